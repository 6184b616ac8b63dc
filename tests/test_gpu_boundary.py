"""The drop-in boundary on an MI355X, through the C ABI: setup validation,
setup-pool reuse, CSR capacity, the masked-logit sampler and its rollout, the
reference's host-copy API of the device state, the multi-tile CSR scan, and the
12 reference games replayed on the device against the vectors junqi_core wrote.
"""

from __future__ import annotations

import ctypes
import hashlib
import json

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests import gpu_compare as G  # noqa: E402
from tests import helpers as H  # noqa: E402


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


# ------------------------------------------------------------ setup validation

def test_invalid_setups_are_rejected(jq):
    print("[boundary] invalid setups", flush=True)
    n = 8
    b = jq.JunqiBatch(n, show_mode=2, pool_size=16)
    b.reset(5)
    z0 = b.get_field("zobrist").copy()
    good = jq.generate_lineups(77, n)
    cases = 0
    for path in H.scenario_files("setup_validation"):
        su = json.loads(path.read_text())["setup_only"]
        lu = [H.TYPE_OF[x] for x in su["lineups"][0]]
        if su["expect_valid"] or len(lu) != 30:
            continue
        bad = good.copy()
        bad[5, 60:90] = lu          # env 5, seat 2
        with pytest.raises(ValueError, match="env 5 seat 2"):
            b.reset_lineups(bad)
        assert np.array_equal(b.get_field("zobrist"), z0), "a rejected reset touched the state"
        cases += 1
    assert cases >= 6
    bad = good.copy()
    bad[0, 3] = 14                  # not a PieceType
    with pytest.raises(ValueError, match="TYPE"):
        b.reset_lineups(bad)
    # a bad pool entry: the upload fails and the handle keeps its old pool
    old_pool = b.pool.copy()
    pool = jq.generate_pool(3, 40)
    pool[17, 6] = H.TYPE_OF["PAIZH"]   # a piece in camp 6 of seat 0
    with pytest.raises(ValueError, match="pool entry 17 seat 0 breaks C1"):
        b.upload_setup_pool(pool)
    b.reset_lineups(good)
    b.set_termination(np.ones(n, bool), np.zeros(n, np.int8), np.zeros(n, bool))
    b.reset_terminated(9)
    games = [O.Game(old_pool[G.reset_pool_index(i, 9, len(old_pool))], show_mode=2) for i in range(n)]
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="reset from the kept pool")
    b.close()


def test_setup_pool_upload_reuses_its_buffer(jq):
    print("[boundary] pool reuse", flush=True)
    b = jq.JunqiBatch(64, show_mode=2, pool_size=4096)
    pools = [jq.generate_pool(s, 4096 - 37 * s) for s in range(20)]
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for rep in range(10):
        for p in pools:
            b.upload_setup_pool(p)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 - free1 < (4 << 20), f"device memory fell by {free0 - free1} bytes over 200 uploads"
    # the last pool is the one resets read
    last = pools[-1]
    b.reset(1)
    b.set_termination(np.ones(64, bool), np.zeros(64, np.int8), np.zeros(64, bool))
    b.reset_terminated(4)
    games = [O.Game(last[G.reset_pool_index(i, 4, len(last))], show_mode=2) for i in range(64)]
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="reset after re-uploads")
    b.close()


# ------------------------------------------------------------ CSR capacity

def test_csr_capacity(jq):
    print("[boundary] CSR capacity", flush=True)
    from junqi_amd import _lib as L
    n = 96
    b = jq.JunqiBatch(n, show_mode=2, pool_size=16)
    b.reset(8)
    h = b._h
    counts = torch.zeros(n, dtype=torch.int32, device=b.device)
    offs = torch.zeros(n + 1, dtype=torch.int32, device=b.device)
    b.legal()
    total = int(b.offsets[-1])
    want = b.values[:total].clone()
    for cap, ok in ((total, True), (total + 5, True), (total - 1, False), (0, False)):
        vals = torch.full((total + 64,), -7, dtype=torch.int32, device=b.device)
        rc = L.lib.jq_legal(h, None, counts.data_ptr(), offs.data_ptr(), vals.data_ptr(), cap, None, None, b.stream)
        torch.cuda.synchronize()
        assert torch.equal(offs, b.offsets) and torch.equal(counts, b.counts)
        if ok:
            assert rc == 0
            assert torch.equal(vals[:total], want)
            assert bool((vals[total:] == -7).all()), "values written past the ids"
        else:
            assert rc == L.JQ_E_CAPACITY, rc
            assert "buffer holds" in L.lib.jq_last_error().decode()
            assert bool((vals == -7).all()), "values written although they do not fit"
    # the fused env-step with a small buffer: the step applies, counts and offsets follow, values do not
    small = torch.full((10,), -7, dtype=torch.int32, device=b.device)
    acts = torch.empty(n, dtype=torch.int32, device=b.device)
    with pytest.raises(L.CapacityError):
        L.check(L.lib.jq_env_step(h, None, L.SAMPLE_UNIFORM, 3, 0, 0, b.counts.data_ptr(), b.offsets.data_ptr(),
                                  small.data_ptr(), small.numel(), None, L.OBS_U8, None, None, None, None, None,
                                  None, acts.data_ptr(), b.stream))
    assert bool((small == -7).all())
    b.close()


def test_env_step_rejects_bad_observation_buffers_before_stepping(jq):
    """jq_env_step checks its observation arguments (alignment, format, tables)
    before it launches anything: a rejected call leaves the state, the CSR and
    the outputs as they were."""
    print("[boundary] env_step argument checks", flush=True)
    from junqi_amd import _lib as L
    n = 64
    b = jq.JunqiBatch(n, show_mode=2, pool_size=16)
    b.reset(12)
    b.legal()
    dev = b.device
    z0, c0, o0 = b.get_field("zobrist").copy(), b.counts.clone(), b.offsets.clone()
    sp = torch.empty((n, 317, 17, 17), dtype=torch.uint8, device=dev)
    aux = torch.empty(n * L.AUX_BYTES + 16, dtype=torch.uint8, device=dev)
    gl = torch.empty(n * 28 + 1, dtype=torch.float32, device=dev)
    bf = torch.empty(n * 317 * 289 + 1, dtype=torch.int16, device=dev)
    acts = torch.full((n,), -5, dtype=torch.int32, device=dev)
    bad = [  # (fmt, spatial, aux, global): misaligned aux, misaligned bf16 rows, unknown format
        (L.OBS_U8, sp.data_ptr(), aux.data_ptr() + 4, gl.data_ptr()),
        (L.OBS_BF16, bf.data_ptr() + 1, None, gl.data_ptr()),
        (7, sp.data_ptr(), None, None),
    ]
    for fmt, s_ptr, a_ptr, g_ptr in bad:
        rc = L.lib.jq_env_step(b._h, None, L.SAMPLE_LOGITS, 1, 0, 0, b.counts.data_ptr(), b.offsets.data_ptr(),
                               b.values.data_ptr(), b.values.numel(), b.mask_words.data_ptr(), fmt, s_ptr, a_ptr,
                               g_ptr, None, None, None, acts.data_ptr(), b.stream)
        torch.cuda.synchronize()
        assert rc == L.JQ_E_ARG, (fmt, rc)
        assert np.array_equal(b.get_field("zobrist"), z0), "a rejected call stepped the games"
        assert torch.equal(b.counts, c0) and torch.equal(b.offsets, o0)
        assert bool((acts == -5).all()), "a rejected call sampled actions"
    b.close()


def test_env_step_side_stream_csr(jq):
    """jq_env_step with a u8 observation and a full-size values buffer runs the
    CSR pass on a side stream beside the observation; with a smaller buffer it
    runs in line (after the total is read back). Both must give the same rows,
    masks, observations and step results, on a non-default caller stream whose
    later work sees the joined results; the observation timing hooks count every
    launch."""
    print("[boundary] side-stream CSR pass", flush=True)
    from junqi_amd import _lib as L
    n, steps = 3000, 24
    side, inline = (jq.JunqiBatch(n, show_mode=2, pool_size=64) for _ in range(2))
    for b in (side, inline):
        b.reset(31)
        b.legal()
    dev = side.device
    st = torch.cuda.Stream(dev)
    mk = lambda: (torch.empty((n, 317, 17, 17), dtype=torch.uint8, device=dev),  # noqa: E731
                  torch.empty((n, L.AUX_BYTES), dtype=torch.uint8, device=dev),
                  torch.empty((n, 28), dtype=torch.float32, device=dev),
                  torch.empty(n, dtype=torch.uint8, device=dev), torch.empty(n, dtype=torch.float32, device=dev),
                  torch.empty(n, dtype=torch.int64, device=dev), torch.empty(n, dtype=torch.int32, device=dev))
    outs = {"side": mk(), "inline": mk()}
    caps = {"side": side.values.numel(), "inline": n * 200}
    assert caps["inline"] < n * L.MAX_LEGAL <= caps["side"]
    L.check(L.lib.jq_obs_timing(side._h, 1))
    with torch.cuda.stream(st):
        for k in range(steps):
            snap = {}
            for name, b in (("side", side), ("inline", inline)):
                sp, aux, gl, te, rw, hs, ac = outs[name]
                L.check(L.lib.jq_env_step(b._h, None, L.SAMPLE_LOGITS, 5, k, k, b.counts.data_ptr(),
                                          b.offsets.data_ptr(), b.values.data_ptr(), caps[name],
                                          b.mask_words.data_ptr(), L.OBS_U8, sp.data_ptr(), aux.data_ptr(),
                                          gl.data_ptr(), te.data_ptr(), rw.data_ptr(), hs.data_ptr(), ac.data_ptr(),
                                          st.cuda_stream))
                # read on the caller's stream right after the call
                tot = b.offsets[-1].clone()
                snap[name] = (b.counts.clone(), b.offsets.clone(), b.values[:n * 200].clone(), b.mask_words.clone(),
                              tot, sp.clone(), aux.clone(), gl.clone(), te.clone(), rw.clone(), hs.clone(), ac.clone())
            st.synchronize()
            a, c = snap["side"], snap["inline"]
            t = int(a[4])
            assert t == int(c[4]) and t <= n * 200
            for i, (x, y) in enumerate(zip(a, c)):
                if i == 2:
                    x, y = x[:t], y[:t]
                assert torch.equal(x, y), f"step {k}: output {i} differs"
    total_ms, launches = ctypes.c_double(), ctypes.c_int64()
    L.check(L.lib.jq_obs_timing_read(side._h, ctypes.byref(total_ms), ctypes.byref(launches)))
    L.check(L.lib.jq_obs_timing(side._h, 0))
    assert launches.value == steps and total_ms.value > 0.0
    side.close()
    inline.close()


def test_multi_tile_scan(jq):
    """n > 32,768 runs the scan's tile carry: offsets are the exclusive cumsum of
    counts and every row is its env's ascending legal ids (rows on both sides of
    the tile edge and the last ones checked against the oracle)."""
    print("[boundary] multi-tile scan n=40000", flush=True)
    n = 40000
    b = jq.JunqiBatch(n, show_mode=2, pool_size=64)
    b.reset(21)
    b.legal()
    counts = b.counts.cpu().numpy().astype(np.int64)
    offs = b.offsets.cpu().numpy().astype(np.int64)
    assert offs[0] == 0 and np.array_equal(np.diff(offs), counts)
    vals = b.values[: int(offs[-1])].cpu().numpy()
    rows = [vals[offs[i]:offs[i + 1]] for i in range(n)]
    assert all((np.diff(r) > 0).all() for r in rows[::97])
    lineups = jq.generate_lineups(21, n)
    for i in list(range(32760, 32780)) + [0, n - 1, n - 2]:
        g = O.Game(lineups[i], show_mode=2)
        assert np.array_equal(rows[i], g.legal_ids()), i
    b.close()


# ------------------------------------------------------------ the masked-logit sampler

def test_logit_sampler_matches_oracle(jq):
    print("[boundary] logit sampler", flush=True)
    n = 300
    b = jq.JunqiBatch(n, show_mode=2, pool_size=64)
    b.reset(31)
    games = G.oracle_games_from_lineups(jq.generate_lineups(31, n), 2)
    rng = np.random.default_rng(1)
    for ply in range(30):
        b.legal()
        canon = torch.empty(n, dtype=torch.int32, device=b.device)
        got = b.sample_logits(0xC5, ply, canonical_out=canon).cpu().numpy()
        canon = canon.cpu().numpy()
        acts = np.zeros(n, np.int32)
        for i, g in enumerate(games):
            ids = g.legal_ids()
            w, c = O.sample_logits(ids, int(g.turn), i, 0xC5, ply)
            assert (int(got[i]), int(canon[i])) == (w, c), f"ply {ply} env {i}"
            acts[i] = ids[rng.integers(len(ids))]   # play on with another stream
        b.step(torch.from_numpy(acts).to(b.device))
        for i, g in enumerate(games):
            assert g.step_id(int(acts[i]))[0] == 0
    # an explicit acting seat other than the turn maps the same row through that seat's rotation
    b.legal()
    seats = torch.full((n,), 2, dtype=torch.int8, device=b.device)
    canon = torch.empty(n, dtype=torch.int32, device=b.device)
    got = b.sample_logits(7, 3, acting=seats, canonical_out=canon).cpu().numpy()
    canon = canon.cpu().numpy()
    for i, g in enumerate(games[:50]):
        w, c = O.sample_logits(g.legal_ids(), 2, i, 7, 3)
        assert (int(got[i]), int(canon[i])) == (w, c)
    b.close()


@pytest.mark.parametrize("sampler", ["logits", "uniform"])
def test_rollout_streams_match_oracle(jq, sampler):
    """The c5 loop at 2,048 games x 256 env-steps (fused jq_env_step: sample ->
    step -> pool restart -> legal), every game's per-step reward, done, hash and
    action equal to the oracle's batched rollout. A 120-move cap makes every
    game end and restart twice inside the window."""
    print(f"[boundary] rollout {sampler}", flush=True)
    n, steps, seed = 2048, 256, 0xC5
    b = jq.JunqiBatch(n, show_mode=2, pool_size=128, max_num_moves=120)
    b.reset(41)
    b.legal()
    dev = b.device
    rew = torch.empty((steps, n), dtype=torch.float32, device=dev)
    done = torch.empty((steps, n), dtype=torch.uint8, device=dev)
    hsh = torch.empty((steps, n), dtype=torch.int64, device=dev)
    act = torch.empty((steps, n), dtype=torch.int32, device=dev)
    for k in range(steps):
        b.env_step(sampler=sampler, sample_seed=seed, ply=k, reset_seed=k, spatial=None, terminated=done[k],
                   reward=rew[k], hash_out=hsh[k], actions_out=act[k])
    torch.cuda.synchronize()
    ob = O.Batch(jq.generate_lineups(41, n), show_mode=2, max_num_moves=120)
    ref = O.rollout(ob, b.pool, sampler=1 if sampler == "logits" else 0, seed=seed, ply0=0, reset_seed0=0,
                    steps=steps)
    assert np.array_equal(act.cpu().numpy(), ref["actions"])
    assert np.array_equal(done.cpu().numpy(), ref["done"])
    assert np.array_equal(rew.cpu().numpy(), ref["reward"])
    assert np.array_equal(hsh.cpu().numpy().view(np.uint64), ref["hash"])
    assert int(ref["done"].sum()) > 0, "no game ended: the restart path went untested"
    G.compare_state(G.device_fields(b), G.oracle_fields([_game_of(ob, i) for i in range(n)]), ctx="after rollout")
    b.close()


def _game_of(batch, i):
    g = O.Game(None)
    g.buf[0] = batch.games[i]
    return g


# ------------------------------------------------------------ host-copy API

def test_v1_collector_host_copy_reset(jq):
    """The v1 PPO collector's reset of finished envs through the state's host
    copies (junqi_rl/training/gpu_collector.py:596-650): copy_to_host, fresh
    games written into the finished slots, copy_from_host,
    copy_termination_from_host. Untouched envs keep their whole state (combat
    memory, beliefs, history); reset slots start as new games; play continues in
    step with the oracle."""
    print("[boundary] v1 host copies", flush=True)
    n, show = 48, 1
    b = jq.JunqiBatch(n, show_mode=show, pool_size=32, max_num_moves=30)
    b.reset(51)
    games = G.oracle_games_from_lineups(jq.generate_lineups(51, n), show, 30)
    rng = np.random.default_rng(2)

    def play(plies):
        for _ in range(plies):
            acts = np.full(n, -1, np.int32)
            for i, g in enumerate(games):
                if not g.terminated:
                    ids = g.legal_ids()
                    acts[i] = ids[rng.integers(len(ids))]
                    assert g.step_id(int(acts[i]))[0] == 0
            b.step(torch.from_numpy(acts).to(b.device))

    play(20 + 0)
    for i in range(0, n, 3):       # end a third of the games
        games[i].buf[0]["terminated"] = 1
    t = b.copy_termination_to_host()
    t["terminated"][0::3] = True
    b.copy_termination_from_host(t["terminated"], t["winner_team"], t["draw"])
    for g in games:
        g.buf[0]["zobrist"] = np.uint64(g.recompute_zobrist())
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="terminated by hand")
    # the collector's reset (gpu_collector.py:596-650)
    assert np.array_equal(b.copy_turn_to_host(), np.array([int(g.turn) for g in games], np.int8))
    host = b.copy_to_host()
    assert set(host) == set(G.oracle_pack(games))
    for k, v in G.oracle_pack(games).items():
        if k != "zobrist":
            assert np.array_equal(host[k], v), k
    term = b.copy_termination_to_host()
    idxs = np.where(term["terminated"])[0]
    fresh = [O.Game(O.random_setup(900 + int(i)), show_mode=show, max_num_moves=30) for i in idxs]
    packed = G.oracle_pack(fresh)
    per = {"cell_piece_id": 289, "seat_dead_arr": 4, "seat_flag_revealed_arr": 4, "turn": 1, "zobrist": 1,
           "move_counter": 1, "moves_since_last_combat": 1}
    for k in host:
        w = per.get(k, 120)
        host[k].reshape(n, w)[idxs] = packed[k].reshape(len(idxs), w)
    b.copy_from_host(host)
    term["terminated"][idxs] = False
    term["winner_team"][idxs] = -1
    term["draw"][idxs] = False
    b.copy_termination_from_host(term["terminated"], term["winner_team"], term["draw"])
    for j, i in enumerate(idxs):
        games[i] = fresh[j]
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="after the host-copy reset")
    play(12)
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="play after the reset")
    sp, gl = b.observe(fmt="f32", all_seats=True)
    sp, gl = sp.cpu().numpy(), gl.cpu().numpy()
    for i in range(0, n, 5):
        for s in range(4):
            osp, ogl = games[i].observe(s)
            assert np.array_equal(sp[i, s], osp) and np.array_equal(gl[i, s], ogl), (i, s)
    b.close()


# ------------------------------------------------------------ reference vectors on the device

def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("mode", ["BRIGHT", "DARK", "HALF_DARK"])
def test_reference_games_on_device(jq, mode):
    """The 12 complete games junqi_core played (tests/golden/reference_vectors.json):
    the device's Zobrist hash after every ply, the acting seat's CSR legal row
    before every ply and at the end (size and digest of the reference's
    GameState.legal_actions), and all four observers' float32 observations and
    globals at the recorded plies, bit for bit."""
    print(f"[boundary] reference games {mode}", flush=True)
    doc = json.loads((H.GOLDEN / "reference_vectors.json").read_text())
    recs = [r for r in doc["games"] if r["show_mode"] == mode]
    n = len(recs)
    show = {"BRIGHT": 0, "DARK": 1, "HALF_DARK": 2}[mode]
    b = jq.JunqiBatch(n, show_mode=show, pool_size=8)
    b.reset_lineups(np.stack([np.asarray(r["setup"], np.int8) for r in recs]))
    cps = [{cp["ply"]: cp for cp in r["checkpoints"]} for r in recs]
    plies = max(len(r["actions"]) for r in recs)

    def check(ply):
        due = [i for i in range(n) if ply in cps[i]]
        if not due:
            return
        sp, gl = b.observe(fmt="f32", all_seats=True)
        sp, gl = sp.cpu().numpy(), gl.cpu().numpy()
        for i in due:
            for s in range(4):
                assert _sha(sp[i, s]) == cps[i][ply]["obs_f32"][s], f"game {i} ply {ply} observer {s}"
                assert _sha(gl[i, s]) == cps[i][ply]["glob_f32"][s], f"game {i} ply {ply} globals {s}"

    def check_legal(ply):   # the sets before ply + 1
        b.legal()
        offs = b.offsets.cpu().numpy()
        vals = b.values[: int(offs[-1])].cpu().numpy()
        for i, r in enumerate(recs):
            if ply < len(r["legal_count"]):
                row = vals[offs[i]:offs[i + 1]].astype("<i4")
                assert len(row) == r["legal_count"][ply], f"game {i} before ply {ply + 1}: legal count"
                assert _sha(row)[:16] == r["legal_digest"][ply], f"game {i} before ply {ply + 1}: legal set"

    check(0)
    for ply in range(1, plies + 1):
        check_legal(ply - 1)
        acts = np.array([r["actions"][ply - 1][0] * 289 + r["actions"][ply - 1][1] if ply <= len(r["actions"])
                         else -1 for r in recs], np.int32)
        out = b.step(torch.from_numpy(acts).to(b.device))
        valid = out["valid"].cpu().numpy()
        z = b.get_field("zobrist")[:, 0]
        for i, r in enumerate(recs):
            if ply <= len(r["actions"]):
                assert valid[i], f"game {i} ply {ply}: reference action rejected"
                assert format(int(z[i]), "016x") == r["zobrist"][ply - 1], f"game {i} ply {ply}: Zobrist"
        check(ply)
    check_legal(plies)
    assert [bool(t) for t in b.termination()["terminated"]] == [r["terminated"] for r in recs]
    b.close()
