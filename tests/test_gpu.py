"""Parity of the HIP path (through the C ABI) with the oracle, on an MI355X.

Every comparison is bit-exact: state fields, Zobrist hashes, step results,
sorted legal-id rows, canonical masks and float32 observations. bf16 must equal
round-to-nearest-even of the float32 values; u8 codes must decode exactly.
"""

from __future__ import annotations

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


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def _play(jq, n, plies, show_mode, seed, check_every=1, obs_every=1, all_seats_every=50, max_moves=4000):
    """Random legal play on device and oracle side by side, auto-reset from the pool."""
    print(f"[play] n={n} plies={plies} show_mode={show_mode} seed={seed}", flush=True)
    b = jq.JunqiBatch(n, show_mode=show_mode, max_num_moves=max_moves, pool_size=256)
    b.reset(seed)
    lineups = jq.generate_lineups(seed, n)
    games = G.oracle_games_from_lineups(lineups, show_mode, max_moves)
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="reset")
    rng = np.random.default_rng(seed)
    tables = O.tables()
    for ply in range(plies):
        if ply % 40 == 0:
            print(f"[play] ply {ply}", flush=True)
        b.legal()   # CSR and packed canonical mask in one call
        offs = b.offsets.cpu().numpy()
        vals = b.values[: int(offs[-1])].cpu().numpy()
        mw = b.mask_words.cpu().numpy()
        actions = np.zeros(n, np.int32)
        for i, g in enumerate(games):
            ids = g.legal_ids()
            row = vals[offs[i]:offs[i + 1]]
            assert np.array_equal(row, ids), f"ply {ply} env {i}: legal row differs"
            assert np.array_equal(mw[i], G.canonical_mask_words(ids, int(g.turn), tables)), \
                f"ply {ply} env {i}: canonical mask differs"
            actions[i] = ids[rng.integers(len(ids))] if len(ids) else -1
        if ply % obs_every == 0:
            sp, gl = b.observe(fmt="f32")
            sp, gl = sp.cpu().numpy(), gl.cpu().numpy()
            for i, g in enumerate(games):
                osp, ogl = g.observe(int(g.turn))
                if not np.array_equal(sp[i].view(np.uint32), osp.view(np.uint32)):
                    bad = np.argwhere(sp[i] != osp)[:5]
                    raise AssertionError(f"ply {ply} env {i}: obs differs at {bad.tolist()} "
                                         f"dev {sp[i][tuple(bad[0])]} oracle {osp[tuple(bad[0])]}")
                assert np.array_equal(gl[i], ogl), f"ply {ply} env {i}: globals differ"
        if ply % all_seats_every == 0:
            sp4, gl4 = b.observe(fmt="f32", all_seats=True)
            sp4, gl4 = sp4.cpu().numpy(), gl4.cpu().numpy()
            for i, g in enumerate(games[:8]):
                for o in range(4):
                    osp, ogl = g.observe(o)
                    assert np.array_equal(sp4[i, o], osp) and np.array_equal(gl4[i, o], ogl), (ply, i, o)
        out = b.step(torch.from_numpy(actions).to(b.device))
        res = {k: v.cpu().numpy() for k, v in out.items()}
        seed_reset = seed * 7919 + ply
        for i, g in enumerate(games):
            if actions[i] < 0:
                continue
            seat = int(g.turn)
            rc, r = g.step_id(int(actions[i]))
            assert rc == 0
            assert bool(res["valid"][i]) and res["event"][i] == r["event"], (ply, i, r, res["event"][i])
            assert bool(res["terminated"][i]) == bool(r["terminated"])
            assert res["winner_team"][i] == r["winner"] and bool(res["draw"][i]) == bool(r["draw"])
            assert bool(res["flag_captured"][i]) == bool(r["flag_captured"])
            assert res["seats_died"][i] == r["seats_died_mask"]
            want = 0.0
            if r["terminated"] and not r["draw"] and r["winner"] >= 0:
                want = 1.0 if (seat & 1) == r["winner"] else -1.0
            assert res["rewards"][i] == want
        if ply % check_every == 0:
            G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"ply {ply}")
        term = [i for i, g in enumerate(games) if g.terminated]
        if term:
            b.reset_terminated(seed_reset)
            for i in term:
                idx = G.reset_pool_index(i, seed_reset, b.pool.shape[0])
                games[i] = O.Game(b.pool[idx], show_mode=show_mode, max_num_moves=max_moves)
            G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"reset after ply {ply}")
    b.close()


def test_play_half_dark(jq):
    _play(jq, 48, 260, 2, seed=11)


def test_play_bright_and_dark(jq):
    _play(jq, 24, 160, 0, seed=5, check_every=2, obs_every=2)
    _play(jq, 24, 160, 1, seed=6, check_every=2, obs_every=2)


@pytest.mark.parametrize("show_mode", [0, 1, 2])
def test_c1_64_games_200_plies(jq, show_mode):
    # the CPU-reference plumbing configuration: 64 four-player games from seeded
    # random legal setups, 200 plies of seeded uniform-random legal actions; hash,
    # state, CSR rows, canonical masks and observations after every ply
    _play(jq, 64, 200, show_mode, seed=64 + show_mode, check_every=1, obs_every=1)


def test_play_move_cap(jq):
    # the env cap (max_num_moves) ends games in a draw after the turn advance
    _play(jq, 16, 90, 2, seed=3, max_moves=60, check_every=3, obs_every=3)


def test_obs_formats_agree(jq):
    print("[formats]", flush=True)
    b = jq.JunqiBatch(64, show_mode=2)
    b.reset(100)
    rng = np.random.default_rng(0)
    for ply in range(60):
        offs, vals = b.legal_csr_numpy()
        acts = np.array([vals[offs[i] + rng.integers(offs[i + 1] - offs[i])] for i in range(b.n)], np.int32)
        b.step(torch.from_numpy(acts).to(b.device))
    f32, g32 = b.observe(fmt="f32")
    bf, gbf = b.observe(fmt="bf16")
    u8, gu8, aux = b.observe(fmt="u8")
    f32 = f32.cpu().numpy()
    assert np.array_equal(bf.view(torch.int16).cpu().numpy().view(np.uint16), _bf16_rne(f32))
    u8n = u8.cpu().numpy()
    for ch in jq.AUX_CHANNELS:
        assert np.all(u8n[:, ch] == 0)
    dec = jq.decode_u8(u8n, aux.cpu().numpy())
    assert np.array_equal(dec.view(np.uint32), f32.view(np.uint32))
    assert torch.equal(jq.decode_u8(u8, aux).cpu(), torch.from_numpy(dec))   # the device decode too
    assert np.array_equal(g32.cpu().numpy(), gu8.cpu().numpy())
    b.close()


def test_mask_bool_matches_words(jq):
    b = jq.JunqiBatch(32, show_mode=2)
    b.reset(7)
    out = b.legal(mask_bool=True)
    words = out["mask_words"].cpu().numpy().view(np.uint32)
    bits = ((words[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(32, -1)[:, :16641]
    assert np.array_equal(bits.astype(bool), out["mask_bool"].cpu().numpy())
    b.close()


def test_sampler_is_philox_uniform(jq):
    b = jq.JunqiBatch(256, show_mode=2)
    b.reset(1)
    b.legal()
    acts = b.sample_uniform(seed=0x4A51, ply=12).cpu().numpy()
    counts = b.counts.cpu().numpy()
    offs = b.offsets.cpu().numpy()
    vals = b.values.cpu().numpy()
    for i in range(b.n):
        u = G.philox_first_word(i, 12, 0, 0, 0x4A51, 0)
        assert acts[i] == vals[offs[i] + ((u * int(counts[i])) >> 32)]
    b.close()


def test_canonical_action_step_matches_world(jq):
    """step_device_torch's canonical compact ids unrotate to the same world move."""
    b1 = jq.JunqiBatch(32, show_mode=2)
    b2 = jq.JunqiBatch(32, show_mode=2)
    b1.reset(9); b2.reset(9)
    rng = np.random.default_rng(2)
    tables = O.tables()
    c2f = tables["compact_to_flat"]
    f2c = np.full(289, -1, np.int32); f2c[c2f] = np.arange(129)
    for _ in range(40):
        offs, vals = b1.legal_csr_numpy()
        seats = b1.field_tensor("turn").cpu().numpy().astype(np.int64)
        w = np.array([vals[offs[i] + rng.integers(offs[i + 1] - offs[i])] for i in range(32)], np.int32)
        can = np.zeros(32, np.int32)
        for i in range(32):
            s, d = divmod(int(w[i]), 289)
            rot = lambda f, st=seats[i]: [(f % 17, f // 17), (f // 17, 16 - f % 17), (16 - f % 17, 16 - f // 17), (16 - f // 17, f % 17)][st]
            cs = rot(s); cd = rot(d)
            can[i] = f2c[cs[1] * 17 + cs[0]] * 129 + f2c[cd[1] * 17 + cd[0]]
        r1 = b1.step(torch.from_numpy(w).cuda())
        r2 = b2.step(torch.from_numpy(can).cuda(), torch.from_numpy(seats.astype(np.int8)).cuda(), canonical=True)
        assert torch.equal(r2["world_action"], torch.from_numpy(w).cuda())
        assert torch.equal(r1["event"], r2["event"])
    assert np.array_equal(b1.get_field("zobrist"), b2.get_field("zobrist"))
    b1.close(); b2.close()


def _import_positions(jq, b, positions):
    """positions: list of dicts(pieces=[(pid,type,x,y)], turn, mc, mslc, dead, flag)."""
    n = b.n
    cell = np.full((n, 292), -1, np.int8)
    ptype = np.full((n, 128), -1, np.int8)
    pos = np.full((n, 128), -1, np.int16)
    for i, p in enumerate(positions):
        for pid, t, x, y in p["pieces"]:
            cell[i, y * 17 + x] = pid
            ptype[i, pid] = t
            pos[i, pid] = y * 17 + x
    zero = np.full((n, 128), -1, np.int16)
    b.set_field("cell", cell); b.set_field("ptype", ptype); b.set_field("pos", pos); b.set_field("zero", zero)
    for f in ("move_count", "active_eat", "passive_surv"):
        b.set_field(f, np.zeros((n, 128), np.int16))
    b.set_field("death_reason", np.full((n, 128), -1, np.int8))
    b.set_field("death_step", np.full((n, 128), -1, np.int16))
    b.set_field("death_loc", np.full((n, 128), -1, np.int16))
    for dev, _ in G.CM_FIELDS:
        e, by = jq._lib.field_info(dev)
        fill = -1 if dev in ("cm_last_direct", "cm_last_chain", "cm_floor_step") else 0
        b.set_field(dev, np.full((n, e), fill, np.int64))
    b.set_field("cm_flags", np.zeros((n, 512), np.uint8))
    b.set_field("hist_meta", np.zeros((n, 1), np.int32))
    b.set_field("turn", np.array([p["turn"] for p in positions], np.int8))
    b.set_field("move_counter", np.array([p["mc"] for p in positions], np.int32))
    b.set_field("mslc", np.array([p["mslc"] for p in positions], np.int32))
    b.set_field("seat_dead", np.array([sum(v << s for s, v in enumerate(p["dead"])) for p in positions], np.uint8))
    b.set_field("flag_rev", np.array([sum(v << s for s, v in enumerate(p["flag"])) for p in positions], np.uint8))
    b.set_field("terminated", np.zeros(n, np.uint8)); b.set_field("draw", np.zeros(n, np.uint8))
    b.set_field("winner", np.full(n, -1, np.int8))
    b.finalize_import()


def test_golden_scenarios_on_device(jq):
    cases = [json.loads(p.read_text()) for c in ("battle", "siling_flag", "stronghold", "inference",
                                                 "full_game", "move_gen") for p in H.scenario_files(c)]
    positions = []
    for d in cases:
        pre = d["pre_state"]
        dead, fr = H.scenario_info(pre)
        positions.append(dict(pieces=H.scenario_pieces(pre), turn=pre["turn"], mc=pre["move_counter"],
                              mslc=pre["moves_since_last_combat"], dead=dead, flag=fr))
    b = jq.JunqiBatch(len(cases), show_mode=2)
    _import_positions(jq, b, positions)
    games = [O.Game.from_pieces(p["pieces"], turn=p["turn"], move_counter=p["mc"], mslc=p["mslc"],
                                seat_dead=p["dead"], flag_rev=p["flag"]) for p in positions]
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx="import")
    nsteps = max(len(d["actions"]) for d in cases)
    for k in range(nsteps):
        acts = np.full(len(cases), -1, np.int32)
        for i, d in enumerate(cases):
            if k < len(d["actions"]):
                a = d["actions"][k]
                acts[i] = H.flat(a["src"]) * 289 + H.flat(a["dst"])
        out = b.step(torch.from_numpy(acts).cuda())
        ev = out["event"].cpu().numpy()
        for i, d in enumerate(cases):
            if acts[i] < 0:
                continue
            exp = d["expected"]["results"][k]
            assert ev[i] == H.EVENT_OF[exp["event"]], (d["id"], k)
            games[i].step_id(int(acts[i]))
        G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"scenario step {k}")
    term = b.get_field("terminated")[:, 0]
    for i, d in enumerate(cases):
        assert bool(term[i]) == d["expected"]["terminated"], d["id"]
    b.close()


def _engineer_positions(n, seed):
    """Config c4: every seat keeps 3 engineers and at most 6 other pieces on rail
    cells, plus random nine-grid occupancy."""
    rng = np.random.default_rng(seed)
    t = O.tables()
    rail = [f for f in range(289) if t["rail"][f]]
    out = []
    for _ in range(n):
        cells = rng.permutation(rail).tolist()
        pieces = []
        for s in range(4):
            kinds = [13, 13, 13] + list(rng.choice([4, 5, 6, 7, 8, 9, 10, 11, 12], size=rng.integers(0, 7)))
            for j, k in enumerate(kinds):
                f = cells.pop()
                pieces.append((s * 30 + j, int(k), f % 17, f // 17))
        out.append(dict(pieces=pieces, turn=int(rng.integers(4)), mc=0, mslc=0, dead=[0] * 4, flag=[0] * 4))
    return out


def test_engineer_stress_legal_sets(jq):
    positions = _engineer_positions(512, 4)
    b = jq.JunqiBatch(len(positions), show_mode=2)
    _import_positions(jq, b, positions)
    games = [O.Game.from_pieces(p["pieces"], turn=p["turn"]) for p in positions]
    for seat in range(4):
        acting = torch.full((b.n,), seat, dtype=torch.int8, device=b.device)
        offs, vals = b.legal_csr_numpy(acting)
        for i, g in enumerate(games):
            assert np.array_equal(vals[offs[i]:offs[i + 1]], g.legal_ids(seat)), (i, seat)
    # a few plies from these positions too
    rng = np.random.default_rng(1)
    for ply in range(20):
        offs, vals = b.legal_csr_numpy()
        acts = np.array([vals[offs[i] + rng.integers(offs[i + 1] - offs[i])] if offs[i + 1] > offs[i] else -1
                         for i in range(b.n)], np.int32)
        b.step(torch.from_numpy(acts).cuda())
        for i, g in enumerate(games):
            if acts[i] >= 0:
                g.step_id(int(acts[i]))
        G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"engineer ply {ply}")
    b.close()


def test_slot_mask_matches_oracle(jq):
    """legal_action_mask_batch layout: device slot rows equal the oracle's for
    every seat, during play (with resets) and on engineer-dense positions."""
    n, seed = 48, 23
    print(f"[slots] play n={n} seed={seed}", flush=True)
    b = jq.JunqiBatch(n, show_mode=2, pool_size=64)
    b.reset(seed)
    games = G.oracle_games_from_lineups(jq.generate_lineups(seed, n), 2, 4000)
    rng = np.random.default_rng(seed)
    for ply in range(120):
        if ply % 10 == 0:
            for seat in range(4):
                got = b.legal_slots(torch.full((n,), seat, dtype=torch.int8, device=b.device)).cpu().numpy()
                for i, g in enumerate(games):
                    assert np.array_equal(got[i], g.legal_slots(seat)), (ply, i, seat)
        got = b.legal_slots().cpu().numpy()
        offs, vals = b.legal_csr_numpy()
        acts = np.full(n, -1, np.int32)
        for i, g in enumerate(games):
            assert np.array_equal(got[i], g.legal_slots()), (ply, i)
            row = vals[offs[i]:offs[i + 1]]
            assert int(got[i].sum()) == len(row)
            if len(row):
                acts[i] = row[rng.integers(len(row))]
        b.step(torch.from_numpy(acts).to(b.device))
        for i, g in enumerate(games):
            if acts[i] >= 0:
                g.step_id(int(acts[i]))
        term = [i for i, g in enumerate(games) if g.terminated]
        if term:
            b.reset_terminated(ply)
            for i in term:
                games[i] = O.Game(b.pool[G.reset_pool_index(i, ply, b.pool.shape[0])], show_mode=2)
    b.close()
    positions = _engineer_positions(256, 9)
    print(f"[slots] engineer positions n={len(positions)}", flush=True)
    b = jq.JunqiBatch(len(positions), show_mode=2)
    _import_positions(jq, b, positions)
    games = [O.Game.from_pieces(p["pieces"], turn=p["turn"]) for p in positions]
    out = torch.empty((b.n, 120, 80), dtype=torch.bool, device=b.device)
    for seat in range(4):
        got = b.legal_slots(torch.full((b.n,), seat, dtype=torch.int8, device=b.device), out=out).cpu().numpy()
        for i, g in enumerate(games):
            assert np.array_equal(got[i], g.legal_slots(seat)), (i, seat)
    b.close()


def test_imported_state_observes_like_the_oracle(jq):
    """Every state field of oracle-played games (combat memory, beliefs and the
    move ring included) set through jq_set_field, then jq_rehash: observations
    of all four seats equal the oracle's bit for bit, so the compact
    combat-memory summaries the observation reads are rebuilt from the import."""
    games = []
    for k in range(24):
        g = O.Game(O.random_setup(300 + k), show_mode=2)
        rng = np.random.default_rng(k)
        for _ in range(30 + 8 * k):
            ids = g.legal_ids()
            if not len(ids) or g.terminated:
                break
            g.step_id(int(ids[rng.integers(len(ids))]))
        games.append(g)
    n = len(games)
    print(f"[import] n={n}", flush=True)
    b = jq.JunqiBatch(n, show_mode=2)
    f = G.oracle_fields(games)
    for name, v in f.items():
        if name != "hist_list":
            b.set_field(name, v)
    ring = np.zeros((n, 32), np.int32)
    meta = np.zeros((n, 1), np.int32)
    for i, h in enumerate(f["hist_list"]):
        for j, (src, dst) in enumerate(h):
            ring[i, j] = src | (dst << 16)
        meta[i, 0] = len(h) | ((len(h) & 31) << 8)
    b.set_field("hist", ring)
    b.set_field("hist_meta", meta)
    b.rehash()
    G.compare_state(G.device_fields(b), f, ctx="imported")
    sp4, gl4 = b.observe(fmt="f32", all_seats=True)
    sp4, gl4 = sp4.cpu().numpy(), gl4.cpu().numpy()
    for i, g in enumerate(games):
        for o in range(4):
            osp, ogl = g.observe(o)
            assert np.array_equal(sp4[i, o].view(np.uint32), osp.view(np.uint32)), (i, o)
            assert np.array_equal(gl4[i, o], ogl), (i, o)
    b.close()


def test_invalid_actions_leave_state(jq):
    b = jq.JunqiBatch(8, show_mode=2)
    b.reset(3)
    before = G.device_fields(b)
    bad = torch.tensor([-1, 0, 289 * 289, 5 * 289 + 6, 200 * 289 + 201, 100, 8 * 289 + 8, 83520],
                       dtype=torch.int32, device=b.device)
    out = b.step(bad)
    assert not out["valid"].any()
    after = G.device_fields(b)
    for k in before:
        if k != "hist_list":
            assert np.array_equal(before[k], after[k]), k
    # the same with the legal sets current (the step then tests membership in
    # them): another seat's legal move, a destination the piece cannot reach,
    # a move of a flag or mine
    b.legal()
    games = G.oracle_games_from_lineups(jq.generate_lineups(3, 8), 2)
    rng = np.random.default_rng(5)
    for kind in range(3):
        acts = np.full(8, -1, np.int32)
        for i, g in enumerate(games):
            seat = int(g.turn)
            if kind == 0:
                acts[i] = rng.choice(g.legal_ids((seat + 1) % 4))
            elif kind == 1:
                ids = g.legal_ids(seat)
                src = int(ids[0]) // 289
                own = set(int(x) % 289 for x in ids if int(x) // 289 == src)
                acts[i] = src * 289 + next(d for d in range(289) if d not in own and d != src)
            else:
                pid = next(p for p in range(seat * 30, seat * 30 + 30) if g.ptype[p] in (2, 3) and g.alive[p])
                f = int(g.pos_y[pid]) * 17 + int(g.pos_x[pid])
                acts[i] = f * 289 + (f + 1 if f % 17 < 16 else f - 1)
        out = b.step(torch.from_numpy(acts).to(b.device))
        assert not out["valid"].any(), kind
        after = G.device_fields(b)
        for k in before:
            if k != "hist_list":
                assert np.array_equal(before[k], after[k]), (kind, k)
    ok = np.array([g.legal_ids()[0] for g in games], np.int32)
    assert b.step(torch.from_numpy(ok).to(b.device))["valid"].all()
    b.close()


@pytest.mark.parametrize("max_moves,plies,n,fmt,given,show", [
    (4000, 120, 64, "u8", False, 2), (25, 90, 62, "u8", False, 2), (25, 40, 33, "f32", False, 2),
    (25, 60, 40, "u8", True, 2), (25, 60, 36, "u8", False, 1), (25, 60, 36, "f32", False, 0)])
def test_env_step_fused_matches_oracle(jq, max_moves, plies, n, fmt, given, show):
    """The env-step (sample, step, auto-reset, legal, observation) agrees with
    the oracle stepped with the same Philox choices: state, sorted CSR rows,
    canonical mask words and observations after every step. A 25-move cap
    makes games end and restart from the pool every 25 plies. Odd batch
    sizes, the u8 and the f32 observation, HALF_DARK, DARK and BRIGHT.
    `given`: the caller passes the actions instead, legal ones mixed with -1
    and arbitrary (mostly illegal) world ids, which leave their env as it was."""
    print(f"[env_step] max_moves={max_moves} plies={plies} n={n} fmt={fmt} given={given} show={show}", flush=True)
    rng = np.random.default_rng(n)
    b = jq.JunqiBatch(n, show_mode=show, pool_size=128, max_num_moves=max_moves)
    b.reset(21)
    games = G.oracle_games_from_lineups(jq.generate_lineups(21, n), show, max_moves)
    b.legal()
    u8 = fmt == "u8"
    sp = torch.empty((n, 317, 17, 17), dtype=torch.uint8 if u8 else torch.float32, device=b.device)
    aux = torch.empty((n, jq._lib.AUX_BYTES), dtype=torch.uint8, device=b.device) if u8 else None
    gl = torch.empty((n, 28), dtype=torch.float32, device=b.device)
    term = torch.empty(n, dtype=torch.uint8, device=b.device)
    rew = torch.empty(n, dtype=torch.float32, device=b.device)
    acts = torch.empty(n, dtype=torch.int32, device=b.device)
    dec = jq.decode_table()
    tables = O.tables()
    resets = 0
    for ply in range(plies):
        offs = b.offsets.cpu().numpy(); vals = b.values.cpu().numpy(); counts = b.counts.cpu().numpy()
        chosen = None
        if given:
            chosen = np.full(n, -1, np.int32)
            for i, g in enumerate(games):
                r, ids = rng.random(), g.legal_ids()
                if r < 0.15:
                    chosen[i] = int(rng.integers(289 * 289))
                elif r >= 0.25 and len(ids):
                    chosen[i] = int(ids[rng.integers(len(ids))])
        b.env_step(actions=None if chosen is None else torch.from_numpy(chosen).to(b.device),
                   sample_seed=77, ply=ply, reset_seed=ply, obs_fmt=fmt, spatial=sp, aux=aux, glob=gl,
                   terminated=term, reward=rew, actions_out=acts)
        a = acts.cpu().numpy()
        tm = term.cpu().numpy()
        for i, g in enumerate(games):
            if given:
                want = chosen[i]
            else:
                u = G.philox_first_word(i, ply, 0, 0, 77, 0)
                want = vals[offs[i] + ((u * int(counts[i])) >> 32)] if counts[i] else -1
            assert a[i] == want
            if want >= 0:
                g.step_id(int(want))
        for i, g in enumerate(games):
            assert bool(tm[i]) == bool(g.terminated), (ply, i)
            if g.terminated:
                resets += 1
                games[i] = O.Game(b.pool[G.reset_pool_index(i, ply, b.pool.shape[0])], show_mode=show,
                                  max_num_moves=max_moves)
        G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"fused ply {ply}")
        offs = b.offsets.cpu().numpy(); vals = b.values.cpu().numpy(); mw = b.mask_words.cpu().numpy()
        spn = sp.cpu().numpy(); ax = aux.cpu().numpy() if u8 else None; g2 = gl.cpu().numpy()
        for i, g in enumerate(games):
            ids = g.legal_ids()
            assert np.array_equal(vals[offs[i]:offs[i + 1]], ids), (ply, i)
            assert np.array_equal(mw[i], G.canonical_mask_words(ids, int(g.turn), tables)), (ply, i)
            osp, ogl = g.observe(int(g.turn))
            if u8:
                d = jq.decode_u8(spn[i], ax[i])
            else:
                d = spn[i]
            assert np.array_equal(d.view(np.uint32), osp.view(np.uint32)), (ply, i)
            assert np.array_equal(g2[i], ogl)
    if max_moves < 100:
        assert resets >= n, resets
    b.close()
