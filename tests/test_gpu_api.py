"""The drop-in interfaces (GpuRollout, GpuWorld) against the oracle, on an MI355X.

test_rollout_collector_loop drives GpuRollout through the per-step call order of
the reference collector (junqi_rl/training/gpu_collector.py:763-975): turn view,
acting-seat observation, canonical mask, step_device_torch with compact canonical
ids, update_beliefs_device, reset_terminated_device. Every output is compared
bit-exactly with the oracle stepped with the same moves.
"""

from __future__ import annotations

import types

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests import gpu_compare as G  # noqa: E402


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


def _f2c():
    c2f = O.tables()["compact_to_flat"]
    f2c = np.full(289, -1, np.int64)
    f2c[c2f] = np.arange(129)
    return c2f, f2c


def _rot(f: int, seat: int) -> int:
    x, y = f % 17, f // 17
    cx, cy = [(x, y), (y, 16 - x), (16 - x, 16 - y), (16 - y, x)][seat]
    return cy * 17 + cx


def _canonical_ids(world_ids: np.ndarray, seat: int) -> np.ndarray:
    _, f2c = _f2c()
    s, d = np.divmod(world_ids.astype(np.int64), 289)
    return np.array([f2c[_rot(int(a), seat)] * 129 + f2c[_rot(int(b), seat)] for a, b in zip(s, d)], np.int64)


def test_rollout_collector_loop(jq):
    n, show, seed_base = 40, 1, 77   # DARK, the reference's default show mode
    print(f"[rollout] n={n} show={show}", flush=True)
    ro = jq.GpuRollout(n, show_mode=show, max_num_moves=150)
    ro.reset(seed_base)
    games = G.oracle_games_from_lineups(jq.generate_lineups(seed_base, n), show, 150)
    G.compare_state(G.device_fields(ro.batch), G.oracle_fields(games), ctx="reset")
    rng = np.random.default_rng(5)
    pool = ro.batch.pool
    resets = 0
    for step in range(170):
        acting_t = ro.turn_torch().clone()
        sp_t, gl_t = ro.build_acting_seat_observation_torch(acting_t)
        lm_t = ro.legal_mask_canonical_torch_device(acting_t)
        acting = acting_t.cpu().numpy()
        sp, gl, lm = sp_t.cpu().numpy(), gl_t.cpu().numpy(), lm_t.cpu().numpy()
        acts = np.zeros(n, np.int32)
        world = np.zeros(n, np.int64)
        for i, g in enumerate(games):
            assert int(g.turn) == acting[i]
            osp, ogl = g.observe(int(acting[i]))
            assert np.array_equal(sp[i].view(np.uint32), osp.view(np.uint32)), (step, i, "obs")
            assert np.array_equal(gl[i], ogl), (step, i, "globals")
            ids = g.legal_ids()
            can = _canonical_ids(ids, int(acting[i]))
            want = np.zeros(16641, bool)
            want[can] = True
            assert np.array_equal(lm[i], want), (step, i, "canonical mask")
            k = rng.integers(len(ids))
            acts[i], world[i] = can[k], ids[k]
        res = ro.step_device_torch(torch.from_numpy(acts).cuda(), acting_t)
        ro.update_beliefs_device(res, acting_t)
        r = {k: v.cpu().numpy() for k, v in res.items()}
        for i, g in enumerate(games):
            seat = int(g.turn)
            rc, o = g.step_id(int(world[i]))
            assert rc == 0 and r["event"][i] == o["event"], (step, i)
            assert bool(r["terminated"][i]) == bool(o["terminated"]) and bool(r["draw"][i]) == bool(o["draw"])
            assert r["winner_team"][i] == o["winner"]
            want = 0.0
            if o["terminated"] and not o["draw"] and o["winner"] >= 0:
                want = 1.0 if (seat & 1) == o["winner"] else -1.0
            assert r["rewards"][i] == want
        seed = seed_base + step * 1_000_003
        ro.reset_terminated_device(seed=seed)
        for i, g in enumerate(games):
            if g.terminated:
                resets += 1
                games[i] = O.Game(pool[G.reset_pool_index(i, seed, pool.shape[0])], show_mode=show,
                                  max_num_moves=150)
        assert not ro.terminated_torch().any()
        G.compare_state(G.device_fields(ro.batch), G.oracle_fields(games), ctx=f"step {step}")
    assert resets > 0, "the move cap should have ended some games"
    term = ro.read_termination()
    assert set(term) == {"terminated", "winner_team", "draw"} and term["terminated"].dtype == bool
    ro.close()


def test_rollout_all_seat_observations_with_observer_map(jq):
    n = 12
    ro = jq.GpuRollout(n, show_mode=2)
    ro.reset(3)
    games = G.oracle_games_from_lineups(jq.generate_lineups(3, n), 2)
    rng = np.random.default_rng(1)
    for _ in range(30):
        ids, counts = ro.legal_actions_dense(ro.turn_torch().cpu().numpy())
        acts = np.array([ids[i, rng.integers(counts[i])] for i in range(n)], np.int32)
        out = ro.step(acts)
        assert out["valid"].all()
        for i, g in enumerate(games):
            g.step_id(int(acts[i]))
    seats = np.array([rng.permutation(4) for _ in range(n)], np.int8)
    ro.set_observer_seats(seats)
    sp, gl = ro.build_all_seat_observations()
    assert sp.shape == (n, 4, 317, 17, 17) and gl.shape == (n, 4, 28)
    for i, g in enumerate(games):
        for k in range(4):
            osp, ogl = g.observe(int(seats[i, k]))
            assert np.array_equal(sp[i, k], osp) and np.array_equal(gl[i, k], ogl), (i, k)
    with pytest.raises(ValueError):
        ro.set_observer_seats(np.zeros((n, 3), np.int8))
    ro.close()


def test_rollout_dense_legal_and_reset_from_pool(jq):
    n = 16
    ro = jq.GpuRollout(n, show_mode=2)
    ro.reset(11)
    games = G.oracle_games_from_lineups(jq.generate_lineups(11, n), 2)
    seats = np.array([i % 4 for i in range(n)], np.int8)
    ids, counts = ro.legal_actions_dense(seats)
    assert ids.shape == (n, 512) and ids.dtype == np.int32 and counts.dtype == np.int32
    for i, g in enumerate(games):
        want = g.legal_ids(int(seats[i]))
        assert counts[i] == len(want)
        assert np.array_equal(ids[i, :counts[i]], want) and np.all(ids[i, counts[i]:] == -1)
    m = ro.legal_actions_mask(seats)
    assert m.shape == (n, 120, 80) and m.dtype == bool
    for i, g in enumerate(games):
        assert np.array_equal(m[i], g.legal_slots(int(seats[i]))), i
        assert int(m[i].sum()) == counts[i]
    ro.reset_from_setup_pool(seed=9)
    pool = ro.batch.pool
    games = [O.Game(pool[G.reset_pool_index(i, 9, pool.shape[0])], show_mode=2) for i in range(n)]
    G.compare_state(G.device_fields(ro.batch), G.oracle_fields(games), ctx="reset_from_setup_pool")
    with pytest.raises(ValueError):
        ro.step(np.zeros(n + 1, np.int32))
    ro.close()


def _fake_envs(games):
    """Objects shaped like junqi_rl JunqiEnv: a GameState's SoA arrays at .state."""
    envs = []
    for g in games:
        b = g.buf[0]
        st = types.SimpleNamespace(
            alive=b["alive"].astype(bool), piece_type_arr=b["ptype"].copy(), piece_seat_arr=b["pseat"].copy(),
            pos_x=b["pos_x"].copy(), pos_y=b["pos_y"].copy(), zero_x=b["zero_x"].copy(), zero_y=b["zero_y"].copy(),
            move_count_arr=b["move_count"].copy(), active_eat_arr=b["active_eat"].copy(),
            passive_surv_arr=b["passive_surv"].copy(), death_reason_arr=b["death_reason"].copy(),
            death_step_arr=b["death_step"].copy(), death_loc_flat_arr=b["death_loc"].copy(),
            cell_piece_id=b["cell_pid"].copy(), seat_dead_arr=b["seat_dead"].astype(bool),
            seat_flag_revealed_arr=b["flag_rev"].astype(bool), turn=int(b["turn"]),
            move_counter=int(b["move_counter"]), moves_since_last_combat=int(b["mslc"]),
            terminated=bool(b["terminated"]), winner_team=None if int(b["winner"]) < 0 else int(b["winner"]),
            draw=bool(b["draw"]),
            move_history=[(int(s), int(d)) for s, d in b["hist"][: int(b["hist_len"])]])
        envs.append(types.SimpleNamespace(state=st))
    return envs


def test_world_push_state_step_and_legal(jq):
    n = 24
    lineups = jq.generate_lineups(40, n)
    games = G.oracle_games_from_lineups(lineups, 2)
    rng = np.random.default_rng(2)
    for ply in range(60):   # advance on the CPU only, then hand the states over
        for g in games:
            ids = g.legal_ids()
            if len(ids) and not g.terminated:
                g.step_id(int(ids[rng.integers(len(ids))]))
    w = jq.GpuWorld(n)
    w.push_state_from_envs(_fake_envs(games))
    dev = G.device_fields(w.state)
    orc = G.oracle_fields(games)
    for k in ("cell", "ptype", "pos", "zero", "move_count", "death_step", "turn", "move_counter", "mslc",
              "seat_dead", "flag_rev", "terminated", "zobrist", "hist_list"):
        G.compare_state({k: dev[k]}, {k: orc[k]}, ctx=f"push_state_from_envs {k}")

    for ply in range(25):
        seats = w.state.field_tensor("turn").cpu().numpy().astype(np.int8)
        offs, vals = w.legal_actions_csr(seats)
        acts = np.full(n, -1, np.int32)
        for i, g in enumerate(games):
            want = g.legal_ids(int(seats[i]))
            assert np.array_equal(vals[offs[i]:offs[i + 1]], want), (ply, i)
            if len(want):
                acts[i] = want[rng.integers(len(want))]
        out = w.step_batch(acts)
        assert set(out) == {"valid", "event", "terminated", "winner_team", "draw", "flag_captured"}
        for i, g in enumerate(games):
            if acts[i] < 0:
                assert not out["valid"][i]
                continue
            rc, o = g.step_id(int(acts[i]))
            assert out["valid"][i] and out["event"][i] == o["event"] and bool(out["flag_captured"][i]) == bool(
                o["flag_captured"]), (ply, i)
        z = w.state.get_field("zobrist")[:, 0]
        assert all(int(z[i]) == int(g.zobrist) for i, g in enumerate(games)), ply
    seats = w.state.field_tensor("turn").cpu().numpy().astype(np.int8)
    m = w.legal_actions_mask(seats)
    assert m.shape == (n, 120, jq.SLOTS_PER_PIECE) and m.dtype == bool
    for i, g in enumerate(games):
        assert np.array_equal(m[i], g.legal_slots(int(seats[i]))), i
    with pytest.raises(ValueError):
        w.legal_actions_csr(np.zeros(n, np.int32))
    with pytest.raises(ValueError):
        w.legal_actions_mask(np.zeros(n, np.int32))
    term = w.pull_termination_state()
    w.push_termination_state(np.ones(n, bool), np.zeros(n, np.int8), np.zeros(n, bool))
    assert w.pull_termination_state()["terminated"].all()
    assert not w.step_batch(np.zeros(n, np.int32))["valid"].any()
    assert term["terminated"].dtype == bool
    w.state.close()


def test_uploaded_beliefs_feed_the_observation(jq):
    """upload_beliefs (gpu_rollout.py:966-981): the belief planes take the
    observer's uploaded value at each teammate / enemy piece's cell (> 0 only),
    bit-exact against the oracle's uploaded-belief observation, for the acting
    seat, every seat, bf16 and GpuWorld.build_observation; u8 is refused and
    clear_beliefs returns to the BeliefTensor planes."""
    from tests.test_gpu import _bf16_rne
    n, show = 10, 2
    ro = jq.GpuRollout(n, show_mode=show)
    ro.reset(21)
    games = G.oracle_games_from_lineups(jq.generate_lineups(21, n), show)
    rng = np.random.default_rng(8)
    for _ in range(25):
        ids, counts = ro.legal_actions_dense(ro.turn_torch().cpu().numpy())
        acts = np.array([ids[i, rng.integers(counts[i])] if counts[i] else -1 for i in range(n)], np.int32)
        ro.step(acts)
        for i, g in enumerate(games):
            if acts[i] >= 0:
                g.step_id(int(acts[i]))
    bel = (rng.random((n, 4, 12, 289), dtype=np.float32) - np.float32(0.25)).astype(np.float32)
    ro.upload_beliefs(bel)
    acting = ro.turn_torch().clone()
    sp, gl = ro.build_acting_seat_observation_torch(acting)
    sp, gl = sp.cpu().numpy(), gl.cpu().numpy()
    for i, g in enumerate(games):
        seat = int(g.turn)
        osp, ogl = g.observe(seat, bel[i, seat])
        assert np.array_equal(sp[i].view(np.uint32), osp.view(np.uint32)), i
        assert np.array_equal(gl[i], ogl), i
    sp4, _ = ro.build_all_seat_observations()
    for i, g in enumerate(games):
        for k in range(4):
            assert np.array_equal(sp4[i, k], g.observe(k, bel[i, k])[0]), (i, k)
    bf, _ = ro.state.observe(acting, fmt="bf16")
    bf = bf.view(torch.int16).cpu().numpy().view(np.uint16)
    for i, g in enumerate(games):
        assert np.array_equal(bf[i], _bf16_rne(g.observe(int(g.turn), bel[i, int(g.turn)])[0])), i
    with pytest.raises(jq.JunqiError):
        ro.state.observe(acting, fmt="u8")
    ro.clear_beliefs()
    sp, _ = ro.build_acting_seat_observation_torch(acting)
    for i, g in enumerate(games):
        assert np.array_equal(sp[i].cpu().numpy(), g.observe(int(g.turn))[0]), i
    with pytest.raises(ValueError):
        ro.upload_beliefs(bel[:, :3])
    ro.close()
    # GpuWorld: beliefs for one call only. The pushed state carries no combat
    # memory (as push_state_from_envs in the reference), so only the belief
    # planes are compared with the oracle; the others equal the world's own
    # observation without uploaded beliefs.
    w = jq.GpuWorld(n, show_mode=show)
    w.push_state_from_envs(_fake_envs(games))
    wsp, _ = w.build_observation(bel, show_mode=show)
    wsp0, _ = w.build_observation(None, show_mode=show)
    planes = list(range(12, 24)) + list(range(27, 51))
    other = [c for c in range(317) if c not in planes]
    for i, g in enumerate(games):
        for k in range(4):
            assert np.array_equal(wsp[i, k][planes], g.observe(k, bel[i, k])[0][planes]), (i, k)
            assert np.array_equal(wsp[i, k][other], wsp0[i, k][other]), (i, k)
    w.state.close()


def test_setup_styles_and_arrangement_pools(jq):
    """Canonical / mixed setup styles and arrangement pools
    (gpu_rollout.py:498-744,1034-1100; tests/test_gpu_rollout.py:165-207)."""
    import json

    from tests import helpers as H

    lu = json.loads((H.GOLDEN / "canonical_lineups.json").read_text())
    n = 16
    print("[styles] canonical reset", flush=True)
    ro = jq.GpuRollout(n, canonical_setup_styles=("T", "D"))
    ro.reset(seed_base=5)
    want = O.styled_setups("canonical", 5, n, ("T", "D"), lu, per_game_seed=True)
    games = [O.Game(w, show_mode=1) for w in want]
    G.compare_state(G.device_fields(ro.batch), G.oracle_fields(games), ctx="canonical reset")
    ro.close()
    with pytest.raises(ValueError, match="unknown canonical setup styles"):
        jq.GpuRollout(2, canonical_setup_styles=("Q",))
    with pytest.raises(ValueError, match="non-empty"):
        jq.GpuRollout(2, mixed_setup=True, mixed_own_team_styles=())

    print("[styles] mixed pool through evaluation", flush=True)
    ro = jq.GpuRollout(n, mixed_setup=True, mixed_own_team_styles=("T",))
    ro.reset(seed_base=0)
    want = O.styled_setups("mixed", 0, n, ("T",), lu, per_game_seed=True)
    assert np.array_equal(ro.batch.get_field("ptype")[:, :120].reshape(n, 120).clip(0), want.clip(0))

    def own_lineups() -> set:
        pt = ro.batch.get_field("ptype")[:, :120].reshape(n, 4, 30).clip(0)   # camps hold -1 on device
        return {tuple(int(v) for v in r) for r in pt[:, 0, :]}

    def restart(seed: int) -> None:
        ro.batch.set_field("terminated", np.ones(n, np.uint8))
        ro.reset_terminated_device(seed=seed)

    restart(1)
    assert own_lineups() == {tuple(lu["T"])}
    ro.upload_fixed_evaluation_setup_pool(seed=20_260_817)
    restart(2)
    assert len(own_lineups()) > 1
    assert ro.restore_training_setup_pool() > 0
    restart(3)
    assert own_lineups() == {tuple(lu["T"])}

    print("[styles] arrangement pool refresh", flush=True)
    base = O.setup_pool(11, 8)
    from junqi_amd.setups import lineups_to_vocab
    vocab = torch.from_numpy(lineups_to_vocab(base).reshape(32, 30))
    samples = torch.nn.functional.one_hot(vocab, 13).float()
    seat_idx = torch.arange(4).repeat(8)
    assert ro.refresh_setup_pool_from_arrangements(samples, seat_idx) == 8
    assert ro.last_setup_pool_unique == len({tuple(r) for r in base})
    ro.reset_from_setup_pool(seed=4)
    pool = ro.batch.pool
    assert np.array_equal(pool, base)
    games = [O.Game(pool[G.reset_pool_index(i, 4, pool.shape[0])], show_mode=1) for i in range(n)]
    G.compare_state(G.device_fields(ro.batch), G.oracle_fields(games), ctx="arrangement pool reset")
    arr = ro.snapshot_env_arrangements()
    assert arr.shape == (n, 4, 30) and arr.dtype == np.int64
    assert np.array_equal(arr, lineups_to_vocab(np.stack([g.buf[0]["ptype"] for g in games])))
    ro.close()
