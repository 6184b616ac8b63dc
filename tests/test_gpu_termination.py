"""Termination thresholds on the device, both sides of each threshold.

The reference's Q10 draw rules (junqi_core/rules.py:444-445: MAX_NUM_MOVES 4000,
MAX_NUM_MOVES_BETWEEN_ATTACKS 200, applied with >= by _check_victory,
state.py:1721-1724, before the turn advance, which termination skips,
state.py:914-941) and the env's move cap (junqi_rl/env.py:295-305, applied after
the turn advance, game_state.cu:1651-1656) are run from imported positions that
sit one and two plies before each threshold, with the cap far above 4000 where
the rules draw is under test (so the cap cannot stand in for it). After every
ply the whole device state (turn, terminated, draw, winner, counters, Zobrist
hash, ...) and the step results must equal the oracle's; the oracle's clauses
are pinned by the restated reference KATs in test_oracle_kats.py.

Both step paths run: jq_step (k_step) and the fused jq_env_step with given
actions (k_env_step), whose finished games restart from the setup pool.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests import gpu_compare as G  # noqa: E402
from tests.test_gpu import _import_positions  # noqa: E402

SOUTH, WEST, NORTH, EAST = 0, 1, 2, 3
NO_CAP = 2**30
PAIZH, SILING = 12, 5
_QUIET = [(0, PAIZH, 8, 11), (30, PAIZH, 5, 8), (60, PAIZH, 8, 0), (90, PAIZH, 11, 8)]
_COMBAT = [(0, SILING, 6, 11), (30, PAIZH, 6, 10), (60, PAIZH, 8, 0), (90, PAIZH, 11, 8)]
_QUIET_MOVE = (11 * 17 + 8) * 289 + 12 * 17 + 8     # SOUTH (8,11) -> (8,12)
_COMBAT_MOVE = (11 * 17 + 6) * 289 + 10 * 17 + 6    # SOUTH (6,11) x (6,10)


def _cases(cap):
    """(pieces, mc, mslc, first action) around the thresholds that matter for `cap`."""
    if cap == NO_CAP or cap == 4000:
        return [
            (_QUIET, 3999, 0, _QUIET_MOVE),     # rules draw at 4000, turn frozen
            (_QUIET, 3998, 0, _QUIET_MOVE),     # 3999: live; next ply draws
            (_QUIET, 3997, 0, _QUIET_MOVE),     # live for two plies
            (_QUIET, 500, 199, _QUIET_MOVE),    # no-combat draw at 200
            (_QUIET, 500, 198, _QUIET_MOVE),    # 199: live; next quiet ply draws
            (_COMBAT, 500, 199, _COMBAT_MOVE),  # combat resets the counter
            (_COMBAT, 3999, 199, _COMBAT_MOVE),  # combat at move 4000 still draws
            (_QUIET, 3999, 199, _QUIET_MOVE),   # both thresholds at once
        ]
    return [
        (_QUIET, cap - 1, 0, _QUIET_MOVE),      # cap draw after the turn advance
        (_QUIET, cap - 2, 0, _QUIET_MOVE),      # live, then the cap
        (_COMBAT, cap - 1, 5, _COMBAT_MOVE),    # seat death + advance, then the cap
        (_QUIET, cap - 1, 199, _QUIET_MOVE),    # rules draw before the cap: turn frozen
    ]


def _positions(cases):
    return [dict(pieces=p, turn=SOUTH, mc=mc, mslc=ms, dead=[0] * 4, flag=[0] * 4) for p, mc, ms, _ in cases]


def _games(cases, cap):
    return [O.Game.from_pieces(p, turn=SOUTH, move_counter=mc, mslc=ms, max_num_moves=cap)
            for p, mc, ms, _ in cases]


def _next_actions(games):
    acts = np.full(len(games), -1, np.int32)
    for i, g in enumerate(games):
        if not g.terminated:
            ids = g.legal_ids()
            if len(ids):
                acts[i] = ids[0]
    return acts


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


@pytest.mark.parametrize("cap", [NO_CAP, 4000, 600, 3])
def test_thresholds_step(jq, cap):
    print(f"[termination] jq_step cap={cap}", flush=True)
    cases = _cases(cap)
    n = len(cases)
    b = jq.JunqiBatch(n, show_mode=2, max_num_moves=cap)
    _import_positions(jq, b, _positions(cases))
    games = _games(cases, cap)
    G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"cap {cap} import")
    acts = np.array([a for *_, a in cases], np.int32)
    seen_draw = 0
    for ply in range(3):
        out = b.step(torch.from_numpy(acts).to(b.device))
        res = [g.step_id(int(a))[1] if a >= 0 else None for g, a in zip(games, acts)]
        got = {k: v.cpu().numpy() for k, v in out.items()}
        for i, r in enumerate(res):
            if r is None:
                assert not got["valid"][i], (cap, ply, i)
                continue
            assert got["valid"][i], (cap, ply, i)
            assert int(got["event"][i]) == r["event"], (cap, ply, i)
            assert bool(got["terminated"][i]) == bool(r["terminated"]), (cap, ply, i)
            assert bool(got["draw"][i]) == bool(r["draw"]), (cap, ply, i)
            assert int(got["winner_team"][i]) == r["winner"], (cap, ply, i)
            assert int(got["seats_died"][i]) == r["seats_died_mask"], (cap, ply, i)
            assert got["rewards"][i] == 0.0, (cap, ply, i)
            seen_draw += r["draw"]
        G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"cap {cap} ply {ply}")
        acts = _next_actions(games)
    # every case reaches its draw within the three plies, except the combat reset
    expected = {NO_CAP: 7, 4000: 7}.get(cap, 4)
    assert seen_draw == expected, (cap, seen_draw)
    b.close()


@pytest.mark.parametrize("cap", [NO_CAP, 600])
def test_thresholds_fused_env_step(jq, cap):
    """The fused step on the same positions: terminated / reward / hash outputs
    per ply equal the oracle's, finished games restart from the pool (pool pick
    of the reference's reset hash) and live ones match the oracle's state."""
    print(f"[termination] jq_env_step cap={cap}", flush=True)
    cases = _cases(cap)
    n = len(cases)
    b = jq.JunqiBatch(n, show_mode=2, max_num_moves=cap, pool_size=16)
    _import_positions(jq, b, _positions(cases))
    games = _games(cases, cap)
    b.legal()
    dev = b.device
    term = torch.empty(n, dtype=torch.uint8, device=dev)
    rew = torch.empty(n, dtype=torch.float32, device=dev)
    hsh = torch.empty(n, dtype=torch.int64, device=dev)
    aout = torch.empty(n, dtype=torch.int32, device=dev)
    acts = np.array([a for *_, a in cases], np.int32)
    for ply in range(3):
        b.env_step(actions=torch.from_numpy(acts).to(dev), sample_seed=5, ply=ply, reset_seed=100 + ply,
                   spatial=None, terminated=term, reward=rew, hash_out=hsh, actions_out=aout)
        tm, rw, hs = term.cpu().numpy(), rew.cpu().numpy(), hsh.cpu().numpy().view(np.uint64)
        for i, g in enumerate(games):
            if acts[i] >= 0:
                rc, _ = g.step_id(int(acts[i]))
                assert rc == 0
                assert hs[i] == np.uint64(g.zobrist), (cap, ply, i)
            assert bool(tm[i]) == bool(g.terminated), (cap, ply, i)
            assert rw[i] == 0.0, (cap, ply, i)
            if g.terminated:
                games[i] = O.Game(b.pool[G.reset_pool_index(i, 100 + ply, b.pool.shape[0])], show_mode=2,
                                  max_num_moves=cap)
        G.compare_state(G.device_fields(b), G.oracle_fields(games), ctx=f"fused cap {cap} ply {ply}")
        offs = b.offsets.cpu().numpy()
        vals = b.values.cpu().numpy()
        for i, g in enumerate(games):
            assert np.array_equal(vals[offs[i]:offs[i + 1]], g.legal_ids()), (cap, ply, i)
        acts = np.array([g.legal_ids()[0] if len(g.legal_ids()) else -1 for g in games], np.int32)
    b.close()


@pytest.mark.parametrize("device_step", [False, True])
def test_custom_move_limit_is_per_rollout_and_survives_reset(jq, device_step):
    """tests/test_gpu_rollout.py:211-245 through the GpuRollout mirror: a limit of
    one move draws after one step, a limit of three is live after one step and
    draws after three, and both limits hold again after reset_terminated_device."""
    print(f"[termination] GpuRollout move limit device_step={device_step}", flush=True)
    short = jq.GpuRollout(num_envs=2, max_num_moves=1)
    longer = jq.GpuRollout(num_envs=2, max_num_moves=3)
    for world in (short, longer):
        world.reset(seed_base=100)

    def step(world):
        if device_step:
            acting = world.turn_torch().clone()
            mask = world.legal_mask_canonical_torch_device(acting)
            actions = mask.long().argmax(-1).to(torch.int32)
            world.step_device_torch(actions, acting)
        else:
            acting = world.state.copy_to_host()["turn"].reshape(-1)
            ids, counts = world.legal_actions_dense(acting)
            assert (counts > 0).all()
            world.step(ids[:, 0].copy())

    step(short)
    step(longer)
    assert short.read_termination()["draw"].all()
    assert not longer.read_termination()["terminated"].any()
    step(longer)
    step(longer)
    assert longer.read_termination()["draw"].all()
    for world in (short, longer):
        world.reset_terminated_device(seed=103)
        assert not world.read_termination()["terminated"].any()
    step(short)
    step(longer)
    assert short.read_termination()["draw"].all()
    assert not longer.read_termination()["terminated"].any()
    short.close()
    longer.close()
