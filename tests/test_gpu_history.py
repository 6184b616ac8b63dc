"""Compact rollout history (GpuRolloutHistory over jq_history_*) on an MI355X.

Games are played with a snapshot of the pre-action state at every step, as the
reference collector does (junqi_rl/training/gpu_collector.py:872); rows chosen
beforehand are then rebuilt from the history and compared bit-exactly with the
oracle's observation, globals and canonical legal mask at that step, for the
acting seat and for other seats (junqi_rl/gpu_rollout.py:164-217).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests import gpu_compare as G  # noqa: E402
from tests.test_gpu import _bf16_rne  # noqa: E402
from tests.test_gpu_api import _canonical_ids  # noqa: E402

ROW_BYTES = 35972


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


def test_history_reconstructs_observations_and_masks(jq):
    n, steps, show = 20, 16, 2
    print(f"[history] n={n} steps={steps} show={show}", flush=True)
    ro = jq.GpuRollout(n, show_mode=show, max_num_moves=400)
    ro.reset(31)
    games = G.oracle_games_from_lineups(jq.generate_lineups(31, n), show, 400)
    hist = ro.create_rollout_history(steps)
    assert hist.history_bytes == steps * n * ROW_BYTES
    rng = np.random.default_rng(4)
    # rows to rebuild: (step, env, seat offset from the acting seat)
    picks = [(int(t), int(i), int(k)) for t, i, k in zip(rng.integers(steps, size=40), rng.integers(n, size=40),
                                                         rng.integers(4, size=40))]
    want = {}
    seats = {}
    for t in range(steps):
        acting = ro.turn_torch().clone()
        hist.snapshot(ro.state, acting, t)
        for (pt, i, k) in picks:
            if pt == t:
                seat = (int(games[i].turn) + k) & 3
                sp, gl = games[i].observe(seat)
                want[(pt, i, k)] = (sp, gl, _canonical_ids(games[i].legal_ids(seat), seat))
                seats[(pt, i, k)] = seat
        acts = np.full(n, -1, np.int32)
        for i, g in enumerate(games):
            ids = g.legal_ids()
            if len(ids) and not g.terminated:
                acts[i] = ids[rng.integers(len(ids))]
        out = ro.step(acts)
        for i, g in enumerate(games):
            if acts[i] >= 0:
                rc, o = g.step_id(int(acts[i]))
                assert rc == 0 and bool(out["valid"][i])
    flat = torch.tensor([t * n + i for (t, i, k) in picks], dtype=torch.int64, device=ro.device)
    obs = torch.tensor([seats[p] for p in picks], dtype=torch.int8, device=ro.device)
    sp, gl, mask = hist.reconstruct(flat, obs, dtype=torch.float32)
    assert sp.shape == (len(picks), 317, 17, 17) and gl.shape == (len(picks), 28) and mask.dtype == torch.bool
    sp, gl, mask = sp.cpu().numpy(), gl.cpu().numpy(), mask.cpu().numpy()
    for b, p in enumerate(picks):
        wsp, wgl, wids = want[p]
        assert np.array_equal(sp[b].view(np.uint32), wsp.view(np.uint32)), (p, "obs")
        assert np.array_equal(gl[b], wgl), (p, "globals")
        wm = np.zeros(16641, bool)
        wm[wids] = True
        assert np.array_equal(mask[b], wm), (p, "mask")
    # bf16 storage dtype: round-to-nearest-even of the f32 observation
    sb, gb, mb = hist.reconstruct(flat, obs, dtype=torch.bfloat16)
    assert sb.dtype == torch.bfloat16 and gb.dtype == torch.bfloat16
    for b, p in enumerate(picks):
        assert np.array_equal(sb[b].view(torch.int16).cpu().numpy().view(np.uint16), _bf16_rne(want[p][0])), p
    assert np.array_equal(mb.cpu().numpy(), mask)
    # a smaller batch after a larger one reuses the scratch rows
    s2, g2, m2 = hist.reconstruct(flat[:3].flip(0), obs[:3].flip(0), dtype=torch.float32)
    for b, p in enumerate(reversed(picks[:3])):
        assert np.array_equal(s2[b].cpu().numpy().view(np.uint32), want[p][0].view(np.uint32)), p
    # rows outside the history rebuild the empty terminated state: no legal action
    bad = torch.tensor([-1, steps * n], dtype=torch.int64, device=ro.device)
    _, _, mbad = hist.reconstruct(bad, torch.zeros(2, dtype=torch.int8, device=ro.device), dtype=torch.float32)
    assert not mbad.any()
    with pytest.raises(ValueError):
        hist.reconstruct(flat[:0], obs[:0], dtype=torch.float32)
    with pytest.raises(ValueError):
        hist.reconstruct(flat, obs[:2], dtype=torch.float32)
    with pytest.raises(IndexError):
        hist.snapshot(ro.state, ro.turn_torch().clone(), steps)
    hist.close()
    ro.close()


def test_history_rejects_a_mismatched_state(jq):
    ro = jq.GpuRollout(8, show_mode=2)
    ro.reset(1)
    hist = jq.GpuRolloutHistory(num_steps=2, num_envs=9, show_mode=2)
    with pytest.raises(jq.JunqiError):
        hist.snapshot(ro.state, torch.zeros(9, dtype=torch.int8, device=ro.device), 0)
    other = jq.GpuRolloutHistory(num_steps=2, num_envs=8, show_mode=0)
    with pytest.raises(jq.JunqiError):
        other.snapshot(ro.state, ro.turn_torch().clone(), 0)
    hist.close()
    other.close()
    ro.close()
