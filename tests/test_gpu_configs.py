"""The workload configurations at their stated sizes, on an MI355X, against the
oracle's OpenMP batch path (every game, not a sample):

* c2: 4,096 games, step + CSR, Philox-uniform actions, games at staggered
  stages with auto-reset: every game's Zobrist hash and legal row (count and
  digest) after every one of 1,024 env-steps (> 2.6 M plies), the whole state
  and every CSR row at the end.
* c3: 16,384 games staggered to plies 0-400 in BRIGHT, DARK and HALF_DARK;
  hash and legal-row streams through the warm-up, then the acting seat's u8
  and bf16 observations of every game bit-exact against the oracle's float32.
* c4: 8,192 engineer-dense positions (3 engineers + <= 6 pieces per seat on
  rail cells, random nine-grid occupancy), all four seats' legal sets.
* c5: 32,768 games, the fused loop (masked-logit sampler -> step -> restart
  -> legal + mask + u8 observation) for 256 recorded env-steps after a
  staggered warm-up: every game's reward, done, hash, action and legal row per
  step equal to the oracle's rollout.

The staggering pauses game i for its first S_i env-steps (its action is -1);
both sides do the same, so games finish and restart at different steps.
"""

from __future__ import annotations

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


def _pow_table(m: int) -> torch.Tensor:
    w, x = [], 1
    for _ in range(m):
        w.append(x)
        x = (x * O.LEGAL_DIGEST_P) & (2**64 - 1)
    return torch.from_numpy(np.array(w, np.uint64).view(np.int64))


def _row_digests(b, pw: torch.Tensor) -> torch.Tensor:
    """Per-env digest of the device CSR rows, sum values[j] * P^j mod 2^64
    (oracle.legal_digest), as int64 bits."""
    n = b.n
    counts = b.counts.to(torch.int64)
    total = int(b.offsets[-1])
    row = torch.repeat_interleave(torch.arange(n, device=b.device), counts)
    j = torch.arange(total, device=b.device) - torch.repeat_interleave(b.offsets[:-1].to(torch.int64), counts)
    v = b.values[:total].to(torch.int64) * pw[j]
    return torch.zeros(n, dtype=torch.int64, device=b.device).index_add_(0, row, v)


def _drive(b, steps, *, sampler, seed, active_from, obs_from=None, obs=None):
    """Device side of O.rollout: per step, sample from the current CSR rows,
    pause games before their start step, apply (fused env-step), record.
    obs_from: from that step on the fused path samples itself and writes the u8
    observation into obs (spatial, aux, glob)."""
    n, dev = b.n, b.device
    pw = _pow_table(4096).to(dev)
    af = torch.from_numpy(active_from.astype(np.int64)).to(dev) if active_from is not None else None
    rec = {k: torch.empty((steps, n), dtype=t, device=dev) for k, t in
           (("reward", torch.float32), ("done", torch.uint8), ("hash", torch.int64), ("actions", torch.int32),
            ("legal_count", torch.int32), ("legal_digest", torch.int64))}
    for k in range(steps):
        if k % 128 == 0:
            print(f"[configs] step {k}", flush=True)
        if obs_from is not None and k >= obs_from:
            sp, aux, gl = obs
            b.env_step(sampler=sampler, sample_seed=seed, ply=k, reset_seed=k, obs_fmt="u8", spatial=sp, aux=aux,
                       glob=gl, terminated=rec["done"][k], reward=rec["reward"][k], hash_out=rec["hash"][k],
                       actions_out=rec["actions"][k])
        else:
            a = b.sample_logits(seed, k) if sampler == "logits" else b.sample_uniform(seed, k)
            if af is not None:
                a = torch.where(af > k, torch.full_like(a, -1), a)
            b.env_step(actions=a, sample_seed=seed, ply=k, reset_seed=k, spatial=None,
                       terminated=rec["done"][k], reward=rec["reward"][k], hash_out=rec["hash"][k],
                       actions_out=rec["actions"][k])
        rec["legal_count"][k] = b.counts
        rec["legal_digest"][k] = _row_digests(b, pw)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in rec.items()}


def _compare_streams(dev: dict, ref: dict, ctx: str) -> None:
    for key, view in (("actions", None), ("done", None), ("reward", None), ("hash", np.uint64),
                      ("legal_count", None), ("legal_digest", np.uint64)):
        d = dev[key] if view is None else dev[key].view(view)
        if not np.array_equal(d, ref[key]):
            k, i = np.argwhere(d != ref[key])[0]
            raise AssertionError(f"{ctx}: {key} differs first at step {k} game {i}: {d[k, i]} vs {ref[key][k, i]}")


def _game(batch, i):
    g = O.Game(None)
    g.buf[0] = batch.games[i]
    return g


def test_c2_step_and_csr_4096(jq):
    n, steps, seed = 4096, 1024, 0x4A51
    print(f"[configs] c2 n={n} steps={steps}", flush=True)
    b = jq.JunqiBatch(n, show_mode=2, pool_size=1024, max_num_moves=4000)
    b.reset(202)
    b.legal()
    start = np.random.default_rng(2).integers(0, 768, n).astype(np.int32)
    dev = _drive(b, steps, sampler="uniform", seed=seed, active_from=start)
    ob = O.Batch(jq.generate_lineups(202, n), show_mode=2)
    ref = O.rollout(ob, b.pool, sampler=0, seed=seed, ply0=0, reset_seed0=0, steps=steps, active_from=start)
    _compare_streams(dev, ref, "c2")
    assert ref["applied"] > 2_500_000 and int(ref["done"].sum()) > 1000
    G.compare_state(G.device_fields(b), G.oracle_fields([_game(ob, i) for i in range(n)]), ctx="c2 end")
    offs, vals = b.legal_csr_numpy()
    for i in range(n):
        assert np.array_equal(vals[offs[i]:offs[i + 1]], _game(ob, i).legal_ids()), i
    b.close()


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


@pytest.mark.parametrize("show_mode", [0, 1, 2])
def test_c3_mixed_stage_observations_16384(jq, show_mode):
    n, warm, seed = 16384, 400, 0x3C3
    print(f"[configs] c3 n={n} show_mode={show_mode}", flush=True)
    b = jq.JunqiBatch(n, show_mode=show_mode, pool_size=2048, max_num_moves=4000)
    b.reset(303 + show_mode)
    b.legal()
    start = (warm - np.random.default_rng(3).integers(0, warm + 1, n)).astype(np.int32)  # plies 0-400
    dev = _drive(b, warm, sampler="uniform", seed=seed, active_from=start)
    ob = O.Batch(jq.generate_lineups(303 + show_mode, n), show_mode=show_mode)
    ref = O.rollout(ob, b.pool, sampler=0, seed=seed, ply0=0, reset_seed0=0, steps=warm, active_from=start)
    _compare_streams(dev, ref, f"c3 warm-up mode {show_mode}")
    mc = b.get_field("move_counter")[:, 0]
    assert mc.min() <= 10 and mc.max() >= 390, (mc.min(), mc.max())
    dec = jq.decode_table()
    sp8 = torch.empty((n, 317, 17, 17), dtype=torch.uint8, device=b.device)
    aux = torch.empty((n, jq._lib.AUX_BYTES), dtype=torch.uint8, device=b.device)
    gl8 = torch.empty((n, 28), dtype=torch.float32, device=b.device)
    for extra in range(2):
        k = warm + extra
        b.env_step(sampler="uniform", sample_seed=seed, ply=k, reset_seed=k, obs_fmt="u8", spatial=sp8, aux=aux,
                   glob=gl8)
        O.rollout(ob, b.pool, sampler=0, seed=seed, ply0=k, reset_seed0=k, steps=1)
        sp16, gl16 = b.observe(fmt="bf16") if extra == 1 else (None, None)
        torch.cuda.synchronize()
        for g0 in range(0, n, 2048):
            g1 = min(n, g0 + 2048)
            osp, ogl = O.batch_observe(ob, g0, g1)
            u8 = sp8[g0:g1].cpu().numpy()
            assert int(u8.max()) < 32, "u8 code outside the decode table"
            got = jq.decode_u8(u8, aux[g0:g1].cpu().numpy())
            assert np.array_equal(got, osp), f"c3 u8 observation, games {g0}-{g1}, ply {k}"
            assert np.array_equal(gl8[g0:g1].cpu().numpy(), ogl)
            if sp16 is not None:
                assert np.array_equal(sp16[g0:g1].view(torch.int16).cpu().numpy().view(np.uint16), _bf16_rne(osp)), \
                    f"c3 bf16 observation, games {g0}-{g1}"
                assert np.array_equal(gl16[g0:g1].cpu().numpy(), ogl)
    b.close()


def test_c4_engineer_positions_8192(jq):
    from tests.test_gpu import _engineer_positions, _import_positions
    positions = _engineer_positions(8192, 44)
    print(f"[configs] c4 n={len(positions)}", flush=True)
    b = jq.JunqiBatch(len(positions), show_mode=2)
    _import_positions(jq, b, positions)
    games = [O.Game.from_pieces(p["pieces"], turn=p["turn"]) for p in positions]
    total = 0
    for seat in range(4):
        acting = torch.full((b.n,), seat, dtype=torch.int8, device=b.device)
        offs, vals = b.legal_csr_numpy(acting)
        for i, g in enumerate(games):
            ids = g.legal_ids(seat)
            assert np.array_equal(vals[offs[i]:offs[i + 1]], ids), (i, seat)
            total += len(ids)
    assert total > 8192 * 4 * 20
    b.close()


def test_c5_rollout_32768(jq):
    n, warm, rec_steps, seed = 32768, 512, 256, 0xC5
    steps = warm + rec_steps
    print(f"[configs] c5 n={n} warm={warm} recorded={rec_steps}", flush=True)
    b = jq.JunqiBatch(n, show_mode=2, pool_size=10000, max_num_moves=4000)
    b.reset(505)
    b.legal()
    start = np.random.default_rng(5).integers(0, warm, n).astype(np.int32)
    dev = b.device
    obs = (torch.empty((n, 317, 17, 17), dtype=torch.uint8, device=dev),
           torch.empty((n, jq._lib.AUX_BYTES), dtype=torch.uint8, device=dev),
           torch.empty((n, 28), dtype=torch.float32, device=dev))
    got = _drive(b, steps, sampler="logits", seed=seed, active_from=start, obs_from=warm, obs=obs)
    ob = O.Batch(jq.generate_lineups(505, n), show_mode=2)
    ref = O.rollout(ob, b.pool, sampler=1, seed=seed, ply0=0, reset_seed0=0, steps=steps, active_from=start)
    _compare_streams(got, ref, "c5")
    window = slice(warm, steps)
    assert int(ref["done"][window].sum()) > 5000, "too few games ended inside the recorded window"
    assert (np.abs(ref["reward"][window]).sum() > 0)
    # the last step's observations: codes valid everywhere, exact on a block of games
    u8 = obs[0]
    assert int(u8.max()) < 32
    osp, ogl = O.batch_observe(ob, 0, 1024)
    dec = jq.decode_table()
    gotsp = jq.decode_u8(u8[:1024].cpu().numpy(), obs[1][:1024].cpu().numpy())
    assert np.array_equal(gotsp, osp)
    assert np.array_equal(obs[2][:1024].cpu().numpy(), ogl)
    b.close()
