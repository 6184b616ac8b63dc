"""The env-step at its full benchmark size (32,768 games, u8 observation), on an
MI355X: properties that hold at any size checked over every game, and exact
parity with the oracle on a sample of games tracked through every ply.

Properties over all games, every ply: offsets are the exclusive scan of counts,
each count is the popcount of the env's canonical mask words, every CSR row is
strictly ascending, every sampled action is the Philox pick from the env's
previous CSR row, every u8 code is a valid decode-table index. After the last
ply: no env is left terminated (finished games restart from the pool), the
incrementally kept Zobrist hash equals a full recompute for every game, and a
second batch run from the same seeds reproduces the outputs byte for byte.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests import gpu_compare as G  # noqa: E402

N = 32768
CAP = 60          # move cap: every game ends and restarts from the pool once
PLIES = 70
SAMPLE = 48


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


def _run(jq, plies, sample, check):
    """Step a full-size batch `plies` times; with `check`, verify the per-ply
    properties over all games and track `sample` games with the oracle.
    Returns the batch and a digest of every ply's outputs."""
    b = jq.JunqiBatch(N, show_mode=2, pool_size=512, max_num_moves=CAP)
    b.reset(3)
    b.legal()
    dev = b.device
    sp = torch.empty((N, 317, 17, 17), dtype=torch.uint8, device=dev)
    aux = torch.empty((N, jq._lib.AUX_BYTES), dtype=torch.uint8, device=dev)
    gl = torch.empty((N, 28), dtype=torch.float32, device=dev)
    term = torch.empty(N, dtype=torch.uint8, device=dev)
    rew = torch.empty(N, dtype=torch.float32, device=dev)
    acts = torch.empty(N, dtype=torch.int32, device=dev)
    bitcount = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int32, device=dev)
    games = G.oracle_games_from_lineups(jq.generate_lineups(3, N)[sample], 2, CAP) if check else None
    dec = jq.decode_table()
    tables = O.tables()
    digest = []
    idx = torch.as_tensor(sample, device=dev)
    sample = [int(i) for i in sample]
    for ply in range(plies):
        offs = b.offsets.cpu().numpy()
        vals = b.values.cpu().numpy()
        counts = b.counts.cpu().numpy()
        b.env_step(sample_seed=11, ply=ply, reset_seed=ply, obs_fmt="u8", spatial=sp, aux=aux, glob=gl,
                   terminated=term, reward=rew, actions_out=acts)
        torch.cuda.synchronize()
        digest.append(torch.stack([b.counts.sum().long(), b.values[: int(b.offsets[-1])].long().sum(),
                                   sp.view(N, -1)[:, ::97].long().sum(), acts.long().sum(),
                                   b.mask_words.long().sum()]).cpu().numpy())
        if not check:
            continue
        # every game: the pick is the Philox-chosen entry of the previous row
        a = acts.cpu().numpy()
        u = G.philox_first_word_np(np.arange(N), ply, 0, 0, 11, 0)
        pick = ((u * counts.astype(np.uint64)) >> np.uint64(32)).astype(np.int64)
        want = np.where(counts > 0, vals[np.minimum(offs[:-1] + pick, max(len(vals) - 1, 0))], -1)
        assert np.array_equal(a, want), ply
        # every game: scan, count / mask agreement, sorted rows, code range
        c = b.counts.long()
        o = b.offsets.long()
        assert int(o[0]) == 0 and torch.equal(o[1:] - o[:-1], c), ply
        pop = bitcount[b.mask_words.view(torch.uint8).long()].view(N, -1).sum(1)
        assert torch.equal(pop.long(), c), ply
        v = b.values[: int(o[-1])].long()
        starts = torch.zeros(int(o[-1]), dtype=torch.bool, device=dev)
        starts[o[:-1][c > 0]] = True
        assert bool(((v[1:] > v[:-1]) | starts[1:]).all()), ply
        assert int(sp.max()) < 17, ply
        # sampled games: oracle stepped with the same actions, restarted alike
        tm = term.cpu().numpy()
        for j, i in enumerate(sample):
            if a[i] >= 0:
                games[j].step_id(int(a[i]))
            assert bool(tm[i]) == bool(games[j].terminated), (ply, i)
            if games[j].terminated:
                games[j] = O.Game(b.pool[G.reset_pool_index(i, ply, b.pool.shape[0])], show_mode=2,
                                  max_num_moves=CAP)
        offs = b.offsets.cpu().numpy()
        vals = b.values.cpu().numpy()
        mw = b.mask_words[idx].cpu().numpy()
        u8 = sp[idx].cpu().numpy()
        ax = aux[idx].cpu().numpy()
        g2 = gl[idx].cpu().numpy()
        for j, i in enumerate(sample):
            g = games[j]
            ids = g.legal_ids()
            assert np.array_equal(vals[offs[i]:offs[i + 1]], ids), (ply, i)
            assert np.array_equal(mw[j], G.canonical_mask_words(ids, int(g.turn), tables)), (ply, i)
            osp, ogl = g.observe(int(g.turn))
            d = jq.decode_u8(u8[j], ax[j])
            assert np.array_equal(d.view(np.uint32), osp.view(np.uint32)), (ply, i)
            assert np.array_equal(g2[j], ogl), (ply, i)
    return b, games, np.stack(digest)


def test_full_size_env_step(jq):
    rng = np.random.default_rng(7)
    sample = np.unique(np.concatenate([[0, 1, N // 2, N - 2, N - 1],
                                       rng.choice(np.arange(2, N - 2), SAMPLE - 5, replace=False)]))
    print(f"[full] n={N} plies={PLIES} sample={len(sample)}", flush=True)
    b, games, digest = _run(jq, PLIES, sample, check=True)
    dev = G.device_fields(b)
    sub = {k: (v[sample] if k != "hist_list" else [v[i] for i in sample]) for k, v in dev.items()}
    G.compare_state(sub, G.oracle_fields(games), ctx="full size, final")
    assert not dev["terminated"].any()
    z = dev["zobrist"].copy()
    b.rehash()
    assert np.array_equal(b.get_field("zobrist")[:, 0], z)
    b.close()
    print("[full] replay from the same seeds", flush=True)
    b2, _, digest2 = _run(jq, 12, sample, check=False)
    assert np.array_equal(digest[:12], digest2)
    b2.close()
