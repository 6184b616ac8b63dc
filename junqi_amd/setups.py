"""Setup pools beyond the uniform-random one.

* Canonical and mixed setup styles of ``GpuRollout`` (junqi_rl/gpu_rollout.py:
  278-382, 498-560, 701-728): the four canonical opening lineups of
  junqi_core/setup_canonical.py ("T", "D", "G", "F"), drawn with
  ``random.Random.choice`` and generated on the host by the library
  (``jq_generate_styled``), bit-identical to the reference's CPython streams.
* Arrangement-net samples to a setup pool and back
  (junqi_rl/arrangement/pool_upload.py): one-hot (n, 30, 13) samples with a
  seat per sample become (P, 120) int8 pools with the reference's zip and
  independent pairing; a batch's current lineups read back as vocabulary
  indices.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib as L
from ._lib import check, lib

CANONICAL_STYLES = ("T", "D", "G", "F")
ARRANGEMENT_SIZE = 30
N_PIECE_TYPE_WITH_NONE = 13
# vocabulary index -> PieceType value: NONE, then the placeable types JUNQI..GONGB
# (junqi_rl/networks/arrangement_net.py:61-75; rules.py:110-125)
VOCAB_IDX_TO_PIECE_TYPE_VALUE = (0,) + tuple(range(2, 14))


def _check_styles(styles, what: str) -> tuple[str, ...]:
    styles = tuple(styles)
    unknown = [s for s in styles if s not in CANONICAL_STYLES]
    if unknown:
        raise ValueError(f"unknown {what} {unknown}; valid: {sorted(CANONICAL_STYLES)}")
    if not styles:
        raise ValueError(f"{what} must be non-empty")
    return styles


def generate_styled(mode: str, seed: int, count: int, styles, *, per_game_seed: bool) -> np.ndarray:
    """(count, 120) int8 setups. mode "canonical": all four seats share one
    style's lineup; "mixed": seats 0 and 2 share it, seats 1 and 3 draw
    uniform-random lineups. per_game_seed: setup i comes from
    random.Random(seed + i) (GpuRollout.reset); else one random.Random(seed)
    stream feeds every setup (the pool builders)."""
    code = {"canonical": L.SETUP_CANONICAL, "mixed": L.SETUP_MIXED}[mode]
    styles = _check_styles(styles, "setup styles")
    out = np.zeros((int(count), 120), dtype=np.int8)
    letters = "".join(styles).encode()
    check(lib.jq_generate_styled(code, int(seed), int(count), int(bool(per_game_seed)), letters, len(styles),
                                 out.ctypes.data))
    return out


def canonical_lineup(style: str) -> np.ndarray:
    """The 30 seat-local piece types of one canonical style (0 in the camps)."""
    return generate_styled("canonical", 0, 1, (style,), per_game_seed=False)[0, :30].copy()


def arrangements_to_pool(samples: torch.Tensor, seat_idx: torch.Tensor, *, pool_size: int = 0,
                         seed: int = 0) -> np.ndarray:
    """(n_arr, 30, 13) one-hot samples and their (n_arr,) seats -> (P, 120) int8
    pool (pool_upload.py:62-150). Zip pairing: row k takes the k-th sample of
    every seat, P = the fewest samples of any seat. pool_size > 0 keeps that
    prefix and fills up to max(pool_size, P) rows with one independently drawn
    sample per seat from numpy.random.default_rng(seed)."""
    if samples.ndim != 3 or samples.size(1) != ARRANGEMENT_SIZE or samples.size(2) != N_PIECE_TYPE_WITH_NONE:
        raise ValueError(f"samples must be (n_arr, {ARRANGEMENT_SIZE}, {N_PIECE_TYPE_WITH_NONE}), "
                         f"got {tuple(samples.shape)}")
    if seat_idx.shape != (samples.size(0),):
        raise ValueError(f"seat_idx shape {seat_idx.shape} must match samples.size(0)")
    if int(pool_size) < 0:
        raise ValueError(f"pool_size must be >= 0, got {pool_size}")
    vocab = samples.argmax(dim=-1).to("cpu").numpy().astype(np.int64)
    types = np.asarray(VOCAB_IDX_TO_PIECE_TYPE_VALUE, dtype=np.int8)[vocab]
    seats = seat_idx.cpu().numpy().astype(np.int64)
    per_seat = [np.nonzero(seats == s)[0] for s in range(4)]
    zip_size = min(len(ids) for ids in per_seat)
    if zip_size == 0:
        raise ValueError("Cannot build pool: at least one seat has zero arrangement samples. "
                         "Call generate_arrangements with seats covering all 4 indices.")
    target = zip_size if int(pool_size) <= 0 else max(int(pool_size), zip_size)
    pool = np.zeros((target, 120), dtype=np.int8)
    for s in range(4):
        pool[:zip_size, 30 * s:30 * (s + 1)] = types[per_seat[s][:zip_size]]
    if target > zip_size:
        rng = np.random.default_rng(int(seed))
        extra = target - zip_size
        for s in range(4):
            ids = per_seat[s]
            pool[zip_size:, 30 * s:30 * (s + 1)] = types[ids[rng.integers(0, len(ids), size=extra)]]
    return pool


def lineups_to_vocab(ptype: np.ndarray) -> np.ndarray:
    """(N, 120) piece types per pid -> (N, 4, 30) int64 vocabulary indices
    (pool_upload.py:158-203); values outside 0..13 read as NONE."""
    t = np.asarray(ptype, dtype=np.int64).reshape(-1, 4, 30)
    inv = np.zeros(14, dtype=np.int64)
    for idx, v in enumerate(VOCAB_IDX_TO_PIECE_TYPE_VALUE):
        inv[v] = idx
    t = np.where((t >= 0) & (t < 14), t, 0)
    return inv[t]
