"""``GpuRollout``: the device-resident rollout interface of the reference
(junqi_rl/gpu_rollout.py:486-1243), over the MI355X library.

Same class and method names, argument meaning, dtypes, shapes and error types,
so ``junqi_rl/training/gpu_collector.py`` can drive it unchanged. Results
follow ``junqi_core.state.GameState`` semantics; where the reference's CUDA path
diverged from them (full Zobrist hash after device resets, sorted legal ids,
BeliefTensor-exact beliefs updated inside the step) this class follows the
Python rules.

Returned device tensors are views of buffers this object owns, overwritten by
the next call of the same method, as in the reference.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib as L
from .batch import JunqiBatch, generate_pool
from .history import GpuRolloutHistory
from .setups import _check_styles, arrangements_to_pool, generate_styled, lineups_to_vocab

DEFAULT_POOL_SIZE = 10000
OBS_CHANNELS = L.OBS_CHANNELS
FLAT_ACTION_DIM = L.ACTION_DIM
MAX_ACTIONS_PER_ENV = 512
_SHOW_DARK = 1


def _show_value(show_mode) -> int:
    v = int(getattr(show_mode, "value", show_mode))
    if v not in (0, 1, 2):
        raise ValueError(f"show_mode must be BRIGHT(0), DARK(1) or HALF_DARK(2), got {show_mode!r}")
    return v


class GpuRollout:
    """N Junqi games resident on one GPU (junqi_rl/gpu_rollout.py:486)."""

    def __init__(self, num_envs: int, *, show_mode=_SHOW_DARK, device_id: int = 0,
                 canonical_setup_styles: tuple[str, ...] | None = None, mixed_setup: bool = False,
                 mixed_own_team_styles: tuple[str, ...] = ("T",), max_num_moves: int | None = None) -> None:
        if num_envs <= 0:
            raise ValueError(f"num_envs must be positive, got {num_envs}")
        if not torch.cuda.is_available() or torch.cuda.device_count() == 0:
            raise RuntimeError("No GPU found")
        self._canonical_setup_styles = canonical_setup_styles
        self._mixed_setup = bool(mixed_setup)
        self._mixed_own_team_styles = tuple(mixed_own_team_styles)
        if self._mixed_setup and not self._mixed_own_team_styles:
            raise ValueError("mixed_setup=True requires mixed_own_team_styles to be non-empty")
        # setup mode by precedence mixed > canonical > uniform (gpu_rollout.py:560-651)
        if self._mixed_setup:
            self._setup_mode = ("mixed", _check_styles(self._mixed_own_team_styles, "mixed_own_team_styles"))
        elif canonical_setup_styles:
            self._setup_mode = ("canonical", _check_styles(canonical_setup_styles, "canonical setup styles"))
        else:
            self._setup_mode = None
        move_limit = 4000 if max_num_moves is None else max_num_moves
        if move_limit <= 0:
            raise ValueError("max_num_moves must be positive")
        self.num_envs = int(num_envs)
        self.show_mode = show_mode
        self._device_id = int(device_id)
        if self._setup_mode is None:
            self._training_pool = generate_pool(42, DEFAULT_POOL_SIZE)
        else:
            self._training_pool = generate_styled(self._setup_mode[0], 42, DEFAULT_POOL_SIZE, self._setup_mode[1],
                                                  per_game_seed=False)
        self.last_setup_pool_unique = 0
        self._b = JunqiBatch(self.num_envs, show_mode=_show_value(show_mode), max_num_moves=move_limit,
                             device=self._device_id, setup_pool=self._training_pool)
        dev = self._b.device
        self.device = dev
        n = self.num_envs
        self._observer_seats = torch.arange(4, dtype=torch.int8, device=dev).repeat(n, 1).contiguous()
        self._sp1 = self._gl1 = self._sp4 = self._gl4 = None
        self._mask_bool = None
        self._step_out = {
            "terminated": torch.empty(n, dtype=torch.bool, device=dev),
            "rewards": torch.empty(n, dtype=torch.float32, device=dev),
            "event": torch.empty(n, dtype=torch.int8, device=dev),
            "draw": torch.empty(n, dtype=torch.bool, device=dev),
            "winner_team": torch.empty(n, dtype=torch.int8, device=dev),
        }
        self._last_result: dict[str, np.ndarray] | None = None

    # ------------------------------------------------------------ setup pools
    def upload_setup_pool(self, pool: np.ndarray) -> int:
        """Install a (pool_size, 120) int8 setup pool for device resets."""
        pool = np.ascontiguousarray(pool, dtype=np.int8).reshape(-1, 120)
        self._b.upload_setup_pool(pool)
        return int(pool.shape[0])

    def upload_fixed_evaluation_setup_pool(self, *, seed: int, pool_size: int = DEFAULT_POOL_SIZE) -> int:
        """Deterministic uniform setup pool for an evaluation (gpu_rollout.py:654-669)."""
        return self.upload_setup_pool(generate_pool(int(seed), int(pool_size)))

    def restore_training_setup_pool(self) -> int:
        """Re-install the training pool after an evaluation (gpu_rollout.py:671-688)."""
        if self._training_pool is None:
            return 0
        return self.upload_setup_pool(self._training_pool)

    def refresh_setup_pool_from_arrangements(self, samples: torch.Tensor, seat_idx: torch.Tensor, *,
                                             pool_size: int = 0, seed: int = 0) -> int:
        """Install a pool built from arrangement-net samples as the training pool
        (gpu_rollout.py:1034-1081): (n_arr, 30, 13) one-hot samples and their
        (n_arr,) seats, zip or independent pairing. Returns the pool size."""
        pool = arrangements_to_pool(samples, seat_idx, pool_size=int(pool_size), seed=int(seed))
        self.upload_setup_pool(pool)
        self._training_pool = pool
        self.last_setup_pool_unique = int(np.unique(pool, axis=0).shape[0])
        return int(pool.shape[0])

    def snapshot_env_arrangements(self) -> np.ndarray:
        """(N, 4, 30) int64 vocabulary indices of each env's lineup
        (gpu_rollout.py:1083-1100)."""
        return lineups_to_vocab(self._b.get_field("ptype")[:, :120])

    # ------------------------------------------------------------ lifecycle
    def reset(self, seed_base: int = 0) -> None:
        """Fresh games from random.Random(seed_base + i) per env: uniform-random
        setups, or the canonical / mixed style draw (gpu_rollout.py:690-744)."""
        if self._setup_mode is None:
            self._b.reset(int(seed_base))
        else:
            mode, styles = self._setup_mode
            self._b.reset_lineups(generate_styled(mode, int(seed_base), self.num_envs, styles, per_game_seed=True))
        self._last_result = None

    def reset_from_setup_pool(self, seed: int = 0) -> None:
        """Reset every env from the uploaded pool (gpu_rollout.py:746-761)."""
        n = self.num_envs
        self._b.set_termination(np.ones(n, bool), np.full(n, -1, np.int8), np.zeros(n, bool), finalize=False)
        self.reset_terminated_device(seed=int(seed))
        self._last_result = None

    def reset_terminated_device(self, seed: int) -> None:
        """Reset terminated envs from the pool, entry hash(env, seed) % pool_size
        (gpu_rollout.py:1007-1028). Beliefs of a reset env start fresh."""
        self._b.reset_terminated(int(seed))

    # ------------------------------------------------------------ step
    def step(self, action_ids: np.ndarray) -> dict[str, np.ndarray]:
        """World action ids (src_flat*289 + dst_flat) → MoveResultBatch dict on the
        host (gpu_rollout.py:765-778)."""
        action_ids = np.asarray(action_ids)
        if action_ids.shape != (self.num_envs,):
            raise ValueError(f"action_ids shape mismatch: expected ({self.num_envs},), got {action_ids.shape}")
        out = self._b.step(torch.from_numpy(action_ids.astype(np.int32, copy=False)).to(self.device))
        res = {k: out[k].cpu().numpy() for k in ("valid", "event", "terminated", "winner_team", "draw",
                                                  "flag_captured")}
        self._last_result = res
        return res

    def step_device_torch(self, canonical_actions: torch.Tensor, acting_seats: torch.Tensor) -> dict:
        """Compact canonical ids (src_c*129 + dst_c in the acting seat's frame) →
        device dict terminated / rewards / event / draw / winner_team
        (gpu_rollout.py:780-848). Move history and beliefs are updated here."""
        b, o = self._b, self._step_out
        a = canonical_actions.to(device=self.device, dtype=torch.int32).contiguous()
        s = acting_seats.to(device=self.device, dtype=torch.int8).contiguous()
        if a.shape != (self.num_envs,) or s.shape != (self.num_envs,):
            raise ValueError(f"expected ({self.num_envs},) actions and acting seats")
        L.check(L.lib.jq_step(b._h, a.data_ptr(), s.data_ptr(), L.ACT_CANONICAL, None, o["event"].data_ptr(),
                              o["terminated"].data_ptr(), o["winner_team"].data_ptr(), o["draw"].data_ptr(),
                              None, None, o["rewards"].data_ptr(), None, b.stream))
        return dict(o)

    def update_beliefs_device(self, step_result: dict, acting_seats: torch.Tensor) -> None:
        """Beliefs (BeliefTensor semantics, info_model.py:271-429) are updated by
        the step itself, so this is a no-op kept for the collector's call order
        (gpu_rollout.py:1103-1157)."""
        return None

    @property
    def last_result(self) -> dict[str, np.ndarray] | None:
        return self._last_result

    # ------------------------------------------------------------ legal actions
    def _seats_np(self, acting_seats) -> np.ndarray:
        a = np.asarray(acting_seats)
        if a.shape != (self.num_envs,):
            raise ValueError(f"acting_seats: expected shape ({self.num_envs},), got {a.shape}")
        return a.astype(np.int8, copy=False)

    def legal_actions_dense(self, acting_seats: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """(action_ids (N,512) int32, counts (N,) int32); ids ascending in each
        row, unused slots -1 (gpu_rollout.py:854-860)."""
        s = torch.from_numpy(self._seats_np(acting_seats)).to(self.device)
        ids, counts = _dense_from_csr(self._b, s)
        return ids.cpu().numpy(), counts.cpu().numpy()

    def legal_actions_mask(self, acting_seats: np.ndarray) -> np.ndarray:
        """(N, 120, 80) bool per-piece slot mask (gpu_rollout.py:862-869): slot
        layout of legal_action_mask_batch (game_state.cu:1964-2197)."""
        s = torch.from_numpy(self._seats_np(acting_seats)).to(self.device)
        return self._b.legal_slots(s).cpu().numpy()

    def legal_mask_canonical_torch(self, acting_seats: np.ndarray | None = None) -> torch.Tensor:
        """(N, 16641) bool device mask over compact canonical ids
        (gpu_rollout.py:1195-1218)."""
        s = None if acting_seats is None else torch.from_numpy(self._seats_np(acting_seats)).to(self.device)
        return self._canonical_mask(s)

    def legal_mask_canonical_torch_device(self, acting_seats_t: torch.Tensor) -> torch.Tensor:
        """As legal_mask_canonical_torch with device int8 seats (gpu_rollout.py:1220-1238)."""
        return self._canonical_mask(acting_seats_t)

    def _canonical_mask(self, seats: torch.Tensor | None) -> torch.Tensor:
        b = self._b
        if self._mask_bool is None:
            self._mask_bool = torch.empty((self.num_envs, FLAT_ACTION_DIM), dtype=torch.bool, device=self.device)
        s = None if seats is None else seats.to(device=self.device, dtype=torch.int8).contiguous()
        L.check(L.lib.jq_legal(b._h, None if s is None else s.data_ptr(), b.counts.data_ptr(), None, None, 0, None,
                               self._mask_bool.data_ptr(), b.stream))
        return self._mask_bool

    # ------------------------------------------------------------ observations
    def build_acting_seat_observation_torch(self, acting_seats_t: torch.Tensor):
        """(N,317,17,17) f32 and (N,28) f32 device views for one observer per env
        (gpu_rollout.py:927-964)."""
        if self._sp1 is None:
            self._sp1 = torch.empty((self.num_envs, OBS_CHANNELS, 17, 17), dtype=torch.float32, device=self.device)
            self._gl1 = torch.empty((self.num_envs, L.OBS_GLOBALS), dtype=torch.float32, device=self.device)
        s = acting_seats_t.to(device=self.device, dtype=torch.int8).contiguous()
        return self._b.observe(s, fmt="f32", out_spatial=self._sp1, out_global=self._gl1)

    def build_all_seat_observations_torch(self):
        """(N,4,317,17,17) and (N,4,28) f32 device views; slot k observes the seat
        set by set_observer_seats (gpu_rollout.py:888-925)."""
        if self._sp4 is None:
            self._sp4 = torch.empty((self.num_envs, 4, OBS_CHANNELS, 17, 17), dtype=torch.float32,
                                    device=self.device)
            self._gl4 = torch.empty((self.num_envs, 4, L.OBS_GLOBALS), dtype=torch.float32, device=self.device)
        return self._b.observe(self._observer_seats, fmt="f32", all_seats=True, out_spatial=self._sp4,
                               out_global=self._gl4)

    def build_all_seat_observations(self) -> tuple[np.ndarray, np.ndarray]:
        """Host copies of build_all_seat_observations_torch (gpu_rollout.py:875-886)."""
        sp, gl = self.build_all_seat_observations_torch()
        return sp.cpu().numpy(), gl.cpu().numpy()

    def set_observer_seats(self, observer_seats: np.ndarray) -> None:
        """Per-env observer mapping (N,4) int8 (gpu_rollout.py:983-1001)."""
        a = np.asarray(observer_seats)
        if a.shape != (self.num_envs, 4):
            raise ValueError(f"observer_seats shape must be ({self.num_envs}, 4), got {a.shape}")
        if np.any((a < 0) | (a > 3)):
            raise ValueError("observer_seats values must be seats 0..3")
        self._observer_seats = torch.from_numpy(a.astype(np.int8)).to(self.device).contiguous()

    def upload_beliefs(self, beliefs: np.ndarray) -> None:
        """Replace the beliefs the observations read (gpu_rollout.py:966-981):
        (N, 4, 12, 289) float32 world-cell beliefs per (env, observer); the
        belief planes take the observer's value at each teammate / enemy piece's
        cell. Until then (and after ``clear_beliefs``) the device's own
        BeliefTensor beliefs are used."""
        if beliefs.shape != (self.num_envs, 4, 12, 289):
            raise ValueError(f"beliefs shape must be ({self.num_envs}, 4, 12, 289), got {beliefs.shape}")
        if beliefs.dtype != np.float32:
            beliefs = beliefs.astype(np.float32, copy=False)
        self._beliefs = beliefs
        self._b.upload_beliefs(beliefs)

    def clear_beliefs(self) -> None:
        self._beliefs = None
        self._b.clear_beliefs()

    # ------------------------------------------------------------ termination, views
    def read_termination(self) -> dict[str, np.ndarray]:
        """terminated / winner_team / draw on the host (gpu_rollout.py:1003-1005)."""
        return self._b.termination()

    def turn_torch(self) -> torch.Tensor:
        """Zero-copy int8 (N,) view of the acting seats (gpu_rollout.py:1159-1169)."""
        return self._b.field_tensor("turn")

    def terminated_torch(self) -> torch.Tensor:
        return self._b.field_tensor("terminated", torch.bool)

    def winner_team_torch(self) -> torch.Tensor:
        return self._b.field_tensor("winner")

    def draw_torch(self) -> torch.Tensor:
        return self._b.field_tensor("draw", torch.bool)

    @property
    def state(self) -> JunqiBatch:
        """The device game-state batch (the reference's DeviceGameStateBatch)."""
        return self._b

    def create_rollout_history(self, num_steps: int) -> GpuRolloutHistory:
        """Allocate compact pre-action state history for one PPO rollout
        (gpu_rollout.py:579-585)."""
        return GpuRolloutHistory(num_steps=num_steps, num_envs=self.num_envs, show_mode=self.show_mode,
                                 device_id=self._device_id)

    def close(self) -> None:
        self._b.close()

    @property
    def batch(self) -> JunqiBatch:
        """The underlying JunqiBatch (all library entry points)."""
        return self._b


def _dense_from_csr(b: JunqiBatch, seats: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """(N,512) int32 ids (ascending, -1 padded) and (N,) counts from the CSR rows."""
    b.legal(seats, csr=True, mask_words=False)
    counts = b.counts.clone()
    n = b.n
    total = int(b.offsets[-1].item())
    idx = torch.arange(MAX_ACTIONS_PER_ENV, device=b.device).unsqueeze(0)
    take = idx < counts.clamp(max=MAX_ACTIONS_PER_ENV).unsqueeze(1)
    dense = torch.full((n, MAX_ACTIONS_PER_ENV), -1, dtype=torch.int32, device=b.device)
    src = b.offsets[:-1].unsqueeze(1) + idx
    dense[take] = b.values[: max(total, 1)].gather(0, src[take].long().clamp(max=max(total - 1, 0)))
    return dense, counts
