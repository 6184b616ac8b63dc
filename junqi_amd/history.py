"""``GpuRolloutHistory``: compact device rollout history with train-time
observation reconstruction (junqi_rl/gpu_rollout.py:107-217), over the
jq_history_* C ABI.

A PPO rollout snapshots the pre-action state of every env at each step; a
minibatch is rebuilt from the (step, env) rows it samples: observations and
canonical legal masks are recomputed on the device instead of being stored
(35,972 bytes per env-step instead of 366 KB of float32 observations).
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L
from ._lib import check, lib

OBS_CHANNELS = L.OBS_CHANNELS
OBS_GLOBAL_DIMS = L.OBS_GLOBALS
FLAT_ACTION_DIM = L.ACTION_DIM


def _show_value(show_mode) -> int:
    v = int(getattr(show_mode, "value", show_mode))
    if v not in (0, 1, 2):
        raise ValueError(f"show_mode must be BRIGHT(0), DARK(1) or HALF_DARK(2), got {show_mode!r}")
    return v


class GpuRolloutHistory:
    """Compact device history with train-time observation reconstruction."""

    def __init__(self, *, num_steps: int, num_envs: int, show_mode, device_id: int = 0) -> None:
        self.num_steps = int(num_steps)
        self.num_envs = int(num_envs)
        self.show_mode = show_mode
        self.device = torch.device("cuda", int(device_id))
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            check(lib.jq_history_create(C.byref(h), self.num_envs, self.num_steps, _show_value(show_mode),
                                        int(device_id)))
        self._h = h
        self._mask_words = None

    @property
    def history_bytes(self) -> int:
        v = C.c_int64()
        check(lib.jq_history_bytes(self._h, C.byref(v)))
        return int(v.value)

    def snapshot(self, state, acting_seats: torch.Tensor, step: int) -> None:
        """Save the pre-action state of every env as row block `step`
        (``state`` is the rollout's JunqiBatch, GpuRollout.state)."""
        if acting_seats.device.type != "cuda":
            raise ValueError("acting_seats must be a CUDA tensor")
        if acting_seats.dtype != torch.int8:
            acting_seats = acting_seats.to(torch.int8)
        if not acting_seats.is_contiguous():
            acting_seats = acting_seats.contiguous()
        if acting_seats.shape != (self.num_envs,):
            raise ValueError(f"acting_seats must have shape ({self.num_envs},), got {tuple(acting_seats.shape)}")
        if not 0 <= int(step) < self.num_steps:
            raise IndexError(f"history snapshot step {step} out of range [0, {self.num_steps})")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        check(lib.jq_history_snapshot(self._h, state._h, acting_seats.data_ptr(), int(step), stream))

    def reconstruct(self, flat_indices: torch.Tensor, acting_seats: torch.Tensor, *,
                    dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Rebuild one PPO minibatch entirely from device history: rows
        ``flat_indices`` (step * num_envs + env), observed by ``acting_seats``.
        Returns spatial (B,317,17,17) and global (B,28) in ``dtype`` and the
        (B,16641) bool canonical legal mask."""
        if flat_indices.device.type != "cuda" or acting_seats.device.type != "cuda":
            raise ValueError("history indices and seats must be CUDA tensors")
        if flat_indices.dtype != torch.int64:
            flat_indices = flat_indices.to(torch.int64)
        if acting_seats.dtype != torch.int8:
            acting_seats = acting_seats.to(torch.int8)
        flat_indices = flat_indices.contiguous()
        acting_seats = acting_seats.contiguous()
        if flat_indices.ndim != 1 or acting_seats.shape != flat_indices.shape:
            raise ValueError("history indices and seats must be matching 1-D tensors")
        b = int(flat_indices.numel())
        if b <= 0:
            raise ValueError("cannot reconstruct an empty history minibatch")
        dev = flat_indices.device
        fmt, sdt = (L.OBS_BF16, torch.bfloat16) if dtype == torch.bfloat16 else (L.OBS_F32, torch.float32)
        spatial = torch.empty((b, OBS_CHANNELS, 17, 17), dtype=sdt, device=dev)
        glob = torch.empty((b, OBS_GLOBAL_DIMS), dtype=torch.float32, device=dev)
        mask = torch.empty((b, FLAT_ACTION_DIM), dtype=torch.bool, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        check(lib.jq_history_reconstruct(self._h, flat_indices.data_ptr(), acting_seats.data_ptr(), b, fmt,
                                         spatial.data_ptr(), None, glob.data_ptr(), None, mask.data_ptr(), stream))
        if spatial.dtype != dtype:
            spatial = spatial.to(dtype)
        return spatial, glob.to(dtype), mask

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            check(lib.jq_history_destroy(self._h))
            self._h = C.c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
