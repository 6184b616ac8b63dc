"""Legal-support storage of rollout buffers: dense bool mask rows <-> per-row id
lists (junqi_rl/training/rollout_gpu.py:119-198), on the device through the
jq_mask_count / jq_mask_to_ids / jq_ids_to_mask kernels.

Same arguments, shapes, dtypes and ValueError checks as the reference's
``_dense_mask_to_csr`` and ``_csr_to_dense_selected``; tensors must be on the
GPU (there is no host path).
"""

from __future__ import annotations

import torch

from ._lib import check, lib


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dense_mask_to_csr(mask: torch.Tensor, out_ids: torch.Tensor, out_counts: torch.Tensor) -> None:
    """Write the True columns of each row of ``mask`` (N, FLAT) bool into
    ``out_ids`` (N, K_MAX) int32, in order, zero-padded, and the per-row count
    into ``out_counts`` (N,) int32. Overflow raises before any output changes."""
    if mask.ndim != 2 or mask.dtype != torch.bool or out_ids.ndim != 2:
        raise ValueError("CSR encoding requires a 2-D bool mask and 2-D ids")
    n, k_max = out_ids.shape
    if k_max <= 0 or mask.shape[0] != n or out_counts.shape != (n,):
        raise ValueError("CSR output shapes must be (N, K>0) and (N,)")
    if out_ids.dtype != torch.int32 or out_counts.dtype != torch.int32:
        raise ValueError("CSR ids and counts must be int32")
    if out_ids.device != mask.device or out_counts.device != mask.device:
        raise ValueError("CSR inputs and outputs must share a device")
    if mask.device.type != "cuda":
        raise ValueError("CSR encoding runs on the GPU: mask must be a CUDA tensor")
    mask = mask.contiguous()
    if not out_ids.is_contiguous() or not out_counts.is_contiguous():
        raise ValueError("CSR outputs must be contiguous")
    counts = torch.empty(n, dtype=torch.int32, device=mask.device)
    s = _stream(mask)
    check(lib.jq_mask_count(mask.data_ptr(), n, int(mask.shape[1]), counts.data_ptr(), s))
    if n and bool((counts > k_max).any()):   # synchronises, like the reference's guard
        required = int(counts.max().item())
        raise ValueError(
            f"CSR legal-mask overflow: need {required} entries, capacity {k_max}; "
            "increase rollout.csr_k_max or disable CSR legal-mask storage")
    out_counts.copy_(counts)
    check(lib.jq_mask_to_ids(mask.data_ptr(), n, int(mask.shape[1]), k_max, out_ids.data_ptr(), s))


def csr_to_dense_selected(legal_ids: torch.Tensor, legal_counts: torch.Tensor, idx: torch.Tensor,
                          flat_action_dim: int) -> torch.Tensor:
    """Dense (B, flat_action_dim) bool mask of the transitions ``idx`` (B,)
    int64 from (T*N, K_MAX) int32 id lists and their (T*N,) counts."""
    if legal_ids.ndim != 2 or legal_counts.shape != (legal_ids.shape[0],):
        raise ValueError("legal_ids must be (rows, K_MAX) with legal_counts (rows,)")
    if legal_ids.dtype != torch.int32 or legal_counts.dtype != torch.int32:
        raise ValueError("legal_ids and legal_counts must be int32")
    if legal_ids.device.type != "cuda" or legal_counts.device != legal_ids.device or idx.device != legal_ids.device:
        raise ValueError("legal ids, counts and indices must be CUDA tensors on one device")
    ids = legal_ids.contiguous()
    cnt = legal_counts.contiguous()
    sel = idx.to(torch.int64).contiguous().reshape(-1)
    b = int(sel.numel())
    out = torch.empty((b, int(flat_action_dim)), dtype=torch.bool, device=ids.device)
    check(lib.jq_ids_to_mask(ids.data_ptr(), cnt.data_ptr(), int(ids.shape[0]), int(ids.shape[1]), sel.data_ptr(),
                             b, int(flat_action_dim), out.data_ptr(), _stream(ids)))
    return out
