"""GEMV y = A.x (fp32, and fp16 weights with fp32 accumulation).

Mirrors the reference GEMV application (applications/gemv/src/gemv_k1024_persistent_subwarp.cu):
`mode` "baseline"/"oblivious" is gemv_baseline_kernel (:199-231), "aware" is
gemv_partitioned_kernel (:163-197), "swapped"/"rotated" is its swapped=1 launch (:176).
"""
from __future__ import annotations

import torch

from . import _lib
from ._torch import mode_id, ptr, stream_handle


def workspace(M: int, K: int, dtype: torch.dtype, device="cuda") -> torch.Tensor | None:
    """Zero-filled workspace for the split-row home routing of an M x K matrix, or None when
    that route does not apply to the shape (rows not a whole number >= 2 of 8 KiB chunks).
    Every gemv call leaves it zeroed,
    so it is allocated once and reused."""
    elem = torch.empty((), dtype=dtype).element_size()
    n = int(_lib.lib.xd_gemv_workspace_size(M, K, elem))
    return torch.zeros(n, dtype=torch.uint8, device=device) if n else None


def gemv(A: torch.Tensor, x: torch.Tensor, y: torch.Tensor | None = None, mode="aware",
         stream: torch.cuda.Stream | None = None, home_attr: torch.Tensor | None = None,
         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y[M] (fp32) = A[M,K] . x[K]. A/x are both float32 or both float16. home_attr: the
    xd_home_map of A (domain.home_map(A)); used by the aware/rotated modes only. workspace:
    from gemv.workspace(M, K, A.dtype); without it rows of several 8 KiB chunks fall back to
    XCD-slice placement in the aware/rotated modes."""
    if A.dim() != 2 or x.dim() != 1 or A.shape[1] != x.shape[0]:
        raise ValueError("gemv: expected A[M,K] and x[K]")
    M, K = A.shape
    if y is None:
        y = torch.empty(M, dtype=torch.float32, device=A.device)
    if y.dtype != torch.float32 or y.numel() != M:
        raise ValueError("gemv: y must be float32[M]")
    ws, wsb = (ptr(workspace), workspace.numel() * workspace.element_size()) if workspace is not None else (None, 0)
    if A.dtype == torch.float32 and x.dtype == torch.float32:
        _lib.call("xd_gemv_f32", ptr(A), ptr(x), ptr(y), M, K, mode_id(mode), ptr(home_attr), ws, wsb,
                  stream_handle(stream))
    elif A.dtype == torch.float16 and x.dtype == torch.float16:
        _lib.call("xd_gemv_f16f32", ptr(A), ptr(x), ptr(y), M, K, mode_id(mode), ptr(home_attr), ws, wsb,
                  stream_handle(stream))
    else:
        raise TypeError("gemv: A and x must both be float32 or both float16")
    return y
