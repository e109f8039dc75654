"""Small-M linear layers of the decode step on the HIP kernel (nc_linear).

nanochat runs every projection of a decode step as ``F.linear(x,
W.to(x.dtype))`` on a (B, 1, C) activation (nanochat/gpt.py:45-50, callers
:87-89, :125, :136-138, :469).  With B rows against an (N, K) weight these are
weight-streaming problems; ``linear`` runs them on the library's small-M
kernel, and ``logits_head`` fuses the lm_head with the vocabulary slice, the
fp32 cast and the tanh softcap of gpt.py:468-472.

Only shapes the kernel takes are accepted (``supported``); the caller keeps
F.linear for the others (prefill, M > 64).  There is no torch fallback inside
these functions: without libnc_kv.so they raise.
"""
from __future__ import annotations

import ctypes

import torch

from . import _ext

MAX_M = 64
_DTYPES = (torch.bfloat16, torch.float16)


def supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True if nc_linear takes y = x @ weight.T (x: (..., K), weight: (N, K))."""
    if not (x.is_cuda and weight.is_cuda) or x.device != weight.device:
        return False
    if x.dtype not in _DTYPES or weight.dtype != x.dtype or weight.dim() != 2 or x.dim() < 1:
        return False
    k = weight.shape[1]
    if x.shape[-1] != k or k % 8 != 0:
        return False
    m = x.numel() // k if k else 0
    return 1 <= m <= MAX_M


# Block projections of a decode step go to the kernel only where it measured faster than the
# library GEMM (MI355X, HIP graph replays, bf16, weights streamed from HBM): at most 16 rows and
# K <= 2048, e.g. 16 x 4608 x 1536 in 8.0 vs 9.6 us and 16 x 1280 x 1280 in 4.7 vs 6.3 us.  At 32
# rows the two are level or the library is faster (32 x 5120 x 1280: 10.8 vs 8.7 us), and so it is
# at K >= 5120 (16 x 1280 x 5120: 12.4 vs 9.4 us); tiny weights are launch-bound either way.
PROJ_MAX_M, PROJ_MAX_K, PROJ_MIN_DIM = 16, 2048, 512


def prefer_for_projection(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True if F.linear(x, weight) should run on the kernel: a supported, inference-only
    (no autograd) shape in the region where it beats the library GEMM."""
    if torch.is_grad_enabled() or not supported(x, weight):
        return False
    n, k = weight.shape
    m = x.numel() // k
    return m <= PROJ_MAX_M and PROJ_MIN_DIM <= k <= PROJ_MAX_K and n >= PROJ_MIN_DIM


def _rows(t: torch.Tensor, cols: int) -> torch.Tensor:
    """t as an (rows, cols) matrix with unit column stride, without copying when possible."""
    t2 = t.reshape(-1, cols)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) % 8 != 0) or t2.data_ptr() % 16 != 0:
        t2 = t2.contiguous()
    return t2


def _call(x: torch.Tensor, weight: torch.Tensor, n: int, y_dtype: torch.dtype, softcap: float) -> torch.Tensor:
    if not supported(x, weight):
        raise ValueError(f"nc_linear does not take x {tuple(x.shape)} {x.dtype} @ weight {tuple(weight.shape)} "
                         f"{weight.dtype} (CUDA tensors, bf16/fp16, K % 8 == 0, at most {MAX_M} rows)")
    k = weight.shape[1]
    x2 = _rows(x, k)
    w2 = weight if (weight.stride(-1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0) \
        else weight.contiguous()
    m = x2.shape[0]
    y = torch.empty((m, n), dtype=y_dtype, device=x.device)
    L = _ext.lib()
    a = _ext.LinearArgs()
    a.x, a.w, a.y = x2.data_ptr(), w2.data_ptr(), y.data_ptr()
    a.m, a.n, a.k = m, n, k
    a.x_stride_m, a.w_stride_n, a.y_stride_m = x2.stride(0), w2.stride(0), n
    a.dtype = _ext.DTYPE_CODE[x.dtype]
    a.y_dtype = _ext.DTYPE_CODE[y_dtype]
    a.softcap = softcap
    stream = _ext.stream_handle(x.device)
    need = L.nc_linear_workspace_bytes(m, n, k)
    if need:
        ws = _ext.workspace(x.device, stream, need)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _ext.check(L.nc_linear(ctypes.byref(a), stream), "nc_linear")
    return y.view(*x.shape[:-1], n)


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.linear(x, weight) (no bias) on the small-M kernel: (..., K) x (N, K) -> (..., N), x's dtype."""
    return _call(x, weight, weight.shape[0], x.dtype, 0.0)


def logits_head(x: torch.Tensor, weight: torch.Tensor, vocab_size: int, softcap: float) -> torch.Tensor:
    """gpt.py:468-472 in one kernel: softcap * tanh(F.linear(x, W)[..., :vocab_size].float() / softcap).

    Returns fp32 (..., vocab_size).  Only the first vocab_size rows of W are read.
    """
    if not 0 < vocab_size <= weight.shape[0]:
        raise ValueError(f"vocab_size {vocab_size} outside (0, {weight.shape[0]}]")
    if not softcap > 0:
        raise ValueError("softcap must be > 0")
    return _call(x, weight[:vocab_size], vocab_size, torch.float32, float(softcap))
