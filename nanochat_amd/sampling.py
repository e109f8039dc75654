"""Next-token sampling on the HIP kernel (nc_sample): nanochat/engine.py:141-156 in one launch.

``sample_next_token(logits, rng, temperature, top_k)`` keeps the reference's signature: greedy
(temperature 0) gives torch.argmax's tokens; otherwise one uniform per row is drawn from ``rng``
(``torch.rand``) and the kernel returns the inverse-CDF token of softmax(logits / T) over the
row or over its top_k logits.  The distribution is the reference's; the reference draws from
torch.multinomial's own stream, so a given seed picks different tokens.  ``sample_with_uniforms``
takes the draws from the caller (e.g. a buffer a HIP graph reads).  No torch fallback: without
libnc_kv.so these functions raise.
"""
from __future__ import annotations

import ctypes

import torch

from . import _ext

MAX_TOP_K = 1024


def sample_with_uniforms(logits: torch.Tensor, uniforms: torch.Tensor | None, temperature: float,
                         top_k: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """(B, V) fp32 logits -> (B, 1) int64 token ids; `uniforms` (B,) fp32 in [0, 1) unless greedy."""
    if not logits.is_cuda or logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(-1) != 1:
        raise ValueError("logits must be a (B, V) fp32 CUDA tensor with unit column stride")
    if temperature < 0:
        raise ValueError("temperature must be non-negative")
    B, V = logits.shape
    k = 0 if top_k is None or top_k <= 0 or top_k >= V else int(top_k)
    if k > MAX_TOP_K:
        raise ValueError(f"top_k {top_k} > {MAX_TOP_K} is not supported")
    if temperature > 0:
        if uniforms is None or not uniforms.is_cuda or uniforms.dtype != torch.float32 or uniforms.numel() != B:
            raise ValueError("sampling needs (B,) fp32 CUDA uniforms")
        uniforms = uniforms.contiguous()
    if out is None:
        out = torch.empty((B, 1), dtype=torch.int64, device=logits.device)
    a = _ext.SampleArgs()
    a.logits = logits.data_ptr()
    a.uniforms = uniforms.data_ptr() if temperature > 0 else None
    a.out = out.data_ptr()
    a.error_flag = _ext.error_flag(logits.device).data_ptr()
    a.batch, a.vocab, a.logits_stride = B, V, logits.stride(0)
    a.temperature = float(temperature)
    a.top_k = k
    _ext.check(_ext.lib().nc_sample(ctypes.byref(a), _ext.stream_handle(logits.device)), "nc_sample")
    return out


def sample_next_token(logits: torch.Tensor, rng: torch.Generator, temperature: float = 1.0,
                      top_k: int | None = None) -> torch.Tensor:
    """engine.py:141-156 on the GPU: (B, V) logits -> (B, 1) ids."""
    assert temperature >= 0.0, "temperature must be non-negative"
    u = None
    if temperature > 0:
        u = torch.rand(logits.size(0), generator=rng, device=logits.device, dtype=torch.float32)
    return sample_with_uniforms(logits.float(), u, temperature, top_k)
