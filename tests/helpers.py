"""Shared helpers for the parity tests: seeded inputs, an independent fp64
brute-force attention, and comparison utilities."""
from __future__ import annotations

import math

import numpy as np
import torch


def gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn(shape, g, dtype=torch.float32):
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def brute_attention(q, k_cache, v_cache, seqlens, window):
    """Softmax attention written out key by key in float64 (tiny inputs only).

    q: (B, T, H, D); caches (B, T_max, H_kv, D) already holding the appended
    tokens.  Query i of row b sits at position p = seqlens[b] + i and sees keys
    j <= p with p - j <= window when window >= 0.  Head h reads kv head
    h // (H // H_kv).  Scale 1/sqrt(D).
    """
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    B, T, H, D = q.shape
    H_kv = kc.shape[2]
    G = H // H_kv
    out = np.zeros((B, T, H, D))
    for b in range(B):
        for i in range(T):
            p = int(seqlens[b]) + i
            keys = [j for j in range(p + 1) if window < 0 or p - j <= window]
            for h in range(H):
                hk = h // G
                s = np.array([float(np.dot(q[b, i, h], kc[b, j, hk])) for j in keys]) / math.sqrt(D)
                w = np.exp(s - s.max())
                w /= w.sum()
                acc = np.zeros(D)
                for wj, j in zip(w, keys):
                    acc += wj * vc[b, j, hk]
                out[b, i, h] = acc
    return out


def max_rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    denom = ref.abs().max().item()
    return (got - ref).abs().max().item() / max(denom, 1e-30)


def bits(t: torch.Tensor) -> torch.Tensor:
    """Raw bit pattern of a tensor (for bit-exact comparisons)."""
    t = t.detach().contiguous().cpu()
    view = {2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.view(view)
