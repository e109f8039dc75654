"""nc_attn_kvcache_noalloc: the no-allocation variant of nc_attn_kvcache (no counterpart in the
reference; for callers that cannot allocate).  Its split-K scratch is a device array of the
library instead of the caller's workspace, so through the C ABI it must reproduce the existing
entry point bit for bit (same kernels and plans): outputs and the appended caches, on calls in a
row where a later call is smaller, with in-kernel ticket merges (which need the array's counters
back at zero after every call), merge launches and chunk partials.  A call needing more scratch
than NC_NOALLOC_SCRATCH_BYTES is rejected with NC_ERR_SCRATCH_LIMIT and touches nothing.
"""
import ctypes

import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import _attn_call, flash_attn
from tests.helpers import bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


def _case(seed, B, T_new, H, H_kv, D, T_max, seqlens):
    g = gen(seed)
    q = randn((B, T_new, H, D), g, BF16)
    k = randn((B, T_new, H_kv, D), g, BF16)
    v = randn((B, T_new, H_kv, D), g, BF16)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=BF16)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, BF16)
        vc[b, :s] = randn((s, H_kv, D), g, BF16)
    sl = torch.tensor(seqlens, dtype=torch.int32)
    return [t.to(DEV) for t in (q, k, v, kc, vc, sl)]


def _noalloc(q, kc, vc, k, v, sl, window, kps):
    """One nc_attn_kvcache_noalloc call through the C ABI (the test allocates only the output)."""
    a, out, dev, sl = _attn_call("nc_attn_kvcache_noalloc", q, kc, vc, k, v, sl, True, (window, 0), kps)
    status = _ext.lib().nc_attn_kvcache_noalloc(ctypes.byref(a), _ext.stream_handle(dev))
    return status, out


def _agree(seed, B, T_new, H, H_kv, D, T_max, seqlens, window=-1, kps=0):
    q, k, v, kc, vc, sl = _case(seed, B, T_new, H, H_kv, D, T_max, seqlens)
    kc2, vc2 = kc.clone(), vc.clone()
    want = flash_attn.flash_attn_with_kvcache(q, kc2, vc2, k=k, v=v, cache_seqlens=sl, causal=True,
                                              window_size=(window, 0), keys_per_split=kps)
    status, got = _noalloc(q, kc, vc, k, v, sl, window, kps)
    assert status == 0, _ext.lib().nc_strerror(status).decode()
    torch.cuda.synchronize()
    assert torch.equal(bits(got), bits(want)), "output differs from nc_attn_kvcache"
    assert torch.equal(bits(kc), bits(kc2)) and torch.equal(bits(vc), bits(vc2)), "caches differ"


def test_noalloc_equals_workspace_entry_point_on_calls_in_a_row():
    g = gen(900)
    c2 = torch.randint(512, 2049, (32,), generator=g, dtype=torch.int32).tolist()
    # d20 decode layer (B=32, 9 splits per row, merge launch): 1.5 MB of partials in the array
    _agree(901, 32, 1, 10, 10, 128, 2304, c2)
    # smaller: 32 groups of 64-key splits merged in-kernel by tickets, twice (counters back at zero)
    _agree(902, 4, 1, 8, 8, 128, 3000, [2999, 7, 64, 2500], kps=64)
    _agree(903, 4, 1, 8, 8, 128, 3000, [1500, 2998, 1, 640], kps=64)
    # smaller still: GQA chunk rows with 2048-key splits (chunk partials, merge launch), windowed decode
    _agree(904, 3, 128, 16, 4, 128, 6200, [6000, 100, 3000])
    _agree(905, 2, 1, 4, 2, 64, 700, [699, 300], window=100, kps=64)


def test_noalloc_rejects_calls_beyond_its_scratch():
    """16 rows x 128-token chunks, 16/4 heads, 16384-key cache: 136 MB of partials > 64 MiB."""
    B, T_new, H, H_kv, D, T_max = 16, 128, 16, 4, 128, 16384
    q = torch.ones(B, T_new, H, D, dtype=BF16, device=DEV)
    k = torch.ones(B, T_new, H_kv, D, dtype=BF16, device=DEV)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=BF16, device=DEV)
    vc = torch.zeros_like(kc)
    sl = torch.full((B,), 5000, dtype=torch.int32, device=DEV)
    a, _, _, _ = _attn_call("x", q, kc, vc, k, k, sl, True, (-1, 0), 0)
    assert _ext.lib().nc_attn_workspace_bytes(ctypes.byref(a)) > _ext.NC_NOALLOC_SCRATCH_BYTES
    status, _ = _noalloc(q, kc, vc, k, k, sl, -1, 0)
    assert status == _ext.NC_ERR_SCRATCH_LIMIT
    assert "NC_NOALLOC_SCRATCH_BYTES" in _ext.lib().nc_strerror(status).decode()
    torch.cuda.synchronize()
    assert int(kc.count_nonzero()) == 0 and int(vc.count_nonzero()) == 0, "a rejected call launched"
    # and the next call in range still agrees
    _agree(906, 2, 1, 4, 4, 128, 512, [511, 3], kps=64)
