"""GPU parity of single-token decode on length-balanced pieces.

A single-token call with the library's split size (keys_per_split=0) and a plain cache layout
(no cache_batch_idx, cu_seqlens_q or page table) of at most 256 rows, whose uniform split plan
would give rows longer than num_splits x 256 keys longer splits (the grid cap of about 4096
workgroups binds), cuts every row's key span into pieces of one common size instead: a multiple
of 64 keys, at least 256, chosen on the device from cache_seqlens so that all pieces fit the
grid.  One workgroup per piece; one merge block per (row, kv head, head block) combines that
group's contiguous partial slots.  The cases below are such calls (the plan rule is worked out in
each comment): skewed GQA rows as in C5, more than 64 rows (the prefix sums run in passes of 64
rows), the 256-row maximum, a sliding window, head blocks of 8, fp16 / fp32 caches, calls
without new k/v, two consecutive steps, the fused QK prologue.  257 rows, and cache_batch_idx
calls, keep the uniform split plan (long rows spread over the bounded splits).

Reference: the oracle (nanochat/flash_attention.py:155-177 + :69-102 applied row by row) in
float32 on the CPU from the same seeded inputs.  Tolerances as the other decode parity tests:
bf16/fp16 max rel err <= 2e-2 and allclose(atol=rtol=1e-2) (nanochat
tests/test_attention_fallback.py:39), fp32 1e-4; caches and cache_seqlens bit-exact.
"""
import numpy as np
import pytest
import torch

from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn
from tests.test_gpu_attention import _check
from tests.test_gpu_rope import _run as _run_prologue

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _skewed(B, hi, seed, lo=128):
    """Zipf(1.2) lengths clipped to [lo, hi] (C5's distribution), rows 0 and 1 at 0 and 1 keys."""
    s = np.clip(np.random.RandomState(seed).zipf(1.2, B), lo, hi).astype(int).tolist()
    s[0], s[1] = 0, 1
    return s


def _ragged(B, hi, seed):
    """Uniform lengths in [0, hi] with the tile edges 63, 64, 65 and the maximum hi."""
    s = np.random.RandomState(seed).randint(0, hi + 1, B).tolist()
    s[:4] = [63, 64, 65, hi]
    return s


CASES = {
    # name: (B, H, H_kv, D, T_max, seqlens, window)
    # 48 rows x 4 kv heads = 192 groups: 21 splits (4096 // 192), 21 x 256 < 8192 keys
    "gqa_skewed": (48, 16, 4, 128, 8192, _skewed(48, 8000, 0), -1),
    # 300 groups: 13 splits, 13 x 256 < 4096; 150 rows = 3 passes of the prefix sums
    "mha_150_rows": (150, 2, 2, 128, 4096, _ragged(150, 4094, 1), -1),
    # 512 groups: 8 splits, 8 x 256 < 3000; the 256-row maximum (4 passes)
    "max_rows": (256, 2, 2, 64, 3000, _ragged(256, 2998, 2), -1),
    # 1024 groups: 4 splits, 4 x 256 < the 1025-key window span
    "window": (256, 4, 4, 64, 2048, _ragged(256, 2046, 3), 1024),
    # head blocks of 8 q heads: 100 groups, 40 splits, 40 x 256 < 12288
    "mqa_8_heads": (100, 8, 1, 64, 12288, _skewed(100, 12286, 4, lo=1), -1),
}


@pytest.mark.parametrize("name", list(CASES))
def test_balanced_pieces_match_oracle(name):
    B, H, H_kv, D, T_max, seqlens, window = CASES[name]
    _check(700 + list(CASES).index(name), B, 1, H, H_kv, D, T_max, seqlens, window)


@pytest.mark.parametrize("q_dtype,cache_dtype", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                                 (torch.float32, torch.bfloat16)])
def test_balanced_pieces_dtypes(q_dtype, cache_dtype):
    B, H, H_kv, D, T_max, seqlens, window = CASES["gqa_skewed"]
    _check(710, B, 1, H, H_kv, D, T_max, seqlens, window, q_dtype=q_dtype, cache_dtype=cache_dtype)


def test_balanced_pieces_without_new_kv():
    """k=v=None: the call reads the cache only (keys [0, s_b] of row b)."""
    B, H, H_kv, D, T_max, seqlens, window = CASES["gqa_skewed"]
    _check(720, B, 1, H, H_kv, D, T_max, seqlens, window, with_kv=False)


def test_balanced_pieces_consecutive_steps():
    """Two decode steps on one cache: the second step's pieces (from the advanced cache_seqlens)
    read the token the first one appended; the workspace slots are rewritten in between."""
    B, H, H_kv, D, T_max = 48, 16, 4, 128, 8192
    seqlens = _skewed(B, 8000, 5)
    g = gen(730)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
        vc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
    sl = torch.tensor(seqlens, dtype=torch.int32)
    kc_d, vc_d, sl_d = kc.to(DEV), vc.to(DEV), sl.to(DEV)
    for step in range(2):
        q, k, v = (randn((B, 1, n, D), g, torch.bfloat16) for n in (H, H_kv, H_kv))
        out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV),
                                                 cache_seqlens=sl_d, causal=True, window_size=(-1, 0))
        ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True,
                                          window_size=(-1, 0), compute_dtype=torch.float32)
        err = max_rel_err(out, ref.float())
        assert err <= 2e-2, f"step {step}: max rel err {err:.3e}"
        assert torch.allclose(out.float().cpu(), ref.float(), atol=1e-2, rtol=1e-2)
        assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc)), f"step {step}: caches"
        sl += 1
        sl_d += 1


def test_balanced_pieces_with_fused_prologue():
    """The fused QK prologue (rotary + RMS norm + scale on q and the appended k) on the same
    balanced plan."""
    B, H, H_kv, D, T_max, seqlens, window = CASES["gqa_skewed"]
    _run_prologue(740, B, 1, H, H_kv, D, T_max, seqlens, window)


def test_more_rows_than_the_balanced_maximum_keep_the_split_plan():
    """257 rows (one past the maximum): the uniform split plan, long rows spread over its 7 splits."""
    B, H, H_kv, D, T_max = 257, 2, 2, 64, 3000
    _check(750, B, 1, H, H_kv, D, T_max, _ragged(B, 2998, 6), -1)


def test_cache_batch_idx_calls_keep_the_split_plan():
    """A cache_batch_idx call on the gqa_skewed shape runs the lookup kernels on the uniform split
    plan (rows longer than 21 x 256 keys spread over the 21 splits); the identity index equals
    the plain call's oracle."""
    B, H, H_kv, D, T_max, seqlens, window = CASES["gqa_skewed"]
    g = gen(760)
    q = randn((B, 1, H, D), g, torch.bfloat16)
    k = randn((B, 1, H_kv, D), g, torch.bfloat16)
    v = randn((B, 1, H_kv, D), g, torch.bfloat16)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
        vc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
    sl = torch.tensor(seqlens, dtype=torch.int32)
    idx = torch.arange(B, dtype=torch.int32)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                             causal=True, window_size=(window, 0), cache_batch_idx=idx.to(DEV))
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(window, 0),
                                      compute_dtype=torch.float32)
    err = max_rel_err(out, ref.float())
    assert err <= 2e-2, f"max rel err {err:.3e}"
    assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc))
