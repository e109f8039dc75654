"""GPU parity of the varlen layout (FA3's cu_seqlens_q / max_seqlen_q): packed tokens, row b owning
tokens [cu[b], cu[b+1]) appended at cache_seqlens[b]; rows may hold 0, 1 or many tokens.

Oracle: kvcache_oracle.flash_attn_with_kvcache(..., cu_seqlens_q=cu), pinned in test_oracle.py by
the uniform-length and one-call-per-row identities.  Caches are compared bit-exactly as whole
tensors; outputs within max rel err 2e-2 of fp32 (1e-4 for fp32 caches).
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, lens, seqlens, H, H_kv, D, T_max, dtype, Bc=None):
    g = gen(seed)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    total = int(cu[-1])
    q = randn((total, H, D), g, dtype)
    k = randn((total, H_kv, D), g, dtype)
    v = randn((total, H_kv, D), g, dtype)
    Bc = Bc or len(lens)
    kc = torch.zeros(Bc, T_max, H_kv, D, dtype=dtype)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, dtype)
        vc[b, :s] = randn((s, H_kv, D), g, dtype)
    return q, k, v, kc, vc, torch.tensor(seqlens, dtype=torch.int32), cu


def _check(seed, lens, seqlens, H, H_kv, D, T_max, window=-1, dtype=torch.bfloat16, kps=0, idx=None, Bc=None):
    q, k, v, kc, vc, sl, cu = _inputs(seed, lens, seqlens, H, H_kv, D, T_max, dtype, Bc)
    ix = torch.tensor(idx, dtype=torch.int32) if idx is not None else None
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                             causal=True, window_size=(window, 0), cu_seqlens_q=cu.to(DEV),
                                             max_seqlen_q=max(max(lens), 1), keys_per_split=kps,
                                             cache_batch_idx=ix.to(DEV) if ix is not None else None)
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(window, 0),
                                      compute_dtype=torch.float32, cu_seqlens_q=cu, cache_batch_idx=ix)
    assert out.shape == q.shape
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    if q.shape[0]:
        assert max_rel_err(out, ref.float()) <= tol
    assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc))
    return out


def test_varlen_decode_rows_of_zero_and_one_token():
    """max_seqlen_q = 1: the decode kernel with the fused append; rows of 0 tokens are left alone."""
    _check(600, [1, 0, 1, 1, 0, 1], [100, 50, 0, 700, 3, 1023], 8, 8, 128, 1100)


def test_varlen_decode_many_splits_in_kernel_merge():
    _check(601, [1, 1, 0, 1], [3000, 7, 900, 2500], 16, 4, 128, 3100, kps=64)


def test_varlen_short_rows_per_query_decode():
    """max_seqlen_q below the chunk threshold: standalone append + per-query decode."""
    _check(602, [3, 0, 5, 1, 2], [10, 40, 0, 99, 300], 8, 2, 64, 320, window=30)


@pytest.mark.parametrize("lens,seqlens,H,H_kv,D,window,kps", [
    ([1, 128, 0, 37, 1, 64], [500, 0, 64, 1000, 2, 333], 16, 4, 128, -1, 0),   # C5-like mix on the MFMA kernel
    ([40, 9, 17], [0, 128, 70], 8, 8, 64, 50, 0),                              # windows, D=64
    ([100, 3, 60], [2500, 4000, 10], 16, 2, 128, -1, 128),                     # chunk split-K
])
def test_varlen_mixed_rows_on_the_chunk_kernel(lens, seqlens, H, H_kv, D, window, kps):
    T_max = max(s + n for s, n in zip(seqlens, lens)) + 5
    _check(610 + len(lens) + H, lens, seqlens, H, H_kv, D, T_max, window=window, kps=kps)


def test_varlen_fp32_cache():
    _check(620, [2, 1, 0, 4], [5, 60, 1, 33], 4, 4, 64, 80, dtype=torch.float32)


def test_varlen_with_cache_batch_idx():
    _check(621, [1, 12, 0, 30], [40, 0, 99, 200], 8, 4, 128, 260, idx=[4, 1, 0, 2], Bc=5)


def test_varlen_uniform_rows_equal_the_fixed_length_call_bit_for_bit():
    B, T, T_max, H, H_kv, D = 3, 16, 200, 8, 4, 128
    q, k, v, kc, vc, sl, cu = _inputs(630, [T] * B, [5, 100, 0], H, H_kv, D, T_max, torch.bfloat16)
    kc1, vc1, kc2, vc2 = kc.to(DEV), vc.to(DEV), kc.to(DEV), vc.to(DEV)
    o1 = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc1, vc1, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                            causal=True, cu_seqlens_q=cu.to(DEV), max_seqlen_q=T)
    o2 = flash_attn.flash_attn_with_kvcache(q.reshape(B, T, H, D).to(DEV), kc2, vc2, k=k.reshape(B, T, H_kv, D).to(DEV),
                                            v=v.reshape(B, T, H_kv, D).to(DEV), cache_seqlens=sl.to(DEV), causal=True)
    assert torch.equal(bits(o1), bits(o2.reshape(B * T, H, D)))
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))


@pytest.mark.parametrize("T_max_q", [1, 24])
def test_varlen_with_fused_prologue(T_max_q):
    lens = [1, 0, 1] if T_max_q == 1 else [24, 3, 0, 11]
    seqlens = [17, 5, 200] if T_max_q == 1 else [0, 90, 7, 150]
    H, H_kv, D, T_max = 8, 4, 128, 240
    q, k, v, kc, vc, sl, cu = _inputs(640 + T_max_q, lens, seqlens, H, H_kv, D, T_max, torch.bfloat16)
    cos_t, sin_t = orc.rotary_tables(T_max + 8, D, dtype=torch.bfloat16)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache_rope(q.to(DEV), kc_d, vc_d, k.to(DEV), v.to(DEV), sl.to(DEV),
                                                  cos_t.to(DEV), sin_t.to(DEV), cu_seqlens_q=cu.to(DEV),
                                                  max_seqlen_q=T_max_q)
    eps = torch.finfo(torch.bfloat16).eps
    # token positions: cache_seqlens[b] + t for row b's t-th token
    pos = torch.cat([torch.arange(n, dtype=torch.int32) + int(s) for n, s in zip(lens, seqlens)])
    # each packed token as a row of one token at its own position
    qx = orc.qk_prologue(q.float()[:, None], cos_t.float(), sin_t.float(), pos, 1.2, eps)[:, 0].to(torch.bfloat16)
    kx = orc.qk_prologue(k.float()[:, None], cos_t.float(), sin_t.float(), pos, 1.2, eps)[:, 0].to(torch.bfloat16)
    ref_kc, ref_vc = kc.clone(), vc.clone()
    ref = orc.flash_attn_with_kvcache(qx, ref_kc, ref_vc, k=kx, v=v, cache_seqlens=sl, causal=True,
                                      compute_dtype=torch.float32, cu_seqlens_q=cu)
    assert max_rel_err(out, ref.float()) <= 2e-2
    assert torch.equal(bits(vc_d), bits(ref_vc))
    diff = (kc_d.float().cpu() - ref_kc.float()).abs()
    assert float((diff > 0).float().mean()) <= 0.02


def test_varlen_malformed_rows_are_skipped_and_flagged():
    """A row past total_q or longer than max_seqlen_q is skipped (no reads or writes) and flagged."""
    H, D, T_max = 4, 64, 64
    q, k, v, kc, vc, sl, _ = _inputs(650, [1, 1, 1], [5, 9, 20], H, H, D, T_max, torch.bfloat16)
    cu = torch.tensor([0, 1, 3, 9], dtype=torch.int32)   # row 1 holds 2 > max_seqlen_q tokens; row 2 ends past 3
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    dev = kc_d.device
    _ext.read_and_clear_device_errors(dev)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                             causal=True, cu_seqlens_q=cu.to(DEV), max_seqlen_q=1)
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_QLEN
    ref_kc, ref_vc = kc.clone(), vc.clone()
    ref = orc.flash_attn_with_kvcache(q[:1], ref_kc, ref_vc, k=k[:1], v=v[:1], cache_seqlens=sl[:1], causal=True,
                                      compute_dtype=torch.float32, cu_seqlens_q=torch.tensor([0, 1], dtype=torch.int32))
    assert max_rel_err(out[:1], ref.float()) <= 2e-2
    assert torch.equal(bits(kc_d), bits(ref_kc)) and torch.equal(bits(vc_d), bits(ref_vc))


@pytest.mark.parametrize("kps", [0, 64])
def test_varlen_mixed_batch_splits_single_token_rows_to_the_decode_kernel(kps):
    """Single-token rows next to chunk rows: the decode kernel takes the former and the chunk kernel
    the latter, each with split-K partials in its own workspace region (64-key splits)."""
    lens = [1, 1, 40, 1, 0, 9, 1, 1, 128]
    seqlens = [3000, 17, 2500, 1, 700, 2999, 64, 1500, 800]
    _check(660 + kps, lens, seqlens, 16, 4, 128, 3200, kps=kps)
