"""GPU parity of cache_batch_idx (FA3's flash_attn_with_kvcache argument): batch row b reads and
appends cache row idx[b] of a larger cache; cache_seqlens stays indexed by b.

Oracle: kvcache_oracle.flash_attn_with_kvcache(..., cache_batch_idx=idx), pinned by the
permutation identity in test_oracle.py.  Caches are compared bit-exactly as whole tensors (rows
not named by idx must not change); outputs within max rel err 2e-2 of fp32 (1e-4 for fp32 caches).
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, Bc, idx, T_new, H, H_kv, D, T_max, seqlens, dtype):
    g = gen(seed)
    B = len(idx)
    q = randn((B, T_new, H, D), g, dtype)
    k = randn((B, T_new, H_kv, D), g, dtype)
    v = randn((B, T_new, H_kv, D), g, dtype)
    kc = randn((Bc, T_max, H_kv, D), g, dtype)   # every cache row filled: stray reads or writes show
    vc = randn((Bc, T_max, H_kv, D), g, dtype)
    return q, k, v, kc, vc, torch.tensor(seqlens, dtype=torch.int32), torch.tensor(idx, dtype=torch.int32)


@pytest.mark.parametrize("T_new,H,H_kv,D,dtype,kps,window", [
    (1, 8, 8, 128, torch.bfloat16, 0, -1),      # decode, fused append
    (1, 16, 4, 128, torch.bfloat16, 64, -1),    # GQA, many splits (in-kernel merge)
    (1, 4, 4, 64, torch.float32, 64, 100),      # fp32 cache (unpacked decode path), window
    (3, 8, 2, 64, torch.bfloat16, 0, -1),       # short chunk: standalone append + per-query decode
    (40, 8, 2, 128, torch.bfloat16, 0, 50),     # MFMA chunk, fused append, window
    (40, 4, 4, 64, torch.float16, 128, -1),     # MFMA chunk split-K
])
def test_cache_batch_idx_matches_oracle(T_new, H, H_kv, D, dtype, kps, window):
    Bc, idx, seqlens, T_max = 6, [5, 0, 3, 1], [300, 0, 511, 77], 600
    q, k, v, kc, vc, sl, ix = _inputs(500 + T_new + H, Bc, idx, T_new, H, H_kv, D, T_max, seqlens, dtype)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                             causal=True, window_size=(window, 0), cache_batch_idx=ix.to(DEV),
                                             keys_per_split=kps)
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(window, 0),
                                      compute_dtype=torch.float32, cache_batch_idx=ix)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert max_rel_err(out, ref.float()) <= tol
    assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc))


@pytest.mark.parametrize("T_new", [1, 20])
def test_cache_batch_idx_with_fused_prologue(T_new):
    """The fused QK prologue call appends the transformed k into row idx[b]."""
    Bc, idx, seqlens, T_max, H, H_kv, D = 5, [2, 4, 0], [10, 200, 99], 260, 8, 4, 128
    q, k, v, kc, vc, sl, ix = _inputs(520 + T_new, Bc, idx, T_new, H, H_kv, D, T_max, seqlens, torch.bfloat16)
    cos_t, sin_t = orc.rotary_tables(T_max + 8, D, dtype=torch.bfloat16)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache_rope(q.to(DEV), kc_d, vc_d, k.to(DEV), v.to(DEV), sl.to(DEV),
                                                  cos_t.to(DEV), sin_t.to(DEV), cache_batch_idx=ix.to(DEV))
    eps = torch.finfo(torch.bfloat16).eps
    qx = orc.qk_prologue(q.float(), cos_t.float(), sin_t.float(), sl, 1.2, eps).to(torch.bfloat16)
    kx = orc.qk_prologue(k.float(), cos_t.float(), sin_t.float(), sl, 1.2, eps).to(torch.bfloat16)
    ref_kc, ref_vc = kc.clone(), vc.clone()
    ref = orc.flash_attn_with_kvcache(qx, ref_kc, ref_vc, k=kx, v=v, cache_seqlens=sl, causal=True,
                                      compute_dtype=torch.float32, cache_batch_idx=ix)
    assert max_rel_err(out, ref.float()) <= 2e-2
    # rows not in idx untouched; V bit-exact; K within one bf16 ulp (one rounding vs the oracle's)
    for r in (1, 3):
        assert torch.equal(bits(kc_d[r]), bits(kc[r])) and torch.equal(bits(vc_d[r]), bits(vc[r]))
    assert torch.equal(bits(vc_d), bits(ref_vc))
    diff = (kc_d.float().cpu() - ref_kc.float()).abs()
    assert float((diff > 0).float().mean()) <= 0.02


def test_cache_batch_idx_out_of_range_skips_the_row_and_sets_the_flag():
    Bc, T_max, H, D = 4, 64, 4, 64
    q, k, v, kc, vc, sl, _ = _inputs(530, Bc, [2, 0], 1, H, H, D, T_max, [5, 9], torch.bfloat16)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    dev = kc_d.device   # the indexed device the library's error flag is kept for
    _ext.read_and_clear_device_errors(dev)
    ix = torch.tensor([2, 9], dtype=torch.int32)   # row 1 names cache row 9 of 4
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                             causal=True, cache_batch_idx=ix.to(DEV))
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_BATCH_IDX
    # row 0 attends and appends into cache row 2 as usual; nothing else changes
    ref_kc, ref_vc = kc.clone(), vc.clone()
    ref = orc.flash_attn_with_kvcache(q[:1], ref_kc, ref_vc, k=k[:1], v=v[:1], cache_seqlens=sl[:1], causal=True,
                                      compute_dtype=torch.float32, cache_batch_idx=ix[:1])
    assert max_rel_err(out[:1], ref.float()) <= 2e-2
    assert torch.equal(bits(kc_d), bits(ref_kc)) and torch.equal(bits(vc_d), bits(ref_vc))


def test_identity_cache_batch_idx_equals_no_index():
    Bc, T_max, H, D = 3, 128, 8, 128
    q, k, v, kc, vc, sl, _ = _inputs(540, Bc, [0, 1, 2], 1, H, H, D, T_max, [100, 3, 64], torch.bfloat16)
    kc1, vc1, kc2, vc2 = kc.to(DEV), vc.to(DEV), kc.to(DEV), vc.to(DEV)
    ix = torch.arange(3, dtype=torch.int32, device=DEV)
    o1 = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc1, vc1, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                            causal=True, cache_batch_idx=ix)
    o2 = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc2, vc2, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl.to(DEV),
                                            causal=True)
    assert torch.equal(bits(o1), bits(o2))
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))
