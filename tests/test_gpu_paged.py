"""GPU parity of the paged KV cache (FA3's page_table argument): caches are (num_blocks, P, H_kv, D)
blocks and position j of row b is slot j % P of block page_table[b, j // P].

Oracle: kvcache_oracle.flash_attn_with_kvcache(..., page_table=) (the call on the rows the table
assembles, written back block by block), pinned by the block-shuffle identity in test_oracle.py.
The whole block pool is compared bit-exactly, so stray writes into spare blocks or other rows'
blocks fail; outputs within max rel err 2e-2 of fp32 (1e-4 for fp32 caches).
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _paged_inputs(seed, B, T_new, H, H_kv, D, P, nb, seqlens, dtype, spare=3):
    g = gen(seed)
    q = randn((B, T_new, H, D), g, dtype)
    k = randn((B, T_new, H_kv, D), g, dtype)
    v = randn((B, T_new, H_kv, D), g, dtype)
    n_blocks = B * nb + spare
    kp = randn((n_blocks, P, H_kv, D), g, dtype)      # every block filled: stray reads or writes show
    vp = randn((n_blocks, P, H_kv, D), g, dtype)
    table = torch.randperm(n_blocks, generator=g)[:B * nb].view(B, nb).to(torch.int32)
    return q, k, v, kp, vp, torch.tensor(seqlens, dtype=torch.int32), table


@pytest.mark.parametrize("T_new,H,H_kv,D,P,dtype,kps,window", [
    (1, 8, 8, 128, 64, torch.bfloat16, 0, -1),      # decode, fused append
    (1, 16, 4, 128, 16, torch.bfloat16, 64, -1),    # GQA, many splits, pages smaller than a split
    (1, 4, 4, 64, 256, torch.float32, 64, 100),     # fp32 cache, window, pages larger than a split
    (3, 8, 2, 64, 32, torch.bfloat16, 0, -1),       # short chunk: standalone append + per-query decode
    (40, 8, 2, 128, 64, torch.bfloat16, 0, 50),     # MFMA chunk, fused append, window
    (40, 4, 4, 64, 16, torch.float16, 128, -1),     # MFMA chunk split-K, 16-token pages (tiles span pages)
])
def test_paged_cache_matches_oracle(T_new, H, H_kv, D, P, dtype, kps, window):
    B, nb = 4, -(-640 // P)   # at least 640 logical positions per row
    seqlens = [300, 0, 600 - T_new, 77]
    q, k, v, kp, vp, sl, table = _paged_inputs(600 + T_new + P, B, T_new, H, H_kv, D, P, nb, seqlens, dtype)
    kp_d, vp_d = kp.to(DEV), vp.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kp_d, vp_d, k=k.to(DEV), v=v.to(DEV),
                                             cache_seqlens=sl.to(DEV), causal=True, window_size=(window, 0),
                                             page_table=table.to(DEV), keys_per_split=kps)
    ref = orc.flash_attn_with_kvcache(q, kp, vp, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(window, 0),
                                      compute_dtype=torch.float32, page_table=table)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert max_rel_err(out, ref.float()) <= tol
    assert torch.equal(bits(kp_d), bits(kp)) and torch.equal(bits(vp_d), bits(vp))


def test_paged_without_append_and_with_varlen():
    """No k/v (attention over the paged cache only), then a varlen batch (rows of 0, 1, 12 tokens)."""
    B, H, H_kv, D, P, nb = 3, 8, 4, 128, 32, 12
    q, _, _, kp, vp, sl, table = _paged_inputs(640, B, 1, H, H_kv, D, P, nb, [100, 5, 380], torch.bfloat16)
    kp_d, vp_d = kp.to(DEV), vp.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kp_d, vp_d, cache_seqlens=sl.to(DEV), causal=True,
                                             page_table=table.to(DEV))
    ref = orc.flash_attn_with_kvcache(q, kp, vp, cache_seqlens=sl, causal=True, compute_dtype=torch.float32,
                                      page_table=table)
    assert max_rel_err(out, ref.float()) <= 2e-2
    assert torch.equal(bits(kp_d), bits(kp))
    lens = [0, 1, 12]
    cu = torch.tensor([0, 0, 1, 13], dtype=torch.int32)
    sl = torch.tensor([100, 5, 360], dtype=torch.int32)   # 360 + 12 new tokens within the 384 positions
    g = gen(641)
    qv = randn((13, H, D), g, torch.bfloat16)
    kv = randn((13, H_kv, D), g, torch.bfloat16)
    vv = randn((13, H_kv, D), g, torch.bfloat16)
    out = flash_attn.flash_attn_with_kvcache(qv.to(DEV), kp_d, vp_d, k=kv.to(DEV), v=vv.to(DEV),
                                             cache_seqlens=sl.to(DEV), causal=True, cu_seqlens_q=cu.to(DEV),
                                             max_seqlen_q=max(lens), page_table=table.to(DEV))
    ref = orc.flash_attn_with_kvcache(qv, kp, vp, k=kv, v=vv, cache_seqlens=sl, causal=True,
                                      compute_dtype=torch.float32, cu_seqlens_q=cu, page_table=table)
    assert max_rel_err(out, ref.float()) <= 2e-2
    assert torch.equal(bits(kp_d), bits(kp)) and torch.equal(bits(vp_d), bits(vp))


@pytest.mark.parametrize("T_new", [1, 20])
def test_paged_with_fused_prologue(T_new):
    """The fused QK prologue call appends the transformed k into the row's pages."""
    B, H, H_kv, D, P, nb = 3, 8, 4, 128, 64, 5
    q, k, v, kp, vp, sl, table = _paged_inputs(650 + T_new, B, T_new, H, H_kv, D, P, nb, [10, 200, 99],
                                               torch.bfloat16)
    cos_t, sin_t = orc.rotary_tables(nb * P + 8, D, dtype=torch.bfloat16)
    kp_d, vp_d = kp.to(DEV), vp.to(DEV)
    out = flash_attn.flash_attn_with_kvcache_rope(q.to(DEV), kp_d, vp_d, k.to(DEV), v.to(DEV), sl.to(DEV),
                                                  cos_t.to(DEV), sin_t.to(DEV), page_table=table.to(DEV))
    eps = torch.finfo(torch.bfloat16).eps
    qx = orc.qk_prologue(q.float(), cos_t.float(), sin_t.float(), sl, 1.2, eps).to(torch.bfloat16)
    kx = orc.qk_prologue(k.float(), cos_t.float(), sin_t.float(), sl, 1.2, eps).to(torch.bfloat16)
    ref_kp, ref_vp = kp.clone(), vp.clone()
    ref = orc.flash_attn_with_kvcache(qx, ref_kp, ref_vp, k=kx, v=v, cache_seqlens=sl, causal=True,
                                      compute_dtype=torch.float32, page_table=table)
    assert max_rel_err(out, ref.float()) <= 2e-2
    assert torch.equal(bits(vp_d), bits(ref_vp))
    diff = (kp_d.float().cpu() - ref_kp.float()).abs()   # K within one bf16 ulp (one rounding vs several)
    assert float((diff > 0).float().mean()) <= 0.02


def test_paged_identity_table_equals_the_dense_cache():
    """Blocks laid out in order (table = arange) are the dense cache: same bits as the plain call."""
    B, T_max, H, D, P = 3, 256, 8, 128, 64
    g = gen(660)
    q = randn((B, 1, H, D), g, torch.bfloat16).to(DEV)
    k = randn((B, 1, H, D), g, torch.bfloat16).to(DEV)
    v = randn((B, 1, H, D), g, torch.bfloat16).to(DEV)
    kc = randn((B, T_max, H, D), g, torch.bfloat16).to(DEV)
    vc = randn((B, T_max, H, D), g, torch.bfloat16).to(DEV)
    sl = torch.tensor([100, 3, 200], dtype=torch.int32, device=DEV)
    kc2, vc2 = kc.clone(), vc.clone()
    o1 = flash_attn.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True)
    table = torch.arange(B * T_max // P, dtype=torch.int32, device=DEV).view(B, T_max // P)
    o2 = flash_attn.flash_attn_with_kvcache(q, kc2.view(-1, P, H, D), vc2.view(-1, P, H, D), k=k, v=v,
                                            cache_seqlens=sl, causal=True, page_table=table)
    assert torch.equal(bits(o1), bits(o2))
    assert torch.equal(bits(kc), bits(kc2)) and torch.equal(bits(vc), bits(vc2))


@pytest.mark.parametrize("T_new", [1, 3, 40])
def test_page_index_outside_the_pool_is_never_dereferenced(T_new):
    """A table entry outside [0, num_blocks) sets NC_DEVERR_PAGE; rows with valid tables are unaffected
    and no block changes except the valid rows' appends."""
    B, H, H_kv, D, P, nb = 2, 8, 2, 128, 32, 4
    q, k, v, kp, vp, sl, table = _paged_inputs(670 + T_new, B, T_new, H, H_kv, D, P, nb, [20, 40], torch.bfloat16)
    bad = table.clone()
    bad[1, 0] = kp.shape[0] + 7        # row 1's first block: past the pool
    bad[1, 2] = -1
    kp_d, vp_d = kp.to(DEV), vp.to(DEV)
    dev = kp_d.device
    _ext.read_and_clear_device_errors(dev)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kp_d, vp_d, k=k.to(DEV), v=v.to(DEV),
                                             cache_seqlens=sl.to(DEV), causal=True, page_table=bad.to(DEV))
    torch.cuda.synchronize()
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_PAGE
    ref_kp, ref_vp = kp.clone(), vp.clone()
    ref = orc.flash_attn_with_kvcache(q[:1], ref_kp, ref_vp, k=k[:1], v=v[:1], cache_seqlens=sl[:1], causal=True,
                                      compute_dtype=torch.float32, page_table=table[:1])
    assert max_rel_err(out[:1], ref.float()) <= 2e-2
    # row 1 appends positions 40.. : those in its valid block 1 (slots 8..31) hold its k/v; those in the
    # bad block 2 are not stored; every other slot is as the oracle left it after row 0's call
    blk1 = int(table[1, 1])
    mask = torch.ones(kp.shape[:2], dtype=torch.bool)
    for t in range(T_new):
        j = 40 + t
        if j // P == 1:
            mask[blk1, j % P] = False
            assert torch.equal(bits(kp_d[blk1, j % P].cpu()), bits(k[1, t]))
            assert torch.equal(bits(vp_d[blk1, j % P].cpu()), bits(v[1, t]))
    assert torch.equal(bits(kp_d.cpu()[mask]), bits(ref_kp[mask]))
    assert torch.equal(bits(vp_d.cpu()[mask]), bits(ref_vp[mask]))


def test_page_table_rejections():
    B, H, D, P = 2, 4, 64, 32
    q = torch.zeros(B, 1, H, D, dtype=torch.bfloat16, device=DEV)
    kp = torch.zeros(8, P, H, D, dtype=torch.bfloat16, device=DEV)
    sl = torch.zeros(B, dtype=torch.int32, device=DEV)
    table = torch.zeros(B, 2, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):   # with cache_batch_idx
        flash_attn.flash_attn_with_kvcache(q, kp, kp, cache_seqlens=sl, page_table=table,
                                           cache_batch_idx=torch.zeros(B, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError):   # page size not a power of two
        flash_attn.flash_attn_with_kvcache(q, kp[:, :24], kp[:, :24], cache_seqlens=sl, page_table=table)
    with pytest.raises(ValueError):   # wrong table shape
        flash_attn.flash_attn_with_kvcache(q, kp, kp, cache_seqlens=sl, page_table=table[:1])
