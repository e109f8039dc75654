"""GPU parity of the cache writes: ragged append and prefill fan-out.

The bar is bit-exactness of the whole cache tensors against the oracle
(torch slice / broadcast assignment, nanochat/flash_attention.py:160-162 and
nanochat/engine.py:132-134), so stray writes anywhere are caught too.
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.engine import KVCache
from nanochat_amd.flash_attention import kv_append
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("in_dtype,cache_dtype", [
    (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16), (torch.float32, torch.float32),
    (torch.float32, torch.bfloat16), (torch.float32, torch.float16), (torch.bfloat16, torch.float32),
])
@pytest.mark.parametrize("T_new", [1, 3, 64])
def test_append_bit_exact(in_dtype, cache_dtype, T_new):
    g = gen(100 + T_new)
    B, T_max, H_kv, D = 5, 160, 3, 64
    seqlens = torch.randint(0, T_max - T_new + 1, (B,), generator=g, dtype=torch.int32)
    kc = randn((B, T_max, H_kv, D), g, cache_dtype)
    vc = randn((B, T_max, H_kv, D), g, cache_dtype)
    k = randn((B, T_new, H_kv, D), g, in_dtype)
    v = randn((B, T_new, H_kv, D), g, in_dtype)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    sl_d = seqlens.to(DEV)
    kv_append(kc_d, vc_d, k.to(DEV), v.to(DEV), sl_d)
    orc.kv_append(kc, vc, k, v, seqlens)
    assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc))
    assert torch.equal(sl_d.cpu(), seqlens)


def test_append_rounding_edge_cases_match_torch():
    """fp32 -> bf16 / fp16 ties, NaN, inf, denormals, overflow: identical bits to torch's
    device-side cast (the copy the reference's slice assignment performs on a GPU cache)."""
    specials = torch.tensor([
        1.0, 1.00390625, 1.01171875, 1.005859375, -2.5, 3.0e38, -3.4e38, 1e-40, -1e-42, 0.0, -0.0,
        float("inf"), float("-inf"), float("nan"), 65504.0, 65520.0, 70000.0, 6e-8, 1e-8, 2.0 ** -149,
    ], dtype=torch.float32)
    g = gen(7)
    noise = randn((1, 1, 1, 108), g) * 1e3
    k = torch.cat([specials.view(1, 1, 1, -1), noise], dim=-1).to(DEV)  # D = 128
    v = -k
    for cache_dtype in (torch.bfloat16, torch.float16):
        kc = torch.zeros(1, 4, 1, 128, dtype=cache_dtype, device=DEV)
        vc = torch.zeros(1, 4, 1, 128, dtype=cache_dtype, device=DEV)
        ref_k, ref_v = kc.clone(), vc.clone()
        ref_k[:, 2:3] = k  # torch's own copy kernel on the device
        ref_v[:, 2:3] = v
        kv_append(kc, vc, k, v, torch.tensor([2], dtype=torch.int32, device=DEV))
        for got, want in ((kc, ref_k), (vc, ref_v)):
            diff = (bits(got) != bits(want)).nonzero().tolist()
            assert not diff, f"{cache_dtype}: differing elements {diff[:8]}"


def test_append_overflow_sets_flag_and_writes_nothing_out_of_range():
    B, T_max, H_kv, D = 2, 16, 2, 32
    kc = torch.zeros(B, T_max + 4, H_kv, D, dtype=torch.bfloat16, device=DEV)  # guard band of 4 rows
    vc = torch.zeros_like(kc)
    view_k, view_v = kc[:, :T_max], vc[:, :T_max]
    k = torch.ones(B, 3, H_kv, D, dtype=torch.bfloat16, device=DEV)
    sl = torch.tensor([2, T_max - 1], dtype=torch.int32, device=DEV)
    dev = torch.device(DEV, torch.cuda.current_device())
    _ext.read_and_clear_device_errors(dev)
    kv_append(view_k, view_v, k, k, sl)
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_OVERFLOW
    assert (kc[0, 2:5] == 1).all() and (kc[1, T_max - 1] == 1).all()
    assert (kc[1, T_max:] == 0).all(), "guard band written"
    assert (kc[0, 5:] == 0).all() and (kc[1, :T_max - 1] == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_prefill_fanout_bit_exact(dtype):
    g = gen(11)
    L, H, D, P, T_src, T_dst, N = 3, 4, 64, 37, 40, 50, 6
    src = orc.KVCache(1, H, T_src, D, L, "cpu", dtype)
    src.k_cache.copy_(randn(src.k_cache.shape, g, dtype))
    src.v_cache.copy_(randn(src.v_cache.shape, g, dtype))
    src.advance(P)
    src.prev_embedding = randn((1, 1, 16), g, dtype)
    dst_ref = orc.KVCache(N, H, T_dst, D, L, "cpu", dtype)
    dst_ref.prefill(src)

    src_d = KVCache(1, H, T_src, D, L, DEV, dtype)
    src_d.k_cache.copy_(src.k_cache)
    src_d.v_cache.copy_(src.v_cache)
    src_d.advance(P)
    src_d.prev_embedding = src.prev_embedding.to(DEV)
    dst = KVCache(N, H, T_dst, D, L, DEV, dtype)
    dst.prefill(src_d)
    assert torch.equal(bits(dst.k_cache), bits(dst_ref.k_cache))
    assert torch.equal(bits(dst.v_cache), bits(dst_ref.v_cache))
    assert torch.equal(dst.cache_seqlens.cpu(), dst_ref.cache_seqlens)
    assert dst.get_pos() == P
    assert torch.equal(dst.prev_embedding.cpu(), dst_ref.prev_embedding)


def test_prefill_known_answer_from_reference_tests():
    """nanochat tests/test_engine.py:124-155 on the GPU cache."""
    src = KVCache(batch_size=1, num_heads=4, seq_len=32, head_dim=8, num_layers=2, device=DEV, dtype=torch.float32)
    src.k_cache[0, 0, :16, :, :] = 1.0
    src.v_cache[0, 0, :16, :, :] = 2.0
    src.advance(16)
    dst = KVCache(batch_size=1, num_heads=4, seq_len=64, head_dim=8, num_layers=2, device=DEV, dtype=torch.float32)
    dst.prefill(src)
    assert dst.get_pos() == 16
    assert (dst.k_cache[0, 0, :16, :, :] == 1.0).all()
    assert (dst.v_cache[0, 0, :16, :, :] == 2.0).all()
    assert (dst.k_cache[:, :, 16:] == 0).all() and (dst.k_cache[1] == 0).all()


def test_prefill_odd_sizes_use_narrow_units():
    """head_dim 5 (10-byte rows) still copies exactly (2-byte copy units)."""
    g = gen(12)
    src = KVCache(1, 3, 9, 5, 2, DEV, torch.bfloat16)
    src.k_cache.copy_(randn(src.k_cache.shape, g, torch.bfloat16).to(DEV))
    src.v_cache.copy_(randn(src.v_cache.shape, g, torch.bfloat16).to(DEV))
    src.advance(7)
    dst = KVCache(3, 3, 11, 5, 2, DEV, torch.bfloat16)
    dst.prefill(src)
    ref = torch.zeros_like(dst.k_cache)
    ref[:, :, :7] = src.k_cache[:, :, :7]
    assert torch.equal(bits(dst.k_cache), bits(ref))


def test_prefill_preconditions_raise_assertion():
    a = KVCache(1, 2, 8, 32, 1, DEV, torch.bfloat16)
    b = KVCache(1, 2, 4, 32, 1, DEV, torch.bfloat16)
    with pytest.raises(AssertionError):
        b.prefill(a)
    a.advance(1)
    with pytest.raises(AssertionError):
        a.prefill(b)


def test_d24_fanout_full_size():
    """C3 shapes (24 layers, 12 kv heads x 128, P = 1024 -> 16 rows of 1152): checksum of rows."""
    L, H, D, P, N = 24, 12, 128, 1024, 16
    src = KVCache(1, H, P, D, L, DEV, torch.bfloat16)
    gd = torch.Generator(device=DEV)
    gd.manual_seed(0)
    src.k_cache.normal_(generator=gd)
    src.v_cache.normal_(generator=gd)
    src.advance(P)
    dst = KVCache(N, H, P + 128, D, L, DEV, torch.bfloat16)
    dst.prefill(src)
    torch.cuda.synchronize()
    for n in (0, 7, N - 1):
        assert torch.equal(dst.k_cache[:, n, :P], src.k_cache[:, 0])
        assert torch.equal(dst.v_cache[:, n, :P], src.v_cache[:, 0])
    assert (dst.k_cache[:, :, P:] == 0).all() and (dst.v_cache[:, :, P:] == 0).all()
    assert (dst.cache_seqlens == P).all()


def test_reset_on_gpu_zeroes_positions_and_keeps_cache_bytes():
    """KVCache.reset (nanochat/engine.py:106-109) on the GPU: positions back to 0, prev_embedding
    dropped, cache bytes kept; the next append then writes at position 0 again (mirrors
    nanochat tests/test_engine.py:114-116)."""
    from nanochat_amd.flash_attention import flash_attn
    B, T_max, H, D = 3, 32, 2, 64
    cache = KVCache(batch_size=B, num_heads=H, seq_len=T_max, head_dim=D, num_layers=2, device=DEV,
                    dtype=torch.bfloat16)
    g = gen(401)
    for layer in range(2):
        kc, vc = cache.get_layer_cache(layer)
        q, k, v = (randn((B, 5, H, D), g, torch.bfloat16).to(DEV) for _ in range(3))
        flash_attn.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=cache.cache_seqlens, causal=True)
    cache.advance(5)
    cache.prev_embedding = torch.ones(B, 1, 8, device=DEV)
    assert cache.get_pos() == 5
    k_before, v_before = cache.k_cache.clone(), cache.v_cache.clone()
    cache.reset()
    assert cache.get_pos() == 0 and cache.cache_seqlens.tolist() == [0] * B
    assert cache.prev_embedding is None
    assert torch.equal(bits(cache.k_cache), bits(k_before)) and torch.equal(bits(cache.v_cache), bits(v_before))
    kc, vc = cache.get_layer_cache(0)
    k1 = randn((B, 1, H, D), g, torch.bfloat16).to(DEV)
    flash_attn.flash_attn_with_kvcache(k1, kc, vc, k=k1, v=k1, cache_seqlens=cache.cache_seqlens)
    want = k_before.clone()
    want[0, :, 0] = k1[:, 0]
    assert torch.equal(bits(cache.k_cache), bits(want)), "after reset the append lands at position 0"


def test_overflow_raises_at_get_pos():
    """An append past the cache length raises RuntimeError at the next host read of the positions
    (KVCache.get_pos, which GPT.forward and prefill make anyway), as the reference's slice
    assignment raises at the call (nanochat/flash_attention.py:160-162); the flag is then clear."""
    from nanochat_amd.flash_attention import flash_attn
    dev = torch.device(DEV, torch.cuda.current_device())
    _ext.read_and_clear_device_errors(dev)
    B, T_max, H, D = 2, 8, 2, 64
    cache = KVCache(batch_size=B, num_heads=H, seq_len=T_max, head_dim=D, num_layers=1, device=DEV,
                    dtype=torch.bfloat16)
    cache.advance(T_max)                              # full
    kc, vc = cache.get_layer_cache(0)
    x = torch.ones(B, 1, H, D, dtype=torch.bfloat16, device=DEV)
    before = cache.k_cache.clone()
    flash_attn.flash_attn_with_kvcache(x, kc, vc, k=x, v=x, cache_seqlens=cache.cache_seqlens)
    with pytest.raises(RuntimeError, match="exceeds the cache length"):
        cache.get_pos()
    assert cache.get_pos() == T_max                   # cleared: the next read is clean
    assert torch.equal(bits(cache.k_cache), bits(before)), "nothing stored past the end"
