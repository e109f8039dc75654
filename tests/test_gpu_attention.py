"""GPU parity of flash_attn_with_kvcache (decode split-K and chunk paths).

Reference: the oracle (nanochat/flash_attention.py:155-177 + :69-102 applied
row by row) evaluated on the CPU in float32 from the same seeded inputs.
Tolerances (written per test): bf16/fp16 caches max rel err <= 2e-2 and
torch.allclose(atol=1e-2, rtol=1e-2) (nanochat tests/test_attention_fallback.py:39);
fp32 caches 1e-4.  Cache contents after the call are compared bit-exactly.
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, B, T_new, H, H_kv, D, T_max, seqlens, q_dtype, cache_dtype):
    g = gen(seed)
    q = randn((B, T_new, H, D), g, q_dtype)
    k = randn((B, T_new, H_kv, D), g, q_dtype)
    v = randn((B, T_new, H_kv, D), g, q_dtype)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=cache_dtype)
    vc = torch.zeros(B, T_max, H_kv, D, dtype=cache_dtype)
    for b, s in enumerate(seqlens):
        s = int(s)
        kc[b, :s] = randn((s, H_kv, D), g, cache_dtype)
        vc[b, :s] = randn((s, H_kv, D), g, cache_dtype)
    return q, k, v, kc, vc, torch.as_tensor(seqlens, dtype=torch.int32)


def _tol(q_dtype, cache_dtype):
    if q_dtype == torch.float32 and cache_dtype == torch.float32:
        return 1e-4, 1e-4
    return 2e-2, 1e-2


def _check(seed, B, T_new, H, H_kv, D, T_max, seqlens, window, q_dtype=torch.bfloat16,
           cache_dtype=torch.bfloat16, kps=0, with_kv=True):
    q, k, v, kc, vc, sl = _inputs(seed, B, T_new, H, H_kv, D, T_max, seqlens, q_dtype, cache_dtype)
    kc_d, vc_d, sl_d = kc.to(DEV), vc.to(DEV), sl.to(DEV)
    kk = k.to(DEV) if with_kv else None
    vv = v.to(DEV) if with_kv else None
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=kk, v=vv, cache_seqlens=sl_d, causal=True,
                                             window_size=(window, 0), keys_per_split=kps)
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k if with_kv else None, v=v if with_kv else None,
                                      cache_seqlens=sl, causal=True, window_size=(window, 0),
                                      compute_dtype=torch.float32)
    assert out.shape == (B, T_new, H, D) and out.dtype == q_dtype
    rel_tol, atol = _tol(q_dtype, cache_dtype)
    err = max_rel_err(out, ref.float())
    assert err <= rel_tol, f"max rel err {err:.3e}"
    assert torch.allclose(out.float().cpu(), ref.float(), atol=atol, rtol=atol)
    assert torch.equal(bits(kc_d), bits(kc)), "k_cache bytes differ from the oracle"
    assert torch.equal(bits(vc_d), bits(vc)), "v_cache bytes differ from the oracle"
    assert torch.equal(sl_d.cpu(), sl), "cache_seqlens must not be modified"
    return out


# ---- nanochat tests/test_attention_fallback.py scenarios, re-expressed ----
def test_reference_scenario_prefill_into_empty_cache():
    _check(1, 2, 16, 4, 4, 32, 64, [0, 0], 64)


def test_reference_scenario_single_token():
    _check(2, 2, 1, 4, 4, 32, 64, [16, 16], 64)


def test_reference_scenario_single_token_sliding_window():
    _check(3, 2, 1, 4, 4, 32, 64, [32, 32], 8)


def test_reference_scenario_sdpa_only_kvcache_flow():
    """TestSDPAOnly.test_kvcache: prefill 16 then decode 1 through KVCache and advance."""
    from nanochat_amd.engine import KVCache
    B, T_max, H, D = 2, 64, 4, 32
    cache = KVCache(batch_size=B, num_heads=H, seq_len=T_max, head_dim=D, num_layers=1, device=DEV,
                    dtype=torch.bfloat16)
    k_cache, v_cache = cache.get_layer_cache(0)
    g = gen(4)
    q, k, v = (randn((B, 16, H, D), g, torch.bfloat16).to(DEV) for _ in range(3))
    y = flash_attn.flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens=cache.cache_seqlens,
                                           causal=True, window_size=(T_max, 0))
    cache.advance(16)
    assert y.shape == (B, 16, H, D) and cache.get_pos() == 16
    q1, k1, v1 = (randn((B, 1, H, D), g, torch.bfloat16).to(DEV) for _ in range(3))
    y1 = flash_attn.flash_attn_with_kvcache(q1, k_cache, v_cache, k=k1, v=v1, cache_seqlens=cache.cache_seqlens,
                                            causal=True, window_size=(T_max, 0))
    cache.advance(1)
    assert y1.shape == (B, 1, H, D) and cache.get_pos() == 17
    assert not torch.isnan(y).any() and not torch.isnan(y1).any()


# ---- decode (T_new = 1) ----
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_decode_head_dims(D):
    _check(10 + D, 3, 1, 4, 4, D, 200, [0, 77, 199], -1, kps=64)


@pytest.mark.parametrize("H,H_kv", [(4, 4), (8, 2), (16, 4), (12, 4), (6, 2), (16, 2), (24, 3)])
def test_decode_gqa(H, H_kv):
    _check(20 + H, 4, 1, H, H_kv, 128, 300, [5, 130, 299, 64], -1, kps=64)


@pytest.mark.parametrize("window", [0, 1, 37, 128, 511])
def test_decode_sliding_window_ragged(window):
    _check(30 + window, 5, 1, 4, 2, 128, 700, [0, 3, 250, 600, 699], window, kps=64)


@pytest.mark.parametrize("q_dtype,cache_dtype", [
    (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16), (torch.float32, torch.float32),
    (torch.float32, torch.bfloat16), (torch.float16, torch.bfloat16), (torch.bfloat16, torch.float32),
])
def test_decode_dtypes(q_dtype, cache_dtype):
    _check(40, 3, 1, 8, 4, 128, 400, [17, 256, 399], 100, q_dtype=q_dtype, cache_dtype=cache_dtype, kps=128)


@pytest.mark.parametrize("kps", [0, 64, 128, 512, 1152])
def test_decode_split_sizes_agree(kps):
    _check(50, 6, 1, 10, 10, 128, 1100, [0, 1, 511, 512, 513, 1099], -1, kps=kps)


def test_chunk_split_merge():
    _check(51, 2, 5, 8, 2, 128, 900, [0, 700], -1, kps=64)


def test_decode_many_splits_cap():
    """16384 keys at 64 keys per split exceed the 256-split cap: the plan widens the splits."""
    _check(52, 2, 1, 4, 1, 64, 16384, [16383, 9000], -1, kps=64)


def test_decode_without_new_kv_reads_cache_only():
    _check(60, 3, 1, 4, 4, 64, 100, [10, 50, 98], -1, with_kv=False, kps=64)


def test_decode_repeated_calls_reuse_workspace():
    """The per-stream workspace is reused: many calls in a row stay correct."""
    for i in range(5):
        _check(70 + i, 4, 1, 8, 8, 128, 600, [100 * (i + 1), 7, 599 - i, 300], -1, kps=64)


def test_decode_d20_shapes_ragged_batch():
    """C2 shapes at B = 32 with the library's default split (one layer)."""
    g = gen(0)
    seqlens = torch.randint(512, 2049, (32,), generator=g, dtype=torch.int32).tolist()
    _check(80, 32, 1, 10, 10, 128, 2304, seqlens, -1)


# ---- chunk (T_new > 1) ----
@pytest.mark.parametrize("T_new", [2, 7, 33])
def test_chunk_ragged_window_gqa(T_new):
    _check(90 + T_new, 3, T_new, 8, 2, 64, 300, [0, 41, 300 - T_new], 50, kps=64)


def test_chunk_full_causal_into_nonempty_cache():
    _check(95, 2, 24, 6, 6, 128, 400, [100, 376], -1)


def test_chunk_fp32_compute_bf16_cache():
    _check(96, 2, 9, 4, 4, 128, 128, [0, 60], 20, q_dtype=torch.float32, cache_dtype=torch.bfloat16)


def test_chunk_equals_sequential_decode_on_gpu():
    """Incremental-equals-full invariant through the HIP path itself."""
    q, k, v, kc, vc, sl = _inputs(97, 2, 12, 4, 2, 128, 200, [30, 111], torch.bfloat16, torch.bfloat16)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    qd, kd, vd, sld = q.to(DEV), k.to(DEV), v.to(DEV), sl.to(DEV)
    full = flash_attn.flash_attn_with_kvcache(qd, kc1, vc1, k=kd, v=vd, cache_seqlens=sld, window_size=(40, 0))
    steps = []
    pos = sld.clone()
    for t in range(12):
        steps.append(flash_attn.flash_attn_with_kvcache(qd[:, t:t + 1], kc2, vc2, k=kd[:, t:t + 1],
                                                        v=vd[:, t:t + 1], cache_seqlens=pos, window_size=(40, 0)))
        pos += 1
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))
    assert max_rel_err(full, torch.cat(steps, dim=1)) <= 1e-2


def test_flash_attn_func_forward_matches_oracle():
    g = gen(98)
    q, k, v = (randn((2, 40, 4, 64), g, torch.bfloat16) for _ in range(3))
    with torch.no_grad():
        out = flash_attn.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, window_size=(9, 0))
    ref = orc.sdpa_attention(q.float().transpose(1, 2), k.float().transpose(1, 2), v.float().transpose(1, 2),
                             (9, 0), False).transpose(1, 2)
    assert max_rel_err(out, ref) <= 2e-2


# ---- error behaviour ----
def test_overflow_sets_device_flag():
    dev = torch.device(DEV, torch.cuda.current_device())
    _ext.read_and_clear_device_errors(dev)
    q, k, v, kc, vc, sl = _inputs(99, 2, 1, 4, 4, 64, 16, [3, 16], torch.bfloat16, torch.bfloat16)
    kc_d = kc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc.to(DEV), k=k.to(DEV), v=v.to(DEV),
                                             cache_seqlens=sl.to(DEV))
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_OVERFLOW
    assert torch.isfinite(out.float()).all()
    assert torch.equal(bits(kc_d[1]), bits(kc[1])), "row past the end must not be written"


def test_mismatched_dtypes_raise():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(1, 8, 4, 64, dtype=torch.bfloat16, device=DEV)
    sl = torch.zeros(1, dtype=torch.int32, device=DEV)
    with pytest.raises(TypeError):
        flash_attn.flash_attn_with_kvcache(q, kc, kc.clone(), k=q.float(), v=q.float(), cache_seqlens=sl)
    with pytest.raises(RuntimeError, match="head_dim"):
        q2 = torch.zeros(1, 1, 4, 48, dtype=torch.bfloat16, device=DEV)
        kc2 = torch.zeros(1, 8, 4, 48, dtype=torch.bfloat16, device=DEV)
        flash_attn.flash_attn_with_kvcache(q2, kc2, kc2.clone(), cache_seqlens=sl)


# ---- MFMA chunk kernel (T_new >= 8, bf16/fp16 caches, head_dim 64/128) ----
@pytest.mark.parametrize("T_new,H,H_kv,D,seqlens,window,dtype", [
    (8, 4, 4, 128, [0, 50], -1, torch.bfloat16),             # threshold, one q tile
    (70, 6, 6, 128, [0, 130], -1, torch.bfloat16),           # partial second q tile
    (64, 16, 4, 128, [0, 333, 1000, 1900], -1, torch.bfloat16),  # C5-like GQA 4:1 chunk rows
    (128, 16, 2, 64, [5, 700], 100, torch.bfloat16),         # GQA 8:1, window
    (96, 8, 8, 128, [0, 64], 31, torch.float16),             # fp16, small window
    (40, 12, 4, 64, [17, 0, 250], -1, torch.float16),        # GQA 3:1 (head blocks of 1)
])
def test_mfma_chunk_matches_oracle(T_new, H, H_kv, D, seqlens, window, dtype):
    T_max = max(seqlens) + T_new + 3
    _check(200 + T_new, len(seqlens), T_new, H, H_kv, D, T_max, seqlens, window, q_dtype=dtype, cache_dtype=dtype)


@pytest.mark.parametrize("H,H_kv", [(16, 4), (4, 4)])
def test_mfma_chunk_default_split_of_long_spans(H, H_kv):
    """Spans beyond 2048 keys with the library's split size (2048 keys for 16/4 heads, 512 for
    4/4): one long row next to short ones, merged by the split-merge kernel."""
    _check(260 + H, 3, 128, H, H_kv, 128, 6200, [6000, 100, 3000], -1)


@pytest.mark.parametrize("window", [-1, 512])
def test_mfma_chunk_c3_prefill(window):
    """C3 prefill shape: one row, 1024 tokens into an empty cache, 12 heads x 128 (S and L windows)."""
    _check(210, 1, 1024, 12, 12, 128, 1152, [0], window)


@pytest.mark.parametrize("kps,window", [(64, -1), (128, 200), (320, -1), (4096, 50)])
def test_mfma_chunk_split_sizes(kps, window):
    """Split-K of the chunk kernel: q tiles of one call have different split counts (ragged rows, causal
    spans, windows); one-split tiles write directly, the others go through the merge."""
    _check(220, 3, 100, 8, 2, 128, 1200, [0, 37, 1000], window, kps=kps)


def test_mfma_chunk_overflow_stores_in_range_tokens_and_flags():
    """Chunk append past t_max (the reference raises at flash_attention.py:161): the kernel stores the
    tokens below t_max, skips the rest, sets the overflow flag, and leaves other rows' bytes alone."""
    dev = torch.device(DEV, torch.cuda.current_device())
    _ext.read_and_clear_device_errors(dev)
    T_new, T_max = 20, 40
    q, k, v, kc, vc, sl = _inputs(98, 2, T_new, 4, 2, 64, T_max, [5, 30], torch.bfloat16, torch.bfloat16)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV),
                                             cache_seqlens=sl.to(DEV), causal=True)
    assert _ext.read_and_clear_device_errors(dev) & _ext.NC_DEVERR_OVERFLOW
    assert torch.isfinite(out.float()).all()
    kc_exp, vc_exp = kc.clone(), vc.clone()
    kc_exp[0, 5:25] = k[0]
    vc_exp[0, 5:25] = v[0]
    kc_exp[1, 30:40] = k[1, :10]
    vc_exp[1, 30:40] = v[1, :10]
    assert torch.equal(bits(kc_d), bits(kc_exp))
    assert torch.equal(bits(vc_d), bits(vc_exp))
    # the in-range row is exact attention
    ref = orc.flash_attn_with_kvcache(q[:1], kc[:1].clone(), vc[:1].clone(), k=k[:1], v=v[:1],
                                      cache_seqlens=sl[:1], causal=True, compute_dtype=torch.float32)
    assert max_rel_err(out[:1], ref.float()) <= 2e-2


def test_mfma_chunk_reads_strided_new_kv():
    """k/v as views of a fused (B, T, 2, H_kv, D) projection output: the chunk kernel takes the new
    tokens straight from the strided k/v and stores them into the cache."""
    g = gen(97)
    B, T_new, H, H_kv, D, T_max = 2, 48, 8, 4, 128, 300
    seqlens = [0, 211]
    q = randn((B, T_new, H, D), g, torch.bfloat16)
    kv = randn((B, T_new, 2, H_kv, D), g, torch.bfloat16)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[1, :211] = randn((211, H_kv, D), g, torch.bfloat16)
    vc[1, :211] = randn((211, H_kv, D), g, torch.bfloat16)
    sl = torch.tensor(seqlens, dtype=torch.int32)
    kv_d = kv.to(DEV)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=kv_d[:, :, 0], v=kv_d[:, :, 1],
                                             cache_seqlens=sl.to(DEV), causal=True, window_size=(100, 0))
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=kv[:, :, 0], v=kv[:, :, 1], cache_seqlens=sl, causal=True,
                                      window_size=(100, 0), compute_dtype=torch.float32)
    assert max_rel_err(out, ref.float()) <= 2e-2
    assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc))


@pytest.mark.parametrize("H,H_kv,kps", [(16, 4, 128), (8, 1, 64), (6, 6, 128)])
def test_decode_merge_beyond_16_splits(H, H_kv, kps):
    """Rows of 40+ splits take the 32-slot merge (float4 per thread), short rows in the same call
    write directly or merge a few slots."""
    _check(230 + H, 3, 1, H, H_kv, 128, 5200, [5000, 70, 2100], -1, kps=kps)


@pytest.mark.parametrize("B,H,H_kv,D,seqlens,window", [
    (16, 12, 12, 128, [1024] * 16, 512),            # C3 decode shape, S layer (8-wave workgroups, no split)
    (12, 13, 13, 128, [3072, 3000, 2999, 3072, 1, 0, 3100, 3071, 4095, 2, 64, 65], -1),  # ragged, up to 4096 keys
    (40, 16, 4, 128, [(i * 977) % 4000 for i in range(40)], -1),  # GQA 4:1 head blocks, 160 groups
    (20, 8, 8, 256, [(i * 613) % 4090 for i in range(20)], 700),  # head_dim 256, window
])
def test_decode_wide_workgroups_no_split(B, H, H_kv, D, seqlens, window):
    """128..256 groups with rows <= 4096 keys take 8-wave workgroups with one split (no merge launch)."""
    _check(240 + B, B, 1, H, H_kv, D, max(seqlens) + 4, seqlens, window)


def _sync_region_is_zero():
    """Every stream workspace's leading split counters are back at zero."""
    torch.cuda.synchronize()
    for buf in list(_ext._workspaces.values()):
        head = buf[:_ext.NC_WORKSPACE_SYNC_BYTES]
        assert int(head.count_nonzero()) == 0


def test_decode_in_kernel_merge_counters_return_to_zero():
    """Split merges by the last workgroup of each group: calls whose split
    counts per row change from call to call (ragged rows, 64-key splits, more
    than 8 slots per row), a chunk call in between, and the counters are zero
    after each call."""
    cases = [
        (4, 8, 8, [3000, 7, 64, 65]),           # up to 47 splits: several merge rounds
        (6, 16, 4, [1, 640, 2999, 128, 129, 0]),
        (2, 4, 4, [2500, 2501]),
    ]
    for i, (B, H, H_kv, seqlens) in enumerate(cases):
        _check(300 + i, B, 1, H, H_kv, 128, 3072, seqlens, -1, kps=64)
        _sync_region_is_zero()
        _check(310 + i, B, 16, H, H_kv, 128, 3072, [min(s, 3000) for s in seqlens], -1)  # chunk partials
        _sync_region_is_zero()
        _check(320 + i, B, 1, H, H_kv, 128, 3072, [max(s - 1, 0) for s in seqlens], 700, kps=128)
        _sync_region_is_zero()


def test_decode_more_groups_than_counters_uses_merge_launch():
    """16640 (row, head) groups exceed the 16384 counters of the sync region:
    the plan falls back to the merge kernel; same results."""
    B, H = 65, 256
    seqlens = [(b * 37) % 200 for b in range(B)]
    _check(330, B, 1, H, H, 32, 200, seqlens, -1, kps=64)
    _sync_region_is_zero()


def test_decode_long_rows_spread_over_bounded_splits():
    """96 groups in a 16384-key cache: the default plan keeps 4096 // 96 = 42 splits per group, so
    rows longer than 42 x 256 keys take longer splits (multiples of 64); short rows in the same
    call keep 256-key splits."""
    B = 24
    seqlens = [16000, 12000, 7000, 2689, 128, 10751, 10752, 10753] + [(i * 331) % 900 for i in range(B - 8)]
    _check(340, B, 1, 8, 4, 64, 16384, seqlens, -1)
