"""C-ABI checks that need no GPU: the library loads, exports every function
include/nc_kv.h declares, and its host-side validation and planning behave.
(No kernel is launched here.)"""
import ctypes
import re

import pytest
import torch

from nanochat_amd import _ext
from tests.conftest import ROOT

HEADER = ROOT / "include" / "nc_kv.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(nc_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    assert _declared_functions() == sorted(_ext.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _ext.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.nc_abi_version() == _ext.ABI_VERSION


def test_header_constants_match_python_mirror():
    text = HEADER.read_text()
    for name in ("NC_KV_ABI_VERSION", "NC_WORKSPACE_SYNC_BYTES", "NC_DEVERR_OVERFLOW", "NC_DEVERR_ROPE_RANGE",
                 "NC_DEVERR_BATCH_IDX", "NC_DEVERR_QLEN", "NC_DEVERR_SAMPLE"):
        value = int(re.search(r"#define %s (\d+)" % name, text).group(1))
        py = _ext.ABI_VERSION if name == "NC_KV_ABI_VERSION" else getattr(_ext, name)
        assert py == value, name


def test_struct_layouts_match_header_field_order():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for cname, pystruct in (("nc_append_args", _ext.AppendArgs), ("nc_fanout_args", _ext.FanoutArgs),
                            ("nc_attn_args", _ext.AttnArgs), ("nc_qk_prologue", _ext.QKPrologue),
                            ("nc_linear_args", _ext.LinearArgs), ("nc_sample_args", _ext.SampleArgs)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), text, flags=re.S).group(1)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            decl = re.sub(r"^(const\s+)?[\w]+\s*\*?\s*", "", decl)
            names += [n.strip().lstrip("*") for n in decl.split(",")]
        assert names == [f[0] for f in pystruct._fields_], cname


def test_strerror_names_every_status():
    lib = _ext.lib()
    for code in range(9):
        assert lib.nc_strerror(code).decode()
    assert lib.nc_strerror(0).decode() == "ok"
    assert lib.nc_strerror(99).decode() == "unknown nc_status"


def test_supported_head_dims():
    lib = _ext.lib()
    assert [d for d in (16, 32, 64, 96, 128, 256) if lib.nc_supports_head_dim(d)] == [32, 64, 128, 256]


def _attn_args(B=32, T_new=1, T_max=2304, H=10, H_kv=10, D=128, window=-1, dtype=2, kps=0):
    a = _ext.AttnArgs()
    a.batch, a.t_new, a.t_max, a.n_heads, a.n_kv_heads, a.head_dim = B, T_new, T_max, H, H_kv, D
    a.window_left = window
    a.q_dtype = a.cache_dtype = dtype
    a.keys_per_split = kps
    a.softmax_scale = D ** -0.5
    return a


def test_workspace_plan_for_d20_decode():
    lib = _ext.lib()
    a = _attn_args()
    # 64 KiB of K per head per split -> 256 keys; 2304 / 256 = 9 splits;
    # (m, l) and o partials per (row, head, split)
    pairs = 32 * 10
    expect = _ext.NC_WORKSPACE_SYNC_BYTES + 256 * ((pairs * 9 * 8 + 255) // 256) + pairs * 9 * 128 * 4
    assert lib.nc_attn_workspace_bytes(ctypes.byref(a)) == expect


def test_workspace_zero_for_single_split_and_window_caps_keys():
    lib = _ext.lib()
    assert lib.nc_attn_workspace_bytes(ctypes.byref(_attn_args(T_max=256))) == 0
    assert lib.nc_attn_workspace_bytes(ctypes.byref(_attn_args(T_max=4096, window=255))) == 0
    assert lib.nc_attn_workspace_bytes(ctypes.byref(_attn_args(T_max=4096, window=256))) > 0
    # split cap: 65536 keys at the 256-key default is exactly 256 splits; 80000 keys keep 256
    # splits (the kernels spread a longer row evenly over them)
    assert lib.nc_attn_workspace_bytes(ctypes.byref(_attn_args(B=1, H=1, H_kv=1, T_max=80000))) == \
        _ext.NC_WORKSPACE_SYNC_BYTES + 256 * ((1 * 256 * 8 + 255) // 256) + 256 * 128 * 4


def test_default_decode_grid_is_bounded():
    lib = _ext.lib()
    # 192 (row, kv head) groups (48 rows, GQA 16/4 -> one head block of 4): 4096 // 192 = 21 splits
    # per group instead of 16384 / 256 = 64.  Rows longer than 21 x 256 keys then take
    # length-balanced pieces, on the same grid of 192 x 21 workgroups with one partial slot per
    # workgroup and q head of its block.  An explicit split size keeps every split.
    pairs = 48 * 16
    slots = 192 * 21 * 4
    a = _attn_args(B=48, T_max=16384, H=16, H_kv=4)
    assert lib.nc_attn_workspace_bytes(ctypes.byref(a)) == \
        _ext.NC_WORKSPACE_SYNC_BYTES + 256 * ((slots * 8 + 255) // 256) + slots * 128 * 4
    a = _attn_args(B=48, T_max=16384, H=16, H_kv=4, kps=256)
    assert lib.nc_attn_workspace_bytes(ctypes.byref(a)) == \
        _ext.NC_WORKSPACE_SYNC_BYTES + 256 * ((pairs * 64 * 8 + 255) // 256) + pairs * 64 * 128 * 4


def _chunk_workspace(pairs, splits, D=128):
    return _ext.NC_WORKSPACE_SYNC_BYTES + 256 * ((pairs * splits * 8 + 255) // 256) + pairs * splits * D * 4


def test_chunk_split_size_gives_each_row_about_256_workgroups():
    lib = _ext.lib()
    # 16/4 heads, 128 tokens: 8 q tiles x 4 kv heads = 32 workgroups per split of a row;
    # 16384 keys * 32 / 256 = 2048-key splits -> 8 splits
    a = _attn_args(B=1, T_new=128, T_max=16384, H=16, H_kv=4)
    assert lib.nc_attn_workspace_bytes(ctypes.byref(a)) == _chunk_workspace(128 * 16, 8)
    # 4/4 heads: 2 q tiles x 4 kv heads = 8 per split -> 512-key splits (the unit) -> 32 splits
    a = _attn_args(B=1, T_new=128, T_max=16384, H=4, H_kv=4)
    assert lib.nc_attn_workspace_bytes(ctypes.byref(a)) == _chunk_workspace(128 * 4, 32)
    # spans up to 2048 keys run unsplit: no workspace
    assert lib.nc_attn_workspace_bytes(ctypes.byref(_attn_args(B=1, T_new=128, T_max=2048, H=4, H_kv=4))) == 0


def test_invalid_arguments_are_rejected_before_launch():
    lib = _ext.lib()
    a = _attn_args()
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 1  # NULL pointers
    fake = 1 << 20
    a.q = a.out = a.k_cache = a.v_cache = a.cache_seqlens = fake
    a.n_kv_heads = 3
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 2  # 10 % 3 != 0
    a.n_kv_heads = 10
    a.head_dim = 96
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 4  # head_dim
    a.head_dim = 128
    a.cache_dtype = 7
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 3  # dtype
    a.cache_dtype = 2
    a.kc_stride_t = 3  # 6 bytes: not 16-byte aligned
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 5
    a.kc_stride_t = a.vc_stride_t = 1280
    a.q_stride_h = 128
    a.workspace = None
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 6  # 9 splits need a workspace
    a.keys_per_split = 100
    assert lib.nc_attn_kvcache(ctypes.byref(a), None) == 2  # not a multiple of 64


def test_linear_plan_splits_k_to_fill_the_gpu():
    lib = _ext.lib()
    sync = _ext.NC_WORKSPACE_SYNC_BYTES
    # (m, n, k) -> splits, for m > 32: 64-column blocks x splits reaches about 512 workgroups, with
    # at least one 128-wide chunk of k per split and at most 4 splits; partials are 64 columns x
    # m_tiles x 16 rows fp32 per (block, split)
    for (m, n, k), splits in {(64, 1280, 1280): 4, (64, 1280, 5120): 4, (48, 5120, 1280): 4,
                              (33, 1536, 6144): 4, (48, 640, 896): 4, (33, 20000, 1280): 2,
                              (64, 64, 256): 2}.items():
        m_tiles, n_blocks = (m + 15) // 16, (n + 63) // 64
        assert lib.nc_linear_workspace_bytes(m, n, k) == sync + n_blocks * splits * 64 * m_tiles * 64, (m, n, k)
    # m <= 32 where the 64-column plan would split K: the narrow kernel (K split over the waves of
    # one workgroup, summed in LDS), no workspace ...
    for m, n, k in [(32, 1280, 1280), (32, 5120, 1280), (1, 1280, 1280), (32, 640, 896), (32, 20000, 1280),
                    (8, 64, 256), (16, 1536, 1536)]:
        assert lib.nc_linear_workspace_bytes(m, n, k) == 0, (m, n, k)
    # ... unless K is long and there are fewer than 256 blocks of 16 columns: then K is split over 2
    # workgroups as well (at least one 128-wide chunk per wave and split; 16 waves here), partials of
    # 64 lanes x m_tiles x 4 fp32 per (block, split)
    for (m, n, k), (blocks, splits) in {(32, 1280, 5120): (80, 2), (16, 1536, 6144): (96, 2),
                                        (32, 136, 4104): (9, 2)}.items():
        m_tiles = (m + 15) // 16
        assert lib.nc_linear_workspace_bytes(m, n, k) == sync + blocks * splits * m_tiles * 64 * 4 * 4, (m, n, k)
    # no split: at least 512 column blocks (lm_head)
    assert lib.nc_linear_workspace_bytes(32, 32768, 1280) == 0
    assert lib.nc_linear_workspace_bytes(64, 32768, 1280) == 0
    assert lib.nc_linear_workspace_bytes(32, 65536, 2048) == 0
    assert lib.nc_linear_workspace_bytes(0, 16, 16) == 0


def test_linear_rejects_bad_arguments_before_launch():
    lib = _ext.lib()
    a = _ext.LinearArgs()
    assert lib.nc_linear(ctypes.byref(a), None) == 1          # NULL pointers
    fake = 1 << 20
    a.x = a.w = a.y = fake
    a.m, a.n, a.k = 32, 64, 128
    a.x_stride_m, a.w_stride_n, a.y_stride_m = 128, 128, 64
    a.dtype = a.y_dtype = 2
    for field, bad in (("m", 65), ("m", 0), ("k", 12), ("n", 0), ("x_stride_m", 64), ("y_stride_m", 32),
                       ("w_stride_n", 1 << 24)):
        good = getattr(a, field)
        setattr(a, field, bad)
        assert lib.nc_linear(ctypes.byref(a), None) == 2, field
        setattr(a, field, good)
    a.dtype = a.y_dtype = 0                                    # fp32 operands are not taken
    assert lib.nc_linear(ctypes.byref(a), None) == 3
    a.dtype, a.y_dtype = 2, 1                                  # bf16 operands, fp16 output
    assert lib.nc_linear(ctypes.byref(a), None) == 3
    a.y_dtype, a.softcap = 2, 15.0                             # the logits head writes fp32
    assert lib.nc_linear(ctypes.byref(a), None) == 3
    a.softcap = float("nan")
    assert lib.nc_linear(ctypes.byref(a), None) == 2
    a.softcap = 0.0
    a.x_stride_m = 132                                         # rows not 16-byte aligned
    assert lib.nc_linear(ctypes.byref(a), None) == 5
    a.x_stride_m = 128
    a.x = fake + 8
    assert lib.nc_linear(ctypes.byref(a), None) == 5
    a.x = fake
    a.m, a.n, a.k, a.w_stride_n, a.x_stride_m, a.y_stride_m = 64, 1280, 1280, 1280, 1280, 1280
    assert lib.nc_linear(ctypes.byref(a), None) == 6          # K split: needs a workspace
    a.workspace, a.workspace_bytes = fake, lib.nc_linear_workspace_bytes(64, 1280, 1280) - 16
    assert lib.nc_linear(ctypes.byref(a), None) == 6


def test_sample_rejects_bad_arguments_before_launch():
    lib = _ext.lib()
    a = _ext.SampleArgs()
    assert lib.nc_sample(ctypes.byref(a), None) == 1           # NULL pointers
    fake = 1 << 20
    a.logits, a.out = fake, fake
    a.batch, a.vocab, a.logits_stride, a.temperature, a.top_k = 4, 5000, 5000, 1.0, 0
    assert lib.nc_sample(ctypes.byref(a), None) == 1           # sampling needs uniforms
    a.uniforms = fake
    for field, bad in (("batch", 0), ("vocab", 0), ("logits_stride", 4999), ("logits_stride", -1), ("top_k", -1),
                       ("top_k", 1025),
                       ("temperature", -1.0), ("temperature", float("nan"))):
        good = getattr(a, field)
        setattr(a, field, bad)
        assert lib.nc_sample(ctypes.byref(a), None) == 2, field
        setattr(a, field, good)
    a.out = fake + 4                                            # int64 ids need 8-byte alignment
    assert lib.nc_sample(ctypes.byref(a), None) == 5
    a.out = fake


def test_fanout_and_append_reject_bad_arguments():
    lib = _ext.lib()
    f = _ext.FanoutArgs()
    assert lib.nc_kv_fanout(ctypes.byref(f), None) == 1
    f.k_src = f.v_src = f.k_dst = f.v_dst = 1 << 20
    f.n_layers, f.n_rows, f.prefix_len, f.row_elems = 0, 1, 1, 1
    assert lib.nc_kv_fanout(ctypes.byref(f), None) == 2
    a = _ext.AppendArgs()
    assert lib.nc_kv_append(ctypes.byref(a), None) == 1
    a.k_cache = a.v_cache = a.k = a.v = a.cache_seqlens = 1 << 20
    a.batch, a.t_new, a.t_max, a.n_kv_heads, a.head_dim = 1, 1, 4, 1, 5
    a.cache_dtype = a.in_dtype = 2
    assert lib.nc_kv_append(ctypes.byref(a), None) == 4  # 10-byte rows cannot be 16-byte vectors


def test_python_surface_rejects_cpu_tensors_and_bad_shapes():
    from nanochat_amd.flash_attention import flash_attn
    q = torch.zeros(2, 1, 4, 32)
    kc = torch.zeros(2, 8, 4, 32)
    sl = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_attn.flash_attn_with_kvcache(q, kc, kc.clone(), k=q, v=q, cache_seqlens=sl)
    with pytest.raises(ValueError):
        flash_attn.flash_attn_with_kvcache(q, kc[:, :, :3], kc[:, :, :3].clone(), cache_seqlens=sl)
    with pytest.raises(ValueError):
        flash_attn.flash_attn_with_kvcache(q, kc, kc.clone(), k=q, v=None, cache_seqlens=sl)
    with pytest.raises(ValueError):
        flash_attn.flash_attn_with_kvcache(q, kc, kc.clone(), cache_seqlens=sl.long())


def test_override_mechanism_mirrors_reference():
    """nanochat tests/test_attention_fallback.py:340-359 on this module."""
    import nanochat_amd.flash_attention as fa
    fa._override_impl = 'sdpa'
    fa.USE_FA3 = fa._resolve_use_fa3()
    assert fa.USE_FA3 is False
    fa._override_impl = None
    fa.USE_FA3 = fa._resolve_use_fa3()
    assert fa.USE_FA3 == fa.HAS_FA3
    fa._override_impl = 'fa3'
    with pytest.raises(AssertionError):
        fa._resolve_use_fa3()
    fa._override_impl = None


def test_kv_cache_basic_on_cpu():
    """nanochat tests/test_engine.py:84-121 against nanochat_amd.KVCache."""
    from nanochat_amd.engine import KVCache
    c = KVCache(batch_size=2, num_heads=3, seq_len=64, head_dim=5, num_layers=6, device="cpu", dtype=torch.float32)
    assert c.get_pos() == 0
    assert c.k_cache.shape == (6, 2, 64, 3, 5) and c.v_cache.shape == (6, 2, 64, 3, 5)
    c.advance(10)
    assert c.get_pos() == 10
    c.advance(5)
    assert c.get_pos() == 15
    c.reset()
    assert c.get_pos() == 0
    k0, v0 = c.get_layer_cache(0)
    assert k0.shape == (2, 64, 3, 5) and v0.shape == (2, 64, 3, 5)
    assert k0.data_ptr() == c.k_cache.data_ptr()  # views, not copies


def test_prefill_on_cpu_fails_loudly():
    from nanochat_amd.engine import KVCache
    src = KVCache(1, 2, 8, 8, 1, "cpu", torch.float32)
    src.advance(4)
    dst = KVCache(2, 2, 8, 8, 1, "cpu", torch.float32)
    with pytest.raises(RuntimeError, match="GPU"):
        dst.prefill(src)


def test_invariant_divisor_method_is_exact():
    """The kernels split block indices with q = (mulhi(m, n) + n) >> l, m = floor(2^32 (2^l - d) / d) + 1,
    l = ceil(log2 d) (Granlund & Montgomery 1994, sec. 4), for n < 2^31.  Check the identity against
    integer division: every n < 4096 for d <= 300, and the extremes of the range for larger d."""
    def make(d):
        l = (d - 1).bit_length()
        return ((1 << 32) * ((1 << l) - d)) // d + 1, l

    def fdiv(n, m, l):
        return (((m * n) >> 32) + n) >> l

    for d in range(1, 301):
        m, l = make(d)
        assert m < (1 << 32)
        for n in range(4096):
            assert fdiv(n, m, l) == n // d, (n, d)
    g = torch.Generator().manual_seed(0)
    big = [2**31 - 1, 2**31 - 2, 2**30, 2**30 + 1, 3 * 2**29, 65537, 1 << 20, (1 << 20) + 1]
    big += torch.randint(1, 2**31 - 1, (200,), generator=g).tolist()
    for d in big:
        m, l = make(d)
        assert m < (1 << 32)
        ns = [0, 1, d - 1, d, d + 1, 2**31 - 1, (2**31 - 1) // d * d, (2**31 - 1) // d * d - 1]
        ns += torch.randint(0, 2**31, (64,), generator=g).tolist()
        for n in ns:
            if 0 <= n < 2**31:
                assert fdiv(n, m, l) == n // d, (n, d)
