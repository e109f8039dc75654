"""Drop-in for ``nanochat.flash_attention`` backed by gfx950 HIP kernels.

Same public surface as nanochat/flash_attention.py:
  - ``flash_attn`` namespace with ``flash_attn_with_kvcache`` and
    ``flash_attn_func`` (nanochat/flash_attention.py:184-187);
  - the module globals ``HAS_FA3``, ``USE_FA3``, ``_override_impl`` and
    ``_resolve_use_fa3`` that nanochat's tests flip (:41-63).  There is no FA3
    on MI355X and no SDPA fallback here: every call runs libnc_kv.so.

Semantics of ``flash_attn_with_kvcache`` (nanochat/flash_attention.py:131-177):
  - k/v (if given) are written in place into k_cache/v_cache at each row's own
    position ``cache_seqlens[b]`` (FA3's contract; the reference fallback uses
    row 0's position for all rows, :157, which is the same for uniform batches);
  - cache_seqlens is read, never advanced (the caller advances, gpt.py:119-121);
  - query i of row b sits at absolute position s_b + i (bottom-right aligned,
    :94) and sees keys j <= s_b + i with s_b + i - j <= window_size[0] when
    window_size[0] >= 0 (:96-100, :84-88);
  - ``causal`` and ``window_size[1]`` are accepted and, as in the fallback,
    do not change the mask;
  - GQA maps q head h to kv head h // (H / H_kv) (SDPA enable_gqa, :174);
  - the result is a new (B, T_new, H, D) tensor in q's dtype; k/v are stored
    in the cache dtype with round-to-nearest-even; scores and sums are fp32.
"""
from __future__ import annotations

import ctypes
import os
from types import SimpleNamespace

import torch

from . import _ext

# FA3 is a Hopper-only binary (nanochat/flash_attention.py:23-38); it does not
# exist on MI355X.  The names stay so callers and tests that read them work.
HAS_FA3 = False
_override_impl = None

_CHECK_ERRORS = os.environ.get("NANOCHAT_AMD_CHECK", "0") == "1"


def _resolve_use_fa3():
    """Mirror of nanochat/flash_attention.py:48-61: always False on MI355X."""
    if _override_impl == 'fa3':
        assert HAS_FA3, "Cannot override to FA3: not available on this hardware"
        return True
    return False


USE_FA3 = _resolve_use_fa3()


def _require_gpu(name: str, *tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"{name}: the MI355X KV-cache path runs on the GPU only (got device {dev})")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"{name}: all tensors must be on {dev}, got {t.device}")
    return dev


def _dtype_code(t: torch.Tensor, name: str) -> int:
    code = _ext.DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(f"{name} has unsupported dtype {t.dtype} (float32, float16, bfloat16)")
    return code


def _attn_call(name, q, k_cache, v_cache, k, v, cache_seqlens, causal, window_size, keys_per_split,
               cache_batch_idx=None, cu_seqlens_q=None, max_seqlen_q=None, page_table=None):
    """Validate the arguments of one attention call and fill nc_attn_args (workspace left empty).

    With cu_seqlens_q, q/k/v are packed tokens (total_q, H or H_kv, D) and the
    output is (total_q, H, D); otherwise (B, T_new, ...).
    """
    if cache_seqlens is None:
        raise ValueError(f"{name}: cache_seqlens is required")
    if (k is None) != (v is None):
        raise ValueError(f"{name}: pass both k and v, or neither")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError(f"{name}: k_cache, v_cache must be 4-D (B, T_max, H_kv, D)")
    varlen = cu_seqlens_q is not None
    if varlen:
        if q.dim() != 3:
            raise ValueError(f"{name}: with cu_seqlens_q, q must be (total_q, H, D)")
        if max_seqlen_q is None:
            raise ValueError(f"{name}: max_seqlen_q is required with cu_seqlens_q")
        if cu_seqlens_q.dim() != 1 or cu_seqlens_q.dtype != torch.int32 or cu_seqlens_q.numel() < 2:
            raise ValueError(f"{name}: cu_seqlens_q must be a (B+1,) int32 tensor")
        cu_seqlens_q = cu_seqlens_q.contiguous()
        total_q, H, D = q.shape
        B, T_new = cu_seqlens_q.numel() - 1, int(max_seqlen_q)
        if T_new < 1:
            raise ValueError(f"{name}: max_seqlen_q must be >= 1")
    else:
        if q.dim() != 4:
            raise ValueError(f"{name}: q must be 4-D (B, T, H, D)")
        B, T_new, H, D = q.shape
    Bc, T_max, H_kv, Dc = k_cache.shape
    if tuple(v_cache.shape) != (Bc, T_max, H_kv, Dc):
        raise ValueError(f"v_cache shape {tuple(v_cache.shape)} != k_cache shape {tuple(k_cache.shape)}")
    paged = page_table is not None
    if paged:
        # FA3's paged cache: (num_blocks, page_size, H_kv, D) blocks, row b's logical positions
        # through page_table[b] (B, max_blocks_per_seq) int32
        if cache_batch_idx is not None:
            raise ValueError(f"{name}: page_table and cache_batch_idx cannot be combined")
        if page_table.dim() != 2 or page_table.shape[0] != B or page_table.dtype != torch.int32:
            raise ValueError(f"{name}: page_table must be a (B, max_blocks) int32 tensor")
        if page_table.stride(-1) != 1:
            page_table = page_table.contiguous()
        page_size, num_blocks = T_max, Bc
        if page_size < 16 or page_size & (page_size - 1):
            raise ValueError(f"{name}: the page size (k_cache.shape[1] = {page_size}) must be a power of two >= 16")
        T_max = page_table.shape[1] * page_size   # logical positions of a row
    if (cache_batch_idx is None and not paged and Bc != B) or Dc != D:
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match q shape {tuple(q.shape)}")
    if cache_batch_idx is not None:
        if tuple(cache_batch_idx.shape) != (B,) or cache_batch_idx.dtype != torch.int32:
            raise ValueError("cache_batch_idx must be a (B,) int32 tensor")
        cache_batch_idx = cache_batch_idx.contiguous()
    if H % H_kv != 0:
        raise ValueError(f"n_heads {H} is not a multiple of n_kv_heads {H_kv}")
    if k is not None:
        kv_shape = (total_q, H_kv, D) if varlen else (B, T_new, H_kv, D)
        if tuple(k.shape) != kv_shape or tuple(v.shape) != kv_shape:
            raise ValueError(f"k/v must have shape {kv_shape}, got {tuple(k.shape)}, {tuple(v.shape)}")
        if k.dtype != q.dtype or v.dtype != q.dtype:
            raise TypeError(f"k/v dtype ({k.dtype}, {v.dtype}) must equal q dtype {q.dtype}")
    if tuple(cache_seqlens.shape) != (B,) or cache_seqlens.dtype != torch.int32:
        raise ValueError("cache_seqlens must be a (B,) int32 tensor")
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must have the same dtype")
    tensors = [q, k_cache, v_cache, cache_seqlens] + ([k, v] if k is not None else [])
    tensors += [cache_batch_idx] if cache_batch_idx is not None else []
    tensors += [cu_seqlens_q] if varlen else []
    tensors += [page_table] if paged else []
    dev = _require_gpu(name, *tensors)
    for tname, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("k", k), ("v", v)):
        if t is not None and t.stride(-1) != 1:
            raise ValueError(f"{tname} must be contiguous in its last (head_dim) dimension")
    if not cache_seqlens.is_contiguous():
        cache_seqlens = cache_seqlens.contiguous()

    out = torch.empty((total_q, H, D) if varlen else (B, T_new, H, D), dtype=q.dtype, device=dev)
    window = int(window_size[0]) if window_size is not None else -1
    a = _ext.AttnArgs()
    a.q = q.data_ptr(); a.out = out.data_ptr()
    a.k_cache = k_cache.data_ptr(); a.v_cache = v_cache.data_ptr()
    a.k = k.data_ptr() if k is not None else None
    a.v = v.data_ptr() if v is not None else None
    a.cache_seqlens = cache_seqlens.data_ptr()
    a.error_flag = _ext.error_flag(dev).data_ptr()
    if cache_batch_idx is not None:
        a.cache_batch_idx, a.cache_batch = cache_batch_idx.data_ptr(), Bc
    if varlen:
        a.cu_seqlens_q, a.total_q = cu_seqlens_q.data_ptr(), total_q
    if paged:
        a.page_table, a.page_table_stride = page_table.data_ptr(), page_table.stride(0)
        a.page_size, a.num_blocks = page_size, num_blocks
    a.batch, a.t_new, a.t_max = B, T_new, T_max
    a.n_heads, a.n_kv_heads, a.head_dim = H, H_kv, D
    if varlen:  # packed tokens: token stride and head stride (the batch stride is unused)
        a.q_stride_b, a.q_stride_t, a.q_stride_h = 0, q.stride(0), q.stride(1)
    else:
        a.q_stride_b, a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.kc_stride_b, a.kc_stride_t, a.kc_stride_h = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.vc_stride_b, a.vc_stride_t, a.vc_stride_h = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    if k is not None and varlen:
        a.k_stride_b, a.k_stride_t, a.k_stride_h = 0, k.stride(0), k.stride(1)
        a.v_stride_b, a.v_stride_t, a.v_stride_h = 0, v.stride(0), v.stride(1)
    elif k is not None:
        a.k_stride_b, a.k_stride_t, a.k_stride_h = k.stride(0), k.stride(1), k.stride(2)
        a.v_stride_b, a.v_stride_t, a.v_stride_h = v.stride(0), v.stride(1), v.stride(2)
    a.window_left = window if window >= 0 else -1
    a.causal = 1 if causal else 0
    a.softmax_scale = D ** -0.5
    a.q_dtype = _dtype_code(q, "q")
    a.cache_dtype = _dtype_code(k_cache, "k_cache")
    a.keys_per_split = int(keys_per_split)
    return a, out, dev, cache_seqlens


def _attach_workspace(a, dev, stream, need):
    ws = _ext.workspace(dev, stream, need)
    if ws is not None:
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()


def _check_device_errors(name, dev):
    """NANOCHAT_AMD_CHECK=1: read the device error flag after every call (one host sync each).

    By default the flag is read, and raised as RuntimeError, at the host synchronisations the
    callers already make: KVCache.get_pos and the engine's per-step sampled ids."""
    if _CHECK_ERRORS:
        _ext.raise_device_errors(_ext.read_and_clear_device_errors(dev), name)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                            causal=False, window_size=(-1, -1), *, cache_batch_idx=None, cu_seqlens_q=None,
                            max_seqlen_q=None, page_table=None, keys_per_split: int = 0):
    """Append k/v into the cache in place, then attend (see the module docstring).

    q: (B, T_new, H, D); k_cache, v_cache: (B, T_max, H_kv, D), or (B_cache, T_max,
    H_kv, D) with cache_batch_idx: (B,) int32, FA3's argument (row b uses cache
    row cache_batch_idx[b]; indices must be distinct when k/v are given);
    k, v: (B, T_new, H_kv, D) or None; cache_seqlens: (B,) int32 on the GPU.
    cu_seqlens_q: (B+1,) int32 with max_seqlen_q (FA3's varlen layout): q, k, v
    are packed tokens (total_q, H or H_kv, D), row b owning tokens
    [cu[b], cu[b+1]); rows may hold 0, 1 or many tokens.
    page_table: (B, max_blocks) int32 (FA3's paged cache): k_cache, v_cache are
    (num_blocks, page_size, H_kv, D) blocks and position j of row b is slot
    j % page_size of block page_table[b, j // page_size]; page_size a power of two >= 16.
    Returns (B, T_new, H, D), or (total_q, H, D) with cu_seqlens_q, in q's dtype.
    """
    a, out, dev, _ = _attn_call("flash_attn_with_kvcache", q, k_cache, v_cache, k, v, cache_seqlens, causal,
                                window_size, keys_per_split, cache_batch_idx, cu_seqlens_q, max_seqlen_q,
                                page_table)
    L = _ext.lib()
    ref = ctypes.byref(a)
    stream = _ext.stream_handle(dev)
    _attach_workspace(a, dev, stream, L.nc_attn_workspace_bytes(ref))
    _ext.check(L.nc_attn_kvcache(ref, stream), "nc_attn_kvcache")
    _check_device_errors("flash_attn_with_kvcache", dev)
    return out


def flash_attn_with_kvcache_rope(q, k_cache, v_cache, k, v, cache_seqlens, cos, sin, causal=True,
                                 window_size=(-1, -1), *, qk_scale: float = 1.2, eps=None,
                                 cache_batch_idx=None, cu_seqlens_q=None, max_seqlen_q=None, page_table=None,
                                 keys_per_split: int = 0):
    """flash_attn_with_kvcache with nanochat's QK prologue fused (nanochat/gpt.py:98-102).

    q and k are the raw projections; inside the call each token t of row b is
    rotated with table row cache_seqlens[b] + t of cos/sin (the model's
    (1, T_rot, 1, D/2) buffers or (T_rot, D/2) tables), RMS-normalised over D
    with `eps` (default torch.finfo(q.dtype).eps, F.rms_norm's default) and
    scaled by qk_scale; k is appended in that form, v as given.  Equivalent to
    rotary + norm + scale in torch followed by flash_attn_with_kvcache, with
    one rounding instead of one per op.
    """
    if k is None or v is None:
        raise ValueError("flash_attn_with_kvcache_rope: k and v are required")
    D = q.shape[-1]
    if D % 2 != 0:
        raise ValueError("flash_attn_with_kvcache_rope: head_dim must be even")
    cos2 = cos.reshape(-1, cos.shape[-1])
    sin2 = sin.reshape(-1, sin.shape[-1])
    if cos2.shape != sin2.shape or cos2.shape[1] != D // 2:
        raise ValueError(f"rotary tables must be (T, {D // 2}); got {tuple(cos.shape)}, {tuple(sin.shape)}")
    if cos2.dtype != sin2.dtype:
        raise TypeError("cos and sin must have the same dtype")
    if not cos2.is_contiguous() or cos2.data_ptr() % 16 != 0:
        cos2 = cos2.clone(memory_format=torch.contiguous_format)
    if not sin2.is_contiguous() or sin2.data_ptr() % 16 != 0:
        sin2 = sin2.clone(memory_format=torch.contiguous_format)
    a, out, dev, _ = _attn_call("flash_attn_with_kvcache_rope", q, k_cache, v_cache, k, v, cache_seqlens, causal,
                                window_size, keys_per_split, cache_batch_idx, cu_seqlens_q, max_seqlen_q,
                                page_table)
    _require_gpu("flash_attn_with_kvcache_rope", cos2, sin2)
    pro = _ext.QKPrologue()
    pro.cos, pro.sin = cos2.data_ptr(), sin2.data_ptr()
    pro.rot_len = cos2.shape[0]
    pro.rot_dtype = _dtype_code(cos2, "cos")
    pro.qk_scale = float(qk_scale)
    pro.eps = float(torch.finfo(q.dtype).eps if eps is None else eps)
    L = _ext.lib()
    ref = ctypes.byref(a)
    stream = _ext.stream_handle(dev)
    _attach_workspace(a, dev, stream, L.nc_attn_rope_workspace_bytes(ref))
    _ext.check(L.nc_attn_kvcache_rope(ref, ctypes.byref(pro), stream), "nc_attn_kvcache_rope")
    _check_device_errors("flash_attn_with_kvcache_rope", dev)
    return out


def flash_attn_func(q, k, v, causal=False, window_size=(-1, -1)):
    """Forward-only attention without a cache (nanochat/flash_attention.py:107-128).

    Runs the cache kernel with k/v as a filled cache and zero positions, which
    is exactly the reference's causal/windowed mask.  Training (autograd) is
    not part of this library.
    """
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise NotImplementedError("flash_attn_func: backward is not implemented by the MI355X KV-cache library")
    B = q.shape[0]
    zeros = torch.zeros(B, dtype=torch.int32, device=q.device)
    return flash_attn_with_kvcache(q, k, v, cache_seqlens=zeros, causal=causal, window_size=window_size)


def kv_append(k_cache, v_cache, k, v, cache_seqlens):
    """Standalone ragged append (the first half of flash_attn_with_kvcache)."""
    B, T_new, H_kv, D = k.shape
    _, T_max, _, _ = k_cache.shape
    dev = _require_gpu("kv_append", k_cache, v_cache, k, v, cache_seqlens)
    if tuple(v.shape) != tuple(k.shape) or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("kv_append: k/v and k_cache/v_cache shapes must match")
    if k_cache.shape[0] != B or k_cache.shape[2] != H_kv or k_cache.shape[3] != D:
        raise ValueError("kv_append: k does not match the cache shape")
    if k.dtype != v.dtype or k_cache.dtype != v_cache.dtype:
        raise TypeError("kv_append: k/v dtypes and cache dtypes must match pairwise")
    a = _ext.AppendArgs()
    a.k_cache = k_cache.data_ptr(); a.v_cache = v_cache.data_ptr()
    a.k = k.data_ptr(); a.v = v.data_ptr()
    a.cache_seqlens = cache_seqlens.data_ptr()
    a.error_flag = _ext.error_flag(dev).data_ptr()
    a.batch, a.t_new, a.t_max, a.n_kv_heads, a.head_dim = B, T_new, T_max, H_kv, D
    a.kc_stride_b, a.kc_stride_t, a.kc_stride_h = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.vc_stride_b, a.vc_stride_t, a.vc_stride_h = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    a.k_stride_b, a.k_stride_t, a.k_stride_h = k.stride(0), k.stride(1), k.stride(2)
    a.v_stride_b, a.v_stride_t, a.v_stride_h = v.stride(0), v.stride(1), v.stride(2)
    a.in_dtype = _dtype_code(k, "k")
    a.cache_dtype = _dtype_code(k_cache, "k_cache")
    _ext.check(_ext.lib().nc_kv_append(ctypes.byref(a), _ext.stream_handle(dev)), "nc_kv_append")


flash_attn = SimpleNamespace(
    flash_attn_func=flash_attn_func,
    flash_attn_with_kvcache=flash_attn_with_kvcache,
    flash_attn_with_kvcache_rope=flash_attn_with_kvcache_rope,
)
