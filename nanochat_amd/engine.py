"""KV cache and inference engine with nanochat's interfaces, MI355X-native.

``KVCache`` keeps the surface of nanochat/engine.py:82-137 (attributes
k_cache, v_cache, cache_seqlens, prev_embedding, n_layers, max_seq_len and the
methods reset / get_pos / get_layer_cache / advance / prefill).  The fan-out
copy in ``prefill`` is one HIP launch (nc_kv_fanout) that reads the prefilled
row once and writes it into every destination row, K and V of all layers,
and sets cache_seqlens on the device.
"""
from __future__ import annotations

import ctypes

import torch

from . import _ext


class KVCache:
    """Preallocated (L, B, T, H_kv, D) K and V caches plus per-row positions.

    Layout and dtype follow nanochat/engine.py:92-104: zero-filled, contiguous,
    layer outermost, so ``get_layer_cache(l)`` returns (B, T, H_kv, D) views
    that flash_attn_with_kvcache updates in place.
    """

    def __init__(self, batch_size, num_heads, seq_len, head_dim, num_layers, device, dtype):
        self.batch_size = batch_size
        self.max_seq_len = seq_len
        self.n_layers = num_layers
        self.n_heads = num_heads
        self.head_dim = head_dim
        shape = (num_layers, batch_size, seq_len, num_heads, head_dim)
        self.k_cache = torch.zeros(shape, device=device, dtype=dtype)
        self.v_cache = torch.zeros(shape, device=device, dtype=dtype)
        self.cache_seqlens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self.prev_embedding = None

    def reset(self):
        """Positions back to 0 (cache bytes are kept), nanochat/engine.py:106-109."""
        self.cache_seqlens.zero_()
        self.prev_embedding = None

    def get_pos(self):
        """Row 0's position (uniform-batch assumption of nanochat/engine.py:111-113)."""
        return self.cache_seqlens[0].item()

    def get_layer_cache(self, layer_idx):
        """(k_cache, v_cache) views of one layer, nanochat/engine.py:115-117."""
        return self.k_cache[layer_idx], self.v_cache[layer_idx]

    def advance(self, num_tokens):
        """cache_seqlens += num_tokens on the device, nanochat/engine.py:119-121."""
        self.cache_seqlens += num_tokens

    def prefill(self, other):
        """Copy other's first get_pos() positions into every row of this cache.

        Preconditions and effects of nanochat/engine.py:123-137: this cache is
        empty, layer/head/head_dim match, it is at least as long as `other`;
        afterwards every row holds other's row 0 prefix and cache_seqlens is
        other's position.  K and V of all layers move in one HIP launch.
        """
        assert self.get_pos() == 0, "Cannot prefill a non-empty KV cache"
        assert self.n_layers == other.n_layers and self.n_heads == other.n_heads and self.head_dim == other.head_dim
        assert self.max_seq_len >= other.max_seq_len
        other_pos = other.get_pos()
        if not 0 <= other_pos <= other.max_seq_len:
            raise ValueError(f"KVCache.prefill: source position {other_pos} outside [0, {other.max_seq_len}]")
        src_k, src_v, dst_k, dst_v = other.k_cache, other.v_cache, self.k_cache, self.v_cache
        dev = dst_k.device
        if dev.type != "cuda" or src_k.device != dev:
            raise RuntimeError("KVCache.prefill: the fan-out copy runs on the GPU only (both caches on one GPU)")
        if src_k.dtype != dst_k.dtype:
            raise TypeError(f"KVCache.prefill: cache dtypes differ ({src_k.dtype} vs {dst_k.dtype})")
        for t in (src_k, src_v, dst_k, dst_v):
            if not t.is_contiguous():
                raise ValueError("KVCache.prefill: caches must be contiguous")
        a = _ext.FanoutArgs()
        a.k_src, a.v_src = src_k.data_ptr(), src_v.data_ptr()
        a.k_dst, a.v_dst = dst_k.data_ptr(), dst_v.data_ptr()
        a.dst_seqlens = self.cache_seqlens.data_ptr()
        a.n_layers = self.n_layers
        a.n_rows = self.batch_size
        a.prefix_len = other_pos
        a.row_elems = self.n_heads * self.head_dim
        a.src_stride_l = src_k.stride(0)
        a.dst_stride_l = dst_k.stride(0)
        a.dst_stride_b = dst_k.stride(1)
        a.dtype = _ext.DTYPE_CODE[dst_k.dtype]
        _ext.check(_ext.lib().nc_kv_fanout(ctypes.byref(a), _ext.stream_handle(dev)), "nc_kv_fanout")
        if other.prev_embedding is not None:
            self.prev_embedding = other.prev_embedding.expand(self.batch_size, -1, -1).clone()
