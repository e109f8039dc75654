"""CPU restatement of nanochat's inference KV-cache path -- TEST INFRASTRUCTURE.

This module is the parity checker for the HIP library.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only as the checker or as the timed CPU baseline; the product (nanochat_amd/)
never imports it.

It restates, with the same torch operations the reference uses:
  - _sdpa_attention            nanochat/flash_attention.py:69-102
  - flash_attn_func            nanochat/flash_attention.py:107-128
  - flash_attn_with_kvcache    nanochat/flash_attention.py:155-177, applied row
                               by row with each row's own cache_seqlens[b] (FA3's
                               per-row contract, nanochat/engine.py:84-90); for a
                               uniform batch this is the reference fallback itself
  - KVCache                    nanochat/engine.py:82-137
  - compute_window_sizes       nanochat/gpt.py:285-312
  - rotary / qk_prologue       nanochat/gpt.py:57-63 (apply_rotary_emb), :42-43
                               (norm), :98-102 (rotary, QK norm, x1.2) with each
                               row's own position s_b (the fused prologue's contract;
                               the reference slices the table at row 0's position)
  - rotary_tables              nanochat/gpt.py:268-283
  - cache_batch_idx            FA3's flash_attn_with_kvcache argument, reached through
                               nanochat/flash_attention.py:149-153 (the FA3 branch;
                               flash-attention 3 from the 'varunneal/flash-attention-3'
                               kernel-hub build, not vendored): batch row b reads and
                               appends cache row cache_batch_idx[b]; cache_seqlens
                               stays indexed by b.  Pinned by the permutation
                               identity in tests/test_oracle.py (no golden vectors:
                               the reference never passes it).
  - page_table                 FA3's paged KV cache through the same branch: caches
                               are (num_blocks, P, H_kv, D) blocks, position j of row b
                               is slot j % P of block page_table[b, j // P]; restated as
                               the call on the rows the table assembles (gather), written
                               back block by block.  Pinned by the block-shuffle identity
                               in tests/test_oracle.py (a dense cache cut into blocks and
                               stored in a shuffled pool gives the dense call's results).
  - cu_seqlens_q               FA3's varlen layout through the same branch: packed
                               tokens, row b owning [cu[b], cu[b+1]); restated as one
                               call per row of the function above, pinned by the
                               uniform-length and per-row identities in
                               tests/test_oracle.py.
The pins for each function (brute force, closed forms, the reference's own
known-answer test) live in tests/test_oracle.py.

Mixed dtypes (F7 of the path analysis: fp32 compute with a bf16 cache on the
GPU) are defined as: k/v are rounded into the cache dtype on store (torch
copy_ semantics), the cache is upcast to q's dtype for attention, and the
output has q's dtype.  ``compute_dtype`` lets a test run the same algorithm
in float32 or float64 as the high-precision reference.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def sdpa_attention(q, k, v, window_size, enable_gqa):
    """nanochat/flash_attention.py:69-102.  q, k, v are (B, H, T, D)."""
    Tq = q.size(2)
    Tk = k.size(2)
    window = window_size[0]
    # :78-80 full context, same length
    if (window < 0 or window >= Tq) and Tq == Tk:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=enable_gqa)
    # :82-89 single query: keep the last window+1 keys
    if Tq == 1:
        if 0 <= window < Tk:
            start = max(0, Tk - (window + 1))
            k = k[:, :, start:, :]
            v = v[:, :, start:, :]
        return F.scaled_dot_product_attention(q, k, v, is_causal=False, enable_gqa=enable_gqa)
    # :91-102 explicit bottom-right aligned causal (+ window) mask
    row_idx = (Tk - Tq) + torch.arange(Tq, device=q.device).unsqueeze(1)
    col_idx = torch.arange(Tk, device=q.device).unsqueeze(0)
    mask = col_idx <= row_idx
    if 0 <= window < Tk:
        mask = mask & ((row_idx - col_idx) <= window)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=enable_gqa)


def flash_attn_func(q, k, v, causal=False, window_size=(-1, -1)):
    """nanochat/flash_attention.py:107-128 (the SDPA fallback): (B, T, H, D) in and out."""
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    y = sdpa_attention(q, k, v, window_size, q.size(1) != k.size(1))
    return y.transpose(1, 2)


def kv_append(k_cache, v_cache, k, v, cache_seqlens):
    """In-place append at each row's position: nanochat/flash_attention.py:160-162 per row."""
    T_new = k.size(1)
    for b in range(k.size(0)):
        pos = int(cache_seqlens[b])
        k_cache[b, pos:pos + T_new, :, :] = k[b]
        v_cache[b, pos:pos + T_new, :, :] = v[b]


def paged_to_dense(cache_blocks, page_table):
    """(num_blocks, P, H, D) blocks and a (B, nb) table -> (B, nb * P, H, D) row caches (a copy)."""
    B, nb = page_table.shape
    P = cache_blocks.shape[1]
    return cache_blocks[page_table.long()].reshape(B, nb * P, *cache_blocks.shape[2:])


def dense_to_paged(dense, cache_blocks, page_table):
    """Write (B, nb * P, H, D) row caches back into the blocks their table names."""
    B, nb = page_table.shape
    P = cache_blocks.shape[1]
    for b in range(B):
        for j in range(nb):
            cache_blocks[int(page_table[b, j])] = dense[b, j * P:(j + 1) * P]


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                            causal=False, window_size=(-1, -1), compute_dtype=None, cache_batch_idx=None,
                            cu_seqlens_q=None, page_table=None):
    """nanochat/flash_attention.py:155-177, one batch row at a time.

    Mutates k_cache/v_cache like the reference.  ``compute_dtype`` (default:
    q's dtype) is the dtype q and the cache slices are cast to before SDPA;
    the result is returned in q's dtype.  ``cache_batch_idx`` (FA3): row b
    uses cache row cache_batch_idx[b].  ``cu_seqlens_q`` (FA3 varlen): q, k, v
    are packed tokens (total_q, H, D) and row b owns [cu[b], cu[b+1]); the
    output is packed the same way.  ``page_table`` (FA3's paged cache): the
    caches are (num_blocks, P, H, D) blocks and position j of row b is slot
    j % P of block page_table[b, j // P]; restated as the call on the rows the
    table assembles, written back block by block.
    """
    if page_table is not None:
        kd, vd = paged_to_dense(k_cache, page_table), paged_to_dense(v_cache, page_table)
        y = flash_attn_with_kvcache(q, kd, vd, k=k, v=v, cache_seqlens=cache_seqlens, causal=causal,
                                    window_size=window_size, compute_dtype=compute_dtype,
                                    cu_seqlens_q=cu_seqlens_q)
        dense_to_paged(kd, k_cache, page_table)
        dense_to_paged(vd, v_cache, page_table)
        return y
    if cu_seqlens_q is not None:
        outs = []
        for b in range(len(cu_seqlens_q) - 1):
            a, e = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
            if e == a:
                continue
            c = int(cache_batch_idx[b]) if cache_batch_idx is not None else b
            y = flash_attn_with_kvcache(q[a:e].unsqueeze(0), k_cache, v_cache,
                                        k=k[a:e].unsqueeze(0) if k is not None else None,
                                        v=v[a:e].unsqueeze(0) if v is not None else None,
                                        cache_seqlens=cache_seqlens[b:b + 1], causal=causal,
                                        window_size=window_size, compute_dtype=compute_dtype,
                                        cache_batch_idx=torch.tensor([c], dtype=torch.int32))
            outs.append(y[0])
        return torch.cat(outs, dim=0) if outs else q.new_empty((0,) + tuple(q.shape[1:]))
    B, T_new, H, D = q.shape
    cdt = compute_dtype if compute_dtype is not None else q.dtype
    outs = []
    for b in range(B):
        pos = int(cache_seqlens[b])
        c = int(cache_batch_idx[b]) if cache_batch_idx is not None else b
        if k is not None and v is not None:
            k_cache[c:c + 1, pos:pos + T_new, :, :] = k[b:b + 1]
            v_cache[c:c + 1, pos:pos + T_new, :, :] = v[b:b + 1]
        end_pos = pos + T_new
        k_full = k_cache[c:c + 1, :end_pos, :, :].to(cdt)
        v_full = v_cache[c:c + 1, :end_pos, :, :].to(cdt)
        q_sdpa = q[b:b + 1].to(cdt).transpose(1, 2)
        k_sdpa = k_full.transpose(1, 2)
        v_sdpa = v_full.transpose(1, 2)
        enable_gqa = q_sdpa.size(1) != k_sdpa.size(1)
        y = sdpa_attention(q_sdpa, k_sdpa, v_sdpa, window_size, enable_gqa)
        outs.append(y.transpose(1, 2))
    return torch.cat(outs, dim=0).to(q.dtype)


class KVCache:
    """nanochat/engine.py:82-137 (CPU or any torch device)."""

    def __init__(self, batch_size, num_heads, seq_len, head_dim, num_layers, device, dtype):
        self.batch_size = batch_size
        self.max_seq_len = seq_len
        self.n_layers = num_layers
        self.n_heads = num_heads
        self.head_dim = head_dim
        self.k_cache = torch.zeros(num_layers, batch_size, seq_len, num_heads, head_dim, device=device, dtype=dtype)
        self.v_cache = torch.zeros(num_layers, batch_size, seq_len, num_heads, head_dim, device=device, dtype=dtype)
        self.cache_seqlens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self.prev_embedding = None

    def reset(self):
        self.cache_seqlens.zero_()
        self.prev_embedding = None

    def get_pos(self):
        return self.cache_seqlens[0].item()

    def get_layer_cache(self, layer_idx):
        return self.k_cache[layer_idx], self.v_cache[layer_idx]

    def advance(self, num_tokens):
        self.cache_seqlens += num_tokens

    def prefill(self, other):
        assert self.get_pos() == 0, "Cannot prefill a non-empty KV cache"
        assert self.n_layers == other.n_layers and self.n_heads == other.n_heads and self.head_dim == other.head_dim
        assert self.max_seq_len >= other.max_seq_len
        other_pos = other.get_pos()
        self.k_cache[:, :, :other_pos, :, :] = other.k_cache[:, :, :other_pos, :, :]
        self.v_cache[:, :, :other_pos, :, :] = other.v_cache[:, :, :other_pos, :, :]
        self.cache_seqlens.fill_(other_pos)
        if other.prev_embedding is not None:
            self.prev_embedding = other.prev_embedding.expand(self.batch_size, -1, -1).clone()


def compute_window_sizes(sequence_len, window_pattern, n_layer):
    """nanochat/gpt.py:285-312: per-layer (left, right) windows, last layer long."""
    pattern = window_pattern.upper()
    assert all(c in "SL" for c in pattern), f"Invalid window_pattern: {pattern}. Use only S and L."
    long_window = sequence_len
    short_window = -(-long_window // 4 // 128) * 128
    char_to_window = {"L": (long_window, 0), "S": (short_window, 0)}
    sizes = [char_to_window[pattern[i % len(pattern)]] for i in range(n_layer)]
    sizes[-1] = (long_window, 0)
    return sizes


def decode_bytes(seqlens, n_layers, n_heads, n_kv_heads, head_dim, elem_bytes, windows=None):
    """Algorithmic HBM bytes of one decode step (T_new = 1) over all layers.

    Per layer and row: K and V of n_keys cached/new tokens read once, the new
    K and V token written once, q read and the output written once, with
    n_keys = min(s_b + 1, w + 1) (w < 0: s_b + 1).
    """
    total = 0
    kv_tok = 2 * n_kv_heads * head_dim * elem_bytes
    qo = 2 * n_heads * head_dim * elem_bytes
    for layer in range(n_layers):
        w = -1 if windows is None else windows[layer]
        for s in seqlens:
            s = int(s)
            n_keys = s + 1 if w < 0 else min(s + 1, w + 1)
            total += kv_tok * n_keys + kv_tok + qo
    return total


def softmax_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)


def rotary_tables(seq_len, head_dim, base=100000, dtype=torch.float32):
    """nanochat/gpt.py:268-283: cos/sin of t * base^(-2i/D), shape (seq_len, D/2), cast to dtype."""
    channel_range = torch.arange(0, head_dim, 2, dtype=torch.float32)
    inv_freq = 1.0 / (base ** (channel_range / head_dim))
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def rotary(x, cos, sin):
    """nanochat/gpt.py:57-63 on (B, T, H, D) with cos/sin broadcastable to (B, T, 1, D/2)."""
    d = x.shape[3] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * cos + x2 * sin, x1 * (-sin) + x2 * cos], 3)


def qk_prologue(x, cos_tab, sin_tab, positions, scale=1.2, eps=None):
    """Rotary at each row's positions, RMS norm over D, times scale (nanochat/gpt.py:98-102).

    x is (B, T, H, D); token t of row b uses table row positions[b] + t.  Every
    operation runs in x's dtype, as the reference's do in COMPUTE_DTYPE.
    """
    T = x.shape[1]
    idx = positions.long()[:, None] + torch.arange(T)[None, :]
    cos = cos_tab[idx][:, :, None, :].to(x.dtype)
    sin = sin_tab[idx][:, :, None, :].to(x.dtype)
    y = rotary(x, cos, sin)
    y = F.rms_norm(y, (y.size(-1),), eps=eps)
    return y * scale
