/*
 * nc_kv.h -- C ABI of libnc_kv.so, the MI355X (gfx950) KV-cache inference path.
 *
 * The library replaces the compute inside nanochat's inference KV-cache path:
 *   - nanochat/flash_attention.py:131-177  flash_attn_with_kvcache (append + attention)
 *   - nanochat/flash_attention.py:69-102   _sdpa_attention masks (causal, sliding window, GQA)
 *   - nanochat/engine.py:123-137           KVCache.prefill (broadcast fan-out copy)
 *   - nanochat/gpt.py:45-50, 468-472       the decode step's linear layers and logits head
 * Host code (Python, ctypes) validates shapes and dtypes, then calls these
 * functions with raw device pointers, element strides and the caller's stream.
 *
 * Conventions
 *   - Every pointer is a device pointer (hipMalloc'd / torch CUDA tensor data).
 *   - Strides are in ELEMENTS of the tensor they describe; the innermost
 *     (head_dim) stride is always 1.
 *   - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *   - Nothing here synchronises the host or allocates memory.
 *   - Return value: NC_OK (0) or an nc_status code; nc_strerror() names it.
 */
#ifndef NC_KV_H
#define NC_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_KV_ABI_VERSION 8

/* Element types (the torch dtypes the reference path uses). */
enum nc_dtype {
  NC_DTYPE_F32 = 0,
  NC_DTYPE_F16 = 1,
  NC_DTYPE_BF16 = 2
};

enum nc_status {
  NC_OK = 0,
  NC_ERR_NULL_ARG = 1,          /* a required pointer is NULL               */
  NC_ERR_BAD_SHAPE = 2,         /* a size is <= 0 or inconsistent           */
  NC_ERR_DTYPE = 3,             /* unsupported dtype combination            */
  NC_ERR_HEAD_DIM = 4,          /* head_dim not in the compiled set         */
  NC_ERR_ALIGNMENT = 5,         /* pointer / stride not 16-byte aligned     */
  NC_ERR_WORKSPACE = 6,         /* workspace NULL or smaller than required  */
  NC_ERR_LAUNCH = 7,            /* hipLaunchKernel / hipGetLastError failed */
  NC_ERR_SCRATCH_LIMIT = 8      /* nc_attn_kvcache_noalloc: the call needs more than
                                   NC_NOALLOC_SCRATCH_BYTES of scratch */
};

/* Bit set in *error_flag by a kernel when a row would write past t_max
 * (cache_seqlens[b] + t_new > t_max).  Such writes are skipped, never done
 * out of bounds.  The reference raises a torch size-mismatch RuntimeError at
 * nanochat/flash_attention.py:161 for the same condition. */
#define NC_DEVERR_OVERFLOW 1

/* Bit set in *error_flag when cache_batch_idx[b] is outside [0, cache_batch).
 * Nothing of batch row b is read, written or stored.  FA3's
 * flash_attn_with_kvcache indexes the cache with it unchecked. */
#define NC_DEVERR_BATCH_IDX 4

/* Bit set in *error_flag when row b's tokens [cu_seqlens_q[b],
 * cu_seqlens_q[b+1]) are not a range inside [0, total_q) of at most t_new
 * (max_seqlen_q) tokens.  Nothing of that row is read, written or stored. */
#define NC_DEVERR_QLEN 8

/* cu_seqlens_q (optional, FA3's varlen layout): q, k, v and out hold packed
 * tokens (total_q, H or H_kv, D); batch row b owns tokens [cu_seqlens_q[b],
 * cu_seqlens_q[b+1]) and appends them at cache_seqlens[b].  t_new is then the
 * bound max_seqlen_q, the *_stride_b fields are ignored, and out is
 * (total_q, H, D) contiguous.  A batch may mix rows of 0, 1 and many tokens.
 *
 * cache_batch_idx (optional, FA3's flash_attn_with_kvcache argument): batch
 * row b reads and appends cache row cache_batch_idx[b] instead of row b;
 * cache_seqlens stays indexed by b.  cache_batch is the number of cache rows.
 * With k/v given the indices must be distinct (rows sharing a cache row race,
 * as in FA3).
 *
 * page_table (optional, FA3's paged KV cache; not together with
 * cache_batch_idx): k_cache / v_cache are (num_blocks, page_size, H_kv, D)
 * blocks, and logical position j of batch row b is slot j % page_size of
 * block page_table[b * page_table_stride + j / page_size].  t_max is the
 * logical capacity of a row (at most page_table_stride * page_size);
 * kc_stride_b / vc_stride_b are the block strides and must equal page_size
 * times kc_stride_t / vc_stride_t.  page_size is a power of two, at least 16.
 * A table entry outside [0, num_blocks) is never dereferenced: that key is
 * not read or stored, the row's output is undefined, and NC_DEVERR_PAGE is
 * set. */
#define NC_DEVERR_PAGE 32

/* ---------------------------------------------------------------------------
 * Ragged KV append: k_cache[b, cache_seqlens[b] + t] = k[b, t] (and v), t < t_new.
 * Replaces nanochat/flash_attention.py:160-162 with FA3's per-row positions
 * (the fallback uses row 0's position for every row).  Values are converted
 * to the cache dtype with round-to-nearest-even (NaN -> canonical quiet NaN),
 * exactly as torch's copy_ does.  cache_seqlens is read, never written.
 * ------------------------------------------------------------------------- */
typedef struct nc_append_args {
  void* k_cache;                 /* (B, T_max, H_kv, D) */
  void* v_cache;
  const void* k;                 /* (B, T_new, H_kv, D) */
  const void* v;
  const int32_t* cache_seqlens;  /* (B,) */
  int32_t* error_flag;           /* optional (NULL): NC_DEVERR_* bits are OR-ed in */
  const int32_t* cache_batch_idx;  /* (B,) or NULL (row b is cache row b) */
  int64_t cache_batch;           /* cache rows (with cache_batch_idx) */
  const int32_t* cu_seqlens_q;   /* (B+1,) or NULL: packed new tokens */
  int64_t total_q;               /* tokens in k, v (with cu_seqlens_q) */
  const int32_t* page_table;     /* (B, page_table_stride) or NULL: paged cache */
  int64_t page_table_stride, page_size, num_blocks;
  int64_t batch, t_new, t_max, n_kv_heads, head_dim;
  int64_t kc_stride_b, kc_stride_t, kc_stride_h;
  int64_t vc_stride_b, vc_stride_t, vc_stride_h;
  int64_t k_stride_b, k_stride_t, k_stride_h;
  int64_t v_stride_b, v_stride_t, v_stride_h;
  int32_t in_dtype;              /* dtype of k, v */
  int32_t cache_dtype;           /* dtype of k_cache, v_cache */
} nc_append_args;

int nc_kv_append(const nc_append_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Prefill fan-out: for every layer l and destination row n < n_rows,
 *   dst[l, n, 0:prefix_len] = src[l, 0, 0:prefix_len]     (K and V)
 * and, if dst_seqlens != NULL, dst_seqlens[n] = prefix_len.
 * Replaces nanochat/engine.py:132-134.  One launch covers K and V of every
 * layer; each source byte is read once and written n_rows times.
 * Each [l, row, 0:prefix_len] region must be contiguous (row_elems = H_kv*D
 * elements per token), which holds for KVCache's (L, B, T, H_kv, D) slabs.
 * ------------------------------------------------------------------------- */
typedef struct nc_fanout_args {
  const void* k_src;             /* (L, 1, T_src, H_kv, D) */
  const void* v_src;
  void* k_dst;                   /* (L, N, T_dst, H_kv, D) */
  void* v_dst;
  int32_t* dst_seqlens;          /* optional (N,) */
  int64_t n_layers, n_rows, prefix_len, row_elems;
  int64_t src_stride_l;          /* elements between layers of src        */
  int64_t dst_stride_l;          /* elements between layers of dst        */
  int64_t dst_stride_b;          /* elements between rows of dst          */
  int32_t dtype;                 /* same dtype for src and dst            */
} nc_fanout_args;

int nc_kv_fanout(const nc_fanout_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * flash_attn_with_kvcache: optional append of (k, v) at cache_seqlens, then
 *   out[b,i,h] = softmax_j( q[b,i,h] . K[b,j,h/G] * scale ) . V[b,j,h/G]
 * over keys j with  j <= s_b + i  and  (window_left < 0 || s_b + i - j <= window_left),
 * where s_b = cache_seqlens[b] and G = n_heads / n_kv_heads.
 * This is nanochat/flash_attention.py:155-177 + :69-102 (queries bottom-right
 * aligned, row_idx = Tk - Tq + i) applied with each row's own s_b.
 * `causal` is accepted and, like the reference fallback, does not change the
 * mask.  Output is (B, T_new, H, D), contiguous, in q's dtype; accumulation
 * is fp32.  The fused path (t_new == 1) appends and attends in one launch;
 * t_new > 1 appends first and then attends (two launches, same stream).
 * When a row's keys span several splits, partial results go to the workspace
 * (nc_attn_workspace_bytes; 0 bytes when every row fits one split) and are
 * merged by the last split of each (row, query, head block) in the same
 * launch, or by a second small kernel (chunk splits; more than
 * NC_WORKSPACE_SYNC_BYTES / 4 groups).  A non-empty workspace begins with
 * NC_WORKSPACE_SYNC_BYTES of split counters: they must be zero before the
 * buffer's first use (e.g. allocate it zeroed), and every call leaves them
 * zero; the rest needs no initialisation.  Calls sharing a workspace must not
 * overlap in time (use one per stream).
 * ------------------------------------------------------------------------- */
typedef struct nc_attn_args {
  const void* q;                 /* (B, T_new, H, D) */
  void* out;                     /* (B, T_new, H, D) contiguous */
  void* k_cache;                 /* (B, T_max, H_kv, D) */
  void* v_cache;
  const void* k;                 /* (B, T_new, H_kv, D) or NULL (no append) */
  const void* v;
  const int32_t* cache_seqlens;  /* (B,) read-only */
  int32_t* error_flag;           /* optional */
  const int32_t* cache_batch_idx;  /* (B,) or NULL (row b is cache row b) */
  int64_t cache_batch;           /* cache rows (with cache_batch_idx) */
  const int32_t* cu_seqlens_q;   /* (B+1,) or NULL: packed query tokens */
  int64_t total_q;               /* tokens in q, k, v, out (with cu_seqlens_q) */
  const int32_t* page_table;     /* (B, page_table_stride) or NULL: paged cache */
  int64_t page_table_stride, page_size, num_blocks;
  void* workspace;
  size_t workspace_bytes;
  int64_t batch, t_new, t_max, n_heads, n_kv_heads, head_dim;
  int64_t q_stride_b, q_stride_t, q_stride_h;
  int64_t kc_stride_b, kc_stride_t, kc_stride_h;
  int64_t vc_stride_b, vc_stride_t, vc_stride_h;
  int64_t k_stride_b, k_stride_t, k_stride_h;
  int64_t v_stride_b, v_stride_t, v_stride_h;
  int32_t window_left;           /* < 0: unlimited */
  int32_t causal;
  float softmax_scale;           /* > 0, finite (nanochat: head_dim ** -0.5) */
  int32_t q_dtype;               /* dtype of q, k, v and out */
  int32_t cache_dtype;
  int32_t keys_per_split;        /* keys one workgroup covers before a split-K merge;
                                    0: library default; else a multiple of 64 */
} nc_attn_args;

/* Leading bytes of every non-empty workspace that hold split counters
 * (zero before first use, left zero by every call). */
#define NC_WORKSPACE_SYNC_BYTES 65536

/* Bytes of workspace nc_attn_kvcache needs for these arguments. */
size_t nc_attn_workspace_bytes(const nc_attn_args* args);

int nc_attn_kvcache(const nc_attn_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * nc_attn_kvcache_noalloc: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The same call as nc_attn_kvcache
 * (same kernels, plans and results), except that its split-K scratch (split
 * counters and partials) lives in a device array of the library, of
 * NC_NOALLOC_SCRATCH_BYTES on each GPU it runs on, held until the process
 * ends; args->workspace and args->workspace_bytes are ignored.  It calls no
 * hipMalloc / hipFree.  A call needing more scratch than that
 * (nc_attn_workspace_bytes(args) > NC_NOALLOC_SCRATCH_BYTES) returns
 * NC_ERR_SCRATCH_LIMIT and launches nothing.  Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (other streams,
 * other host threads) race and must be serialised by the caller.  The first
 * call on a GPU looks the array up and launches one small kernel on `stream`
 * that zeroes its split counters; every call leaves them zero.
 * ------------------------------------------------------------------------- */
#define NC_NOALLOC_SCRATCH_BYTES (64 << 20)

int nc_attn_kvcache_noalloc(const nc_attn_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * QK prologue fused into the call: nanochat/gpt.py:98-102 (rotary, QK RMS
 * norm, x qk_scale), which the reference computes with separate torch ops
 * before flash_attn_with_kvcache (gpt.py:112-118), applied here to the raw q
 * and k projections with each row's position from cache_seqlens:
 *   token t of row b uses table row r = cache_seqlens[b] + t;
 *   y1 = x1 cos[r] + x2 sin[r],  y2 = -x1 sin[r] + x2 cos[r]
 *        (x1, x2: dims [0, D/2) and [D/2, D); nanochat/gpt.py:57-63);
 *   y  = qk_scale * y / sqrt(mean(y^2) + eps)            (gpt.py:42-43).
 * q is transformed for the attention only (rounded to q's dtype); k is
 * transformed, rounded to the cache dtype (RNE) and appended with v, which is
 * appended unchanged.  Arithmetic is fp32 with one rounding at the end (the
 * reference rounds after every op in its compute dtype).  The reference
 * slices the tables at row 0's position (gpt.py:424-425); per-row positions
 * equal that for uniform batches.  A table row at or past rot_len is read as
 * row rot_len - 1 and sets NC_DEVERR_ROPE_RANGE (the reference asserts,
 * gpt.py:420).  k and v are required.  T_new == 1 runs in the decode kernel
 * itself; T_new > 1 runs a prologue kernel (q into the workspace, k/v into
 * the cache) and then the attention of nc_attn_kvcache without append.
 * ------------------------------------------------------------------------- */
#define NC_DEVERR_ROPE_RANGE 2

typedef struct nc_qk_prologue {
  const void* cos;               /* (rot_len, head_dim / 2), contiguous, 16-byte aligned (gpt.py:268-283) */
  const void* sin;
  int64_t rot_len;
  int32_t rot_dtype;             /* dtype of cos / sin */
  float qk_scale;                /* nanochat: 1.2 */
  float eps;                     /* rms_norm eps: torch.finfo(compute dtype).eps */
} nc_qk_prologue;

/* Bytes of workspace nc_attn_kvcache_rope needs (>= nc_attn_workspace_bytes). */
size_t nc_attn_rope_workspace_bytes(const nc_attn_args* args);

int nc_attn_kvcache_rope(const nc_attn_args* args, const nc_qk_prologue* prologue, void* stream);

/* ---------------------------------------------------------------------------
 * Small-M linear layer of the decode step: y = x W^T (bias-free), for the
 * projections nanochat runs on a (B, 1, C) activation with F.linear
 * (nanochat/gpt.py:45-50 Linear.forward; callers gpt.py:87-89 c_q/c_k/c_v,
 * :125 c_proj, :136-138 MLP, :469 lm_head).  x is (m, k), W is
 * (n, k) (nn.Linear's layout), y is (m, n); m <= 64.  Accumulation is fp32
 * with one rounding at the end (round to nearest even).  x and W have the
 * same dtype (bf16 or fp16); y is that dtype or fp32.
 *
 * softcap > 0 selects the logits head of gpt.py:468-472 instead: the fp32
 * accumulator is rounded to x's dtype (the lm_head output), widened, and
 * y (fp32) = softcap * tanh(v * (1 / softcap)) -- the operations torch runs
 * for `softcap * torch.tanh(logits.float() / softcap)`.  Passing n = the
 * vocabulary size (not the padded row count of W) gives the sliced logits
 * `[..., :vocab_size]` directly.
 *
 * With few 64-column blocks, K is split: for m <= 32 over the waves of one
 * workgroup (no workspace), otherwise over workgroups.  In that case
 * nc_linear_workspace_bytes() is non-zero and the workspace follows the same
 * rule as nc_attn_kvcache's (first NC_WORKSPACE_SYNC_BYTES zero before the
 * first call, left zero by every call).  Results do not depend on the order
 * in which workgroups run.
 * ------------------------------------------------------------------------- */
typedef struct nc_linear_args {
  const void* x;                 /* (m, k), rows x_stride_m elements apart, 16-byte aligned */
  const void* w;                 /* (n, k), rows w_stride_n elements apart, 16-byte aligned */
  void* y;                       /* (m, n), rows y_stride_m elements apart */
  void* workspace;
  size_t workspace_bytes;
  int64_t m, n, k;               /* 1 <= m <= 64; k a multiple of 8 */
  int64_t x_stride_m, w_stride_n, y_stride_m;
  int32_t dtype;                 /* x and w: NC_DTYPE_BF16 or NC_DTYPE_F16 */
  int32_t y_dtype;               /* dtype, or NC_DTYPE_F32; NC_DTYPE_F32 when softcap > 0 */
  float softcap;                 /* 0: plain linear */
} nc_linear_args;

/* Bytes of workspace nc_linear needs for these sizes (0: none). */
size_t nc_linear_workspace_bytes(int64_t m, int64_t n, int64_t k);

int nc_linear(const nc_linear_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Next-token sampling, one launch for the batch (nanochat/engine.py:141-156
 * sample_next_token, applied to the fp32 logits of gpt.py:472):
 *   temperature == 0: argmax of each row (first maximum; NaN counts as the
 *     maximum, as torch.argmax does);
 *   0 < top_k < vocab: the top_k largest logits (equal values at the cut:
 *     lower indices first), softmax of logit / temperature over them, one
 *     categorical draw;
 *   otherwise: softmax of logit / temperature over the whole row, one draw.
 * The draw is the inverse CDF at uniforms[b] in [0, 1): the first category
 * whose running sum of exp(x - max) exceeds u times the total, categories in
 * torch.topk's order (value descending) for top-k and in index order for the
 * whole row.  The reference draws with torch.multinomial and its generator:
 * the distribution is the same, the stream of draws is the caller's.  NaN
 * logits are never drawn; a row with no finite logit yields 0 and sets
 * NC_DEVERR_SAMPLE (torch.multinomial raises for it).
 * ------------------------------------------------------------------------- */
#define NC_DEVERR_SAMPLE 16

typedef struct nc_sample_args {
  const float* logits;           /* (batch, vocab) fp32, rows logits_stride elements apart (0: one row for all) */
  const float* uniforms;         /* (batch,): one draw per row (unused when temperature == 0) */
  int64_t* out;                  /* (batch,) token ids */
  int32_t* error_flag;           /* optional (NULL): NC_DEVERR_SAMPLE is OR-ed in */
  int64_t batch, vocab, logits_stride;
  float temperature;             /* >= 0 */
  int32_t top_k;                 /* 0 or >= vocab: whole row; else at most 1024 */
} nc_sample_args;

int nc_sample(const nc_sample_args* args, void* stream);

/* Name of an nc_status code (static string). */
const char* nc_strerror(int status);

/* NC_KV_ABI_VERSION of the built library. */
int nc_abi_version(void);

/* Non-zero if the library was built with kernels for `head_dim`. */
int nc_supports_head_dim(int64_t head_dim);

#ifdef __cplusplus
}
#endif

#endif /* NC_KV_H */
