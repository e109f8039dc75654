// C ABI entry points of libnc_kv.so: argument validation, launch planning and
// dispatch.  Nothing here allocates or synchronises.  The only mutable state is
// the per-device address of the no-allocation entry point's scratch array
// (set once per device, under a mutex).

#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "nc_kv.h"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

// Chunks of at least this many new tokens run on the MFMA chunk kernel.
constexpr int64_t kChunkMinTokens = 8;
// Chunk-kernel splits, used when a workgroup's span can exceed
// kChunkSplitAbove keys (shorter spans run unsplit: measured on MI355X, the
// merge launch costs more than the shorter critical path saves; d24 1024-token
// prefill: 0.65 ms unsplit, 0.86 ms at 512-key splits).  The split size is a
// multiple of kChunkSplitUnit chosen so that one row of the batch alone gives
// about kChunkWGPerRow workgroups: many q tiles and heads per row need few
// splits.  Measured (us per call): one 14k-key row, 16/4 heads x 128 tokens
// (32 workgroups per split): 94 at 512, 78 at 2048; 4/4 heads (8 per split):
// 34 at 512, 58 at 2048; C5's 16 chunk rows: 136 at 512, 121 at 2048.
constexpr int64_t kChunkSplitUnit = 512;
constexpr int64_t kChunkWGPerRow = 256;
constexpr int64_t kChunkSplitAbove = 2048;
// Default decode plans size their split count so the grid has about this
// many workgroups (long rows then take longer splits).
#ifndef NC_DECODE_GRID_TARGET
#define NC_DECODE_GRID_TARGET 4096
#endif
constexpr int64_t kDecodeGridTarget = NC_DECODE_GRID_TARGET;
// Decode with wide workgroups and no split: at most this many groups (one per
// CU) and this many keys per row.
constexpr int64_t kWideMinGroups = 128;
#ifndef NC_DECODE_WIDE_MAX_GROUPS
#define NC_DECODE_WIDE_MAX_GROUPS 256
#endif
constexpr int64_t kWideMaxGroups = NC_DECODE_WIDE_MAX_GROUPS;
constexpr int64_t kWideMaxKeys = 4096;
// Decode splits merged by their last workgroup (one uint32 ticket per group at
// the start of every non-empty workspace) instead of a merge launch, for grids
// of at most kMergeInKernelMaxWG workgroups.  Each workgroup then ends with a
// ticket round trip while holding its CU slot, which costs more than the
// merge launch once there are many workgroups per CU.  Measured on MI355X
// (us per call, merge launch -> in-kernel): d26 S layers (104 groups x 5
// splits) 15.3 -> 13.8; B=1 at 32k keys (10 x 129) 58.3 -> 52.5; d20 B=32
// at 1088 keys (320 x 5) 34.5 -> 33.7; but C2 (320 x 9) 39.5 -> 40.3 and
// B=32 at 4k keys (320 x 17) 108.4 -> 113.
#ifndef NC_DECODE_MERGE_IN_KERNEL
#define NC_DECODE_MERGE_IN_KERNEL 1  // 0: decode splits always use the merge launch
#endif
#ifndef NC_MERGE_IN_KERNEL_MAX_WG
#define NC_MERGE_IN_KERNEL_MAX_WG 2048
#endif
constexpr int64_t kMaxTickets = NC_WORKSPACE_SYNC_BYTES / 4;
constexpr int64_t kMergeInKernelMaxWG = NC_DECODE_MERGE_IN_KERNEL ? NC_MERGE_IN_KERNEL_MAX_WG : 0;

bool valid_dtype(int d) { return d == NC_DTYPE_F32 || d == NC_DTYPE_F16 || d == NC_DTYPE_BF16; }
int64_t dtype_bytes(int d) { return d == NC_DTYPE_F32 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A paged cache (page_table given): a power-of-two page of at least 16 tokens,
// blocks of page_size token rows, a table wide enough for t_max positions, and
// no cache_batch_idx beside it.
bool valid_pages(const int32_t* table, int64_t stride, int64_t page_size, int64_t num_blocks, int64_t t_max,
                 const int32_t* cache_batch_idx, int64_t kc_sb, int64_t kc_st, int64_t vc_sb, int64_t vc_st) {
  if (table == nullptr) return true;
  if (cache_batch_idx != nullptr) return false;
  if (page_size < 16 || page_size > (int64_t(1) << 24) || (page_size & (page_size - 1)) != 0) return false;
  if (num_blocks <= 0 || num_blocks > INT32_MAX || stride < (t_max + page_size - 1) / page_size) return false;
  return kc_sb == page_size * kc_st && vc_sb == page_size * vc_st;
}
bool strides16(int64_t ebytes, int64_t s0, int64_t s1, int64_t s2) {
  return (s0 * ebytes) % 16 == 0 && (s1 * ebytes) % 16 == 0 && (s2 * ebytes) % 16 == 0;
}
size_t round256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace

int plan_attention(const nc_attn_args& a, AttnPlan* plan) {
  if (a.batch <= 0 || a.t_new <= 0 || a.t_max <= 0 || a.n_heads <= 0 || a.n_kv_heads <= 0 ||
      a.head_dim <= 0) {
    return NC_ERR_BAD_SHAPE;
  }
  if (a.n_heads % a.n_kv_heads != 0) return NC_ERR_BAD_SHAPE;
  if (a.t_max > INT32_MAX / 2 || a.t_new > INT32_MAX / 2) return NC_ERR_BAD_SHAPE;
  if (!valid_dtype(a.q_dtype) || !valid_dtype(a.cache_dtype)) return NC_ERR_DTYPE;
  if (!decode_supports(a.cache_dtype, a.head_dim)) return NC_ERR_HEAD_DIM;
  if (a.keys_per_split < 0 || a.keys_per_split % 64 != 0) return NC_ERR_BAD_SHAPE;
  // the kernels take running maxima of unscaled scores: the scale must be positive (and finite)
  if (!(a.softmax_scale > 0.0f) || !(a.softmax_scale < 3.0e38f)) return NC_ERR_BAD_SHAPE;
  if (a.cache_batch_idx != nullptr && a.cache_batch <= 0) return NC_ERR_BAD_SHAPE;
  if (a.cu_seqlens_q != nullptr && (a.total_q < 0 || a.total_q > INT32_MAX)) return NC_ERR_BAD_SHAPE;
  if (!valid_pages(a.page_table, a.page_table_stride, a.page_size, a.num_blocks, a.t_max, a.cache_batch_idx,
                   a.kc_stride_b, a.kc_stride_t, a.vc_stride_b, a.vc_stride_t)) {
    return NC_ERR_BAD_SHAPE;
  }

  const int group = static_cast<int>(a.n_heads / a.n_kv_heads);
  int hb = 1;
  for (int c : {8, 4, 2}) {
    if (group % c == 0) { hb = c; break; }
  }
  plan->group = group;
  plan->head_block = hb;
  plan->n_hblocks = group / hb;
  if (a.n_kv_heads * plan->n_hblocks > INT32_MAX / 2) return NC_ERR_BAD_SHAPE;
  plan->n_units = static_cast<int>(a.n_kv_heads) * plan->n_hblocks;
  plan->n_groups = a.batch * a.t_new * plan->n_units;

  const int64_t ebytes = dtype_bytes(a.cache_dtype);
  const int64_t max_keys = a.window_left >= 0 ? std::min<int64_t>(a.t_max, int64_t(a.window_left) + 1) : a.t_max;
  int64_t kps = a.keys_per_split;
  if (kps == 0) {
    kps = std::max<int64_t>(64, (default_split_bytes() / (a.head_dim * ebytes) + 63) / 64 * 64);
  }
  // Splits per group: enough for the longest possible row at kps keys, but at
  // most max_splits() and, for the library default, at most about
  // kDecodeGridTarget workgroups in all.  Rows longer than ns * kps are spread
  // evenly over the ns splits by the kernels (multiples of 64 keys), so the
  // grid follows the cache length only up to that bound: workgroups past a
  // row's end still cost a dispatch each (48 rows x 128 keys, GQA 16/4: 9.5 us
  // per call in a 4096-key cache, 20.2 us in a 16384-key one).
  const int64_t cap = max_splits();
  const int64_t grid_cap = a.keys_per_split > 0 ? cap : std::max<int64_t>(1, kDecodeGridTarget / plan->n_groups);
  int64_t ns = std::min((max_keys + kps - 1) / kps, std::min(cap, grid_cap));
  // Between half and one chip's worth of groups with short rows: one 8-wave
  // workgroup per group streams the whole row (no split, so no merge launch).
  // Measured on MI355X: d24 decode (192 groups x 513-1153 keys) 0.469 -> 0.391
  // ms/step; fewer groups leave CUs idle (d26 SSSL decode, 104 groups x
  // 1025-3328 keys: 0.562 -> 0.606), so they keep the split plan.
  plan->wide = false;
  if (a.t_new == 1 && a.keys_per_split == 0 && plan->n_groups >= kWideMinGroups && plan->n_groups <= kWideMaxGroups &&
      max_keys <= kWideMaxKeys &&
      decode_wide_supported(hb, a.head_dim)) {
    plan->wide = true;
    kps = (max_keys + 63) / 64 * 64;
    ns = 1;
  }
  plan->keys_per_split = static_cast<int>(kps);
  plan->num_splits = static_cast<int>(ns);
  plan->n_wg = decode_grid(plan->n_groups, plan->num_splits);
  if (plan->n_groups <= 0 || plan->n_wg <= 0 || plan->n_wg > INT32_MAX) return NC_ERR_BAD_SHAPE;
  // Length-balanced pieces where the uniform split count would stretch long
  // rows' splits past keys_per_split (the grid cap binds) and there are rows
  // to balance: n_groups * num_splits workgroups (no XCD rounding: pieces are
  // not mapped to XCDs), one piece size for the call chosen on the device
  // from cache_seqlens.  Rows of equal length get the pieces the splits had.
  const int64_t row_tiles = (a.t_max + 63) / 64;
  plan->bal = NC_DECODE_BAL && !plan->wide && a.t_new == 1 && a.keys_per_split == 0 &&
              a.cache_batch_idx == nullptr && a.cu_seqlens_q == nullptr && a.page_table == nullptr &&
              a.batch >= 2 && a.batch <= kDecodeBalMaxRows && ns >= 2 && max_keys > ns * kps &&
              a.batch * row_tiles * plan->n_units <= INT32_MAX / 2;
  // (A cap of n_groups + 3136 workgroups, fewer of them past the last piece,
  // measured 1.742 vs 1.785 ms/step on C5 at 16 steps but 1.88 vs 1.81 at
  // bench.py's default 8 steps, with the same pieces: no cap.)
  if (plan->bal) plan->n_wg = plan->n_groups * ns;

  plan->use_chunk = a.t_new >= kChunkMinTokens && chunk_supports(a);
  plan->chunk_keys_per_split = 0;
  plan->chunk_splits = 1;
  plan->chunk_rows = kChunkRowsSmall;
  if (plan->use_chunk) {
    const int64_t units = (a.t_new + kChunkRowsSmall / hb - 1) / (kChunkRowsSmall / hb) * a.batch * a.n_kv_heads *
                          plan->n_hblocks;
    if (units >= kChunkLargeAt) plan->chunk_rows = kChunkRowsLarge;
    // one workgroup's keys span at most (window + its queries) or the cache length
    const int64_t qb = plan->chunk_rows / hb;
    const int64_t span = a.window_left >= 0 ? std::min<int64_t>(a.t_max, int64_t(a.window_left) + qb) : a.t_max;
    int64_t ckps = a.keys_per_split;
    if (ckps == 0) {
      // workgroups of one row per split: q tiles x kv heads x head blocks
      const int64_t per_row = (a.t_new + qb - 1) / qb * a.n_kv_heads * plan->n_hblocks;
      // 128-row workgroups aim at half as many per row: C5's chunk rows get 2048-key splits
      // (fewer partials for the merge).  Measured on one box, C5 chunk part, 1024 vs 2048:
      // 3.378 vs 3.467 ms/step at 16 steps (lengths to 14336), but 3.064 vs 2.886 at 8 steps
      // (lengths to 15360); one varlen call per layer 6.51 vs 6.37.
      const int64_t wg_per_row = kChunkWGPerRow * kChunkRowsSmall / plan->chunk_rows;
      const int64_t want = (span * per_row + wg_per_row - 1) / wg_per_row;
      ckps = span > kChunkSplitAbove
                 ? std::min(span, std::max(kChunkSplitUnit, (want + kChunkSplitUnit - 1) / kChunkSplitUnit * kChunkSplitUnit))
                 : span;
    }
    int64_t cns = (span + ckps - 1) / ckps;
    if (cns > cap) {
      ckps = ((span + cap - 1) / cap + 63) / 64 * 64;
      cns = (span + ckps - 1) / ckps;
    }
    plan->chunk_keys_per_split = static_cast<int>(ckps);
    plan->chunk_splits = static_cast<int>(cns);
    // the chunk grid (block indices are decomposed in 32-bit arithmetic)
    const int64_t cgroups = (a.batch * a.n_kv_heads * plan->n_hblocks + 7) / 8 * 8;
    if (cgroups * ((a.t_new + qb - 1) / qb) * cns > INT32_MAX) return NC_ERR_BAD_SHAPE;
  }
  const int64_t merge_splits = plan->use_chunk ? plan->chunk_splits : ns;
  // decode splits: the last workgroup of each group merges (no merge launch)
  plan->merge_in_kernel = !plan->use_chunk && !plan->bal && ns > 1 && plan->n_groups <= kMaxTickets &&
                          plan->n_groups * ns <= kMergeInKernelMaxWG;
  if (merge_splits > 1) {
    const size_t pairs = static_cast<size_t>(a.batch * a.t_new * a.n_heads);
    // balanced pieces: one slot per workgroup of the grid and head of its unit
    const size_t slots = plan->bal ? static_cast<size_t>(plan->n_wg * hb) : pairs * merge_splits;
    plan->ml_bytes = round256(slots * 2 * 4);
    plan->o_bytes = round256(slots * static_cast<size_t>(a.head_dim) * 4);
  } else {
    plan->ml_bytes = plan->o_bytes = 0;
  }
  // A varlen batch on the chunk kernel sends its single-token rows to the
  // decode kernel (a t_new = 1 plan of their own, partials after the chunk
  // partials): on the chunk kernel each of them fills 1 query of a 16-query
  // tile (C5 as one call per layer: 12.4 ms/step on the chunk kernel alone,
  // two calls 7.2).
  plan->split_rows = a.cu_seqlens_q != nullptr && plan->use_chunk;
  plan->dec_bytes = 0;
  if (plan->split_rows) {
    nc_attn_args d = a;
    d.t_new = 1;
    AttnPlan dp;
    const int st = plan_attention(d, &dp);
    if (st != NC_OK) return st;
    plan->dec_bytes = dp.ml_bytes + dp.o_bytes;
  }
  // every non-empty workspace starts with the sync region, whether or not
  // this call uses it, so no call's scratch ever lands on the counters
  const size_t scratch = plan->ml_bytes + plan->o_bytes + plan->dec_bytes;
  plan->total_bytes = scratch > 0 ? NC_WORKSPACE_SYNC_BYTES + scratch : 0;
  return NC_OK;
}

}  // namespace nckv

using namespace nckv;

extern "C" {

int nc_abi_version(void) { return NC_KV_ABI_VERSION; }

int nc_supports_head_dim(int64_t head_dim) { return decode_supports(NC_DTYPE_BF16, head_dim) ? 1 : 0; }

const char* nc_strerror(int status) {
  switch (status) {
    case NC_OK: return "ok";
    case NC_ERR_NULL_ARG: return "a required pointer argument is NULL";
    case NC_ERR_BAD_SHAPE: return "invalid or inconsistent sizes";
    case NC_ERR_DTYPE: return "unsupported dtype combination";
    case NC_ERR_HEAD_DIM: return "head_dim not supported by the compiled kernels (32, 64, 128, 256)";
    case NC_ERR_ALIGNMENT: return "pointer or stride not 16-byte aligned";
    case NC_ERR_WORKSPACE: return "workspace missing or too small";
    case NC_ERR_LAUNCH: return "kernel launch failed";
    case NC_ERR_SCRATCH_LIMIT:
      return "the call needs more split-K scratch than nc_attn_kvcache_noalloc holds (NC_NOALLOC_SCRATCH_BYTES); "
             "use nc_attn_kvcache with a workspace";
    default: return "unknown nc_status";
  }
}

int nc_kv_append(const nc_append_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  const nc_append_args& a = *args;
  if (!a.k_cache || !a.v_cache || !a.k || !a.v || !a.cache_seqlens) return NC_ERR_NULL_ARG;
  if (a.batch <= 0 || a.t_new <= 0 || a.t_max <= 0 || a.n_kv_heads <= 0 || a.head_dim <= 0) {
    return NC_ERR_BAD_SHAPE;
  }
  if (a.cache_batch_idx != nullptr && a.cache_batch <= 0) return NC_ERR_BAD_SHAPE;
  if (a.cu_seqlens_q != nullptr && (a.total_q < 0 || a.total_q > INT32_MAX)) return NC_ERR_BAD_SHAPE;
  if (!valid_pages(a.page_table, a.page_table_stride, a.page_size, a.num_blocks, a.t_max, a.cache_batch_idx,
                   a.kc_stride_b, a.kc_stride_t, a.vc_stride_b, a.vc_stride_t)) {
    return NC_ERR_BAD_SHAPE;
  }
  if (!valid_dtype(a.in_dtype) || !valid_dtype(a.cache_dtype)) return NC_ERR_DTYPE;
  const int64_t eb = dtype_bytes(a.cache_dtype);
  if ((a.head_dim * eb) % 16 != 0) return NC_ERR_HEAD_DIM;
  if (!aligned16(a.k_cache) || !aligned16(a.v_cache) ||
      !strides16(eb, a.kc_stride_b, a.kc_stride_t, a.kc_stride_h) ||
      !strides16(eb, a.vc_stride_b, a.vc_stride_t, a.vc_stride_h)) {
    return NC_ERR_ALIGNMENT;
  }
  if (a.in_dtype == a.cache_dtype &&
      (!aligned16(a.k) || !aligned16(a.v) || !strides16(eb, a.k_stride_b, a.k_stride_t, a.k_stride_h) ||
       !strides16(eb, a.v_stride_b, a.v_stride_t, a.v_stride_h))) {
    return NC_ERR_ALIGNMENT;
  }
  return launch_append(a, static_cast<hipStream_t>(stream)) == hipSuccess ? NC_OK : NC_ERR_LAUNCH;
}

int nc_kv_fanout(const nc_fanout_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  const nc_fanout_args& a = *args;
  if (!a.k_src || !a.v_src || !a.k_dst || !a.v_dst) return NC_ERR_NULL_ARG;
  if (a.n_layers <= 0 || a.n_rows <= 0 || a.prefix_len < 0 || a.row_elems <= 0) return NC_ERR_BAD_SHAPE;
  if (a.n_layers > 65535 || a.n_rows > INT32_MAX || a.prefix_len > INT32_MAX) return NC_ERR_BAD_SHAPE;
  if (!valid_dtype(a.dtype)) return NC_ERR_DTYPE;
  const int64_t eb = dtype_bytes(a.dtype);
  const int64_t region = a.prefix_len * a.row_elems * eb;
  const uintptr_t ptr_or = reinterpret_cast<uintptr_t>(a.k_src) | reinterpret_cast<uintptr_t>(a.v_src) |
                           reinterpret_cast<uintptr_t>(a.k_dst) | reinterpret_cast<uintptr_t>(a.v_dst);
  const int64_t size_or = region | (a.src_stride_l * eb) | (a.dst_stride_l * eb) | (a.dst_stride_b * eb);
  int unit = 2;
  if ((ptr_or & 15u) == 0 && (size_or & 15) == 0) {
    unit = 16;
  } else if ((ptr_or & 3u) == 0 && (size_or & 3) == 0) {
    unit = 4;
  }
  return launch_fanout(a, unit, static_cast<hipStream_t>(stream)) == hipSuccess ? NC_OK : NC_ERR_LAUNCH;
}

size_t nc_attn_workspace_bytes(const nc_attn_args* args) {
  if (args == nullptr) return 0;
  AttnPlan plan;
  if (plan_attention(*args, &plan) != NC_OK) return 0;
  return plan.total_bytes;
}

namespace {

// Validation shared by both attention entry points; fills the plan.
int check_attention(const nc_attn_args& a, AttnPlan* plan) {
  if (!a.q || !a.out || !a.k_cache || !a.v_cache || !a.cache_seqlens) return NC_ERR_NULL_ARG;
  if ((a.k == nullptr) != (a.v == nullptr)) return NC_ERR_NULL_ARG;
  const int st = plan_attention(a, plan);
  if (st != NC_OK) return st;
  const int64_t eb = dtype_bytes(a.cache_dtype);
  if (!aligned16(a.k_cache) || !aligned16(a.v_cache) ||
      !strides16(eb, a.kc_stride_b, a.kc_stride_t, a.kc_stride_h) ||
      !strides16(eb, a.vc_stride_b, a.vc_stride_t, a.vc_stride_h)) {
    return NC_ERR_ALIGNMENT;
  }
  const bool same = a.q_dtype == a.cache_dtype;
  if (same && (!aligned16(a.q) || !strides16(eb, a.q_stride_b, a.q_stride_t, a.q_stride_h))) {
    return NC_ERR_ALIGNMENT;
  }
  if (a.k != nullptr && same &&
      (!aligned16(a.k) || !aligned16(a.v) || !strides16(eb, a.k_stride_b, a.k_stride_t, a.k_stride_h) ||
       !strides16(eb, a.v_stride_b, a.v_stride_t, a.v_stride_h))) {
    return NC_ERR_ALIGNMENT;
  }
  return NC_OK;
}

AttnScratch carve(const nc_attn_args& a, const AttnPlan& plan) {
  AttnScratch s;
  char* ws = static_cast<char*>(a.workspace);
  s.tickets = reinterpret_cast<uint32_t*>(ws);
  s.part_ml = reinterpret_cast<float*>(ws + NC_WORKSPACE_SYNC_BYTES);
  s.part_o = reinterpret_cast<float*>(ws + NC_WORKSPACE_SYNC_BYTES + plan.ml_bytes);
  return s;
}

// Append (unless a prologue already did) and attend: decode kernel for
// t_new == 1 (append and, with `prologue`, the QK prologue fused), MFMA chunk
// kernel for chunks, the decode kernel per query otherwise.
int run_attention(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                  const nc_qk_prologue* prologue, hipStream_t hs) {
  bool fused = false;
  if (a.k != nullptr) {
    if (a.t_new == 1 || plan.use_chunk) {
      fused = true;  // the decode / chunk kernel appends the new tokens itself
    } else {
      nc_append_args ap;
      ap.k_cache = a.k_cache; ap.v_cache = a.v_cache; ap.k = a.k; ap.v = a.v;
      ap.cache_seqlens = a.cache_seqlens; ap.error_flag = a.error_flag;
      ap.cache_batch_idx = a.cache_batch_idx; ap.cache_batch = a.cache_batch;
      ap.cu_seqlens_q = a.cu_seqlens_q; ap.total_q = a.total_q;
      ap.page_table = a.page_table; ap.page_table_stride = a.page_table_stride;
      ap.page_size = a.page_size; ap.num_blocks = a.num_blocks;
      ap.batch = a.batch; ap.t_new = a.t_new; ap.t_max = a.t_max;
      ap.n_kv_heads = a.n_kv_heads; ap.head_dim = a.head_dim;
      ap.kc_stride_b = a.kc_stride_b; ap.kc_stride_t = a.kc_stride_t; ap.kc_stride_h = a.kc_stride_h;
      ap.vc_stride_b = a.vc_stride_b; ap.vc_stride_t = a.vc_stride_t; ap.vc_stride_h = a.vc_stride_h;
      ap.k_stride_b = a.k_stride_b; ap.k_stride_t = a.k_stride_t; ap.k_stride_h = a.k_stride_h;
      ap.v_stride_b = a.v_stride_b; ap.v_stride_t = a.v_stride_t; ap.v_stride_h = a.v_stride_h;
      ap.in_dtype = a.q_dtype; ap.cache_dtype = a.cache_dtype;
      if (launch_append(ap, hs) != hipSuccess) return NC_ERR_LAUNCH;
    }
  }
  if (plan.use_chunk) {
    RowFilter chunk_rows{0, static_cast<int>(a.t_new), static_cast<int>(a.t_new)};
    if (plan.split_rows) {
      // single-token rows on the decode kernel, the others on the chunk kernel
      nc_attn_args d = a;
      d.t_new = 1;
      AttnPlan dp;
      if (plan_attention(d, &dp) != NC_OK) return NC_ERR_BAD_SHAPE;
      AttnScratch ds = s;
      char* base = static_cast<char*>(a.workspace) + NC_WORKSPACE_SYNC_BYTES + plan.ml_bytes + plan.o_bytes;
      ds.part_ml = reinterpret_cast<float*>(base);
      ds.part_o = reinterpret_cast<float*>(base + dp.ml_bytes);
      const RowFilter dec_rows{1, 1, static_cast<int>(a.t_new)};
      if (launch_decode(d, dp, ds, fused, nullptr, hs, &dec_rows) != hipSuccess) return NC_ERR_LAUNCH;
      chunk_rows.lo = 2;
    }
    if (launch_chunk(a, plan, s, hs, &chunk_rows) != hipSuccess) return NC_ERR_LAUNCH;
    if (plan.chunk_splits > 1 && launch_chunk_merge(a, plan, s, hs, &chunk_rows) != hipSuccess) return NC_ERR_LAUNCH;
    return NC_OK;
  }
  return launch_decode(a, plan, s, fused, prologue, hs) == hipSuccess ? NC_OK : NC_ERR_LAUNCH;
}

// Bytes of q after the prologue kept in the workspace (t_new > 1).
size_t rope_q_bytes(const nc_attn_args& a) {
  if (a.t_new <= 1) return 0;
  return round256(static_cast<size_t>(a.batch * a.t_new * a.n_heads * a.head_dim) *
                  static_cast<size_t>(dtype_bytes(a.q_dtype)));
}

// Workspace offset of the prologue's q (after the sync region and partials).
size_t rope_q_offset(const AttnPlan& plan) {
  return NC_WORKSPACE_SYNC_BYTES + plan.ml_bytes + plan.o_bytes + plan.dec_bytes;
}

// Workspace bytes of nc_attn_kvcache_rope.
size_t rope_need(const nc_attn_args& a, const AttnPlan& plan) {
  const size_t q = rope_q_bytes(a);
  return q > 0 ? rope_q_offset(plan) + q : plan.total_bytes;
}

}  // namespace

int nc_attn_kvcache(const nc_attn_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  const nc_attn_args& a = *args;
  AttnPlan plan;
  const int st = check_attention(a, &plan);
  if (st != NC_OK) return st;
  if (plan.total_bytes > 0 && (a.workspace == nullptr || a.workspace_bytes < plan.total_bytes ||
                               !aligned16(a.workspace))) {
    return NC_ERR_WORKSPACE;
  }
  return run_attention(a, plan, carve(a, plan), nullptr, static_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Scratch of nc_attn_kvcache_noalloc: the split counters (first
// NC_WORKSPACE_SYNC_BYTES, zero between calls) and split partials that
// nc_attn_kvcache takes from the caller's workspace.  Each GPU holds its own
// copy at its own address until the process ends.  In host code this name is
// not a device address: host code only ever uses the address
// hipGetSymbolAddress returns for a device (kept in g_scratch_addr).
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[NC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 1024;
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxScratchDevices];  // device address of `scratch` per device; null until set up

__global__ __launch_bounds__(256) void clear_counters_kernel(uint32_t* counters) {
  counters[blockIdx.x * 256 + threadIdx.x] = 0u;
}

// Device address of `scratch` on the GPU that `stream` belongs to.  The first
// call on a device looks the address up with that device current and clears
// the split counters with a fill kernel on `stream`, ordered before the
// call's own kernels (static device memory is zero at load, but the counters
// must be zero whatever the loader did).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream != nullptr ? hipStreamGetDevice(stream, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) {
    return NC_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return NC_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_addr[dev] == nullptr) {
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) return NC_ERR_LAUNCH;
    if (prev != dev && hipSetDevice(dev) != hipSuccess) return NC_ERR_LAUNCH;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p != nullptr) {
      static_assert(NC_WORKSPACE_SYNC_BYTES % (4 * 256) == 0, "counter region: whole 256-thread blocks");
      hipLaunchKernelGGL(clear_counters_kernel, dim3(NC_WORKSPACE_SYNC_BYTES / (4 * 256)), dim3(256), 0, stream,
                         static_cast<uint32_t*>(p));
      e = hipGetLastError();
    }
    if (prev != dev) (void)hipSetDevice(prev);
    if (e != hipSuccess || p == nullptr) return NC_ERR_LAUNCH;
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return NC_OK;
}

}  // namespace

extern "C" {

int nc_attn_kvcache_noalloc(const nc_attn_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  AttnPlan plan;
  const int st = check_attention(*args, &plan);
  if (st != NC_OK) return st;
  if (plan.total_bytes > static_cast<size_t>(NC_NOALLOC_SCRATCH_BYTES)) return NC_ERR_SCRATCH_LIMIT;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  nc_attn_args a = *args;
  a.workspace = nullptr;
  a.workspace_bytes = 0;
  if (plan.total_bytes > 0) {
    const int s2 = scratch_address(hs, &a.workspace);
    if (s2 != NC_OK) return s2;
    a.workspace_bytes = NC_NOALLOC_SCRATCH_BYTES;
  }
  return run_attention(a, plan, carve(a, plan), nullptr, hs);
}

size_t nc_attn_rope_workspace_bytes(const nc_attn_args* args) {
  if (args == nullptr) return 0;
  AttnPlan plan;
  if (plan_attention(*args, &plan) != NC_OK) return 0;
  return rope_need(*args, plan);
}

int nc_attn_kvcache_rope(const nc_attn_args* args, const nc_qk_prologue* prologue, void* stream) {
  if (args == nullptr || prologue == nullptr) return NC_ERR_NULL_ARG;
  const nc_attn_args& a = *args;
  const nc_qk_prologue& pro = *prologue;
  if (a.k == nullptr || a.v == nullptr || pro.cos == nullptr || pro.sin == nullptr) return NC_ERR_NULL_ARG;
  if (pro.rot_len <= 0 || pro.rot_len > INT32_MAX) return NC_ERR_BAD_SHAPE;
  if (!valid_dtype(pro.rot_dtype)) return NC_ERR_DTYPE;
  // tables are read with 8-32 byte vector loads at multiples of 4 entries
  if (!aligned16(pro.cos) || !aligned16(pro.sin) || (a.head_dim / 2 * dtype_bytes(pro.rot_dtype)) % 16 != 0) {
    return NC_ERR_ALIGNMENT;
  }
  AttnPlan plan;
  const int st = check_attention(a, &plan);
  if (st != NC_OK) return st;
  const size_t need = rope_need(a, plan);
  if (need > 0 && (a.workspace == nullptr || a.workspace_bytes < need || !aligned16(a.workspace))) {
    return NC_ERR_WORKSPACE;
  }
  const int64_t rows = a.batch * a.t_new * (a.n_heads + 2 * a.n_kv_heads);
  if (rows / 4 > INT32_MAX) return NC_ERR_BAD_SHAPE;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const AttnScratch s = carve(a, plan);
  if (a.t_new == 1) return run_attention(a, plan, s, &pro, hs);
  // t_new > 1: prologue kernel (q -> workspace, k/v -> cache), then attention without append
  void* q_out = static_cast<char*>(a.workspace) + rope_q_offset(plan);
  if (launch_rope_append(a, pro, q_out, hs) != hipSuccess) return NC_ERR_LAUNCH;
  nc_attn_args b = a;
  b.q = q_out;
  b.q_stride_h = a.head_dim;
  b.q_stride_t = a.n_heads * a.head_dim;
  b.q_stride_b = a.t_new * a.n_heads * a.head_dim;
  b.k = nullptr;
  b.v = nullptr;
  return run_attention(b, plan, s, nullptr, hs);
}

size_t nc_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return plan_linear(m, n, k).total_bytes;
}

int nc_linear(const nc_linear_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  const nc_linear_args& a = *args;
  if (!a.x || !a.w || !a.y) return NC_ERR_NULL_ARG;
  if (a.m <= 0 || a.m > kLinMaxM || a.n <= 0 || a.k <= 0 || a.k % 8 != 0) return NC_ERR_BAD_SHAPE;
  if (a.n > INT32_MAX / 2 || a.k > INT32_MAX / 2) return NC_ERR_BAD_SHAPE;
  if (a.x_stride_m >= kLinMaxStride || a.w_stride_n >= kLinMaxStride || a.k >= kLinMaxStride) {
    return NC_ERR_BAD_SHAPE;
  }
  if ((a.m > 1 && (a.x_stride_m < a.k || a.y_stride_m < a.n)) || (a.n > 1 && a.w_stride_n < a.k)) {
    return NC_ERR_BAD_SHAPE;
  }
  if (!(a.softcap >= 0.0f) || a.softcap > 3.0e38f) return NC_ERR_BAD_SHAPE;  // also rejects NaN
  if (a.dtype != NC_DTYPE_BF16 && a.dtype != NC_DTYPE_F16) return NC_ERR_DTYPE;
  if (a.y_dtype != a.dtype && a.y_dtype != NC_DTYPE_F32) return NC_ERR_DTYPE;
  if (a.softcap > 0.0f && a.y_dtype != NC_DTYPE_F32) return NC_ERR_DTYPE;
  if (!aligned16(a.x) || !aligned16(a.w) || (a.x_stride_m % 8) != 0 || (a.w_stride_n % 8) != 0) {
    return NC_ERR_ALIGNMENT;
  }
  if ((reinterpret_cast<uintptr_t>(a.y) % dtype_bytes(a.y_dtype)) != 0) return NC_ERR_ALIGNMENT;
  const LinearPlan pl = plan_linear(a.m, a.n, a.k);
  if (pl.total_bytes > 0 &&
      (a.workspace == nullptr || a.workspace_bytes < pl.total_bytes || !aligned16(a.workspace))) {
    return NC_ERR_WORKSPACE;
  }
  return launch_linear(a, pl, a.workspace, static_cast<hipStream_t>(stream)) == hipSuccess ? NC_OK : NC_ERR_LAUNCH;
}

int nc_sample(const nc_sample_args* args, void* stream) {
  if (args == nullptr) return NC_ERR_NULL_ARG;
  const nc_sample_args& a = *args;
  if (!a.logits || !a.out || (a.temperature > 0.0f && !a.uniforms)) return NC_ERR_NULL_ARG;
  if (a.batch <= 0 || a.batch > INT32_MAX || a.vocab <= 0 || a.vocab > INT32_MAX / 2) return NC_ERR_BAD_SHAPE;
  // rows logits_stride apart; 0 broadcasts one row to the batch (an expanded tensor)
  if (a.logits_stride < 0 || (a.batch > 1 && a.logits_stride != 0 && a.logits_stride < a.vocab)) {
    return NC_ERR_BAD_SHAPE;
  }
  if (!(a.temperature >= 0.0f) || a.temperature > 3.0e38f) return NC_ERR_BAD_SHAPE;   // also NaN
  if (a.top_k < 0 || (a.top_k > kMaxTopK && a.top_k < a.vocab)) return NC_ERR_BAD_SHAPE;
  if ((reinterpret_cast<uintptr_t>(a.logits) & 3u) != 0 || (reinterpret_cast<uintptr_t>(a.out) & 7u) != 0) {
    return NC_ERR_ALIGNMENT;
  }
  return launch_sample(a, static_cast<hipStream_t>(stream)) == hipSuccess ? NC_OK : NC_ERR_LAUNCH;
}

}  // extern "C"
