// Host-side launch interfaces between the C ABI (nc_kv_abi.hip) and the
// kernel translation units.  Arguments have been validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "nc_kv.h"
#include "nc_kv_common.hpp"

namespace nckv {

// The device-side page map of a call (table NULL when the cache is not paged).
inline PageMap page_map(const int32_t* table, int64_t stride, int64_t page_size, int64_t n_blocks) {
  PageMap pm{table, stride, 0, n_blocks};
  while (table != nullptr && (int64_t(1) << pm.shift) < page_size) ++pm.shift;
  return pm;
}

// Split-K scratch carved out of the caller's workspace.
struct AttnScratch {
  float* part_ml;      // (pair, split, 2): running max (log2 domain) and sum
  float* part_o;       // (pair, split, D): unnormalised output
  uint32_t* tickets;   // (group,): split arrival counters, zero between calls
};

// Launch plan shared by nc_attn_workspace_bytes and nc_attn_kvcache.
struct AttnPlan {
  int group;           // q heads per kv head
  int head_block;      // q heads one workgroup scores together (divides group)
  int n_hblocks;       // group / head_block
  int n_units;         // n_kv_heads * n_hblocks
  int64_t n_groups;    // batch * t_new * n_units: one merge block each
  int keys_per_split;
  int num_splits;
  int64_t n_wg;        // decode grid size
  bool wide;           // decode with 8-wave workgroups and one split (few groups, short rows)
  bool bal;            // decode with length-balanced pieces (see kDecodeBalMaxRows)
  bool merge_in_kernel;  // decode splits merged by their last workgroup (tickets), no merge launch
  bool use_chunk;      // T_new > 1 on the MFMA chunk kernel
  int chunk_rows;      // (query, head) rows per chunk workgroup: kChunkRowsSmall or kChunkRowsLarge
  int chunk_keys_per_split;
  int chunk_splits;    // > 1: chunk partials merged by the split-merge kernel
  // varlen batch on the chunk kernel: its single-token rows run on the decode
  // kernel (a t_new = 1 plan of their own; dec_bytes of partials after the
  // chunk partials)
  bool split_rows;
  size_t ml_bytes, o_bytes, dec_bytes, total_bytes;
};

// Returns NC_OK and fills `plan`, or an error code.
int plan_attention(const nc_attn_args& a, AttnPlan* plan);

// Single-token decode over rows of very unequal lengths: the uniform split
// count of the plan leaves the long rows' workgroups with long splits that
// finish last.  Such calls (plain layout, the library's split size, rows
// longer than num_splits * keys_per_split possible, at most this many rows)
// cut every row into pieces of one common size instead, sized on the device
// from cache_seqlens so that all pieces fit the grid.
constexpr int kDecodeBalMaxRows = 256;
#ifndef NC_DECODE_BAL
#define NC_DECODE_BAL 1  // 0: such calls keep the uniform split plan
#endif
#ifndef NC_DECODE_BAL_MIN_TILES
#define NC_DECODE_BAL_MIN_TILES 4  // least 64-key tiles per piece
#endif

hipError_t launch_append(const nc_append_args& a, hipStream_t stream);
hipError_t launch_fanout(const nc_fanout_args& a, int unit_bytes, hipStream_t stream);
// prologue != nullptr: the fused QK prologue on q and the appended k (t_new == 1 with k/v).
// Rows one launch takes from a varlen batch (cu_seqlens_q) that is split
// between the kernels: rows whose token count len satisfies lo <= len <= hi;
// `bound` (the call's max_seqlen_q) is the validity limit of len.
struct RowFilter {
  int lo, hi, bound;
};

hipError_t launch_decode(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                         bool fused_append, const nc_qk_prologue* prologue, hipStream_t stream,
                         const RowFilter* rows = nullptr);
// QK prologue for t_new > 1: q -> q_out (contiguous (B, T, H, D), q's dtype), k (transformed) and
// v appended into the cache.
hipError_t launch_rope_append(const nc_attn_args& a, const nc_qk_prologue& pro, void* q_out, hipStream_t stream);

bool decode_supports(int cache_dtype, int64_t head_dim);
bool decode_wide_supported(int head_block, int64_t head_dim);
bool chunk_supports(const nc_attn_args& a);
hipError_t launch_chunk(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s, hipStream_t stream,
                        const RowFilter* rows = nullptr);
// Chunk workgroups own 64 (query, head) rows (two wave groups share each key
// tile) while the call has fewer than kChunkLargeAt (q tile, kv head, head
// block) units at 64 rows, and 128 rows (each key tile feeds twice the rows)
// from there on.  Measured on MI355X (ms): d24 1024-token prefill (192 units)
// 0.54 at 64 rows, 0.75 at 128; C5's 16 chunk rows (512 units) 4.39 at 64
// rows, 4.01 at 128.
constexpr int kChunkRowsSmall = 64;
constexpr int kChunkRowsLarge = 128;
#ifndef NC_CHUNK_LARGE_AT
#define NC_CHUNK_LARGE_AT 512
#endif
constexpr int64_t kChunkLargeAt = NC_CHUNK_LARGE_AT;
// Split merge of the chunk kernel's partials (plan.chunk_splits > 1).
hipError_t launch_chunk_merge(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                              hipStream_t stream, const RowFilter* rows = nullptr);
int max_splits();
int default_split_bytes();
int64_t decode_grid(int64_t n_groups, int num_splits);

// ---- small-M linear (linear_small_m.hip) ----
// Columns of W per workgroup (4 waves x 16).
constexpr int64_t kLinCols = 64;
// Workgroups one call aims for (two per CU); the K range is split to reach it.
#ifndef NC_LIN_TARGET_WG
#define NC_LIN_TARGET_WG 512
#endif
constexpr int64_t kLinTargetWG = NC_LIN_TARGET_WG;
// At most this many K splits (each adds a partial tile the last workgroup reads back).
#ifndef NC_LIN_MAX_SPLITS
#define NC_LIN_MAX_SPLITS 4
#endif
constexpr int64_t kLinMaxSplits = NC_LIN_MAX_SPLITS;
// Column blocks that can take split-K tickets (one uint32 each in the sync region).
constexpr int64_t kLinMaxTickets = NC_WORKSPACE_SYNC_BYTES / 4;
constexpr int64_t kLinMaxM = 64;
// Narrow plan: M <= kLinNarrowMaxM with few column blocks; waves per workgroup
// sized so the grid holds about kLinNarrowWaves waves.
constexpr int64_t kLinNarrowMaxM = 32;
#ifndef NC_LIN_NARROW_WAVES
#define NC_LIN_NARROW_WAVES 1024
#endif
constexpr int64_t kLinNarrowWaves = NC_LIN_NARROW_WAVES;
// narrow plans with fewer column blocks than this split long K across workgroups too
constexpr int64_t kLinNarrowMinBlocks = 256;

// Row strides (elements) the kernel's 32-bit buffer offsets cover.
constexpr int64_t kLinMaxStride = int64_t(1) << 24;

struct LinearPlan {
  int m_tiles;            // ceil(m / 16)
  int64_t n_blocks;       // ceil(n / 64): one column block per workgroup (per split)
  int64_t chunks;         // ceil(k / 128)
  int64_t chunks_per_split;
  int64_t splits;         // > 1: partials summed by the last workgroup of a block
  int narrow_waves;       // > 0: the narrow kernel (16 * narrow_tiles columns per workgroup, K split over this many waves)
  int narrow_tiles;       // 16-column MFMA tiles per wave of the narrow kernel (1 or 2)
  size_t part_bytes, total_bytes;
};

LinearPlan plan_linear(int64_t m, int64_t n, int64_t k);

// ---- next-token sampling (sample.hip) ----
constexpr int kMaxTopK = 1024;
hipError_t launch_sample(const nc_sample_args& a, hipStream_t stream);
hipError_t launch_linear(const nc_linear_args& a, const LinearPlan& plan, void* workspace, hipStream_t stream);

}  // namespace nckv
