// Chunked prefill into the KV cache on MFMA (nanochat/flash_attention.py:91-102:
// queries bottom-right aligned at s_b + i, causal, sliding window, GQA),
// for T_new > 1 with bf16 / fp16 caches.
//
// Fused append: with k/v given, keys at positions >= s_b are read from k/v
// (token j - s_b) instead of the cache, and the workgroup whose queries are
// those tokens (head block 0, the split holding the position) also stores
// them into the cache, so each new position is written once and no
// workgroup of the launch reads a cache position another one writes.
// Positions outside [0, t_max) are not stored and set NC_DEVERR_OVERFLOW,
// as the standalone append does.
//
// Tiling.  A workgroup owns ROWS = 64 or 128 "rows" = (query, q head) pairs of
// one (row b, kv head, q-head block): ROWS / GB queries x GB heads, so the GB
// heads that share a kv head read each K/V tile once.  8 waves: with 128 rows
// each wave owns 16 rows and scores whole 64-key tiles; with 64 rows (calls of
// few workgroups) two groups of 4 waves take the two 32-key halves of every
// tile for the same rows and merge their (m, l, o) in LDS at the end.
//
// K/V tiles go through a ring of LDS stages filled by direct loads
// (global_load_lds_dwordx4: no registers, no LDS store instructions), the next
// tile in flight while the current one is consumed.  Tile rows are unpadded
// 256-byte rows whose 16-byte chunks sit in slots chunk ^ swz(row), chosen on
// the global side of the load, so the MFMA operand reads hit all 64 banks.
// The waits are counted: every lane issues every load (lanes past the span or
// outside the page pool read a valid key, zeroed once landed), so a wave has a
// fixed number of loads per tile in flight, and each stage is a separate
// __shared__ array named statically at every access (the compiler then sees
// that a stage being filled is not the one being read).
//
// Per tile and wave (v_mfma_f32_16x16x32_{bf16,f16}; lane l, q = l / 16):
//   S^T = K . Q^T   A = K[16 keys][32 dims] (LDS), B = Q^T (registers);
//                   lane l holds S[row l%16][keys 16kb + 4q + r], r < 4.
//   softmax         each lane owns one query row: running max / sum in fp32
//                   (maxima of the unscaled scores, the scale folded into the
//                   exponent's fma), cross-lane reductions over the 4 lane
//                   groups only.
//   O^T += V^T . P^T  B = P^T straight from the S registers (the 32 keys of a
//                   chunk are enumerated in the order the lanes hold them), so
//                   P never leaves registers.  A = V^T in that same key order
//                   comes from the [key][dim] LDS rows through two gfx950
//                   transpose reads (ds_read_b64_tr_b16: in each 16-lane group,
//                   lane i receives element i of the four 8-byte rows its
//                   neighbours point at, i.e. 4 keys of dim i).
//                   Lane l holds O[row l%16][dims 16db + 4q + r].
// Scores and the softmax state are fp32; P is rounded to the cache dtype for
// the second MFMA, as flash-attention kernels do.
//
// Split-K: a workgroup's key span [lo, hi) is cut into `keys_per_split`
// pieces handled by separate workgroups, so long caches keep the chip busy.
// A span that fits one split writes the output directly; otherwise each split
// writes (o, m, l) partials per (query, head) and the split-merge kernel of
// the decode path combines them (chunk_span gives both sides the same split
// count; workgroups past it return at once).

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

// Every workgroup has 8 waves.  With ROWS = 128 each wave owns 16 of the rows
// and scores whole key tiles; with ROWS = 64, two wave groups of 4 split every
// key tile: group g scores keys [g, g + 1) * kBN / 2 of each tile for the same
// 64 rows, and the groups' (m, l, o) meet in LDS at the end (twice the waves of
// a 4-wave workgroup, to hide latency, without more LDS).
constexpr int kChunkWaves = 8;
#ifndef NC_CHUNK_TILE_KEYS
#define NC_CHUNK_TILE_KEYS 64         // keys per tile, 128-row kernels
#endif
#ifndef NC_CHUNK_TILE_KEYS_SMALL
#define NC_CHUNK_TILE_KEYS_SMALL 64   // keys per tile, 64-row kernels
#endif
#ifndef NC_CHUNK_STAGES
#define NC_CHUNK_STAGES 2         // 128-row kernels (two workgroups per CU share the LDS)
#endif
#ifndef NC_CHUNK_STAGES_SMALL  // 64-row kernels (one workgroup per CU: at most 160 KiB of ring)
#define NC_CHUNK_STAGES_SMALL (NC_CHUNK_TILE_KEYS_SMALL >= 128 ? 2 : 3)
#endif
// keys per tile (multiples of 32), the larger of the two
constexpr int kBNMax = NC_CHUNK_TILE_KEYS > NC_CHUNK_TILE_KEYS_SMALL ? NC_CHUNK_TILE_KEYS : NC_CHUNK_TILE_KEYS_SMALL;
constexpr int kChunkStagePages = 512;  // page numbers a workgroup stages in LDS (paged cache)
constexpr float kNegBigC = -1.0e30f;
// exponent-base slack of the online softmax (log2 units: P <= 256)
constexpr float kRebaseSlack = 8.0f;
constexpr int kXcdsC = 8;

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) char lds_char;

// ds_read_b64_tr_b16 from a generic pointer into a __shared__ array.
__device__ __forceinline__ i16x4 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((lds_char*)(p)));
}


// One wave's 16-byte direct load into LDS (global_load_lds_dwordx4): lane l's
// 16 bytes from `src` land at dst + 16 * l.  `dst` must be wave-uniform.  The
// load counts in the wave's vector-memory counter like any other load.
//
// Issued as inline asm, so the compiler does not track it: with the builtin,
// the compiler put an s_waitcnt vmcnt(0) before the transposed V reads
// (ds_read_b64_tr_b16 carries no alias information), a wait for the next
// tile's prefetch issued just before, which serialised every tile's load
// latency with its compute.  The kernel's own counted waits (wait_vmcnt
// before the barrier of each step) are what order a stage's loads before its
// reads; the compiler's waits for its own vector loads stay conservative,
// since loads complete in order and these only add younger ones.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)(p)));
}
// `dst` is wave-uniform by contract; readfirstlane states it to the compiler,
// whose uniformity analysis does not always see it (an "s" operand it could
// not prove uniform was handed a VGPR).
// m0 (the LDS base of the load) is a reserved register: nothing else in these
// kernels reads it (LDS instructions do not use m0 on gfx9 and later), so
// clobbering it here is safe and the compiler's warning about it is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const char* src, char* dst) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one query row's
// lane groups) with the gfx950 lane-half swaps v_permlane16_swap (rows of 16
// lanes: odd rows of the first operand with even rows of the second) and
// v_permlane32_swap (upper 32 lanes with lower 32): swapping x with itself
// leaves {x[l], x[l ^ 16]} (then {., x[l ^ 32]}) in the two results at every
// lane, with no LDS round trip (ds_bpermute) in the softmax's dependency
// chain.  The four lanes end with bitwise-equal values (the pairs are the
// same, max and + commute).
__device__ __forceinline__ float lane_group_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_group_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wait until at most N of this wave's vector-memory operations are outstanding
// (s_waitcnt vmcnt(N); expcnt and lgkmcnt left alone).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS layout of a K or V tile: key row r holds its CPR 16-byte chunks in
// slots permuted by chunk ^ swz(r), so that the MFMA operand reads (8 rows x
// 16 bytes of one chunk per phase for K; 4 rows x 2 chunks, 8 bytes each,
// per 16 lanes for the transposed V reads) spread over all 64 banks.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
  if constexpr (CPR == 16) return 2 * (r & 7);
  else if constexpr (CPR == 8) return 2 * ((r >> 1) & 3);
  else return 0;
}

struct ChunkParams {
  const void* q;
  void* out;
  const char* kc;
  const char* vc;
  const int32_t* seqlens;
  const int32_t* cache_idx;  // cache_batch_idx or NULL
  int64_t cache_batch;
  const int32_t* cu_q;       // cu_seqlens_q (packed query tokens) or NULL
  int64_t total_q;
  PageMap pages;             // paged cache (page_table), or pages.table == NULL
  int32_t indirect;          // cache_idx, cu_q or a page table given: per-row lookups (else row b, t_new queries)
  int32_t q_bound, len_lo, len_hi;  // varlen rows: validity bound, and the token counts this launch takes
  int64_t q_sb, q_st, q_sh;
  int64_t kc_sb, kc_st, kc_sh;
  int64_t vc_sb, vc_st, vc_sh;
  int32_t t_new, t_max, n_heads, n_kv_heads, group, n_hblocks;
  int32_t n_qtiles;
  int64_t n_groups;  // B * n_kv_heads * n_hblocks
  int32_t window;
  float scale_log2;
  int32_t num_splits, keys_per_split;
  float* part_ml;
  float* part_o;
  FastDiv fd_members, fd_qtiles, fd_hblocks, fd_kv_heads;  // block-index divisors (indices < 2^31)
  // fused append (k/v given): positions >= s_b are read from k/v, and each new
  // token is stored into the cache by the one workgroup that owns it
  const char* k_new;
  const char* v_new;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int32_t* err;
  int32_t fused;
};

// MFMA accumulators as the builtin's own vector type (no float4 round trips,
// which cost AGPR <-> VGPR copies around every MFMA).
typedef float f4v __attribute__((ext_vector_type(4)));

template <typename TC> struct mfma_t;
template <> struct mfma_t<bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static void run(const v8& a, const v8& b, f4v& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint16_t from_float(float x) { return f32_to_bf16_rne(x); }
  // two values rounded to nearest even, packed (v_cvt_pk_bf16_f32)
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 h2 __attribute__((ext_vector_type(2)));
    const f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
  }
};
template <> struct mfma_t<f16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static void run(const v8& a, const v8& b, f4v& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint16_t from_float(float x) { return f32_to_f16_rne(x); }
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
  }
};

// LK: 0 plain launch, with no lookup code (it cost 3% on the C5 batch); 1
// cache_batch_idx / cu_seqlens_q lookups; 2 those and a page table (kernels of
// their own, so the lookup kernels keep their code).
// Register budget: waves per SIMD the 128-row kernels are built for (two
// 8-wave workgroups per CU, their LDS rings fitting), and the 64-row ones
// (launches of few workgroups, one per CU: registers are not what limits them).
#ifndef NC_CHUNK_WAVES_PER_EU
#define NC_CHUNK_WAVES_PER_EU 4
#endif
#ifndef NC_CHUNK_PIPE_LARGE
#define NC_CHUNK_PIPE_LARGE 0  // 1: 128-row kernels pipeline their operand reads too (needs the 2-wave budget)
#endif
#ifndef NC_CHUNK_WAVES_PER_EU_SMALL
#define NC_CHUNK_WAVES_PER_EU_SMALL 2
#endif
#define NC_CHUNK_OCC __attribute__((amdgpu_waves_per_eu(ROWS == 64 ? NC_CHUNK_WAVES_PER_EU_SMALL : NC_CHUNK_WAVES_PER_EU)))

template <typename TC, int D, int GB, int LK, int ROWS>
__global__ __launch_bounds__(kChunkWaves * kWave) NC_CHUNK_OCC void chunk_attn_kernel(const ChunkParams p) {
  typedef typename mfma_t<TC>::v8 v8;
  constexpr int kRowWaves = ROWS / 16;    // waves covering the rows, 16 each
  constexpr int kKeyGroups = kChunkWaves / kRowWaves;  // wave groups splitting each key tile
  static_assert(kRowWaves * kKeyGroups == kChunkWaves && (kKeyGroups == 1 || kKeyGroups == 2), "rows");
  constexpr int QB = ROWS / GB;           // queries per workgroup
  constexpr int DC = D / 32;              // 32-dim chunks (MFMA K for S)
  constexpr int DB = D / 16;              // 16-dim output blocks
  constexpr int kBN = ROWS == 64 ? NC_CHUNK_TILE_KEYS_SMALL : NC_CHUNK_TILE_KEYS;  // keys per tile
  constexpr int KG = kBN / kKeyGroups;    // keys of a tile one wave group scores
  constexpr int KB = KG / 16;             // 16-key blocks per wave and tile (S MFMAs)
  constexpr int KC = KG / 32;             // 32-key chunks per wave and tile (P.V MFMAs)
  constexpr int CPR = D / 8;              // 16-byte chunks per key row
  constexpr int ROWB = D * 2;             // bytes per key row in LDS (unpadded, swizzled)
  constexpr int TILEB = kBN * ROWB;       // bytes of a K (or V) tile
  constexpr int NI = kBN * CPR / kWave / kChunkWaves;  // direct loads per wave per tile, K (V the same)
  constexpr int LPT = 2 * NI;             // vector-memory operations per wave per tile
  static_assert(NI * kWave * kChunkWaves == kBN * CPR && KG % 32 == 0, "tile / workgroup shape");
  // software-pipelined operand reads (64-row kernels)
  constexpr bool kPipe = ROWS == 64 || NC_CHUNK_PIPE_LARGE;
  // K/V tiles of the LDS ring (>= 2): kStages - 1 in flight
  constexpr int kStages = ROWS == 64 ? NC_CHUNK_STAGES_SMALL : NC_CHUNK_STAGES;
  static_assert(kStages >= 2 && (kStages - 2) * LPT < 64, "ring depth");

  // ring of kStages tiles, one __shared__ array per stage (K at [0], V at [1]):
  // every access below names its stage statically, so the compiler can tell a
  // stage being filled by direct loads from the stage being read
  static_assert(kStages <= 4, "ring stages");
  __shared__ __attribute__((aligned(1024))) char ring0[2][TILEB];
  __shared__ __attribute__((aligned(1024))) char ring1[2][TILEB];
  __shared__ __attribute__((aligned(1024))) char ring2[kStages > 2 ? 2 : 1][kStages > 2 ? TILEB : 16];
  __shared__ __attribute__((aligned(1024))) char ring3[kStages > 3 ? 2 : 1][kStages > 3 ? TILEB : 16];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // the wave index, provably wave-uniform (so tile bounds and masks derived
  // from it compile to scalar branches, not per-lane exec masking)
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lq = lane / 16;               // lane group 0..3
  const int lr = lane % 16;
  const int rw = wave % kRowWaves;        // row block of this wave
  const int kg = wave / kRowWaves;        // key group of this wave
  const int kgo = kg * KG;                // its first key within a tile

  // the arguments of the prologue, in one batch of scalar loads
  pin_args(p.fd_members, p.fd_qtiles, p.fd_hblocks, p.fd_kv_heads, p.n_groups, p.seqlens, p.t_new, p.t_max,
           p.window, p.keys_per_split, p.q, p.q_sb, p.q_st, p.q_sh, p.kc, p.vc, p.kc_sb, p.kc_st, p.kc_sh, p.vc_sb,
           p.vc_st, p.vc_sh, p.n_heads, p.group, p.fused);

  // ---- block -> (group = (b, kv head, head block), key split, q tile) ----
  // A group's blocks run on one XCD (workgroups go round-robin over the 8 XCDs)
  // and, within it, the q tiles of one key split are neighbours in dispatch
  // order, so they read that split's K/V tiles from the XCD's L2 while it still
  // holds them.  (Measured on a GQA batch with one 14k-key row: q tile fastest
  // 7.0 ms/step, split fastest 8.1, splits spread over the XCDs 8.9, no XCD
  // grouping 23.8.)
  const uint32_t pb = blockIdx.x;
  uint32_t member, rem;
  const uint32_t gq = fdivmod(pb / kXcdsC, p.fd_members, member);
  const uint32_t group = gq * kXcdsC + pb % kXcdsC;
  const int split = static_cast<int>(fdivmod(member, p.fd_qtiles, rem));
  const int qt = static_cast<int>(rem);
  if (group >= p.n_groups) return;
  uint32_t gtmp = fdivmod(group, p.fd_hblocks, rem);
  const int hb = static_cast<int>(rem);
  const int64_t b = fdivmod(gtmp, p.fd_kv_heads, rem);
  const int hk = static_cast<int>(rem);
  // cache row and queries of batch row b (cache_batch_idx, cu_seqlens_q); an
  // invalid entry skips the row in every workgroup of it
  int64_t cb = b;
  RowQ rq{b * p.t_new, p.t_new};
  if constexpr (LK != 0) {
    const bool report = qt == 0 && split == 0 && hk == 0 && hb == 0 && tid == 0;
    if constexpr (LK == 2) {
      cb = 0;  // paged: every position is addressed through the page table
    } else {
      cb = cache_row(p.cache_idx, p.cache_batch, b, p.err, report);
      if (cb < 0) return;
    }
    rq = row_queries(p.cu_q, p.total_q, b, p.q_bound, p.err, report);
    if (rq.len < p.len_lo || rq.len > p.len_hi) return;  // another launch's row (or skipped)
  }
  const int q0 = qt * QB;
  if (q0 >= rq.len) return;  // no queries of this row in the tile (or the row was skipped)

  const int s = p.seqlens[b];
  const int q_end = min(q0 + QB, rq.len);
  if (p.fused && p.err != nullptr && qt == 0 && split == 0 && hk == 0 && hb == 0 && tid == 0 &&
      (s < 0 || s > p.t_max - rq.len)) {
    atomicOr(p.err, NC_DEVERR_OVERFLOW);  // a new token falls outside [0, t_max): not stored
  }

  // this lane's query row
  const int row = rw * 16 + lr;
  const int qi = q0 + row / GB;
  const int h = hk * p.group + hb * GB + row % GB;
  const bool row_ok = qi < rq.len;
  const int qpos = s + qi;
  const int row_lo = p.window >= 0 ? max(0, qpos - p.window) : 0;

  // keys of this split: [lo, hi) within the workgroup's span; splits past the
  // span's own split count have nothing to do (the merge never reads them)
  const ChunkSpan span = chunk_span(s, q0, q_end, p.t_max, p.window, p.keys_per_split);
  if (split >= span.nsplit) return;
  const int lo = span.lo + split * p.keys_per_split;
  const int hi = min(span.hi, lo + p.keys_per_split);
  const int64_t pair_row = (b * p.t_new + qi) * p.n_heads + h;   // this lane's (query, head): partials
  const int64_t out_row = (rq.tok0 + qi) * p.n_heads + h;        // its row of `out`

  // ---- Q^T fragments (B operand): lane holds Q[row][32c + 8*lq + e] ----
  v8 qf[DC];
  {
    const TC* qp = reinterpret_cast<const TC*>(static_cast<const char*>(p.q) +
                                              (token_offset(p.cu_q, rq, b, qi, p.q_sb, p.q_st) + h * p.q_sh) *
                                                  elem<TC>::kBytes);
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (row_ok) w = *reinterpret_cast<const uint4*>(qp + 32 * c + 8 * lq);
      qf[c] = __builtin_bit_cast(v8, w);
    }
  }

  float m_run = kNegBigC, l_run = 0.0f;
  f4v acc_o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc_o[db] = f4v{0.f, 0.f, 0.f, 0.f};

  constexpr int EB = elem<TC>::kBytes;
  const char* kbase = p.kc + (cb * p.kc_sb + hk * p.kc_sh) * EB;
  const char* vbase = p.vc + (cb * p.vc_sb + hk * p.vc_sh) * EB;
  const int64_t kst = p.kc_st * EB;
  const int64_t vst = p.vc_st * EB;
  // new tokens: position j >= s is token j - s of k/v; this workgroup stores the
  // ones of its own queries, [s + q0, s + q_end), once per kv head (hb == 0)
  const int new_lo = p.fused ? s : INT32_MAX;
  const int own_lo = (p.fused && hb == 0) ? s + q0 : INT32_MAX;
  const char* knew = p.k_new + (token_offset(p.cu_q, rq, b, 0, p.k_sb, p.k_st) + hk * p.k_sh) * EB;
  const char* vnew = p.v_new + (token_offset(p.cu_q, rq, b, 0, p.v_sb, p.v_st) + hk * p.v_sh) * EB;
  const int64_t knst = p.k_st * EB;
  const int64_t vnst = p.v_st * EB;

  // ---- key tiles: a ring of kStages LDS tiles filled by direct loads, kStages - 1 tiles ahead ----
  // Load slot i of this wave covers the 64 16-byte LDS chunks [64 n, 64 n + 64) of a tile,
  // n = wave * NI + i: key row lrow[i], holding global chunk (chunk slot ^ swz(row)) at byte
  // column lcol[i] (the plan keeps a tile's byte span below 2^31, so offsets are 32-bit).
  constexpr int RPI = kWave / CPR;        // key rows one direct load covers
  auto lrow = [&](int i) __attribute__((always_inline)) { return (wave * NI + i) * RPI + lane / CPR; };
  auto lcol = [&](int i) __attribute__((always_inline)) {
    return static_cast<uint32_t>(((lane % CPR) ^ swz<CPR>(lrow(i))) * 16);
  };
  // paged cache: the page numbers of this workgroup's keys [lo, hi), read from
  // the table once into LDS (entries outside the pool become -1 and set
  // NC_DEVERR_PAGE), so a tile's K/V loads wait on LDS rather than on a table
  // load of their own.  Spans of more pages fall back to per-key lookups, and
  // so do workgroups that read no cached key (a prefill from position 0: only
  // their stores look pages up, and a staging prologue would only add latency).
  [[maybe_unused]] int page_lo = 0;
  [[maybe_unused]] bool pages_staged = false;
  [[maybe_unused]] bool pages_bad = false;
  [[maybe_unused]] const int32_t* sm_pg = nullptr;
  if constexpr (LK == 2) {
    __shared__ int32_t sm_pages[kChunkStagePages];
    __shared__ int sm_bad;
    page_lo = lo >> p.pages.shift;
    const int npages = hi > lo ? ((hi - 1) >> p.pages.shift) - page_lo + 1 : 0;
    pages_staged = npages <= kChunkStagePages && min(hi, new_lo) > lo;
    if (pages_staged) {
      if (tid == 0) sm_bad = 0;
      __syncthreads();
      for (int i = tid; i < npages; i += kChunkWaves * kWave) {
        const int32_t blk = p.pages.table[b * p.pages.stride + page_lo + i];
        const bool ok = blk >= 0 && blk < p.pages.n_blocks;
        if (!ok) {
          sm_bad = 1;
          if (p.err != nullptr) atomicOr(p.err, NC_DEVERR_PAGE);
        }
        sm_pages[i] = ok ? blk : -1;
      }
      __syncthreads();
      pages_bad = sm_bad != 0;
    } else {
      pages_bad = true;  // per-key lookups: any tile may hold a key outside the pool
    }
    sm_pg = sm_pages;
  }
  // physical cache position of logical key j in [lo, hi): j, or its page-table
  // slot (-1: not addressable)
  auto cache_pos = [&](int j) __attribute__((always_inline)) -> int64_t {
    if constexpr (LK == 2) {
      if (pages_staged) {
        const int32_t blk = sm_pg[(j >> p.pages.shift) - page_lo];
        return blk >= 0 ? ((static_cast<int64_t>(blk) << p.pages.shift) | (j & ((1 << p.pages.shift) - 1))) : -1;
      }
      return page_pos(p.pages, b, j, p.err);
    }
    return j;
  };
  constexpr bool contiguous = LK != 2;  // positions are cache rows (no page table)
  // Issue tile t's direct loads into its ring stage.  Every lane issues every
  // load (so each wave always has LPT operations per tile in flight, which the
  // waits below count on): keys past the span read the span's last key and
  // keys outside the page pool read block 0, and both are zeroed once landed.
  const int ntiles = hi > lo ? (hi - lo + kBN - 1) / kBN : 0;
  // the K and V tiles of ring stage st (a compile-time index at every use)
  auto stage_k = [&](auto st) __attribute__((always_inline)) -> char* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return ring0[0]; else if constexpr (S == 1) return ring1[0];
    else if constexpr (S == 2) return ring2[0]; else return ring3[0];
  };
  auto stage_v = [&](auto st) __attribute__((always_inline)) -> char* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return ring0[1]; else if constexpr (S == 1) return ring1[1];
    else if constexpr (S == 2) return ring2[1]; else return ring3[1];
  };
  auto issue = [&](int t, auto st) __attribute__((always_inline)) {
    const int kt0 = lo + t * kBN;
    char* kd = stage_k(st) + wave * NI * kWave * 16;
    char* vd = stage_v(st) + wave * NI * kWave * 16;
    if (contiguous && kt0 + kBN <= hi && kt0 + kBN <= new_lo) {
      // whole tile inside the span and in the cache: no per-key checks
      const char* kt = kbase + kt0 * kst;
      const char* vt = vbase + kt0 * vst;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        dma16(kt + (static_cast<uint32_t>(lrow(i) * kst) + lcol(i)), kd + i * kWave * 16);
        dma16(vt + (static_cast<uint32_t>(lrow(i) * vst) + lcol(i)), vd + i * kWave * 16);
      }
      return;
    }
    if (ROWS == 64 && kt0 >= new_lo && kt0 + kBN <= hi) {
      // whole tile inside the span and of new tokens (a prefill's tiles): k/v rows kt0 - s on
      // (64-row kernels: the 128-row ones have no registers for a second fast path)
      const char* kt = knew + static_cast<int64_t>(kt0 - s) * knst;
      const char* vt = vnew + static_cast<int64_t>(kt0 - s) * vnst;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        dma16(kt + (lrow(i) * knst + lcol(i)), kd + i * kWave * 16);
        dma16(vt + (lrow(i) * vnst + lcol(i)), vd + i * kWave * 16);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int j = min(kt0 + lrow(i), hi - 1);
      const char* ks_;
      const char* vs_;
      if (j >= new_lo) {
        ks_ = knew + (j - s) * knst;
        vs_ = vnew + (j - s) * vnst;
      } else {
        const int64_t pj = contiguous ? j : max(cache_pos(j), int64_t(0));
        ks_ = kbase + pj * kst;
        vs_ = vbase + pj * vst;
      }
      dma16(ks_ + lcol(i), kd + i * kWave * 16);
      dma16(vs_ + lcol(i), vd + i * kWave * 16);
    }
  };

  // wave-uniform bounds of this wave's query rows: tiles wholly inside every
  // row's mask skip the per-element mask
  const int qi_first = q0 + (rw * 16) / GB, qi_last = q0 + (rw * 16 + 15) / GB;
  const bool wave_rows_full = qi_last < rq.len;
  const int qpos_first = s + qi_first, qpos_last = s + qi_last;
  // this lane's LDS read offsets (the swizzle depends only on the row within a 16-row block):
  // K chunk (4c + lq) of row lr; V row 4 lq + lr / 4 of a 32-key chunk (the +16 half has the
  // same swizzle), 8 bytes at dims 16 db + 4 (lr % 4)
  const int k_sw = swz<CPR>(lr);
  const int v_row = 4 * lq + lr / 4;
  const int v_sw = swz<CPR>(v_row);
  auto k_rd = [&](int c) __attribute__((always_inline)) { return lr * ROWB + (((4 * c + lq) ^ k_sw) * 16); };
  auto v_rd = [&](int db) __attribute__((always_inline)) {
    return v_row * ROWB + (((2 * db + (lr % 4) / 2) ^ v_sw) * 16) + ((lr % 4) % 2) * 8;
  };

  // ---- S^T = K . Q^T for the KB key blocks of a tile ----
  // 64-row kernels (register budget of 2 waves per SIMD): software-pipelined
  // operand reads, block kb + 1's K reads issued before block kb's MFMAs (the
  // scheduling barriers keep that order; left alone, the compiler waited for
  // each read right before its MFMA, one LDS round trip per MFMA).  The
  // 128-row kernels have no registers for it (spills) and keep the
  // compiler's order.
  auto s_phase = [&](const char* ks, f4v (&acc_s)[KB]) __attribute__((always_inline)) {
    uint4 ka[2][DC];
    auto k_load = [&](int kb, uint4 (&dst)[DC]) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < DC; ++c) dst[c] = *reinterpret_cast<const uint4*>(ks + (kgo + 16 * kb) * ROWB + k_rd(c));
    };
    if constexpr (kPipe) {
      k_load(0, ka[0]);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb + 1 < KB) k_load(kb + 1, ka[(kb + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        acc_s[kb] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < DC; ++c) mfma_t<TC>::run(__builtin_bit_cast(v8, ka[kb & 1][c]), qf[c], acc_s[kb]);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        acc_s[kb] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const uint4 a = *reinterpret_cast<const uint4*>(ks + (kgo + 16 * kb) * ROWB + k_rd(c));
          mfma_t<TC>::run(__builtin_bit_cast(v8, a), qf[c], acc_s[kb]);
        }
      }
    }
  };

  // ---- mask, scale, online softmax (each lane: one query row), then O += P.V ----
  auto finish = [&](int kt0, const f4v (&acc_s)[KB], const char* vs) __attribute__((always_inline)) {
    const bool interior = wave_rows_full && kt0 + kBN <= hi && kt0 + kBN - 1 <= qpos_first &&
                          (p.window < 0 || kt0 >= qpos_last - p.window);
    // raw scores (the scale is positive: the running max is taken before scaling
    // and the scale folded into the exponent's fma)
    float sv[KB][4];
    float mt = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const float a4[4] = {acc_s[kb][0], acc_s[kb][1], acc_s[kb][2], acc_s[kb][3]};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[kb][r] = a4[r];
        if (!interior) {
          const int j = kt0 + kgo + 16 * kb + 4 * lq + r;
          const bool ok = row_ok && j >= row_lo && j <= qpos && j < hi;
          sv[kb][r] = ok ? sv[kb][r] : -__builtin_inff();
        }
        mt = fmaxf(mt, sv[kb][r]);
      }
    }
    mt = lane_group_max(mt);
    // Lazy rebase: the exponent base m_run (log2 units) moves to the row's
    // running max only when that max exceeds it by more than kRebaseSlack, so
    // the rescale of the output accumulators runs on few tiles (in practice
    // the first ones) instead of on every tile where some row's max grows.
    // Until then P <= 2^kRebaseSlack, well inside fp32 sums and the P dtype's
    // range; (m, l, o) stay consistent for any base, which is all the merges
    // rely on.
    const float m_tile = mt * p.scale_log2;
    if (__any(m_tile > m_run + kRebaseSlack)) {
      const float m_new = fmaxf(m_run, m_tile);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc_o[db] *= alpha;
      m_run = m_new;
    }
    float rs = 0.0f;
    uint32_t pk[KB][2];  // P packed in the cache dtype: [key block][pair of r]
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float pv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[r] = fast_exp2(__builtin_fmaf(sv[kb][r], p.scale_log2, -m_run));
        rs += pv[r];
      }
      pk[kb][0] = mfma_t<TC>::pack2(pv[0], pv[1]);
      pk[kb][1] = mfma_t<TC>::pack2(pv[2], pv[3]);
    }
    rs = lane_group_sum(rs);
    l_run += rs;

    // ---- O^T += V^T . P^T over the KC 32-key chunks ----
    // V^T operands in groups of VG output blocks, the next group's reads
    // issued before this group's MFMAs (as for K above).  Lane lr of group lq
    // points at key (kgo + 32kc + 4lq + lr/4), dims 16db + 4*(lr%4) .. +3.
    constexpr int VG = DB < 4 ? DB : 4;   // output blocks per group
    constexpr int NG = KC * DB / VG;      // groups per tile
    v8 va[2][VG];
    auto v_load = [&](int gi, v8 (&dst)[VG]) __attribute__((always_inline)) {
      const int kc = gi / (DB / VG), db0 = (gi % (DB / VG)) * VG;
#pragma unroll
      for (int i = 0; i < VG; ++i) {
        const char* src0 = vs + (kgo + 32 * kc) * ROWB + v_rd(db0 + i);
        const i16x4 lo4 = lds_read_tr16(src0);
        const i16x4 hi4 = lds_read_tr16(src0 + 16 * ROWB);
        dst[i] = __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    if constexpr (kPipe) {
      v_load(0, va[0]);
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        if (gi + 1 < NG) v_load(gi + 1, va[(gi + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        const int kc = gi / (DB / VG), db0 = (gi % (DB / VG)) * VG;
        const v8 bp = __builtin_bit_cast(v8, make_uint4(pk[2 * kc][0], pk[2 * kc][1], pk[2 * kc + 1][0], pk[2 * kc + 1][1]));
#pragma unroll
        for (int i = 0; i < VG; ++i) mfma_t<TC>::run(va[gi & 1][i], bp, acc_o[db0 + i]);
      }
    } else {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const v8 bp = __builtin_bit_cast(v8, make_uint4(pk[2 * kc][0], pk[2 * kc][1], pk[2 * kc + 1][0], pk[2 * kc + 1][1]));
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const char* src0 = vs + (kgo + 32 * kc) * ROWB + v_rd(db);
          const i16x4 lo4 = lds_read_tr16(src0);
          const i16x4 hi4 = lds_read_tr16(src0 + 16 * ROWB);
          const v8 av = __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
          mfma_t<TC>::run(av, bp, acc_o[db]);
        }
      }
    }
  };
  auto compute = [&](int kt0, const char* ks, const char* vs) __attribute__((always_inline)) {
    f4v acc_s[KB];
    s_phase(ks, acc_s);
    finish(kt0, acc_s, vs);
  };

  bool stores_pending = false;  // cache stores of new tokens issued after the loads still counted on
  // a landed tile: keys past the span (or outside the page pool) zeroed, and
  // this workgroup's new tokens stored into the cache
  auto fix_tile = [&](int kt0, char* ks, char* vs) __attribute__((always_inline)) {
    char* kme = ks + wave * NI * kWave * 16 + lane * 16;  // this lane's landed chunks (slot i at + i * 1 KiB)
    char* vme = vs + wave * NI * kWave * 16 + lane * 16;
    if (kt0 + kBN > hi || (LK == 2 && pages_bad)) {
      // keys past the span (and outside the page pool) are zero, as if never loaded
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int j = kt0 + lrow(i);
        bool zero = j >= hi;
        if constexpr (LK == 2) zero = zero || (j < new_lo && cache_pos(j) < 0);
        if (zero) {
          *reinterpret_cast<uint4*>(kme + i * kWave * 16) = make_uint4(0, 0, 0, 0);
          *reinterpret_cast<uint4*>(vme + i * kWave * 16) = make_uint4(0, 0, 0, 0);
        }
      }
      __syncthreads();
    }
    if (kt0 + kBN > own_lo) {
      // the tile holds new tokens this workgroup stores into the cache
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int j = kt0 + lrow(i);
        const int64_t pj = (j >= own_lo && j < hi) ? (contiguous ? j : cache_pos(j)) : -1;
        if (pj >= 0) {
          *reinterpret_cast<uint4*>(const_cast<char*>(kbase) + pj * kst + lcol(i)) =
              *reinterpret_cast<const uint4*>(kme + i * kWave * 16);
          *reinterpret_cast<uint4*>(const_cast<char*>(vbase) + pj * vst + lcol(i)) =
              *reinterpret_cast<const uint4*>(vme + i * kWave * 16);
        }
      }
      stores_pending = true;
    }
  };
  // one tile: wait for its loads, free the oldest stage, refill it kStages - 1 tiles ahead, compute
  auto step = [&](int t, auto st) __attribute__((always_inline)) {
    constexpr int S = decltype(st)::value;
    const int kt0 = lo + t * kBN;
    // this wave's loads of tile t have landed: later tiles' loads (at most
    // kStages - 2 of them, LPT operations each) may still be in flight
    const int later = min(kStages - 2, ntiles - 1 - t);
    if (stores_pending || later <= 0) {
      wait_vmcnt<0>();
      stores_pending = false;
    } else if (later == 1) {
      wait_vmcnt<LPT>();
    } else {
      wait_vmcnt<(kStages >= 4 ? 2 * LPT : LPT)>();
    }
    __syncthreads();  // every wave's loads of tile t landed; tile t - 1's stage is free
    char* ks = stage_k(st);
    char* vs = stage_v(st);
    fix_tile(kt0, ks, vs);
    if (t + kStages - 1 < ntiles) issue(t + kStages - 1, std::integral_constant<int, (S + kStages - 1) % kStages>{});
    compute(kt0, ks, vs);
  };

  if (ntiles > 0) issue(0, std::integral_constant<int, 0>{});
  if (kStages >= 3 && ntiles > 1) issue(1, std::integral_constant<int, 1 % kStages>{});
  if (kStages >= 4 && ntiles > 2) issue(2, std::integral_constant<int, 2 % kStages>{});
  for (int t = 0; t < ntiles; t += kStages) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
    if (kStages >= 3 && t + 2 < ntiles) step(t + 2, std::integral_constant<int, 2 % kStages>{});
    if (kStages >= 4 && t + 3 < ntiles) step(t + 3, std::integral_constant<int, 3 % kStages>{});
  }

  if constexpr (kKeyGroups == 2) {
    // ---- the second key group's (m, l, o) join the first's through LDS (the ring is free) ----
    __syncthreads();
    f4v* xo = reinterpret_cast<f4v*>(ring0[0]);          // [row wave][db][lane]: 32 KiB for D = 128
    float2* xml = reinterpret_cast<float2*>(ring1[0]);   // [row wave][lane]
    static_assert(kRowWaves * DB * kWave * 16 <= 2 * TILEB, "merge buffer");
    if (kg == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db) xo[(rw * DB + db) * kWave + lane] = acc_o[db];
      xml[rw * kWave + lane] = make_float2(m_run, l_run);
    }
    __syncthreads();
    if (kg == 1) return;
    const float2 ml1 = xml[rw * kWave + lane];
    const float m_all = fmaxf(m_run, ml1.x);
    const float a0 = fast_exp2(m_run - m_all), a1 = fast_exp2(ml1.x - m_all);
    l_run = l_run * a0 + ml1.y * a1;
    m_run = m_all;
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_o[db] = acc_o[db] * a0 + xo[(rw * DB + db) * kWave + lane] * a1;
  }
  if (!row_ok) return;
  if (span.nsplit > 1) {
    // ---- partials for the merge kernel: o unnormalised, (m, l) once per row ----
    float* po = p.part_o + (pair_row * p.num_splits + split) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) *reinterpret_cast<f4v*>(po + 16 * db + 4 * lq) = acc_o[db];
    if (lq == 0) {
      *reinterpret_cast<float2*>(p.part_ml + (pair_row * p.num_splits + split) * 2) = make_float2(m_run, l_run);
    }
    return;
  }
  // ---- normalise and store: lane holds O[row][16db + 4lq + r] ----
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + out_row * static_cast<int64_t>(D);
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const float o4[4] = {acc_o[db][0] * inv, acc_o[db][1] * inv, acc_o[db][2] * inv, acc_o[db][3] * inv};
    uint2 w;
    w.x = static_cast<uint32_t>(mfma_t<TC>::from_float(o4[0])) | (static_cast<uint32_t>(mfma_t<TC>::from_float(o4[1])) << 16);
    w.y = static_cast<uint32_t>(mfma_t<TC>::from_float(o4[2])) | (static_cast<uint32_t>(mfma_t<TC>::from_float(o4[3])) << 16);
    *reinterpret_cast<uint2*>(op + 16 * db + 4 * lq) = w;
  }
}

// Split merge of the chunk kernel's partials: block (group, q tile, slice of
// kMergeRows rows) combines the slots of the slice's (query, head) rows with
// the log-sum-exp rule.  A chunk workgroup's key span, hence its split count,
// is the same for all its rows, so a block whose tile ran unsplit returns after
// one read of cache_seqlens.  kMergeTPR threads per row, each folding D /
// kMergeTPR consecutive dims over the splits; every slot load of a chunk of
// kMergeCH splits is in flight together (the slot index clamped to the last
// split, not branched on), so up to kMergeCH splits cost one memory round trip
// after the cache_seqlens read (C5's chunk rows have 8).
constexpr int kMergeRows = 32;
constexpr int kMergeTPR = 16;
// slots per round trip: 8 keeps the kernel at ~108 VGPRs, two 512-thread blocks per CU (16: 200
// VGPRs, one block per CU; C5's merges 8.9 and 16.0 us against 7.4 and 11.7 at 8)
#ifndef NC_CHUNK_MERGE_CH
#define NC_CHUNK_MERGE_CH 8
#endif
constexpr int kMergeCH = NC_CHUNK_MERGE_CH;

template <typename TC, int D, int GB, int ROWS, bool IND>
__global__ __launch_bounds__(kMergeRows * kMergeTPR) void chunk_merge_kernel(const ChunkParams p) {
  constexpr int QB = ROWS / GB;
  constexpr int SLICES = ROWS / kMergeRows;
  constexpr int DT = D / kMergeTPR;       // dims per thread
  static_assert(DT % 4 == 0 && ROWS % kMergeRows == 0, "merge shape");
  pin_args(p.fd_qtiles, p.n_groups, p.n_hblocks, p.n_kv_heads, p.t_new, p.seqlens, p.t_max, p.window,
           p.keys_per_split, p.group, p.n_heads, p.num_splits, p.part_ml, p.part_o, p.out);
  const uint32_t pb = blockIdx.x;
  const int slice = static_cast<int>(pb % SLICES);
  uint32_t rem;
  const uint32_t gt = pb / SLICES;
  const uint32_t gq = fdivmod(gt, p.fd_qtiles, rem);
  const int qt = static_cast<int>(rem);
  uint32_t group = gq;
  if (group >= p.n_groups) return;
  const int hb = static_cast<int>(group % static_cast<uint32_t>(p.n_hblocks));
  group /= static_cast<uint32_t>(p.n_hblocks);
  const int hk = static_cast<int>(group % static_cast<uint32_t>(p.n_kv_heads));
  const int64_t b = group / static_cast<uint32_t>(p.n_kv_heads);
  RowQ rq{b * p.t_new, p.t_new};
  if constexpr (IND) {
    if (cache_row(p.cache_idx, p.cache_batch, b, nullptr, false) < 0) return;  // the row was skipped
    rq = row_queries(p.cu_q, p.total_q, b, p.q_bound, nullptr, false);
    if (rq.len < p.len_lo || rq.len > p.len_hi) return;  // another launch's row (or skipped)
  }
  const int q0 = qt * QB;
  if (q0 >= rq.len) return;
  const int q_end = min(q0 + QB, rq.len);
  const int nsplit = chunk_span(p.seqlens[b], q0, q_end, p.t_max, p.window, p.keys_per_split).nsplit;
  if (nsplit <= 1) return;  // the chunk workgroup wrote these outputs itself
  const int row = slice * kMergeRows + static_cast<int>(threadIdx.x) / kMergeTPR;
  const int qi = q0 + row / GB;
  if (qi >= rq.len) return;
  const int h = hk * p.group + hb * GB + row % GB;
  const int d0 = (static_cast<int>(threadIdx.x) % kMergeTPR) * DT;
  const int64_t pair_row = (b * p.t_new + qi) * p.n_heads + h;
  const float* ml = p.part_ml + pair_row * p.num_splits * 2;
  const float* po = p.part_o + pair_row * p.num_splits * D + d0;
  float M = kNegBigC, L = 0.0f, O[DT];
#pragma unroll
  for (int e = 0; e < DT; ++e) O[e] = 0.0f;
  for (int sp0 = 0; sp0 < nsplit; sp0 += kMergeCH) {
    float ms[kMergeCH], ls[kMergeCH];
    float4 os[kMergeCH][DT / 4];
#pragma unroll
    for (int u = 0; u < kMergeCH; ++u) {
      const int sp = min(sp0 + u, nsplit - 1);  // clamped: an in-bounds duplicate, masked below
      const float2 v = *reinterpret_cast<const float2*>(ml + 2 * sp);
      ms[u] = v.x;
      ls[u] = v.y;
#pragma unroll
      for (int e = 0; e < DT / 4; ++e) os[u][e] = *reinterpret_cast<const float4*>(po + static_cast<int64_t>(sp) * D + 4 * e);
    }
    __builtin_amdgcn_sched_barrier(0);  // no use of a slot scheduled between the loads
#pragma unroll
    for (int u = 0; u < kMergeCH; ++u) {
      if (sp0 + u >= nsplit) ls[u] = 0.0f;
    }
    float mx = M;
#pragma unroll
    for (int u = 0; u < kMergeCH; ++u) mx = ls[u] > 0.0f ? fmaxf(mx, ms[u]) : mx;
    const float a = fast_exp2(M - mx);
    L *= a;
#pragma unroll
    for (int e = 0; e < DT; ++e) O[e] *= a;
#pragma unroll
    for (int u = 0; u < kMergeCH; ++u) {
      const bool live = ls[u] > 0.0f;  // l == 0: every key of the split masked for this row, or a duplicate
      const float w = live ? fast_exp2(ms[u] - mx) : 0.0f;
      L = __builtin_fmaf(ls[u], w, L);
#pragma unroll
      for (int e = 0; e < DT / 4; ++e) {
        O[4 * e + 0] = live ? __builtin_fmaf(os[u][e].x, w, O[4 * e + 0]) : O[4 * e + 0];
        O[4 * e + 1] = live ? __builtin_fmaf(os[u][e].y, w, O[4 * e + 1]) : O[4 * e + 1];
        O[4 * e + 2] = live ? __builtin_fmaf(os[u][e].z, w, O[4 * e + 2]) : O[4 * e + 2];
        O[4 * e + 3] = live ? __builtin_fmaf(os[u][e].w, w, O[4 * e + 3]) : O[4 * e + 3];
      }
    }
    M = mx;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + ((rq.tok0 + qi) * p.n_heads + h) * static_cast<int64_t>(D) + d0;
#pragma unroll
  for (int e = 0; e < DT; e += 2) {
    const uint32_t w = mfma_t<TC>::pack2(O[e] * inv, O[e + 1] * inv);
    *reinterpret_cast<uint32_t*>(op + e) = w;
  }
}

template <typename TC, int D, int LK, int ROWS>
hipError_t launch_cr(const ChunkParams& p, int gb, hipStream_t stream) {
  const int64_t n_wg = static_cast<int64_t>(kXcdsC) * p.n_qtiles * p.num_splits * ((p.n_groups + kXcdsC - 1) / kXcdsC);
  const dim3 grid(static_cast<unsigned>(n_wg)), block(kChunkWaves * kWave);
  switch (gb) {
    case 8: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 8, LK, ROWS>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 4, LK, ROWS>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 2, LK, ROWS>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 1, LK, ROWS>), grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

template <typename TC, int D, int LK>
hipError_t launch_ci(const ChunkParams& p, int gb, int rows, hipStream_t stream) {
  return rows == kChunkRowsLarge ? launch_cr<TC, D, LK, kChunkRowsLarge>(p, gb, stream)
                                 : launch_cr<TC, D, LK, kChunkRowsSmall>(p, gb, stream);
}

template <typename TC, int D>
hipError_t launch_c(const ChunkParams& p, int gb, int rows, hipStream_t stream) {
  if (p.pages.table != nullptr) return launch_ci<TC, D, 2>(p, gb, rows, stream);
  return p.indirect ? launch_ci<TC, D, 1>(p, gb, rows, stream) : launch_ci<TC, D, 0>(p, gb, rows, stream);
}

template <typename TC, int D, bool IND, int ROWS>
hipError_t launch_merge_cr(const ChunkParams& p, int gb, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.n_groups * p.n_qtiles * (ROWS / kMergeRows))), block(kMergeRows * kMergeTPR);
  switch (gb) {
    case 8: hipLaunchKernelGGL((chunk_merge_kernel<TC, D, 8, ROWS, IND>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((chunk_merge_kernel<TC, D, 4, ROWS, IND>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((chunk_merge_kernel<TC, D, 2, ROWS, IND>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((chunk_merge_kernel<TC, D, 1, ROWS, IND>), grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

template <typename TC, int D>
hipError_t launch_merge_c(const ChunkParams& p, int gb, int rows, hipStream_t stream) {
  if (p.indirect) {
    return rows == kChunkRowsLarge ? launch_merge_cr<TC, D, true, kChunkRowsLarge>(p, gb, stream)
                                   : launch_merge_cr<TC, D, true, kChunkRowsSmall>(p, gb, stream);
  }
  return rows == kChunkRowsLarge ? launch_merge_cr<TC, D, false, kChunkRowsLarge>(p, gb, stream)
                                 : launch_merge_cr<TC, D, false, kChunkRowsSmall>(p, gb, stream);
}

// Launch parameters of a chunk call (and of its split merge).
ChunkParams make_chunk_params(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                              const RowFilter* rows) {
  ChunkParams p;
  p.q = a.q; p.out = a.out;
  p.kc = static_cast<const char*>(a.k_cache); p.vc = static_cast<const char*>(a.v_cache);
  p.seqlens = a.cache_seqlens;
  p.cache_idx = a.cache_batch_idx; p.cache_batch = a.cache_batch;
  p.cu_q = a.cu_seqlens_q; p.total_q = a.total_q;
  p.pages = page_map(a.page_table, a.page_table_stride, a.page_size, a.num_blocks);
  p.indirect = (a.cache_batch_idx != nullptr || a.cu_seqlens_q != nullptr || a.page_table != nullptr) ? 1 : 0;
  p.q_bound = p.len_hi = static_cast<int32_t>(a.t_new);
  p.len_lo = 0;
  if (rows != nullptr) {
    p.len_lo = rows->lo;
    p.len_hi = rows->hi;
    p.q_bound = rows->bound;
  }
  p.q_sb = a.q_stride_b; p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
  p.kc_sb = a.kc_stride_b; p.kc_st = a.kc_stride_t; p.kc_sh = a.kc_stride_h;
  p.vc_sb = a.vc_stride_b; p.vc_st = a.vc_stride_t; p.vc_sh = a.vc_stride_h;
  p.t_new = static_cast<int32_t>(a.t_new);
  p.t_max = static_cast<int32_t>(a.t_max);
  p.n_heads = static_cast<int32_t>(a.n_heads);
  p.n_kv_heads = static_cast<int32_t>(a.n_kv_heads);
  p.group = plan.group;
  p.n_hblocks = plan.n_hblocks;
  const int qb = plan.chunk_rows / plan.head_block;
  p.n_qtiles = static_cast<int32_t>((a.t_new + qb - 1) / qb);
  p.n_groups = a.batch * a.n_kv_heads * plan.n_hblocks;
  p.window = a.window_left;
  p.scale_log2 = a.softmax_scale * 1.4426950408889634f;
  p.num_splits = plan.chunk_splits;
  p.keys_per_split = plan.chunk_keys_per_split;
  p.part_ml = s.part_ml;
  p.part_o = s.part_o;
  p.fd_members = make_fastdiv(static_cast<uint32_t>(p.n_qtiles * p.num_splits));
  p.fd_qtiles = make_fastdiv(static_cast<uint32_t>(p.n_qtiles));
  p.fd_hblocks = make_fastdiv(static_cast<uint32_t>(p.n_hblocks));
  p.fd_kv_heads = make_fastdiv(static_cast<uint32_t>(p.n_kv_heads));
  p.fused = a.k != nullptr ? 1 : 0;
  p.k_new = static_cast<const char*>(a.k);
  p.v_new = static_cast<const char*>(a.v);
  p.k_sb = a.k_stride_b; p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
  p.v_sb = a.v_stride_b; p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
  p.err = a.error_flag;
  return p;
}

}  // namespace

bool chunk_supports(const nc_attn_args& a) {
  // a key tile's byte span (64 cache rows) must fit the kernel's 32-bit offsets
  const int64_t tile_bytes = kBNMax * std::max(std::abs(a.kc_stride_t), std::abs(a.vc_stride_t)) * 2;
  return a.t_new > 1 && a.q_dtype == a.cache_dtype &&
         (a.cache_dtype == NC_DTYPE_BF16 || a.cache_dtype == NC_DTYPE_F16) &&
         (a.head_dim == 64 || a.head_dim == 128) && tile_bytes < (int64_t(1) << 31);
}

hipError_t launch_chunk(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s, hipStream_t stream,
                        const RowFilter* rows) {
  const ChunkParams p = make_chunk_params(a, plan, s, rows);
  const int wg_rows = plan.chunk_rows;
  if (a.cache_dtype == NC_DTYPE_BF16) {
    return a.head_dim == 64 ? launch_c<bf16, 64>(p, plan.head_block, wg_rows, stream)
                            : launch_c<bf16, 128>(p, plan.head_block, wg_rows, stream);
  }
  return a.head_dim == 64 ? launch_c<f16, 64>(p, plan.head_block, wg_rows, stream)
                          : launch_c<f16, 128>(p, plan.head_block, wg_rows, stream);
}

hipError_t launch_chunk_merge(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                              hipStream_t stream, const RowFilter* rows) {
  const ChunkParams p = make_chunk_params(a, plan, s, rows);
  const int wg_rows = plan.chunk_rows;
  if (a.cache_dtype == NC_DTYPE_BF16) {
    return a.head_dim == 64 ? launch_merge_c<bf16, 64>(p, plan.head_block, wg_rows, stream)
                            : launch_merge_c<bf16, 128>(p, plan.head_block, wg_rows, stream);
  }
  return a.head_dim == 64 ? launch_merge_c<f16, 64>(p, plan.head_block, wg_rows, stream)
                          : launch_merge_c<f16, 128>(p, plan.head_block, wg_rows, stream);
}

}  // namespace nckv
