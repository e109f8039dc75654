// Split-K flash-decoding over the KV cache (nanochat/flash_attention.py:82-89,
// 155-177 with FA3's per-row cache_seqlens), GQA and sliding window.
//
// Work decomposition.  A "unit" is one (kv head, q-head block): the GB query
// heads of a kv head scored together (GQA packing: K/V bytes are read once for
// all of them).  A workgroup is (row b, query t, unit, key split): 4 waves
// that stream `keys_per_split` cache positions of the unit's kv head, tiles
// interleaved across the waves.
//
// Lane layout inside a wave (D = head_dim, VEC = elements per 16 bytes):
//   LPK = D / VEC lanes hold one key row (16 bytes each), KPI = 64 / LPK keys
//   are covered by one 128-bit load instruction.  q . k is a per-lane partial
//   dot product finished by a DPP all-reduce over the LPK lanes, so every lane
//   of a key group ends up with that key's score and no LDS traffic is needed
//   in the streaming loop.  Each key group (`row`) keeps its own online-softmax
//   state (max m, sum l, output o); rows are merged by a butterfly and waves
//   through LDS once at the end.
//
// Split merge: a query whose key range fits one split (always, when the plan
// has one split) gets its output from the decode kernel directly.  Otherwise
// each of its splits writes (o, m, l) partials to the workspace (a split past
// the end of the range does nothing) and the partials are combined with the
// log-sum-exp rule, in one of two ways:
//  - in-kernel (the plan passes `tickets`): partials are written with
//    agent-coherent stores (sc1: written through the XCD's L2), each thread
//    waits for its stores to complete (vmcnt(0)), then the workgroup takes a
//    ticket with an agent-scope atomic add.  The split that draws the last
//    ticket reads the slots back with agent-coherent loads, merges them and
//    resets the ticket to zero.  No L2 write-back or invalidate (the
//    release/acquire fences, buffer_wbl2 / buffer_inv, which measured 3-10x
//    slower on MI355X) and no waiting on other workgroups: the last arrival
//    finds every partial complete.
//  - merge_splits_kernel, the next launch on the stream (decode plans with
//    more groups or workgroups than the in-kernel merge takes): it recomputes
//    the query's split count from cache_seqlens and combines exactly those
//    slots.  (The chunk kernel's splits have a merge kernel of their own.)
// The splits of one (b, t, unit) run on one XCD (workgroups are dispatched
// round-robin over the 8 XCDs), next to each other in launch order.
//
// Fused append (t_new == 1 with k/v given): the split owning position s_b
// takes the new key/value from the k/v inputs (converted to the cache dtype,
// RNE) instead of the cache, and the hb == 0 unit of each kv head stores them
// into the cache.  No other workgroup reads position s_b, so the store does
// not race.

#pragma once

#include <algorithm>
#include <type_traits>

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

// Compile-time tuning (defaults are the measured best on MI355X; see the
// per-option notes).
#ifndef NC_DECODE_WAVES
#define NC_DECODE_WAVES 4       // waves per workgroup (8: -1%, 2: -6%)
#endif
#ifndef NC_DECODE_NI
#define NC_DECODE_NI 8          // 16-byte K (and V) loads per lane per tile, GB < 4
#endif
#ifndef NC_DECODE_NI_GQA
#define NC_DECODE_NI_GQA 4      // same for head blocks of 4 or 8 q heads
#endif
#ifndef NC_DECODE_GQA4_WAVES
#define NC_DECODE_GQA4_WAVES 3  // occupancy floor (waves per SIMD) of 4-head blocks
#endif
#ifndef NC_DECODE_XCD_MAP
#define NC_DECODE_XCD_MAP 1     // 1: the splits of a unit run on the XCD of its merge block
#endif
#ifndef NC_DECODE_NT_LOADS
#define NC_DECODE_NT_LOADS 1    // 1: K/V loads carry the non-temporal hint (+12% measured)
#endif
#ifndef NC_DECODE_PV_DOT2
#define NC_DECODE_PV_DOT2 1     // 1: P.V with v_dot2 on key pairs (packed caches)
#endif
#ifndef NC_DECODE_WIDE_EAGER
// 1: 8-wave workgroups rescale on every tile instead of moving the exponent
// base lazily (2 waves per SIMD: the per-tile vote and branch sit on the
// critical path; C3 decode 0.3864 -> 0.3827 ms/step)
#define NC_DECODE_WIDE_EAGER 1
#endif
#ifndef NC_DECODE_KEY_BYTES
#define NC_DECODE_KEY_BYTES 65536  // default split: this many K bytes per unit (and as many V)
#endif

namespace nckv {

// Kernel arguments of the decode and split-merge kernels (shared by the
// translation units that instantiate them).
struct DecodeParams {
  const void* q;
  void* out;
  char* kc;
  char* vc;
  const void* k_new;
  const void* v_new;
  const int32_t* seqlens;
  int32_t* err;
  const int32_t* cache_idx;  // cache_batch_idx or NULL
  int64_t cache_batch;
  const int32_t* cu_q;       // cu_seqlens_q (packed query tokens) or NULL
  int64_t total_q;
  PageMap pages;             // paged cache (page_table), or pages.table == NULL
  int32_t indirect;          // cache_idx, cu_q or a page table given: per-row lookups (else row b, t_new queries)
  int32_t q_bound, len_lo, len_hi;  // varlen rows: validity bound, and the token counts this launch takes
  float* part_ml;
  float* part_o;
  uint32_t* tickets;  // non-null: splits merge in-kernel (one zeroed counter per group)
  int64_t q_sb, q_st, q_sh;
  int64_t kc_sb, kc_st, kc_sh;
  int64_t vc_sb, vc_st, vc_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int32_t t_new, t_max, n_heads, n_kv_heads, group, n_hblocks;
  int32_t n_units;   // n_kv_heads * n_hblocks
  int64_t n_groups;  // B * t_new * n_units
  int32_t window;
  float scale_log2;
  int32_t q_dtype;
  int32_t num_splits, keys_per_split;
  int32_t fused;
  // length-balanced pieces (LK == 3 kernels): the call's rows, the least
  // 64-key tiles per piece, and the grid size minus n_groups
  int32_t bal_rows, bal_min_tiles, bal_den;
  // fused QK prologue (rotary, RMS norm, scale) on q and the appended k; rope == 0: off
  const void* rope_cos;
  const void* rope_sin;
  int32_t rope, rope_len, rope_dtype, rope_half;  // rope_half = head_dim / 2 (table row length)
  float rope_scale, rope_eps;
  // divisors of the block-index decompositions (every index is < 2^31: the plan caps the grid)
  FastDiv fd_hblocks, fd_kv_heads, fd_t_new, fd_splits, fd_kps;
};

namespace {

constexpr int kWavesPerWG = NC_DECODE_WAVES;
// Wide workgroups: 8 waves, for plans whose groups fit one workgroup per CU
// and need no split (see plan_attention); their LDS merge arrays bound GB * D,
// and GB <= 4 keeps every instantiation within 256 VGPRs.
constexpr int kWideWaves = 8;
constexpr int kWideMaxElems = 512;
constexpr float kNegBig = -1.0e30f;   // finite "minus infinity" for running maxima
// a decode tile moves its exponent base only past this many log2 units
constexpr float kDecodeRebaseSlack = 8.0f;
constexpr int kMaxMergeSplits = 256;  // split cap of the launch plan
constexpr int kXcds = 8;              // MI355X: workgroups go round-robin over 8 XCDs


template <typename TC> struct dot_packed;
template <> struct dot_packed<bf16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  // two fp32 values rounded to nearest-even and packed (x0 low)
  __device__ __forceinline__ static uint32_t pack(float x0, float x1) {
    const v2 v = {static_cast<__bf16>(x0), static_cast<__bf16>(x1)};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct dot_packed<f16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  __device__ __forceinline__ static uint32_t pack(float x0, float x1) {
    const v2 v = {static_cast<_Float16>(x0), static_cast<_Float16>(x1)};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Query fragment of one lane for one head: either the raw 16-byte vector in
// the cache dtype (QPK, packed dot2 path) or VEC fp32 values.
template <typename TC, bool QPK> struct QFrag;
template <typename TC> struct QFrag<TC, true> {
  uint4 w;
  __device__ __forceinline__ float dot(const uint4& k) const {
    float acc = dot_packed<TC>::run(w.x, k.x, 0.0f);
    acc = dot_packed<TC>::run(w.y, k.y, acc);
    acc = dot_packed<TC>::run(w.z, k.z, acc);
    acc = dot_packed<TC>::run(w.w, k.w, acc);
    return acc;
  }
};
template <typename TC> struct QFrag<TC, false> {
  static constexpr int VEC = widen<TC>::N;
  float f[VEC];
  __device__ __forceinline__ float dot(const uint4& k) const {
    float kf[VEC];
    widen<TC>::run(k, kf);
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc = __builtin_fmaf(f[e], kf[e], acc);
    return acc;
  }
};

__device__ __forceinline__ uint4 load16(const char* p) {
#if NC_DECODE_NT_LOADS
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
#else
  return *reinterpret_cast<const uint4*>(p);
#endif
}

// Key range [lo, hi) of query t of row b and its split count.
struct KeyRange {
  int qpos, lo, hi, n, nsplit, kps;
};

// A row's split size is keys_per_split, or, for rows longer than
// num_splits * keys_per_split, the row spread evenly over the num_splits
// splits (multiples of 64 keys): the grid is sized for num_splits per group
// and no split of a long row is left without keys.
__device__ __forceinline__ KeyRange key_range(const DecodeParams& p, int64_t b, int t) {
  KeyRange r;
  r.qpos = p.seqlens[b] + t;  // absolute position of the query
  r.hi = min(r.qpos + 1, p.t_max);
  r.lo = p.window >= 0 ? max(0, r.qpos - p.window) : 0;
  r.n = r.hi - r.lo;
  r.kps = p.keys_per_split;
  if (r.n > r.kps * p.num_splits) r.kps = ((r.n + p.num_splits - 1) / p.num_splits + 63) / 64 * 64;
  r.nsplit = r.n > 0 ? static_cast<int>(fdiv(static_cast<uint32_t>(r.n + r.kps - 1), p.fd_kps)) : 1;
  if (r.kps != p.keys_per_split) r.nsplit = (r.n + r.kps - 1) / r.kps;
  return r;
}

// ---- length-balanced pieces (LK == 3: single-token plain decode) ----
// Row b's key span of T_b 64-key tiles is cut into P_b = max(1, ceil(T_b / c))
// pieces per unit, c being one value for the whole call: the least c >=
// bal_min_tiles with U * sum_b T_b <= c * bal_den (U units per row).  Then
// sum_b U * P_b <= U * sum_b T_b / c + B * U <= bal_den + n_groups = grid
// size, so every piece has a workgroup.  Pieces are numbered row by row, unit
// by unit, piece by piece; workgroup w takes piece w and writes its partial
// to slot w, so the slots of one (row, unit) are contiguous.  Workgroups past
// the last piece exit (they are the last ones dispatched).  Every workgroup
// and merge block derives the numbering from cache_seqlens itself: one load
// per lane for every 64 rows, a wave sum and a wave prefix sum, no LDS.
constexpr int kBalPasses = kDecodeBalMaxRows / kWave;

__device__ __forceinline__ int wave_sum_int(int x) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off /= 2) x += __shfl_xor(x, off, kWave);
  return x;
}

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off *= 2) {
    const int y = __shfl_up(x, off, kWave);
    x += lane >= off ? y : 0;
  }
  return x;
}

// Per lane, rows lane + 64 i: cache_seqlens, pieces per unit, and the
// inclusive prefix of pieces (all units) over the rows up to that one.
struct BalScan {
  int s[kBalPasses];
  int pieces[kBalPasses];
  int incl[kBalPasses];
  int c;  // tiles per piece
};

__device__ __forceinline__ BalScan bal_scan(const DecodeParams& p, int lane) {
  BalScan r;
  const int nrows = p.bal_rows;
  // every pass's load in flight together (row index clamped, masked below)
#pragma unroll
  for (int i = 0; i < kBalPasses; ++i) r.s[i] = p.seqlens[min(lane + i * kWave, nrows - 1)];
  __builtin_amdgcn_sched_barrier(0);
  int tiles[kBalPasses];
  int tsum = 0;
#pragma unroll
  for (int i = 0; i < kBalPasses; ++i) {
    // the key span of the row's query, as key_range computes it
    const int qpos = r.s[i];
    const int hi = min(qpos + 1, p.t_max);
    const int lo = p.window >= 0 ? max(0, qpos - p.window) : 0;
    tiles[i] = lane + i * kWave < nrows ? (max(hi - lo, 0) + 63) >> 6 : 0;
    tsum += tiles[i];
  }
  const int total = wave_sum_int(tsum) * p.n_units;  // the plan bounds it below 2^31
  r.c = max(p.bal_min_tiles, (total + p.bal_den - 1) / p.bal_den);
  int carry = 0;
#pragma unroll
  for (int i = 0; i < kBalPasses; ++i) {
    r.pieces[i] = lane + i * kWave < nrows ? max(1, (tiles[i] + r.c - 1) / r.c) : 0;
    r.incl[i] = carry;
    if (i * kWave < nrows) {
      r.incl[i] = wave_incl_scan(r.pieces[i] * p.n_units, lane) + carry;
      carry = __builtin_amdgcn_readlane(r.incl[i], kWave - 1);
    }
  }
  return r;
}

// The piece of workgroup w: its row, unit, index within the (row, unit), and
// that row's pieces per unit and cache_seqlens.
struct BalPiece {
  bool found;
  int b, u, j, pieces, s, c;
};

__device__ __forceinline__ BalPiece bal_piece(const DecodeParams& p, int w, int lane) {
  const BalScan sc = bal_scan(p, lane);
  BalPiece r{false, 0, 0, 0, 1, 0, sc.c};
  int first = 0;
#pragma unroll
  for (int i = 0; i < kBalPasses; ++i) {
    if (!r.found && i * kWave < p.bal_rows) {
      // the first row whose inclusive prefix exceeds w (the prefix never decreases)
      const uint64_t hit = __ballot(sc.incl[i] > w);
      if (hit != 0) {
        const int l = __builtin_ctzll(hit);
        r.found = true;
        r.b = i * kWave + l;
        r.pieces = __builtin_amdgcn_readlane(sc.pieces[i], l);
        r.s = __builtin_amdgcn_readlane(sc.s[i], l);
        first = __builtin_amdgcn_readlane(sc.incl[i], l) - r.pieces * p.n_units;
      }
    }
  }
  if (r.found) {
    const int rem = w - first;
    r.u = rem / r.pieces;
    r.j = rem - r.u * r.pieces;
  }
  return r;
}

// Group (b, unit u) of a balanced call: its first slot and piece count.
__device__ __forceinline__ void bal_group_slots(const DecodeParams& p, int b, int u, int lane, int& first,
                                                int& pieces) {
  const BalScan sc = bal_scan(p, lane);
  first = 0;
  pieces = 1;
#pragma unroll
  for (int i = 0; i < kBalPasses; ++i) {
    if (b / kWave == i) {
      const int l = b % kWave;
      pieces = __builtin_amdgcn_readlane(sc.pieces[i], l);
      first = __builtin_amdgcn_readlane(sc.incl[i], l) - (p.n_units - u) * pieces;
    }
  }
}

// Key range of a balanced piece: [lo + j * c * 64, ...) of its row's span.
__device__ __forceinline__ KeyRange bal_range(const DecodeParams& p, const BalPiece& bp) {
  KeyRange r;
  r.qpos = bp.s;
  r.hi = min(r.qpos + 1, p.t_max);
  r.lo = p.window >= 0 ? max(0, r.qpos - p.window) : 0;
  r.n = r.hi - r.lo;
  r.kps = bp.c * 64;
  r.nsplit = bp.pieces;
  return r;
}

// Group index -> (b, t, kv head, head block).
struct GroupIdx {
  int64_t b;
  int t, hk, hb;
};

__device__ __forceinline__ GroupIdx group_index(const DecodeParams& p, uint32_t group) {
  GroupIdx r;
  uint32_t rem;
  group = fdivmod(group, p.fd_hblocks, rem);
  r.hb = static_cast<int>(rem);
  group = fdivmod(group, p.fd_kv_heads, rem);
  r.hk = static_cast<int>(rem);
  r.b = fdivmod(group, p.fd_t_new, rem);
  r.t = static_cast<int>(rem);
  return r;
}

// Threads of a merge block: one per VE outputs of the group's GB heads.
__host__ __device__ constexpr int merge_threads(int d, int gb, int ve) {
  return (gb * d / ve + kWave - 1) / kWave * kWave < 256 ? (gb * d / ve + kWave - 1) / kWave * kWave : 256;
}

template <int VE> struct MergeVec;
template <> struct MergeVec<1> {
  typedef float T;
  __device__ __forceinline__ static void get(const T& v, float (&o)[1]) { o[0] = v; }
};
template <> struct MergeVec<4> {
  typedef float4 T;
  __device__ __forceinline__ static void get(const T& v, float (&o)[4]) {
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
};

// Second pass of the decode splits: block g combines the split partials of
// group g's GB heads.  The block recomputes how many splits its query's
// producer used (from the query's key range) and reads exactly those slots;
// a query with one split was written directly by its producer.  Each
// thread owns VE consecutive output elements of one head and folds the slots
// in chunks of CH with every load of a chunk in flight together ((m, l) reads
// are uniform per head), so up to CH splits cost one memory round trip.  The
// number of dependent round trips, not the bytes, sets this kernel's time:
// EAGER kernels (the plan's split count is at most CH) load every allocated
// slot right after the kernel arguments, without waiting for cache_seqlens,
// and mask the slots past the query's split count afterwards.  Shapes:
// <CH 16, VE 1> (few VGPRs, high occupancy: many merge blocks, few splits)
// and <CH 32, VE 4> (more than 16 splits: one or two round trips for up to
// 64 splits).  Slots with l == 0 (every key of the split masked for this
// query) contribute nothing.
// IND: the launch passes cache_batch_idx or cu_seqlens_q (per-row lookups).
// Plain launches use IND = false kernels, which hold no lookup code at all:
// its mere presence, never executed, measured 3% slower on the C5 batch.
template <int D, int GB, int CH, int VE, bool IND, bool EAGER>
__global__ __launch_bounds__(256) void merge_splits_kernel(const DecodeParams p) {
  typedef typename MergeVec<VE>::T VT;
  constexpr int TPH = D / VE;  // threads per head
  pin_args(p.fd_hblocks, p.fd_kv_heads, p.fd_t_new, p.fd_kps, p.seqlens, p.part_ml, p.part_o, p.out,
           p.num_splits, p.keys_per_split, p.t_new, p.t_max, p.window, p.n_heads, p.group, p.q_dtype);
  const GroupIdx gi = group_index(p, blockIdx.x);
  RowQ rq{gi.b * p.t_new, p.t_new};
  if constexpr (IND) {
    if (cache_row(p.cache_idx, p.cache_batch, gi.b, nullptr, false) < 0) return;  // the row was skipped
    rq = row_queries(p.cu_q, p.total_q, gi.b, p.q_bound, nullptr, false);
    // no such query in this row, the row is another launch's, or it was skipped
    if (rq.len < p.len_lo || rq.len > p.len_hi || gi.t >= rq.len) return;
  }
  int nsplit = 0;
  if constexpr (!EAGER) {
    nsplit = key_range(p, gi.b, gi.t).nsplit;
    if (nsplit <= 1) return;
  }
  const int lim = EAGER ? p.num_splits : nsplit;
  const int64_t pair0 = (gi.b * p.t_new + gi.t) * p.n_heads + gi.hk * p.group + gi.hb * GB;
  const int64_t opair0 = (rq.tok0 + gi.t) * p.n_heads + gi.hk * p.group + gi.hb * GB;  // row of `out`
  for (int e = threadIdx.x; e < GB * TPH; e += blockDim.x) {
    const int g = e / TPH, d0 = (e % TPH) * VE;
    const float* ml = p.part_ml + (pair0 + g) * p.num_splits * 2;
    const float* po = p.part_o + (pair0 + g) * p.num_splits * D + d0;
    float M = kNegBig, L = 0.0f, O[VE];
#pragma unroll
    for (int v = 0; v < VE; ++v) O[v] = 0.0f;
    for (int sp0 = 0; sp0 < lim; sp0 += CH) {
      float ms[CH], ls[CH];
      VT os[CH];
      // Slot indices past `lim` are clamped to the last allocated slot (an
      // in-bounds duplicate, masked below) rather than branched around: a
      // branch per slot made the compiler wait for each load before issuing
      // the next (one round trip per slot).
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int sp = min(sp0 + u, lim - 1);
        const float2 v = *reinterpret_cast<const float2*>(ml + 2 * sp);
        ms[u] = v.x;
        ls[u] = v.y;
        os[u] = *reinterpret_cast<const VT*>(po + static_cast<int64_t>(sp) * D);
      }
      __builtin_amdgcn_sched_barrier(0);  // no use of a slot scheduled between the loads
      // eager: the query's split count, read while the slot loads are in flight
      if constexpr (EAGER) nsplit = key_range(p, gi.b, gi.t).nsplit;
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (sp0 + u >= nsplit) ls[u] = 0.0f;  // slot not written by this call, or a clamped duplicate
      }
      float mx = M;
#pragma unroll
      for (int u = 0; u < CH; ++u) mx = ls[u] > 0.0f ? fmaxf(mx, ms[u]) : mx;
      const float a = fast_exp2(M - mx);
      L *= a;
#pragma unroll
      for (int v = 0; v < VE; ++v) O[v] *= a;
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const bool live = ls[u] > 0.0f;
        const float w = live ? fast_exp2(ms[u] - mx) : 0.0f;
        L = __builtin_fmaf(ls[u], w, L);
        float ov[VE];
        MergeVec<VE>::get(os[u], ov);
#pragma unroll
        for (int v = 0; v < VE; ++v) O[v] = live ? __builtin_fmaf(ov[v], w, O[v]) : O[v];
      }
      M = mx;
    }
    if (nsplit <= 1) return;  // the producer wrote this query's output
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const int64_t o0 = (opair0 + g) * D + d0;
#pragma unroll
    for (int v = 0; v < VE; ++v) store_any(p.out, o0 + v, p.q_dtype, O[v] * inv);
  }
}

template <int D, int GB, bool IND>
void launch_merge_i(const DecodeParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.n_groups));
  if (p.num_splits > 32) {
    hipLaunchKernelGGL((merge_splits_kernel<D, GB, 32, 4, IND, false>), grid, dim3(merge_threads(D, GB, 4)), 0,
                       stream, p);
  } else if (p.num_splits > 16) {
    hipLaunchKernelGGL((merge_splits_kernel<D, GB, 32, 4, IND, true>), grid, dim3(merge_threads(D, GB, 4)), 0,
                       stream, p);
  } else {
    hipLaunchKernelGGL((merge_splits_kernel<D, GB, 16, 1, IND, true>), grid, dim3(merge_threads(D, GB, 1)), 0,
                       stream, p);
  }
}

// Merge of length-balanced pieces (LK == 3 decode kernels): block g combines
// the contiguous partial slots of group g, which it locates from
// cache_seqlens as the producers did.  S slices of TPG threads: thread (k, e)
// owns VE outputs e of the group and folds the slots k, k + S, k + 2S, ...,
// CH of them per round trip (every load of a round trip in flight together);
// the slices then combine through LDS.  With GB * D = 512 (GQA 16/4 at 128),
// 4 slices of 128 threads take up to 64 slots in one round trip.
template <int D, int GB>
struct BalMerge {
  static constexpr int VE = 4;
  static constexpr int TPG = GB * D / VE;
  static constexpr int S = TPG >= 512 ? 1 : (512 / TPG > 16 ? 16 : 512 / TPG);
  static constexpr int NT = S * TPG;
  static constexpr int CH = 16;
  static_assert(NT % kWave == 0 && NT <= 1024, "merge block");
};

template <int D, int GB>
__global__ __launch_bounds__((BalMerge<D, GB>::NT)) void merge_bal_kernel(const DecodeParams p) {
  using M_ = BalMerge<D, GB>;
  constexpr int VE = M_::VE, TPG = M_::TPG, S = M_::S, CH = M_::CH;
  constexpr int TPH = D / VE;  // threads per head
  __shared__ float sm_m[S][TPG];
  __shared__ float sm_l[S][TPG];
  __shared__ float4 sm_o[S][TPG];
  pin_args(p.fd_hblocks, p.fd_kv_heads, p.fd_t_new, p.seqlens, p.part_ml, p.part_o, p.out, p.bal_rows,
           p.bal_min_tiles, p.bal_den, p.n_units, p.t_max, p.window, p.n_heads, p.group, p.q_dtype);
  const GroupIdx gi = group_index(p, blockIdx.x);
  int first, nsplit;
  bal_group_slots(p, static_cast<int>(gi.b), gi.hk * p.n_hblocks + gi.hb, threadIdx.x % kWave, first, nsplit);
  if (nsplit <= 1) return;  // one piece: its workgroup wrote the output
  const int k = threadIdx.x / TPG, e = threadIdx.x % TPG;
  const int g = e / TPH, d0 = (e % TPH) * VE;
  const int64_t slot0 = static_cast<int64_t>(first) * GB + g;  // slot `first`, head g; slots step GB
  const float* ml = p.part_ml + slot0 * 2;
  const float* po = p.part_o + slot0 * D + d0;
  float M = kNegBig, L = 0.0f, O[VE];
#pragma unroll
  for (int v = 0; v < VE; ++v) O[v] = 0.0f;
  for (int sp0 = k; sp0 < nsplit; sp0 += S * CH) {
    float ms[CH], ls[CH];
    float4 os[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int sp = min(sp0 + u * S, nsplit - 1);  // clamped: an in-bounds duplicate, masked below
      const float2 v = *reinterpret_cast<const float2*>(ml + static_cast<int64_t>(2 * GB) * sp);
      ms[u] = v.x;
      ls[u] = v.y;
      os[u] = *reinterpret_cast<const float4*>(po + static_cast<int64_t>(GB) * D * sp);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (sp0 + u * S >= nsplit) ls[u] = 0.0f;
    }
    float mx = M;
#pragma unroll
    for (int u = 0; u < CH; ++u) mx = ls[u] > 0.0f ? fmaxf(mx, ms[u]) : mx;
    const float a = fast_exp2(M - mx);
    L *= a;
#pragma unroll
    for (int v = 0; v < VE; ++v) O[v] *= a;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const bool live = ls[u] > 0.0f;
      const float w = live ? fast_exp2(ms[u] - mx) : 0.0f;
      L = __builtin_fmaf(ls[u], w, L);
      const float ov[VE] = {os[u].x, os[u].y, os[u].z, os[u].w};
#pragma unroll
      for (int v = 0; v < VE; ++v) O[v] = live ? __builtin_fmaf(ov[v], w, O[v]) : O[v];
    }
    M = mx;
  }
  sm_m[k][e] = M;
  sm_l[k][e] = L;
  sm_o[k][e] = make_float4(O[0], O[1], O[2], O[3]);
  __syncthreads();
  if (k != 0) return;
  float mx = kNegBig;
#pragma unroll
  for (int kk = 0; kk < S; ++kk) mx = sm_l[kk][e] > 0.0f ? fmaxf(mx, sm_m[kk][e]) : mx;
  float Lt = 0.0f, Ot[VE] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kk = 0; kk < S; ++kk) {
    const float l = sm_l[kk][e];
    const float w = l > 0.0f ? fast_exp2(sm_m[kk][e] - mx) : 0.0f;
    const float4 o = sm_o[kk][e];
    Lt = __builtin_fmaf(l, w, Lt);
    Ot[0] = __builtin_fmaf(o.x, w, Ot[0]);
    Ot[1] = __builtin_fmaf(o.y, w, Ot[1]);
    Ot[2] = __builtin_fmaf(o.z, w, Ot[2]);
    Ot[3] = __builtin_fmaf(o.w, w, Ot[3]);
  }
  const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
  const int64_t opair0 = gi.b * p.n_heads + gi.hk * p.group + gi.hb * GB;  // t_new = 1, row b's query
  const int64_t o0 = (opair0 + g) * D + d0;
#pragma unroll
  for (int v = 0; v < VE; ++v) store_any(p.out, o0 + v, p.q_dtype, Ot[v] * inv);
}

template <int D, int GB>
void launch_merge_bal(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((merge_bal_kernel<D, GB>), dim3(static_cast<unsigned>(p.n_groups)), dim3(BalMerge<D, GB>::NT),
                     0, stream, p);
}

template <int D, int GB>
void launch_merge_g(const DecodeParams& p, hipStream_t stream) {
  if (p.indirect) {
    launch_merge_i<D, GB, true>(p, stream);
  } else {
    launch_merge_i<D, GB, false>(p, stream);
  }
}

// Agent-coherent accesses for the in-kernel split merge: relaxed agent-scope
// atomics compile to plain vector loads/stores with the sc1 bit (coherent
// across the XCDs' L2s), without the L2 write-back / invalidate that a
// release / acquire fence adds.
__device__ __forceinline__ void coherent_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// slots folded per round trip by the in-kernel merge (the default split
// gives at most 8 slots per row at 2048 keys)
constexpr int kInKernelMergeChunk = 8;
// Paged cache: a split's page numbers are staged in LDS when it spans at most
// this many pages (else each key reads the table itself).
constexpr int kMaxSplitPages = 64;

// LK: 0 plain launch (no lookup code); 1 cache_batch_idx / cu_seqlens_q
// lookups; 2 those and a page table; 3 plain launch of length-balanced
// pieces.  Paged launches have kernels of their own so the lookup kernels
// keep the code they had without paging.
template <typename TC, bool QPK, int D, int GB, int NW, int LK>
// Occupancy floor per head block: 3 waves per SIMD (168 VGPRs) for blocks of
// 4 q heads, 2 (256) for 8; the compiler otherwise spends registers on
// issuing the next tile's loads early and drops a wave.
__global__ __launch_bounds__(NW * kWave, GB == 4 ? NC_DECODE_GQA4_WAVES : (GB == 8 ? 2 : 1)) void decode_attn_kernel(const DecodeParams p) {
  constexpr int VEC = widen<TC>::N;
  constexpr int LPK = D / VEC;            // lanes per key row
  constexpr int KPI = kWave / LPK;        // keys per load instruction
  constexpr int NI = (GB >= 4) ? NC_DECODE_NI_GQA : NC_DECODE_NI;  // loads per tile (K and V each)
  constexpr int TILE = KPI * NI;          // keys per wave tile
  constexpr int EB = elem<TC>::kBytes;
  static_assert(LPK >= 1 && LPK <= kWave && KPI * LPK == kWave, "head_dim / dtype");

  __shared__ float sm_o[NW][GB][D];
  __shared__ float sm_m[NW][GB];
  __shared__ float sm_l[NW][GB];
  __shared__ float sm_w[NW][GB];
  __shared__ float sm_L[GB];
  __shared__ int sm_last;  // this split drew the group's last ticket: it merges

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // the wave index, provably wave-uniform (so tile bounds and masks derived
  // from it compile to scalar branches, not per-lane exec masking)
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int row = lane / LPK;
  const int col = lane % LPK;

  // the arguments on the path to the first K/V load, in one batch (head
  // blocks of 4 or 8 q heads: measured 2% slower, their loads already batch)
  if constexpr (GB < 4) pin_args(p.fd_splits, p.n_groups, p.fd_hblocks, p.fd_kv_heads, p.fd_t_new, p.fd_kps, p.seqlens, p.t_max,
           p.window, p.keys_per_split, p.num_splits, p.t_new, p.n_heads, p.group, p.fused, p.kc, p.vc, p.kc_sb,
           p.kc_sh, p.kc_st, p.vc_sb, p.vc_sh, p.vc_st);

  constexpr bool kLookups = LK == 1 || LK == 2;
  constexpr bool kBal = LK == 3;

  // ---- block -> (group, split) ----
  uint32_t group;
  int split;
  [[maybe_unused]] BalPiece bp;
  if constexpr (kBal) {
    bp = bal_piece(p, static_cast<int>(blockIdx.x), lane);
    if (!bp.found) return;  // past the call's last piece
    group = static_cast<uint32_t>(bp.b * p.n_units + bp.u);
    split = bp.j;
  } else {
#if NC_DECODE_XCD_MAP
    const uint32_t pb = blockIdx.x;
    uint32_t split_u;
    const uint32_t gq = fdivmod(pb / kXcds, p.fd_splits, split_u);
    split = static_cast<int>(split_u);
    group = gq * kXcds + pb % kXcds;
    if (group >= p.n_groups) return;
#else
    uint32_t split_u;
    group = fdivmod(blockIdx.x, p.fd_splits, split_u);
    split = static_cast<int>(split_u);
#endif
  }
  const GroupIdx gi = group_index(p, group);
  const int64_t b = gi.b;
  const int t = gi.t, hk = gi.hk, hb = gi.hb;
  // cache row and queries of batch row b (cache_batch_idx, cu_seqlens_q); an
  // invalid entry skips the row in every workgroup of it
  int64_t cb = b;
  RowQ rq{b * p.t_new, p.t_new};
  if constexpr (kLookups) {
    const bool report = split == 0 && t == 0 && hk == 0 && hb == 0 && threadIdx.x == 0;
    if constexpr (LK == 2) {
      cb = 0;  // paged: every position is addressed through the page table
    } else {
      cb = cache_row(p.cache_idx, p.cache_batch, b, p.err, report);
      if (cb < 0) return;
    }
    rq = row_queries(p.cu_q, p.total_q, b, p.q_bound, p.err, report);
    // no such query in this row, the row is another launch's, or it was skipped
    if (rq.len < p.len_lo || rq.len > p.len_hi || t >= rq.len) return;
  }

  const KeyRange kr = [&] {
    if constexpr (kBal) {
      return bal_range(p, bp);
    } else {
      return key_range(p, b, t);
    }
  }();
  const int64_t pair0 = (b * p.t_new + t) * p.n_heads + hk * p.group + hb * GB;  // (b, t, first q head)
  const int64_t opair0 = (rq.tok0 + t) * p.n_heads + hk * p.group + hb * GB;     // its row of `out`
  // partial slots: (pair, split) order, or (piece, head) order for balanced
  // pieces (this piece is slot blockIdx.x, the group's pieces contiguous)
  const int64_t slot_first = kBal ? (static_cast<int64_t>(blockIdx.x) - split) * GB : pair0 * p.num_splits;
  const int64_t slot_head = kBal ? 1 : p.num_splits;  // head g's slots start at slot_first + g * slot_head
  constexpr int64_t kSlotStep = kBal ? GB : 1;        // from one split's slot to the next one's
  const int64_t slot_mine = slot_first + split * kSlotStep;
  if (split >= kr.nsplit) return;  // past this query's keys: the merge never reads this slot
  const int qpos = kr.qpos;
  const int k0 = kr.lo + split * kr.kps;
  const int k1 = kr.n > 0 ? min(k0 + kr.kps, kr.hi) : k0;
  const bool new_in_range = p.fused && qpos >= 0 && qpos < p.t_max;
  const bool own_new = new_in_range && kr.n > 0 && k1 == qpos + 1;
  const int kc_end = own_new ? k1 - 1 : k1;       // keys read from the cache: [k0, kc_end)

  // paged cache: the page numbers of this split's positions [k0, k1), read
  // from the table once into LDS (entries outside the pool become -1 and set
  // NC_DEVERR_PAGE).  Per-key lookups then wait on LDS, not on the vector
  // memory counter the K/V loads in flight also use.
  [[maybe_unused]] int page_lo = 0;
  [[maybe_unused]] bool pages_staged = false;
  [[maybe_unused]] const int32_t* sm_pg = nullptr;
  if constexpr (LK == 2) {
    __shared__ int32_t sm_pages[kMaxSplitPages];
    page_lo = k0 >> p.pages.shift;
    const int npages = k1 > k0 ? ((k1 - 1) >> p.pages.shift) - page_lo + 1 : 0;
    pages_staged = npages <= kMaxSplitPages;
    if (pages_staged) {
      for (int i = tid; i < npages; i += NW * kWave) {
        const int32_t blk = p.pages.table[b * p.pages.stride + page_lo + i];
        const bool ok = blk >= 0 && blk < p.pages.n_blocks;
        if (!ok && p.err != nullptr) atomicOr(p.err, NC_DEVERR_PAGE);
        sm_pages[i] = ok ? blk : -1;
      }
      __syncthreads();
    }
    sm_pg = sm_pages;
  }
  // physical row of cached position j (paged: its page-table slot; -1 if not addressable)
  auto paged_row = [&](int j) -> int64_t {
    if (pages_staged) {
      const int32_t blk = sm_pg[(j >> p.pages.shift) - page_lo];
      return blk >= 0 ? ((static_cast<int64_t>(blk) << p.pages.shift) | (j & ((1 << p.pages.shift) - 1))) : -1;
    }
    return page_pos(p.pages, b, j, p.err);
  };

  if (p.fused && (qpos < 0 || qpos >= p.t_max) && split == 0 && hk == 0 && hb == 0 && tid == 0 &&
      p.err != nullptr) {
    atomicOr(p.err, NC_DEVERR_OVERFLOW);
  }

  const int h0 = hk * p.group + hb * GB;          // first q head of this unit

  // table row of the fused QK prologue: the query's position, clamped into the table
  const int rope_row = min(max(qpos, 0), p.rope_len - 1);
  if (p.rope && (qpos < 0 || qpos >= p.rope_len) && split == 0 && hk == 0 && hb == 0 && tid == 0 &&
      p.err != nullptr) {
    atomicOr(p.err, NC_DEVERR_ROPE_RANGE);
  }

  QFrag<TC, QPK> qf[GB];  // filled once the first tile's loads are in flight

  float m[GB], l[GB], o[GB][VEC];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = kNegBig;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[g][e] = 0.0f;
  }

  const char* kbase = p.kc + (cb * p.kc_sb + hk * p.kc_sh + col * VEC) * EB;
  const char* vbase = p.vc + (cb * p.vc_sb + hk * p.vc_sh + col * VEC) * EB;
  const int64_t kst = p.kc_st * EB;
  const int64_t vst = p.vc_st * EB;

  // ---- stream the split's cache keys, TILE keys per wave per step ----
  auto load_tile = [&](int base, uint4 (&kv)[NI], uint4 (&vv)[NI]) {
    if constexpr (LK == 2) {  // paged cache: each key's slot from the page table
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int j = base + i * KPI + row;
        const int64_t pj = j < kc_end ? paged_row(j) : -1;
        kv[i] = pj >= 0 ? load16(kbase + pj * kst) : make_uint4(0, 0, 0, 0);
        vv[i] = pj >= 0 ? load16(vbase + pj * vst) : make_uint4(0, 0, 0, 0);
      }
      return;
    }
    // the index is clamped to the split's last cached key (load_tile runs only
    // while base < kc_end) rather than branched on: keys past the end load a
    // duplicate that the tile step masks (weight 0), and the loads need no
    // zero-filled copies
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int j = min(base + i * KPI + row, kc_end - 1);
      kv[i] = load16(kbase + j * kst);
      vv[i] = load16(vbase + j * vst);
    }
  };
  // One tile step.  Scores stay unscaled (q . k) and the weights are
  // exp2(s * scale_log2 - m) in one fma.  m[g] is an exponent base (log2
  // units) that moves only when a score of the tile exceeds it by more than
  // kDecodeRebaseSlack, so most tiles skip the rescale of o and l (the
  // weights then reach up to 2^8 before the final normalisation).  Only a
  // tile that runs past the split's end masks its keys (MASKED).
  auto consume_tile = [&](auto masked, int base, const uint4 (&kv)[NI], const uint4 (&vv)[NI]) {
    constexpr bool kMasked = decltype(masked)::value;
    const float c2 = p.scale_log2;
    float sc[GB][NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool valid = !kMasked || base + i * KPI + row < kc_end;
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const float d = group_sum<LPK>(qf[g].dot(kv[i]));
        sc[g][i] = valid ? d : -__builtin_inff();
      }
    }
    float mt[GB];
    bool grow = false;
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float x = sc[g][0];
#pragma unroll
      for (int i = 1; i < NI; ++i) x = fmaxf(x, sc[g][i]);
      mt[g] = x * c2;
      grow = grow || mt[g] > m[g] + kDecodeRebaseSlack;
    }
    if (NC_DECODE_WIDE_EAGER && NW == kWideWaves ? true : __any(grow)) {
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const float mn = fmaxf(m[g], mt[g]);
        const float alpha = fast_exp2(m[g] - mn);
        m[g] = mn;
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[g][e] *= alpha;
      }
    }
    if constexpr (QPK && NC_DECODE_PV_DOT2 && NI % 2 == 0) {
      // P.V on key pairs with v_dot2: P rounded to the cache dtype (as in
      // flash-attention's second matmul), the two keys' elements of one dim
      // paired by v_perm; the sum l stays in fp32.
#pragma unroll
      for (int i = 0; i < NI; i += 2) {
        const uint32_t a[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
        const uint32_t c[4] = {vv[i + 1].x, vv[i + 1].y, vv[i + 1].z, vv[i + 1].w};
        uint32_t pairs[VEC];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pairs[2 * w] = __builtin_amdgcn_perm(c[w], a[w], 0x05040100u);      // element 2w of keys i, i+1
          pairs[2 * w + 1] = __builtin_amdgcn_perm(c[w], a[w], 0x07060302u);  // element 2w+1
        }
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          const float p0 = fast_exp2(__builtin_fmaf(sc[g][i], c2, -m[g]));
          const float p1 = fast_exp2(__builtin_fmaf(sc[g][i + 1], c2, -m[g]));
          l[g] += p0 + p1;
          const uint32_t pp = dot_packed<TC>::pack(p0, p1);
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[g][e] = dot_packed<TC>::run(pp, pairs[e], o[g][e]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float vf[VEC];
        widen<TC>::run(vv[i], vf);
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          const float pr = fast_exp2(__builtin_fmaf(sc[g][i], c2, -m[g]));
          l[g] += pr;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[g][e] = __builtin_fmaf(pr, vf[e], o[g][e]);
        }
      }
    }
  };
  constexpr int STEP = NW * TILE;
  // the first tile's loads go out before q is prepared (the QK prologue's
  // table loads and shuffles then overlap them); afterwards each tile's loads
  // are issued right after the previous one is consumed
  uint4 kv[NI], vv[NI];
  int base = k0 + wave * TILE;
  if (base < kc_end) load_tile(base, kv, vv);
  float rcos[VEC], rsin[VEC];  // this lane's table entries (fused QK prologue)
  if (p.rope) {
    const int64_t toff = static_cast<int64_t>(rope_row) * p.rope_half + (col % (LPK / 2)) * VEC;
    load_table_vec<VEC>(p.rope_cos, toff, p.rope_dtype, rcos);
    load_table_vec<VEC>(p.rope_sin, toff, p.rope_dtype, rsin);
  }
  // ---- query fragments (raw, or through the QK prologue and rounded to q's dtype), built while
  // the first tile's K/V loads are in flight ----
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const int64_t qoff = token_offset(p.cu_q, rq, b, t, p.q_sb, p.q_st) + (h0 + g) * p.q_sh + col * VEC;
    if (p.rope) {
      float xf[VEC];
      if constexpr (QPK) {
        widen<TC>::run(*reinterpret_cast<const uint4*>(static_cast<const char*>(p.q) + qoff * EB), xf);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xf[e] = load_any(p.q, qoff + e, p.q_dtype);
      }
      qk_prologue_apply<LPK, VEC>(xf, col, rcos, rsin, p.rope_scale, p.rope_eps);
      if constexpr (QPK) {
        qf[g].w = pack_cache_vec<TC>(xf);  // q's dtype is the cache dtype on this path
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) qf[g].f[e] = round_to(xf[e], p.q_dtype);
      }
    } else if constexpr (QPK) {
      qf[g].w = *reinterpret_cast<const uint4*>(static_cast<const char*>(p.q) + qoff * EB);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qf[g].f[e] = load_any(p.q, qoff + e, p.q_dtype);
    }
  }

  while (base < kc_end) {
    consume_tile(std::true_type{}, base, kv, vv);
    base += STEP;
    if (base < kc_end) load_tile(base, kv, vv);
  }

  // ---- the appended token (fused path): read from k/v, store into the cache ----
  if (own_new && wave == NW - 1) {
    const int64_t koff = token_offset(p.cu_q, rq, b, 0, p.k_sb, p.k_st) + hk * p.k_sh + col * VEC;
    const int64_t voff = token_offset(p.cu_q, rq, b, 0, p.v_sb, p.v_st) + hk * p.v_sh + col * VEC;
    uint4 kn;
    if (p.rope) {
      float xf[VEC];
      if constexpr (QPK) {
        widen<TC>::run(*reinterpret_cast<const uint4*>(static_cast<const char*>(p.k_new) + koff * EB), xf);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xf[e] = load_any(p.k_new, koff + e, p.q_dtype);
      }
      qk_prologue_apply<LPK, VEC>(xf, col, rcos, rsin, p.rope_scale, p.rope_eps);
      kn = pack_cache_vec<TC>(xf);
    } else {
      kn = load_as_cache_vec<TC>(p.k_new, koff, p.q_dtype);
    }
    const uint4 vn = load_as_cache_vec<TC>(p.v_new, voff, p.q_dtype);
    if (hb == 0 && row == 0) {
      int64_t pq = qpos;
      if constexpr (LK == 2) pq = paged_row(qpos);
      if (pq >= 0) {
        *reinterpret_cast<uint4*>(const_cast<char*>(kbase) + pq * kst) = kn;
        *reinterpret_cast<uint4*>(const_cast<char*>(vbase) + pq * vst) = vn;
      }
    }
    float vf[VEC];
    widen<TC>::run(vn, vf);
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const float d = group_sum<LPK>(qf[g].dot(kn)) * p.scale_log2;
      const float sc = row == 0 ? d : -__builtin_inff();
      const float mn = fmaxf(m[g], sc);
      const float alpha = fast_exp2(m[g] - mn);
      const float pr = fast_exp2(sc - mn);
      m[g] = mn;
      l[g] = l[g] * alpha + pr;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[g][e] = __builtin_fmaf(pr, vf[e], o[g][e] * alpha);
    }
  }

  // ---- merge the KPI key groups of each wave (butterfly over lane offsets LPK..32) ----
#pragma unroll
  for (int off = LPK; off < kWave; off *= 2) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const float mo = __shfl_xor(m[g], off, kWave);
      const float lo_ = __shfl_xor(l[g], off, kWave);
      const float mn = fmaxf(m[g], mo);
      const float a_self = fast_exp2(m[g] - mn);
      const float a_other = fast_exp2(mo - mn);
      l[g] = l[g] * a_self + lo_ * a_other;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float oo = __shfl_xor(o[g][e], off, kWave);
        o[g][e] = o[g][e] * a_self + oo * a_other;
      }
      m[g] = mn;
    }
  }
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) sm_o[wave][g][col * VEC + e] = o[g][e];
      if (col == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves ----
  if (tid < GB) {
    const int g = tid;
    float mx = sm_m[0][g];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, sm_m[w][g]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(sm_m[w][g] - mx);
      sm_w[w][g] = wt;
      L += sm_l[w][g] * wt;
    }
    sm_L[g] = L;
    sm_m[0][g] = mx;  // merged max, read below
  }
  __syncthreads();

  if (kr.nsplit == 1) {
    for (int idx = tid; idx < GB * D; idx += NW * kWave) {
      const int g = idx / D, d = idx % D;
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) acc += sm_o[w][g][d] * sm_w[w][g];
      const float L = sm_L[g];
      store_any(p.out, (opair0 + g) * D + d, p.q_dtype, L > 0.0f ? acc / L : 0.0f);
    }
    return;
  }
  if (p.tickets == nullptr) {  // merge_splits_kernel combines the partials
    for (int idx = tid; idx < GB * D; idx += NW * kWave) {
      const int g = idx / D, d = idx % D;
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) acc += sm_o[w][g][d] * sm_w[w][g];
      p.part_o[(slot_mine + g * slot_head) * D + d] = acc;
    }
    if (tid < GB) {
      *reinterpret_cast<float2*>(p.part_ml + (slot_mine + tid * slot_head) * 2) =
          make_float2(sm_m[0][tid], sm_L[tid]);
    }
    return;
  }

  // ---- in-kernel merge: publish the partial, take a ticket, the last split merges ----
  for (int idx = tid; idx < GB * D; idx += NW * kWave) {
    const int g = idx / D, d = idx % D;
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += sm_o[w][g][d] * sm_w[w][g];
    coherent_store(p.part_o + (slot_mine + g * slot_head) * D + d, acc);
  }
  if (tid < GB) {
    float* ml = p.part_ml + (slot_mine + tid * slot_head) * 2;
    coherent_store(ml, sm_m[0][tid]);
    coherent_store(ml + 1, sm_L[tid]);
  }
  // every thread's partial stores have completed (reached the agent's point
  // of coherence) before the barrier, hence before the ticket is taken
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t tk = __hip_atomic_fetch_add(p.tickets + group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = tk + 1 == static_cast<uint32_t>(kr.nsplit);
    // every split of this group has drawn its ticket: back to zero for the next call
    if (last) __hip_atomic_store(p.tickets + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_last = last;
  }
  __syncthreads();
  if (!sm_last) return;
  __asm__ volatile("" ::: "memory");
  const int nsplit = kr.nsplit;
  for (int idx = tid; idx < GB * D; idx += NW * kWave) {
    const int g = idx / D, d = idx % D;
    const float* ml = p.part_ml + (slot_first + g * slot_head) * 2;
    const float* po = p.part_o + (slot_first + g * slot_head) * D + d;
    float M = kNegBig, L = 0.0f, O = 0.0f;
    for (int sp0 = 0; sp0 < nsplit; sp0 += kInKernelMergeChunk) {
      float ms[kInKernelMergeChunk], ls[kInKernelMergeChunk], os[kInKernelMergeChunk];
#pragma unroll
      for (int u = 0; u < kInKernelMergeChunk; ++u) {
        // clamped, not branched: every load of the chunk in flight together
        const int sp = min(sp0 + u, nsplit - 1);
        ms[u] = coherent_load(ml + 2 * kSlotStep * sp);
        ls[u] = coherent_load(ml + 2 * kSlotStep * sp + 1);
        os[u] = coherent_load(po + kSlotStep * D * sp);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kInKernelMergeChunk; ++u) {
        if (sp0 + u >= nsplit) ls[u] = 0.0f;  // a clamped duplicate
      }
      float mx = M;
#pragma unroll
      for (int u = 0; u < kInKernelMergeChunk; ++u) mx = ls[u] > 0.0f ? fmaxf(mx, ms[u]) : mx;
      const float a = fast_exp2(M - mx);
      L *= a;
      O *= a;
#pragma unroll
      for (int u = 0; u < kInKernelMergeChunk; ++u) {
        const bool live = ls[u] > 0.0f;
        const float w = live ? fast_exp2(ms[u] - mx) : 0.0f;
        L = __builtin_fmaf(ls[u], w, L);
        O = live ? __builtin_fmaf(os[u], w, O) : O;
      }
      M = mx;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    store_any(p.out, (opair0 + g) * D + d, p.q_dtype, O * inv);
  }
}


template <typename TC, bool QPK, int D, int GB, int LK>
hipError_t launch_gi(const DecodeParams& p, int64_t n_wg, bool wide, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(n_wg));
  if constexpr (LK == 3) {  // balanced pieces: the plan never combines them with wide workgroups
    hipLaunchKernelGGL((decode_attn_kernel<TC, QPK, D, GB, kWavesPerWG, LK>), grid, dim3(kWavesPerWG * kWave), 0,
                       stream, p);
    if (p.tickets == nullptr) launch_merge_bal<D, GB>(p, stream);
    return hipGetLastError();
  }
  if constexpr (LK != 3 && GB <= 4 && GB * D <= kWideMaxElems) {
    if (wide) {
      hipLaunchKernelGGL((decode_attn_kernel<TC, QPK, D, GB, kWideWaves, LK>), grid, dim3(kWideWaves * kWave), 0,
                         stream, p);
      if (p.num_splits > 1 && p.tickets == nullptr) launch_merge_i<D, GB, (LK != 0)>(p, stream);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((decode_attn_kernel<TC, QPK, D, GB, kWavesPerWG, LK>), grid, dim3(kWavesPerWG * kWave), 0,
                     stream, p);
  if (p.num_splits > 1 && p.tickets == nullptr) launch_merge_i<D, GB, (LK != 0)>(p, stream);
  return hipGetLastError();
}

template <typename TC, bool QPK, int D, int GB>
hipError_t launch_g(const DecodeParams& p, int64_t n_wg, bool wide, hipStream_t stream) {
  if (p.bal_rows > 0) return launch_gi<TC, QPK, D, GB, 3>(p, n_wg, wide, stream);
  if (p.pages.table != nullptr) return launch_gi<TC, QPK, D, GB, 2>(p, n_wg, wide, stream);
  return p.indirect ? launch_gi<TC, QPK, D, GB, 1>(p, n_wg, wide, stream)
                    : launch_gi<TC, QPK, D, GB, 0>(p, n_wg, wide, stream);
}

template <typename TC, bool QPK, int D>
hipError_t launch_d(const DecodeParams& p, int gb, int64_t n_wg, bool wide, hipStream_t stream) {
  switch (gb) {
    case 8: return launch_g<TC, QPK, D, 8>(p, n_wg, wide, stream);
    case 4: return launch_g<TC, QPK, D, 4>(p, n_wg, wide, stream);
    case 2: return launch_g<TC, QPK, D, 2>(p, n_wg, wide, stream);
    default: return launch_g<TC, QPK, D, 1>(p, n_wg, wide, stream);
  }
}

template <typename TC, bool QPK>
hipError_t launch_dt(const DecodeParams& p, int64_t head_dim, int gb, int64_t n_wg, bool wide, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_d<TC, QPK, 32>(p, gb, n_wg, wide, stream);
    case 64: return launch_d<TC, QPK, 64>(p, gb, n_wg, wide, stream);
    case 128: return launch_d<TC, QPK, 128>(p, gb, n_wg, wide, stream);
    default: return launch_d<TC, QPK, 256>(p, gb, n_wg, wide, stream);
  }
}

}  // namespace

// Decode launches for one cache dtype, each instantiated in its own
// translation unit (attn_decode_{bf16,f16,f32}.hip) so they compile in parallel.
hipError_t launch_decode_bf16(const DecodeParams& p, bool qpk, int64_t head_dim, int gb, int64_t n_wg, bool wide,
                              hipStream_t stream);
hipError_t launch_decode_f16(const DecodeParams& p, bool qpk, int64_t head_dim, int gb, int64_t n_wg, bool wide,
                             hipStream_t stream);
hipError_t launch_decode_f32(const DecodeParams& p, int64_t head_dim, int gb, int64_t n_wg, bool wide,
                             hipStream_t stream);

}  // namespace nckv
