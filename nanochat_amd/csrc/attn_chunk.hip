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
// Tiling.  A workgroup owns 64 "rows" = (query, q head) pairs of one
// (row b, kv head, q-head block): 64 / GB queries x GB heads, so the GB heads
// that share a kv head read each K/V tile once.  4 waves x 16 rows.  Key tiles
// of 64 positions are staged in LDS as [key][dim] rows (16-byte stores), padded
// so the MFMA operand reads are bank-conflict free.
//
// Per tile and wave (v_mfma_f32_16x16x32_{bf16,f16}; lane l, q = l / 16):
//   S^T = K . Q^T   A = K[16 keys][32 dims] (LDS), B = Q^T (registers);
//                   lane l holds S[row l%16][keys 16kb + 4q + r], r < 4.
//   softmax         each lane owns one query row: running max / sum in fp32,
//                   cross-lane reductions over the 4 lane groups only.
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
// count; workgroups past it return at once).  The next key tile is
// loaded into registers while the current one is consumed from LDS.

#include <algorithm>
#include <cstdlib>

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

constexpr int kChunkWaves = 4;
constexpr int kRows = 64;        // (query, head) rows per workgroup
constexpr int kBN = 64;          // keys per tile
constexpr int kChunkStagePages = 512;  // page numbers a workgroup stages in LDS (paged cache)
constexpr float kNegBigC = -1.0e30f;
constexpr int kXcdsC = 8;

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) char lds_char;

// ds_read_b64_tr_b16 from a generic pointer into a __shared__ array.
__device__ __forceinline__ i16x4 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((lds_char*)(p)));
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
template <typename TC, int D, int GB, int LK>
__global__ __launch_bounds__(kChunkWaves * kWave) void chunk_attn_kernel(const ChunkParams p) {
  typedef typename mfma_t<TC>::v8 v8;
  constexpr int QB = kRows / GB;          // queries per workgroup
  constexpr int DC = D / 32;              // 32-dim chunks (MFMA K for S)
  constexpr int DB = D / 16;              // 16-dim output blocks
  constexpr int KROW = D * 2 + 16;        // bytes per K row in LDS (padded: 16-byte reads, 8 lanes/cycle)
  constexpr int VROW = D * 2 + 32;        // bytes per V row in LDS (padded: transpose reads, 16 lanes/cycle)
  constexpr int CHUNKS = kBN * D / 8;     // 16-byte chunks per tile (K or V)
  constexpr int PER_THREAD = CHUNKS / (kChunkWaves * kWave);
  static_assert(PER_THREAD * kChunkWaves * kWave == CHUNKS, "tile / workgroup shape");

  __shared__ __attribute__((aligned(16))) char ks[kBN * KROW];
  __shared__ __attribute__((aligned(16))) char vs[kBN * VROW];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // the wave index, provably wave-uniform (so tile bounds and masks derived
  // from it compile to scalar branches, not per-lane exec masking)
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lq = lane / 16;               // lane group 0..3
  const int lr = lane % 16;

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
  const int row = wave * 16 + lr;
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

  // ---- key tiles: registers hold the next tile while the current one is
  // consumed from LDS (a second register stage measured no faster) ----
  // Thread chunk u of a tile is key key0 + u * KSTEP, 16-byte column dc0 (the
  // plan keeps a tile's byte span below 2^31, so offsets are 32-bit).
  constexpr int CPR = D / 8;                          // 16-byte chunks per key row
  constexpr int KSTEP = kChunkWaves * kWave / CPR;    // keys between a thread's chunks
  const int key0 = tid / CPR, dc0 = tid % CPR;
  uint32_t koff[PER_THREAD], voff[PER_THREAD];
#pragma unroll
  for (int u = 0; u < PER_THREAD; ++u) {
    koff[u] = static_cast<uint32_t>((key0 + u * KSTEP) * kst + dc0 * 16);
    voff[u] = static_cast<uint32_t>((key0 + u * KSTEP) * vst + dc0 * 16);
  }
  // paged cache: the page numbers of this workgroup's keys [lo, hi), read from
  // the table once into LDS (entries outside the pool become -1 and set
  // NC_DEVERR_PAGE), so a tile's K/V loads wait on LDS rather than on a table
  // load of their own.  Spans of more pages fall back to per-key lookups, and
  // so do workgroups that read no cached key (a prefill from position 0: only
  // their stores look pages up, and a staging prologue would only add latency).
  [[maybe_unused]] int page_lo = 0;
  [[maybe_unused]] bool pages_staged = false;
  [[maybe_unused]] const int32_t* sm_pg = nullptr;
  if constexpr (LK == 2) {
    __shared__ int32_t sm_pages[kChunkStagePages];
    page_lo = lo >> p.pages.shift;
    const int npages = hi > lo ? ((hi - 1) >> p.pages.shift) - page_lo + 1 : 0;
    pages_staged = npages <= kChunkStagePages && min(hi, new_lo) > lo;
    if (pages_staged) {
      for (int i = tid; i < npages; i += kChunkWaves * kWave) {
        const int32_t blk = p.pages.table[b * p.pages.stride + page_lo + i];
        const bool ok = blk >= 0 && blk < p.pages.n_blocks;
        if (!ok && p.err != nullptr) atomicOr(p.err, NC_DEVERR_PAGE);
        sm_pages[i] = ok ? blk : -1;
      }
      __syncthreads();
    }
    sm_pg = sm_pages;
  }
  // physical cache position of logical key j in [lo, hi): j, or its page-table
  // slot (-1: not addressable)
  auto cache_pos = [&](int j) -> int64_t {
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
  uint4 kreg[PER_THREAD], vreg[PER_THREAD];
  auto load_regs = [&](int kt0, uint4 (&kr)[PER_THREAD], uint4 (&vr)[PER_THREAD]) {
    if (contiguous && kt0 + kBN <= hi && kt0 + kBN <= new_lo) {
      // whole tile inside the span and in the cache: no per-chunk checks
      const char* kt = kbase + kt0 * kst;
      const char* vt = vbase + kt0 * vst;
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        kr[u] = *reinterpret_cast<const uint4*>(kt + koff[u]);
        vr[u] = *reinterpret_cast<const uint4*>(vt + voff[u]);
      }
      return;
    }
    if (!contiguous) {  // paged cache: each cached key's slot from the page table
      if (pages_staged && kt0 + kBN <= hi && kt0 + kBN <= new_lo) {
        // whole tile in the cache: branch-free loads (a key of a page outside
        // the pool reads block 0, which exists, and is then zeroed)
        const int pmask = (1 << p.pages.shift) - 1;
#pragma unroll
        for (int u = 0; u < PER_THREAD; ++u) {
          const int j = kt0 + key0 + u * KSTEP;
          const int32_t blk = sm_pg[(j >> p.pages.shift) - page_lo];
          const int64_t pj = (static_cast<int64_t>(max(blk, 0)) << p.pages.shift) | (j & pmask);
          const uint4 kx = *reinterpret_cast<const uint4*>(kbase + pj * kst + dc0 * 16);
          const uint4 vx = *reinterpret_cast<const uint4*>(vbase + pj * vst + dc0 * 16);
          kr[u] = blk >= 0 ? kx : make_uint4(0, 0, 0, 0);
          vr[u] = blk >= 0 ? vx : make_uint4(0, 0, 0, 0);
        }
        return;
      }
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        const int j = kt0 + key0 + u * KSTEP;
        const bool from_new = j >= new_lo;
        const int64_t pj = (j < hi && !from_new) ? cache_pos(j) : 0;
        if (j < hi && pj >= 0) {
          const char* kp = from_new ? knew + (j - s) * knst : kbase + pj * kst;
          const char* vp = from_new ? vnew + (j - s) * vnst : vbase + pj * vst;
          kr[u] = *reinterpret_cast<const uint4*>(kp + dc0 * 16);
          vr[u] = *reinterpret_cast<const uint4*>(vp + dc0 * 16);
        } else {
          kr[u] = make_uint4(0, 0, 0, 0);
          vr[u] = make_uint4(0, 0, 0, 0);
        }
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < PER_THREAD; ++u) {
      const int j = kt0 + key0 + u * KSTEP;
      if (j < hi) {
        const bool from_new = j >= new_lo;
        const char* kp = from_new ? knew + (j - s) * knst : kbase + j * kst;
        const char* vp = from_new ? vnew + (j - s) * vnst : vbase + j * vst;
        kr[u] = *reinterpret_cast<const uint4*>(kp + dc0 * 16);
        vr[u] = *reinterpret_cast<const uint4*>(vp + dc0 * 16);
      } else {
        kr[u] = make_uint4(0, 0, 0, 0);
        vr[u] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  // wave-uniform bounds of this wave's query rows: tiles wholly inside every
  // row's mask skip the per-element mask
  const int qi_first = q0 + (wave * 16) / GB, qi_last = q0 + (wave * 16 + 15) / GB;
  const bool wave_rows_full = qi_last < rq.len;
  const int qpos_first = s + qi_first, qpos_last = s + qi_last;
  auto tile_step = [&](int kt0, uint4 (&kr)[PER_THREAD], uint4 (&vr)[PER_THREAD]) {
    __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
    for (int u = 0; u < PER_THREAD; ++u) {
      const int key = key0 + u * KSTEP;
      *reinterpret_cast<uint4*>(ks + key * KROW + dc0 * 16) = kr[u];
      *reinterpret_cast<uint4*>(vs + key * VROW + dc0 * 16) = vr[u];
    }
    if (kt0 + kBN > own_lo) {  // the tile holds new tokens this workgroup stores
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        const int j = kt0 + key0 + u * KSTEP;
        const bool own = j >= own_lo && j < hi;
        const int64_t pj = own ? (contiguous ? j : cache_pos(j)) : -1;
        if (pj >= 0) {
          *reinterpret_cast<uint4*>(const_cast<char*>(kbase) + pj * kst + dc0 * 16) = kr[u];
          *reinterpret_cast<uint4*>(const_cast<char*>(vbase) + pj * vst + dc0 * 16) = vr[u];
        }
      }
    }
    __syncthreads();
    if (kt0 + kBN < hi) load_regs(kt0 + kBN, kr, vr);

    // ---- S^T = K . Q^T for the 4 key blocks of the tile ----
    f4v acc_s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      acc_s[kb] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const uint4 a = *reinterpret_cast<const uint4*>(ks + (16 * kb + lr) * KROW + (32 * c + 8 * lq) * 2);
        mfma_t<TC>::run(__builtin_bit_cast(v8, a), qf[c], acc_s[kb]);
      }
    }

    // ---- mask, scale, online softmax (each lane: one query row) ----
    const bool interior = wave_rows_full && kt0 + kBN <= hi && kt0 + kBN - 1 <= qpos_first &&
                          (p.window < 0 || kt0 >= qpos_last - p.window);
    float sv[4][4];
    float mt = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float a4[4] = {acc_s[kb][0], acc_s[kb][1], acc_s[kb][2], acc_s[kb][3]};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[kb][r] = a4[r] * p.scale_log2;
        if (!interior) {
          const int j = kt0 + 16 * kb + 4 * lq + r;
          const bool ok = row_ok && j >= row_lo && j <= qpos && j < hi;
          sv[kb][r] = ok ? sv[kb][r] : -__builtin_inff();
        }
        mt = fmaxf(mt, sv[kb][r]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = fast_exp2(m_run - m_new);
    float rs = 0.0f;
    uint32_t pk[4][2];  // P packed in the cache dtype: [key block][pair of r]
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      float pv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[r] = fast_exp2(sv[kb][r] - m_new);
        rs += pv[r];
      }
      pk[kb][0] = mfma_t<TC>::pack2(pv[0], pv[1]);
      pk[kb][1] = mfma_t<TC>::pack2(pv[2], pv[3]);
    }
    rs += __shfl_xor(rs, 16, kWave);
    rs += __shfl_xor(rs, 32, kWave);
    l_run = l_run * alpha + rs;
    // rescale the output only when some row's running max moved
    if (__any(m_new != m_run)) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc_o[db] *= alpha;
      }
    }
    m_run = m_new;

    // ---- O^T += V^T . P^T over the two 32-key chunks ----
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const v8 bp = __builtin_bit_cast(v8, make_uint4(pk[2 * kc][0], pk[2 * kc][1], pk[2 * kc + 1][0], pk[2 * kc + 1][1]));
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        // lane lr of group lq points at key (base + lr/4), dims 16db + 4*(lr%4) .. +3
        const char* src0 = vs + (32 * kc + 4 * lq + lr / 4) * VROW + (16 * db + 4 * (lr % 4)) * 2;
        const char* src1 = src0 + 16 * VROW;
        const i16x4 lo4 = lds_read_tr16(src0);
        const i16x4 hi4 = lds_read_tr16(src1);
        const v8 av = __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        mfma_t<TC>::run(av, bp, acc_o[db]);
      }
    }
  };
  load_regs(lo, kreg, vreg);
  for (int kt0 = lo; kt0 < hi; kt0 += kBN) tile_step(kt0, kreg, vreg);

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

template <typename TC, int D, int LK>
hipError_t launch_ci(const ChunkParams& p, int gb, hipStream_t stream) {
  const int64_t n_wg = static_cast<int64_t>(kXcdsC) * p.n_qtiles * p.num_splits * ((p.n_groups + kXcdsC - 1) / kXcdsC);
  const dim3 grid(static_cast<unsigned>(n_wg)), block(kChunkWaves * kWave);
  switch (gb) {
    case 8: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 8, LK>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 4, LK>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 2, LK>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((chunk_attn_kernel<TC, D, 1, LK>), grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

template <typename TC, int D>
hipError_t launch_c(const ChunkParams& p, int gb, hipStream_t stream) {
  if (p.pages.table != nullptr) return launch_ci<TC, D, 2>(p, gb, stream);
  return p.indirect ? launch_ci<TC, D, 1>(p, gb, stream) : launch_ci<TC, D, 0>(p, gb, stream);
}

}  // namespace

bool chunk_supports(const nc_attn_args& a) {
  // a key tile's byte span (64 cache rows) must fit the kernel's 32-bit offsets
  const int64_t tile_bytes = kBN * std::max(std::abs(a.kc_stride_t), std::abs(a.vc_stride_t)) * 2;
  return a.t_new > 1 && a.q_dtype == a.cache_dtype &&
         (a.cache_dtype == NC_DTYPE_BF16 || a.cache_dtype == NC_DTYPE_F16) &&
         (a.head_dim == 64 || a.head_dim == 128) && tile_bytes < (int64_t(1) << 31);
}

int chunk_rows_per_wg() { return kRows; }

hipError_t launch_chunk(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s, hipStream_t stream,
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
  const int qb = kRows / plan.head_block;
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
  if (a.cache_dtype == NC_DTYPE_BF16) {
    return a.head_dim == 64 ? launch_c<bf16, 64>(p, plan.head_block, stream)
                            : launch_c<bf16, 128>(p, plan.head_block, stream);
  }
  return a.head_dim == 64 ? launch_c<f16, 64>(p, plan.head_block, stream)
                          : launch_c<f16, 128>(p, plan.head_block, stream);
}

}  // namespace nckv
