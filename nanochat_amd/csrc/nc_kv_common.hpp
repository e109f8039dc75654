// Device-side helpers shared by the KV-cache kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nc_kv.h"

namespace nckv {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element types.  Each cache element type knows how many elements a 16-byte
// vector holds and how to widen a 16-byte vector to fp32.
// ---------------------------------------------------------------------------
struct bf16 { uint16_t bits; };
struct f16 { uint16_t bits; };

template <typename T> struct elem;
template <> struct elem<float> {
  static constexpr int kBytes = 4;
  static constexpr int kDtype = NC_DTYPE_F32;
};
template <> struct elem<f16> {
  static constexpr int kBytes = 2;
  static constexpr int kDtype = NC_DTYPE_F16;
};
template <> struct elem<bf16> {
  static constexpr int kBytes = 2;
  static constexpr int kDtype = NC_DTYPE_BF16;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float half_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> bf16, round to nearest even; NaN becomes the canonical quiet NaN
// 0x7FC0.  This is the rounding torch's Tensor.to(torch.bfloat16) applies.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Widen the 16-byte vector `w` holding elements of type T to fp32.
template <typename T> struct widen;
template <> struct widen<bf16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void run(const uint4& w, float* o) {
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x);
    o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
    o[4] = bf16_lo(w.z); o[5] = bf16_hi(w.z);
    o[6] = bf16_lo(w.w); o[7] = bf16_hi(w.w);
  }
};
template <> struct widen<f16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void run(const uint4& w, float* o) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = half_bits_to_f32(static_cast<uint16_t>(v[i] & 0xffffu));
      o[2 * i + 1] = half_bits_to_f32(static_cast<uint16_t>(v[i] >> 16));
    }
  }
};
template <> struct widen<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void run(const uint4& w, float* o) {
    o[0] = __uint_as_float(w.x); o[1] = __uint_as_float(w.y);
    o[2] = __uint_as_float(w.z); o[3] = __uint_as_float(w.w);
  }
};

// Scalar load of element i of a tensor whose dtype is known only at run
// time (q, k, v inputs; a handful of elements per workgroup).
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == NC_DTYPE_BF16) {
    const uint16_t b = static_cast<const uint16_t*>(p)[i];
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  if (dtype == NC_DTYPE_F16) return half_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float x) {
  if (dtype == NC_DTYPE_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(x);
  } else if (dtype == NC_DTYPE_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_rne(x);
  } else {
    static_cast<float*>(p)[i] = x;
  }
}

// Cache-element encoding of an fp32 value (the value torch's copy_ stores).
template <typename T> struct narrow;
template <> struct narrow<bf16> {
  __device__ __forceinline__ static uint16_t run(float x) { return f32_to_bf16_rne(x); }
};
template <> struct narrow<f16> {
  __device__ __forceinline__ static uint16_t run(float x) { return f32_to_f16_rne(x); }
};

// Convert VEC consecutive elements of a runtime-typed input into one 16-byte
// vector of cache type T.  When the input dtype equals T the bits are copied
// unchanged (a plain 16-byte load), which is what a same-dtype copy_ does.
template <typename T>
__device__ __forceinline__ uint4 load_as_cache_vec(const void* base, int64_t off, int in_dtype) {
  if (in_dtype == elem<T>::kDtype) {
    return *reinterpret_cast<const uint4*>(static_cast<const char*>(base) + off * elem<T>::kBytes);
  }
  if constexpr (elem<T>::kBytes == 4) {
    uint4 r;
    r.x = __float_as_uint(load_any(base, off + 0, in_dtype));
    r.y = __float_as_uint(load_any(base, off + 1, in_dtype));
    r.z = __float_as_uint(load_any(base, off + 2, in_dtype));
    r.w = __float_as_uint(load_any(base, off + 3, in_dtype));
    return r;
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = narrow<T>::run(load_any(base, off + 2 * i, in_dtype));
      const uint32_t hi = narrow<T>::run(load_any(base, off + 2 * i + 1, in_dtype));
      w[i] = lo | (hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// VEC fp32 values -> one 16-byte vector of cache type T (RNE, as copy_ rounds).
template <typename T>
__device__ __forceinline__ uint4 pack_cache_vec(const float* x) {
  if constexpr (elem<T>::kBytes == 4) {
    return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = static_cast<uint32_t>(narrow<T>::run(x[2 * i])) | (static_cast<uint32_t>(narrow<T>::run(x[2 * i + 1])) << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------------------
// Cross-lane sums inside groups of N consecutive lanes (N a power of two,
// N <= 64).  N <= 16 stays inside a DPP row: quad_perm swaps for 1 and 2,
// row_half_mirror for 4, row_mirror for 8.  Each step pairs lanes that already
// hold equal partial sums, so the result is an all-reduce over the group.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group size");
  if constexpr (N >= 2) x += dpp_move<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) x += dpp_move<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) x += dpp_move<0x141>(x);  // row_half_mirror
  if constexpr (N >= 16) x += dpp_move<0x140>(x); // row_mirror
  if constexpr (N >= 32) x += __shfl_xor(x, 16, kWave);
  if constexpr (N >= 64) x += __shfl_xor(x, 32, kWave);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// VE consecutive table entries starting at element `off` (runtime dtype),
// with 8/16/32-byte vector loads (tables are 16-byte aligned and the offsets
// are multiples of VE).
template <int VE>
__device__ __forceinline__ void load_table_vec(const void* tab, int64_t off, int dtype, float (&out)[VE]) {
  if (dtype == NC_DTYPE_F32) {
    const float4* p4 = reinterpret_cast<const float4*>(static_cast<const float*>(tab) + off);
#pragma unroll
    for (int i = 0; i < VE / 4; ++i) {
      const float4 v = p4[i];
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  } else {
    const uint16_t* p16 = static_cast<const uint16_t*>(tab) + off;
    uint32_t w[VE / 2];
    if constexpr (VE == 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(p16);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(p16);
      w[0] = v.x; w[1] = v.y;
    }
#pragma unroll
    for (int i = 0; i < VE / 2; ++i) {
      if (dtype == NC_DTYPE_BF16) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        out[2 * i] = half_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
        out[2 * i + 1] = half_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
      }
    }
  }
}

// QK prologue of one head vector (nanochat/gpt.py:98-102): rotary with this
// lane's table entries cs/sn (y1 = x1 cos + x2 sin, y2 = -x1 sin + x2 cos
// over the halves [0, D/2), [D/2, D); gpt.py:57-63), RMS norm over D with eps
// (gpt.py:42-43), times `scale`.  The vector is held VE values per lane by G
// consecutive lanes (lane c of the group: dims [VE c, VE c + VE); its table
// entries are columns [VE (c mod G/2), +VE)), so the rotary partner of a lane
// is lane c ^ G/2 and the norm is a G-lane sum.  fp32 throughout; every lane
// of the wave must take part (cross-lane exchange).
template <int G, int VE>
__device__ __forceinline__ void qk_prologue_apply(float (&x)[VE], int c, const float (&cs)[VE],
                                                  const float (&sn)[VE], float scale, float eps) {
  static_assert(G >= 2 && (G & (G - 1)) == 0, "lanes per head vector");
  constexpr int D = G * VE;
  float y[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) y[e] = __shfl_xor(x[e], G / 2, kWave);
  const bool first = c < G / 2;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < VE; ++e) {
    x[e] = first ? __builtin_fmaf(x[e], cs[e], y[e] * sn[e]) : __builtin_fmaf(x[e], cs[e], -(y[e] * sn[e]));
    ss = __builtin_fmaf(x[e], x[e], ss);
  }
  ss = group_sum<G>(ss);
  const float inv = scale / sqrtf(ss * (1.0f / D) + eps);
#pragma unroll
  for (int e = 0; e < VE; ++e) x[e] *= inv;
}

// Same, loading the table entries of table row `row` first.
template <int G, int VE>
__device__ __forceinline__ void qk_prologue_lanes(float (&x)[VE], int c, const void* cos_tab, const void* sin_tab,
                                                  int64_t row, int tab_dtype, float scale, float eps) {
  constexpr int D = G * VE;
  float cs[VE], sn[VE];
  const int64_t off = row * (D / 2) + static_cast<int64_t>(c % (G / 2)) * VE;
  load_table_vec<VE>(cos_tab, off, tab_dtype, cs);
  load_table_vec<VE>(sin_tab, off, tab_dtype, sn);
  qk_prologue_apply<G, VE>(x, c, cs, sn, scale, eps);
}

// Round to a storage dtype and back (the value a tensor of that dtype holds).
__device__ __forceinline__ float round_to(float x, int dtype) {
  if (dtype == NC_DTYPE_BF16) return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_rne(x)) << 16);
  if (dtype == NC_DTYPE_F16) return half_bits_to_f32(f32_to_f16_rne(x));
  return x;
}

// Division of integers in [0, 2^31) by a divisor fixed for the whole launch,
// as a multiply-high and a shift (Granlund & Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, sec. 4: with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1, n / d =
// (mulhi(m, n) + n) >> l; the sum cannot overflow for n < 2^31).  The
// block-index decompositions of the kernels use it instead of the 32/64-bit
// division sequences the compiler would emit for runtime divisors.
struct FastDiv {
  uint32_t d, m, l;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  f.l = 0;
  while ((uint64_t(1) << f.l) < d) ++f.l;
  f.m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << f.l) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.l;
}

// q = n / d and r = n % d.
__device__ __forceinline__ uint32_t fdivmod(uint32_t n, const FastDiv& f, uint32_t& r) {
  const uint32_t q = fdiv(n, f);
  r = n - q * f.d;
  return q;
}

// Kernel arguments in scalar registers from this point on.  The compiler
// loads each argument next to its first use, after whatever early-exit
// branches come before it, so a kernel prologue otherwise waits on one
// scalar-cache round trip per branch (4-6 before the first vector load on the
// decode kernels).  Naming the prologue's arguments here, before any branch,
// issues all their loads as one batch.
__device__ __forceinline__ void pin_arg(int32_t v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void pin_arg(uint32_t v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void pin_arg(int64_t v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void pin_arg(float v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void pin_arg(const void* v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void pin_arg(const FastDiv& f) {
  pin_arg(f.d);
  pin_arg(f.m);
  pin_arg(f.l);
}
template <typename... T>
__device__ __forceinline__ void pin_args(const T&... v) {
  (pin_arg(v), ...);
}

// Key span [lo, hi) of the chunk-kernel workgroup that owns queries
// [q0, q_end) of a row whose cache held s tokens, and its split count (>= 1;
// an empty span is one split).  The chunk kernel and the split merge both use
// it, so they agree on which partial slots exist.
struct ChunkSpan {
  int lo, hi, nsplit;
};

__device__ __forceinline__ ChunkSpan chunk_span(int s, int q0, int q_end, int t_max, int window, int kps) {
  ChunkSpan c;
  c.lo = window >= 0 ? max(0, s + q0 - window) : 0;
  c.hi = min(s + q_end, t_max);
  c.nsplit = c.hi > c.lo ? (c.hi - c.lo + kps - 1) / kps : 1;
  return c;
}

// Cache row of batch row b: cache_batch_idx[b] when given (FA3's argument),
// else b.  -1 when the index is outside [0, n_rows); `report` sets
// NC_DEVERR_BATCH_IDX (one reporting thread per row keeps the atomics few).
__device__ __forceinline__ int64_t cache_row(const int32_t* idx, int64_t n_rows, int64_t b, int32_t* err,
                                             bool report) {
  if (idx == nullptr) return b;
  const int64_t r = idx[b];
  if (r < 0 || r >= n_rows) {
    if (report && err != nullptr) atomicOr(err, NC_DEVERR_BATCH_IDX);
    return -1;
  }
  return r;
}

// Queries of batch row b.  With cu_seqlens_q (packed tokens, FA3's varlen
// layout) they are tokens [cu[b], cu[b+1]); without, row b holds t_new
// queries starting at token b * t_new.  A range that is not inside
// [0, total_q) or longer than t_new (the launch's bound, max_seqlen_q) gives
// len = -1: the row is skipped and `report` sets NC_DEVERR_QLEN.
// Paged cache (page_table): logical position j of batch row b is slot
// j & (2^shift - 1) of block table[b * stride + (j >> shift)]; the returned
// physical position indexes the cache as block * 2^shift + slot token rows
// (the block stride is 2^shift rows).  A block outside [0, n_blocks) returns
// -1 and sets NC_DEVERR_PAGE: the caller neither reads nor stores that key.
struct PageMap {
  const int32_t* table;   // NULL: the cache is not paged
  int64_t stride;
  int32_t shift;
  int64_t n_blocks;
};
__device__ __forceinline__ int64_t page_pos(const PageMap& pm, int64_t b, int j, int32_t* err) {
  const int32_t blk = pm.table[b * pm.stride + (j >> pm.shift)];
  if (blk < 0 || blk >= pm.n_blocks) {
    if (err != nullptr) atomicOr(err, NC_DEVERR_PAGE);
    return -1;
  }
  return (static_cast<int64_t>(blk) << pm.shift) | (j & ((1 << pm.shift) - 1));
}

struct RowQ {
  int64_t tok0;  // token index of the row's first query (row of `out`)
  int len;       // queries of the row
};
__device__ __forceinline__ RowQ row_queries(const int32_t* cu, int64_t total_q, int64_t b, int t_new, int32_t* err,
                                            bool report) {
  if (cu == nullptr) return RowQ{b * t_new, t_new};
  const int a = cu[b], e = cu[b + 1];
  if (a < 0 || e < a || e - a > t_new || e > total_q) {
    if (report && err != nullptr) atomicOr(err, NC_DEVERR_QLEN);
    return RowQ{a, -1};
  }
  return RowQ{a, e - a};
}

// Element offset of query/new token t of row b in q, k or v (batch stride sb
// and token stride st; packed tokens ignore sb).
__device__ __forceinline__ int64_t token_offset(const int32_t* cu, const RowQ& rq, int64_t b, int t, int64_t sb,
                                                int64_t st) {
  return cu != nullptr ? (rq.tok0 + t) * st : b * sb + t * st;
}

}  // namespace nckv
