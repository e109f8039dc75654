// Small-M linear layer y = x W^T for decode steps (M = batch rows <= 64), and
// the GPT logits head fused into it.
//
// nanochat's decode step runs every projection as F.linear on a (B, 1, C)
// activation: M = B rows against an (N, K) weight, a weight-streaming problem
// (every weight byte is used by all M rows once).  The last one, lm_head, is
// followed by a vocabulary slice, a cast to fp32 and a tanh softcap, each a
// separate pass over the (B, vocab) logits.  Here they are one kernel.
//
// A workgroup (4 waves) owns a 64-column block of W (16 columns per wave)
// over a range of K.  Per 128-wide chunk of K each wave runs four MFMAs
// v_mfma_f32_16x16x32 (A = its W tile straight from HBM into registers,
// B = the x^T tile, one per 32-wide k-block).  The x chunk is loaded once
// per workgroup into a 2-deep LDS ring and read by all 4 waves; W and x of
// the next chunks are loaded kLinPD chunks ahead.  Loads are buffer loads with
// 32-bit offsets.  When K is split over workgroups (few column blocks), each
// publishes its fp32 partial with coherent stores and takes a ticket; the
// workgroup that draws the last ticket sums the partials in split order (the
// result does not depend on the order in which workgroups run) and writes y.
//
// Measured on MI355X (HIP graph replays, bf16): the vocabulary-sized shapes
// stream W at 5.5-5.9 TB/s (32 x 32768 x 1280: 15.3 us, the library GEMM
// 15.1; at M = 16 and M = 1 this kernel is 11-16% faster), and the fused
// head takes 16.2 us against 26.0 us for the library GEMM plus torch's slice,
// cast and softcap.  The block projections (3-13 MB of W) are latency-bound:
// there split K across workgroups costs two more memory round trips, so for
// m <= 32 the narrow kernel below splits K over the waves of one workgroup
// instead (32 x 3840 x 1280: 10.3 -> 6.5 us; 16 rows: 4.7-8.4 us, 15-40%
// below the library GEMM at K <= 2048; at 32 rows, and at K >= 5120, the
// library is level or faster, as each workgroup then reads all of x from L2).
//
// Epilogue: fp32 accumulator -> output dtype (round to nearest even), or,
// with softcap > 0, the logits head: the accumulator is rounded to the input
// dtype (the reference's bf16 lm_head output), widened, and written as fp32
// softcap * tanh(v * (1/softcap)) -- the operations torch performs for
// softcap * torch.tanh(logits / softcap) on a float tensor and a scalar.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

constexpr int kLinWaves = 4;      // one 16-column tile each: 64 columns per workgroup
constexpr int kLinChunk = 128;   // K elements per step (four 32-wide MFMA k-blocks)
static_assert(kLinWaves * kWave == 16 * 16, "x staging: 16 rows x 16 segments of 16 bytes per m-tile");

typedef float lin_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int lin_u4 __attribute__((ext_vector_type(4)));

template <typename TC> struct lin_mfma;
template <> struct lin_mfma<bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static void run(const lin_u4& a, const lin_u4& b, lin_f4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static float round_trip(float x) { return __uint_as_float(uint32_t(f32_to_bf16_rne(x)) << 16); }
};
template <> struct lin_mfma<f16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static void run(const lin_u4& a, const lin_u4& b, lin_f4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static float round_trip(float x) { return static_cast<float>(static_cast<_Float16>(x)); }
};

struct LinearParams {
  const uint16_t* x;
  const uint16_t* w;
  void* y;
  int64_t x_st, w_st, y_st;   // row strides, elements
  int m, n, k;
  int chunks;                 // ceil(k / kLinChunk)
  int chunks_per_split;
  int splits;
  int out_dtype;
  float softcap;              // > 0: fp32 logits head epilogue
  float inv_softcap;
  float* part;                // [block][split][wave][MT][64 lanes][4] fp32, splits > 1
  uint32_t* tickets;          // [block], zero between calls
};

__device__ __forceinline__ void lin_coherent_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float lin_coherent_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Buffer resource over [base, base + bytes): loads take 32-bit byte offsets.
// Every offset used below is inside the range (masked lanes read element 0
// and their values are replaced by zero), so the hardware range check is
// never relied on.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lin_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}
#ifndef NC_LIN_NT
#define NC_LIN_NT 0
#endif
// Cache policy of the W loads.  Plain loads: a W load instruction reads 64 of
// the 128 bytes of a line per row and the next one reads the other half, so the
// line must stay in L2 between them (the non-temporal hint cost 35% on the
// logits head: 23.5 vs 15.1 us at 32 x 32768 x 1280).
constexpr int kLinNT = NC_LIN_NT;

// Output of lane (lr, lq) for m-tile mt: y[mt*16 + lr][n0 + 4 lq + r], r = 0..3.
template <typename TC>
__device__ __forceinline__ void lin_store(const LinearParams& p, int row, int col0, const lin_f4& v) {
  if (row >= p.m) return;
  const int64_t base = static_cast<int64_t>(row) * p.y_st + col0;
  if (p.softcap > 0.0f) {
    float* y = static_cast<float*>(p.y) + base;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (col0 + r < p.n) y[r] = tanhf(lin_mfma<TC>::round_trip(v[r]) * p.inv_softcap) * p.softcap;
    }
    return;
  }
  if (p.out_dtype == NC_DTYPE_F32) {
    float* y = static_cast<float*>(p.y) + base;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (col0 + r < p.n) y[r] = v[r];
    }
    return;
  }
  uint16_t h[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    h[r] = p.out_dtype == NC_DTYPE_BF16 ? f32_to_bf16_rne(v[r]) : f32_to_f16_rne(v[r]);
  }
  uint16_t* y = static_cast<uint16_t*>(p.y) + base;
  if (col0 + 4 <= p.n && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
    *reinterpret_cast<uint2*>(y) = make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (col0 + r < p.n) y[r] = h[r];
    }
  }
}

// W operand of chunk c for lane (lr, lq): sub-load j holds W[row][c*128 + 32 j + 8 lq, +8), the
// MFMA A layout of k-block j (16 rows x 64 contiguous bytes per load instruction).
__device__ __forceinline__ void lin_load_w(__amdgpu_buffer_rsrc_t rw, uint32_t row_off, int k, int lq, int c,
                                           lin_u4 (&w)[4]) {
  const int k0 = c * kLinChunk + 8 * lq;
  if ((c + 1) * kLinChunk <= k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, row_off + 2u * (k0 + 32 * j), 0, kLinNT);
    }
  } else {
    const lin_u4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = k0 + 32 * j < k;
      const lin_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, in ? row_off + 2u * (k0 + 32 * j) : 0u, 0, kLinNT);
      w[j] = in ? v : zero;
    }
  }
}

// x rows of chunk c staged by thread t: row mt*16 + t/16, elements c*128 + 8 (t % 16), +8.
template <int MT>
__device__ __forceinline__ void lin_load_x(const LinearParams& p, __amdgpu_buffer_rsrc_t rx, int tid, int c,
                                           lin_u4 (&xr)[MT]) {
  const int kk = c * kLinChunk + 8 * (tid % 16);
  const bool k_ok = kk < p.k;
  const lin_u4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = min(mt * 16 + tid / 16, p.m - 1);   // rows past m feed only unstored outputs
    const uint32_t off = k_ok ? 2u * static_cast<uint32_t>(row * p.x_st + kk) : 0u;
    const lin_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    xr[mt] = k_ok ? v : zero;
  }
}

constexpr int kLinMergeBatch = 4;                // split partials loaded together by the merging workgroup
constexpr int kLinXPitch = kLinChunk * 2 + 16;   // bytes per staged x row (padded: conflict-free 16-byte reads)
#ifndef NC_LIN_PD
#define NC_LIN_PD 2
#endif
constexpr int kLinPD = NC_LIN_PD;                // chunks of W and x loaded ahead per wave (2 measured best of 2-6)

template <typename TC, int MT>
__global__ __launch_bounds__(kLinWaves * kWave) void linear_small_m_kernel(const LinearParams p) {
  __shared__ __attribute__((aligned(16))) char xs[2][MT * 16 * kLinXPitch];
  __shared__ int sm_last;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lq = lane / 16;
  const int lr = lane % 16;

  // ---- block -> (64-column block, K split); wave -> its 16 columns ----
  const int blk = blockIdx.x / p.splits;
  const int split = blockIdx.x - blk * p.splits;
  const int nb0 = blk * kLinCols;
  const int rows_in_blk = min(kLinCols, p.n - nb0);
  const int n0 = nb0 + 16 * wave;
  // rows past n read the block's last row: they feed only outputs that are not stored
  const int wrow = min(16 * wave + lr, rows_in_blk - 1);
  const __amdgpu_buffer_rsrc_t rw = lin_rsrc(
      p.w + static_cast<int64_t>(nb0) * p.w_st,
      static_cast<uint32_t>(2 * (static_cast<int64_t>(rows_in_blk - 1) * p.w_st + p.k)));
  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(
      p.x, static_cast<uint32_t>(2 * (static_cast<int64_t>(p.m - 1) * p.x_st + p.k)));
  const uint32_t w_row_off = 2u * static_cast<uint32_t>(wrow * p.w_st);

  lin_f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = lin_f4{0.0f, 0.0f, 0.0f, 0.0f};

  const int c_begin = split * p.chunks_per_split;
  const int c_end = min(p.chunks, c_begin + p.chunks_per_split);

  // ---- prologue: W and x of the first kLinPD chunks in flight, x of the first chunk into LDS ----
  // x(c) is loaded right after W(c), kLinPD chunks ahead of its use, so the wait for x(c + 1)
  // (before it is staged) only drains loads up to W(c + 1): kLinPD - 1 chunks stay in flight.
  lin_u4 wr[kLinPD][4];
  lin_u4 xr[kLinPD][MT];
#pragma unroll
  for (int s = 0; s < kLinPD; ++s) {
    if (c_begin + s < c_end) {
      lin_load_w(rw, w_row_off, p.k, lq, c_begin + s, wr[s]);
      lin_load_x<MT>(p, rx, tid, c_begin + s, xr[s]);
    }
  }
  const int xs_off = (tid / 16) * kLinXPitch + (tid % 16) * 16;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<lin_u4*>(xs[0] + mt * 16 * kLinXPitch + xs_off) = xr[0][mt];

  // ---- chunk loop: x through a 2-deep LDS ring (one barrier per chunk) ----
  const int rd_off = lr * kLinXPitch + lq * 16;
  for (int c0 = c_begin; c0 < c_end; c0 += kLinPD) {
#pragma unroll
    for (int s = 0; s < kLinPD; ++s) {
      const int c = c0 + s;
      if (c < c_end) {
        __syncthreads();   // x(c) is in xs[(c - c_begin) & 1]; the other buffer's readers are done
        const char* xb = xs[(c - c_begin) & 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const lin_u4 xf = *reinterpret_cast<const lin_u4*>(xb + mt * 16 * kLinXPitch + rd_off + 64 * j);
            lin_mfma<TC>::run(wr[s][j], xf, acc[mt]);
          }
        }
        if (c + 1 < c_end) {
          const int sn = (s + 1) % kLinPD;   // a constant once the loop over s is unrolled
          char* xn = xs[(c + 1 - c_begin) & 1];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<lin_u4*>(xn + mt * 16 * kLinXPitch + xs_off) = xr[sn][mt];
        }
        if (c + kLinPD < c_end) {
          lin_load_w(rw, w_row_off, p.k, lq, c + kLinPD, wr[s]);
          lin_load_x<MT>(p, rx, tid, c + kLinPD, xr[s]);
        }
      }
    }
  }

  const int col0 = n0 + 4 * lq;
  if (p.splits == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) lin_store<TC>(p, mt * 16 + lr, col0, acc[mt]);
    return;
  }

  // ---- split K: publish the partial, take a ticket, the last split sums in split order ----
  const int64_t slot_stride = static_cast<int64_t>(kLinWaves) * MT * kWave * 4;
  float* slot = p.part + (static_cast<int64_t>(blk) * p.splits + split) * slot_stride + (wave * MT * kWave + lane) * 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) lin_coherent_store(slot + mt * kWave * 4 + r, acc[mt][r]);
  }
  // the partial stores have completed before the barrier, hence before the ticket
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t tk = __hip_atomic_fetch_add(p.tickets + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = tk + 1 == static_cast<uint32_t>(p.splits);
    if (last) __hip_atomic_store(p.tickets + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_last = last;
  }
  __syncthreads();
  if (!sm_last) return;
  __asm__ volatile("" ::: "memory");
  const float* src = p.part + static_cast<int64_t>(blk) * p.splits * slot_stride + (wave * MT * kWave + lane) * 4;
  // splits summed in order; each batch's loads are issued together (one memory round trip per batch)
  lin_f4 sum[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sum[mt] = lin_f4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int sp0 = 0; sp0 < p.splits; sp0 += kLinMergeBatch) {
    float v[kLinMergeBatch][MT][4];
#pragma unroll
    for (int u = 0; u < kLinMergeBatch; ++u) {
      const bool in = sp0 + u < p.splits;
      const float* q = src + (in ? sp0 + u : 0) * slot_stride;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[u][mt][r] = in ? lin_coherent_load(q + mt * kWave * 4 + r) : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < kLinMergeBatch; ++u) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[mt][r] += v[u][mt][r];
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) lin_store<TC>(p, mt * 16 + lr, col0, sum[mt]);
}

// x^T operand of chunk c for lane (lr, lq) and m-tile mt: x[mt*16 + lr][c*128 + 32 j + 8 lq, +8)
// (K % 8 == 0, so an 8-element group is wholly inside or outside K).
template <int MT>
__device__ __forceinline__ void lin_load_xb(__amdgpu_buffer_rsrc_t rx, const uint32_t (&x_off)[MT], int k, int lq,
                                            int c, lin_u4 (&xb)[MT][4]) {
  const int k0 = c * kLinChunk + 8 * lq;
  const lin_u4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = k0 + 32 * j < k;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const lin_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, in ? x_off[mt] + 2u * (k0 + 32 * j) : 0u, 0, 0);
      xb[mt][j] = in ? v : zero;
    }
  }
}

// Narrow plan (M <= 32 and few 64-column blocks: the decode step's own
// projections, 3-13 MB of W).  A workgroup owns 16 columns and its KW waves
// split K among themselves (chunk c goes to wave c % KW), each streaming W
// and x straight into registers kLinNarrowPD chunks ahead.  The waves' fp32
// partials meet in LDS and wave 0 adds them in wave order, so the result does
// not depend on timing, and nothing crosses workgroups: one pass, no
// workspace, no ticket.  (x is read once per workgroup from L2; at these
// sizes that costs less than the split plan's two extra memory round trips.)
constexpr int kLinNarrowPD = 2;
template <typename TC, int MT, int KW, int NT>
__global__ __launch_bounds__(KW * kWave) void linear_narrow_kernel(const LinearParams p) {
  __shared__ lin_f4 red[KW - 1][NT][MT][kWave];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lq = lane / 16;
  const int lr = lane % 16;

  // the workgroup's 16 * NT columns; each wave runs all NT column tiles on its chunks, so one x
  // load feeds NT MFMAs.  With splits > 1 (long K, few column blocks) the workgroup takes chunks
  // [split * chunks_per_split, +chunks_per_split) of its column block.
  const int blk = static_cast<int>(blockIdx.x) / p.splits;
  const int split = static_cast<int>(blockIdx.x) - blk * p.splits;
  const int c_begin = split * p.chunks_per_split;
  const int c_end = min(p.chunks, c_begin + p.chunks_per_split);
  const int n0 = blk * 16 * NT;
  const int rows_in_blk = min(16 * NT, p.n - n0);
  // rows past n read the block's last row, rows past m the last x row: they feed only unstored outputs
  const __amdgpu_buffer_rsrc_t rw = lin_rsrc(
      p.w + static_cast<int64_t>(n0) * p.w_st,
      static_cast<uint32_t>(2 * (static_cast<int64_t>(rows_in_blk - 1) * p.w_st + p.k)));
  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(
      p.x, static_cast<uint32_t>(2 * (static_cast<int64_t>(p.m - 1) * p.x_st + p.k)));
  uint32_t w_row_off[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) w_row_off[nt] = 2u * static_cast<uint32_t>(min(16 * nt + lr, rows_in_blk - 1) * p.w_st);
  uint32_t x_off[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) x_off[mt] = 2u * static_cast<uint32_t>(min(mt * 16 + lr, p.m - 1) * p.x_st);

  lin_f4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = lin_f4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  lin_u4 wr[kLinNarrowPD][NT][4];
  lin_u4 xr[kLinNarrowPD][MT][4];
#pragma unroll
  for (int s = 0; s < kLinNarrowPD; ++s) {
    const int c = c_begin + wave + s * KW;
    if (c < c_end) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) lin_load_w(rw, w_row_off[nt], p.k, lq, c, wr[s][nt]);
      lin_load_xb<MT>(rx, x_off, p.k, lq, c, xr[s]);
    }
  }
  for (int c0 = c_begin + wave; c0 < c_end; c0 += kLinNarrowPD * KW) {
#pragma unroll
    for (int s = 0; s < kLinNarrowPD; ++s) {
      const int c = c0 + s * KW;
      if (c < c_end) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) lin_mfma<TC>::run(wr[s][nt][j], xr[s][mt][j], acc[nt][mt]);
          }
        }
        const int cn = c + kLinNarrowPD * KW;
        if (cn < c_end) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) lin_load_w(rw, w_row_off[nt], p.k, lq, cn, wr[s][nt]);
          lin_load_xb<MT>(rx, x_off, p.k, lq, cn, xr[s]);
        }
      }
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[wave - 1][nt][mt][lane] = acc[nt][mt];
    }
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < KW - 1; ++w) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] += red[w][nt][mt][lane];
    }
  }
  if (p.splits > 1) {
    // split K across workgroups as well: wave 0 publishes the workgroup's partial with coherent
    // stores, waits for them, and takes a ticket; the last split sums the partials in split order
    constexpr int64_t slot = static_cast<int64_t>(NT) * MT * kWave * 4;
    float* mine = p.part + (static_cast<int64_t>(blk) * p.splits + split) * slot + lane * 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) lin_coherent_store(mine + (nt * MT + mt) * kWave * 4 + r, acc[nt][mt][r]);
      }
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the wave's partial stores have completed
    uint32_t tk = 0;
    if (lane == 0) tk = __hip_atomic_fetch_add(p.tickets + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tk = __shfl(tk, 0);
    if (tk + 1 != static_cast<uint32_t>(p.splits)) return;
    if (lane == 0) __hip_atomic_store(p.tickets + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __asm__ volatile("" ::: "memory");
    const float* src_part = p.part + static_cast<int64_t>(blk) * p.splits * slot + lane * 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = lin_f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int sp = 0; sp < p.splits; ++sp) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[nt][mt][r] += lin_coherent_load(src_part + sp * slot + (nt * MT + mt) * kWave * 4 + r);
        }
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int col0 = n0 + 16 * nt + 4 * lq;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) lin_store<TC>(p, mt * 16 + lr, col0, acc[nt][mt]);
  }
}

template <typename TC, int MT, int KW, int NT>
hipError_t launch_narrow_t(const LinearParams& p, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL((linear_narrow_kernel<TC, MT, KW, NT>), dim3(static_cast<unsigned>(blocks * p.splits)),
                     dim3(KW * kWave), 0, stream, p);
  return hipGetLastError();
}

// tiles = 1: one 16-column tile per wave, 4-16 waves; tiles = 2 (16 < m <= 32, wide n): two tiles per
// wave sharing each x load, 4-8 waves (VGPRs)
template <typename TC>
hipError_t launch_narrow(const LinearParams& p, int64_t blocks, int kw, int tiles, hipStream_t stream) {
  if (p.m > 16) {
    if (tiles == 2) {
      return kw >= 8 ? launch_narrow_t<TC, 2, 8, 2>(p, blocks, stream) : launch_narrow_t<TC, 2, 4, 2>(p, blocks, stream);
    }
    switch (kw) {
      case 16: return launch_narrow_t<TC, 2, 16, 1>(p, blocks, stream);
      case 8: return launch_narrow_t<TC, 2, 8, 1>(p, blocks, stream);
      default: return launch_narrow_t<TC, 2, 4, 1>(p, blocks, stream);
    }
  }
  switch (kw) {
    case 16: return launch_narrow_t<TC, 1, 16, 1>(p, blocks, stream);
    case 8: return launch_narrow_t<TC, 1, 8, 1>(p, blocks, stream);
    default: return launch_narrow_t<TC, 1, 4, 1>(p, blocks, stream);
  }
}

template <typename TC, int MT>
hipError_t launch_lin_t(const LinearParams& p, int64_t blocks, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(blocks * p.splits));
  hipLaunchKernelGGL((linear_small_m_kernel<TC, MT>), grid, dim3(kLinWaves * kWave), 0, stream, p);
  return hipGetLastError();
}

template <typename TC>
hipError_t launch_lin_m(const LinearParams& p, int64_t blocks, hipStream_t stream) {
  switch ((p.m + 15) / 16) {
    case 1: return launch_lin_t<TC, 1>(p, blocks, stream);
    case 2: return launch_lin_t<TC, 2>(p, blocks, stream);
    case 3: return launch_lin_t<TC, 3>(p, blocks, stream);
    default: return launch_lin_t<TC, 4>(p, blocks, stream);
  }
}

}  // namespace

LinearPlan plan_linear(int64_t m, int64_t n, int64_t k) {
  LinearPlan pl{};
  pl.m_tiles = static_cast<int>((m + 15) / 16);
  pl.n_blocks = (n + kLinCols - 1) / kLinCols;
  pl.chunks = (k + kLinChunk - 1) / kLinChunk;
  // split K until the grid covers every CU about twice (at least one chunk per split)
  int64_t splits = (kLinTargetWG + pl.n_blocks - 1) / pl.n_blocks;
  if (m <= kLinNarrowMaxM && splits > 1) {
    // the narrow kernel instead.  Two column tiles per wave for m > 16 when 8-wave workgroups of
    // 32 columns already give about kLinNarrowWaves waves (x loads then feed twice the MFMAs;
    // with fewer columns the lost workgroups cost more: 32 x 3840 x 1280 6.5 us at one tile,
    // 8.3 at two; 32 x 5120 x 1280 10.8 and 8.9).  Waves per workgroup doubled from 4 (at most
    // 16, 8 with two tiles, and not past the chunk count) until the grid holds about that many.
    const int tiles = (m > 16 && (n + 31) / 32 * 8 >= kLinNarrowWaves) ? 2 : 1;
    const int64_t cols = 16 * tiles;
    const int64_t nb = (n + cols - 1) / cols;
    const int kw_max = tiles == 2 ? 8 : 16;
    int kw = 4;
    while (kw < kw_max && nb * kw < kLinNarrowWaves && kw < pl.chunks) kw *= 2;
    pl.narrow_waves = kw;
    pl.narrow_tiles = tiles;
    pl.n_blocks = nb;
    // long K with fewer column blocks than CUs: K split over 2-4 workgroups as well, while each
    // split keeps at least one chunk per wave
    int64_t ns = 1;
    while (ns < kLinMaxSplits && nb * ns < kLinNarrowMinBlocks && pl.chunks >= 2 * ns * kw) ns *= 2;
    pl.chunks_per_split = (pl.chunks + ns - 1) / ns;
    pl.splits = (pl.chunks + pl.chunks_per_split - 1) / pl.chunks_per_split;
    pl.part_bytes = pl.splits > 1 ? static_cast<size_t>(nb) * pl.splits * tiles * pl.m_tiles * kWave * 4 * sizeof(float)
                                  : 0;
    pl.total_bytes = pl.splits > 1 ? NC_WORKSPACE_SYNC_BYTES + pl.part_bytes : 0;
    return pl;
  }
  splits = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(splits, pl.chunks), kLinMaxSplits));
  if (pl.n_blocks > kLinMaxTickets) splits = 1;
  pl.chunks_per_split = (pl.chunks + splits - 1) / splits;
  pl.splits = (pl.chunks + pl.chunks_per_split - 1) / pl.chunks_per_split;
  pl.part_bytes = pl.splits > 1
      ? static_cast<size_t>(pl.n_blocks) * pl.splits * kLinCols * pl.m_tiles * 16 * sizeof(float) : 0;
  pl.total_bytes = pl.splits > 1 ? NC_WORKSPACE_SYNC_BYTES + pl.part_bytes : 0;
  return pl;
}

hipError_t launch_linear(const nc_linear_args& a, const LinearPlan& pl, void* workspace, hipStream_t stream) {
  LinearParams p{};
  p.x = static_cast<const uint16_t*>(a.x);
  p.w = static_cast<const uint16_t*>(a.w);
  p.y = a.y;
  p.x_st = a.x_stride_m;
  p.w_st = a.w_stride_n;
  p.y_st = a.y_stride_m;
  p.m = static_cast<int>(a.m);
  p.n = static_cast<int>(a.n);
  p.k = static_cast<int>(a.k);
  p.chunks = static_cast<int>(pl.chunks);
  p.chunks_per_split = static_cast<int>(pl.chunks_per_split);
  p.splits = static_cast<int>(pl.splits);
  p.out_dtype = a.y_dtype;
  p.softcap = a.softcap;
  p.inv_softcap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
  if (pl.splits > 1) {
    p.tickets = static_cast<uint32_t*>(workspace);
    p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + NC_WORKSPACE_SYNC_BYTES);
  }
  if (pl.narrow_waves > 0) {
    return a.dtype == NC_DTYPE_BF16 ? launch_narrow<bf16>(p, pl.n_blocks, pl.narrow_waves, pl.narrow_tiles, stream)
                                    : launch_narrow<f16>(p, pl.n_blocks, pl.narrow_waves, pl.narrow_tiles, stream);
  }
  return a.dtype == NC_DTYPE_BF16 ? launch_lin_m<bf16>(p, pl.n_blocks, stream)
                                  : launch_lin_m<f16>(p, pl.n_blocks, stream);
}

}  // namespace nckv
