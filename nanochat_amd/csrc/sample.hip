// Next-token sampling from fp32 logits, one workgroup per row
// (nanochat/engine.py:141-156 sample_next_token):
//   temperature == 0  -> argmax (first maximum; NaN counts as the maximum,
//                        as torch.argmax does);
//   top_k in [1, V)   -> the k largest logits, softmax of logits / T over
//                        them, one categorical draw;
//   otherwise         -> softmax of logits / T over the whole row, one draw.
// The draw is an inverse-CDF lookup with the caller's uniform u in [0, 1):
// the first category, in the order torch.topk returns them (value
// descending; equal values by index) or in index order for the whole row,
// whose running sum of exp(x - max) exceeds u times the total.  NaN logits
// are never drawn (treated as -inf); a row with no finite logit yields token
// 0 and sets NC_DEVERR_SAMPLE (torch.multinomial raises for such a row).
//
// Top-k: the k-th largest value is found by a radix select over the
// order-preserving 32-bit key of each logit (3 passes over digits of 11, 11
// and 10 bits, histograms in LDS); the k candidates (all larger values, then the first equal ones in
// index order) are compacted into LDS, sorted by a bitonic network, and
// scanned.  Whole-row draws scan per-thread contiguous segments.
// Every reduction and scan has a fixed order: results do not vary between
// runs.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

constexpr int kSmpThreads = 1024;
constexpr int kSmpWaves = kSmpThreads / kWave;
constexpr int kSmpBins = 2048;   // radix-select histogram: 11-bit digits, two bins per thread
static_assert(kSmpBins == 2 * kSmpThreads, "bin choice: each thread scans two adjacent bins");

struct SampleParams {
  const float* logits;
  int64_t stride;
  int vocab;
  int top_k;                 // 0: whole row
  float inv_temp;            // 0: argmax
  const float* uniforms;
  int64_t* out;
  int32_t* err;
};

// Larger float -> larger key; NaN maps to the key of -inf.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0xff800000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
constexpr uint32_t kKeyNegInf = 0x007fffffu;   // order_key(-inf)

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SmpShared {
  float f[kSmpWaves];
  int i[kSmpWaves];
  uint32_t u[kSmpWaves];
};

// f(i, v) for every element of the row, threads striding over 16-byte groups
// (coalesced), 4 groups in flight per thread; each thread sees its indices in
// increasing order.
template <typename F>
__device__ __forceinline__ void for_strided(const float* row, int vocab, F f) {
  int tail = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
    const int n4 = vocab / 4;
    const float4* r4 = reinterpret_cast<const float4*>(row);
    int g = threadIdx.x;
    for (; g + 3 * kSmpThreads < n4; g += 4 * kSmpThreads) {
      float4 a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = r4[g + u * kSmpThreads];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int b = 4 * (g + u * kSmpThreads);
        f(b, a[u].x); f(b + 1, a[u].y); f(b + 2, a[u].z); f(b + 3, a[u].w);
      }
    }
    for (; g < n4; g += kSmpThreads) {
      const float4 a = r4[g];
      f(4 * g, a.x); f(4 * g + 1, a.y); f(4 * g + 2, a.z); f(4 * g + 3, a.w);
    }
    tail = 4 * n4;
  }
  for (int j = tail + static_cast<int>(threadIdx.x); j < vocab; j += kSmpThreads) f(j, row[j]);
}

// f(i, v) for i in [i0, i1) in order, with 16-byte loads where aligned.
template <typename F>
__device__ __forceinline__ void for_segment(const float* row, int i0, int i1, F f) {
  int i = i0;
  if ((reinterpret_cast<uintptr_t>(row + i0) & 15u) == 0) {
    for (; i + 16 <= i1; i += 16) {
      float4 a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = *reinterpret_cast<const float4*>(row + i + 4 * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f(i + 4 * u, a[u].x); f(i + 4 * u + 1, a[u].y); f(i + 4 * u + 2, a[u].z); f(i + 4 * u + 3, a[u].w);
      }
    }
    for (; i + 4 <= i1; i += 4) {
      const float4 a = *reinterpret_cast<const float4*>(row + i);
      f(i, a.x); f(i + 1, a.y); f(i + 2, a.z); f(i + 3, a.w);
    }
  }
  for (; i < i1; ++i) f(i, row[i]);
}

// Thread t's contiguous segment of the row (a multiple of 4 elements long).
__device__ __forceinline__ void row_segment(int vocab, int& i0, int& i1) {
  const int seg = (((vocab + kSmpThreads - 1) / kSmpThreads) + 3) & ~3;
  i0 = min(vocab, static_cast<int>(threadIdx.x) * seg);
  i1 = min(vocab, i0 + seg);
}

// Exclusive prefix sum over the block's threads (thread order), and the total.
template <typename T>
__device__ T block_exclusive_scan(T v, T* wave_tot, T& total) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  T inc = v;
#pragma unroll
  for (int o = 1; o < kWave; o *= 2) {
    const T y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  __syncthreads();
  if (lane == kWave - 1) wave_tot[w] = inc;
  __syncthreads();
  T base = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < kSmpWaves; ++i) {
    base += i < w ? wave_tot[i] : T(0);
    tot += wave_tot[i];
  }
  total = tot;
  return base + inc - v;
}

// Argmax with torch's rule: NaN is the largest value, the first index wins.
__device__ void row_argmax(const float* row, int vocab, int64_t* out, SmpShared& sh) {
  float best = -INFINITY;
  int bi = INT32_MAX;
  bool bnan = false;
  for_strided(row, vocab, [&](int i, float v) __attribute__((always_inline)) {
    const bool nan = v != v;
    // strictly larger (NaN above everything) replaces; ties keep the earlier index
    const bool take = bi == INT32_MAX || (nan && !bnan) || (!bnan && !nan && v > best);
    if (take) { best = v; bi = i; bnan = nan; }
  });
  // wave reduce on (nan, value, -index)
#pragma unroll
  for (int o = kWave / 2; o > 0; o /= 2) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    const bool on = __shfl_xor(static_cast<int>(bnan), o) != 0;
    bool take;
    if (oi == INT32_MAX) take = false;
    else if (bi == INT32_MAX) take = true;
    else if (on != bnan) take = on;
    else if (!on && ov != best) take = ov > best;
    else take = oi < bi;
    if (take) { best = ov; bi = oi; bnan = on; }
  }
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) { sh.f[w] = best; sh.i[w] = bi; sh.u[w] = bnan; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sh.f[0];
    int idx = sh.i[0];
    bool n = sh.u[0] != 0;
    for (int k = 1; k < kSmpWaves; ++k) {
      const int oi = sh.i[k];
      const bool on = sh.u[k] != 0;
      bool take;
      if (oi == INT32_MAX) take = false;
      else if (idx == INT32_MAX) take = true;
      else if (on != n) take = on;
      else if (!on && sh.f[k] != b) take = sh.f[k] > b;
      else take = oi < idx;
      if (take) { b = sh.f[k]; idx = oi; n = on; }
    }
    *out = idx == INT32_MAX ? 0 : idx;
  }
}

__device__ __forceinline__ float finite_or_neg_inf(float v) { return v != v ? -INFINITY : v; }

// Whole-row draw: thread t owns the contiguous segment [t*seg, (t+1)*seg).
__device__ void row_sample_full(const SampleParams& p, const float* row, float u, int64_t* out, SmpShared& sh,
                                float* scan_tmp, int* pick) {
  const int vocab = p.vocab;
  int i0, i1;
  row_segment(vocab, i0, i1);
  float mx = -INFINITY;
  for_strided(row, vocab, [&](int, float v) __attribute__((always_inline)) { mx = fmaxf(mx, finite_or_neg_inf(v) * p.inv_temp); });
  // block max
#pragma unroll
  for (int o = kWave / 2; o > 0; o /= 2) mx = fmaxf(mx, __shfl_xor(mx, o));
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh.f[threadIdx.x / kWave] = mx;
  __syncthreads();
  float rmax = sh.f[0];
#pragma unroll
  for (int k = 1; k < kSmpWaves; ++k) rmax = fmaxf(rmax, sh.f[k]);
  if (rmax == -INFINITY) {   // no finite logit
    if (threadIdx.x == 0) {
      *out = 0;
      if (p.err) atomicOr(p.err, NC_DEVERR_SAMPLE);
    }
    return;
  }
  float local = 0.0f;
  int last_pos = -1;
  for_segment(row, i0, i1, [&](int i, float v) __attribute__((always_inline)) {
    const float e = expf(finite_or_neg_inf(v) * p.inv_temp - rmax);
    local += e;
    if (e > 0.0f) last_pos = i;
  });
  float total;
  const float excl = block_exclusive_scan<float>(local, scan_tmp, total);
  const float target = u * total;
  if (threadIdx.x == 0) { pick[0] = INT32_MAX; pick[1] = -1; }
  __syncthreads();
  // The segments' fp32 intervals [excl, excl + local) need not tile exactly
  // (excl of thread t + 1 can differ from excl + local of thread t by a
  // rounding), so there is no lower bound: every segment whose upper end lies
  // above the target looks for its first drawable element whose running sum
  // passes the target (its last drawable one if rounding leaves none), and
  // the lowest index wins.  A target in a rounding gap between two segments
  // then draws the first drawable element after the gap.
  if (local > 0.0f && target < excl + local) {
    float run = excl;
    int chosen = last_pos;
    for (int i = i0; i < i1; ++i) {
      const float e = expf(finite_or_neg_inf(row[i]) * p.inv_temp - rmax);
      run += e;
      if (e > 0.0f && run > target) { chosen = i; break; }
    }
    atomicMin(pick, chosen);
  }
  __syncthreads();
  if (*pick == INT32_MAX) {   // u * total rounded past the end: the last drawable index
    int lp = last_pos;
#pragma unroll
    for (int o = kWave / 2; o > 0; o /= 2) lp = max(lp, __shfl_xor(lp, o));
    if (threadIdx.x % kWave == 0) atomicMax(pick + 1, lp);
    __syncthreads();
    if (threadIdx.x == 0) *out = pick[1];
    return;
  }
  if (threadIdx.x == 0) *out = *pick;
}

// Top-k draw (1 <= k < vocab, k <= kMaxTopK).
__device__ void row_sample_topk(const SampleParams& p, const float* row, float u, int64_t* out, SmpShared& sh,
                                uint32_t* hist, uint32_t* ckey, int* cidx, float* scan_tmp, int* misc) {
  const int vocab = p.vocab, k = p.top_k;
  // ---- radix select: key of the k-th largest, and how many equal keys to take ----
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  // three passes over digits of 11, 11 and 10 bits (2048 bins; the last pass uses the lower 1024)
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 1023u : 2047u;
    for (int b = threadIdx.x; b < kSmpBins; b += kSmpThreads) hist[b] = 0;
    __syncthreads();
    for_strided(row, vocab, [&](int, float v) __attribute__((always_inline)) {
      const uint32_t key = order_key(v);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & dmask], 1u);
    });
    __syncthreads();
    // the bin holding the remaining-th largest key: thread t takes bins 2047 - 2t and 2046 - 2t,
    // in that order; an exclusive scan over the pairs gives the count of keys in higher bins
    const int hi_bin = kSmpBins - 1 - 2 * static_cast<int>(threadIdx.x);
    const int c_hi = static_cast<int>(hist[hi_bin]), c_lo = static_cast<int>(hist[hi_bin - 1]);
    int all;
    const int above = block_exclusive_scan<int>(c_hi + c_lo, reinterpret_cast<int*>(scan_tmp), all);
    if (c_hi > 0 && above < remaining && remaining <= above + c_hi) {
      misc[0] = hi_bin;
      misc[1] = remaining - above;
    } else if (c_lo > 0 && above + c_hi < remaining && remaining <= above + c_hi + c_lo) {
      misc[0] = hi_bin - 1;
      misc[1] = remaining - above - c_hi;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(misc[0]) << shift;
    mask |= dmask << shift;
    remaining = misc[1];
    __syncthreads();
  }
  const uint32_t kth = prefix;   // candidates: keys > kth, then the first `remaining` keys == kth
  // ---- compact the k candidates in index order (contiguous per-thread segments) ----
  int i0, i1;
  row_segment(vocab, i0, i1);
  int n_gt = 0, n_eq = 0;
  for_segment(row, i0, i1, [&](int, float v) __attribute__((always_inline)) {
    const uint32_t key = order_key(v);
    n_gt += key > kth;
    n_eq += key == kth;
  });
  int tot_gt, tot_eq;
  int* wt = reinterpret_cast<int*>(scan_tmp);
  int o_gt = block_exclusive_scan<int>(n_gt, wt, tot_gt);
  int o_eq = block_exclusive_scan<int>(n_eq, wt, tot_eq);
  if (n_gt + n_eq > 0) {
    for_segment(row, i0, i1, [&](int i, float v) __attribute__((always_inline)) {
      const uint32_t key = order_key(v);
      const bool gt = key > kth, eq = key == kth;
      if (gt) { ckey[o_gt] = key; cidx[o_gt] = i; }
      if (eq && o_eq < remaining) { ckey[tot_gt + o_eq] = key; cidx[tot_gt + o_eq] = i; }
      o_gt += gt;
      o_eq += eq;
    });
  }
  // pad to a power of two with entries that sort last
  int np2 = 1;
  while (np2 < k) np2 *= 2;
  for (int j = k + static_cast<int>(threadIdx.x); j < np2; j += kSmpThreads) { ckey[j] = 0u; cidx[j] = INT32_MAX; }
  __syncthreads();
  // ---- bitonic sort: key descending, index ascending ----
  for (int size = 2; size <= np2; size *= 2) {
    for (int stride = size / 2; stride > 0; stride /= 2) {
      for (int t = threadIdx.x; t < np2 / 2; t += kSmpThreads) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint32_t ka = ckey[lo], kb = ckey[hi];
        const int ia = cidx[lo], ib = cidx[hi];
        const bool a_first = ka > kb || (ka == kb && ia < ib);
        if (a_first != desc) {
          ckey[lo] = kb; ckey[hi] = ka; cidx[lo] = ib; cidx[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
  // ---- softmax over the sorted candidates and the inverse-CDF draw ----
  if (ckey[0] == kKeyNegInf) {   // no finite candidate
    if (threadIdx.x == 0) {
      *out = 0;
      if (p.err) atomicOr(p.err, NC_DEVERR_SAMPLE);
    }
    return;
  }
  const float x0 = key_value(ckey[0]) * p.inv_temp;
  // thread t owns candidates 2t, 2t+1 (k <= 2 * kSmpThreads)
  float e[2];
  float local = 0.0f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = 2 * static_cast<int>(threadIdx.x) + q;
    e[q] = j < k ? expf(key_value(ckey[j]) * p.inv_temp - x0) : 0.0f;
    local += e[q];
  }
  float total;
  const float excl = block_exclusive_scan<float>(local, scan_tmp + kSmpWaves, total);
  const float target = u * total;
  if (threadIdx.x == 0) misc[2] = INT32_MAX;
  __syncthreads();
  const int j0 = 2 * static_cast<int>(threadIdx.x);
  const float run0 = excl + e[0], run1 = run0 + e[1];
  const int found = (j0 < k && e[0] > 0.0f && run0 > target) ? j0
                  : ((j0 + 1 < k && e[1] > 0.0f && run1 > target) ? j0 + 1 : INT32_MAX);
  if (found != INT32_MAX) atomicMin(&misc[2], found);
  __syncthreads();
  if (threadIdx.x == 0) {
    int j = misc[2];
    if (j == INT32_MAX) {   // rounding past the end: the last candidate with weight
      j = k - 1;
      while (j > 0 && ckey[j] == kKeyNegInf) --j;
    }
    *out = cidx[j];
  }
}

__global__ __launch_bounds__(kSmpThreads) void sample_kernel(const SampleParams p) {
  __shared__ SmpShared sh;
  __shared__ uint32_t hist[kSmpBins];
  __shared__ uint32_t ckey[kMaxTopK];
  __shared__ int cidx[kMaxTopK];
  __shared__ float scan_tmp[2 * kSmpWaves];
  __shared__ int misc[4];
  const int b = blockIdx.x;
  const float* row = p.logits + static_cast<int64_t>(b) * p.stride;
  int64_t* out = p.out + b;
  if (p.inv_temp == 0.0f) {
    row_argmax(row, p.vocab, out, sh);
    return;
  }
  float u = p.uniforms[b];
  u = u < 0.0f ? 0.0f : (u >= 1.0f ? 0x1.fffffep-1f : u);
  if (p.top_k > 0 && p.top_k < p.vocab) {
    row_sample_topk(p, row, u, out, sh, hist, ckey, cidx, scan_tmp, misc);
  } else {
    row_sample_full(p, row, u, out, sh, scan_tmp, misc);
  }
}

}  // namespace

hipError_t launch_sample(const nc_sample_args& a, hipStream_t stream) {
  SampleParams p{};
  p.logits = a.logits;
  p.stride = a.logits_stride;
  p.vocab = static_cast<int>(a.vocab);
  p.top_k = a.top_k >= a.vocab ? 0 : a.top_k;
  p.inv_temp = a.temperature > 0.0f ? 1.0f / a.temperature : 0.0f;
  p.uniforms = a.uniforms;
  p.out = a.out;
  p.err = a.error_flag;
  hipLaunchKernelGGL(sample_kernel, dim3(static_cast<unsigned>(a.batch)), dim3(kSmpThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nckv
