// Cache write kernels: the ragged KV append and the prefill fan-out copy.
//
// append : nanochat/flash_attention.py:160-162 with FA3's per-row positions.
// fan-out: nanochat/engine.py:132-134 (+ :134 cache_seqlens.fill_).
// Both are pure HBM streams; every thread moves 16-byte vectors so each wave
// issues fully coalesced 1 KiB loads and stores.

#include "nc_kv_common.hpp"
#include "nc_kv_internal.hpp"

namespace nckv {

namespace {

struct AppendParams {
  void* kc;
  void* vc;
  const void* k;
  const void* v;
  const int32_t* seqlens;
  int32_t* err;
  int64_t kc_sb, kc_st, kc_sh, vc_sb, vc_st, vc_sh;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
  int32_t t_new, t_max, h_kv, vecs_per_head;  // vecs_per_head = D / VEC
  int64_t n_vec;                                 // B * t_new * h_kv * vecs_per_head
  int32_t in_dtype;
};

// One thread per 16-byte cache vector; blockIdx.y selects K (0) or V (1).
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParams p) {
  constexpr int VEC = 16 / elem<T>::kBytes;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= p.n_vec) return;
  const bool is_v = blockIdx.y != 0;
  int64_t r = i;
  const int c = static_cast<int>(r % p.vecs_per_head); r /= p.vecs_per_head;
  const int h = static_cast<int>(r % p.h_kv); r /= p.h_kv;
  const int t = static_cast<int>(r % p.t_new);
  const int64_t b = r / p.t_new;
  const int pos = p.seqlens[b] + t;
  if (pos < 0 || pos >= p.t_max) {
    if (p.err != nullptr && c == 0 && h == 0 && !is_v) atomicOr(p.err, NC_DEVERR_OVERFLOW);
    return;
  }
  const void* src = is_v ? p.v : p.k;
  const int64_t soff = is_v ? (b * p.v_sb + t * p.v_st + h * p.v_sh)
                            : (b * p.k_sb + t * p.k_st + h * p.k_sh);
  const uint4 val = load_as_cache_vec<T>(src, soff + static_cast<int64_t>(c) * VEC, p.in_dtype);
  char* dst = static_cast<char*>(is_v ? p.vc : p.kc);
  const int64_t doff = is_v ? (b * p.vc_sb + pos * p.vc_st + h * p.vc_sh)
                            : (b * p.kc_sb + pos * p.kc_st + h * p.kc_sh);
  *reinterpret_cast<uint4*>(dst + (doff + static_cast<int64_t>(c) * VEC) * elem<T>::kBytes) = val;
}

struct FanoutParams {
  const char* src[2];
  char* dst[2];
  int32_t* seqlens;
  int64_t units;          // copy units per layer region
  int64_t src_stride_l;   // bytes
  int64_t dst_stride_l;   // bytes
  int64_t dst_stride_b;   // bytes
  int32_t n_rows;
  int32_t prefix_len;
};

constexpr int kFanoutUnitsPerThread = 4;

// grid: x over the per-layer region, y = layer, z = K/V.  Each thread loads
// kFanoutUnitsPerThread units of the source once and stores them into every
// destination row.
template <typename U>
__global__ __launch_bounds__(256) void kv_fanout_kernel(const FanoutParams p) {
  if (p.seqlens != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {
    for (int n = threadIdx.x; n < p.n_rows; n += blockDim.x) p.seqlens[n] = p.prefix_len;
  }
  const int z = blockIdx.z;
  const int64_t l = blockIdx.y;
  const U* src = reinterpret_cast<const U*>(p.src[z] + l * p.src_stride_l);
  char* dst_layer = p.dst[z] + l * p.dst_stride_l;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x * kFanoutUnitsPerThread + threadIdx.x;
  U val[kFanoutUnitsPerThread];
#pragma unroll
  for (int u = 0; u < kFanoutUnitsPerThread; ++u) {
    const int64_t idx = base + static_cast<int64_t>(u) * blockDim.x;
    if (idx < p.units) val[u] = src[idx];
  }
  for (int n = 0; n < p.n_rows; ++n) {
    U* dst = reinterpret_cast<U*>(dst_layer + n * p.dst_stride_b);
#pragma unroll
    for (int u = 0; u < kFanoutUnitsPerThread; ++u) {
      const int64_t idx = base + static_cast<int64_t>(u) * blockDim.x;
      if (idx < p.units) dst[idx] = val[u];
    }
  }
}

}  // namespace

hipError_t launch_append(const nc_append_args& a, hipStream_t stream) {
  AppendParams p;
  p.kc = a.k_cache; p.vc = a.v_cache; p.k = a.k; p.v = a.v;
  p.seqlens = a.cache_seqlens; p.err = a.error_flag;
  p.kc_sb = a.kc_stride_b; p.kc_st = a.kc_stride_t; p.kc_sh = a.kc_stride_h;
  p.vc_sb = a.vc_stride_b; p.vc_st = a.vc_stride_t; p.vc_sh = a.vc_stride_h;
  p.k_sb = a.k_stride_b; p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
  p.v_sb = a.v_stride_b; p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
  p.t_new = static_cast<int32_t>(a.t_new);
  p.t_max = static_cast<int32_t>(a.t_max);
  p.h_kv = static_cast<int32_t>(a.n_kv_heads);
  p.in_dtype = a.in_dtype;
  const int ebytes = a.cache_dtype == NC_DTYPE_F32 ? 4 : 2;
  const int vec = 16 / ebytes;
  p.vecs_per_head = static_cast<int32_t>(a.head_dim / vec);
  p.n_vec = a.batch * a.t_new * a.n_kv_heads * p.vecs_per_head;
  const dim3 block(256);
  const dim3 grid(static_cast<unsigned>((p.n_vec + 255) / 256), 2);
  switch (a.cache_dtype) {
    case NC_DTYPE_BF16: hipLaunchKernelGGL(kv_append_kernel<bf16>, grid, block, 0, stream, p); break;
    case NC_DTYPE_F16: hipLaunchKernelGGL(kv_append_kernel<f16>, grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL(kv_append_kernel<float>, grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

hipError_t launch_fanout(const nc_fanout_args& a, int unit_bytes, hipStream_t stream) {
  const int64_t ebytes = a.dtype == NC_DTYPE_F32 ? 4 : 2;
  FanoutParams p;
  p.src[0] = static_cast<const char*>(a.k_src);
  p.src[1] = static_cast<const char*>(a.v_src);
  p.dst[0] = static_cast<char*>(a.k_dst);
  p.dst[1] = static_cast<char*>(a.v_dst);
  p.seqlens = a.dst_seqlens;
  p.units = a.prefix_len * a.row_elems * ebytes / unit_bytes;
  p.src_stride_l = a.src_stride_l * ebytes;
  p.dst_stride_l = a.dst_stride_l * ebytes;
  p.dst_stride_b = a.dst_stride_b * ebytes;
  p.n_rows = static_cast<int32_t>(a.n_rows);
  p.prefix_len = static_cast<int32_t>(a.prefix_len);
  const int64_t per_block = 256 * kFanoutUnitsPerThread;
  const int64_t gx = p.units > 0 ? (p.units + per_block - 1) / per_block : 1;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(a.n_layers), 2);
  const dim3 block(256);
  if (unit_bytes == 16) {
    hipLaunchKernelGGL(kv_fanout_kernel<uint4>, grid, block, 0, stream, p);
  } else if (unit_bytes == 4) {
    hipLaunchKernelGGL(kv_fanout_kernel<uint32_t>, grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(kv_fanout_kernel<uint16_t>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace nckv
