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
  const int32_t* cache_idx;  // cache_batch_idx or NULL
  int64_t cache_batch;
  const int32_t* cu_q;       // cu_seqlens_q (packed new tokens) or NULL
  int64_t total_q;
  PageMap pages;             // paged cache (page_table), or pages.table == NULL
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
  const int64_t cb = p.pages.table != nullptr
      ? 0 : cache_row(p.cache_idx, p.cache_batch, b, p.err, c == 0 && h == 0 && t == 0 && !is_v);
  if (cb < 0) return;
  const RowQ rq = row_queries(p.cu_q, p.total_q, b, p.t_new, p.err, c == 0 && h == 0 && t == 0 && !is_v);
  if (t >= rq.len) return;
  const int lpos = p.seqlens[b] + t;
  if (lpos < 0 || lpos >= p.t_max) {
    if (p.err != nullptr && c == 0 && h == 0 && !is_v) atomicOr(p.err, NC_DEVERR_OVERFLOW);
    return;
  }
  // cache row of the position: the page table's slot for paged caches
  const int64_t pos = p.pages.table != nullptr ? page_pos(p.pages, b, lpos, c == 0 ? p.err : nullptr) : lpos;
  if (pos < 0) return;
  const void* src = is_v ? p.v : p.k;
  const int64_t soff = is_v ? token_offset(p.cu_q, rq, b, t, p.v_sb, p.v_st) + h * p.v_sh
                            : token_offset(p.cu_q, rq, b, t, p.k_sb, p.k_st) + h * p.k_sh;
  const uint4 val = load_as_cache_vec<T>(src, soff + static_cast<int64_t>(c) * VEC, p.in_dtype);
  char* dst = static_cast<char*>(is_v ? p.vc : p.kc);
  const int64_t doff = is_v ? (cb * p.vc_sb + pos * p.vc_st + h * p.vc_sh)
                            : (cb * p.kc_sb + pos * p.kc_st + h * p.kc_sh);
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
// Non-temporal store of one copy unit (the fan-out writes far more than the
// L2s hold and nothing reads it back in the same launch).
__device__ __forceinline__ void store_nt(uint4* p, const uint4& v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void store_nt(uint32_t* p, uint32_t v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_nt(uint16_t* p, uint16_t v) { __builtin_nontemporal_store(v, p); }

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
  // every element defined on every path, so the values stay in registers
  // (a conditionally written array was placed in LDS by the compiler and
  // re-read, bank-conflicted, for each destination row)
  U val[kFanoutUnitsPerThread];
  bool in[kFanoutUnitsPerThread];
#pragma unroll
  for (int u = 0; u < kFanoutUnitsPerThread; ++u) {
    const int64_t idx = base + static_cast<int64_t>(u) * blockDim.x;
    in[u] = idx < p.units;
    val[u] = in[u] ? src[idx] : U{};
  }
  for (int n = 0; n < p.n_rows; ++n) {
    U* dst = reinterpret_cast<U*>(dst_layer + n * p.dst_stride_b);
#pragma unroll
    for (int u = 0; u < kFanoutUnitsPerThread; ++u) {
      if (in[u]) store_nt(dst + base + static_cast<int64_t>(u) * blockDim.x, val[u]);
    }
  }
}

// QK prologue for chunks (t_new > 1): one row of D elements per G = D/8 lanes,
// rows enumerated (b, t, slot) with slots [0, H) the q heads, [H, H + H_kv)
// the k heads and [H + H_kv, H + 2 H_kv) the v heads.  q and k go through
// qk_prologue_lanes (rotary at table row s_b + t, RMS norm, scale); q is
// written to q_out (contiguous, q's dtype), k and v are appended into the
// cache at s_b + t (k rounded RNE to the cache dtype; v copied as copy_ does).
struct RopeAppendParams {
  const void* q;
  void* q_out;
  const void* k;
  const void* v;
  char* kc;
  char* vc;
  const int32_t* seqlens;
  int32_t* err;
  const int32_t* cache_idx;  // cache_batch_idx or NULL
  int64_t cache_batch;
  const int32_t* cu_q;       // cu_seqlens_q (packed tokens) or NULL
  int64_t total_q;
  PageMap pages;             // paged cache (page_table), or pages.table == NULL
  const void* cos;
  const void* sin;
  int64_t q_sb, q_st, q_sh, k_sb, k_st, k_sh, v_sb, v_st, v_sh;
  int64_t kc_sb, kc_st, kc_sh, vc_sb, vc_st, vc_sh;
  int64_t n_rows;                 // B * t_new * (H + 2 H_kv)
  int32_t t_new, t_max, n_heads, n_kv_heads, q_dtype, cache_dtype, rot_len, rot_dtype;
  float scale, eps;
};

// One element of a runtime-typed input into a runtime-typed tensor, as copy_
// does (same dtype: the bits).
__device__ __forceinline__ void copy_elem(void* dst, int64_t di, int out_dtype, const void* src, int64_t si,
                                          int in_dtype) {
  if (in_dtype == out_dtype) {
    if (in_dtype == NC_DTYPE_F32) {
      static_cast<uint32_t*>(dst)[di] = static_cast<const uint32_t*>(src)[si];
    } else {
      static_cast<uint16_t*>(dst)[di] = static_cast<const uint16_t*>(src)[si];
    }
  } else {
    store_any(dst, di, out_dtype, load_any(src, si, in_dtype));
  }
}

template <int D>
__global__ __launch_bounds__(256) void qk_rope_append_kernel(const RopeAppendParams p) {
  constexpr int VE = 8;
  constexpr int G = D / VE;          // lanes per row
  constexpr int RPW = kWave / G;     // rows per wave
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % G;
  const int64_t r = (static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave) * RPW + lane / G;
  const bool live = r < p.n_rows;
  const int per = p.n_heads + 2 * p.n_kv_heads;
  int64_t rr = live ? r : 0;
  const int slot = static_cast<int>(rr % per);
  rr /= per;
  const int t = static_cast<int>(rr % p.t_new);
  const int64_t b = rr / p.t_new;
  const int pos = p.seqlens[b] + t;
  const int kind = slot < p.n_heads ? 0 : (slot < p.n_heads + p.n_kv_heads ? 1 : 2);  // q, k, v
  const int h = kind == 0 ? slot : (kind == 1 ? slot - p.n_heads : slot - p.n_heads - p.n_kv_heads);
  // every lane of a row group takes part in the prologue's shuffles, so rows
  // past a row's query count still run it (on zeros) and skip their stores
  const RowQ rq = row_queries(p.cu_q, p.total_q, b, p.t_new, p.err, live && c == 0 && t == 0 && slot == 0);
  const bool active = live && t < rq.len;
  const void* src = kind == 0 ? p.q : (kind == 1 ? p.k : p.v);
  const int64_t soff = kind == 0 ? token_offset(p.cu_q, rq, b, t, p.q_sb, p.q_st) + h * p.q_sh
                                 : (kind == 1 ? token_offset(p.cu_q, rq, b, t, p.k_sb, p.k_st) + h * p.k_sh
                                              : token_offset(p.cu_q, rq, b, t, p.v_sb, p.v_st) + h * p.v_sh);
  float x[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) x[e] = active ? load_any(src, soff + c * VE + e, p.q_dtype) : 0.0f;
  const int row = min(max(pos, 0), p.rot_len - 1);
  qk_prologue_lanes<G, VE>(x, c, p.cos, p.sin, row, p.rot_dtype, p.scale, p.eps);  // every lane takes part
  if (!active) return;
  if (kind == 0) {
    if (c == 0 && (pos < 0 || pos >= p.rot_len) && p.err != nullptr) atomicOr(p.err, NC_DEVERR_ROPE_RANGE);
    const int64_t o0 = ((rq.tok0 + t) * p.n_heads + h) * D + c * VE;
#pragma unroll
    for (int e = 0; e < VE; ++e) store_any(p.q_out, o0 + e, p.q_dtype, x[e]);
    return;
  }
  const int64_t cb = p.pages.table != nullptr
      ? 0 : cache_row(p.cache_idx, p.cache_batch, b, p.err, c == 0 && h == 0 && t == 0 && kind == 1);
  if (cb < 0) return;
  if (pos < 0 || pos >= p.t_max) {
    if (c == 0 && h == 0 && kind == 1 && p.err != nullptr) atomicOr(p.err, NC_DEVERR_OVERFLOW);
    return;
  }
  // cache row of the position: the page table's slot for paged caches
  const int64_t cpos = p.pages.table != nullptr ? page_pos(p.pages, b, pos, c == 0 ? p.err : nullptr) : pos;
  if (cpos < 0) return;
  if (kind == 1) {
    const int64_t d0 = cb * p.kc_sb + cpos * p.kc_st + h * p.kc_sh + c * VE;
#pragma unroll
    for (int e = 0; e < VE; ++e) store_any(p.kc, d0 + e, p.cache_dtype, x[e]);
  } else {
    const int64_t d0 = cb * p.vc_sb + cpos * p.vc_st + h * p.vc_sh + c * VE;
#pragma unroll
    for (int e = 0; e < VE; ++e) copy_elem(p.vc, d0 + e, p.cache_dtype, p.v, soff + c * VE + e, p.q_dtype);
  }
}

}  // namespace

hipError_t launch_append(const nc_append_args& a, hipStream_t stream) {
  AppendParams p;
  p.kc = a.k_cache; p.vc = a.v_cache; p.k = a.k; p.v = a.v;
  p.seqlens = a.cache_seqlens; p.err = a.error_flag;
  p.cache_idx = a.cache_batch_idx; p.cache_batch = a.cache_batch;
  p.cu_q = a.cu_seqlens_q; p.total_q = a.total_q;
  p.pages = page_map(a.page_table, a.page_table_stride, a.page_size, a.num_blocks);
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

hipError_t launch_rope_append(const nc_attn_args& a, const nc_qk_prologue& pro, void* q_out, hipStream_t stream) {
  RopeAppendParams p;
  p.q = a.q; p.q_out = q_out; p.k = a.k; p.v = a.v;
  p.kc = static_cast<char*>(a.k_cache); p.vc = static_cast<char*>(a.v_cache);
  p.seqlens = a.cache_seqlens; p.err = a.error_flag;
  p.cache_idx = a.cache_batch_idx; p.cache_batch = a.cache_batch;
  p.cu_q = a.cu_seqlens_q; p.total_q = a.total_q;
  p.pages = page_map(a.page_table, a.page_table_stride, a.page_size, a.num_blocks);
  p.cos = pro.cos; p.sin = pro.sin;
  p.q_sb = a.q_stride_b; p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
  p.k_sb = a.k_stride_b; p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
  p.v_sb = a.v_stride_b; p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
  p.kc_sb = a.kc_stride_b; p.kc_st = a.kc_stride_t; p.kc_sh = a.kc_stride_h;
  p.vc_sb = a.vc_stride_b; p.vc_st = a.vc_stride_t; p.vc_sh = a.vc_stride_h;
  p.n_rows = a.batch * a.t_new * (a.n_heads + 2 * a.n_kv_heads);
  p.t_new = static_cast<int32_t>(a.t_new);
  p.t_max = static_cast<int32_t>(a.t_max);
  p.n_heads = static_cast<int32_t>(a.n_heads);
  p.n_kv_heads = static_cast<int32_t>(a.n_kv_heads);
  p.q_dtype = a.q_dtype;
  p.cache_dtype = a.cache_dtype;
  p.rot_len = static_cast<int32_t>(pro.rot_len);
  p.rot_dtype = pro.rot_dtype;
  p.scale = pro.qk_scale;
  p.eps = pro.eps;
  const int64_t rows_per_block = 4 * (kWave / (a.head_dim / 8));
  const dim3 grid(static_cast<unsigned>((p.n_rows + rows_per_block - 1) / rows_per_block)), block(256);
  switch (a.head_dim) {
    case 32: hipLaunchKernelGGL(qk_rope_append_kernel<32>, grid, block, 0, stream, p); break;
    case 64: hipLaunchKernelGGL(qk_rope_append_kernel<64>, grid, block, 0, stream, p); break;
    case 128: hipLaunchKernelGGL(qk_rope_append_kernel<128>, grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL(qk_rope_append_kernel<256>, grid, block, 0, stream, p); break;
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
