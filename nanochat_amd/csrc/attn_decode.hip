// Decode attention host side: launch parameters, plans' helpers, and the
// dispatch to the per-dtype translation units.  The kernels (and their
// description) are in attn_decode_kernels.hpp.

#include "attn_decode_kernels.hpp"

namespace nckv {

bool decode_wide_supported(int head_block, int64_t head_dim) {
  return head_block <= 4 && head_block * head_dim <= kWideMaxElems;
}

bool decode_supports(int cache_dtype, int64_t head_dim) {
  (void)cache_dtype;
  return head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
}

int max_splits() { return kMaxMergeSplits; }

int default_split_bytes() { return NC_DECODE_KEY_BYTES; }

int64_t decode_grid(int64_t n_groups, int num_splits) {
#if NC_DECODE_XCD_MAP
  return kXcds * num_splits * ((n_groups + kXcds - 1) / kXcds);
#else
  return num_splits * n_groups;
#endif
}

namespace {

void set_divisors(DecodeParams& p) {
  p.fd_hblocks = make_fastdiv(static_cast<uint32_t>(p.n_hblocks));
  p.fd_kv_heads = make_fastdiv(static_cast<uint32_t>(p.n_kv_heads));
  p.fd_t_new = make_fastdiv(static_cast<uint32_t>(p.t_new));
  p.fd_splits = make_fastdiv(static_cast<uint32_t>(p.num_splits));
  p.fd_kps = make_fastdiv(static_cast<uint32_t>(p.keys_per_split));
}

DecodeParams make_params(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s, bool fused_append) {
  DecodeParams p;
  p.q = a.q; p.out = a.out;
  p.kc = static_cast<char*>(a.k_cache); p.vc = static_cast<char*>(a.v_cache);
  p.k_new = a.k; p.v_new = a.v;
  p.seqlens = a.cache_seqlens; p.err = a.error_flag;
  p.cache_idx = a.cache_batch_idx; p.cache_batch = a.cache_batch;
  p.cu_q = a.cu_seqlens_q; p.total_q = a.total_q;
  p.pages = page_map(a.page_table, a.page_table_stride, a.page_size, a.num_blocks);
  p.indirect = (a.cache_batch_idx != nullptr || a.cu_seqlens_q != nullptr || a.page_table != nullptr) ? 1 : 0;
  p.q_bound = p.len_hi = static_cast<int32_t>(a.t_new);
  p.len_lo = 0;
  p.part_ml = s.part_ml; p.part_o = s.part_o;
  p.tickets = plan.merge_in_kernel ? s.tickets : nullptr;
  p.q_sb = a.q_stride_b; p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
  p.kc_sb = a.kc_stride_b; p.kc_st = a.kc_stride_t; p.kc_sh = a.kc_stride_h;
  p.vc_sb = a.vc_stride_b; p.vc_st = a.vc_stride_t; p.vc_sh = a.vc_stride_h;
  p.k_sb = a.k_stride_b; p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
  p.v_sb = a.v_stride_b; p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
  p.t_new = static_cast<int32_t>(a.t_new);
  p.t_max = static_cast<int32_t>(a.t_max);
  p.n_heads = static_cast<int32_t>(a.n_heads);
  p.n_kv_heads = static_cast<int32_t>(a.n_kv_heads);
  p.group = plan.group;
  p.n_hblocks = plan.n_hblocks;
  p.n_units = plan.n_units;
  p.n_groups = plan.n_groups;
  p.window = a.window_left;
  p.scale_log2 = a.softmax_scale * 1.4426950408889634f;
  p.q_dtype = a.q_dtype;
  p.num_splits = plan.num_splits;
  p.keys_per_split = plan.keys_per_split;
  p.fused = fused_append ? 1 : 0;
  p.bal_rows = plan.bal ? static_cast<int32_t>(a.batch) : 0;
  p.bal_min_tiles = NC_DECODE_BAL_MIN_TILES;
  p.bal_den = static_cast<int32_t>(plan.n_wg - plan.n_groups);
  p.rope_cos = p.rope_sin = nullptr;
  p.rope = 0;
  p.rope_len = 1;
  p.rope_half = static_cast<int32_t>(a.head_dim / 2);
  p.rope_dtype = NC_DTYPE_F32;
  p.rope_scale = 1.0f;
  p.rope_eps = 0.0f;
  set_divisors(p);
  return p;
}

}  // namespace

hipError_t launch_decode(const nc_attn_args& a, const AttnPlan& plan, const AttnScratch& s,
                         bool fused_append, const nc_qk_prologue* prologue, hipStream_t stream,
                         const RowFilter* rows) {
  DecodeParams p = make_params(a, plan, s, fused_append);
  if (rows != nullptr) {
    p.len_lo = rows->lo;
    p.len_hi = rows->hi;
    p.q_bound = rows->bound;
  }
  if (prologue != nullptr) {
    p.rope = 1;
    p.rope_cos = prologue->cos;
    p.rope_sin = prologue->sin;
    p.rope_len = static_cast<int32_t>(prologue->rot_len);
    p.rope_dtype = prologue->rot_dtype;
    p.rope_scale = prologue->qk_scale;
    p.rope_eps = prologue->eps;
  }
  const bool qpk = a.q_dtype == a.cache_dtype && a.cache_dtype != NC_DTYPE_F32;
  const int gb = plan.head_block;
  switch (a.cache_dtype) {
    case NC_DTYPE_BF16: return launch_decode_bf16(p, qpk, a.head_dim, gb, plan.n_wg, plan.wide, stream);
    case NC_DTYPE_F16: return launch_decode_f16(p, qpk, a.head_dim, gb, plan.n_wg, plan.wide, stream);
    default: return launch_decode_f32(p, a.head_dim, gb, plan.n_wg, plan.wide, stream);
  }
}

}  // namespace nckv
