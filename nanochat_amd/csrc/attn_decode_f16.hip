// Decode kernels for f16 caches (attn_decode_kernels.hpp), in a translation
// unit of their own.

#include "attn_decode_kernels.hpp"

namespace nckv {

hipError_t launch_decode_f16(const DecodeParams& p, bool qpk, int64_t head_dim, int gb, int64_t n_wg, bool wide,
                              hipStream_t stream) {
  return qpk ? launch_dt<f16, true>(p, head_dim, gb, n_wg, wide, stream)
             : launch_dt<f16, false>(p, head_dim, gb, n_wg, wide, stream);
}

}  // namespace nckv
