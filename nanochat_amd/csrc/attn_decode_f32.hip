// Decode kernels for fp32 caches (attn_decode_kernels.hpp), in a translation
// unit of their own.

#include "attn_decode_kernels.hpp"

namespace nckv {

hipError_t launch_decode_f32(const DecodeParams& p, int64_t head_dim, int gb, int64_t n_wg, bool wide,
                             hipStream_t stream) {
  return launch_dt<float, false>(p, head_dim, gb, n_wg, wide, stream);
}

}  // namespace nckv
