// Instantiation unit of the tiled GEMM kernel (see gemm_kernel.h).
#include "gemm_kernel.h"

namespace afhip {

int gemm_dispatch_f16_a32(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
                          hipStream_t s) {
  return gemm_detail::dispatch_b_f16<float>(g, t, v, vec, label, s);
}

}  // namespace afhip
