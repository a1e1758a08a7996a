// jh_mfma.hip -- batched decode (B >= 16) through LDS dequant + fp16 MFMA.
#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {

hipError_t launch_gemm_mfma(const GemvArgs &, hipStream_t) { return hipErrorNotSupported; }

}  // namespace jh
