// 256x256 gathered-row encode kernels (sf_encode_gather) for bf16 MFMA inputs, 16-bit and fp32
// outputs.
#include "encode_kernels.h"

namespace sfenc {
template hipError_t launch_live<SF_BF16, 2>(const GemmArgs&, int, int, hipStream_t);
template hipError_t launch_live<SF_BF16, 4>(const GemmArgs&, int, int, hipStream_t);
}  // namespace sfenc
