// 256x256 gathered-row encode kernels (sf_encode_gather) for f32 MFMA inputs, 16-bit and fp32
// outputs.
#include "encode_kernels.h"

namespace sfenc {
template hipError_t launch_live<SF_F32, 2>(const GemmArgs&, int, int, hipStream_t);
template hipError_t launch_live<SF_F32, 4>(const GemmArgs&, int, int, hipStream_t);
}  // namespace sfenc
