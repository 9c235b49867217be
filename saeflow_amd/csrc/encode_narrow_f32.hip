// 256x128 encode kernels for f32 MFMA inputs (16-bit and fp32 outputs).
#include "encode_kernels.h"

namespace sfenc {
template hipError_t launch_narrow<SF_F32, 2>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_narrow<SF_F32, 4>(const GemmArgs&, int, hipStream_t);
}  // namespace sfenc
