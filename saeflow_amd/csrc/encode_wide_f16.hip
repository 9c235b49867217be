// 256x256 encode kernels for f16 MFMA inputs (16-bit and fp32 outputs, 8 and 4 waves).
#include "encode_kernels.h"

namespace sfenc {
template hipError_t launch_wide<SF_F16, 2>(const GemmArgs&, int, int, hipStream_t);
template hipError_t launch_wide<SF_F16, 4>(const GemmArgs&, int, int, hipStream_t);
}  // namespace sfenc
