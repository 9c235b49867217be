// 256x256 encode kernels with the row-candidate epilogue for bf16 MFMA inputs, one per output
// type, without and with a row floor.
#include "encode_kernels.h"

namespace sfenc {
template hipError_t launch_rows<SF_BF16, SF_F32, EPI_ROWS>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_rows<SF_BF16, SF_BF16, EPI_ROWS>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_rows<SF_BF16, SF_F16, EPI_ROWS>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_rows<SF_BF16, SF_F32, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_rows<SF_BF16, SF_BF16, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t);
template hipError_t launch_rows<SF_BF16, SF_F16, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t);
}  // namespace sfenc
