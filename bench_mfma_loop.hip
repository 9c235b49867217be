// Measurement aid, not part of the SAE path: a register-only bf16 MFMA loop on every CU.
//
// It gives the rate at which this board sustains v_mfma_f32_32x32x16_bf16 when nothing
// else runs: no LDS, no memory traffic, no epilogue. Operands are 8 random fragments per
// lane, cycled so that every MFMA sees new inputs (operand toggling, like a real GEMM), and
// each wave keeps 8 accumulator tiles (128 registers), as the 8-wave encode GEMM does. The
// encode kernel's TFLOP/s divided by this rate is the share of the board's sustainable
// MFMA rate it reaches; the ratio of this rate to the datasheet peak is the clock the board
// holds at full MFMA load under its power limit.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NACC = 8;  // accumulator tiles per wave

// src: at least 1 << 20 16-B fragments; out: one float per thread of the grid.
__global__ __launch_bounds__(512, 1) void mfma_loop_kernel(const u32x4* __restrict__ src, float* __restrict__ out,
                                                           int iters, int active_threads) {
  if ((int)threadIdx.x >= active_threads) return;
  const int gid = blockIdx.x * 512 + threadIdx.x;
  u32x4 a[8], b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = src[(gid * 16 + j) & 0xFFFFF];
    b[j] = src[(gid * 16 + 8 + j) & 0xFFFFF];
  }
  f32x16 acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < NACC; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[(i + u) & 7]),
                                                         __builtin_bit_cast(bf16x8, b[(i + 3 * u) & 7]), acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NACC; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  out[gid] = s;  // keeps the loop live
}

}  // namespace

// Launches one workgroup per CU with `waves` (1..8) active waves, each running `iters`
// iterations of 64 MFMAs (32x32x16 bf16, 32768 flops each). src must hold 2^20 16-B
// fragments (16 MiB) of bf16 pairs; out must hold cus * 512 floats. Returns 0, or 1 for bad
// arguments, 2 for a HIP error. Flops per launch = cus * waves * iters * 64 * 32768.
extern "C" __attribute__((visibility("default"))) int sfp_mfma_loop(const void* src, float* out, int cus, int waves, int iters, void* stream) {
  if (!src || !out || cus <= 0 || waves < 1 || waves > 8 || iters <= 0) return 1;
  hipLaunchKernelGGL(mfma_loop_kernel, dim3((unsigned)cus), dim3(512), 0, (hipStream_t)stream,
                     (const u32x4*)src, out, iters, waves * 64);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
