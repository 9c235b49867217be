// Shared device/host helpers for the gfx950 kernels of libsaeflow_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/saeflow_hip.h"

// ---------------------------------------------------------------------------
// host-side error reporting (thread-local message, see sf_last_error)
// ---------------------------------------------------------------------------
int sf_fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void sf_clear_error();

#define SF_REQUIRE(cond, ...)                          \
  do {                                                 \
    if (!(cond)) return sf_fail(SF_EINVAL, __VA_ARGS__); \
  } while (0)

#define SF_HIP_CHECK(expr)                                                          \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess)                                                           \
      return sf_fail(SF_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));       \
  } while (0)

// Launch-error check right after a <<<>>> launch.
#define SF_LAUNCH_CHECK(name)                                                       \
  do {                                                                              \
    hipError_t e_ = hipGetLastError();                                              \
    if (e_ != hipSuccess)                                                           \
      return sf_fail(SF_EHIP, "launch of %s failed: %s", name, hipGetErrorString(e_)); \
  } while (0)

__host__ __device__ static inline bool sf_valid_dtype(int dt) { return dt == SF_F32 || dt == SF_BF16 || dt == SF_F16; }
__host__ __device__ static inline int sf_dtype_size(int dt) { return dt == SF_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// device-side scalar conversions
// ---------------------------------------------------------------------------
typedef unsigned short u16;

// bf16 bits -> fp32 (exact)
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
// fp16 bits -> fp32 (exact)
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  u16 b = (u16)bits16;
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}
// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  u16 b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}
// fp32 -> fp16 bits, round to nearest even
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  u16 b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Load element i of a buffer of runtime dtype `dt` as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == SF_F32) return ((const float*)p)[i];
  uint32_t b = ((const u16*)p)[i];
  return dt == SF_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

// Raw bits of element i of a buffer of runtime dtype `dt` (16-bit types zero-extended), and
// those bits as fp32: load_as_f32 in two steps, so a load can be issued well before its use.
__device__ __forceinline__ uint32_t load_bits(const void* p, int dt, int64_t i) {
  return dt == SF_F32 ? ((const uint32_t*)p)[i] : (uint32_t)((const u16*)p)[i];
}
__device__ __forceinline__ float bits_as_f32(uint32_t b, int dt) {
  return dt == SF_F32 ? __uint_as_float(b) : (dt == SF_BF16 ? bf16_to_f32(b) : f16_to_f32(b));
}

// buffer_load_dwordx4 ... idxen through a structured buffer resource: 16 B at base + vindex *
// stride + voffset; a vindex at or past the resource's record count reads zeros without a
// memory access. The hardware forms vindex * stride + voffset in 32 bits, so the records must
// end below 2^31 bytes from the base, and the stride field holds at most 16383 bytes.
typedef uint32_t sf_u32x4 __attribute__((ext_vector_type(4)));
__device__ sf_u32x4 sf_struct_load_b128(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
constexpr uint32_t SF_RSRC_W3 = 0x00020000;  // buffer resource dword 3 for untyped loads (gfx9 family)

// Bits of fp32 value v rounded to dtype dt (low 16 bits used for 16-bit types).
__device__ __forceinline__ uint32_t f32_to_bits(float v, int dt) {
  if (dt == SF_F32) return __float_as_uint(v);
  return dt == SF_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
}

// Nonzero test on stored bits: +-0 are zero, everything else (NaN included) is not,
// which is exactly `f != 0.0` on the stored value.
__device__ __forceinline__ bool bits_nonzero(uint32_t bits, int esize) {
  return esize == 4 ? (bits & 0x7fffffffu) != 0 : (bits & 0x7fffu) != 0;
}

// Ordered key of a float's bits: unsigned order of keys == numeric order of values
// (NaN sorts above +inf for positive NaN, as in a total order).
__device__ __forceinline__ uint32_t float_key16(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
__device__ __forceinline__ uint32_t float_key32(uint32_t b) {
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Bit mask of the lanes below `lane` in a 64-lane wave.
__device__ __forceinline__ uint64_t lanemask_lt(int lane) { return (1ull << lane) - 1ull; }

// Exclusive prefix of v over the block's 256 threads (and the block total).
__device__ __forceinline__ int64_t block_exclusive_i64(int64_t v, int64_t* s_w, int64_t& total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_w[w] = x;
  __syncthreads();
  int64_t before = 0;
  total = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    before += q < w ? s_w[q] : 0;
    total += s_w[q];
  }
  return before + x - v;
}

// Exclusive prefix over the wave's lanes and wave total of c (0 <= c < 16), from 4 ballots.
__device__ __forceinline__ void wave_scan16(int c, int lane, int& prefix, int& total) {
  prefix = 0;
  total = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint64_t bal = __ballot((c >> b) & 1);
    prefix += __popcll(bal & lanemask_lt(lane)) << b;
    total += __popcll(bal) << b;
  }
}

// In-place bitonic sort of s[0..P) (P a power of two) by the threads of one block
// (nthreads threads, t = threadIdx.x), descending or ascending; ends with a barrier.
__device__ __forceinline__ void block_bitonic_sort(uint64_t* s, int P, int t, int nthreads, bool descending) {
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < P / 2; i += nthreads) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool first = ((lo & size) == 0) == descending;  // larger first in this half
        const uint64_t a = s[lo], b = s[hi];
        if (first ? (a < b) : (a > b)) {
          s[lo] = b;
          s[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

// Largest per-row candidate list the row-candidate consumers sort in LDS.
constexpr int SF_ROWS_CAP_MAX = 4096;
