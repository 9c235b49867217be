#pragma once
// Kernels of the fused SAE encoder on gfx950 MFMA:  out = act((x - b_dec) @ W + b_enc), fp32
// accumulate, with per-row nonzero counting in the epilogue. Included by encode.hip (entry
// points) and by the encode_*.hip files that instantiate the kernels, one tiling and input
// type each, so they compile in parallel.
//
// Reference semantics: saeflow/kernels/encode.py:36-91 (kernel) and :97-139 (wrapper).
//
// Two launches per call:
//  1. prologue pass: x' = cast_to_W_dtype(fp32(x) - fp32(b_dec)) (encode.py:72) written once to
//     a workspace [M, Kp] (Kp = K rounded up to two K-steps, zero padded). Every x row block is
//     reused by all d_sae/256 column tiles, so forming x' once instead of in every tile's
//     staging removes that VALU work from the MFMA loop entirely.
//  2. the GEMM: 256x256 output tiles, 8 waves of 128x64 (two per SIMD; 4 waves of 128x128 and
//     256x128 tiles are compiled as alternatives), 32x32 MFMA tiles. Whole-tile problems run
//     the persistent form (one workgroup per CU walking its XCD's tiles, the next tile's loads
//     under the epilogue); ragged ones one workgroup per tile.
//     * Operand staging is LDS DMA (buffer_load_dwordx4 ... lds): no VGPR round trip, no VALU.
//       Lane l of a DMA lands at LDS base + 16*l, so the XOR-swizzled LDS layout is produced by
//       choosing which global chunk each lane fetches. Buffer resources give 32-bit offsets
//       and return zeros for rows past M / past K.
//     * A feature-contiguous W (the SAELens layout W_enc[d_in, d_sae] row-major) stays
//       [k][n] in LDS; its MFMA fragments are read with ds_read_b64_tr_b16, which transposes a
//       4(k) x 16(n) block across each 16-lane group. A token-contiguous W ([n][k]) and x' are
//       read with ds_read_b128. All layouts are XOR-swizzled for gfx950's 64-bank LDS so the
//       fragment reads are bank-conflict free.
//     * MFMA operands are swapped (A = W^T block, B = x' block) so each lane's accumulators
//       hold runs of 4 consecutive features of one token: the epilogue converts, counts per
//       token row, stages the wave tile through LDS and writes full 128- or 256-B row
//       segments with 16-B stores.
//     * Tile order is XCD-aware: hardware workgroup id b runs on XCD b % 8, so ids are
//       remapped to give each XCD a contiguous run of tiles, walked in runs of GROUP_N
//       feature tiles (or of GROUP_M token tiles).
#include <algorithm>
#include <atomic>
#include <type_traits>

#ifndef SF_DMA_SPLIT
#define SF_DMA_SPLIT 1
#endif
#ifndef SF_WIDE_WAVES
#define SF_WIDE_WAVES 8
#endif

#include "common.h"

namespace sfenc {

constexpr int BM = 256, BN = 256;        // output tile (tokens x features)
constexpr int NT = 256;                  // threads per workgroup (4 waves)
constexpr int ROWB = 128;                // bytes per K-step of one operand row (BK * esize)
constexpr int TILE = 256 * ROWB;         // one operand tile of one stage: 32 KiB
constexpr int STAGE = 2 * TILE;          // [W tile | x' tile]
constexpr uint32_t RSRC_W3 = 0x00020000; // buffer resource dword 3 for raw loads (gfx9 family)
constexpr uint32_t OOB = 0x40000000u;    // an offset past every buffer range used here
constexpr int XCD_CUS = 32;              // CUs per XCD (MI355X: 256 CUs in 8 XCDs)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <int DT> struct Traits;
template <> struct Traits<SF_BF16> { static constexpr int E = 2, EPC = 8, BK = 64; };
template <> struct Traits<SF_F16> { static constexpr int E = 2, EPC = 8, BK = 64; };
template <> struct Traits<SF_F32> { static constexpr int E = 4, EPC = 4, BK = 32; };

enum WPath { W_NMAJOR = 0, W_KMAJOR = 1, W_GENERIC = 2 };

struct GemmArgs {
  const char* xw;  // x' [M, Kp], W dtype, row stride Kp
  int64_t Kp;
  const char* w;
  int64_t swk, swn;
  const void* b_enc;
  int benc_dt;
  const void* thr;
  int thr_dt;
  void* out;
  int64_t som, son;
  int out_dt;
  int32_t* row_nnz;
  int64_t M, N, K;
  int act;
  // Tile order (gemm_kernel): group_n > 0 walks runs of group_n feature panels token panel by
  // token panel; otherwise runs of group_m token panels, feature panel by feature panel.
  int tiles_m, tiles_n, group_m, group_n;
  int ksteps;  // K-steps the kernel runs: ceil(K / BK) rounded up to its pipeline round (<= Kp / BK)
  int vec_store;  // out rows contiguous, 16-B aligned
  // Row-candidate epilogue (no dense output): row m's kept values are appended, as (column,
  // value in out_dt), to cand_idx / cand_val[m * cap ...]; cand_cnt[m] counts them all, also
  // those past cap. row_floor (optional) keeps only stored values >= row_floor[m].
  int32_t* cand_cnt;
  int32_t* cand_idx;
  char* cand_val;
  int64_t cap;
  const float* row_floor;
  // Gathered-row form (LIVE kernels only): rows i < clamp(*n_live - live_off, 0, M) are live.
  const int32_t* n_live;
  int64_t live_off;
  // Persistent kernels: per-XCD tile counters (int, TILE_CTR_STRIDE apart), zeroed by the
  // prologue pass before the GEMM.
  int32_t* tile_ctr;
};
constexpr int TILE_CTR_STRIDE = 16;     // ints between two XCDs' counters (64 B)
constexpr int64_t TILE_CTR_BYTES = 512;  // the counters' share of the workspace


enum Epi { EPI_DENSE = 0, EPI_ROWS = 1, EPI_ROWS_FLOOR = 2 };

// LDS swizzles, derived for gfx950's LDS: 64 banks x 4 B, i.e. 256 B per clock, so a
// 64-lane read of 16 B per lane is serviced 16 lanes per clock and one of 8 B per lane 32
// lanes per clock; a clock is conflict free when its lanes touch 64 distinct banks.
// Token-contiguous operand rows are 128 B (8 chunks of 16 B). A fragment read puts lanes
// 16i..16i+15 on 16 consecutive rows at one logical chunk: rows of equal parity share a
// 128-B bank half, so the 8 even and the 8 odd rows must each land on 8 distinct chunks.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
// Feature-contiguous 16-bit W rows are 512 B (32 chunks, row stride = 2 x 256 B). The
// transpose reads of lanes 0-31 cover rows kb..kb+3 x logical chunks c..c+3 (c % 4 == 0):
// XOR-ing chunk indices with 4*(k%4) spreads those 16 chunks over all 16 bank positions.
__device__ __forceinline__ int wswz(int k) { return 4 * (k & 3); }
// Feature-contiguous fp32 W rows are 1 KiB; lanes 0-31 and 32-63 read rows k and k+4 at the
// same features, so rows with bit 2 set are shifted by 128 B.
__device__ __forceinline__ int wswz32(int k) { return 8 * ((k >> 2) & 1); }
__device__ __forceinline__ int lds_off(int row, int kc) { return row * ROWB + ((kc ^ swz(row)) << 4); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(uint32_t)bytes, (int)RSRC_W3);
}

// 16 B from global (buffer offset voff + soff) to LDS at wave_base + 16*lane
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* wave_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)wave_base, 16, (int)voff, (int)soff, 0, 0);
}

// s_waitcnt vmcnt(0) (expcnt/lgkmcnt left at their maxima): all DMA into LDS has landed
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int DT>
__device__ __forceinline__ void mfma_chunk(f32x16& acc, const u32x4& a, const u32x4& b) {
  if constexpr (DT == SF_BF16) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  } else if constexpr (DT == SF_F16) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[e]), __uint_as_float(b[e]), acc,
                                                 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ uint32_t to_bits_t(float v) {
  if constexpr (DT == SF_F32) return __float_as_uint(v);
  else if constexpr (DT == SF_BF16) return f32_to_bf16(v);
  else return f32_to_f16(v);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// two fp32 values -> packed 16-bit pair (one v_cvt_pk_{bf16,f16}_f32, round to nearest even)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (DT == SF_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

template <int DT>
__device__ __forceinline__ float chunk_elem(const u32x4& c, int e) {
  if constexpr (DT == SF_F32) return __uint_as_float(c[e]);
  else {
    uint32_t h = (c[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
    return DT == SF_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  }
}

template <int DT>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
  u32x4 r;
  if constexpr (DT == SF_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(v[e]);
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = pack2<DT>(v[2 * d], v[2 * d + 1]);
  }
  return r;
}

// ===================================================================================
// 1. prologue pass: x' = cast(fp32(x) - fp32(b_dec)), zero for k >= K
// ===================================================================================
template <int DT, bool FAST>
__global__ __launch_bounds__(256) void xprep_kernel(const void* x, int64_t sxm, int64_t sxk, int x_dt,
                                                    const void* b_dec, int bdec_dt, int64_t M, int64_t K,
                                                    int64_t Kp, char* xw, int32_t* tile_ctr) {
  constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC;
  // the GEMM that follows on the stream claims tiles from these (persistent form)
  if (blockIdx.x == 0 && threadIdx.x < 8) tile_ctr[threadIdx.x * TILE_CTR_STRIDE] = 0;
  const int64_t cpr = Kp / EPC;  // chunks per row
  const int64_t total = M * cpr;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t m = c / cpr, k0 = (c - m * cpr) * EPC;
    float v[EPC];
    if constexpr (FAST) {  // x and b_dec of the W dtype, rows 16-B aligned, K % EPC == 0
      if (k0 < K) {
        const u32x4 xv = *(const u32x4*)((const char*)x + (m * sxm + k0) * E);
        const u32x4 bv = *(const u32x4*)((const char*)b_dec + k0 * E);
#pragma unroll
        for (int e = 0; e < EPC; ++e) v[e] = chunk_elem<DT>(xv, e) - chunk_elem<DT>(bv, e);
      } else {
#pragma unroll
        for (int e = 0; e < EPC; ++e) v[e] = 0.f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const int64_t k = k0 + e;
        v[e] = k < K ? load_as_f32(x, x_dt, m * sxm + k * sxk) - load_as_f32(b_dec, bdec_dt, k) : 0.f;
      }
    }
    *(u32x4*)(xw + c * 16) = pack_chunk<DT>(v);
  }
}

// Gathered-row prologue (sf_encode_gather): x' row i = cast(fp32(x[rows[row_off + i]]) -
// fp32(b_dec)) for the live rows i < clamp(*n_rows - row_off, 0, M), the same arithmetic as
// xprep_kernel; the rest of the last live 256-row block is zeroed. A row id outside [0, Mx)
// gives a zero row. The grid strides over the live chunks only, so with no live row every
// workgroup returns at once.
template <int DT>
__global__ __launch_bounds__(256) void xprep_rows_kernel(const void* x, int64_t sxm, int64_t sxk, int x_dt,
                                                         int64_t Mx, const int32_t* rows, const int32_t* n_rows,
                                                         int64_t row_off, const void* b_dec, int bdec_dt, int64_t M,
                                                         int64_t K, int64_t Kp, char* xw) {
  constexpr int EPC = Traits<DT>::EPC;
  int64_t live = (int64_t)*n_rows - row_off;
  live = live < 0 ? 0 : (live > M ? M : live);
  const int64_t padded = min(M, (live + BM - 1) / BM * BM);
  const int64_t cpr = Kp / EPC;
  const int64_t total = padded * cpr;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t i = c / cpr, k0 = (c - i * cpr) * EPC;
    int64_t src = i < live ? (int64_t)rows[row_off + i] : -1;
    if (src >= Mx) src = -1;
    float v[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t k = k0 + e;
      v[e] = src >= 0 && k < K ? load_as_f32(x, x_dt, src * sxm + k * sxk) - load_as_f32(b_dec, bdec_dt, k) : 0.f;
    }
    *(u32x4*)(xw + c * 16) = pack_chunk<DT>(v);
  }
}

// ===================================================================================
// 2. the GEMM + epilogue
// ===================================================================================

// Tile (pid_m, pid_n) at position lid of the grouped order. With group_n > 0: runs of group_n
// feature panels (tiles_m * group_n positions each), token panel by token panel, feature panel
// fastest, so the W_enc panels of a run stay in cache while the x' panels stream past them;
// otherwise runs of group_m token panels, feature panel by feature panel, token panel fastest.
// Both are bijections of [0, tiles_m * tiles_n).
// (Returned by value: stores through two reference outputs from the two branches get merged
// into a store through a selected pointer, which puts the tile ids in scratch memory and the
// buffer resources built from them in vector registers.)
struct TilePos {
  int m, n;
};
__device__ __forceinline__ TilePos tile_of(const GemmArgs& a, int lid) {
  // the order's parameters: (runs of g panels along the "major" axis, the other axis length)
  const bool by_n = a.group_n > 0;
  const int g = by_n ? a.group_n : a.group_m;
  const int major = by_n ? a.tiles_n : a.tiles_m, minor = by_n ? a.tiles_m : a.tiles_n;
  const int per_group = g * minor;
  const int first = (lid / per_group) * g;
  const int gs = min(major - first, g);
  const int p_major = first + (lid % per_group) % gs, p_minor = (lid % per_group) / gs;
  return by_n ? TilePos{p_minor, p_major} : TilePos{p_major, p_minor};
}

// Per-thread staging plan of one tile for NW waves: the LDS chunk each of the thread's PER x'
// DMAs and PER W DMAs fills is fixed ((i*NW + wave)*64 + lane); the global chunk it fetches
// follows from the swizzle. Offsets are relative to per-tile / per-K-step buffer bases.
template <int DT, int WP, int NW>
struct Plan {
  static constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC;
  static constexpr int PER = 32 / NW;  // 2048 16-B chunks per operand tile / (64 * NW) threads
  uint32_t xo[PER];
  uint32_t wo[PER];
  int kcw[PER];  // token-contiguous W: logical K-chunk of each W DMA (for the K tail)

  __device__ __forceinline__ void init(const GemmArgs& a, int64_t n0, int w, int lane) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int P = (i * NW + w) * 64 + lane;  // 16-B LDS chunk index within the operand tile
      {
        const int m = P >> 3, kc = (P & 7) ^ swz(m);
        xo[i] = (uint32_t)(m * a.Kp * E + kc * 16);
      }
      if constexpr (WP == W_NMAJOR) {
        // feature-contiguous rows of BN features: 16-bit 32 chunks/row x 64 rows; fp32 64 x 32
        constexpr int CPR = BN * E / 16;
        const int k = P / CPR, pc = P % CPR;
        const int c = pc ^ (DT == SF_F32 ? wswz32(k) : wswz(k));
        const int64_t col = min((int64_t)c * EPC, a.N - EPC - n0);  // past-N columns re-read valid data
        wo[i] = (uint32_t)(k * a.swk * E + col * E);
        kcw[i] = 0;
      } else {
        const int n = P >> 3, kc = (P & 7) ^ swz(n);
        const int64_t nc = min((int64_t)n, a.N - 1 - n0);
        wo[i] = (uint32_t)(nc * a.swn * E + kc * 16);
        kcw[i] = kc;
      }
    }
  }
};

// Issue part `part` (0..3) of K-step kt's DMAs into stage buffer `st` ([W tile | x' tile]):
// this thread's x' and W chunks i = part*PPP .. part*PPP + PPP-1. The four parts of a stage are
// spread over the MFMA groups of the K-step before it, so no wave stalls on a burst of DMA
// issues.
template <int DT, int WP, int NW>
__device__ __forceinline__ void issue_part(const GemmArgs& a, const Plan<DT, WP, NW>& p,
                                           __amdgpu_buffer_rsrc_t xr, int64_t n0, int kt, char* st, int w,
                                           int part) {
  constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC, BK = Traits<DT>::BK;
  constexpr int PPP = Plan<DT, WP, NW>::PER / 4;  // chunks per operand per part
  const int64_t k0 = (int64_t)kt * BK;
  char* ws = st;
  char* xs = st + TILE;
#pragma unroll
  for (int j = 0; j < PPP; ++j) {
    const int i = PPP * part + j;
    dma16(xr, xs + (i * NW + w) * 1024, p.xo[i], (uint32_t)(k0 * E));
  }
  if constexpr (WP == W_NMAJOR) {
    // rows past K (and whole K-steps past K) fall outside the range and read as zero; the
    // range is a scalar select, not a branch, so the DMAs stay in the MFMA schedule
    const int64_t rows = min((int64_t)BK, a.K - k0);
    const int64_t span = (rows - 1) * a.swk * E + (a.N - n0) * E;
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w + (k0 * a.swk + n0) * E, rows > 0 ? span : 0);
#pragma unroll
    for (int j = 0; j < PPP; ++j) {
      const int i = PPP * part + j;
      dma16(wr, ws + (i * NW + w) * 1024, p.wo[i], 0);
    }
  } else {
    const int64_t nrows = min((int64_t)BN, a.N - n0);
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w + n0 * a.swn * E, (nrows - 1) * a.swn * E + a.K * E);
#pragma unroll
    for (int j = 0; j < PPP; ++j) {
      const int i = PPP * part + j;
      const uint32_t vo = k0 + p.kcw[i] * EPC >= a.K ? OOB : p.wo[i];  // K chunks past K read zero
      dma16(wr, ws + (i * NW + w) * 1024, vo, (uint32_t)(k0 * E));
    }
  }
}

// Generic W (any strides / alignment): element-wise loads into registers, then the
// token-contiguous LDS layout; x' still arrives by DMA.
template <int DT, int NTH>
__device__ __forceinline__ void stage_generic_w(const GemmArgs& a, int64_t n0, int kt, char* ws, int t) {
  constexpr int EPC = Traits<DT>::EPC, BK = Traits<DT>::BK;
  const int kc = t & 7;
  const int64_t k = (int64_t)kt * BK + kc * EPC;
#pragma unroll 1
  for (int i = 0; i < 2048 / NTH; ++i) {
    const int nl = (t >> 3) + (NTH / 8) * i;
    const int64_t n = n0 + nl;
    u32x4 c = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t kk = k + e;
      uint32_t bits = 0;
      if (n < a.N && kk < a.K) {
        const int64_t off = kk * a.swk + n * a.swn;
        bits = DT == SF_F32 ? ((const uint32_t*)a.w)[off] : ((const u16*)a.w)[off];
      }
      if constexpr (DT == SF_F32) c[e] = bits;
      else c[e >> 1] |= bits << ((e & 1) * 16);
    }
    *(u32x4*)(ws + lds_off(nl, kc)) = c;
  }
}

// A fragment (W^T rows = features) of k16 step s for feature block nb of the wave whose
// features start at cb0 within the tile.
template <int DT, int WP>
__device__ __forceinline__ u32x4 load_a(const char* ws, int cb0, int nb, int s, int lane) {
  if constexpr (WP == W_NMAJOR && DT != SF_F32) {
    // [k][n] rows of 512 B; ds_read_b64_tr_b16 per 16-lane group g: source lane p points at
    // row kb + p/4, features cb + 4*(p%4); lane p receives features cb + p, rows kb..kb+3.
    const int g = lane >> 4, p = lane & 15;
    const int cb = cb0 + nb * 32 + 16 * (g & 1);
    u32x4 r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kb = s * 16 + 8 * (g >> 1) + 4 * h;
      const int k = kb + (p >> 2);
      const int col = cb + 4 * (p & 3);
      const int off = k * 512 + (((col >> 3) ^ wswz(k)) << 4) + ((col >> 2) & 1) * 8;
      const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(ws + off));
      const u32x2 u = __builtin_bit_cast(u32x2, v);
      r[2 * h] = u[0];
      r[2 * h + 1] = u[1];
    }
    return r;
  } else if constexpr (WP == W_NMAJOR) {
    // fp32 [k][n] rows of 1 KiB: lane supplies W[k][n] for MFMA e, k = (2s + lane/32)*4 + e
    const int n = cb0 + nb * 32 + (lane & 31);
    const int kq = (2 * s + (lane >> 5)) * 4;
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = kq + e;
      r[e] = *(const uint32_t*)(ws + k * 1024 + (((n >> 2) ^ wswz32(k)) << 4) + (n & 3) * 4);
    }
    return r;
  } else {
    return *(const u32x4*)(ws + lds_off(cb0 + nb * 32 + (lane & 31), 2 * s + (lane >> 5)));
  }
}

// Epilogue for output element type ODT: activation + cast + count + LDS-staged store. b_enc is
// already in the accumulators (they start at the bias). s_t[n] folds the activation into one
// threshold per feature: a value is kept unless pre <= s_t[n], with s_t = max(thr, h) for
// jumprelu, h for relu, +inf past N and for a NaN threshold, NaN for the bare pre-activation
// (keeps everything), where h is the largest value that rounds to zero in the output type (0
// for fp32, 2^-126 for bf16 as its denormals are not relied on, 2^-25 for fp16). A NaN
// pre-activation is kept, as relu(NaN) = NaN in the reference. Kept values are exactly the
// nonzeros of the stored tile, so the row count is the number of kept values
// (encode.py:78-91).
// STG: bytes of LDS staging per pass (32 KiB: the 16-bit tile in one pass; the persistent form
// has 16 KiB); FULL: the tile lies inside M x N with aligned rows, so only the unconditional
// store path is compiled (NIT stores per pass).
template <int ODT, int STG = 32768, bool FULL = false>
__device__ __forceinline__ void epilogue(const GemmArgs& a, f32x16 (&acc)[4][4], int64_t m0, int64_t n0, int w,
                                         int lane, const float* s_t, char* reg) {
  constexpr int OES = ODT == SF_F32 ? 4 : 2;
  constexpr int RB = 128 * OES;        // bytes per staged row (128 features)
  constexpr int UPR = RB / 16;         // 16-B units per row
  constexpr int RPI = 64 / UPR;        // rows per 64-lane read
  constexpr int EPU = 16 / OES;        // elements per unit
  constexpr int NP = 128 * RB / STG;   // passes over the wave tile
  constexpr int MPP = 4 / NP;          // 32-token blocks per pass
  constexpr int NIT = MPP * 32 / RPI;  // 16-B row-unit reads per lane per pass
  static_assert(NP >= 1 && 4 % NP == 0 && NIT % 8 == 0, "staging of whole 32-token blocks");
  const int wm = w >> 1, wn = w & 1;
  const bool count = a.row_nnz != nullptr;
  // the wave's tile in range with 16-B aligned rows: branch-free stores in batches
  const bool full = FULL || (a.vec_store && m0 + wm * 128 + 128 <= a.M && n0 + wn * 128 + 128 <= a.N);
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    int cnt[MPP];
#pragma unroll
    for (int mi = 0; mi < MPP; ++mi) cnt[mi] = 0;
    // thresholds of the next (nb, g) group are read one group ahead
    float4 thn = *(const float4*)(s_t + wn * 128 + (lane >> 5) * 4);
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
      const int nb = idx >> 2, g = idx & 3;
      // the 4 features of this lane in group (nb, g)
      const int cl = nb * 32 + g * 8 + (lane >> 5) * 4;
      const float4 th = thn;
      if (idx < 15) {
        const int cn = ((idx + 1) >> 2) * 32 + ((idx + 1) & 3) * 8 + (lane >> 5) * 4;
        thn = *(const float4*)(s_t + wn * 128 + cn);
      }
      const float thv[4] = {th.x, th.y, th.z, th.w};
      const int unit = (cl * OES) >> 4;
#pragma unroll
      for (int mi = 0; mi < MPP; ++mi) {
        const int mb = pass * MPP + mi;
        const int rl = mi * 32 + (lane & 31);  // staged row
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pre = acc[nb][mb][g * 4 + r];
          const bool keep = !(pre <= thv[r]);
          o[r] = keep ? pre : 0.f;
          cnt[mi] += keep ? 1 : 0;
        }
        // materialise the count here: left to itself the compiler sinks it past the store
        // phase and keeps every 64-bit compare mask alive in the meantime
        asm volatile("" : "+v"(cnt[mi]));
        char* dst = reg + rl * RB + ((unit ^ (rl & 15)) << 4);
        if constexpr (OES == 2) {
          *(u32x2*)(dst + ((cl >> 2) & 1) * 8) = u32x2{pack2<ODT>(o[0], o[1]), pack2<ODT>(o[2], o[3])};
        } else {
          *(float4*)dst = float4{o[0], o[1], o[2], o[3]};
        }
      }
    }
    if (count) {
      // Columns past N (threshold +inf) are never stored but a NaN there would pass the keep
      // test: drop such counts in the waves that reach past N (NaN inputs only).
      if (!FULL && n0 + wn * 128 + 128 > a.N) {
#pragma unroll
        for (int idx = 0; idx < 16; ++idx)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + wn * 128 + (idx >> 2) * 32 + (idx & 3) * 8 + (lane >> 5) * 4 + r;
#pragma unroll
            for (int mi = 0; mi < MPP; ++mi) {
              const float pre = acc[idx >> 2][pass * MPP + mi][(idx & 3) * 4 + r];
              cnt[mi] -= (n >= a.N && pre != pre) ? 1 : 0;
            }
          }
      }
#pragma unroll
      for (int mi = 0; mi < MPP; ++mi) {
        const int64_t m = m0 + wm * 128 + (pass * MPP + mi) * 32 + (lane & 31);
        const int c = cnt[mi] + __shfl_xor(cnt[mi], 32);
        if (lane < 32 && (FULL || m < a.M) && c > 0) atomicAdd(a.row_nnz + m, c);
      }
    }
    // the staged rows are this wave's own: LDS executes a wave's accesses in order
    __builtin_amdgcn_wave_barrier();
    // read back MPP*32 rows x 128 features of this wave and store whole row segments
    if (full) {
      const int u = lane % UPR;
      char* base = (char*)a.out +
                   ((m0 + wm * 128 + pass * MPP * 32 + lane / UPR) * a.som + n0 + wn * 128 + u * EPU) * OES;
      const int64_t step = (int64_t)RPI * a.som * OES;
#pragma unroll
      for (int it0 = 0; it0 < NIT; it0 += 8) {
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int rl = (it0 + j) * RPI + lane / UPR;
          v[j] = *(const u32x4*)(reg + rl * RB + ((u ^ (rl & 15)) << 4));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) __builtin_nontemporal_store(v[j], (u32x4*)(base + (it0 + j) * step));
      }
    } else if constexpr (!FULL) {
#pragma unroll 4
      for (int it = 0; it < NIT; ++it) {
        const int rl = it * RPI + lane / UPR, u = lane % UPR;
        const u32x4 v = *(const u32x4*)(reg + rl * RB + ((u ^ (rl & 15)) << 4));
        const int64_t m = m0 + wm * 128 + pass * MPP * 32 + rl;
        const int64_t n = n0 + wn * 128 + u * EPU;
        if (m < a.M) {
          char* orow = (char*)a.out + m * a.som * OES;
          if (a.vec_store && n + EPU <= a.N) {
            __builtin_nontemporal_store(v, (u32x4*)(orow + n * OES));
          } else {
#pragma unroll
            for (int e = 0; e < EPU; ++e) {
              if (n + e < a.N) {
                if constexpr (OES == 2)
                  *(u16*)(orow + (n + e) * a.son * 2) = (u16)((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
                else
                  *(uint32_t*)(orow + (n + e) * a.son * 4) = v[e];
              }
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Workgroup barrier without __syncthreads()'s release fence: that fence waits for every
// outstanding vector-memory operation, including the LDS DMA of stages still in flight.
// Ordering is kept explicitly instead: before arriving, each thread waits (vmcnt) for its own
// DMAs of the stage about to be read and (lgkmcnt) for its own LDS reads of the stage that the
// next DMA overwrites. The signal fences only stop the compiler from moving memory accesses
// across the barrier.
__device__ __forceinline__ void barrier_no_fence() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// s_waitcnt lgkmcnt(0) (vmcnt/expcnt at their maxima): this thread's LDS writes have landed
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// The value as stored in output type ODT (round to nearest even), back in fp32.
template <int ODT>
__device__ __forceinline__ float stored_value(float v) {
  if constexpr (ODT == SF_F32) return v;
  else {
    const uint32_t p = pack2<ODT>(v, 0.f) & 0xffffu;
    return ODT == SF_BF16 ? bf16_to_f32(p) : f16_to_f32(p);
  }
}

// Smallest fp32 x whose value stored in ODT (round to nearest even) is >= F: with hi the
// smallest ODT value >= F, the midpoint below hi when hi's last mantissa bit is even (the tie
// rounds up to hi), just above it when odd. Floors <= 0 (or NaN) filter nothing here: every
// kept value is positive.
template <int ODT>
__device__ __forceinline__ float floor_lo(float F) {
  if (!(F > 0.f)) return -__builtin_inff();
  if constexpr (ODT == SF_F32) return F;
  else {
    uint32_t b = pack2<ODT>(F, 0.f) & 0xffffu;
    if ((ODT == SF_BF16 ? bf16_to_f32(b) : f16_to_f32(b)) < F) ++b;  // round F up to an ODT value
    const float hi = ODT == SF_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
    const float lo = ODT == SF_BF16 ? bf16_to_f32(b - 1) : f16_to_f32(b - 1);
    const float mid = 0.5f * (lo + hi);  // exact in fp32
    return (b & 1u) ? __uint_as_float(__float_as_uint(mid) + 1u) : mid;  // mid > 0: next float up
  }
}

// Row-candidate epilogue of a 128x128 wave tile: instead of storing the tile, each token row's
// kept values (the nonzeros the dense epilogue would store; with FLOOR only those whose
// stored value is >= row_floor[m], and NaNs, which rank above every value) are appended to the row's candidate list. Lanes l and l+32
// hold the same token, so one returning atomic per token row per wave reserves the slots.
// Slots past cap are counted but not written: the caller sees cand_cnt[m] > cap. mid() runs
// once the slots are reserved (the atomics have returned) and before the stores.
template <int ODT, bool FLOOR, int NBK, typename Mid>
__device__ __forceinline__ void epilogue_rows(const GemmArgs& a, f32x16 (&acc)[NBK][4], int64_t m0, int64_t n0,
                                              int wm, int wn, int lane, const float* s_t, Mid&& mid) {
  constexpr int OES = ODT == SF_F32 ? 4 : 2;
  constexpr int WNC = NBK * 32;    // features per wave
  constexpr int NG = NBK * 4;      // 8-feature groups per wave tile row
  constexpr int NW32 = NG / 8;     // 32-bit mask words per token block (4 bits per group)
  uint32_t km[4][NW32];  // keep masks per 32-token block: bit (nb*4 + g)*4 + r
  float fl[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int64_t m = m0 + wm * 128 + mb * 32 + (lane & 31);
    fl[mb] = FLOOR && m < a.M ? floor_lo<ODT>(a.row_floor[m]) : -__builtin_inff();
#pragma unroll
    for (int q = 0; q < NW32; ++q) km[mb][q] = 0;
  }
#pragma unroll
  for (int idx = 0; idx < NG; ++idx) {
    const int nb = idx >> 2, g = idx & 3;
    const float4 th = *(const float4*)(s_t + wn * WNC + nb * 32 + g * 8 + (lane >> 5) * 4);
    const float thv[4] = {th.x, th.y, th.z, th.w};
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pre = acc[nb][mb][g * 4 + r];
        bool keep = !(pre <= thv[r]);
        if constexpr (FLOOR) keep = keep && !(pre < fl[mb]);  // a NaN stays a candidate
        const int bit = (idx & 7) * 4 + r;
        km[mb][idx >> 3] |= keep ? (1u << bit) : 0u;
      }
  }
  // Only rows < M and columns < N exist: padded rows compute bias-only values and padded
  // columns (thresholds +inf) could still pass as NaN, so both are masked out here.
  uint32_t colok[NW32];
#pragma unroll
  for (int q = 0; q < NW32; ++q) colok[q] = 0;
#pragma unroll
  for (int idx = 0; idx < NG; ++idx)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = n0 + wn * WNC + (idx >> 2) * 32 + (idx & 3) * 8 + (lane >> 5) * 4 + r;
      colok[idx >> 3] |= n < a.N ? (1u << ((idx & 7) * 4 + r)) : 0u;
    }
  int cnt[4], old[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const bool rowok = m0 + wm * 128 + mb * 32 + (lane & 31) < a.M;
    cnt[mb] = 0;
#pragma unroll
    for (int q = 0; q < NW32; ++q) {
      km[mb][q] = rowok ? km[mb][q] & colok[q] : 0u;
      cnt[mb] += __popc(km[mb][q]);
    }
    const int tot = cnt[mb] + __shfl_xor(cnt[mb], 32);
    const int64_t m = m0 + wm * 128 + mb * 32 + (lane & 31);
    old[mb] = 0;
    if (lane < 32 && m < a.M && tot > 0) old[mb] = atomicAdd(a.cand_cnt + m, tot);
  }
  int jr[4];  // this lane's first slot in each token block's row
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int o = __shfl(old[mb], lane & 31), c = __shfl(cnt[mb], lane & 31);
    jr[mb] = o + (lane >= 32 ? c : 0);
    asm volatile("" : "+v"(jr[mb])::"memory");  // the atomics are awaited before mid()
  }
  mid();
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int64_t m = m0 + wm * 128 + mb * 32 + (lane & 31);
    int64_t j = jr[mb];
    int32_t* idx_row = a.cand_idx + m * a.cap;
    char* val_row = a.cand_val + m * a.cap * OES;
#pragma unroll
    for (int idx = 0; idx < NG; ++idx) {
      const int nb = idx >> 2, g = idx & 3;
      const uint32_t nib = (km[mb][idx >> 3] >> ((idx & 7) * 4)) & 15u;
      if (__ballot(nib != 0) == 0) continue;  // wave-uniform: most groups hold nothing
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (nib & (1u << r)) {
          if (j < a.cap) {
            idx_row[j] = (int32_t)(n0 + wn * WNC + nb * 32 + g * 8 + (lane >> 5) * 4 + r);
            const float v = stored_value<ODT>(acc[nb][mb][g * 4 + r]);
            if constexpr (OES == 4) *(float*)(val_row + j * 4) = v;
            else *(u16*)(val_row + j * 2) = (u16)(pack2<ODT>(v, 0.f) & 0xffffu);
          }
          ++j;
        }
      }
    }
  }
}

// Helpers of the 256x128 tiling (and the 128x64-per-wave epilogue shared with the 8-wave 256x256).
namespace t2 {
constexpr int BM = 256, BN = 128;
constexpr int XROWB = 64;            // bytes of one x' row per K-step
constexpr int XT = BM * XROWB;       // 16 KiB x' tile
constexpr int WT = 8192;             // 8 KiB W tile ([k][128] rows or [128][64 B])
template <int DT> struct Tr;
template <> struct Tr<SF_BF16> { static constexpr int E = 2, EPC = 8, BK = 32; };
template <> struct Tr<SF_F16> { static constexpr int E = 2, EPC = 8, BK = 32; };
template <> struct Tr<SF_F32> { static constexpr int E = 4, EPC = 4, BK = 16; };

// 64-B rows of 4 chunks: a fragment read puts 16 consecutive rows on one logical chunk;
// rows r, r+4, r+8, r+12 share a bank window and get distinct chunks.
__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int off(int row, int kc) { return row * XROWB + ((kc ^ swz(row)) << 4); }
// feature-contiguous 16-bit W rows are 256 B (16 chunks): the transpose reads of lanes 0-31
// cover rows kb..kb+3 x chunks c..c+3, spread over all 16 bank positions by 4*(k%4).
__device__ __forceinline__ int wswz(int k) { return 4 * (k & 3); }
// fp32 W rows are 512 B: rows k and k+4 are read together, so bit 2 of k shifts by 128 B.
__device__ __forceinline__ int wswz32(int k) { return 8 * ((k >> 2) & 1); }

template <int DT, int WP>
struct Plan2 {
  static constexpr int E = Tr<DT>::E, EPC = Tr<DT>::EPC;
  uint32_t xo[4], wo[2];
  int kcw[2];
  __device__ __forceinline__ void init(const GemmArgs& a, int64_t n0, int w, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int P = (i * 4 + w) * 64 + lane;
      const int m = P >> 2, kc = (P & 3) ^ swz(m);
      xo[i] = (uint32_t)(m * a.Kp * E + kc * 16);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int P = (i * 4 + w) * 64 + lane;
      if constexpr (WP == W_NMAJOR) {
        constexpr int CPR = BN * E / 16;  // 16 (16-bit) or 32 (fp32) chunks per row
        const int k = P / CPR, pc = P % CPR;
        const int c = pc ^ (DT == SF_F32 ? wswz32(k) : wswz(k));
        const int64_t col = min((int64_t)c * EPC, a.N - EPC - n0);
        wo[i] = (uint32_t)(k * a.swk * E + col * E);
        kcw[i] = 0;
      } else {
        const int n = P >> 2, kc = (P & 3) ^ swz(n);
        const int64_t nc = min((int64_t)n, a.N - 1 - n0);
        wo[i] = (uint32_t)(nc * a.swn * E + kc * 16);
        kcw[i] = kc;
      }
    }
  }
};

// DMA j (0..5) of K-step kt: j < 4 the x' chunks, j >= 4 the W chunks of this thread's plan.
// Ranges are scalar selects, not branches, so the DMAs stay in the MFMA schedule.
template <int DT, int WP>
__device__ __forceinline__ void issue2_one(const GemmArgs& a, const Plan2<DT, WP>& p, __amdgpu_buffer_rsrc_t xr,
                                           int64_t n0, int kt, char* ws, char* xs, int w, int j) {
  constexpr int E = Tr<DT>::E, EPC = Tr<DT>::EPC, BK = Tr<DT>::BK;
  const int64_t k0 = (int64_t)kt * BK;
  if (j < 4) {
    dma16(xr, xs + (j * 4 + w) * 1024, p.xo[j], (uint32_t)(k0 * E));
    return;
  }
  const int i = j - 4;
  if constexpr (WP == W_NMAJOR) {
    const int64_t rows = min((int64_t)BK, a.K - k0);
    const int64_t span = (rows - 1) * a.swk * E + (a.N - n0) * E;
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w + (k0 * a.swk + n0) * E, rows > 0 ? span : 0);
    dma16(wr, ws + (i * 4 + w) * 1024, p.wo[i], 0);
  } else {
    const int64_t nrows = min((int64_t)BN, a.N - n0);
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w + n0 * a.swn * E, (nrows - 1) * a.swn * E + a.K * E);
    const uint32_t vo = k0 + p.kcw[i] * EPC >= a.K ? OOB : p.wo[i];  // K chunks past K read zero
    dma16(wr, ws + (i * 4 + w) * 1024, vo, (uint32_t)(k0 * E));
  }
}

template <int DT>
__device__ __forceinline__ void stage_generic_w2(const GemmArgs& a, int64_t n0, int kt, char* ws, int t) {
  constexpr int EPC = Tr<DT>::EPC, BK = Tr<DT>::BK;
#pragma unroll 1
  for (int i = 0; i < 2; ++i) {
    const int q = t + 256 * i;
    const int nl = q >> 2, kc = q & 3;
    const int64_t n = n0 + nl, k = (int64_t)kt * BK + kc * EPC;
    u32x4 c = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t kk = k + e;
      uint32_t bits = 0;
      if (n < a.N && kk < a.K) {
        const int64_t o = kk * a.swk + n * a.swn;
        bits = DT == SF_F32 ? ((const uint32_t*)a.w)[o] : ((const u16*)a.w)[o];
      }
      if constexpr (DT == SF_F32) c[e] = bits;
      else c[e >> 1] |= bits << ((e & 1) * 16);
    }
    *(u32x4*)(ws + off(nl, kc)) = c;
  }
}

template <int DT, int WP>
__device__ __forceinline__ u32x4 load_a2(const char* ws, int wn, int nb, int s, int lane) {
  if constexpr (WP == W_NMAJOR && DT != SF_F32) {
    const int g = lane >> 4, p = lane & 15;
    const int cb = wn * 64 + nb * 32 + 16 * (g & 1);
    u32x4 r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = s * 16 + 8 * (g >> 1) + 4 * h + (p >> 2);
      const int col = cb + 4 * (p & 3);
      const int o = k * 256 + (((col >> 3) ^ wswz(k)) << 4) + ((col >> 2) & 1) * 8;
      const u32x2 u = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(ws + o)));
      r[2 * h] = u[0];
      r[2 * h + 1] = u[1];
    }
    return r;
  } else if constexpr (WP == W_NMAJOR) {
    const int n = wn * 64 + nb * 32 + (lane & 31);
    const int kq = (2 * s + (lane >> 5)) * 4;
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = kq + e;
      r[e] = *(const uint32_t*)(ws + k * 512 + (((n >> 2) ^ wswz32(k)) << 4) + (n & 3) * 4);
    }
    return r;
  } else {
    return *(const u32x4*)(ws + off(wn * 64 + nb * 32 + (lane & 31), 2 * s + (lane >> 5)));
  }
}

// Epilogue of a wave's 128 x 64 tile (token block wm, feature block wn of the workgroup
// tile), staged through an STG-byte LDS region per pass (the 256x128 tiling and the
// persistent 256x256 form have 8 KiB per wave, the 8-wave 256x256 tiling 16 KiB: its whole
// 16-bit tile in one pass, 16 stores in flight); s_t holds the tile's thresholds. FULL: the
// tile lies inside M x N and the output rows are 16-B aligned, so only the unconditional store
// path is compiled (NIT stores per pass, always).
template <int ODT, int STG = 8192, bool FULL = false>
__device__ __forceinline__ void epilogue2(const GemmArgs& a, f32x16 (&acc)[2][4], int64_t m0, int64_t n0, int wm,
                                          int wn, int lane, const float* s_t, char* reg) {
  constexpr int OES = ODT == SF_F32 ? 4 : 2;
  constexpr int RB = 64 * OES;          // staged row: 64 features
  constexpr int UPR = RB / 16;          // 8 (16-bit) or 16 (fp32) units per row
  constexpr int RPI = 64 / UPR;         // rows per 64-lane read
  constexpr int EPU = 16 / OES;
  constexpr int MPP = STG / (32 * RB);  // 32-token blocks per pass
  constexpr int NP = 4 / MPP;
  constexpr int NIT = MPP * 32 / RPI;  // 16-B row-unit reads per lane per pass (8)
  const bool count = a.row_nnz != nullptr;
  const bool full = FULL || (a.vec_store && m0 + wm * 128 + 128 <= a.M && n0 + wn * 64 + 64 <= a.N);
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    int cnt[MPP];
#pragma unroll
    for (int mi = 0; mi < MPP; ++mi) cnt[mi] = 0;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = nb * 32 + g * 8 + (lane >> 5) * 4;  // feature within the wave tile
        const float4 th = *(const float4*)(s_t + wn * 64 + cl);
        const float thv[4] = {th.x, th.y, th.z, th.w};
        const int unit = (cl * OES) >> 4;
#pragma unroll
        for (int mi = 0; mi < MPP; ++mi) {
          const int mb = pass * MPP + mi;
          const int rl = mi * 32 + (lane & 31);
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pre = acc[nb][mb][g * 4 + r];  // b_enc is in the accumulators
            const bool keep = !(pre <= thv[r]);
            o[r] = keep ? pre : 0.f;
            cnt[mi] += keep ? 1 : 0;
          }
          asm volatile("" : "+v"(cnt[mi]));  // keep the count from sinking
          char* dst = reg + rl * RB + ((unit ^ (rl & (UPR - 1))) << 4);
          if constexpr (OES == 2)
            *(u32x2*)(dst + ((cl >> 2) & 1) * 8) = u32x2{pack2<ODT>(o[0], o[1]), pack2<ODT>(o[2], o[3])};
          else
            *(float4*)dst = float4{o[0], o[1], o[2], o[3]};
        }
      }
    }
    if (count) {
      if (!FULL && n0 + wn * 64 + 64 > a.N) {  // NaN in columns past N: see the 256x256 epilogue
#pragma unroll
        for (int idx = 0; idx < 8; ++idx)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + wn * 64 + (idx >> 2) * 32 + (idx & 3) * 8 + (lane >> 5) * 4 + r;
#pragma unroll
            for (int mi = 0; mi < MPP; ++mi) {
              const float pre = acc[idx >> 2][pass * MPP + mi][(idx & 3) * 4 + r];
              cnt[mi] -= (n >= a.N && pre != pre) ? 1 : 0;
            }
          }
      }
#pragma unroll
      for (int mi = 0; mi < MPP; ++mi) {
        const int64_t m = m0 + wm * 128 + (pass * MPP + mi) * 32 + (lane & 31);
        const int c = cnt[mi] + __shfl_xor(cnt[mi], 32);
        if (lane < 32 && (FULL || m < a.M) && c > 0) atomicAdd(a.row_nnz + m, c);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the staged rows are this wave's own (in-order LDS)
    if (full) {
      const int u = lane % UPR;
      char* base = (char*)a.out +
                   ((m0 + wm * 128 + pass * MPP * 32 + lane / UPR) * a.som + n0 + wn * 64 + u * EPU) * OES;
      const int64_t step = (int64_t)RPI * a.som * OES;
      u32x4 v[NIT];
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int rl = it * RPI + lane / UPR;
        v[it] = *(const u32x4*)(reg + rl * RB + ((u ^ (rl & (UPR - 1))) << 4));
      }
#pragma unroll
      for (int it = 0; it < NIT; ++it) __builtin_nontemporal_store(v[it], (u32x4*)(base + it * step));
    } else if constexpr (!FULL)
#pragma unroll 4
    for (int it = 0; it < NIT; ++it) {
      const int rl = it * RPI + lane / UPR, u = lane % UPR;
      const u32x4 v = *(const u32x4*)(reg + rl * RB + ((u ^ (rl & (UPR - 1))) << 4));
      const int64_t m = m0 + wm * 128 + pass * MPP * 32 + rl;
      const int64_t n = n0 + wn * 64 + u * EPU;
      if (m < a.M) {
        char* orow = (char*)a.out + m * a.som * OES;
        if (a.vec_store && n + EPU <= a.N) {
          __builtin_nontemporal_store(v, (u32x4*)(orow + n * OES));
        } else {
#pragma unroll
          for (int e = 0; e < EPU; ++e) {
            if (n + e < a.N) {
              if constexpr (OES == 2)
                *(u16*)(orow + (n + e) * a.son * 2) = (u16)((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
              else
                *(uint32_t*)(orow + (n + e) * a.son * 4) = v[e];
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}
}  // namespace t2

// NW = 4 waves of 128x128 (one wave per SIMD, 256 accumulators each) or 8 waves of 128x64
// (two per SIMD, 128 accumulators each, so one wave's LDS / DMA waits run under the other's
// MFMAs).
//
// LIVE: the gathered-row form behind sf_encode_gather. Only the first live = clamp(*n_live -
// live_off, 0, M) rows are wanted, a count that lives on the device, so the grid is one
// workgroup per CU and each workgroup walks the tiles of the row blocks that hold live rows
// (row-major), exiting at once when there are none. Tiles run the same K-steps in the same
// order as the one-tile-per-workgroup form, so results are bit-identical to it.
template <int DT, int WP, int OES, int NW, int EPI = EPI_DENSE, bool LIVE = false>
__global__ __launch_bounds__(NW * 64, 1) void gemm_kernel(GemmArgs a) {
  constexpr int E = Traits<DT>::E, BK = Traits<DT>::BK;
  constexpr int NTH = NW * 64;
  constexpr int WCOLS = NW / 2;          // waves across the 256 features
  constexpr int WNC = BN / WCOLS;        // features per wave: 128 or 64
  constexpr int NBK = WNC / 32;          // 32-feature MFMA blocks per wave: 4 or 2
  constexpr int LWP = WP == W_GENERIC ? W_KMAJOR : WP;  // LDS layout of the W tile
  // Two stage buffers as distinct LDS objects: the compiler's wait-count pass can then tell
  // the DMA into one stage from the fragment reads of the other and keeps them overlapped.
  __shared__ __attribute__((aligned(1024))) char lds0[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds1[STAGE];
  __shared__ __attribute__((aligned(16))) float s_benc[BN];
  __shared__ __attribute__((aligned(16))) float s_thr[BN];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w / WCOLS, wn = w % WCOLS;

  // XCD-aware remap: hardware id b runs on XCD b % 8; give each XCD a contiguous range.
  const int total = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = b % 8, loc = b / 8;
  int live_tiles = 0;
  if constexpr (LIVE) {
    int64_t live = (int64_t)*a.n_live - a.live_off;
    live = live < 0 ? 0 : (live > a.M ? a.M : live);
    live_tiles = (int)((live + BM - 1) / BM) * a.tiles_n;
    if (b >= live_tiles) return;
  }
  for (int it = b;;) {
    int lid, pid_m, pid_n;
    if constexpr (LIVE) {
      lid = it;
      pid_m = it / a.tiles_n;
      pid_n = it % a.tiles_n;
    } else {
      lid = xcd * per + min(xcd, rem) + loc;
      const TilePos tp = tile_of(a, lid);
      pid_m = tp.m;
      pid_n = tp.n;
    }
    const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

    f32x16 acc[NBK][4];

    const __amdgpu_buffer_rsrc_t xr = rsrc(a.xw + m0 * a.Kp * E, min((int64_t)BM, a.M - m0) * a.Kp * E);
    Plan<DT, LWP, NW> plan;
    plan.init(a, n0, w, lane);
    const int KT = a.ksteps;  // even (whole pipeline rounds); x' is zero up to Kp, W reads zero past K

    // DMA part `part` of K-step kt into `st`; a generic W is staged whole with part 0.
    auto stage_part = [&](int kt, char* st, int part) {
      if constexpr (WP == W_GENERIC) {
        if (part == 0) {
#pragma unroll
          for (int i = 0; i < Plan<DT, LWP, NW>::PER; ++i)
            dma16(xr, st + TILE + (i * NW + w) * 1024, plan.xo[i], (uint32_t)((int64_t)kt * BK * E));
          stage_generic_w<DT, NTH>(a, n0, kt, st, t);
        }
      } else {
        issue_part<DT, WP, NW>(a, plan, xr, n0, kt, st, w, part);
      }
    };

    // Fragments of one k16 step (x' rows and W^T rows), double-buffered in registers.
    struct Frag {
      u32x4 a[NBK], b[4];
    };
    auto load_frag = [&](Frag& f, const char* cur, int s) {
      const char* ws = cur;         // W tile
      const char* xs = cur + TILE;  // x' tile
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        f.b[mb] = *(const u32x4*)(xs + lds_off(wm * 128 + mb * 32 + (lane & 31), 2 * s + (lane >> 5)));
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb) f.a[nb] = load_a<DT, LWP>(ws, wn * WNC, nb, s, lane);
    };
    auto mma = [&](const Frag& f) {
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) mfma_chunk<DT>(acc[nb][mb], f.a[nb], f.b[mb]);
    };
    // Schedule of one group: its MFMAs one by one, the next k16 step's fragment reads and
    // NV DMA issues spread evenly between them.
    constexpr int NMF = NBK * 4 * (DT == SF_F32 ? 4 : 1);  // MFMA instructions per k16 step
    constexpr int NRD = 4 + NBK * (LWP == W_NMAJOR ? (DT == SF_F32 ? 4 : 2) : 1);  // LDS reads per step
    constexpr int DPP = 2 * Plan<DT, LWP, NW>::PER / 4;  // DMA instructions per part
    auto interleave = [&](auto nv_tag) {
      constexpr int NV = decltype(nv_tag)::value;
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // MFMA
        if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // DS read
        if (NV > 0 && i % (NMF / (NV > 0 ? NV : 1)) == 0 && i / (NMF / (NV > 0 ? NV : 1)) < NV)
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                 // VMEM (LDS DMA)
      }
    };
    // DMA parts of the next stage issued in each of a region's four MFMA groups
    constexpr int NP0 = SF_DMA_SPLIT == 0 ? 1 : (SF_DMA_SPLIT == 1 ? 2 : 4);
    constexpr int NP1 = SF_DMA_SPLIT == 0 ? 1 : (SF_DMA_SPLIT == 1 ? 2 : 0);
    constexpr int NP2 = SF_DMA_SPLIT == 0 ? 1 : 0;
    constexpr int NP3 = SF_DMA_SPLIT == 0 ? 1 : 0;
    using I0 = std::integral_constant<int, 0>;

    // One K-step region between barriers. On entry F1 holds the previous step's last k16
    // chunk: group 0 reads chunk 0 of `cur` and multiplies that chunk, groups 1-3 read chunk g
    // and multiply chunk g-1. The DMA of step kt+1 into `nxt` (free since the barrier) rides
    // along. kind: 0 = first region (nothing to multiply in group 0), 1 = middle, 2 = last (no
    // next step to stage).
    Frag F0, F1;
    auto region = [&](auto kind_tag, const char* cur, char* nxt, int kt) {
      constexpr int KIND = decltype(kind_tag)::value;
      constexpr int S = KIND == 2 ? 0 : 1;
      load_frag(F0, cur, 0);
#pragma unroll
      for (int q = 0; q < NP0 * S; ++q) stage_part(kt + 1, nxt, q);
      if constexpr (KIND != 0) mma(F1);
      interleave(std::integral_constant<int, KIND == 0 ? 0 : DPP * NP0 * S>{});
      load_frag(F1, cur, 1);
#pragma unroll
      for (int q = 0; q < NP1 * S; ++q) stage_part(kt + 1, nxt, NP0 + q);
      mma(F0);
      interleave(std::integral_constant<int, DPP * NP1 * S>{});
      load_frag(F0, cur, 2);
#pragma unroll
      for (int q = 0; q < NP2 * S; ++q) stage_part(kt + 1, nxt, NP0 + NP1 + q);
      mma(F1);
      interleave(std::integral_constant<int, DPP * NP2 * S>{});
      load_frag(F1, cur, 3);
#pragma unroll
      for (int q = 0; q < NP3 * S; ++q) stage_part(kt + 1, nxt, NP0 + NP1 + NP2 + q);
      mma(F0);
      interleave(std::integral_constant<int, DPP * NP3 * S>{});
      wait_vmcnt0();
      __syncthreads();
    };

#pragma unroll
    for (int q = 0; q < 4; ++q) stage_part(0, lds0, q);
    // bias and effective keep-threshold of this tile's features (fp32 in LDS): their raw bits
    // are loaded beside the stage-0 DMA and awaited with it, one memory latency for both
    uint32_t rb = 0, rt = 0;
    if (t < BN && n0 + t < a.N) {
      rb = load_bits(a.b_enc, a.benc_dt, n0 + t);
      if (a.act == SF_ACT_JUMPRELU) rt = load_bits(a.thr, a.thr_dt, n0 + t);
    }
    wait_vmcnt0();
    if (t < BN) {
      const int64_t n = n0 + t;
      const float h = a.out_dt == SF_F32 ? 0.f : (a.out_dt == SF_BF16 ? __uint_as_float(0x00800000u)  // 2^-126
                                                                      : __uint_as_float(0x33000000u)); // 2^-25
      float tv = a.act == SF_ACT_NONE ? __builtin_nanf("") : h;
      if (n >= a.N) {
        tv = __builtin_inff();
      } else if (a.act == SF_ACT_JUMPRELU) {
        const float th = bits_as_f32(rt, a.thr_dt);
        tv = th != th ? __builtin_inff() : fmaxf(th, h);  // a NaN threshold keeps nothing
      }
      s_benc[t] = n < a.N ? bits_as_f32(rb, a.benc_dt) : 0.f;
      s_thr[t] = tv;
    }
    // the accumulators start at b_enc (the epilogue's bias add, folded in)
    wait_lgkmcnt0();
    barrier_no_fence();
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 be = *(const float4*)(s_benc + wn * WNC + nb * 32 + g * 8 + (lane >> 5) * 4);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          acc[nb][mb][g * 4 + 0] = be.x;
          acc[nb][mb][g * 4 + 1] = be.y;
          acc[nb][mb][g * 4 + 2] = be.z;
          acc[nb][mb][g * 4 + 3] = be.w;
        }
      }
    wait_vmcnt0();
    __syncthreads();
    region(I0{}, lds0, lds1, 0);
    int kt = 1;
    for (; kt + 1 < KT; kt += 2) {
      region(std::integral_constant<int, 1>{}, lds1, lds0, kt);
      region(std::integral_constant<int, 1>{}, lds0, lds1, kt + 1);
    }
    region(std::integral_constant<int, 2>{}, lds1, lds0, kt);  // KT is even: the last step is in lds1
    mma(F1);
    // The W panel of the tile this XCD starts next, when it differs from this tile's, is new
    // to its L2: one load per 128-B line of its first K-step and of its b_enc and threshold
    // slices, issued before the epilogue, so the next workgroup's stage-0 DMA and bias loads
    // find the lines in L2 (1-1.5% at C3 in the token-run order; in the feature-run order the
    // next tile mostly shares the panel, and loading its x' lines instead measured no gain).
    // Workgroups start in id order, one per CU, so on an XCD of XCD_CUS CUs the tile after
    // this one is lid + XCD_CUS; another one starting instead only makes the loads useless.
    uint32_t pf = 0;
    if constexpr (WP == W_NMAJOR && NW == 8 && E == 2 && EPI == EPI_DENSE && !LIVE) {
      const int nlid = lid + XCD_CUS;
      const int xend = xcd * per + min(xcd, rem) + per + (xcd < rem ? 1 : 0);  // end of this XCD's range
      const int npn = nlid < xend ? tile_of(a, nlid).n : pid_n;
      if (npn != pid_n && t < BK * (BN * E / 128) + 16) {
        if (t < BK * (BN * E / 128)) {
          const int64_t k = t / (BN * E / 128);
          const int64_t n = (int64_t)npn * BN + (t % (BN * E / 128)) * (128 / E);
          if (k < a.K && n < a.N) pf = *(const uint32_t*)(a.w + (k * a.swk + n) * E);
        } else {
          const int q = t - BK * (BN * E / 128);  // lines of b_enc (q < 8), of the threshold (q >= 8)
          const bool is_b = q < 8;
          const int dt = is_b ? a.benc_dt : a.thr_dt;
          const int esz = sf_dtype_size(dt);
          const int64_t n = (int64_t)npn * BN + (q & 7) * (128 / esz);
          if ((q & 7) * 128 < BN * esz && n < a.N && (is_b || a.act == SF_ACT_JUMPRELU)) {
            const char* p = (const char*)(is_b ? a.b_enc : a.thr) + n * esz;
            pf = esz == 4 ? *(const uint32_t*)p : (uint32_t)*(const u16*)p;
          }
        }
      }
    }

    // one epilogue body per output width keeps the kernel free of register spills
    if constexpr (EPI != EPI_DENSE) {
      // row-candidate kernels are instantiated per output type: OES carries the sf_dtype code
      epilogue_rows<OES, EPI == EPI_ROWS_FLOOR, NBK>(a, acc, m0, n0, wm, wn, lane, s_thr, [] {});
    } else if constexpr (NW == 4) {
      char* ereg = w < 2 ? lds0 + w * 32768 : lds1 + (w - 2) * 32768;  // this wave's 32 KiB
      if constexpr (OES == 4) {
        epilogue<SF_F32>(a, acc, m0, n0, w, lane, s_thr, ereg);
      } else {
        if (a.out_dt == SF_F16) epilogue<SF_F16>(a, acc, m0, n0, w, lane, s_thr, ereg);
        else epilogue<SF_BF16>(a, acc, m0, n0, w, lane, s_thr, ereg);
      }
    } else {
      // both stage buffers are free after the last K-step's barrier: 16 KiB per wave
      char* ereg = w < 4 ? lds0 + w * 16384 : lds1 + (w - 4) * 16384;
      if constexpr (OES == 4) {
        t2::epilogue2<SF_F32, 16384>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
      } else {
        if (a.out_dt == SF_F16) t2::epilogue2<SF_F16, 16384>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
        else t2::epilogue2<SF_BF16, 16384>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
      }
    }
    // the prefetch's value is unused: this keeps its load, awaited only here at the end (a
    // volatile load would be awaited at once, stalling the epilogue for the L2 miss)
    asm volatile("" ::"v"(pf));
    if constexpr (!LIVE) {
      break;
    } else {
      it += gridDim.x;
      if (it >= live_tiles) break;
      __syncthreads();  // every wave is done with the LDS before the next tile's stage-0 DMA
    }
  }
}



// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt at its maximum), the wait before each K-step barrier
// of the pipeline below: at most n of this thread's DMAs still in flight (those of later
// stages), and every LDS read it issued has returned. The second half matters: the fragment
// reads of a step's last k16 chunk are consumed only after the next barrier, and past that
// barrier other waves start the DMA that overwrites the buffer they read.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0070 | N);
}

// ===================================================================================
// 2b. the overlapped GEMM: 256x128 tiles, BK = 64 bytes per row, 3-stage LDS DMA pipeline.
//     72 KiB of LDS and 128 accumulators per wave let two workgroups share a CU, so one
//     workgroup's epilogue, stores and barrier waits run under the other's MFMA work.
// ===================================================================================
template <int DT, int WP, int OES>
__global__ __launch_bounds__(NT, 2) void gemm2_kernel(GemmArgs a) {
  using t2::Tr; using t2::WT; using t2::XT; using t2::Plan2; using t2::off;
  constexpr int BM = t2::BM, BN = t2::BN;
  constexpr int E = Tr<DT>::E, BK = Tr<DT>::BK;
  constexpr int LWP = WP == W_GENERIC ? W_KMAJOR : WP;
  constexpr int NDMA = WP == W_GENERIC ? 4 : 6;  // DMA instructions per thread per stage
  // three stages, each W tile and x' tile a distinct LDS object, so the compiler's
  // wait-count pass can tell every DMA target from every fragment read
  __shared__ __attribute__((aligned(1024))) char wA[WT];
  __shared__ __attribute__((aligned(1024))) char wB[WT];
  __shared__ __attribute__((aligned(1024))) char wC[WT];
  __shared__ __attribute__((aligned(1024))) char xA[XT];
  __shared__ __attribute__((aligned(1024))) char xB[XT];
  __shared__ __attribute__((aligned(1024))) char xC[XT];
  __shared__ __attribute__((aligned(16))) float s_benc[BN];
  __shared__ __attribute__((aligned(16))) float s_thr[BN];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;

  const int total = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = b % 8, loc = b / 8;
  const int lid = xcd * per + min(xcd, rem) + loc;
  const TilePos tp = tile_of(a, lid);
  const int pid_m = tp.m, pid_n = tp.n;
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  if (t < BN) {
    const int64_t n = n0 + t;
    const float h = a.out_dt == SF_F32 ? 0.f : (a.out_dt == SF_BF16 ? __uint_as_float(0x00800000u)
                                                                    : __uint_as_float(0x33000000u));
    float tv = a.act == SF_ACT_NONE ? __builtin_nanf("") : h;
    if (n >= a.N) {
      tv = __builtin_inff();
    } else if (a.act == SF_ACT_JUMPRELU) {
      const float th = load_as_f32(a.thr, a.thr_dt, n);
      tv = th != th ? __builtin_inff() : fmaxf(th, h);
    }
    s_benc[t] = n < a.N ? load_as_f32(a.b_enc, a.benc_dt, n) : 0.f;
    s_thr[t] = tv;
  }

  f32x16 acc[2][4];

  const __amdgpu_buffer_rsrc_t xr = rsrc(a.xw + m0 * a.Kp * E, min((int64_t)BM, a.M - m0) * a.Kp * E);
  Plan2<DT, LWP> plan;
  plan.init(a, n0, w, lane);
  const int KT = a.ksteps;  // a multiple of 3

  // DMA j of K-step kt; a generic W is staged whole (through registers) with j == 0
  auto dma = [&](int kt, char* ws, char* xs, int j) {
    if constexpr (WP == W_GENERIC) {
      if (j < 4) dma16(xr, xs + (j * 4 + w) * 1024, plan.xo[j], (uint32_t)((int64_t)kt * BK * E));
      if (j == 0) t2::stage_generic_w2<DT>(a, n0, kt, ws, t);
    } else {
      t2::issue2_one<DT, WP>(a, plan, xr, n0, kt, ws, xs, w, j);
    }
  };
  struct Frag {
    u32x4 a[2], b[4];
  };
  auto load_frag = [&](Frag& f, const char* ws, const char* xs, int s) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) f.b[mb] = *(const u32x4*)(xs + off(wm * 128 + mb * 32 + (lane & 31), 2 * s + (lane >> 5)));
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) f.a[nb] = t2::load_a2<DT, LWP>(ws, wn, nb, s, lane);
  };
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) mfma_chunk<DT>(acc[nb][mb], f.a[nb], f.b[mb]);
  };
  constexpr int NMF = DT == SF_F32 ? 32 : 8;  // MFMA instructions per k16 chunk
  constexpr int NRD = 4 + (LWP == W_NMAJOR ? (DT == SF_F32 ? 8 : 4) : 2);  // LDS reads per chunk
  auto interleave = [&](auto nv_tag) {
    constexpr int NV = decltype(nv_tag)::value;
    constexpr int RSTEP = NRD > NMF ? (NRD + NMF - 1) / NMF : 1;  // reads per MFMA slot
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i * RSTEP < NRD) __builtin_amdgcn_sched_group_barrier(0x100, RSTEP, 0);
      if (NV > 0 && i < NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  };

  // One K-step region: wait for stage kt, barrier, then group 0 reads chunk 0 of stage kt
  // and multiplies the previous step's chunk 1, group 1 reads chunk 1 and multiplies chunk 0;
  // the six DMAs of stage kt+2 (into the buffer the previous step released) ride along.
  // kind: 0 first, 1 steady, 2 = no stage kt+2 to issue, 3 = also stage kt+1 absent.
  Frag F0, F1;
  auto region = [&](auto kind_tag, const char* cw, const char* cx, char* nw, char* nx, int kt) {
    constexpr int KIND = decltype(kind_tag)::value;
    if constexpr (KIND == 3) wait_vmcnt_lgkm0<0>();
    else wait_vmcnt_lgkm0<NDMA>();
    barrier_no_fence();
    load_frag(F0, cw, cx, 0);
    if constexpr (KIND <= 1) {
#pragma unroll
      for (int j = 0; j < 3; ++j) dma(kt + 2, nw, nx, j);
    }
    if constexpr (KIND != 0) mma(F1);
    interleave(std::integral_constant<int, KIND <= 1 && KIND != 0 ? 3 : 0>{});
    load_frag(F1, cw, cx, 1);
    if constexpr (KIND <= 1) {
#pragma unroll
      for (int j = 3; j < 6; ++j) dma(kt + 2, nw, nx, j);
    }
    mma(F0);
    interleave(std::integral_constant<int, KIND <= 1 ? 3 : 0>{});
  };

#pragma unroll
  for (int j = 0; j < 6; ++j) dma(0, wA, xA, j);
#pragma unroll
  for (int j = 0; j < 6; ++j) dma(1, wB, xB, j);
  // the accumulators start at b_enc (the epilogue's bias add, folded in) while stages land
  wait_lgkmcnt0();
  barrier_no_fence();
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 be = *(const float4*)(s_benc + wn * 64 + nb * 32 + g * 8 + (lane >> 5) * 4);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        acc[nb][mb][g * 4 + 0] = be.x;
        acc[nb][mb][g * 4 + 1] = be.y;
        acc[nb][mb][g * 4 + 2] = be.z;
        acc[nb][mb][g * 4 + 3] = be.w;
      }
    }
  using K0 = std::integral_constant<int, 0>;
  using K1 = std::integral_constant<int, 1>;
  region(K0{}, wA, xA, wC, xC, 0);
  region(K1{}, wB, xB, wA, xA, 1);
  region(K1{}, wC, xC, wB, xB, 2);
  int kt = 3;
  for (; kt + 3 < KT; kt += 3) {
    region(K1{}, wA, xA, wC, xC, kt);
    region(K1{}, wB, xB, wA, xA, kt + 1);
    region(K1{}, wC, xC, wB, xB, kt + 2);
  }
  // the last three steps (KT is a multiple of 3): stage kt+2 exists only for the first
  region(K1{}, wA, xA, wC, xC, kt);
  region(std::integral_constant<int, 2>{}, wB, xB, wA, xA, kt + 1);
  region(std::integral_constant<int, 3>{}, wC, xC, wB, xB, kt + 2);
  mma(F1);
  __syncthreads();  // all waves are done reading the stages: they become staging space

  char* ereg = (w < 2 ? xA : xB) + (w & 1) * 8192;  // 8 KiB of staging per wave
  if constexpr (OES == 4) {
    t2::epilogue2<SF_F32>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
  } else {
    if (a.out_dt == SF_F16) t2::epilogue2<SF_F16>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
    else t2::epilogue2<SF_BF16>(a, acc, m0, n0, wm, wn, lane, s_thr, ereg);
  }
}


// Persistent form of the 256x256 kernel (8 waves of 128x64, or 4 of 128x128 for the dense
// epilogue), for whole tiles (M and N multiples of 256, 16-B aligned output rows): one
// workgroup per CU walks its XCD's contiguous range of the grouped order. Its first tile is
// fixed (one per workgroup); each later one it claims from the XCD's tile counter at the start
// of the tile before, so tiles start in order, as with one workgroup per tile, and the tiles in
// flight on an XCD stay adjacent in the order, without a workgroup launch between tiles. After
// a tile's last K-step both stage buffers are free: the next tile's stage 0 and the raw bits of
// its b_enc and threshold slices are DMAed into one (the slices into its 2 KiB tail), and the
// epilogue stages through the other (8 KiB per wave in two passes with 8 waves, 16 KiB with 4),
// so the next tile's first loads run under this tile's epilogue. Consecutive tiles alternate buffer roles (parity P); the bias and
// threshold slices are double-buffered. The K loop, the accumulator start and the epilogue
// arithmetic are those of gemm_kernel: results are bit-identical to it. The row-candidate
// epilogues (EPI_ROWS*) keep no staging buffer; there the next tile's stage 0 is issued once
// the epilogue's slot atomics have returned, under its candidate stores.
template <int DT, int WP, int ODT, int EPI = EPI_DENSE, int NW = 8>
__global__ __launch_bounds__(NW * 64, 1) void gemm_persist_kernel(GemmArgs a) {
  constexpr int E = Traits<DT>::E;
  constexpr int WCOLS = NW / 2;    // waves across the 256 features
  constexpr int WNC = BN / WCOLS;  // features per wave: 64 (8 waves) or 128 (4 waves)
  constexpr int NBK = WNC / 32;
  constexpr int OES = ODT == SF_F32 ? 4 : 2;
  // epilogue stores per lane: 8 waves stage 8 KiB per pass (16-bit 2 passes of 8 stores, fp32
  // 4 of 8), 4 waves 16 KiB (16-bit 2 of 16, fp32 4 of 16: vmcnt counts to 63 at most)
  constexpr int NST = NW == 8 ? (OES == 2 ? 16 : 32) : (OES == 2 ? 32 : 63);
  static_assert(NW == 8 || NW == 4, "8 waves of 128x64 or 4 of 128x128");
  constexpr int RAW = STAGE;               // offset of the raw b_enc / threshold slices in a buffer
  static_assert(WP != W_GENERIC, "the generic W is staged through registers");
  __shared__ __attribute__((aligned(1024))) char lds0[STAGE + 2048];
  __shared__ __attribute__((aligned(1024))) char lds1[STAGE + 2048];
  __shared__ __attribute__((aligned(16))) float s_benc[2][BN];
  __shared__ __attribute__((aligned(16))) float s_thr[2][BN];
  __shared__ int s_claim;

  const int t0 = threadIdx.x, lane0 = t0 & 63;
  const int total = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = b % 8, loc = b / 8;
  const int first = xcd * per + min(xcd, rem), last = first + per + (xcd < rem ? 1 : 0);
  const int step = gridDim.x / 8;  // workgroups per XCD: the fixed first tiles
  int32_t* const ctr = a.tile_ctr + xcd * TILE_CTR_STRIDE;
  int lid = first + loc;
  if (lid >= last) return;  // the whole workgroup
  const int KT = a.ksteps;

  // Stage 0 of tile (m0, n0) into buf, and the raw bits of its b_enc (wave 0) and threshold
  // (wave 1) slices into buf's tail: nothing of the next tile lands in registers, so its loads
  // are awaited only where the tile starts.
  auto begin_tile = [&](int64_t m0, int64_t n0, char* buf, int lane, int w) {
    const __amdgpu_buffer_rsrc_t xr = rsrc(a.xw + m0 * a.Kp * E, min((int64_t)BM, a.M - m0) * a.Kp * E);
    Plan<DT, WP, NW> plan;
    plan.init(a, n0, w, lane);
#pragma unroll
    for (int q = 0; q < 4; ++q) issue_part<DT, WP, NW>(a, plan, xr, n0, 0, buf, w, q);
    if (w == 0 || (w == 1 && a.act == SF_ACT_JUMPRELU)) {
      const int dt = w == 0 ? a.benc_dt : a.thr_dt;
      const int64_t esz = sf_dtype_size(dt);
      const char* base = (const char*)(w == 0 ? a.b_enc : a.thr) + n0 * esz;
      dma16(rsrc(base, (a.N - n0) * esz), buf + RAW + w * 1024, (uint32_t)lane * 16, 0);
    }
  };
  // s_benc / s_thr slot from the raw slices in buf's tail (thread t: feature n0 + t < N), as
  // gemm_kernel forms them from its loads
  auto set_bias = [&](int slot, const char* buf, int t) {
    if (t < BN) {
      const char* raw = buf + RAW;
      const int bsz = sf_dtype_size(a.benc_dt), tsz = sf_dtype_size(a.thr_dt);
      const uint32_t rb = bsz == 4 ? *(const uint32_t*)(raw + 4 * t) : *(const u16*)(raw + 2 * t);
      // the output type is ODT (a.out_dt): the floor is a constant, not a register kept across tiles
      constexpr float h = ODT == SF_F32 ? 0.f : (ODT == SF_BF16 ? 0x1p-126f : 0x1p-25f);
      float tv = a.act == SF_ACT_NONE ? __builtin_nanf("") : h;
      if (a.act == SF_ACT_JUMPRELU) {
        const uint32_t rt = tsz == 4 ? *(const uint32_t*)(raw + 1024 + 4 * t) : *(const u16*)(raw + 1024 + 2 * t);
        const float th = bits_as_f32(rt, a.thr_dt);
        tv = th != th ? __builtin_inff() : fmaxf(th, h);  // a NaN threshold keeps nothing
      }
      s_benc[slot][t] = bits_as_f32(rb, a.benc_dt);
      s_thr[slot][t] = tv;
    }
  };

  const TilePos tp0 = tile_of(a, lid);
  int64_t m0 = (int64_t)tp0.m * BM, n0 = (int64_t)tp0.n * BN;
  begin_tile(m0, n0, lds0, lane0, __builtin_amdgcn_readfirstlane(t0 >> 6));
  wait_vmcnt0();

  // One tile with buffer parity P: its stage 0 (and every even K-step) in B0, odd K-steps in
  // B1. Returns whether a next tile was started (its stage 0 in B1).
  auto tile = [&](auto par_tag) -> bool {
    constexpr int P = decltype(par_tag)::value;
    char* const B0 = P ? lds1 : lds0;
    char* const B1 = P ? lds0 : lds1;
    // Opaque copies of the thread index, so nothing derived from it is hoisted out of the tile
    // loop (and kept live, or spilled, across the K loop); the wave index as a scalar.
    int lane = lane0, t = t0;
    asm volatile("" : "+v"(lane), "+v"(t));
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = w / WCOLS, wn = w % WCOLS;
    // every thread has awaited its own DMAs of this tile's stage 0 and slices: past the
    // barrier they are visible; the bias and threshold slices formed from them past the next
    wait_lgkmcnt0();
    barrier_no_fence();
    set_bias(P, B0, t);
    wait_lgkmcnt0();
    barrier_no_fence();
    f32x16 acc[NBK][4];
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 be = *(const float4*)(&s_benc[P][0] + wn * WNC + nb * 32 + g * 8 + (lane >> 5) * 4);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          acc[nb][mb][g * 4 + 0] = be.x;
          acc[nb][mb][g * 4 + 1] = be.y;
          acc[nb][mb][g * 4 + 2] = be.z;
          acc[nb][mb][g * 4 + 3] = be.w;
        }
      }
    // claim the next tile now (the compiler awaits the return at once, behind the last tile's
    // epilogue stores; deferring that wait to the K loop's first one measured no faster)
    int claim = 0;
    if (t == 0) claim = atomicAdd(ctr, 1);
    const __amdgpu_buffer_rsrc_t xr = rsrc(a.xw + m0 * a.Kp * E, min((int64_t)BM, a.M - m0) * a.Kp * E);
    Plan<DT, WP, NW> plan;
    plan.init(a, n0, w, lane);
    auto stage_part = [&](int kt, char* st, int part) { issue_part<DT, WP, NW>(a, plan, xr, n0, kt, st, w, part); };
    // the K loop of gemm_kernel (fragments, MFMA order, DMA schedule and waits)
    struct Frag {
      u32x4 a[NBK], b[4];
    };
    auto load_frag = [&](Frag& f, const char* cur, int s) {
      const char* ws = cur;
      const char* xs = cur + TILE;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        f.b[mb] = *(const u32x4*)(xs + lds_off(wm * 128 + mb * 32 + (lane & 31), 2 * s + (lane >> 5)));
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb) f.a[nb] = load_a<DT, WP>(ws, wn * WNC, nb, s, lane);
    };
    auto mma = [&](const Frag& f) {
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) mfma_chunk<DT>(acc[nb][mb], f.a[nb], f.b[mb]);
    };
    constexpr int NMF = NBK * 4 * (DT == SF_F32 ? 4 : 1);
    constexpr int NRD = 4 + NBK * (WP == W_NMAJOR ? (DT == SF_F32 ? 4 : 2) : 1);
    constexpr int DPP = 2 * Plan<DT, WP, NW>::PER / 4;
    auto interleave = [&](auto nv_tag) {
      constexpr int NV = decltype(nv_tag)::value;
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (NV > 0 && i % (NMF / (NV > 0 ? NV : 1)) == 0 && i / (NMF / (NV > 0 ? NV : 1)) < NV)
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
    };
    constexpr int NP0 = SF_DMA_SPLIT == 0 ? 1 : (SF_DMA_SPLIT == 1 ? 2 : 4);
    constexpr int NP1 = SF_DMA_SPLIT == 0 ? 1 : (SF_DMA_SPLIT == 1 ? 2 : 0);
    constexpr int NP2 = SF_DMA_SPLIT == 0 ? 1 : 0;
    constexpr int NP3 = SF_DMA_SPLIT == 0 ? 1 : 0;
    using I0 = std::integral_constant<int, 0>;
    Frag F0, F1;
    auto region = [&](auto kind_tag, const char* cur, char* nxt, int kt) {
      constexpr int KIND = decltype(kind_tag)::value;
      constexpr int S = KIND == 2 ? 0 : 1;
      load_frag(F0, cur, 0);
#pragma unroll
      for (int q = 0; q < NP0 * S; ++q) stage_part(kt + 1, nxt, q);
      if constexpr (KIND != 0) mma(F1);
      interleave(std::integral_constant<int, KIND == 0 ? 0 : DPP * NP0 * S>{});
      load_frag(F1, cur, 1);
#pragma unroll
      for (int q = 0; q < NP1 * S; ++q) stage_part(kt + 1, nxt, NP0 + q);
      mma(F0);
      interleave(std::integral_constant<int, DPP * NP1 * S>{});
      load_frag(F0, cur, 2);
#pragma unroll
      for (int q = 0; q < NP2 * S; ++q) stage_part(kt + 1, nxt, NP0 + NP1 + q);
      mma(F1);
      interleave(std::integral_constant<int, DPP * NP2 * S>{});
      load_frag(F1, cur, 3);
#pragma unroll
      for (int q = 0; q < NP3 * S; ++q) stage_part(kt + 1, nxt, NP0 + NP1 + NP2 + q);
      mma(F0);
      interleave(std::integral_constant<int, DPP * NP3 * S>{});
      wait_vmcnt0();
      __syncthreads();
    };
    region(I0{}, B0, B1, 0);
    // visible past the next barrier
    if (t == 0) s_claim = claim;
    int kt = 1;
    for (; kt + 1 < KT; kt += 2) {
      region(std::integral_constant<int, 1>{}, B1, B0, kt);
      region(std::integral_constant<int, 1>{}, B0, B1, kt + 1);
    }
    region(std::integral_constant<int, 2>{}, B1, B0, kt);  // KT is even: the last step is in B1
    mma(F1);
    // Both buffers are free past the last barrier: the next tile's stage 0 goes to B1 (its B0),
    // the epilogue stages through B0. Fresh opaque copies again keep the epilogue's per-lane
    // addresses from being formed before the K loop.
    lane = lane0;
    t = t0;
    asm volatile("" : "+v"(lane), "+v"(t));
    const int nlid = first + step + s_claim;  // claims past the range fail: the loop ends
    const bool more = nlid < last;
    int64_t nm0 = 0, nn0 = 0;
    if (more) {
      const TilePos np = tile_of(a, nlid);
      nm0 = (int64_t)np.m * BM;
      nn0 = (int64_t)np.n * BN;
      if constexpr (EPI == EPI_DENSE) begin_tile(nm0, nn0, B1, lane, w);
    }
    if constexpr (EPI == EPI_DENSE) {
      if constexpr (NW == 8) t2::epilogue2<ODT, 8192, true>(a, acc, m0, n0, wm, wn, lane, &s_thr[P][0], B0 + w * 8192);
      else epilogue<ODT, 16384, true>(a, acc, m0, n0, w, lane, &s_thr[P][0], B0 + w * 16384);
      if (!more) return false;
      // A wave's vector-memory operations complete in issue order (gfx9 counts loads and
      // stores in one vmcnt): with the epilogue's NST stores issued after the next tile's DMAs,
      // at most NST outstanding means those DMAs have landed, while the stores drain.
      __builtin_amdgcn_s_waitcnt(0x0F70 | (NST & 15) | (((NST >> 4) & 3) << 14));  // vmcnt(NST)
    } else {
      if (!more) {
        epilogue_rows<ODT, EPI == EPI_ROWS_FLOOR, NBK>(a, acc, m0, n0, wm, wn, lane, &s_thr[P][0], [] {});
        return false;
      }
      epilogue_rows<ODT, EPI == EPI_ROWS_FLOOR, NBK>(a, acc, m0, n0, wm, wn, lane, &s_thr[P][0],
                                                      [&] { begin_tile(nm0, nn0, B1, lane, w); });
      wait_vmcnt0();  // the candidate stores are data-dependent: everything
    }
    lid = nlid;
    m0 = nm0;
    n0 = nn0;
    return true;
  };
  for (;;) {
    if (!tile(std::integral_constant<int, 0>{})) break;
    if (!tile(std::integral_constant<int, 1>{})) break;
  }
}

// Kernel launchers, instantiated one per translation unit (encode_<tiling>_<dtype>.hip).
// CUs of the current device (cached per device), for the persistent grid; 0 on a HIP error.
inline int device_cus() {
  static std::atomic<int> cached[64];  // host threads may launch at once: relaxed, same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

template <int DT, int OES, int NW>
hipError_t launch_wide_nw(const GemmArgs& a, int wp, hipStream_t s) {
  dim3 grid(a.tiles_m * a.tiles_n), block(NW * 64);
  // whole tiles with aligned output rows (the dense epilogue): the persistent form, one
  // workgroup per CU (at most one per tile, whole XCD groups of eight)
  if (wp != W_GENERIC && a.M % BM == 0 && a.N % BN == 0 && a.vec_store && a.M > 0 && a.N > 0) {
    const int cus = device_cus();
    if (cus <= 0) return hipErrorInvalidDevice;
    const int total = a.tiles_m * a.tiles_n;
    const dim3 pg((unsigned)std::max(8, std::min(cus / 8 * 8, (total + 7) / 8 * 8)));
    auto go = [&](auto odt_tag) {
      constexpr int ODT = decltype(odt_tag)::value;
      if (wp == W_NMAJOR) hipLaunchKernelGGL((gemm_persist_kernel<DT, W_NMAJOR, ODT, EPI_DENSE, NW>), pg, block, 0, s, a);
      else hipLaunchKernelGGL((gemm_persist_kernel<DT, W_KMAJOR, ODT, EPI_DENSE, NW>), pg, block, 0, s, a);
    };
    if constexpr (OES == 4) go(std::integral_constant<int, SF_F32>{});
    else if (a.out_dt == SF_F16) go(std::integral_constant<int, SF_F16>{});
    else go(std::integral_constant<int, SF_BF16>{});
    return hipGetLastError();
  }
  switch (wp) {
    case W_NMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_NMAJOR, OES, NW>), grid, block, 0, s, a); break;
    case W_KMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_KMAJOR, OES, NW>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<DT, W_GENERIC, OES, NW>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

template <int DT, int OES>
hipError_t launch_wide(const GemmArgs& a, int wp, int waves, hipStream_t s) {
  return waves == 4 ? launch_wide_nw<DT, OES, 4>(a, wp, s) : launch_wide_nw<DT, OES, 8>(a, wp, s);
}

template <int DT, int OES>
hipError_t launch_narrow(const GemmArgs& a, int wp, hipStream_t s) {
  dim3 grid(a.tiles_m * a.tiles_n), block(NT);
  switch (wp) {
    case W_NMAJOR: hipLaunchKernelGGL((gemm2_kernel<DT, W_NMAJOR, OES>), grid, block, 0, s, a); break;
    case W_KMAJOR: hipLaunchKernelGGL((gemm2_kernel<DT, W_KMAJOR, OES>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm2_kernel<DT, W_GENERIC, OES>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

// Row-candidate kernels: one instantiation per output type ODT (an sf_dtype code), so each
// holds a single epilogue body (two in one kernel spill registers).
template <int DT, int ODT, int EPI>
hipError_t launch_rows(const GemmArgs& a, int wp, hipStream_t s) {
  constexpr int NW = SF_WIDE_WAVES;
  dim3 grid(a.tiles_m * a.tiles_n), block(NW * 64);
  if constexpr (NW == 8) {  // whole tiles: the persistent form
    if (wp != W_GENERIC && a.M % BM == 0 && a.N % BN == 0 && a.M > 0 && a.N > 0) {
      const int cus = device_cus();
      if (cus <= 0) return hipErrorInvalidDevice;
      const int total = a.tiles_m * a.tiles_n;
      const dim3 pg((unsigned)std::max(8, std::min(cus / 8 * 8, (total + 7) / 8 * 8)));
      if (wp == W_NMAJOR) hipLaunchKernelGGL((gemm_persist_kernel<DT, W_NMAJOR, ODT, EPI, NW>), pg, block, 0, s, a);
      else hipLaunchKernelGGL((gemm_persist_kernel<DT, W_KMAJOR, ODT, EPI, NW>), pg, block, 0, s, a);
      return hipGetLastError();
    }
  }
  switch (wp) {
    case W_NMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_NMAJOR, ODT, NW, EPI>), grid, block, 0, s, a); break;
    case W_KMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_KMAJOR, ODT, NW, EPI>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<DT, W_GENERIC, ODT, NW, EPI>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

// Gathered-row dense kernels (sf_encode_gather): 256x256 with SF_WIDE_WAVES waves, one
// workgroup per CU.
template <int DT, int OES>
hipError_t launch_live(const GemmArgs& a, int wp, int cus, hipStream_t s) {
  constexpr int NW = SF_WIDE_WAVES;
  dim3 grid((unsigned)std::max(1, std::min(cus, a.tiles_m * a.tiles_n))), block(NW * 64);
  switch (wp) {
    case W_NMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_NMAJOR, OES, NW, EPI_DENSE, true>), grid, block, 0, s, a); break;
    case W_KMAJOR: hipLaunchKernelGGL((gemm_kernel<DT, W_KMAJOR, OES, NW, EPI_DENSE, true>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<DT, W_GENERIC, OES, NW, EPI_DENSE, true>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

#define SF_ENC_EXTERN(DT)                                                         \
  extern template hipError_t launch_wide<DT, 2>(const GemmArgs&, int, int, hipStream_t); \
  extern template hipError_t launch_wide<DT, 4>(const GemmArgs&, int, int, hipStream_t); \
  extern template hipError_t launch_narrow<DT, 2>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_narrow<DT, 4>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_F32, EPI_ROWS>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_BF16, EPI_ROWS>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_F16, EPI_ROWS>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_F32, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_BF16, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_rows<DT, SF_F16, EPI_ROWS_FLOOR>(const GemmArgs&, int, hipStream_t); \
  extern template hipError_t launch_live<DT, 2>(const GemmArgs&, int, int, hipStream_t); \
  extern template hipError_t launch_live<DT, 4>(const GemmArgs&, int, int, hipStream_t);
SF_ENC_EXTERN(SF_F32)
SF_ENC_EXTERN(SF_BF16)
SF_ENC_EXTERN(SF_F16)
#undef SF_ENC_EXTERN

}  // namespace sfenc
