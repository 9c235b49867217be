// Backward of the sparse SAE path on gfx950: gradients of a loss through
//   x' = cast_W(x - b_dec),  pre = x' W_enc + b_enc,  f = act(pre) (CSR),  x_hat = f W_dec + b_dec
// given g_xhat = dL/dx_hat (and optionally dL/df on the CSR values). The reference lists these
// kernels on its roadmap (saeflow README.md:244, "Backward kernels for training SAEs on sparse
// features"); the forward they differentiate is saeflow/reference.py:36-52 with the CSR of
// ops.encode_sparse (ops.py:29-39).
//
// Every gradient is a sum over the nonzeros of f, so all work is proportional to nnz, and all of
// it is gather / reduce traffic (no dense contraction):
//  - CSR -> CSC, deterministic: a two-level stable counting sort by column (no global atomics),
//    so each column lists its entries in increasing token order.
//  - Per feature j, in work items of at most CHUNK entries, one wave per (item, 512-element
//    slab of d_in): backward_dec_kernel sums dW_dec[j] = sum_m f[m,j] g_xhat[m] and, for each
//    entry, the slab's share of g_xhat[m] . W_dec[j] (W_dec[j]'s slab sits in registers, so the
//    dot products need no gather of their own); gpre_kernel adds the shares in slab order into
//    g_pre = (g_xhat[m] . W_dec[j] + dL/df) * [f > 0]; backward_enc_kernel sums
//    dW_enc^T[j] = sum_m g_pre[m,j] x'[m] and db_enc[j] = sum_m g_pre[m,j]. Columns of more than
//    CHUNK entries write fp32 partials that backward_reduce_kernel sums in chunk order, so
//    results do not depend on timing.
//  - dx' = g_pre W_enc^T is the forward decode over W_enc^T (transpose_kernel makes it
//    row-contiguous), and db_dec = sum_m g_xhat[m] - W_enc db_enc uses col_sums_kernel and
//    matvec_kernel.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WPB = 4;        // waves per 256-thread block
constexpr int64_t CHUNK = 256;  // column entries per work item of backward_units_kernel
constexpr int64_t HEAVY = 64;   // a column with more entries sums into fp32 partial slots
constexpr uint32_t BUF_W3 = 0x00020000;  // buffer resource dword 3 for raw loads (gfx9 family)

__device__ __forceinline__ void clamp_range(const int64_t* ptr, int64_t i, int64_t n, int64_t& lo, int64_t& hi) {
  lo = ptr[i];
  hi = ptr[i + 1];
  lo = lo < 0 ? 0 : (lo > n ? n : lo);
  hi = hi < lo ? lo : (hi > n ? n : hi);
}

// Sum of v over the wave, returned in every lane, with DPP moves (VALU) instead of LDS
// permutes: xor-1 and xor-2 within quads, the half-row and row mirrors give each 16-lane row
// its total, row_bcast:15 / row_bcast:31 carry row totals upward, lane 63 ends with the sum.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xF>(v);  // row_mirror
  v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave sums of 8 values at once: afterwards every lane l holds the total of v[(l >> 3) & 7].
// A reduce-scatter: each of three exchanges (lanes 32, 16 and 8 apart) keeps half of the values
// a lane still carries and adds its partner's copy of that half, then DPP moves sum the 8-lane
// groups (quads, then the half-row mirror). 7 permutes and 10 adds instead of 8 full reductions.
__device__ __forceinline__ float wave_sum8(const float (&v)[8], int lane) {
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
  float w[4], x[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = (b5 ? v[k + 4] : v[k]) + __shfl_xor(b5 ? v[k] : v[k + 4], 32);
#pragma unroll
  for (int k = 0; k < 2; ++k) x[k] = (b4 ? w[k + 2] : w[k]) + __shfl_xor(b4 ? w[k] : w[k + 2], 16);
  float y = (b3 ? x[1] : x[0]) + __shfl_xor(b3 ? x[0] : x[1], 8);
  y = dpp_add<0xB1, 0xF>(y);   // quad_perm [1,0,3,2]
  y = dpp_add<0x4E, 0xF>(y);   // quad_perm [2,3,0,1]
  return dpp_add<0x141, 0xF>(y);  // row_half_mirror: the other quad of the 8-lane group
}

// EPC elements (one 16-B chunk) of row `rowp` starting at element c*EPC, as fp32. VEC: the
// row is 16-B aligned and D % EPC == 0, so the chunk is one load; otherwise element loads
// with elements past D read as 0.
template <int DT, bool VEC>
__device__ __forceinline__ void load_chunk(const char* rowp, int64_t c, int64_t D, float* v) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  if constexpr (VEC) {
    const u32x4 q = *(const u32x4*)(rowp + c * 16);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      if constexpr (DT == SF_F32) v[e] = __uint_as_float(q[e]);
      else {
        const uint32_t h = (q[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        v[e] = DT == SF_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t i = c * EPC + e;
      v[e] = i < D ? load_as_f32(rowp, DT, i) : 0.f;
    }
  }
}

template <int DT, bool VEC>
__device__ __forceinline__ void store_chunk(char* rowp, int64_t c, int64_t D, const float* v) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  if constexpr (VEC) {
    u32x4 q;
    if constexpr (DT == SF_F32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = __float_as_uint(v[e]);
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) q[d] = f32_to_bits(v[2 * d], DT) | (f32_to_bits(v[2 * d + 1], DT) << 16);
    }
    *(u32x4*)(rowp + c * 16) = q;
  } else {
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t i = c * EPC + e;
      if (i < D) {
        if constexpr (ES == 4) ((float*)rowp)[i] = v[e];
        else ((u16*)rowp)[i] = (u16)f32_to_bits(v[e], DT);
      }
    }
  }
}

// --------------------------------------------------------------------------- CSR -> CSC
__global__ __launch_bounds__(256) void col_count_kernel(const int64_t* indptr, const int32_t* indices, int64_t M,
                                                        int64_t N, int64_t nnz, int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= M) return;
  int64_t lo, hi;
  clamp_range(indptr, row, nnz, lo, hi);
  for (int64_t e = lo + lane; e < hi; e += 64) {
    const int32_t c = indices[e];
    if (c >= 0 && c < N) atomicAdd(counts + c, 1);
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// Entry e = (row, c) goes to an unordered slot of column c's segment.
__global__ __launch_bounds__(256) void col_place_kernel(const int64_t* indptr, const int32_t* indices, int64_t M,
                                                        int64_t N, int64_t nnz, const int64_t* colptr,
                                                        int32_t* cursor, int32_t* tmp_row, int32_t* tmp_pos) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= M) return;
  int64_t lo, hi;
  clamp_range(indptr, row, nnz, lo, hi);
  for (int64_t e = lo + lane; e < hi; e += 64) {
    const int32_t c = indices[e];
    if (c >= 0 && c < N) {
      const int64_t slot = colptr[c] + atomicAdd(cursor + c, 1);
      tmp_row[slot] = (int32_t)row;
      tmp_pos[slot] = (int32_t)e;
    }
  }
}

// One block per column: the column's entries in increasing row order (then CSR position).
// Up to 64 entries: one wave ranks them by comparison. More: bit `row` of an LDS bitmap of M
// bits is set per entry, and an entry's rank is the number of set bits below it (a block scan
// of the words' popcounts). A canonical CSR has each row at most once per column; a column
// where a row repeats (duplicate indices in a CSR row) is ranked by comparison instead, so
// every slot of the column is written exactly once.
__device__ __forceinline__ bool key_less(int ra, int pa, int rb, int pb) { return ra < rb || (ra == rb && pa < pb); }

__global__ __launch_bounds__(256) void col_sort_kernel(const int64_t* colptr, int64_t M, const int32_t* tmp_row,
                                                       const int32_t* tmp_pos, int32_t* csc_row, int32_t* csc_pos) {
  extern __shared__ uint32_t s_bits[];  // [W] bitmap, then [W] exclusive prefix of popcounts
  __shared__ uint32_t s_wsum[4];
  __shared__ int s_dup;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t j = blockIdx.x;
  const int64_t lo = colptr[j], n = colptr[j + 1] - lo;
  if (n <= 0) return;
  if (n <= 64) {
    if (w != 0) return;
    const int r = lane < n ? tmp_row[lo + lane] : 0x7fffffff;
    const int p = lane < n ? tmp_pos[lo + lane] : 0x7fffffff;
    int rank = 0;
    for (int q = 0; q < (int)n; ++q)
      rank += key_less(__builtin_amdgcn_readlane(r, q), __builtin_amdgcn_readlane(p, q), r, p) ? 1 : 0;
    if (lane < n) {
      csc_row[lo + rank] = r;
      csc_pos[lo + rank] = p;
    }
    return;
  }
  const int W = (int)((M + 31) / 32);
  uint32_t* bits = s_bits;
  uint32_t* pref = s_bits + W;
  for (int i = t; i < W; i += 256) bits[i] = 0;
  if (t == 0) s_dup = 0;
  __syncthreads();
  for (int64_t i = t; i < n; i += 256) {
    const int r = tmp_row[lo + i];
    const uint32_t bit = 1u << (r & 31);
    if (atomicOr(bits + (r >> 5), bit) & bit) s_dup = 1;
  }
  __syncthreads();
  if (s_dup) {  // block-uniform: rank every entry against all others
    for (int64_t i = t; i < n; i += 256) {
      const int r = tmp_row[lo + i], p = tmp_pos[lo + i];
      int64_t rank = 0;
      for (int64_t q = 0; q < n; ++q) rank += key_less(tmp_row[lo + q], tmp_pos[lo + q], r, p) ? 1 : 0;
      csc_row[lo + rank] = r;
      csc_pos[lo + rank] = p;
    }
    return;
  }
  // exclusive prefix of popcounts: thread t owns words [t*per, (t+1)*per)
  const int per = (W + 255) / 256;
  const int w0 = min(W, t * per), w1 = min(W, w0 + per);
  uint32_t s = 0;
  for (int i = w0; i < w1; ++i) s += __popc(bits[i]);
  uint32_t x = s;  // inclusive wave scan
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_wsum[w] = x;
  __syncthreads();
  uint32_t run = x - s;
  for (int q = 0; q < w; ++q) run += s_wsum[q];
  for (int i = w0; i < w1; ++i) {
    pref[i] = run;
    run += __popc(bits[i]);
  }
  __syncthreads();
  for (int64_t i = t; i < n; i += 256) {
    const int r = tmp_row[lo + i];
    const uint32_t rank = pref[r >> 5] + __popc(bits[r >> 5] & ((1u << (r & 31)) - 1u));
    csc_row[lo + rank] = r;
    csc_pos[lo + rank] = tmp_pos[lo + i];
  }
}

// ------------------------------------------- CSR -> CSC as a two-level stable counting sort
// Used for n_cols <= 2^23 (any number of rows). Columns fall into nb buckets of 2^LB
// consecutive columns (about 2^CSC_BUCKET_BITS buckets). Wave s of S owns the rows
// [s*RW, (s+1)*RW), hence the CSR positions [indptr[s*RW], indptr[(s+1)*RW]).
//  1. csc_count_kernel: wave s counts its valid entries per bucket into hist[b*S + s].
//  2. sf_scan_counts over hist (bucket-major): offs[b*S + s] = first slot of (bucket b, wave s).
//  3. csc_bucket_kernel: wave s walks its entries again in CSR order and writes (row, position,
//     low column bits) to consecutive slots of each bucket; the rank inside a 64-entry chunk
//     comes from ballots on the bucket bits, the running slot of each bucket lives in LDS.
//  4. csc_sort_kernel: a block per bucket counts its entries per column (4 waves on 4
//     consecutive quarters of the bucket), scans the counts into colptr and places the
//     entries the same way.
// Both placements keep CSR order among equal keys, so every column lists its entries by
// increasing row, then position. No global atomics: the result is deterministic. Slots are
// bounds-checked, so a malformed indptr cannot make a pass write outside its arrays.
#ifndef CSC_BUCKET_BITS
#define CSC_BUCKET_BITS 8
#endif
#ifndef CSC_WAVES
#define CSC_WAVES 1024
#endif
constexpr int CSC_MAX_LB = 11;    // pass 4 keeps 4 x 2^LB counters in LDS (32 KB)
constexpr int CSC_MAX_NB = 4096;  // passes 1 and 3 keep 4 x nb counters in LDS (64 KB)
constexpr int CSC_MAX_RW = 32;    // a wave's row offsets sit in its lanes
constexpr int CSC_U = 4;          // 64-entry chunks whose loads are in flight together

struct CscPlan {
  int LB, nb, nb_bits;
  int64_t RW, S;
};

int bits_for(int64_t n) {  // smallest b with n <= 2^b
  int b = 0;
  while (b < 62 && (1LL << b) < n) ++b;
  return b;
}

CscPlan csc_plan(int64_t M, int64_t N) {
  CscPlan p;
  p.LB = std::min(CSC_MAX_LB, std::max(0, bits_for(N) - CSC_BUCKET_BITS));
  p.nb = (int)std::max<int64_t>(1, (N + (1LL << p.LB) - 1) >> p.LB);
  p.nb_bits = bits_for(p.nb);
  p.RW = std::min<int64_t>(CSC_MAX_RW, std::max<int64_t>(1, (M + CSC_WAVES - 1) / CSC_WAVES));
  p.S = std::max<int64_t>(1, (M + p.RW - 1) / p.RW);
  return p;
}

bool csc_sorts(int64_t N) { return (N + (1LL << CSC_MAX_LB) - 1) >> CSC_MAX_LB <= CSC_MAX_NB; }

// Wave s's rows r0 .. r0+nr-1: lane i <= nr returns indptr[r0+i] clamped into [P0, P1], with
// P0 = indptr[r0] clamped to [0, nnz] and P1 = indptr[r0+nr] clamped to [P0, nnz].
__device__ __forceinline__ int wave_rows(const int64_t* indptr, int64_t s, int64_t RW, int64_t M, int64_t nnz,
                                         int lane, int64_t& r0, int& nr, int& P0, int& P1) {
  r0 = s * RW;
  nr = (int)min(RW, M - r0);
  int64_t v = indptr[r0 + min((int64_t)lane, (int64_t)nr)];
  v = v < 0 ? 0 : (v > nnz ? nnz : v);
  P0 = __builtin_amdgcn_readfirstlane((int)v);
  P1 = max(P0, __builtin_amdgcn_readlane((int)v, nr));
  return min(max((int)v, P0), P1);
}

// Lanes whose key equals this lane's among the lanes in `live` (keys < 2^nbits).
__device__ __forceinline__ uint64_t match_key(int key, int nbits, bool in, uint64_t live) {
  uint64_t same = live;
  for (int bit = 0; bit < nbits; ++bit) {
    const bool one = (key >> bit) & 1;
    const uint64_t m = __ballot(in && one);
    same &= one ? m : ~m;
  }
  return same;
}

__global__ __launch_bounds__(256) void csc_count_kernel(const int64_t* indptr, const int32_t* indices, int64_t M,
                                                        int64_t N, int64_t nnz, int LB, int nb, int64_t RW,
                                                        int64_t S, int32_t* hist) {
  extern __shared__ int32_t s_cnt[];  // [4][nb]
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int32_t* cnt = s_cnt + wv * nb;
  for (int i = lane; i < nb; i += 64) cnt[i] = 0;
  __syncthreads();
  const int64_t s = (int64_t)blockIdx.x * 4 + wv;
  if (s < S) {
    int64_t r0;
    int nr, P0, P1;
    wave_rows(indptr, s, RW, M, nnz, lane, r0, nr, P0, P1);
    for (int e0 = P0; e0 < P1; e0 += 256) {
      int c[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) c[u] = indices[min(e0 + u * 64 + lane, P1 - 1)];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (e0 + u * 64 + lane < P1 && c[u] >= 0 && c[u] < N) atomicAdd(cnt + (c[u] >> LB), 1);
    }
  }
  __syncthreads();
  if (s < S)
    for (int i = lane; i < nb; i += 64) hist[(int64_t)i * S + s] = cnt[i];
}

__global__ __launch_bounds__(256) void csc_bucket_kernel(const int64_t* indptr, const int32_t* indices, int64_t M,
                                                         int64_t N, int64_t nnz, int LB, int nb, int nb_bits,
                                                         int64_t RW, int64_t S, const int64_t* offs, int32_t* t_row,
                                                         int32_t* t_pos, int32_t* t_low) {
  extern __shared__ int32_t s_run[];  // [4][nb]: the next slot of each bucket, per wave
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t s = (int64_t)blockIdx.x * 4 + wv;
  if (s >= S) return;
  int32_t* run = s_run + wv * nb;
  for (int i = lane; i < nb; i += 64) run[i] = (int32_t)min(offs[(int64_t)i * S + s], nnz);
  int64_t r0;
  int nr, P0, P1;
  const int ip = wave_rows(indptr, s, RW, M, nnz, lane, r0, nr, P0, P1);
  const int lowmask = (1 << LB) - 1;
  int cur = 0;  // the wave's row holding position e0
  for (int e1 = P0; e1 < P1; e1 += 64 * CSC_U) {
    int cc[CSC_U];  // CSC_U chunks loaded together, then placed in order
#pragma unroll
    for (int u = 0; u < CSC_U; ++u) cc[u] = indices[min(e1 + u * 64 + lane, P1 - 1)];
#pragma unroll
    for (int u = 0; u < CSC_U; ++u) {
      const int e0 = e1 + u * 64;
      if (e0 >= P1) break;
      const int c = cc[u];
      const int e = e0 + lane;
      const bool valid = e < P1 && c >= 0 && c < N;
      while (cur + 1 < nr && __builtin_amdgcn_readlane(ip, cur + 1) <= e0) ++cur;
      int my = cur;
      for (int k = cur + 1; k < nr; ++k) {
        const int start = __builtin_amdgcn_readlane(ip, k);
        if (start > e0 + 63) break;
        if (start <= e) my = k;
      }
      const int bk = valid ? c >> LB : 0;
      const uint64_t same = match_key(bk, nb_bits, valid, __ballot(valid));
      const uint64_t below = same & lanemask_lt(lane);
      if (valid) {
        const int base = run[bk];
        const int dst = base + (int)__popcll(below);
        if (dst < nnz) {
          t_row[dst] = (int32_t)(r0 + my);
          t_pos[dst] = e;
          t_low[dst] = c & lowmask;
        }
        if (below == 0) run[bk] = base + (int)__popcll(same);
      }
    }
  }
}

__global__ __launch_bounds__(256) void csc_sort_kernel(const int64_t* offs, int64_t S, int nb, int LB, int64_t N,
                                                       int64_t nnz, const int32_t* t_row, const int32_t* t_pos,
                                                       const int32_t* t_low, int64_t* colptr, int32_t* csc_row,
                                                       int32_t* csc_pos) {
  extern __shared__ int32_t s_c[];  // [4][K] per-wave counts, then each wave's next slot per column
  __shared__ int32_t s_tot[4];
  const int K = 1 << LB;
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t b = blockIdx.x;
  const int lo = (int)min(offs[b * S], nnz);
  const int hi = max(lo, (int)min(offs[(b + 1) * S], nnz));
  const int n = hi - lo, q = (n + 3) / 4;
  const int q0 = lo + min(n, wv * q), q1 = lo + min(n, (wv + 1) * q);
  int32_t* cnt = s_c + wv * K;
  for (int i = t; i < 4 * K; i += 256) s_c[i] = 0;
  __syncthreads();
  for (int i0 = q0; i0 < q1; i0 += 256) {
    int l[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) l[u] = t_low[min(i0 + u * 64 + lane, q1 - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + u * 64 + lane < q1) atomicAdd(cnt + (l[u] & (K - 1)), 1);
  }
  __syncthreads();
  // exclusive scan over the bucket's K columns; thread t owns columns [t*per, (t+1)*per)
  const int per = (K + 255) / 256;
  const int k0 = min(K, t * per), k1 = min(K, k0 + per);
  int sum = 0;
  for (int k = k0; k < k1; ++k) sum += s_c[k] + s_c[K + k] + s_c[2 * K + k] + s_c[3 * K + k];
  int x = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_tot[wv] = x;
  __syncthreads();
  int run = lo + x - sum;
  for (int w = 0; w < wv; ++w) run += s_tot[w];
  for (int k = k0; k < k1; ++k) {
    const int64_t col = b * K + k;
    if (col < N) colptr[col] = run;
    const int c0 = s_c[k], c1 = s_c[K + k], c2 = s_c[2 * K + k], c3 = s_c[3 * K + k];
    s_c[k] = run;
    s_c[K + k] = run + c0;
    s_c[2 * K + k] = run + c0 + c1;
    s_c[3 * K + k] = run + c0 + c1 + c2;
    run += c0 + c1 + c2 + c3;
  }
  if (b == nb - 1 && t == 0) colptr[N] = hi;
  __syncthreads();
  for (int i1 = q0; i1 < q1; i1 += 64 * CSC_U) {
    int ll[CSC_U], rr[CSC_U], pp[CSC_U];  // CSC_U chunks loaded together, then placed in order
#pragma unroll
    for (int u = 0; u < CSC_U; ++u) {
      const int ic = min(i1 + u * 64 + lane, q1 - 1);
      ll[u] = t_low[ic];
      rr[u] = t_row[ic];
      pp[u] = t_pos[ic];
    }
#pragma unroll
    for (int u = 0; u < CSC_U; ++u) {
      const int i0 = i1 + u * 64;
      if (i0 >= q1) break;
      const int l = ll[u] & (K - 1);
      const bool in = i0 + lane < q1;
      const uint64_t same = match_key(l, LB, in, __ballot(in));
      const uint64_t below = same & lanemask_lt(lane);
      if (in) {
        const int base = cnt[l];
        const int dst = base + (int)__popcll(below);
        if (dst < nnz) {
          csc_row[dst] = rr[u];
          csc_pos[dst] = pp[u];
        }
        if (below == 0) cnt[l] = base + (int)__popcll(same);
      }
    }
  }
}

// --------------------------------------------------------------------------- per-feature sums
struct ColArgs {
  const int64_t* colptr;    // [N+1]
  const int32_t* csc_row;   // [nnz] token of each entry, increasing within a column
  const int32_t* csc_pos;   // [nnz] CSR position of each entry
  const int64_t* item_off;  // [N+1] first work item of each column
  const int64_t* part_off;  // [N+1] first partial slot of each column (slots only for a heavy column)
  const int32_t* item_col;  // [n_items] column of each work item (valid below item_off[N])
  const int32_t* slot_item;  // [n_slots] work item of each partial slot (valid below part_off[N])
  int64_t n_items;
  const void* values;  // f on the CSR positions
  int val_dt;
  const void* g_val;  // optional dL/df on the CSR positions
  int gval_dt;
  const char* w_dec;  // W_dec [N, D] rows of stride sw, dtype DT
  int64_t sw;
  const char* xs;  // x' [M, D] stride sx, dtype DT
  int64_t sx;
  const char* g_xhat;  // [M, D] stride sg, dtype DT
  int64_t sg;
  int64_t N, M, D, nnz;
  float* dots;    // [nslab, nnz] each slab's share of g_xhat[m] . W_dec[j], per CSC entry
  float* g_csc;   // [nnz] dL/dpre per CSC entry
  float* g_pre;   // [nnz] dL/dpre per CSR position
  char* d_wdec;   // [N, D] contiguous, dtype DT
  char* d_wenc;   // [D, N] contiguous, dtype DT
  float* d_benc;  // [N]
  float* part;    // [slots, 2, D] fp32, then [slots] fp32 for b_enc
  int64_t n_slots;
};

// x' = cast_DT(fp32(x) - fp32(b_dec)), the forward's MFMA operand (encode.py:72), [M, D]
// contiguous.
template <int DT>
__global__ __launch_bounds__(256) void shift_kernel(const void* x, int64_t sxm, int64_t sxk, int x_dt,
                                                    const void* b_dec, int bdec_dt, int64_t M, int64_t D, char* xs) {
  constexpr int ES = DT == SF_F32 ? 4 : 2;
  const int64_t total = M * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / D, d = i - m * D;
    const float v = load_as_f32(x, x_dt, m * sxm + d * sxk) - load_as_f32(b_dec, bdec_dt, d);
    if constexpr (ES == 4) ((float*)xs)[i] = v;
    else ((u16*)xs)[i] = (u16)f32_to_bits(v, DT);
  }
}

// The same for x of dtype DT with 16-B aligned rows and D % EPC == 0. Block (x, y) covers the
// chunks [x*64, ...) (one per lane, its b_dec chunk loaded once) of the rows [y*SH_R, ...),
// its 4 waves taking every 4th row, SH_R/4 rows in flight.
constexpr int SH_R = 32;
template <int DT>
__global__ __launch_bounds__(256) void shift_vec_kernel(const char* x, int64_t sxm, const void* b_dec, int bdec_dt,
                                                        int64_t M, int64_t D, char* xs) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES, RW = SH_R / 4;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  if (c * EPC >= D) return;
  float b[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) b[e] = load_as_f32(b_dec, bdec_dt, c * EPC + e);
  const int64_t m0 = (int64_t)blockIdx.y * SH_R + wv;
  float v[RW][EPC];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int64_t m = min(m0 + 4 * i, M - 1);  // rows past M reload row M-1 and are not stored
    load_chunk<DT, true>(x + m * sxm * ES, c, D, v[i]);
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int64_t m = m0 + 4 * i;
    if (m < M) {
#pragma unroll
      for (int e = 0; e < EPC; ++e) v[i][e] -= b[e];
      store_chunk<DT, true>(xs + m * D * ES, c, D, v[i]);
    }
  }
}

// A work item: column j, its chunk q = the CSC entries [e_lo, e_hi) (at most CHUNK, in token
// order), and the column's number of partial slots (0: the column is this one chunk).
struct Item {
  int64_t j, q, e_lo, e_hi, slots;
};
__device__ __forceinline__ Item item_at(const ColArgs& a, int64_t item) {
  Item it;
  it.j = a.item_col[item];
  it.q = item - a.item_off[it.j];
  const int64_t c_lo = a.colptr[it.j], c_hi = a.colptr[it.j + 1];
  it.e_lo = c_lo + it.q * CHUNK;
  it.e_hi = min(c_hi, it.e_lo + CHUNK);
  it.slots = a.part_off[it.j + 1] - a.part_off[it.j];
  return it;
}

template <int DT>
__device__ __forceinline__ float chunk_elem(const u32x4& r, int e) {
  if constexpr (DT == SF_F32) return __uint_as_float(r[e]);
  else {
    const uint32_t h = (r[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
    return DT == SF_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  }
}

// Dot product of two 16-B chunks (16-bit types: packed dot2 instructions on the raw halves,
// products exact in fp32).
template <int DT>
__device__ __forceinline__ float chunk_dot(const u32x4& x, const u32x4& y) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  // the words are copied out before the bit casts: a bit cast of a vector element itself took
  // element 0 for every q in this compiler
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
  float d = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (DT == SF_BF16)
      d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xs[q]), __builtin_bit_cast(bf16x2, ys[q]), d, false);
    else if constexpr (DT == SF_F16)
      d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, xs[q]), __builtin_bit_cast(f16x2, ys[q]), d, false);
    else d = fmaf(__uint_as_float(xs[q]), __uint_as_float(ys[q]), d);
  }
  return d;
}

// Final row chunk of a one-chunk column, or this chunk's fp32 partial (half 0: dW_dec, 1: dW_enc^T).
template <int DT, bool VEC>
__device__ __forceinline__ void put_rows(const ColArgs& a, const Item& it, char* out, int half, int64_t c,
                                         const float* acc) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  if (it.slots == 0) {
    store_chunk<DT, VEC>(out + it.j * a.D * ES, c, a.D, acc);
  } else {
    float* pr = a.part + (a.part_off[it.j] + it.q) * 2 * a.D + half * a.D;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t d = c * EPC + e;
      if (d < a.D) pr[d] = acc[e];
    }
  }
}

// Phase A (DEC) and phase B (!DEC, LIST) of the per-feature sums, one wave per (G consecutive
// work items, slab): slab = 64 consecutive 16-B chunks of the D-wide rows, one per lane. The
// items' entries (token m, CSR position e) are contiguous in the CSC and are walked in order,
// fetched 64 at a time and broadcast with readlane; where an item ends (a wave-uniform test)
// its slab is stored (to dW_dec, or to the item's partial slot in a heavy column) and the next
// item's sums start:
//   A: dW_dec[j] += f[e] g_xhat[m] on the slab, and dots[slab, i] = the slab's share of
//      g_xhat[m] . W_dec[j] for the entry's CSC index i, 8 entries reduced across the wave at
//      once (the W_dec[j] chunks of the wave's items are loaded up front); every work item;
//   B: dW_enc^T[j] += g_pre x'[m] on the slab and, on slab 0, db_enc[j] = sum g_pre; only the
//      work items of heavy columns (listed by slot_item; enc_tile_kernel sums the others).
// Several items per wave amortise the per-wave metadata loads over features of few entries
// (at d_sae = 2^20 a feature has ~1.3). The items, their bounds and the per-entry row and
// scalar are wave-uniform (scalar registers). With 16-B aligned rows (VEC; the gathered
// tensor under 4 GB) a row is one buffer load: the scalar row offset plus the lane's 32-bit
// chunk offset, no vector address arithmetic; lanes past the row's end load the row's last
// chunk instead of branching around the load, their sums are never stored and their phase-A
// dot shares are zeroed (a load past the buffer's end, as with D = 0, returns zeros). U rows
// in flight. Surplus waves (the grid may be sized by a bound of the item count) return at once.
template <int DT, bool VEC, int U, bool DEC, int G, bool LIST>
__global__ __launch_bounds__(256) void backward_units_kernel(ColArgs a, int nslab) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  static_assert(!DEC || U == 8, "phase A reduces 8 entries at once");
  static_assert(DEC != LIST && (!LIST || G == 1), "phase A walks the item table, phase B the slots");
  const int lane = threadIdx.x & 63;
  const uint32_t wid = blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t grp = wid / (uint32_t)nslab;
  const int64_t slab = wid - grp * (uint32_t)nslab;
  const int64_t n_items = LIST ? min(a.n_slots, a.part_off[a.N]) : min(a.n_items, a.item_off[a.N]);
  const int64_t i0 = (int64_t)grp * G;
  if (i0 >= n_items) return;
  const int ni = (int)min((int64_t)G, n_items - i0);
  // the wave's items, head first: column, end of its entries, fp32 partial slot (-1: the item
  // is the whole column)
  int q_j[G], q_slot[G];
  int64_t q_end[G], e_lo = 0, e_hi = 0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    q_j[g] = 0;
    q_slot[g] = -1;
    q_end[g] = 0;
    if (g < ni) {
      const Item it = item_at(a, LIST ? (int64_t)a.slot_item[i0 + g] : i0 + g);
      q_j[g] = (int)it.j;
      // phase A stores the row of a one-item column directly; phase B always fills the slot
      q_slot[g] = it.slots > (DEC ? 1 : 0) ? (int)(a.part_off[it.j] + it.q) : -1;
      q_end[g] = it.e_hi;
      if (g == 0) e_lo = it.e_lo;
      e_hi = it.e_hi;
    }
  }
  const int64_t nch = (a.D + EPC - 1) / EPC, c = slab * 64 + lane;
  const bool cin = c < nch;
  const uint32_t coff = (uint32_t)(min(c, max(nch - 1, (int64_t)0)) * 16);  // the lane's chunk, kept inside the row
  const char* src = DEC ? a.g_xhat : a.xs;
  const int64_t st_bytes = (DEC ? a.sg : a.sx) * ES;
  const int64_t span = a.M > 0 ? (a.M - 1) * st_bytes + a.D * ES : 0;  // < 4 GB on the VEC path
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (int)(uint32_t)span,
                                                                     (int)BUF_W3);
  u32x4 wq[G];       // phase A, VEC: the items' W_dec[j] chunks (raw)
  float wf[G][EPC];  // phase A, otherwise: the same as fp32
#pragma unroll
  for (int g = 0; g < G; ++g) {
    wq[g] = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < EPC; ++e) wf[g][e] = 0.f;
    if constexpr (DEC) {
      if (g < ni && cin) {
        if constexpr (VEC) wq[g] = *(const u32x4*)(a.w_dec + ((int64_t)q_j[g] * a.sw + c * EPC) * ES);
        else load_chunk<DT, false>(a.w_dec + (int64_t)q_j[g] * a.sw * ES, c, a.D, wf[g]);
      }
    }
  }
  float acc[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
  float bsum = 0.f;  // db_enc partial (phase B, slab 0), the same in every lane
  // stores the head item's slab and db_enc share, then pops it
  auto flush = [&]() {
    if (cin) {
      if (DEC && q_slot[0] < 0) {
        store_chunk<DT, VEC>(a.d_wdec + (int64_t)q_j[0] * a.D * ES, c, a.D, acc);
      } else {
        float* pr = a.part + (int64_t)q_slot[0] * 2 * a.D + (DEC ? 0 : a.D);
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const int64_t d = c * EPC + e;
          if (d < a.D) pr[d] = acc[e];
        }
      }
    }
    if (!DEC && slab == 0 && lane == 0) a.part[a.n_slots * 2 * a.D + q_slot[0]] = bsum;
#pragma unroll
    for (int g = 0; g + 1 < G; ++g) {
      q_j[g] = q_j[g + 1];
      q_slot[g] = q_slot[g + 1];
      q_end[g] = q_end[g + 1];
      if constexpr (DEC) {
        wq[g] = wq[g + 1];
#pragma unroll
        for (int e = 0; e < EPC; ++e) wf[g][e] = wf[g + 1][e];
      }
    }
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
    bsum = 0.f;
  };
  for (int64_t k0 = e_lo; k0 < e_hi; k0 += 64) {
    const int kn = (int)min((int64_t)64, e_hi - k0);
    // f (phase A) or dL/dpre (phase B) of entry k0 + lane: the entry's row and its scalar (or,
    // phase A, the CSR position the scalar sits at) are loaded together, then checked (a lane
    // past the batch loads entry k0)
    const int64_t ke = k0 + (lane < kn ? lane : 0);
    const int32_t r = a.csc_row[ke];
    float my_s = 0.f;
    if constexpr (DEC) {
      const int32_t pos = a.csc_pos[ke];
      my_s = pos >= 0 && pos < a.nnz ? load_as_f32(a.values, a.val_dt, pos) : 0.f;
    } else {
      my_s = a.g_csc[ke];
    }
    const bool ok = lane < kn && r >= 0 && r < a.M;  // always in range, for a transpose made by sf_csr_transpose
    const int my_row = ok ? r : 0;
    my_s = ok ? my_s : 0.f;
    for (int kk = 0; kk < kn; kk += U) {
      int rows[U];
      float sv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int sl = min(kk + u, kn - 1);
        rows[u] = __builtin_amdgcn_readlane(my_row, sl);
        sv[u] = kk + u < kn ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_s), sl)) : 0.f;
      }
      u32x4 r[U];       // VEC: raw chunks
      float v[U][EPC];  // otherwise: elements
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (VEC) {
          r[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rs, (int)coff, (int)((uint32_t)rows[u] * (uint32_t)st_bytes), 0));
        } else if (cin) {
          load_chunk<DT, false>(src + (int64_t)rows[u] * st_bytes, c, a.D, v[u]);
        } else {
#pragma unroll
          for (int e = 0; e < EPC; ++e) v[u][e] = 0.f;
        }
      }
      float pd[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = kk + u < kn;  // wave-uniform
        if (live && k0 + kk + u >= q_end[0]) flush();
        if constexpr (DEC) {
          if constexpr (VEC) {
            pd[u] = cin ? chunk_dot<DT>(r[u], wq[0]) : 0.f;
          } else {
            pd[u] = 0.f;
#pragma unroll
            for (int e = 0; e < EPC; ++e) pd[u] = fmaf(v[u][e], wf[0][e], pd[u]);
          }
        } else if (slab == 0) {
          bsum += sv[u];
        }
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[e] = fmaf(sv[u], VEC ? chunk_elem<DT>(r[u], e) : v[u][e], acc[e]);
      }
      if constexpr (DEC) {
        const float sd = wave_sum8(pd, lane);  // entry kk + (lane >> 3)
        const int mine = kk + (lane >> 3);
        if ((lane & 7) == 0 && mine < kn) a.dots[slab * a.nnz + k0 + mine] = sd;
      }
    }
  }
  flush();  // the last item
}

// dL/dpre of CSC entry i: its slab shares of g_xhat[m] . W_dec[j] added in slab order, plus
// dL/df, where f > 0 (else 0), into g_csc[i] and into g_pre at the entry's CSR position.
__global__ __launch_bounds__(256) void gpre_kernel(ColArgs a, int64_t nslab) {
  const int64_t total = min(a.colptr[a.N], a.nnz);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int64_t sl = 0; sl < nslab; ++sl) s += a.dots[sl * a.nnz + i];
    const int32_t pos = a.csc_pos[i];
    float g = 0.f;
    if (pos >= 0 && pos < a.nnz) {
      if (a.g_val) s += load_as_f32(a.g_val, a.gval_dt, pos);
      g = load_as_f32(a.values, a.val_dt, pos) > 0.f ? s : 0.f;
      a.g_pre[pos] = g;
    }
    a.g_csc[i] = g;
  }
}

// Heavy columns (listed in multi_col, multi_off[N] of them): block (x, y) sums the partials of
// column multi_col[x] in chunk order for d in [y*256, (y+1)*256), one d per thread, into its
// dW_dec row and (fp32, for enc_tile_kernel) over the dW_enc^T half of its first slot, and
// its db_enc; a one-item heavy column needs only the db_enc copy.
template <int DT>
__global__ __launch_bounds__(256) void backward_reduce_kernel(ColArgs a, const int32_t* multi_col,
                                                              const int64_t* multi_off) {
  constexpr int ES = DT == SF_F32 ? 4 : 2;
  const int t = threadIdx.x;
  if ((int64_t)blockIdx.x >= multi_off[a.N]) return;  // the grid is a bound
  const int64_t j = multi_col[blockIdx.x];
  const int64_t s0 = a.part_off[j], ns = a.part_off[j + 1] - s0;
  const int64_t d = (int64_t)blockIdx.y * 256 + t;
  if (d < a.D && ns > 1) {  // a one-item column: dW_dec stored by phase A, its slot holds the sum
    float sd = 0.f, se = 0.f;
#pragma unroll 8
    for (int64_t s = 0; s < ns; ++s) {
      const float* pr = a.part + (s0 + s) * 2 * a.D;
      sd += pr[d];
      se += pr[a.D + d];
    }
    const uint32_t bd = f32_to_bits(sd, DT);
    if constexpr (ES == 4) ((uint32_t*)a.d_wdec)[j * a.D + d] = bd;
    else ((u16*)a.d_wdec)[j * a.D + d] = (u16)bd;
    a.part[s0 * 2 * a.D + a.D + d] = se;  // this thread read every slot's element d above
  }
  if (blockIdx.y == 0 && t == 0) {
    float sb = 0.f;
    for (int64_t s = 0; s < ns; ++s) sb += a.part[a.n_slots * 2 * a.D + s0 + s];
    a.d_benc[j] = sb;
  }
}

// A 16-B chunk of DT elements from EPC fp32 values.
template <int DT>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
  u32x4 q;
  if constexpr (DT == SF_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = __float_as_uint(v[e]);
  } else {
#pragma unroll
    for (int h = 0; h < 4; ++h) q[h] = f32_to_bits(v[2 * h], DT) | (f32_to_bits(v[2 * h + 1], DT) << 16);
  }
  return q;
}

__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// dW_enc [D, N] written in place of a dW_enc^T and a transpose: block x makes columns
// [x*TJ, +TJ) of every row, one slab (64 chunks of d) after another. Each of its 16 waves
// takes TILE_CPW consecutive columns. A light column (1..HEAVY entries) is summed here,
// dW_enc^T[j] = sum g_pre x'[m] on the slab and, on slab 0, db_enc[j] = sum g_pre, by one walk
// over the entries of the wave's light columns in CSC order, 64 at a time, U rows in flight,
// with a wave-uniform column change where a column's entries end; a heavy column's sum is the
// one backward_reduce_kernel left in its first slot, an unused column's is zero (and its dW_dec
// row and db_enc are zeroed here too: the work items cover only used columns). Each column's
// slab goes into an LDS row as DT, chunk k of row r at position k ^ (r / EPC) (which spreads
// the column reads below over the banks); after a barrier the block writes, for each d of the
// slab, the TJ consecutive elements of row d of dW_enc with 16-B stores (single elements on
// an edge tile or unaligned output). The column bounds and the first 64 entries of each walk
// are loaded once for all slabs. VEC gathers as backward_units_kernel does.
constexpr int TJ = 64, TILE_WAVES = 16, TILE_CPW = TJ / TILE_WAVES, TILE_THREADS = 64 * TILE_WAVES;
template <int DT, bool VEC>
__global__ __launch_bounds__(TILE_THREADS, VEC ? 8 : 4) void enc_tile_kernel(ColArgs a, int nslab, int out_vec,
                                                                     int dec_vec) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES, SD = 64 * EPC, U = 4;  // U: 64 VGPRs for 32 waves a CU
  typedef typename std::conditional<ES == 4, uint32_t, u16>::type T;
  __shared__ u32x4 tile[TJ * 64];
  auto lds_chunk = [&](int r, int k) -> u32x4& { return tile[r * 64 + (k ^ (r / EPC))]; };
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // block b takes column tile (b % 32) * Q + b / 32: the blocks in flight write 32 windows
  // spread over the whole width of the output rows, not one window (rows N elements apart,
  // 2 MB at d_sae = 2^20, would put one window of every row on the same few HBM channels)
  const int64_t ntiles = (a.N + TJ - 1) / TJ, Q = (ntiles + 31) / 32;
  const int64_t ct = (int64_t)(blockIdx.x % 32) * Q + blockIdx.x / 32;
  if (ct >= ntiles) return;  // the grid is 32 Q blocks
  const int64_t j0 = ct * TJ, jw = j0 + w * TILE_CPW;
  const int64_t nch = (a.D + EPC - 1) / EPC;
  // the wave's columns jw + q, described in lanes q < TILE_CPW
  int64_t lo = 0, slot = 0;
  int len = 0, heavy = 0, used = 1;  // used: a column past N is skipped like a used one
  if (lane < TILE_CPW && jw + lane < a.N) {
    lo = a.colptr[jw + lane];
    used = a.colptr[jw + lane + 1] > lo;
    slot = a.part_off[jw + lane];
    heavy = a.part_off[jw + lane + 1] > slot;
    len = heavy ? 0 : (int)(a.colptr[jw + lane + 1] - lo);
  }
  int64_t q_lo[TILE_CPW];
  int q_pre[TILE_CPW + 1];  // offsets of the columns' light entries in the wave's walk
  q_pre[0] = 0;
#pragma unroll
  for (int q = 0; q < TILE_CPW; ++q) {
    q_lo[q] = readlane_i64(lo, q);
    q_pre[q + 1] = q_pre[q] + __builtin_amdgcn_readlane(len, q);
  }
  const int L = q_pre[TILE_CPW];
  // walk entry k0 + lane: its token row and dL/dpre
  // (the row and the scalar are loaded together, then checked; a lane without an entry loads
  // entry 0, and with no entries at all, nnz = 0, nothing is loaded)
  auto entry = [&](int k0, int kn, int& my_row, float& my_s) {
    const int t = k0 + lane;
    int64_t base = 0;
#pragma unroll
    for (int q = 0; q < TILE_CPW; ++q)
      if (t >= q_pre[q]) base = q_lo[q] - q_pre[q];
    const int64_t i = base + t;
    const bool in = lane < kn && i >= 0 && i < a.nnz;  // always, for a transpose made by sf_csr_transpose
    int32_t r = 0;
    float sv = 0.f;
    if (a.nnz > 0) {  // uniform
      r = a.csc_row[in ? i : 0];
      sv = a.g_csc[in ? i : 0];
    }
    const bool ok = in && r >= 0 && r < a.M;
    my_row = ok ? r : 0;
    my_s = ok ? sv : 0.f;
  };
  int row0;
  float s0;
  entry(0, min(64, L), row0, s0);
  const int64_t st_bytes = a.sx * ES;
  const int64_t span = a.M > 0 ? (a.M - 1) * st_bytes + a.D * ES : 0;  // < 4 GB on the VEC path
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.xs, (short)0, (int)(uint32_t)span,
                                                                     (int)BUF_W3);
  const bool full_cols = out_vec && j0 + TJ <= a.N;
  for (int slab = 0; slab < nslab; ++slab) {
    const int64_t c = (int64_t)slab * 64 + lane;
    const bool cin = c < nch;
    const uint32_t coff = (uint32_t)(min(c, max(nch - 1, (int64_t)0)) * 16);
    // rows without light entries, and the queue of the others (column, end of its entries)
    int e_q[TILE_CPW], e_end[TILE_CPW], nq = 0;
#pragma unroll
    for (int q = 0; q < TILE_CPW; ++q) {
      e_q[q] = 0;
      e_end[q] = L;
    }
#pragma unroll
    for (int q = 0; q < TILE_CPW; ++q) {
      if (q_pre[q + 1] > q_pre[q]) {
#pragma unroll
        for (int p = 0; p < TILE_CPW; ++p) {
          if (p == nq) {
            e_q[p] = q;
            e_end[p] = q_pre[q + 1];
          }
        }
        ++nq;
      } else {
        u32x4 v = u32x4{0, 0, 0, 0};
        if (!__builtin_amdgcn_readlane(used, q)) {  // an unused column: zero dW_dec row and db_enc
          char* rowp = a.d_wdec + (jw + q) * a.D * ES;
          if (dec_vec) {
            if (cin) *(u32x4*)(rowp + c * 16) = v;
          } else {
            const float z[EPC] = {};
            store_chunk<DT, false>(rowp, c, a.D, z);
          }
          if (slab == 0 && lane == 0) a.d_benc[jw + q] = 0.f;
        } else if (__builtin_amdgcn_readlane(heavy, q) && cin) {
          const float* pr = a.part + readlane_i64(slot, q) * 2 * a.D + a.D;
          float f[EPC];
#pragma unroll
          for (int e = 0; e < EPC; ++e) f[e] = c * EPC + e < a.D ? pr[c * EPC + e] : 0.f;
          v = pack_chunk<DT>(f);
        }
        lds_chunk(w * TILE_CPW + q, lane) = v;
      }
    }
    float acc[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
    float bsum = 0.f;
    auto flush = [&]() {  // the head column's slab into its LDS row, then the next column
      lds_chunk(w * TILE_CPW + e_q[0], lane) = pack_chunk<DT>(acc);  // lanes past the row's end: never read
      if (slab == 0 && lane == 0) a.d_benc[jw + e_q[0]] = bsum;
#pragma unroll
      for (int p = 0; p + 1 < TILE_CPW; ++p) {
        e_q[p] = e_q[p + 1];
        e_end[p] = e_end[p + 1];
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
      bsum = 0.f;
    };
    for (int k0 = 0; k0 < L; k0 += 64) {
      const int kn = min(64, L - k0);
      int my_row = row0;
      float my_s = s0;
      if (k0 > 0) entry(k0, kn, my_row, my_s);
      for (int kk = 0; kk < kn; kk += U) {
        int rows[U];
        float sv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int sl = min(kk + u, kn - 1);
          rows[u] = __builtin_amdgcn_readlane(my_row, sl);
          sv[u] = kk + u < kn ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_s), sl)) : 0.f;
        }
        u32x4 r[U];
        float v[U][EPC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if constexpr (VEC) {
            r[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rs, (int)coff, (int)((uint32_t)rows[u] * (uint32_t)st_bytes), 0));
          } else if (cin) {
            load_chunk<DT, false>(a.xs + (int64_t)rows[u] * st_bytes, c, a.D, v[u]);
          } else {
#pragma unroll
            for (int e = 0; e < EPC; ++e) v[u][e] = 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (kk + u < kn && k0 + kk + u >= e_end[0]) flush();  // wave-uniform
          bsum += sv[u];
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[e] = fmaf(sv[u], VEC ? chunk_elem<DT>(r[u], e) : v[u][e], acc[e]);
        }
      }
    }
    if (L > 0) flush();
    __syncthreads();
    const int64_t d0 = (int64_t)slab * SD;
    if (full_cols && d0 + SD <= a.D) {
      if constexpr (ES == 2) {  // chunk k (columns 8k..8k+7) of output rows d0 + 2e and d0 + 2e + 1
#pragma unroll
        for (int i = 0; i < SD / 2 * (TJ / 8) / TILE_THREADS; ++i) {
          const int idx = threadIdx.x + TILE_THREADS * i, k = idx & 7, e = idx >> 3;
          uint32_t wv[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) wv[q] = lds_chunk(8 * k + q, e >> 2)[e & 3];
          u32x4 o0, o1;
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            o0[h] = (wv[2 * h] & 0xffffu) | (wv[2 * h + 1] << 16);
            o1[h] = (wv[2 * h] >> 16) | (wv[2 * h + 1] & 0xffff0000u);
          }
          char* o = a.d_wenc + ((d0 + 2 * e) * a.N + j0 + 8 * k) * ES;
          *(u32x4*)o = o0;
          *(u32x4*)(o + a.N * ES) = o1;
        }
      } else {  // chunk k (columns 4k..4k+3) of output row d0 + d
#pragma unroll
        for (int i = 0; i < SD * (TJ / 4) / TILE_THREADS; ++i) {
          const int idx = threadIdx.x + TILE_THREADS * i, k = idx & 15, d = idx >> 4;
          u32x4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = lds_chunk(4 * k + q, d >> 2)[d & 3];
          *(u32x4*)(a.d_wenc + ((d0 + d) * a.N + j0 + 4 * k) * ES) = o;
        }
      }
    } else {
      for (int idx = threadIdx.x; idx < TJ * SD; idx += TILE_THREADS) {
        const int col = idx % TJ, d = idx / TJ;
        if (j0 + col < a.N && d0 + d < a.D)
          ((T*)a.d_wenc)[(d0 + d) * a.N + j0 + col] = ((const T*)&lds_chunk(col, d / EPC))[d % EPC];
      }
    }
    __syncthreads();  // the next slab rewrites the tile
  }
}

// The work plan's per-column counts, scanned without materialising them: array 0 = work items
// ceil(n / CHUNK) (0 for an unused column, which enc_tile_kernel handles), 1 = partial slots
// (the items of a heavy column: more than HEAVY entries), 2 = 1 for a heavy column. All three are
// scanned by one three-pass tiled scan (grid y = the array) into plan_i64 [3][N+1]: tile totals
// parked in out[tile*PLAN_TILE + 1], turned into tile offsets by one block per array, then
// each tile writes its inclusive prefixes.
constexpr int PLAN_PER = 16, PLAN_TILE = 256 * PLAN_PER;

__device__ __forceinline__ int64_t plan_tile_counts(const int64_t* colptr, int64_t N, int64_t i0, int which,
                                                    int32_t (&c)[PLAN_PER]) {
  int64_t s = 0;
#pragma unroll
  for (int q = 0; q < PLAN_PER; ++q) {
    const int64_t j = i0 + q;
    int64_t k = 0;
    if (j < N) {
      const int64_t n = colptr[j + 1] - colptr[j];
      k = n > 0 ? (n + CHUNK - 1) / CHUNK : 0;
      if (n <= HEAVY && which > 0) k = 0;
    }
    c[q] = (int32_t)(which == 2 ? (k > 0) : k);
    s += c[q];
  }
  return s;
}

__global__ __launch_bounds__(256) void plan_tiles_kernel(const int64_t* colptr, int64_t N, int64_t* out) {
  __shared__ int64_t s_w[4];
  const int which = blockIdx.y;
  const int64_t i0 = (int64_t)blockIdx.x * PLAN_TILE + threadIdx.x * PLAN_PER;
  int32_t c[PLAN_PER];
  const int64_t s = plan_tile_counts(colptr, N, i0, which, c);
  int64_t total;
  block_exclusive_i64(s, s_w, total);
  if (threadIdx.x == 0) out[which * (N + 1) + (int64_t)blockIdx.x * PLAN_TILE + 1] = total;
}

__global__ __launch_bounds__(256) void plan_totals_kernel(int64_t ntiles, int64_t N, int64_t* out) {
  __shared__ int64_t s_w[4];
  int64_t* o = out + blockIdx.x * (N + 1);
  int64_t carry = 0;
  for (int64_t b0 = 0; b0 < ntiles; b0 += 256) {
    const int64_t b = b0 + threadIdx.x;
    const int64_t v = b < ntiles ? o[b * PLAN_TILE + 1] : 0;
    int64_t total;
    const int64_t ex = block_exclusive_i64(v, s_w, total);
    if (b < ntiles) o[b * PLAN_TILE + 1] = carry + ex;
    carry += total;
    __syncthreads();  // s_w is rewritten by the next round
  }
}

__global__ __launch_bounds__(256) void plan_final_kernel(const int64_t* colptr, int64_t N, int64_t* out,
                                                         int has_offsets) {
  __shared__ int64_t s_w[4];
  __shared__ int64_t s_off;
  const int which = blockIdx.y;
  int64_t* o = out + which * (N + 1);
  const int64_t i0 = (int64_t)blockIdx.x * PLAN_TILE + threadIdx.x * PLAN_PER;
  if (threadIdx.x == 0) s_off = has_offsets ? o[(int64_t)blockIdx.x * PLAN_TILE + 1] : 0;
  int32_t c[PLAN_PER];
  const int64_t s = plan_tile_counts(colptr, N, i0, which, c);
  int64_t total;
  int64_t run = block_exclusive_i64(s, s_w, total) + s_off;  // the barrier inside orders s_off
#pragma unroll
  for (int q = 0; q < PLAN_PER; ++q) {
    run += c[q];
    if (i0 + q < N) o[i0 + q + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) o[0] = 0;
}

// item_col[item_off[j] + q] = j for every work item q of column j; slot_item[part_off[j] + q]
// = item_off[j] + q for the items of a heavy column; multi_col lists the heavy columns in
// increasing order.
__global__ __launch_bounds__(256) void item_table_kernel(const int64_t* plan_i64, int64_t N, int32_t* item_col,
                                                         int32_t* multi_col, int32_t* slot_item) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  const int64_t *item_off = plan_i64, *part_off = plan_i64 + (N + 1), *multi_off = plan_i64 + 2 * (N + 1);
  const int64_t i0 = item_off[j];
  for (int64_t i = i0; i < item_off[j + 1]; ++i) item_col[i] = (int32_t)j;
  for (int64_t s = part_off[j]; s < part_off[j + 1]; ++s) slot_item[s] = (int32_t)(i0 + s - part_off[j]);
  if (multi_off[j + 1] > multi_off[j]) multi_col[multi_off[j]] = (int32_t)j;
}

// --------------------------------------------------------------------------- transpose, sums
// dst[c, r] = src[r, c] for a [R, C] source of row stride ss (elements); TR x 64 tiles (TR
// source rows: 256 for 16-bit types, 128 for fp32) through LDS. A full tile with 16-B aligned
// rows on both sides moves 16-B chunks: each thread loads TR/32 source chunks, then gathers
// TR/32 output chunks from LDS columns, so each output row gets a TR-element contiguous
// segment; other tiles move single elements. The source-row tile is the fast grid axis: the
// blocks in flight write different column windows of the output rows rather than one window
// of many output rows R elements apart (with R a power of two those fall on a few HBM
// channels). At d_sae = 2^20 (dW_enc^T -> dW_enc, rows 2 MB apart) 64 x 64 tiles in the other
// order took 2.1 ms.
template <int ES>
constexpr int tr_rows() { return ES == 4 ? 128 : 256; }

template <int ES>
__global__ __launch_bounds__(256) void transpose_kernel(const char* src, int64_t R, int64_t C, int64_t ss,
                                                        char* dst, int vec, const int64_t* skip_ptr) {
  typedef typename std::conditional<ES == 4, uint32_t, u16>::type T;
  constexpr int TR = tr_rows<ES>(), EPC = 16 / ES, CPR = 64 / EPC, PITCH = 64 + 2;  // pitch: spreads column reads over banks
  constexpr int OCR = TR / EPC;  // output chunks per output row of the tile
  __shared__ T tile[TR * PITCH];
  const int t = threadIdx.x, tx = t & 63, ty = t >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * TR, c0 = (int64_t)blockIdx.y * 64;
  const T* s = (const T*)src;
  T* d = (T*)dst;
  // skip_ptr (optional): source row r is all zeros, and is not read, when skip_ptr[r+1] ==
  // skip_ptr[r] (a feature without entries, whose gradient row was never written)
  auto row_used = [&](int64_t r) { return skip_ptr == nullptr || skip_ptr[r + 1] != skip_ptr[r]; };
  if (vec && r0 + TR <= R && c0 + 64 <= C) {
    u32x4 v[TR * CPR / 256];
#pragma unroll
    for (int i = 0; i < TR * CPR / 256; ++i) {
      const int idx = t + 256 * i, r = idx / CPR, k = idx % CPR;
      v[i] = row_used(r0 + r) ? *(const u32x4*)(s + (r0 + r) * ss + c0 + k * EPC) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < TR * CPR / 256; ++i) {
      const int idx = t + 256 * i, r = idx / CPR, k = idx % CPR;
      const T* e = (const T*)&v[i];
#pragma unroll
      for (int q = 0; q < EPC; ++q) tile[r * PITCH + k * EPC + q] = e[q];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 64 * OCR / 256; ++i) {
      const int idx = t + 256 * i, c = idx / OCR, k = idx % OCR;  // output row c, chunk k
      u32x4 o;
      T* e = (T*)&o;
#pragma unroll
      for (int q = 0; q < EPC; ++q) e[q] = tile[(k * EPC + q) * PITCH + c];
      *(u32x4*)(d + (c0 + c) * R + r0 + k * EPC) = o;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TR / 4; ++i) {
    const int r = ty + 4 * i;
    if (r0 + r < R && c0 + tx < C) tile[r * PITCH + tx] = row_used(r0 + r) ? s[(r0 + r) * ss + c0 + tx] : (T)0;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = ty + 4 * i;
#pragma unroll
    for (int h = 0; h < TR / 64; ++h) {
      const int r = h * 64 + tx;
      if (c0 + c < C && r0 + r < R) d[(c0 + c) * R + r0 + r] = tile[r * PITCH + c];
    }
  }
}

// out[r] = sign * sum_c W[r, c] v[c] (+ out[r] when accumulate), fp32, for W of row stride swr
// and column stride swc. Block b sums the columns [p*cols_per, ...) of the MV_RB rows
// [g*MV_RB, ...), g = b / nparts, p = b % nparts, into part[r, p]: a thread loads a chunk of v
// once and the same chunk of every row of its group (16-B loads when VEC: unit column stride,
// aligned rows), so v is read once per row group rather than once per row. Consecutive blocks
// take consecutive column ranges of the same rows, so the blocks in flight read whole rows
// rather than one narrow column window of many rows (which would load only the few HBM channels
// that window maps to). Rows past R load row R-1 and are not stored. matvec_final_kernel adds
// a row's partials in order.
constexpr int MV_RB = 8;
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void matvec_kernel(const char* W, int64_t R, int64_t C, int64_t swr,
                                                     int64_t swc, const float* v, int64_t cols_per, int64_t nparts,
                                                     float* part) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  __shared__ float s_w[MV_RB][4];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)(blockIdx.x / nparts) * MV_RB, p = blockIdx.x % nparts;
  const int64_t c0 = p * cols_per, c1 = min(C, c0 + cols_per);
  const char* rows[MV_RB];
#pragma unroll
  for (int i = 0; i < MV_RB; ++i) rows[i] = W + min(r0 + i, R - 1) * swr * ES;
  float acc[MV_RB];
#pragma unroll
  for (int i = 0; i < MV_RB; ++i) acc[i] = 0.f;
  if constexpr (VEC) {  // cols_per and C are multiples of EPC, v is 16-B aligned
    const int64_t ce = c1 / EPC;
    for (int64_t ch = c0 / EPC + t; ch < ce; ch += 2 * 256) {  // two chunks a trip: 2*MV_RB raw loads in flight
      const bool two = ch + 256 < ce;
      const int64_t chs[2] = {ch, two ? ch + 256 : ch};  // a second chunk past the range reloads the first, unused
      float vv[2][EPC];
      u32x4 w[2][MV_RB];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int q = 0; q < EPC / 4; ++q) {
          const float4 f = *(const float4*)(v + chs[h] * EPC + 4 * q);
          vv[h][4 * q] = f.x; vv[h][4 * q + 1] = f.y; vv[h][4 * q + 2] = f.z; vv[h][4 * q + 3] = f.w;
        }
#pragma unroll
        for (int i = 0; i < MV_RB; ++i) w[h][i] = *(const u32x4*)(rows[i] + chs[h] * 16);
      }
#pragma unroll
      for (int i = 0; i < MV_RB; ++i)
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[i] = fmaf(chunk_elem<DT>(w[0][i], e), vv[0][e], acc[i]);
      if (two) {
#pragma unroll
        for (int i = 0; i < MV_RB; ++i)
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[i] = fmaf(chunk_elem<DT>(w[1][i], e), vv[1][e], acc[i]);
      }
    }
  } else {
    for (int64_t c = c0 + t; c < c1; c += 256) {
      const float vc = v[c];
      float w[MV_RB];
#pragma unroll
      for (int i = 0; i < MV_RB; ++i) w[i] = load_as_f32(rows[i], DT, c * swc);
#pragma unroll
      for (int i = 0; i < MV_RB; ++i) acc[i] = fmaf(w[i], vc, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < MV_RB; ++i) acc[i] = wave_sum(acc[i]);
  if ((t & 63) == 0) {
#pragma unroll
    for (int i = 0; i < MV_RB; ++i) s_w[i][t >> 6] = acc[i];
  }
  __syncthreads();
  if (t < MV_RB && r0 + t < R) part[(r0 + t) * nparts + p] = s_w[t][0] + s_w[t][1] + s_w[t][2] + s_w[t][3];
}

__global__ __launch_bounds__(256) void matvec_final_kernel(const float* part, int64_t R, int64_t nparts, float sign,
                                                           int accumulate, float* out) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= R) return;
  float s = 0.f;
  for (int64_t p = 0; p < nparts; ++p) s += part[r * nparts + p];
  out[r] = accumulate ? out[r] + sign * s : sign * s;
}

// Column sums of A [M, D] (row stride sa, unit column stride), each row optionally weighted by
// w[m] (fp32), in fp32. Block (x, y) covers the columns [x*64*EPC, ...), EPC per lane (one 16-B
// load per row when VEC), and the rows [y*rows_per, ...); its 4 waves take every 4th row, CS_U
// rows in flight, and their sums are added in wave order into part[y, D]. col_sums_final adds
// the partials in order (deterministic).
constexpr int CS_U = 8;
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void col_sums_kernel(const char* A, int64_t M, int64_t D, int64_t sa,
                                                       const float* w, int64_t rows_per, float* part) {
  constexpr int ES = DT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  __shared__ float s_part[3][64 * EPC];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t ch = (int64_t)blockIdx.x * 64 + lane;
  const bool live = ch * EPC < D;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
  const int64_t chc = live ? ch : 0;  // dead lanes load chunk 0 and discard it
  float s[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) s[e] = 0.f;
  int64_t r = r0 + wv;
  for (; r + 4 * (CS_U - 1) < r1; r += 4 * CS_U) {
    float a[CS_U][EPC];
#pragma unroll
    for (int u = 0; u < CS_U; ++u) load_chunk<DT, VEC>(A + (r + 4 * u) * sa * ES, chc, D, a[u]);
#pragma unroll
    for (int u = 0; u < CS_U; ++u) {
      const float wu = w ? w[r + 4 * u] : 1.f;
#pragma unroll
      for (int e = 0; e < EPC; ++e) s[e] = fmaf(wu, a[u][e], s[e]);
    }
  }
  for (; r < r1; r += 4) {
    float a[EPC];
    load_chunk<DT, VEC>(A + r * sa * ES, chc, D, a);
    const float wu = w ? w[r] : 1.f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) s[e] = fmaf(wu, a[e], s[e]);
  }
  if (wv > 0) {
#pragma unroll
    for (int e = 0; e < EPC; ++e) s_part[wv - 1][lane * EPC + e] = s[e];
  }
  __syncthreads();
  if (wv == 0 && live) {
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int64_t d = ch * EPC + e;
      if (d < D) part[blockIdx.y * D + d] = ((s[e] + s_part[0][lane * EPC + e]) + s_part[1][lane * EPC + e]) +
                                            s_part[2][lane * EPC + e];
    }
  }
}

// out[d] = sign * sum_p part[p, d] (+ out[d] when accumulate). Block x covers the columns
// [x*64, ...); wave q adds the partials p = q, q+4, ... and the 4 waves' sums are added in
// order.
__global__ __launch_bounds__(256) void col_sums_final_kernel(const float* part, int64_t nparts, int64_t D,
                                                             float sign, float* out, int accumulate) {
  __shared__ float s_part[3][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t d = (int64_t)blockIdx.x * 64 + lane;
  const int64_t dc = d < D ? d : D - 1;
  float s = 0.f;
#pragma unroll 8
  for (int64_t p = wv; p < nparts; p += 4) s += part[p * D + dc];
  if (wv > 0) s_part[wv - 1][lane] = s;
  __syncthreads();
  if (wv == 0 && d < D) {
    s = ((s + s_part[0][lane]) + s_part[1][lane]) + s_part[2][lane];
    out[d] = accumulate ? out[d] + sign * s : sign * s;
  }
}

bool aligned16(const void* p, int64_t stride_elems, int es) {
  return ((uintptr_t)p % 16) == 0 && ((stride_elems * es) % 16) == 0;
}

constexpr int64_t GRID_BLOCKS = 2048;  // blocks of the grid-stride backward kernels (8 per CU)

// Work items per wave of backward_units_kernel. Measured on MI355X (bf16, d_in 2304): at 16
// entries per feature (d_sae 65536, 16384 tokens, L0 64) one item per wave is fastest (four:
// phase A 0.74 -> 0.88 ms, phase B 0.69 -> 0.77: the queue's registers cost occupancy); at 0.5
// (d_sae 2^20, 4096 tokens, L0 128) four are (phase A 1.27 -> 0.77 ms, phase B 0.84 -> 0.55).
constexpr int units_per_wave(int64_t nnz, int64_t N) { return nnz < 4 * N ? 4 : 1; }

template <int DT, bool VEC, bool DEC, int G>
void launch_units_g(const ColArgs& a, int64_t nslab, hipStream_t s) {
  const int64_t units = ((DEC ? a.n_items : a.n_slots) + G - 1) / G * nslab;
  if (units == 0) return;
  hipLaunchKernelGGL((backward_units_kernel<DT, VEC, 8, DEC, G, !DEC>), dim3((unsigned)((units + WPB - 1) / WPB)),
                     dim3(256), 0, s, a, (int)nslab);
}

// phase A over every work item, phase B over the heavy columns' items (one per wave)
template <int DT, bool VEC, bool DEC>
void launch_units(const ColArgs& a, int64_t nslab, hipStream_t s) {
  if constexpr (DEC) {
    if (units_per_wave(a.nnz, a.N) == 4) {
      launch_units_g<DT, VEC, DEC, 4>(a, nslab, s);
      return;
    }
  }
  launch_units_g<DT, VEC, DEC, 1>(a, nslab, s);
}

template <int DT>
void launch_tile(const ColArgs& a, bool vec, int out_vec, int dec_vec, int64_t nslab, hipStream_t s) {
  const dim3 grid((unsigned)(((a.N + TJ - 1) / TJ + 31) / 32 * 32));
  if (vec) hipLaunchKernelGGL((enc_tile_kernel<DT, true>), grid, dim3(TILE_THREADS), 0, s, a, (int)nslab, out_vec, dec_vec);
  else hipLaunchKernelGGL((enc_tile_kernel<DT, false>), grid, dim3(TILE_THREADS), 0, s, a, (int)nslab, out_vec, dec_vec);
}

template <bool DEC>
void launch_units_dt(const ColArgs& a, int dt, bool vec, int64_t nslab, hipStream_t s) {
  switch (dt) {
    case SF_BF16: vec ? launch_units<SF_BF16, true, DEC>(a, nslab, s) : launch_units<SF_BF16, false, DEC>(a, nslab, s); break;
    case SF_F16: vec ? launch_units<SF_F16, true, DEC>(a, nslab, s) : launch_units<SF_F16, false, DEC>(a, nslab, s); break;
    default: vec ? launch_units<SF_F32, true, DEC>(a, nslab, s) : launch_units<SF_F32, false, DEC>(a, nslab, s); break;
  }
}

// Slabs of 64 16-B chunks covering a D-wide row (at least 1).
int64_t slabs_for(int64_t D, int es) { return std::max<int64_t>(1, ((D + 16 / es - 1) / (16 / es) + 63) / 64); }

}  // namespace

// Workspace of the counting sort: hist int32 [nb*S], offs int64 [nb*S + 1], then (row,
// position, low bits) int32 [nnz] each; of the fallback: counts int32 [N], then (row,
// position) int32 [nnz] each.
static int64_t round256(int64_t n) { return (n + 255) / 256 * 256; }

extern "C" int sf_csr_transpose_workspace_size(int64_t M, int64_t N, int64_t nnz, int64_t* bytes) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0 && nnz >= 0 && bytes, "sf_csr_transpose_workspace_size: bad arguments");
  if (csc_sorts(N)) {
    const CscPlan p = csc_plan(M, N);
    const int64_t cells = (int64_t)p.nb * p.S;
    *bytes = round256(4 * cells) + round256(8 * (cells + 1)) + 3 * round256(4 * nnz);
  } else {
    *bytes = 4 * (N + 2 * nnz) + 256;
  }
  return SF_OK;
}

extern "C" int sf_csr_transpose(const int64_t* indptr, const int32_t* indices, int64_t M, int64_t N, int64_t nnz,
                                int64_t* colptr, int32_t* csc_row, int32_t* csc_pos, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0 && nnz >= 0, "sf_csr_transpose: negative size");
  SF_REQUIRE(M < (1LL << 31) && nnz < (1LL << 31) && N < (1LL << 31), "sf_csr_transpose: size too large");
  SF_REQUIRE(csc_sorts(N) || M <= (1LL << 18),
             "sf_csr_transpose: beyond 2^23 columns at most 2^18 rows (the per-column row bitmap lives in LDS)");
  SF_REQUIRE(colptr && (N == 0 || M == 0 || indptr), "sf_csr_transpose: NULL buffer");
  int64_t need = 0;
  sf_csr_transpose_workspace_size(M, N, nnz, &need);
  SF_REQUIRE(workspace && workspace_bytes >= need, "sf_csr_transpose: workspace of %lld bytes, need %lld",
             (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  if (M == 0 || nnz == 0 || N == 0) {  // every column empty
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>((2 * N + 257) / 256, 4096))),
                       dim3(256), 0, s, (int32_t*)colptr, 2 * (N + 1), 0);
    SF_LAUNCH_CHECK("fill_i32_kernel");
    return SF_OK;
  }
  SF_REQUIRE(indices && csc_row && csc_pos, "sf_csr_transpose: NULL buffer");
  if (csc_sorts(N)) {
    const CscPlan p = csc_plan(M, N);
    const int64_t cells = (int64_t)p.nb * p.S;
    char* w = (char*)workspace;
    int32_t* hist = (int32_t*)w;
    int64_t* offs = (int64_t*)(w + round256(4 * cells));
    int32_t* t_row = (int32_t*)(w + round256(4 * cells) + round256(8 * (cells + 1)));
    int32_t* t_pos = (int32_t*)((char*)t_row + round256(4 * nnz));
    int32_t* t_low = (int32_t*)((char*)t_pos + round256(4 * nnz));
    const unsigned blocks = (unsigned)((p.S + 3) / 4);
    const size_t lds13 = (size_t)4 * 4 * p.nb;
    hipLaunchKernelGGL(csc_count_kernel, dim3(blocks), dim3(256), lds13, s, indptr, indices, M, N, nnz, p.LB, p.nb,
                       p.RW, p.S, hist);
    SF_LAUNCH_CHECK("csc_count_kernel");
    int rc = sf_scan_counts(hist, cells, offs, stream);
    if (rc != SF_OK) return rc;
    hipLaunchKernelGGL(csc_bucket_kernel, dim3(blocks), dim3(256), lds13, s, indptr, indices, M, N, nnz, p.LB, p.nb,
                       p.nb_bits, p.RW, p.S, offs, t_row, t_pos, t_low);
    SF_LAUNCH_CHECK("csc_bucket_kernel");
    hipLaunchKernelGGL(csc_sort_kernel, dim3((unsigned)p.nb), dim3(256), (size_t)4 * 4 * (1 << p.LB), s, offs, p.S,
                       p.nb, p.LB, N, nnz, t_row, t_pos, t_low, colptr, csc_row, csc_pos);
    SF_LAUNCH_CHECK("csc_sort_kernel");
    return SF_OK;
  }
  // beyond 2^23 columns: atomic counts and placement, then a per-column ordering pass
  int32_t* counts = (int32_t*)workspace;
  int32_t* tmp_row = counts + N;
  int32_t* tmp_pos = tmp_row + nnz;
  const unsigned fill_grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((N + 255) / 256, 4096));
  hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_grid), dim3(256), 0, s, counts, N, 0);
  SF_LAUNCH_CHECK("fill_i32_kernel");
  const unsigned rows_grid = (unsigned)((M + WPB - 1) / WPB);
  hipLaunchKernelGGL(col_count_kernel, dim3(rows_grid), dim3(256), 0, s, indptr, indices, M, N, nnz, counts);
  SF_LAUNCH_CHECK("col_count_kernel");
  int rc = sf_scan_counts(counts, N, colptr, stream);
  if (rc != SF_OK) return rc;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_grid), dim3(256), 0, s, counts, N, 0);
  SF_LAUNCH_CHECK("fill_i32_kernel");
  hipLaunchKernelGGL(col_place_kernel, dim3(rows_grid), dim3(256), 0, s, indptr, indices, M, N, nnz, colptr, counts,
                     tmp_row, tmp_pos);
  SF_LAUNCH_CHECK("col_place_kernel");
  const size_t lds = (size_t)2 * 4 * ((M + 31) / 32);
  hipLaunchKernelGGL(col_sort_kernel, dim3((unsigned)N), dim3(256), lds, s, colptr, M, tmp_row, tmp_pos, csc_row,
                     csc_pos);
  SF_LAUNCH_CHECK("col_sort_kernel");
  return SF_OK;
}

extern "C" int sf_backward_bounds(int64_t N, int64_t nnz, int64_t D, int dt, int64_t* max_items, int64_t* max_slots,
                                  int64_t* work_floats) {
  sf_clear_error();
  SF_REQUIRE(N >= 0 && nnz >= 0 && D >= 0 && sf_valid_dtype(dt) && max_items && max_slots && work_floats,
             "sf_backward_bounds: bad arguments");
  *max_items = std::min(N, nnz) + nnz / CHUNK + 1;
  // a heavy column of n > HEAVY entries has ceil(n / CHUNK) <= n / (HEAVY + 1) slots
  *max_slots = nnz / (HEAVY + 1) + 1;
  *work_floats = (slabs_for(D, sf_dtype_size(dt)) + 1) * nnz;
  return SF_OK;
}

extern "C" int sf_backward_plan(const int64_t* colptr, int64_t N, int64_t nnz, int64_t* plan_i64, int32_t* item_col,
                                int32_t* multi_col, int32_t* slot_item, void* stream) {
  sf_clear_error();
  SF_REQUIRE(N >= 0 && nnz >= 0, "sf_backward_plan: bad arguments");
  if (N == 0) return SF_OK;
  SF_REQUIRE(colptr && plan_i64 && item_col && multi_col && slot_item, "sf_backward_plan: NULL buffer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t ntiles = (N + PLAN_TILE - 1) / PLAN_TILE;
  SF_REQUIRE(ntiles < (1LL << 31), "sf_backward_plan: too many columns");
  if (ntiles > 1) {
    hipLaunchKernelGGL(plan_tiles_kernel, dim3((unsigned)ntiles, 3), dim3(256), 0, s, colptr, N, plan_i64);
    SF_LAUNCH_CHECK("plan_tiles_kernel");
    hipLaunchKernelGGL(plan_totals_kernel, dim3(3), dim3(256), 0, s, ntiles, N, plan_i64);
    SF_LAUNCH_CHECK("plan_totals_kernel");
  }
  hipLaunchKernelGGL(plan_final_kernel, dim3((unsigned)ntiles, 3), dim3(256), 0, s, colptr, N, plan_i64,
                     (int)(ntiles > 1));
  SF_LAUNCH_CHECK("plan_final_kernel");
  hipLaunchKernelGGL(item_table_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, s, plan_i64, N, item_col,
                     multi_col, slot_item);
  SF_LAUNCH_CHECK("item_table_kernel");
  return SF_OK;
}

extern "C" int sf_shifted_input(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* b_dec, int bdec_dt,
                                int64_t M, int64_t D, int dt, void* xs, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && D >= 0, "sf_shifted_input: negative size");
  SF_REQUIRE(sf_valid_dtype(x_dt) && sf_valid_dtype(bdec_dt) && sf_valid_dtype(dt), "sf_shifted_input: bad dtype");
  if (M == 0 || D == 0) return SF_OK;
  SF_REQUIRE(x && b_dec && xs, "sf_shifted_input: NULL buffer");
  const unsigned g = (unsigned)std::min<int64_t>(8192, (M * D + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  const int es = sf_dtype_size(dt);
  if (x_dt == dt && sxk == 1 && D % (16 / es) == 0 && aligned16(x, sxm, es) && aligned16(xs, D, es) &&
      (M + SH_R - 1) / SH_R < 65536) {
    const dim3 vg((unsigned)((D / (16 / es) + 63) / 64), (unsigned)((M + SH_R - 1) / SH_R));
    switch (dt) {
      case SF_BF16: hipLaunchKernelGGL(shift_vec_kernel<SF_BF16>, vg, dim3(256), 0, s, (const char*)x, sxm, b_dec, bdec_dt, M, D, (char*)xs); break;
      case SF_F16: hipLaunchKernelGGL(shift_vec_kernel<SF_F16>, vg, dim3(256), 0, s, (const char*)x, sxm, b_dec, bdec_dt, M, D, (char*)xs); break;
      default: hipLaunchKernelGGL(shift_vec_kernel<SF_F32>, vg, dim3(256), 0, s, (const char*)x, sxm, b_dec, bdec_dt, M, D, (char*)xs); break;
    }
    SF_LAUNCH_CHECK("shift_vec_kernel");
    return SF_OK;
  }
  switch (dt) {
    case SF_BF16: hipLaunchKernelGGL(shift_kernel<SF_BF16>, dim3(g), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt, M, D, (char*)xs); break;
    case SF_F16: hipLaunchKernelGGL(shift_kernel<SF_F16>, dim3(g), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt, M, D, (char*)xs); break;
    default: hipLaunchKernelGGL(shift_kernel<SF_F32>, dim3(g), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt, M, D, (char*)xs); break;
  }
  SF_LAUNCH_CHECK("shift_kernel");
  return SF_OK;
}

extern "C" int sf_backward_columns(const int64_t* colptr, const int32_t* csc_row, const int32_t* csc_pos,
                                   const int64_t* plan_i64, const int32_t* item_col, const int32_t* multi_col,
                                   const int32_t* slot_item, int64_t max_items, int64_t max_slots, const void* values, int val_dt,
                                   const void* g_val, int gval_dt, const void* w_dec, int64_t sw, const void* xs,
                                   int64_t sx, const void* g_xhat, int64_t sg, int dt, int64_t N, int64_t M, int64_t D,
                                   int64_t nnz, float* g_pre, void* d_wdec, void* d_wenc, float* d_benc,
                                   float* partials, float* work, int64_t work_floats, void* stream) {
  sf_clear_error();
  SF_REQUIRE(N >= 0 && M >= 0 && D >= 0 && nnz >= 0 && max_items >= 0 && max_slots >= 0,
             "sf_backward_columns: negative size");
  SF_REQUIRE(sf_valid_dtype(val_dt) && sf_valid_dtype(dt) && (g_val == nullptr || sf_valid_dtype(gval_dt)),
             "sf_backward_columns: bad dtype");
  SF_REQUIRE(nnz < (1LL << 31) && D < (1LL << 24), "sf_backward_columns: nnz or D too large");
  const int es = sf_dtype_size(dt);
  const int64_t nslab = slabs_for(D, es);
  // every argument is checked before the first launch
  SF_REQUIRE(nnz == 0 || g_pre, "sf_backward_columns: NULL g_pre");
  if (N > 0) {
    SF_REQUIRE(max_items * nslab < 0x7fffffffLL && max_slots * nslab < 0x7fffffffLL && (N + TJ - 1) / TJ < 0x7fffff00LL,
               "sf_backward_columns: too many work items");
    SF_REQUIRE(colptr && plan_i64 && item_col && multi_col && slot_item && (D == 0 || d_wenc) && d_wdec && d_benc,
               "sf_backward_columns: NULL buffer");
    SF_REQUIRE(nnz == 0 || (csc_row && csc_pos && values && work && partials && (D == 0 || (w_dec && xs && g_xhat))),
               "sf_backward_columns: NULL buffer");
    SF_REQUIRE(work_floats >= (nslab + 1) * nnz, "sf_backward_columns: work of %lld floats, need %lld",
               (long long)work_floats, (long long)((nslab + 1) * nnz));
  }
  hipStream_t s = (hipStream_t)stream;
  if (nnz > 0) {  // entries outside [0, N) keep g_pre = 0
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)std::min<int64_t>(4096, (nnz + 255) / 256)), dim3(256), 0, s,
                       (int32_t*)g_pre, nnz, 0);
    SF_LAUNCH_CHECK("fill_i32_kernel");
  }
  if (N == 0) return SF_OK;
  const int64_t* item_off = plan_i64;
  const int64_t* slot_off = plan_i64 + (N + 1);
  const int64_t* multi_off = plan_i64 + 2 * (N + 1);
  ColArgs a;
  a.colptr = colptr; a.csc_row = csc_row; a.csc_pos = csc_pos; a.item_off = item_off; a.part_off = slot_off;
  a.item_col = item_col; a.slot_item = slot_item; a.n_items = max_items; a.values = values; a.val_dt = val_dt;
  a.g_val = g_val; a.gval_dt = gval_dt; a.w_dec = (const char*)w_dec; a.sw = sw;
  a.xs = (const char*)xs; a.sx = sx; a.g_xhat = (const char*)g_xhat; a.sg = sg;
  a.N = N; a.M = M; a.D = D; a.nnz = nnz;
  a.dots = work; a.g_csc = work ? work + nslab * nnz : nullptr; a.g_pre = g_pre;
  a.d_wdec = (char*)d_wdec; a.d_wenc = (char*)d_wenc; a.d_benc = d_benc;
  a.part = partials; a.n_slots = max_slots;
  const int64_t span_x = M > 0 ? ((M - 1) * sx + D) * es : 0, span_g = M > 0 ? ((M - 1) * sg + D) * es : 0;
  const bool vec = D % (16 / es) == 0 && aligned16(xs, sx, es) && aligned16(g_xhat, sg, es) &&
                   aligned16(w_dec, sw, es) && aligned16(d_wdec, D, es) &&
                   span_x < (1LL << 32) && span_g < (1LL << 32);  // the per-row gathers are buffer loads
  if (nnz > 0) {
    launch_units_dt<true>(a, dt, vec, nslab, s);
    SF_LAUNCH_CHECK("backward_units_kernel (dW_dec)");
    hipLaunchKernelGGL(gpre_kernel, dim3((unsigned)std::min<int64_t>(GRID_BLOCKS, (nnz + 255) / 256)), dim3(256), 0, s,
                       a, nslab);
    SF_LAUNCH_CHECK("gpre_kernel");
    launch_units_dt<false>(a, dt, vec, nslab, s);
    SF_LAUNCH_CHECK("backward_units_kernel (dW_enc)");
  }
  // heavy columns: at most max_slots (each has a slot)
  const dim3 gr((unsigned)std::max<int64_t>(1, std::min<int64_t>(N, max_slots)),
                (unsigned)std::max<int64_t>(1, (D + 255) / 256));
  switch (dt) {
    case SF_BF16: hipLaunchKernelGGL(backward_reduce_kernel<SF_BF16>, gr, dim3(256), 0, s, a, multi_col, multi_off); break;
    case SF_F16: hipLaunchKernelGGL(backward_reduce_kernel<SF_F16>, gr, dim3(256), 0, s, a, multi_col, multi_off); break;
    default: hipLaunchKernelGGL(backward_reduce_kernel<SF_F32>, gr, dim3(256), 0, s, a, multi_col, multi_off); break;
  }
  SF_LAUNCH_CHECK("backward_reduce_kernel");
  {  // with D = 0 it still zeroes db_enc of the unused columns
    const int out_vec = D > 0 && aligned16(d_wenc, N, es), dec_vec = aligned16(d_wdec, D, es);
    switch (dt) {
      case SF_BF16: launch_tile<SF_BF16>(a, vec, out_vec, dec_vec, nslab, s); break;
      case SF_F16: launch_tile<SF_F16>(a, vec, out_vec, dec_vec, nslab, s); break;
      default: launch_tile<SF_F32>(a, vec, out_vec, dec_vec, nslab, s); break;
    }
    SF_LAUNCH_CHECK("enc_tile_kernel");
  }
  return SF_OK;
}

extern "C" int sf_transpose(const void* src, int64_t R, int64_t C, int64_t ss, int dt, const int64_t* skip_ptr,
                            void* dst, void* stream) {
  sf_clear_error();
  SF_REQUIRE(R >= 0 && C >= 0 && sf_valid_dtype(dt), "sf_transpose: bad arguments");
  if (R == 0 || C == 0) return SF_OK;
  SF_REQUIRE(src && dst, "sf_transpose: NULL buffer");
  const int64_t tr = dt == SF_F32 ? tr_rows<4>() : tr_rows<2>();
  SF_REQUIRE((C + 63) / 64 < 65536 && (R + tr - 1) / tr < (1LL << 31), "sf_transpose: too many columns");
  const dim3 grid((unsigned)((R + tr - 1) / tr), (unsigned)((C + 63) / 64));
  hipStream_t s = (hipStream_t)stream;
  const int es = sf_dtype_size(dt);
  const int vec = aligned16(src, ss, es) && aligned16(dst, R, es);
  if (es == 4)
    hipLaunchKernelGGL(transpose_kernel<4>, grid, dim3(256), 0, s, (const char*)src, R, C, ss, (char*)dst, vec,
                       skip_ptr);
  else
    hipLaunchKernelGGL(transpose_kernel<2>, grid, dim3(256), 0, s, (const char*)src, R, C, ss, (char*)dst, vec,
                       skip_ptr);
  SF_LAUNCH_CHECK("transpose_kernel");
  return SF_OK;
}

// Weighted or plain column sums of A [M, D] (row stride sa, unit column stride) into out.
static int column_sums(const void* A, int64_t M, int64_t D, int64_t sa, int dt, const float* w, float sign,
                       int accumulate, float* out, float* workspace, int64_t workspace_floats, hipStream_t s,
                       const char* who) {
  const int64_t nparts = std::max<int64_t>(1, std::min<int64_t>(256, M));
  SF_REQUIRE(workspace_floats >= nparts * D, "%s: workspace of %lld floats, need %lld", who,
             (long long)workspace_floats, (long long)(nparts * D));
  const int es = sf_dtype_size(dt), epc = 16 / es;
  if (M > 0) {
    const bool vec = D % epc == 0 && aligned16(A, sa, es);
    const int64_t rows_per = (M + nparts - 1) / nparts;
    const dim3 grid((unsigned)((D + 64 * epc - 1) / (64 * epc)), (unsigned)nparts);
    const char* a = (const char*)A;
#define SF_CS(DTV, VECV) hipLaunchKernelGGL((col_sums_kernel<DTV, VECV>), grid, dim3(256), 0, s, a, M, D, sa, w, rows_per, workspace)
    switch (dt) {
      case SF_BF16: if (vec) SF_CS(SF_BF16, true); else SF_CS(SF_BF16, false); break;
      case SF_F16: if (vec) SF_CS(SF_F16, true); else SF_CS(SF_F16, false); break;
      default: if (vec) SF_CS(SF_F32, true); else SF_CS(SF_F32, false); break;
    }
#undef SF_CS
    SF_LAUNCH_CHECK("col_sums_kernel");
  } else {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, (int32_t*)workspace, D,
                       0);
    SF_LAUNCH_CHECK("fill_i32_kernel");
  }
  hipLaunchKernelGGL(col_sums_final_kernel, dim3((unsigned)((D + 63) / 64)), dim3(256), 0, s, workspace,
                     M > 0 ? nparts : 1, D, sign, out, accumulate);
  SF_LAUNCH_CHECK("col_sums_final_kernel");
  return SF_OK;
}

extern "C" int sf_column_sums(const void* A, int64_t M, int64_t D, int64_t sa, int dt, float sign, int accumulate,
                              float* out, float* workspace, int64_t workspace_floats, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && D >= 0 && sf_valid_dtype(dt), "sf_column_sums: bad arguments");
  if (D == 0) return SF_OK;
  SF_REQUIRE(out && (M == 0 || (A && workspace)), "sf_column_sums: NULL buffer");
  return column_sums(A, M, D, sa, dt, nullptr, sign, accumulate, out, workspace, workspace_floats,
                     (hipStream_t)stream, "sf_column_sums");
}

extern "C" int sf_matvec(const void* W, int64_t R, int64_t C, int64_t swr, int64_t swc, int w_dt, const float* v,
                         float sign, int accumulate, float* out, float* workspace, int64_t workspace_floats,
                         void* stream) {
  sf_clear_error();
  SF_REQUIRE(R >= 0 && C >= 0 && sf_valid_dtype(w_dt), "sf_matvec: bad arguments");
  SF_REQUIRE(R < (1LL << 31), "sf_matvec: too many rows");
  if (R == 0) return SF_OK;
  SF_REQUIRE(out && (C == 0 || (W && v)) && workspace, "sf_matvec: NULL buffer");
  hipStream_t s = (hipStream_t)stream;
  if (swc != 1 && swr == 1 && C > 0)  // column-contiguous W: the v-weighted column sums of W^T [C, R]
    return column_sums(W, C, R, swc, w_dt, v, sign, accumulate, out, workspace, workspace_floats, s, "sf_matvec");
  const int64_t nparts = std::max<int64_t>(1, std::min<int64_t>(64, (C + 8191) / 8192));
  SF_REQUIRE(workspace_floats >= R * nparts, "sf_matvec: workspace of %lld floats, need %lld",
             (long long)workspace_floats, (long long)(R * nparts));
  const int es = sf_dtype_size(w_dt), epc = 16 / es;
  const bool vec = swc == 1 && C % epc == 0 && aligned16(W, swr, es) && ((uintptr_t)v % 16) == 0;
  const int64_t cols_per = ((C + nparts - 1) / nparts + epc - 1) / epc * epc;
  const char* w = (const char*)W;
  const int64_t blocks = (R + MV_RB - 1) / MV_RB * nparts;
  SF_REQUIRE(blocks < (1LL << 24), "sf_matvec: %lld rows is too many", (long long)R);
  const dim3 grid((unsigned)blocks);
#define SF_MV(DTV, VECV) hipLaunchKernelGGL((matvec_kernel<DTV, VECV>), grid, dim3(256), 0, s, w, R, C, swr, swc, v, cols_per, nparts, workspace)
  switch (w_dt) {
    case SF_BF16: if (vec) SF_MV(SF_BF16, true); else SF_MV(SF_BF16, false); break;
    case SF_F16: if (vec) SF_MV(SF_F16, true); else SF_MV(SF_F16, false); break;
    default: if (vec) SF_MV(SF_F32, true); else SF_MV(SF_F32, false); break;
  }
#undef SF_MV
  SF_LAUNCH_CHECK("matvec_kernel");
  hipLaunchKernelGGL(matvec_final_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, s, workspace, R, nparts,
                     sign, accumulate, out);
  SF_LAUNCH_CHECK("matvec_final_kernel");
  return SF_OK;
}
