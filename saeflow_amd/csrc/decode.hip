// Sparse CSR decode on gfx950: out[m] = b_dec + sum_j values[j] * W_dec[indices[j]], fp32
// accumulation. Reference semantics: _decode_kernel and sparse_decode
// (saeflow/kernels/decode.py:28-55, :97-120).
//
// Decode is a gather, not a dense contraction, so it stays off the matrix cores. Three kernels:
//
// decode_lines_kernel (rows of whole 128-B lines, the default): W_dec is cut into column
// slabs of one or two 128-B lines each, and the (slab, token block) units are split evenly
// over the 8 XCDs in slab-major order, so each XCD's L2 serves the rows of one slab at a
// time: a d_sae x 128 B (or 256 B) working set instead of whole 4.6 KB rows of every feature
// (at d_sae = 65536 the L2-miss traffic falls ~3x). A group of 8 (or 16) lanes owns one token
// (16 B of the slab per lane, 8 or 4 tokens per wavefront): its
// lanes fetch R of the token's (index, value) pairs each, then walk them in CSR order in
// fully unrolled rounds of U rows, the row index moved to the group with ds_bpermute and the
// next round's rows loaded before this round's FMAs. While W_dec is below 2 GiB the rows are
// read through a structured buffer resource (the hardware forms base + row * stride, and a
// row index past d_sae reads zeros, so padding pairs need neither address arithmetic nor a
// branch); larger W_dec uses 64-bit addressed loads.
//
// decode_vec_kernel (any 16-B aligned shape): one wavefront owns one output row (or one
// 512-chunk slab of it when d_in is wide). The row's pairs are fetched 64 at a time and
// broadcast with readlane, which makes every gathered W_dec row address wave-uniform; each
// lane streams its 16-B chunks of U rows at once (U*NC loads in flight per lane).
//
// decode_generic_kernel (any strides or alignment): the same walk, element by element.
//
// All three accumulate per lane in fp32 over the row's entries in CSR order, so they give
// bit-identical results. A padding pair or an invalid index reads no W_dec row and adds
// 0 * 0, as the reference's masked load does (decode.py:46-50).
#include <algorithm>

#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WPB = 4;       // waves (rows) per block
constexpr int MAX_NC = 8;    // 16-B chunks per lane per slab

struct DecArgs {
  const int64_t* indptr;
  const int32_t* indices;
  const void* values;
  int val_dt;
  int64_t nnz;
  const char* w;
  int64_t swn, swd;
  int64_t d_sae;
  const void* b_dec;
  int bdec_dt;
  char* out;
  int64_t som, sod;
  int out_dt;
  int64_t M, D;
  int vec_out;  // out row-contiguous and 16-B aligned
};

template <int WDT>
__device__ __forceinline__ float welem(const u32x4& c, int e) {
  if constexpr (WDT == SF_F32) return __uint_as_float(c[e]);
  else {
    uint32_t h = (c[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
    return WDT == SF_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  }
}

// Fetch this row's entries [j0, j0+64) into one lane each; invalid entries get value 0 and
// row -1, which the kernels skip (no W_dec row is read for them). The index and the value
// are loaded together (a lane past the batch loads entry j0), then checked.
__device__ __forceinline__ void fetch_batch(const DecArgs& a, int64_t j0, int64_t jn, int lane, int& idx,
                                            float& val) {
  const int64_t p = j0 + (lane < jn ? lane : 0);
  const int32_t c = a.indices[p];
  const float v = load_as_f32(a.values, a.val_dt, p);
  const bool ok = lane < jn && c >= 0 && c < a.d_sae;
  idx = ok ? c : -1;  // an invalid entry: no row is read for it
  val = ok ? v : 0.f;
}

__device__ __forceinline__ void row_range(const DecArgs& a, int64_t row, int64_t& lo, int64_t& hi) {
  lo = a.indptr[row];
  hi = a.indptr[row + 1];
  lo = lo < 0 ? 0 : (lo > a.nnz ? a.nnz : lo);
  hi = hi < lo ? lo : (hi > a.nnz ? a.nnz : hi);
}

// Store output chunk d0 .. d0+EPC-1 of `row` (fp32 sums + b_dec, cast to the output type):
// one 16-B store when the output is row-contiguous, aligned and of W_dec's width, else
// element by element through the strides.
template <int ES>
__device__ __forceinline__ void store_chunk(const DecArgs& a, int64_t row, int64_t d0, const float* acc) {
  constexpr int EPC = 16 / ES;
  const int oes = sf_dtype_size(a.out_dt);
  uint32_t bits[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    float o = acc[e];
    if (a.b_dec) o += load_as_f32(a.b_dec, a.bdec_dt, d0 + e);
    bits[e] = f32_to_bits(o, a.out_dt);
  }
  if (a.vec_out && oes == ES) {
    u32x4 c;
    if constexpr (ES == 2) {
#pragma unroll
      for (int d = 0; d < 4; ++d) c[d] = bits[2 * d] | (bits[2 * d + 1] << 16);
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) c[d] = bits[d];
    }
    *(u32x4*)(a.out + (row * a.som + d0) * oes) = c;
  } else {
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      char* p = a.out + (row * a.som + (d0 + e) * a.sod) * oes;
      if (oes == 2) *(u16*)p = (u16)bits[e];
      else *(uint32_t*)p = bits[e];
    }
  }
}

// vector path: W_dec rows contiguous and 16-B aligned, D % EPC == 0
template <int WDT, int NC, int U>
__global__ __launch_bounds__(256) void decode_vec_kernel(DecArgs a) {
  constexpr int ES = WDT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int64_t nch = a.D / EPC;                   // chunks per row
  const int64_t ch0 = (int64_t)blockIdx.y * 64 * NC;  // first chunk of this slab
  int64_t lo, hi;
  row_range(a, row, lo, hi);

  float acc[NC][EPC];
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[i][e] = 0.f;

  bool ok[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) ok[i] = ch0 + i * 64 + lane < nch;

  for (int64_t j0 = lo; j0 < hi; j0 += 64) {
    const int jn = (int)min((int64_t)64, hi - j0);
    int my_idx;
    float my_val;
    fetch_batch(a, j0, jn, lane, my_idx, my_val);
    for (int jj = 0; jj < jn; jj += U) {
      u32x4 w[U][NC];
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int src = min(jj + u, jn - 1);
        const int r = __builtin_amdgcn_readlane(my_idx, src);
        // a pair past the batch or with an invalid index multiplies 0 by 0, never by a W_dec
        // value (0 * inf would be NaN; decode.py:46-50 masks the load the same way)
        const bool live = jj + u < jn && r >= 0;  // wave-uniform
        v[u] = live ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_val), src)) : 0.f;
        const char* wr = a.w + ((int64_t)(live ? r : 0) * a.swn + ch0 * EPC) * ES;
#pragma unroll
        for (int i = 0; i < NC; ++i)
          w[u][i] = live && ok[i] ? *(const u32x4*)(wr + (int64_t)(i * 64 + lane) * 16) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < NC; ++i)
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[i][e] = fmaf(v[u], welem<WDT>(w[u][i], e), acc[i][e]);
    }
  }

#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (ok[i]) store_chunk<ES>(a, row, (ch0 + i * 64 + lane) * EPC, acc[i]);
}

// Line-slab path: rows of D*ES bytes = S whole 128-B lines (S = D*ES/128), 16-B aligned.
// Units (slab, token block) are numbered slab-major and XCD x (hardware workgroup ids
// b = x mod 8) takes units [x*per, (x+1)*per). A slab is SL lines (1 or 2); a workgroup's 4
// wavefronts hold 8 / SL tokens each, one per group of 8 * SL lanes; lane li of group g sums
// chunk li of the slab for its token.
// (pairs per lane per batch, rows per round) of the buffer-resource and the plain-load
// kernels, from sweeps at C1-C5: the buffer kernel's lighter rounds leave registers for 6
// wavefronts per SIMD; the plain kernel's 64-bit addresses need larger rounds to keep loads
// in flight.
constexpr int LR_BUF = 4, LU_BUF = 4;
constexpr int LR_BUF2 = 4, LU_BUF2 = 2;  // two-line slabs: rounds of 2 rows (C3 2-3% faster than 4)
constexpr int LR_GLB = 10, LU_GLB = 4;
constexpr int LG = 8;   // tokens per wavefront with one-line slabs

struct LineArgs {
  DecArgs d;
  int64_t ntb;  // token blocks of WPB * LG / SL tokens
  int64_t per;  // units per XCD
  int64_t tot;  // slabs * ntb
};

// BUF: W_dec is read through a structured buffer resource (row index -> address in the
// hardware, out-of-range rows read zeros), which needs all of W_dec below 2 GiB (the
// hardware's index * stride offset is 32-bit); otherwise plain 64-bit-addressed loads.
// LR (index, value) pairs per lane per batch (8 * LR per token), LU gathered rows per round,
// two rounds in flight per lane.
template <int WDT, bool BUF, int LR, int LU, int SL>
__global__ __launch_bounds__(256) void decode_lines_kernel(LineArgs la) {
  constexpr int ES = WDT == SF_F32 ? 4 : 2, EPC = 16 / ES;
  constexpr int L = 8 * SL, B = LR * L;  // lanes per token (16 B each), pairs per batch
  constexpr int LGT = 64 / L;           // tokens per wavefront
  static_assert(B % LU == 0, "rounds of LU pairs tile a batch");
  const DecArgs& a = la.d;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / L, li = lane % L;
  const int xcd = blockIdx.x & 7;
  const int64_t unit = (int64_t)xcd * la.per + (blockIdx.x >> 3);
  if (unit >= min((int64_t)(xcd + 1) * la.per, la.tot)) return;  // whole workgroup
  const int64_t slab = unit / la.ntb;
  const int64_t row = ((unit - slab * la.ntb) * WPB + wv) * LGT + g;
  const bool tok_on = row < a.M;
  int64_t lo = 0, hi = 0;
  if (tok_on) row_range(a, row, lo, hi);
  const int64_t n = hi - lo;
  int64_t nmax = n;  // the wavefront walks its longest token's pairs
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) nmax = max(nmax, (int64_t)__shfl_xor((long long)nmax, o));
  // equal in every lane: taken from lane 0 so the batch and round bounds are scalar (a row
  // holds at most nnz < 2^31 entries: the launcher takes this kernel only then)
  nmax = __builtin_amdgcn_readfirstlane((int)nmax);

  float acc[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
  const int64_t ch = slab * 8 * SL + li;  // this lane's 16-B chunk of every row
  // The slab as a structured buffer: record r is W_dec row r (stride swn * ES bytes), the
  // lane's chunk at offset 16 * li; a record index at or past d_sae reads zeros and touches
  // no memory, which is how padding and invalid pairs add nothing.
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + slab * 128 * SL), (short)(a.swn * ES), (int)a.d_sae, (int)SF_RSRC_W3);
  const char* wcol = a.w + ch * 16;
  constexpr int NR = B / LU;  // rounds of a batch

  for (int64_t j0 = 0; j0 < nmax; j0 += B) {
    // lane li holds pairs j0 + r*L + li of its token. Every index and value load is issued
    // before any is used (a pair past the token's end loads pair 0, in bounds since nnz > 0
    // here), so the batch costs one memory latency, not a chain of them.
    int32_t craw[LR];
    uint32_t vraw[LR];
#pragma unroll
    for (int r = 0; r < LR; ++r) {
      const int64_t j = j0 + r * L + li;
      craw[r] = a.indices[j < n ? lo + j : 0];
    }
    if (a.val_dt == SF_F32) {
#pragma unroll
      for (int r = 0; r < LR; ++r) {
        const int64_t j = j0 + r * L + li;
        vraw[r] = ((const uint32_t*)a.values)[j < n ? lo + j : 0];
      }
    } else {
#pragma unroll
      for (int r = 0; r < LR; ++r) {
        const int64_t j = j0 + r * L + li;
        vraw[r] = ((const u16*)a.values)[j < n ? lo + j : 0];
      }
    }
    // a pair past the token's end, or with an index outside [0, d_sae), gathers record -1
    // (zeros) with value 0: acc + 0 * 0 == acc exactly, as acc is never -0 (it starts at +0
    // and x + (-x) rounds to +0)
    int idx[LR];
    float val[LR];
#pragma unroll
    for (int r = 0; r < LR; ++r) {
      const bool ok = j0 + r * L + li < n && craw[r] >= 0 && craw[r] < a.d_sae;
      const float v = a.val_dt == SF_F32 ? __uint_as_float(vraw[r])
                                         : (a.val_dt == SF_BF16 ? bf16_to_f32(vraw[r]) : f16_to_f32(vraw[r]));
      idx[r] = ok ? craw[r] : -1;
      val[r] = ok ? v : 0.f;
    }
    const int bn = (int)min((int64_t)B, nmax - j0);
    // Round k gathers pairs k*LU .. k*LU+LU-1 (the row index and value moved to the group's
    // lanes with ds_bpermute); round k+1's gathers are issued before round k's FMAs.
    u32x4 wb[2][LU];
    float vb[2][LU];
    auto issue = [&](int e0, u32x4 (&w)[LU], float (&v)[LU]) {
#pragma unroll
      for (int u = 0; u < LU; ++u) {
        const int e = e0 + u;
        const int src = (g * L + e % L) * 4;  // the lane of the group holding pair e
        const int r = __builtin_amdgcn_ds_bpermute(src, idx[e / L]);
        v[u] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(val[e / L])));
        if constexpr (BUF) {
          w[u] = sf_struct_load_b128(wr, r, li * 16, 0, 0);
        } else {
          w[u] = r >= 0 ? *(const u32x4*)(wcol + (int64_t)r * a.swn * ES) : u32x4{0, 0, 0, 0};
        }
      }
    };
    issue(0, wb[0], vb[0]);
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      if (k * LU < bn) {
        if (k + 1 < NR && (k + 1) * LU < bn) issue((k + 1) * LU, wb[(k + 1) & 1], vb[(k + 1) & 1]);
#pragma unroll
        for (int u = 0; u < LU; ++u)
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[e] = fmaf(vb[k & 1][u], welem<WDT>(wb[k & 1][u], e), acc[e]);
      }
    }
  }
  if (tok_on) store_chunk<ES>(a, row, ch * EPC, acc);
}

// generic path: any W_dec strides/alignment, any D. Lane owns elements lane + 64 i of
// a 512-element slab.
template <int WDT>
__global__ __launch_bounds__(256) void decode_generic_kernel(DecArgs a) {
  constexpr int NE = 8;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int64_t d0 = (int64_t)blockIdx.y * 64 * NE;
  int64_t lo, hi;
  row_range(a, row, lo, hi);
  float acc[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) acc[i] = 0.f;
  for (int64_t j0 = lo; j0 < hi; j0 += 64) {
    const int jn = (int)min((int64_t)64, hi - j0);
    int my_idx;
    float my_val;
    fetch_batch(a, j0, jn, lane, my_idx, my_val);
    for (int jj = 0; jj < jn; ++jj) {
      const int r = __builtin_amdgcn_readlane(my_idx, jj);
      if (r < 0) continue;  // an invalid index adds nothing (wave-uniform)
      const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_val), jj));
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        int64_t d = d0 + i * 64 + lane;
        if (d < a.D) acc[i] = fmaf(v, load_as_f32(a.w, WDT, (int64_t)r * a.swn + d * a.swd), acc[i]);
      }
    }
  }
  const int oes = sf_dtype_size(a.out_dt);
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    int64_t d = d0 + i * 64 + lane;
    if (d >= a.D) continue;
    float o = acc[i];
    if (a.b_dec) o += load_as_f32(a.b_dec, a.bdec_dt, d);
    uint32_t b = f32_to_bits(o, a.out_dt);
    char* p = a.out + (row * a.som + d * a.sod) * oes;
    if (oes == 2) *(u16*)p = (u16)b;
    else *(uint32_t*)p = b;
  }
}

template <int WDT, int NC>
hipError_t launch_vec(const DecArgs& a, dim3 grid, hipStream_t s) {
  constexpr int U = NC <= 4 ? 4 : (NC <= 6 ? 3 : 2);
  hipLaunchKernelGGL((decode_vec_kernel<WDT, NC, U>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// nc_cfg: chunks per lane of a slab (1..MAX_NC) asked for by tile_cfg, 0 = from D.
template <int WDT>
hipError_t launch_wdt(const DecArgs& a, bool vec, int nc_cfg, hipStream_t s) {
  const unsigned gx = (unsigned)((a.M + WPB - 1) / WPB);
  if (!vec) {
    dim3 grid(gx, (unsigned)((a.D + 511) / 512));
    hipLaunchKernelGGL((decode_generic_kernel<WDT>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
  }
  constexpr int EPC = WDT == SF_F32 ? 4 : 8;
  const int64_t nch = a.D / EPC;
  // whole 128-B lines per row: the line-slab kernel. Slabs of two lines (16 lanes per token)
  // when the row holds an even number of lines and d_sae <= 65536: each slab pass reads the
  // CSR again, and two lines per pass halve that while the pair's working set per XCD stays
  // small (C3: 16 MB); at 131072 features and more the doubled working set costs more (C4,
  // C5). Rows read through a structured buffer while they fit its record (14-bit stride)
  // and W_dec stays below 2 GiB, else with 64-bit addresses.
  constexpr int ES = WDT == SF_F32 ? 4 : 2;
  // (the line-slab kernel keeps a wavefront's longest row length in 32 bits: nnz < 2^31)
  if (nc_cfg == 0 && nch % 8 == 0 && a.swn >= 0 && a.d_sae <= 0x7fffffffLL && a.nnz < (1LL << 31)) {
    const int sl = nch % 16 == 0 && a.d_sae <= 65536 ? 2 : 1;
    LineArgs la;
    la.d = a;
    const int tpb = WPB * LG / sl;  // tokens per workgroup
    la.ntb = (a.M + tpb - 1) / tpb;
    la.tot = nch / (8 * sl) * la.ntb;
    la.per = (la.tot + 7) / 8;
    if (la.per * 8 <= 0x7fffffffLL) {  // else the grid would not fit: the row kernel below
      const bool buf = a.swn * ES <= 16383 && a.d_sae * a.swn * ES < (1LL << 31);
      const dim3 grid((unsigned)(la.per * 8)), block(256);
      if (buf && sl == 2)
        hipLaunchKernelGGL((decode_lines_kernel<WDT, true, LR_BUF2, LU_BUF2, 2>), grid, block, 0, s, la);
      else if (buf)
        hipLaunchKernelGGL((decode_lines_kernel<WDT, true, LR_BUF, LU_BUF, 1>), grid, block, 0, s, la);
      else if (sl == 2)
        hipLaunchKernelGGL((decode_lines_kernel<WDT, false, LR_GLB, LU_GLB, 2>), grid, block, 0, s, la);
      else
        hipLaunchKernelGGL((decode_lines_kernel<WDT, false, LR_GLB, LU_GLB, 1>), grid, block, 0, s, la);
      return hipGetLastError();
    }
  }
  // chunks per lane of a slab: the whole row in one slab when it fits MAX_NC, else MAX_NC
  int nc = (int)std::min<int64_t>((nch + 63) / 64, MAX_NC);
  if (nc_cfg > 0) nc = std::min(nc, nc_cfg);
  const int64_t slab = 64 * (int64_t)nc;
  const unsigned gy = (unsigned)((nch + slab - 1) / slab);
  dim3 grid(gx, gy);
  switch (nc) {
    case 1: return launch_vec<WDT, 1>(a, grid, s);
    case 2: return launch_vec<WDT, 2>(a, grid, s);
    case 3: return launch_vec<WDT, 3>(a, grid, s);
    case 4: return launch_vec<WDT, 4>(a, grid, s);
    case 5: return launch_vec<WDT, 5>(a, grid, s);
    case 6: return launch_vec<WDT, 6>(a, grid, s);
    case 7: return launch_vec<WDT, 7>(a, grid, s);
    default: return launch_vec<WDT, 8>(a, grid, s);
  }
}

}  // namespace

extern "C" int sf_decode(const int64_t* indptr, const int32_t* indices, const void* values, int val_dt, int64_t nnz,
                         const void* w_dec, int64_t swn, int64_t swd, int w_dt, int64_t d_sae, const void* b_dec,
                         int bdec_dt, void* out, int64_t som, int64_t sod, int out_dt, int64_t M, int64_t D,
                         const int32_t* tile_cfg, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && D >= 0 && nnz >= 0 && d_sae >= 0, "sf_decode: negative size");
  SF_REQUIRE(sf_valid_dtype(val_dt) && sf_valid_dtype(w_dt) && sf_valid_dtype(out_dt) &&
                 (b_dec == nullptr || sf_valid_dtype(bdec_dt)),
             "sf_decode: bad dtype code");
  if (M == 0 || D == 0) return SF_OK;
  SF_REQUIRE(indptr && out && w_dec, "sf_decode: NULL buffer");
  SF_REQUIRE(nnz == 0 || (indices && values), "sf_decode: NULL indices/values");
  SF_REQUIRE(M <= (int64_t)WPB * 0x7fffffffLL, "sf_decode: M too large");
  int nc_cfg = 0;
  if (tile_cfg) {
    SF_REQUIRE(tile_cfg[0] > 0 && tile_cfg[1] > 0, "sf_decode: tile config {BLOCK_NNZ=%d, BLOCK_D=%d} must be positive",
               tile_cfg[0], tile_cfg[1]);
    const int64_t per_chunk_row = 64LL * (16 / sf_dtype_size(w_dt));  // elements of one chunk per lane
    nc_cfg = (int)std::min<int64_t>((tile_cfg[1] + per_chunk_row - 1) / per_chunk_row, MAX_NC);
  }
  DecArgs a;
  a.indptr = indptr; a.indices = indices; a.values = values; a.val_dt = val_dt; a.nnz = nnz;
  a.w = (const char*)w_dec; a.swn = swn; a.swd = swd; a.d_sae = d_sae;
  a.b_dec = b_dec; a.bdec_dt = bdec_dt;
  a.out = (char*)out; a.som = som; a.sod = sod; a.out_dt = out_dt;
  a.M = M; a.D = D;
  if (d_sae == 0) a.nnz = 0;  // no valid index: no W_dec row may be touched
  const int es = sf_dtype_size(w_dt), epc = 16 / es;
  const int oes = sf_dtype_size(out_dt);
  a.vec_out = sod == 1 && ((uintptr_t)out % 16) == 0 && ((som * oes) % 16) == 0;
  const bool vec = swd == 1 && ((uintptr_t)w_dec % 16) == 0 && ((swn * es) % 16) == 0 && (D % epc) == 0;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (w_dt) {
    case SF_BF16: e = launch_wdt<SF_BF16>(a, vec, nc_cfg, s); break;
    case SF_F16: e = launch_wdt<SF_F16>(a, vec, nc_cfg, s); break;
    default: e = launch_wdt<SF_F32>(a, vec, nc_cfg, s); break;
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "sf_decode: kernel launch failed: %s", hipGetErrorString(e));
  return SF_OK;
}
