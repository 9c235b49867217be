// Fused SAE encoder on gfx950 MFMA:  out = act((x - b_dec) @ W + b_enc), fp32 accumulate,
// with per-row nonzero counting in the epilogue.
//
// Reference semantics: saeflow/kernels/encode.py:36-91 (kernel) and :97-139 (wrapper).
//
// Design (one workgroup = one 256x256 output tile, 4 waves of 128x128):
//  * MFMA operands are swapped: the matrix-core "A" operand is a W^T row block (n, k) and
//    "B" is an x' row block (m, k), so each lane's accumulator holds one token row m and
//    four runs of 4 consecutive features n: the epilogue stores 4 features per instruction
//    and reduces row counts with a single cross-half exchange.
//  * Global -> VGPR -> LDS staging, double-buffered (2 x 64 KiB).  The staging step is the
//    prologue: x' = cast(fp32(x) - fp32(b_dec)) is formed in registers (encode.py:72), and a
//    feature-contiguous W (the SAELens layout, W_enc [d_in, d_sae] row-major) is transposed
//    8x8 in registers so LDS always holds K-contiguous rows for both operands.
//  * LDS rows are 128 B (BK*esize) in 16 B chunks, XOR-swizzled by row so that both the
//    ds_read_b128 fragment reads and the transposed ds_write_b128 stores are bank-conflict
//    free.
//  * Tile order is XCD-aware: consecutive hardware workgroup ids land on different XCDs
//    (round-robin), so ids are remapped to give each XCD a contiguous run of tiles, and the
//    run is walked in GROUP_M-row groups so a W column block is reused from that XCD's L2.
#include "common.h"

namespace {

constexpr int BM = 256, BN = 256;   // output tile (tokens x features)
constexpr int NT = 256;             // threads per workgroup (4 waves)
constexpr int ROWB = 128;           // bytes per LDS row = BK * element size
constexpr int TILE_BYTES = 256 * ROWB;  // one operand tile in LDS: 32 KiB

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int DT> struct Traits;
template <> struct Traits<SF_BF16> { static constexpr int E = 2, EPC = 8, BK = 64; };
template <> struct Traits<SF_F16> { static constexpr int E = 2, EPC = 8, BK = 64; };
template <> struct Traits<SF_F32> { static constexpr int E = 4, EPC = 4, BK = 32; };

enum WPath { W_NMAJOR = 0, W_KMAJOR = 1, W_GENERIC = 2 };

struct EncArgs {
  const void* x;
  int64_t sxm, sxk;
  int x_dt;
  const void* w;
  int64_t swk, swn;
  const void* b_enc;
  int benc_dt;
  const void* b_dec;
  int bdec_dt;
  const void* thr;
  int thr_dt;
  void* out;
  int64_t som, son;
  int out_dt;
  int32_t* row_nnz;
  int64_t M, N, K;
  int act;
  int tiles_m, tiles_n, group_m;
  int vec_store;  // out row-contiguous and 8/16-B aligned rows
};

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int row, int kc) { return row * ROWB + ((kc ^ swz(row)) << 4); }

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

// fp32 -> bits of the MFMA input type
template <int DT>
__device__ __forceinline__ uint32_t to_in_bits(float v) {
  if constexpr (DT == SF_F32) return __float_as_uint(v);
  else if constexpr (DT == SF_BF16) return f32_to_bf16(v);
  else return f32_to_f16(v);
}
// element e (< EPC) of a raw 16-B chunk of type DT, as fp32
template <int DT>
__device__ __forceinline__ float chunk_elem(const u32x4& c, int e) {
  if constexpr (DT == SF_F32) return __uint_as_float(c[e]);
  else {
    uint32_t h = (c[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
    return DT == SF_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  }
}
// pack EPC fp32 values into a 16-B chunk of type DT
template <int DT>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
  u32x4 r;
  if constexpr (DT == SF_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(v[e]);
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = to_in_bits<DT>(v[2 * d]) | (to_in_bits<DT>(v[2 * d + 1]) << 16);
  }
  return r;
}

// ---------------------------------------------------------------------------
// global -> register staging of one K-step (BK elements of K)
// Every thread owns 8 chunks of 16 B for each operand.
// ---------------------------------------------------------------------------
template <int DT, int WP>
struct Stage {
  static constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC;
  u32x4 xa[8];  // x' chunks: row m = (t>>3) + 32 i, chunk kc = t & 7
  u32x4 wb[8];  // W chunks (layout depends on WP)

  // x rows: raw load (vec path) or converted load (generic path)
  __device__ __forceinline__ void load(const EncArgs& a, int64_t m0, int64_t n0, int64_t k0, int t) {
    const int kc = t & 7;
    const int64_t k = k0 + kc * EPC;
    if constexpr (WP != W_GENERIC) {
      const char* xb = (const char*)a.x;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int64_t m = m0 + (t >> 3) + 32 * i;
        if (m < a.M && k < a.K)
          xa[i] = *(const u32x4*)(xb + (m * a.sxm + k) * E);
        else
          xa[i] = u32x4{0, 0, 0, 0};
      }
    }
    if constexpr (WP == W_NMAJOR) {
      // 8x8 (16-bit) or 4x4 (fp32) element blocks: rows k = kg*EPC + r, cols n = ng*EPC..
      constexpr int NGS = 256 / EPC, NB = 8 / EPC;
      const char* wbp = (const char*)a.w;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        int bb = t + 256 * b, ng = bb % NGS, kg = bb / NGS;
        int64_t n = n0 + ng * EPC;
#pragma unroll
        for (int r = 0; r < EPC; ++r) {
          int64_t kk = k0 + kg * EPC + r;
          if (kk < a.K && n < a.N)
            wb[b * EPC + r] = *(const u32x4*)(wbp + (kk * a.swk + n) * E);
          else
            wb[b * EPC + r] = u32x4{0, 0, 0, 0};
        }
      }
    } else if constexpr (WP == W_KMAJOR) {
      const char* wbp = (const char*)a.w;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int64_t n = n0 + (t >> 3) + 32 * i;
        if (n < a.N && k < a.K)
          wb[i] = *(const u32x4*)(wbp + (n * a.swn + k) * E);
        else
          wb[i] = u32x4{0, 0, 0, 0};
      }
    } else {
      // generic: any strides / alignment / x dtype; element-wise, x' formed here
#pragma unroll 1
      for (int i = 0; i < 8; ++i) {
        int64_t m = m0 + (t >> 3) + 32 * i;
        int64_t n = n0 + (t >> 3) + 32 * i;
        float v[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          int64_t kk = k + e;
          v[e] = (m < a.M && kk < a.K)
                     ? load_as_f32(a.x, a.x_dt, m * a.sxm + kk * a.sxk) - load_as_f32(a.b_dec, a.bdec_dt, kk)
                     : 0.f;
        }
        xa[i] = pack_chunk<DT>(v);
        u32x4 c = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          int64_t kk = k + e;
          uint32_t bits = 0;
          if (n < a.N && kk < a.K) {
            int64_t off = kk * a.swk + n * a.swn;
            bits = DT == SF_F32 ? ((const uint32_t*)a.w)[off] : ((const u16*)a.w)[off];
          }
          if constexpr (DT == SF_F32) c[e] = bits;
          else c[e >> 1] |= bits << ((e & 1) * 16);
        }
        wb[i] = c;
      }
    }
  }

  // x' = cast(fp32(x) - fp32(b_dec)) for the vec paths, then registers -> LDS
  __device__ __forceinline__ void store(const EncArgs& a, char* As, char* Bs, int64_t m0, int64_t k0,
                                        int t) {
    const int kc = t & 7;
    if constexpr (WP != W_GENERIC) {
      const int64_t k = k0 + kc * EPC;
      float bd[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) bd[e] = (k + e < a.K) ? load_as_f32(a.b_dec, a.bdec_dt, k + e) : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int64_t m = m0 + (t >> 3) + 32 * i;
        float v[EPC];
        bool ok = m < a.M && k < a.K;
#pragma unroll
        for (int e = 0; e < EPC; ++e) v[e] = ok ? chunk_elem<DT>(xa[i], e) - bd[e] : 0.f;
        xa[i] = pack_chunk<DT>(v);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) *(u32x4*)(Bs + lds_off((t >> 3) + 32 * i, kc)) = xa[i];

    if constexpr (WP == W_NMAJOR) {
      constexpr int NGS = 256 / EPC, NB = 8 / EPC;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        int bb = t + 256 * b, ng = bb % NGS, kg = bb / NGS;
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          u32x4 c;
          if constexpr (DT == SF_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) c[e] = wb[b * 4 + e][j];
          } else {
            const int sh = (j & 1) * 16;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              uint32_t lo = (wb[b * 8 + 2 * d][j >> 1] >> sh) & 0xffffu;
              uint32_t hi = (wb[b * 8 + 2 * d + 1][j >> 1] >> sh) & 0xffffu;
              c[d] = lo | (hi << 16);
            }
          }
          *(u32x4*)(As + lds_off(ng * EPC + j, kg)) = c;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) *(u32x4*)(As + lds_off((t >> 3) + 32 * i, kc)) = wb[i];
    }
  }
};

template <int DT, int WP>
__global__ __launch_bounds__(NT, 1) void encode_kernel(EncArgs a) {
  constexpr int BK = Traits<DT>::BK;
  __shared__ __attribute__((aligned(16))) char smem[2 * 2 * TILE_BYTES];
  __shared__ float s_benc[BN], s_thr[BN];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware remap: hardware id b runs on XCD b % 8; give each XCD a contiguous range.
  const int total = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = b % 8, loc = b / 8;
  const int lid = xcd * per + min(xcd, rem) + loc;
  // grouped order within the range
  const int pids_per_group = a.group_m * a.tiles_n;
  const int first_m = (lid / pids_per_group) * a.group_m;
  const int gm = min(a.tiles_m - first_m, a.group_m);
  const int pid_m = first_m + (lid % pids_per_group) % gm;
  const int pid_n = (lid % pids_per_group) / gm;
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  {  // bias / threshold of this tile's features (fp32 in LDS)
    int64_t n = n0 + t;
    s_benc[t] = n < a.N ? load_as_f32(a.b_enc, a.benc_dt, n) : 0.f;
    s_thr[t] = (a.act == SF_ACT_JUMPRELU && n < a.N) ? load_as_f32(a.thr, a.thr_dt, n) : 0.f;
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  Stage<DT, WP> st;
  const int KT = (int)((a.K + BK - 1) / BK);
  st.load(a, m0, n0, 0, t);
  st.store(a, smem, smem + TILE_BYTES, m0, 0, t);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) st.load(a, m0, n0, (int64_t)(kt + 1) * BK, t);

    const char* As = smem + buf * 2 * TILE_BYTES;  // W^T rows (features)
    const char* Bs = As + TILE_BYTES;              // x' rows (tokens)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kc = s * 2 + (lane >> 5);
      u32x4 fa[4], fb[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) fa[nb] = *(const u32x4*)(As + lds_off(wn * 128 + nb * 32 + (lane & 31), kc));
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) fb[mb] = *(const u32x4*)(Bs + lds_off(wm * 128 + mb * 32 + (lane & 31), kc));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) mfma_chunk<DT>(acc[nb][mb], fa[nb], fb[mb]);
    }

    if (more) {
      char* nAs = smem + (buf ^ 1) * 2 * TILE_BYTES;
      st.store(a, nAs, nAs + TILE_BYTES, m0, (int64_t)(kt + 1) * BK, t);
    }
    __syncthreads();
  }

  // ---------------- epilogue: bias + activation + cast + count + store ----------------
  const int esz = sf_dtype_size(a.out_dt);
  const bool count = a.row_nnz != nullptr;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int64_t m = m0 + wm * 128 + mb * 32 + (lane & 31);
    const bool mok = m < a.M;
    int cnt = 0;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = wn * 128 + nb * 32 + g * 8 + (lane >> 5) * 4;  // local feature of r=0
        const int64_t n = n0 + nl;
        uint32_t bits[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float pre = acc[nb][mb][g * 4 + r] + s_benc[nl + r];
          float o = pre;
          if (a.act != SF_ACT_NONE) {
            o = fmaxf(pre, 0.f);
            if (a.act == SF_ACT_JUMPRELU && !(pre > s_thr[nl + r])) o = 0.f;
          }
          bits[r] = f32_to_bits(o, a.out_dt);
          if (mok && n + r < a.N && bits_nonzero(bits[r], esz)) ++cnt;
        }
        if (!mok) continue;
        if (a.vec_store && n + 3 < a.N) {
          char* p = (char*)a.out + (m * a.som + n) * esz;
          if (esz == 2) {
            u32x2 v = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
            __builtin_nontemporal_store(v, (u32x2*)p);
          } else {
            u32x4 v = {bits[0], bits[1], bits[2], bits[3]};
            __builtin_nontemporal_store(v, (u32x4*)p);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (n + r >= a.N) break;
            int64_t off = m * a.som + (n + r) * a.son;
            if (esz == 2) ((u16*)a.out)[off] = (u16)bits[r];
            else ((uint32_t*)a.out)[off] = bits[r];
          }
        }
      }
    }
    if (count) {
      cnt += __shfl_xor(cnt, 32);
      if (lane < 32 && mok && cnt > 0) atomicAdd(a.row_nnz + m, cnt);
    }
  }
}

template <int DT>
hipError_t launch_dt(const EncArgs& a, int wp, hipStream_t s) {
  dim3 grid(a.tiles_m * a.tiles_n), block(NT);
  switch (wp) {
    case W_NMAJOR: hipLaunchKernelGGL((encode_kernel<DT, W_NMAJOR>), grid, block, 0, s, a); break;
    case W_KMAJOR: hipLaunchKernelGGL((encode_kernel<DT, W_KMAJOR>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((encode_kernel<DT, W_GENERIC>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

constexpr int DEFAULT_GROUP_M = 8;

int bk_of(int w_dt) { return w_dt == SF_F32 ? 32 : 64; }

bool aligned(const void* p, int64_t bytes) { return ((uintptr_t)p % bytes) == 0; }

}  // namespace

extern "C" int sf_encode_config(int64_t M, int64_t N, int64_t K, int w_dt, int32_t* cfg_out) {
  sf_clear_error();
  SF_REQUIRE(cfg_out != nullptr, "sf_encode_config: cfg_out is NULL");
  SF_REQUIRE(sf_valid_dtype(w_dt), "sf_encode_config: bad dtype code %d", w_dt);
  (void)M; (void)N; (void)K;
  cfg_out[0] = BM;
  cfg_out[1] = BN;
  cfg_out[2] = bk_of(w_dt);
  cfg_out[3] = DEFAULT_GROUP_M;
  return SF_OK;
}

extern "C" int sf_encode(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w, int64_t swk,
                         int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec,
                         int bdec_dt, const void* thr, int thr_dt, void* out, int64_t som, int64_t son,
                         int out_dt, int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
                         const int32_t* tile_cfg, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0 && K >= 0, "sf_encode: negative size (M=%lld N=%lld K=%lld)", (long long)M,
             (long long)N, (long long)K);
  SF_REQUIRE(sf_valid_dtype(x_dt) && sf_valid_dtype(w_dt) && sf_valid_dtype(benc_dt) &&
                 sf_valid_dtype(bdec_dt) && sf_valid_dtype(out_dt),
             "sf_encode: bad dtype code");
  SF_REQUIRE(act == SF_ACT_RELU || act == SF_ACT_JUMPRELU || act == SF_ACT_NONE, "sf_encode: bad activation %d",
             act);
  if (act == SF_ACT_JUMPRELU) {
    SF_REQUIRE(thr != nullptr, "sf_encode: jumprelu needs a threshold");
    SF_REQUIRE(sf_valid_dtype(thr_dt), "sf_encode: bad threshold dtype code %d", thr_dt);
  }
  if (M == 0 || N == 0) return SF_OK;
  SF_REQUIRE(x && w && b_enc && b_dec && out, "sf_encode: NULL buffer");
  SF_REQUIRE(M <= INT32_MAX - BM && N <= INT32_MAX - BN, "sf_encode: M or N too large");
  const int bk = bk_of(w_dt);
  int group_m = DEFAULT_GROUP_M;
  if (tile_cfg) {
    SF_REQUIRE(tile_cfg[0] == BM && tile_cfg[1] == BN && tile_cfg[2] == bk && tile_cfg[3] >= 1,
               "sf_encode: unsupported tile config {%d,%d,%d,%d}; compiled tilings: {%d,%d,%d,GROUP_M>=1}",
               tile_cfg[0], tile_cfg[1], tile_cfg[2], tile_cfg[3], BM, BN, bk);
    group_m = tile_cfg[3];
  }

  EncArgs a;
  a.x = x; a.sxm = sxm; a.sxk = sxk; a.x_dt = x_dt;
  a.w = w; a.swk = swk; a.swn = swn;
  a.b_enc = b_enc; a.benc_dt = benc_dt; a.b_dec = b_dec; a.bdec_dt = bdec_dt;
  a.thr = thr; a.thr_dt = act == SF_ACT_JUMPRELU ? thr_dt : SF_F32;
  a.out = out; a.som = som; a.son = son; a.out_dt = out_dt;
  a.row_nnz = row_nnz; a.M = M; a.N = N; a.K = K; a.act = act;
  a.tiles_m = (int)((M + BM - 1) / BM);
  a.tiles_n = (int)((N + BN - 1) / BN);
  a.group_m = group_m;
  SF_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "sf_encode: too many tiles");

  const int esz = sf_dtype_size(w_dt), epc = 16 / esz;
  const int oes = sf_dtype_size(out_dt);
  a.vec_store = son == 1 && (som % 4) == 0 && aligned(out, 4 * oes);

  // vector paths: x and the K-contiguous side of W read as aligned 16-B chunks
  const bool x_vec = x_dt == w_dt && sxk == 1 && (sxm % epc) == 0 && aligned(x, 16) && (K % epc) == 0;
  int wp = W_GENERIC;
  if (x_vec && swn == 1 && (swk % epc) == 0 && (N % epc) == 0 && aligned(w, 16)) wp = W_NMAJOR;
  else if (x_vec && swk == 1 && (swn % epc) == 0 && aligned(w, 16)) wp = W_KMAJOR;

  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (w_dt) {
    case SF_BF16: e = launch_dt<SF_BF16>(a, wp, s); break;
    case SF_F16: e = launch_dt<SF_F16>(a, wp, s); break;
    default: e = launch_dt<SF_F32>(a, wp, s); break;
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "sf_encode: kernel launch failed: %s", hipGetErrorString(e));
  return SF_OK;
}
