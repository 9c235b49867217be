// Fused SAE encoder on gfx950 MFMA: entry points (C ABI) and the x' prologue launch.
// Reference semantics: saeflow/kernels/encode.py:36-91 (kernel) and :97-139 (wrapper). The
// kernels and their design are described in encode_kernels.h.
#include <mutex>

#include "encode_kernels.h"

namespace sfenc {

template <int DT>
hipError_t launch_gemm(const GemmArgs& a, int wp, bool wide, int waves, hipStream_t s) {
  if (wide) return a.out_dt == SF_F32 ? launch_wide<DT, 4>(a, wp, waves, s) : launch_wide<DT, 2>(a, wp, waves, s);
  return a.out_dt == SF_F32 ? launch_narrow<DT, 4>(a, wp, s) : launch_narrow<DT, 2>(a, wp, s);
}

template <int DT>
hipError_t launch_xprep_rows(const void* x, int64_t sxm, int64_t sxk, int x_dt, int64_t Mx, const int32_t* rows,
                             const int32_t* n_rows, int64_t row_off, const void* b_dec, int bdec_dt, int64_t M,
                             int64_t K, int64_t Kp, char* xw, hipStream_t s) {
  const int64_t chunks = M * (Kp / Traits<DT>::EPC);
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 1024);
  hipLaunchKernelGGL((xprep_rows_kernel<DT>), dim3(blocks), dim3(256), 0, s, x, sxm, sxk, x_dt, Mx, rows, n_rows,
                     row_off, b_dec, bdec_dt, M, K, Kp, xw);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_xprep(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* b_dec, int bdec_dt,
                        int64_t M, int64_t K, int64_t Kp, char* xw, int32_t* tile_ctr, hipStream_t s) {
  constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC;
  const bool fast = x_dt == DT && bdec_dt == DT && sxk == 1 && (K % EPC) == 0 && ((uintptr_t)x % 16) == 0 &&
                    ((sxm * E) % 16) == 0 && ((uintptr_t)b_dec % 16) == 0;
  const int64_t chunks = M * (Kp / EPC);
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 65536);
  if (fast)
    hipLaunchKernelGGL((xprep_kernel<DT, true>), dim3(blocks), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt,
                       M, K, Kp, xw, tile_ctr);
  else
    hipLaunchKernelGGL((xprep_kernel<DT, false>), dim3(blocks), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt,
                       M, K, Kp, xw, tile_ctr);
  return hipGetLastError();
}


// Default tile order: runs of 8 feature panels (a run's W_enc panels, 8 x d_in x 256
// elements per XCD, stay in the last-level cache while the x' panels stream past them);
// measured 2-3% faster than runs of 4 token panels at C3 and C5, equal at C2 and C4.
constexpr int DEFAULT_GROUP_M = 1;  // not used while GROUP_N > 0
constexpr int DEFAULT_GROUP_N = 8;
constexpr int DEFAULT_WAVES = SF_WIDE_WAVES;  // the row-candidate kernels' count too

// Tilings: "wide" (default) = 256x256, K-step BK (gemm_kernel) with 8 waves of 128x64
// (default) or 4 waves of 128x128 (dense epilogue only); "narrow" = 256x128, K-step BK/2
// (gemm2_kernel, 4 waves, two workgroups per CU: more overlap, but 1.5x the LDS and L2
// traffic per flop, and it measured slower at the headline shape).
int bk_of(int w_dt) { return w_dt == SF_F32 ? 32 : 64; }
// K padded so both tilings see whole pipeline rounds: an even number of wide K-steps and a
// multiple of three narrow ones: lcm(2*64, 3*32) = 384 (16-bit), lcm(2*32, 3*16) = 192 (fp32).
int64_t padded_k(int64_t K, int w_dt) {
  const int64_t q = w_dt == SF_F32 ? 192 : 384;
  return (K + q - 1) / q * q;
}
bool aligned(const void* p, int64_t bytes) { return ((uintptr_t)p % bytes) == 0; }
// Workspace layout: x' [M, Kp] in the W dtype, rounded up to 256 bytes, then the persistent
// GEMM's per-XCD tile counters.
int64_t xw_bytes(int64_t M, int64_t K, int w_dt) {
  return (M * padded_k(K, w_dt) * sf_dtype_size(w_dt) + 255) / 256 * 256;
}
int64_t workspace_bytes_of(int64_t M, int64_t K, int w_dt) { return xw_bytes(M, K, w_dt) + TILE_CTR_BYTES; }

}  // namespace sfenc

using namespace sfenc;

extern "C" int sf_encode_config(int64_t M, int64_t N, int64_t K, int w_dt, int32_t* cfg_out) {
  sf_clear_error();
  SF_REQUIRE(cfg_out != nullptr, "sf_encode_config: cfg_out is NULL");
  SF_REQUIRE(sf_valid_dtype(w_dt), "sf_encode_config: bad dtype code %d", w_dt);
  (void)M; (void)N; (void)K;
  cfg_out[0] = BM;
  cfg_out[1] = BN;
  cfg_out[2] = bk_of(w_dt);
  cfg_out[3] = DEFAULT_GROUP_M;
  cfg_out[4] = DEFAULT_WAVES;
  cfg_out[5] = DEFAULT_GROUP_N;
  return SF_OK;
}

extern "C" int sf_encode_workspace_size(int64_t M, int64_t K, int w_dt, int64_t* bytes) {
  sf_clear_error();
  SF_REQUIRE(bytes != nullptr, "sf_encode_workspace_size: bytes is NULL");
  SF_REQUIRE(M >= 0 && K >= 0, "sf_encode_workspace_size: negative size");
  SF_REQUIRE(sf_valid_dtype(w_dt), "sf_encode_workspace_size: bad dtype code %d", w_dt);
  *bytes = workspace_bytes_of(M, K, w_dt);
  return SF_OK;
}

namespace {

template <int DT>
hipError_t launch_rows_o(int out_dt, bool floor, const GemmArgs& a, int wp, hipStream_t s) {
  switch (out_dt) {
    case SF_F32:
      return floor ? launch_rows<DT, SF_F32, EPI_ROWS_FLOOR>(a, wp, s) : launch_rows<DT, SF_F32, EPI_ROWS>(a, wp, s);
    case SF_F16:
      return floor ? launch_rows<DT, SF_F16, EPI_ROWS_FLOOR>(a, wp, s) : launch_rows<DT, SF_F16, EPI_ROWS>(a, wp, s);
    default:
      return floor ? launch_rows<DT, SF_BF16, EPI_ROWS_FLOOR>(a, wp, s) : launch_rows<DT, SF_BF16, EPI_ROWS>(a, wp, s);
  }
}

hipError_t launch_rows_dt(int w_dt, int out_dt, bool floor, const GemmArgs& a, int wp, hipStream_t s) {
  switch (w_dt) {
    case SF_BF16: return launch_rows_o<SF_BF16>(out_dt, floor, a, wp, s);
    case SF_F16: return launch_rows_o<SF_F16>(out_dt, floor, a, wp, s);
    default: return launch_rows_o<SF_F32>(out_dt, floor, a, wp, s);
  }
}

// Shared by sf_encode (dense output) and sf_encode_rows (row candidates): validation, the x'
// prologue and the GEMM launch. `fn` names the entry point in error messages.
int encode_impl(const char* fn, int epi, const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w,
                int64_t swk, int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
                const void* thr, int thr_dt, void* out, int64_t som, int64_t son, int out_dt, int32_t* row_nnz,
                int32_t* cand_cnt, int32_t* cand_idx, void* cand_val, int64_t cap, const float* row_floor,
                int64_t M, int64_t N, int64_t K, int act, const int32_t* tile_cfg, void* workspace,
                int64_t workspace_bytes, void* stream, bool gather = false, const int32_t* live_rows = nullptr,
                const int32_t* n_live = nullptr, int64_t live_off = 0, int64_t Mx = 0) {
  SF_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size (M=%lld N=%lld K=%lld)", fn, (long long)M,
             (long long)N, (long long)K);
  SF_REQUIRE(sf_valid_dtype(x_dt) && sf_valid_dtype(w_dt) && sf_valid_dtype(benc_dt) &&
                 sf_valid_dtype(bdec_dt) && sf_valid_dtype(out_dt),
             "%s: bad dtype code", fn);
  SF_REQUIRE(act == SF_ACT_RELU || act == SF_ACT_JUMPRELU || (act == SF_ACT_NONE && epi == EPI_DENSE),
             "%s: bad activation %d", fn, act);
  SF_REQUIRE(!(act == SF_ACT_NONE && row_nnz != nullptr), "%s: row counts need relu or jumprelu", fn);
  if (act == SF_ACT_JUMPRELU) {
    SF_REQUIRE(thr != nullptr, "%s: jumprelu needs a threshold", fn);
    SF_REQUIRE(sf_valid_dtype(thr_dt), "%s: bad threshold dtype code %d", fn, thr_dt);
  }
  const int bk = bk_of(w_dt);
  int group_m = DEFAULT_GROUP_M, group_n = DEFAULT_GROUP_N, waves = DEFAULT_WAVES;
  bool wide = true;
  if (tile_cfg) {
    const bool is_wide = tile_cfg[0] == BM && tile_cfg[1] == BN && tile_cfg[2] == bk &&
                         (tile_cfg[4] == SF_WIDE_WAVES || (tile_cfg[4] == 4 && epi == EPI_DENSE));
    const bool is_narrow = epi == EPI_DENSE && tile_cfg[0] == t2::BM && tile_cfg[1] == t2::BN &&
                           tile_cfg[2] == bk / 2 && tile_cfg[4] == 4;
    SF_REQUIRE((is_wide || is_narrow) && tile_cfg[3] >= 1 && tile_cfg[5] >= 0,
               "%s: unsupported tile config {%d,%d,%d,%d,%d,%d}; compiled tilings: "
               "{%d,%d,%d,GROUP_M>=1,%d%s,GROUP_N>=0}%s", fn, tile_cfg[0], tile_cfg[1], tile_cfg[2], tile_cfg[3],
               tile_cfg[4], tile_cfg[5], BM, BN, bk, SF_WIDE_WAVES, epi == EPI_DENSE ? " or 4" : "",
               epi == EPI_DENSE ? " and {256,128,BLOCK_K/2,GROUP_M>=1,4,GROUP_N>=0}" : "");
    group_m = tile_cfg[3];
    group_n = tile_cfg[5];
    waves = tile_cfg[4];
    wide = is_wide;
  }
  if (epi != EPI_DENSE) {
    SF_REQUIRE(cap >= 0 && cap <= SF_ROWS_CAP_MAX, "%s: capacity %lld out of range [0, %d]", fn, (long long)cap,
               SF_ROWS_CAP_MAX);
    SF_REQUIRE(epi != EPI_ROWS_FLOOR || act == SF_ACT_RELU, "%s: a row floor needs relu", fn);
  }
  if (gather) {
    SF_REQUIRE(epi == EPI_DENSE && tile_cfg == nullptr && row_nnz == nullptr,
               "%s: the gathered-row encode has no tile_cfg and no row counts", fn);
    SF_REQUIRE(Mx >= 0 && live_off >= 0, "%s: negative size (Mx=%lld row_off=%lld)", fn, (long long)Mx,
               (long long)live_off);
  }
  if (M == 0 || N == 0) return SF_OK;
  SF_REQUIRE(x && w && b_enc && b_dec, "%s: NULL buffer", fn);
  SF_REQUIRE(!gather || (live_rows && n_live), "%s: NULL row list or row count", fn);
  if (epi == EPI_DENSE) SF_REQUIRE(out != nullptr, "%s: NULL output", fn);
  else SF_REQUIRE(cand_cnt && (cap == 0 || (cand_idx && cand_val)), "%s: NULL candidate buffer", fn);
  SF_REQUIRE(epi != EPI_ROWS_FLOOR || row_floor != nullptr, "%s: NULL row floor", fn);
  SF_REQUIRE(M <= INT32_MAX - BM && N <= INT32_MAX - BN, "%s: M or N too large", fn);
  const int esz = sf_dtype_size(w_dt), epc = 16 / esz;
  const int64_t Kp = padded_k(K, w_dt);
  SF_REQUIRE(Kp * esz * BM < (1LL << 31), "%s: d_in=%lld too large for 32-bit tile offsets", fn, (long long)K);
  const int64_t need = workspace_bytes_of(M, K, w_dt);
  SF_REQUIRE(workspace != nullptr && workspace_bytes >= need && aligned(workspace, 16),
             "%s: needs a 16-B aligned workspace of %lld bytes (sf_encode_workspace_size), got %lld", fn,
             (long long)need, (long long)workspace_bytes);

  GemmArgs a;
  a.xw = (const char*)workspace; a.Kp = Kp;
  a.w = (const char*)w; a.swk = swk; a.swn = swn;
  a.b_enc = b_enc; a.benc_dt = benc_dt;
  a.thr = thr; a.thr_dt = act == SF_ACT_JUMPRELU ? thr_dt : SF_F32;
  a.out = out; a.som = som; a.son = son; a.out_dt = out_dt;
  a.row_nnz = row_nnz; a.M = M; a.N = N; a.K = K; a.act = act;
  const int tbm = wide ? BM : t2::BM, tbn = wide ? BN : t2::BN;
  // K-steps of the chosen tiling: whole pipeline rounds (2 wide steps of bk, 3 narrow steps of
  // bk/2) covering K; the workspace is padded for both (padded_k), so no zero round is added
  // to the wide kernel where K is not a multiple of 384 (e.g. d_in = 4096: 64 steps, not 66)
  const int64_t round_k = wide ? 2 * bk : 3 * (bk / 2);
  a.ksteps = (int)((K + round_k - 1) / round_k * round_k / (wide ? bk : bk / 2));
  a.tiles_m = (int)((M + tbm - 1) / tbm);
  a.tiles_n = (int)((N + tbn - 1) / tbn);
  // a group wider than the panels there are orders the tiles as one that covers them all (and
  // keeps group * tiles within int)
  a.group_m = std::min(group_m, a.tiles_m);
  a.group_n = std::min(group_n, a.tiles_n);
  SF_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "%s: too many tiles", fn);
  const int oes = sf_dtype_size(out_dt);
  a.vec_store = epi == EPI_DENSE && son == 1 && ((som * oes) % 16) == 0 && aligned(out, 16);
  a.cand_cnt = cand_cnt; a.cand_idx = cand_idx; a.cand_val = (char*)cand_val; a.cap = cap;
  a.row_floor = row_floor;
  a.n_live = n_live;
  a.live_off = live_off;
  a.tile_ctr = (int32_t*)((char*)workspace + xw_bytes(M, K, w_dt));

  // W layouts the DMA paths take; anything else is staged element-wise
  int wp = W_GENERIC;
  if (swn == 1 && swk >= N && (N % epc) == 0 && ((swk * esz) % 16) == 0 && aligned(w, 16) &&
      (int64_t)bk * swk * esz + N * esz < (1LL << 31))
    wp = W_NMAJOR;
  else if (swk == 1 && swn >= K && ((swn * esz) % 16) == 0 && aligned(w, 16) &&
           (int64_t)BN * swn * esz + K * esz < (1LL << 31))
    wp = W_KMAJOR;

  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (gather) {
    int dev = 0, cus = 0;
    SF_HIP_CHECK(hipGetDevice(&dev));
    SF_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    switch (w_dt) {
      case SF_BF16:
        e = launch_xprep_rows<SF_BF16>(x, sxm, sxk, x_dt, Mx, live_rows, n_live, live_off, b_dec, bdec_dt, M, K, Kp,
                                       (char*)workspace, s);
        if (e == hipSuccess) e = out_dt == SF_F32 ? launch_live<SF_BF16, 4>(a, wp, cus, s) : launch_live<SF_BF16, 2>(a, wp, cus, s);
        break;
      case SF_F16:
        e = launch_xprep_rows<SF_F16>(x, sxm, sxk, x_dt, Mx, live_rows, n_live, live_off, b_dec, bdec_dt, M, K, Kp,
                                      (char*)workspace, s);
        if (e == hipSuccess) e = out_dt == SF_F32 ? launch_live<SF_F16, 4>(a, wp, cus, s) : launch_live<SF_F16, 2>(a, wp, cus, s);
        break;
      default:
        e = launch_xprep_rows<SF_F32>(x, sxm, sxk, x_dt, Mx, live_rows, n_live, live_off, b_dec, bdec_dt, M, K, Kp,
                                      (char*)workspace, s);
        if (e == hipSuccess) e = out_dt == SF_F32 ? launch_live<SF_F32, 4>(a, wp, cus, s) : launch_live<SF_F32, 2>(a, wp, cus, s);
        break;
    }
    if (e != hipSuccess) return sf_fail(SF_EHIP, "%s: kernel launch failed: %s", fn, hipGetErrorString(e));
    return SF_OK;
  }
  switch (w_dt) {
    case SF_BF16: e = launch_xprep<SF_BF16>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, a.tile_ctr, s); break;
    case SF_F16: e = launch_xprep<SF_F16>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, a.tile_ctr, s); break;
    default: e = launch_xprep<SF_F32>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, a.tile_ctr, s); break;
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "%s: prologue launch failed: %s", fn, hipGetErrorString(e));
  if (epi == EPI_DENSE) {
    switch (w_dt) {
      case SF_BF16: e = launch_gemm<SF_BF16>(a, wp, wide, waves, s); break;
      case SF_F16: e = launch_gemm<SF_F16>(a, wp, wide, waves, s); break;
      default: e = launch_gemm<SF_F32>(a, wp, wide, waves, s); break;
    }
  } else {
    e = launch_rows_dt(w_dt, out_dt, epi == EPI_ROWS_FLOOR, a, wp, s);
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "%s: kernel launch failed: %s", fn, hipGetErrorString(e));
  return SF_OK;
}

}  // namespace

extern "C" int sf_encode(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w, int64_t swk,
                         int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec,
                         int bdec_dt, const void* thr, int thr_dt, void* out, int64_t som, int64_t son,
                         int out_dt, int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
                         const int32_t* tile_cfg, void* workspace, int64_t workspace_bytes, void* stream) {
  sf_clear_error();
  return encode_impl("sf_encode", EPI_DENSE, x, sxm, sxk, x_dt, w, swk, swn, w_dt, b_enc, benc_dt, b_dec, bdec_dt,
                     thr, thr_dt, out, som, son, out_dt, row_nnz, nullptr, nullptr, nullptr, 0, nullptr, M, N, K,
                     act, tile_cfg, workspace, workspace_bytes, stream);
}

extern "C" int sf_encode_rows(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w, int64_t swk,
                              int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
                              const void* thr, int thr_dt, const float* row_floor, int32_t* cand_cnt,
                              int32_t* cand_idx, void* cand_val, int val_dt, int64_t cap, int64_t M, int64_t N,
                              int64_t K, int act, const int32_t* tile_cfg, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  sf_clear_error();
  return encode_impl("sf_encode_rows", row_floor ? EPI_ROWS_FLOOR : EPI_ROWS, x, sxm, sxk, x_dt, w, swk, swn, w_dt,
                     b_enc, benc_dt, b_dec, bdec_dt, thr, thr_dt, nullptr, 0, 0, val_dt, nullptr, cand_cnt, cand_idx,
                     cand_val, cap, row_floor, M, N, K, act, tile_cfg, workspace, workspace_bytes, stream);
}


extern "C" int sf_encode_gather(const void* x, int64_t sxm, int64_t sxk, int x_dt, int64_t Mx, const int32_t* rows,
                                const int32_t* n_rows, int64_t row_off, const void* w, int64_t swk, int64_t swn,
                                int w_dt, const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
                                const void* thr, int thr_dt, void* out, int64_t som, int64_t son, int out_dt,
                                int64_t M, int64_t N, int64_t K, int act, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  sf_clear_error();
  return encode_impl("sf_encode_gather", EPI_DENSE, x, sxm, sxk, x_dt, w, swk, swn, w_dt, b_enc, benc_dt, b_dec,
                     bdec_dt, thr, thr_dt, out, som, son, out_dt, nullptr, nullptr, nullptr, nullptr, 0, nullptr, M,
                     N, K, act, nullptr, workspace, workspace_bytes, stream, true, rows, n_rows, row_off, Mx);
}

// ----------------------------------------------------------------------------- no allocation
// sf_encode for callers that cannot allocate: the x' workspace is a file-scope device array
// (every GPU the library runs on holds its own copy until the process ends). In host code
// `scratch` names a host-side stand-in, not the device array, so its device address is
// looked up once per device, with that device current, and only that address is used.
static __device__ __align__(256) char scratch[SF_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES];  // device address of `scratch` per device id, set once

int scratch_address(const char* fn, void** out) {
  int dev = -1;
  SF_HIP_CHECK(hipGetDevice(&dev));
  SF_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "%s: device %d out of range", fn, dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return sf_fail(SF_EHIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                     hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return SF_OK;
}
}  // namespace

extern "C" int sf_encode_noalloc(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w, int64_t swk,
                                 int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec,
                                 int bdec_dt, const void* thr, int thr_dt, void* out, int64_t som, int64_t son,
                                 int out_dt, int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
                                 const int32_t* tile_cfg, void* stream) {
  sf_clear_error();
  static const char* fn = "sf_encode_noalloc";
  SF_REQUIRE(M >= 0 && K >= 0, "%s: negative size (M=%lld K=%lld)", fn, (long long)M, (long long)K);
  SF_REQUIRE(M <= INT32_MAX && K < (1LL << 31), "%s: M or d_in too large (M=%lld K=%lld)", fn, (long long)M,
             (long long)K);  // before the byte counts below, which must not overflow
  SF_REQUIRE(sf_valid_dtype(w_dt) && sf_valid_dtype(x_dt) && sf_valid_dtype(out_dt), "%s: bad dtype code", fn);
  // x' rows of whole 256-row tiles that fit the array beside the tile counters (and the x'
  // rounding); larger M runs in chunks of that many rows, each chunk's prologue and GEMM after
  // the previous chunk's on the stream
  const int64_t row_bytes = padded_k(K, w_dt) * sf_dtype_size(w_dt);
  const int64_t chunk = row_bytes > 0 ? (SF_NOALLOC_SCRATCH_BYTES - TILE_CTR_BYTES - 255) / row_bytes / BM * BM : M;
  SF_REQUIRE(chunk >= BM || M == 0,
             "%s: one %d-row block of x' needs %lld bytes (d_in=%lld), above the %lld-byte scratch array; use "
             "sf_encode with a workspace",
             fn, BM, (long long)(BM * row_bytes), (long long)K, (long long)SF_NOALLOC_SCRATCH_BYTES);
  if (M == 0 || N == 0) return SF_OK;
  void* ws = nullptr;
  const int rc = scratch_address(fn, &ws);
  if (rc != SF_OK) return rc;
  const int64_t xes = sf_dtype_size(x_dt), oes = sf_dtype_size(out_dt);
  for (int64_t off = 0; off < M; off += chunk) {
    const int64_t m = std::min(chunk, M - off);
    const int r = encode_impl(fn, EPI_DENSE, (const char*)x + off * sxm * xes, sxm, sxk, x_dt, w, swk, swn, w_dt,
                              b_enc, benc_dt, b_dec, bdec_dt, thr, thr_dt, (char*)out + off * som * oes, som, son,
                              out_dt, row_nnz ? row_nnz + off : nullptr, nullptr, nullptr, nullptr, 0, nullptr, m,
                              N, K, act, tile_cfg, ws, SF_NOALLOC_SCRATCH_BYTES, stream);
    if (r != SF_OK) return r;
  }
  return SF_OK;
}
