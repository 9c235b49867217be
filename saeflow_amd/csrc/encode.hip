// Fused SAE encoder on gfx950 MFMA: entry points (C ABI) and the x' prologue launch.
// Reference semantics: saeflow/kernels/encode.py:36-91 (kernel) and :97-139 (wrapper). The
// kernels and their design are described in encode_kernels.h.
#include "encode_kernels.h"

namespace sfenc {

template <int DT>
hipError_t launch_gemm(const GemmArgs& a, int wp, bool wide, hipStream_t s) {
  if (wide) return a.out_dt == SF_F32 ? launch_wide<DT, 4>(a, wp, s) : launch_wide<DT, 2>(a, wp, s);
  return a.out_dt == SF_F32 ? launch_narrow<DT, 4>(a, wp, s) : launch_narrow<DT, 2>(a, wp, s);
}

template <int DT>
hipError_t launch_xprep(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* b_dec, int bdec_dt,
                        int64_t M, int64_t K, int64_t Kp, char* xw, hipStream_t s) {
  constexpr int E = Traits<DT>::E, EPC = Traits<DT>::EPC;
  const bool fast = x_dt == DT && bdec_dt == DT && sxk == 1 && (K % EPC) == 0 && ((uintptr_t)x % 16) == 0 &&
                    ((sxm * E) % 16) == 0 && ((uintptr_t)b_dec % 16) == 0;
  const int64_t chunks = M * (Kp / EPC);
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 65536);
  if (fast)
    hipLaunchKernelGGL((xprep_kernel<DT, true>), dim3(blocks), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt,
                       M, K, Kp, xw);
  else
    hipLaunchKernelGGL((xprep_kernel<DT, false>), dim3(blocks), dim3(256), 0, s, x, sxm, sxk, x_dt, b_dec, bdec_dt,
                       M, K, Kp, xw);
  return hipGetLastError();
}

constexpr int DEFAULT_GROUP_M = 4;

// Tilings: "wide" (default) = 256x256, K-step BK (gemm_kernel); "narrow" = 256x128, K-step
// BK/2 (gemm2_kernel, two workgroups per CU: more overlap, but 1.5x the LDS and L2 traffic
// per flop, and it measured slower at the headline shape).
int bk_of(int w_dt) { return w_dt == SF_F32 ? 32 : 64; }
// K padded so both tilings see whole pipeline rounds: an even number of wide K-steps and a
// multiple of three narrow ones: lcm(2*64, 3*32) = 384 (16-bit), lcm(2*32, 3*16) = 192 (fp32).
int64_t padded_k(int64_t K, int w_dt) {
  const int64_t q = w_dt == SF_F32 ? 192 : 384;
  return (K + q - 1) / q * q;
}
bool aligned(const void* p, int64_t bytes) { return ((uintptr_t)p % bytes) == 0; }

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
  return SF_OK;
}

extern "C" int sf_encode_workspace_size(int64_t M, int64_t K, int w_dt, int64_t* bytes) {
  sf_clear_error();
  SF_REQUIRE(bytes != nullptr, "sf_encode_workspace_size: bytes is NULL");
  SF_REQUIRE(M >= 0 && K >= 0, "sf_encode_workspace_size: negative size");
  SF_REQUIRE(sf_valid_dtype(w_dt), "sf_encode_workspace_size: bad dtype code %d", w_dt);
  *bytes = M * padded_k(K, w_dt) * sf_dtype_size(w_dt);
  return SF_OK;
}

extern "C" int sf_encode(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* w, int64_t swk,
                         int64_t swn, int w_dt, const void* b_enc, int benc_dt, const void* b_dec,
                         int bdec_dt, const void* thr, int thr_dt, void* out, int64_t som, int64_t son,
                         int out_dt, int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
                         const int32_t* tile_cfg, void* workspace, int64_t workspace_bytes, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0 && K >= 0, "sf_encode: negative size (M=%lld N=%lld K=%lld)", (long long)M,
             (long long)N, (long long)K);
  SF_REQUIRE(sf_valid_dtype(x_dt) && sf_valid_dtype(w_dt) && sf_valid_dtype(benc_dt) &&
                 sf_valid_dtype(bdec_dt) && sf_valid_dtype(out_dt),
             "sf_encode: bad dtype code");
  SF_REQUIRE(act == SF_ACT_RELU || act == SF_ACT_JUMPRELU || act == SF_ACT_NONE, "sf_encode: bad activation %d",
             act);
  SF_REQUIRE(!(act == SF_ACT_NONE && row_nnz != nullptr), "sf_encode: row counts need relu or jumprelu");
  if (act == SF_ACT_JUMPRELU) {
    SF_REQUIRE(thr != nullptr, "sf_encode: jumprelu needs a threshold");
    SF_REQUIRE(sf_valid_dtype(thr_dt), "sf_encode: bad threshold dtype code %d", thr_dt);
  }
  const int bk = bk_of(w_dt);
  int group_m = DEFAULT_GROUP_M;
  bool wide = true;
  if (tile_cfg) {
    const bool is_wide = tile_cfg[0] == BM && tile_cfg[1] == BN && tile_cfg[2] == bk;
    const bool is_narrow = tile_cfg[0] == t2::BM && tile_cfg[1] == t2::BN && tile_cfg[2] == bk / 2;
    SF_REQUIRE((is_wide || is_narrow) && tile_cfg[3] >= 1,
               "sf_encode: unsupported tile config {%d,%d,%d,%d}; compiled tilings: {%d,%d,%d,GROUP_M>=1} "
               "and {%d,%d,%d,GROUP_M>=1}",
               tile_cfg[0], tile_cfg[1], tile_cfg[2], tile_cfg[3], t2::BM, t2::BN, bk / 2, BM, BN, bk);
    group_m = tile_cfg[3];
    wide = is_wide;
  }
  if (M == 0 || N == 0) return SF_OK;
  SF_REQUIRE(x && w && b_enc && b_dec && out, "sf_encode: NULL buffer");
  SF_REQUIRE(M <= INT32_MAX - BM && N <= INT32_MAX - BN, "sf_encode: M or N too large");
  const int esz = sf_dtype_size(w_dt), epc = 16 / esz;
  const int64_t Kp = padded_k(K, w_dt);
  SF_REQUIRE(Kp * esz * BM < (1LL << 31), "sf_encode: d_in=%lld too large for 32-bit tile offsets", (long long)K);
  const int64_t need = M * Kp * esz;
  SF_REQUIRE(workspace != nullptr && workspace_bytes >= need && aligned(workspace, 16),
             "sf_encode: needs a 16-B aligned workspace of %lld bytes (sf_encode_workspace_size), got %lld",
             (long long)need, (long long)workspace_bytes);

  GemmArgs a;
  a.xw = (const char*)workspace; a.Kp = Kp;
  a.w = (const char*)w; a.swk = swk; a.swn = swn;
  a.b_enc = b_enc; a.benc_dt = benc_dt;
  a.thr = thr; a.thr_dt = act == SF_ACT_JUMPRELU ? thr_dt : SF_F32;
  a.out = out; a.som = som; a.son = son; a.out_dt = out_dt;
  a.row_nnz = row_nnz; a.M = M; a.N = N; a.K = K; a.act = act;
  const int tbm = wide ? BM : t2::BM, tbn = wide ? BN : t2::BN;
  a.tiles_m = (int)((M + tbm - 1) / tbm);
  a.tiles_n = (int)((N + tbn - 1) / tbn);
  a.group_m = group_m;
  SF_REQUIRE((int64_t)a.tiles_m * a.tiles_n < (1LL << 31), "sf_encode: too many tiles");
  const int oes = sf_dtype_size(out_dt);
  a.vec_store = son == 1 && ((som * oes) % 16) == 0 && aligned(out, 16);

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
  switch (w_dt) {
    case SF_BF16: e = launch_xprep<SF_BF16>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, s); break;
    case SF_F16: e = launch_xprep<SF_F16>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, s); break;
    default: e = launch_xprep<SF_F32>(x, sxm, sxk, x_dt, b_dec, bdec_dt, M, K, Kp, (char*)workspace, s); break;
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "sf_encode: prologue launch failed: %s", hipGetErrorString(e));
  switch (w_dt) {
    case SF_BF16: e = launch_gemm<SF_BF16>(a, wp, wide, s); break;
    case SF_F16: e = launch_gemm<SF_F16>(a, wp, wide, s); break;
    default: e = launch_gemm<SF_F32>(a, wp, wide, s); break;
  }
  if (e != hipSuccess) return sf_fail(SF_EHIP, "sf_encode: kernel launch failed: %s", hipGetErrorString(e));
  return SF_OK;
}
