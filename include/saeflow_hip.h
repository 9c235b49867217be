/*
 * saeflow_hip.h — C ABI of libsaeflow_hip.so, the gfx950 (MI355X) kernels behind
 * saeflow's SAE hot path: fused encode -> dense->CSR compaction -> sparse CSR decode.
 *
 * Every entry point:
 *   - takes device pointers owned by the caller (no entry point allocates or frees
 *     caller-visible memory), element strides in elements, and a hipStream_t passed
 *     as `void*` (NULL = the legacy default stream);
 *   - launches asynchronously on that stream and returns SF_OK, or a nonzero
 *     sf_status when the arguments are rejected or a HIP call fails; the message
 *     is then in sf_last_error() (thread-local);
 *   - keeps no mutable global state, so calls are reentrant from any host thread.
 *
 * The CSR contract (reference saeflow/kernels/decode.py:3-6, ops.py:4,36): row m's
 * active features are indices[indptr[m] : indptr[m+1]]; indptr is int64 [M+1]
 * starting at 0, indices are int32, values have the feature dtype.
 *
 * All reference citations are file:line into the saeflow Python package.
 */
#ifndef SAEFLOW_HIP_H
#define SAEFLOW_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF_ABI_VERSION 4

/* The library is built with hidden symbol visibility; exactly these entry points are exported. */
#ifndef SF_API
#define SF_API __attribute__((visibility("default")))
#endif

/* element types (torch.float32 / torch.bfloat16 / torch.float16) */
enum sf_dtype { SF_F32 = 0, SF_BF16 = 1, SF_F16 = 2 };

/* activations: reference encode.py:16 numbers relu 0, jumprelu 1; SF_ACT_NONE is
 * the bare pre-activation (reference.py:36-37, SAE.encode_pre). */
enum sf_act { SF_ACT_RELU = 0, SF_ACT_JUMPRELU = 1, SF_ACT_NONE = 2 };

enum sf_status { SF_OK = 0, SF_EINVAL = 1, SF_EHIP = 2, SF_EUNSUPPORTED = 3 };

/* Version of this ABI (SF_ABI_VERSION). No reference counterpart. */
SF_API int sf_abi_version(void);

/* Message describing the last failed call on this host thread ("" if none).
 * Plays the role of the ValueError/RuntimeError texts raised by the reference
 * wrappers (encode.py:107-114). */
SF_API const char* sf_last_error(void);

/*
 * Fused encode: out = act((x - b_dec) @ W + b_enc), fp32 accumulation.
 * Replaces the _encode_kernel launch in fused_encode (reference
 * saeflow/kernels/encode.py:36-91 kernel, :97-139 wrapper).
 *   x      [M, K]  element type x_dt, strides (sxm, sxk)
 *   w      [K, N]  element type w_dt (the MFMA input type), strides (swk, swn): any strides
 *   b_enc  [N], b_dec [K], thr [N] (thr only for SF_ACT_JUMPRELU, else may be NULL);
 *          contiguous, any sf_dtype each, upcast to fp32 (encode.py:67,78,81)
 *   out    [M, N]  element type out_dt, strides (som, son)
 *   row_nnz int32 [M] or NULL: when given, row_nnz[m] += number of nonzero elements
 *          of out row m AS STORED (after rounding to out_dt) (encode.py:89-91)
 * Prologue: x' = cast_to_w_dt(fp32(x) - fp32(b_dec)) (encode.py:72).
 * Epilogue: pre = acc + b_enc; relu: max(pre,0); jumprelu: pre > thr ? max(pre,0) : 0
 *           (encode.py:78-82); none: pre.
 * tile_cfg: NULL (tuned table) or int32[6] {BLOCK_M, BLOCK_N, BLOCK_K, GROUP_M, NUM_WAVES,
 *           GROUP_N} naming one of the compiled tilings (encode.py:104 `config=`, whose Triton
 *           configs carry num_warps likewise): {256, 256, BK, G, 8 or 4, GN} or
 *           {256, 128, BK/2, G, 4, GN}, BK = 64 (16-bit W) or 32 (fp32 W), G >= 1, GN >= 0.
 *           Tile order: GN > 0 walks runs of GN feature tiles, token tile by token tile;
 *           GN = 0 walks runs of G token tiles, feature tile by feature tile (the reference's
 *           GROUP_M order, encode.py:44-52). The order changes speed only, never results.
 * workspace: caller-owned device buffer of at least sf_encode_workspace_size() bytes,
 *           16-B aligned; receives x' = cast(x - b_dec) once per call (the prologue is
 *           hoisted out of the GEMM because every x row block is reused by all d_sae/256
 *           feature tiles) and the GEMM's tile counters, which the prologue zeroes. Its
 *           contents are scratch between calls; calls that overlap must not share one.
 * The fp32 path always computes in IEEE fp32 (gfx950 has no xf32 MFMA): the
 * reference's allow_tf32 (encode.py:105,118-120) has no effect here.
 */
SF_API int sf_encode(const void* x, int64_t sxm, int64_t sxk, int x_dt,
              const void* w, int64_t swk, int64_t swn, int w_dt,
              const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
              const void* thr, int thr_dt,
              void* out, int64_t som, int64_t son, int out_dt,
              int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
              const int32_t* tile_cfg, void* workspace, int64_t workspace_bytes, void* stream);

/* sf_encode without a workspace argument and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). The x' workspace is a
 * library-owned device array of SF_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends). Tokens are encoded in chunks of whole 256-row blocks whose x' fits the array (7168
 * tokens at d_in 2304 in bf16), each chunk's prologue and GEMM after the previous chunk's on
 * the stream, so any M is taken; a d_in whose 256-row block of x' alone exceeds the array
 * (Kp * e > SF_NOALLOC_SCRATCH_BYTES / 256, e.g. d_in > 65536 in bf16) is refused with
 * SF_EINVAL before any launch. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must be serialised by the
 * caller. Arguments and results as sf_encode; the array's address is looked up on the first
 * call on each device. */
#define SF_NOALLOC_SCRATCH_BYTES (32LL << 20)
SF_API int sf_encode_noalloc(const void* x, int64_t sxm, int64_t sxk, int x_dt,
              const void* w, int64_t swk, int64_t swn, int w_dt,
              const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
              const void* thr, int thr_dt,
              void* out, int64_t som, int64_t son, int out_dt,
              int32_t* row_nnz, int64_t M, int64_t N, int64_t K, int act,
              const int32_t* tile_cfg, void* stream);

/* Bytes of workspace sf_encode needs for M tokens of d_in K with MFMA input type w_dt: x'
 * (M * K rounded up to the K-steps * element size, rounded up to 256 bytes) and 512 bytes of
 * tile counters the GEMM claims tiles from. No reference counterpart: the reference's Triton
 * kernel keeps x' in registers (encode.py:72). */
SF_API int sf_encode_workspace_size(int64_t M, int64_t K, int w_dt, int64_t* bytes);

/* Tiling the tuned table picks for sf_encode at this shape: writes
 * {BLOCK_M, BLOCK_N, BLOCK_K, GROUP_M, NUM_WAVES, GROUP_N} to cfg_out (int32[6]). Mirrors
 * best_config() (encode.py:142-144), which reports the autotuner's pick. */
SF_API int sf_encode_config(int64_t M, int64_t N, int64_t K, int w_dt, int32_t* cfg_out);

/*
 * Row-candidate encode: the fused encode without the dense output. Each row's kept values
 * (the nonzeros sf_encode would store, as val_dt) are appended as (column, value) to the
 * row's candidate list cand_idx / cand_val[m * cap ...], in no particular order, and
 * cand_cnt[m] (caller-zeroed int32 [M]) counts them all, also those past cap, so
 * cand_cnt[m] > cap flags a row whose list overflowed. With row_floor (float32 [M], relu
 * only) only stored values >= row_floor[m] are kept.
 * It serves two callers of the reference, without the [M, N] write and read:
 *   - dense_to_csr(fused_encode(...)) in ops.encode_sparse (reference ops.py:37-39), with
 *     sf_rows_to_csr; the candidate counts are the row_nnz counts (encode.py:89-91);
 *   - the TopK select f.topk(k) in ops._topk (reference ops.py:12-16), with sf_rows_topk and
 *     a floor no larger than each row's k-th largest value (NaN values are kept whatever
 *     the floor, as they rank above every value in the top-k).
 * Arguments as sf_encode; only the 256x256 tiling with 8 waves (tile_cfg NULL or {256, 256,
 * BLOCK_K, GROUP_M, 8, GROUP_N}). 0 <= cap <= 4096 (SF_EINVAL otherwise): sf_rows_to_csr and
 * sf_rows_topk read lists of at most 4096 entries.
 */
SF_API int sf_encode_rows(const void* x, int64_t sxm, int64_t sxk, int x_dt,
                   const void* w, int64_t swk, int64_t swn, int w_dt,
                   const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
                   const void* thr, int thr_dt, const float* row_floor,
                   int32_t* cand_cnt, int32_t* cand_idx, void* cand_val, int val_dt, int64_t cap,
                   int64_t M, int64_t N, int64_t K, int act, const int32_t* tile_cfg,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* The rows whose candidate list overflowed: rows[0 .. n) (int32 [M]) = the m with
 * cand_cnt[m] > cap in increasing order, and *n_rows (int32, device memory) = n, written on
 * the stream, so the caller need not read the counts back. Feeds sf_encode_gather and
 * sf_topk_gather, which redo those rows without the candidate lists. No reference counterpart
 * (the reference writes the dense features, ops.py:12-16, 37-39, so no list can overflow). */
SF_API int sf_overflow_rows(const int32_t* cand_cnt, int64_t M, int64_t cap, int32_t* rows, int32_t* n_rows,
                     void* stream);

/* sf_encode of gathered tokens whose number is known only on the device: out row i (of the
 * M rows of out) = the dense encode of token x[rows[row_off + i]] for the live rows
 * i < clamp(*n_rows - row_off, 0, M); the other rows of out hold unspecified values (the
 * rest of the last live 256-row block gets the encode of a zero x' row; past it nothing is
 * written). x has Mx rows; a row id outside [0, Mx) encodes a zero x'; rows (device memory)
 * holds at least *n_rows entries (row_off + i is read for each live i). The values are
 * bit-identical to sf_encode's for the same token. The grid is one workgroup per CU; they
 * walk the live tiles and return at once when there are none, so a call with *n_rows == 0
 * costs two near-empty launches. No row counts and no tile_cfg (the 256x256 tiling with 8
 * waves); workspace as sf_encode's for M rows. It is the TopK select's fallback for rows
 * whose candidate list overflowed (reference ops.py:12-16 makes no host read there, and
 * neither does this path). */
SF_API int sf_encode_gather(const void* x, int64_t sxm, int64_t sxk, int x_dt, int64_t Mx,
                     const int32_t* rows, const int32_t* n_rows, int64_t row_off,
                     const void* w, int64_t swk, int64_t swn, int w_dt,
                     const void* b_enc, int benc_dt, const void* b_dec, int bdec_dt,
                     const void* thr, int thr_dt,
                     void* out, int64_t som, int64_t son, int out_dt,
                     int64_t M, int64_t N, int64_t K, int act,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* Row candidates -> canonical CSR: row m's candidates sorted by column go to
 * indices/values[indptr[m] ...] (indptr = sf_scan_counts of cand_cnt, nnz = indptr[M]).
 * Rows with cand_cnt[m] > cap (overflowed lists) are skipped: their segments are left for
 * the caller to fill. Replaces the compaction of dense_to_csr (reference decode.py:61-94)
 * on the row-candidate path. cap <= 4096. */
SF_API int sf_rows_to_csr(const int32_t* cand_cnt, const int32_t* cand_idx, const void* cand_val, int val_dt,
                   int64_t cap, int64_t M, const int64_t* indptr, int64_t nnz, int32_t* indices,
                   void* values, void* stream);

/* Row-wise top-k of row candidates: values [M, k] (val_dt) sorted descending, indices int32
 * [M, k], equal values by increasing column, as sf_topk. A row with fewer than k candidates
 * is completed with zeros at its lowest columns that are not candidates, which equals
 * sf_topk of the dense row when every nonzero of the row is a candidate. Replaces
 * f.topk(k) in ops._topk (reference ops.py:12-16) on the row-candidate path.
 * 0 <= k <= min(N, 4096), cap <= 4096. */
SF_API int sf_rows_topk(const int32_t* cand_cnt, const int32_t* cand_idx, const void* cand_val, int val_dt,
                 int64_t cap, int64_t M, int64_t N, int64_t k, void* values, int32_t* indices, void* stream);

/* counts[m] = number of nonzero elements of f row m (-0.0 counts as zero, NaN as
 * nonzero, as f != 0). Replaces torch.count_nonzero(f, dim=1) in dense_to_csr
 * (reference decode.py:84-85). f [M, N] any strides. */
SF_API int sf_count_nonzero(const void* f, int64_t sfm, int64_t sfn, int f_dt,
                     int64_t M, int64_t N, int32_t* counts, void* stream);

/* indptr[0] = 0, indptr[m+1] = sum_{i<=m} counts[i] (int64). Replaces
 * `indptr[1:] = row_nnz.cumsum(0)` (reference decode.py:86-87). */
SF_API int sf_scan_counts(const int32_t* counts, int64_t M, int64_t* indptr, void* stream);

/* Compaction: for every row m, the nonzero elements of f row m, in increasing column
 * order, go to indices/values[indptr[m] ...] (canonical CSR, values copied bit-exact).
 * Replaces _compact_kernel (reference decode.py:61-74, launched at :91-93).
 * nnz = indptr[M] = capacity of indices/values; slots outside [indptr[m], indptr[m+1])
 * are never written, so inconsistent counts cannot write out of bounds. */
SF_API int sf_compact(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N,
               const int64_t* indptr, int64_t nnz, int32_t* indices, void* values,
               void* stream);

/* Sparse decode: out[m] = b_dec + sum_{j in row m} values[j] * W_dec[indices[j]],
 * fp32 accumulation. Replaces _decode_kernel (reference decode.py:28-55) launched by
 * sparse_decode (:97-120).
 *   indptr int64 [M+1], indices int32 [nnz], values [nnz] of val_dt
 *   w_dec  [d_sae, D] any strides (swn, swd); b_dec [D] or NULL (HAS_BIAS, decode.py:110)
 *   out    [M, D] of out_dt, strides (som, sod)
 * Entries with indices outside [0, d_sae) contribute nothing; indptr values are
 * clamped to [0, nnz]. tile_cfg NULL: rows of W_dec that are whole 128-B lines (contiguous,
 * 16-B aligned, row stride >= 0) run the line-slab kernel (each XCD's L2 serves one column slab
 * of W_dec at a time: two 128-B lines and 16 lanes per token when the row holds an even number
 * of lines and d_sae <= 65536, else one line and 8 lanes), other shapes one wave per row with
 * the slab width from D.
 * tile_cfg int32[2] {BLOCK_NNZ, BLOCK_D} (decode.py:101), both > 0: one wave per row, and with
 * W_dec rows contiguous BLOCK_D sets the slab of d_in one wave covers, rounded up to whole 16-B
 * chunks per lane (64 * 16/e elements: 512 for 16-bit W_dec, 256 for fp32) and capped at 8 of
 * them; other W_dec strides use 512-element slabs. BLOCK_NNZ is accepted for the reference's
 * signature: entries are always gathered 64 at a time, one per lane. The choice changes speed
 * only: every output element sums its entries in entry order in one lane, so results are
 * bit-identical with and without tile_cfg. */
SF_API int sf_decode(const int64_t* indptr, const int32_t* indices, const void* values, int val_dt,
              int64_t nnz, const void* w_dec, int64_t swn, int64_t swd, int w_dt, int64_t d_sae,
              const void* b_dec, int bdec_dt, void* out, int64_t som, int64_t sod, int out_dt,
              int64_t M, int64_t D, const int32_t* tile_cfg, void* stream);

/* Row-wise top-k of f [M, N]: values [M, k] (f_dt) sorted descending, indices int32
 * [M, k]; equal values are taken and ordered by increasing column. Replaces
 * f.topk(k, dim=-1) in ops._topk (reference ops.py:12-16). 0 <= k <= N: for k <= 1024 the
 * selection is sorted in LDS; above, it is staged and sorted in the output row itself, so
 * any k works without a workspace. */
SF_API int sf_topk(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N,
            int64_t k, void* values, int32_t* indices, void* stream);

/* sf_topk of the live rows i < clamp(*n_rows - row_off, 0, M) of f (a count in device memory),
 * row i written to row out_rows[row_off + i] of values / indices [M_out, k]; out_rows holds at
 * least *n_rows entries and names distinct targets (two rows written to one target race);
 * targets outside [0, M_out) are skipped and no other output row is touched. With sf_encode_gather it replaces
 * the overflowed rows of sf_rows_topk's result without a host read (reference ops.py:12-16). */
SF_API int sf_topk_gather(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N, int64_t k,
                   const int32_t* n_rows, int64_t row_off, const int32_t* out_rows, int64_t M_out,
                   void* values, int32_t* indices, void* stream);

/* Dense [M, d_sae] (out_dt, row-major with row stride som) from CSR; entries outside
 * [0, d_sae) are dropped, duplicate columns are summed in entry order. Replaces
 * torch.sparse_csr_tensor(...).to_dense() in csr_to_dense (reference decode.py:123-126)
 * and zeros.scatter_ in ops.encode's TopK branch (ops.py:21-25). indptr NULL means
 * fixed-width rows of `width` entries (indptr = arange(M+1)*width, ops.py:35), placed as
 * scatter_ places them: each value stored as it is (-0.0 included), and a column repeated
 * in a row (never the case for top-k output) keeps one of its values. */
SF_API int sf_csr_to_dense(const int64_t* indptr, int64_t width, const int32_t* indices,
                    const void* values, int val_dt, int64_t nnz, int64_t M, int64_t d_sae,
                    void* out, int64_t som, int out_dt, void* stream);

/* ---------------------------------------------------------------------------------------
 * Backward of the sparse path, for training SAEs on sparse features. The reference has these
 * only on its roadmap (saeflow README.md:244); they differentiate its forward
 * (reference.py:36-52 with the CSR of ops.encode_sparse, ops.py:29-39):
 *   x' = cast_W(x - b_dec), pre = x' W_enc + b_enc, f = act(pre), x_hat = f W_dec + b_dec.
 * Composition (saeflow_amd/kernels/backward.py): sf_csr_transpose -> sf_shifted_input ->
 * sf_backward_bounds / sf_backward_plan -> sf_backward_columns (dL/dpre, dW_dec, dW_enc,
 * db_enc), then sf_column_sums and sf_matvec for db_dec, and, when x needs a gradient,
 * sf_transpose + sf_decode for dx'. All sums are fp32 in a fixed order.
 * --------------------------------------------------------------------------------------- */

/* Bytes of workspace sf_csr_transpose needs. */
SF_API int sf_csr_transpose_workspace_size(int64_t M, int64_t N, int64_t nnz, int64_t* bytes);

/* CSR [M, N] -> CSC: colptr int64 [N+1]; csc_row / csc_pos int32 [nnz] hold, per column in
 * increasing row order, each entry's row and its position in the CSR arrays. Deterministic.
 * Entries with an index outside [0, N) are left out (colptr[N] counts the rest). Beyond 2^23
 * columns, M <= 2^18. workspace: sf_csr_transpose_workspace_size bytes. */
SF_API int sf_csr_transpose(const int64_t* indptr, const int32_t* indices, int64_t M, int64_t N, int64_t nnz,
                     int64_t* colptr, int32_t* csc_row, int32_t* csc_pos, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* xs [M, D] (dt, contiguous) = cast_dt(fp32(x) - fp32(b_dec)): the encoder's MFMA operand
 * (reference encode.py:72). x [M, D] strides (sxm, sxk). */
SF_API int sf_shifted_input(const void* x, int64_t sxm, int64_t sxk, int x_dt, const void* b_dec, int bdec_dt,
                     int64_t M, int64_t D, int dt, void* xs, void* stream);

/* Bounds of the work plan of sf_backward_columns, on the host: max_items = min(N, nnz) +
 * nnz/256 + 1 work items, max_slots = nnz/65 + 1 fp32 partial slots at most, and the fp32
 * work buffer it needs, (ceil(ceil(D / (16 / sizeof(dt))) / 64) + 1) * nnz floats. */
SF_API int sf_backward_bounds(int64_t N, int64_t nnz, int64_t D, int dt, int64_t* max_items, int64_t* max_slots,
                       int64_t* work_floats);

/* Work plan of sf_backward_columns: a column of n CSC entries is ceil(n / 256) work items (an
 * unused column none: its rows are zero-filled); a heavy column (n > 64) also gets as many
 * fp32 partial slots. plan_i64: int64 [3(N+1)] = item_off, slot_off, multi_off (exclusive
 * scans of the items, slots and heavy flags per column, computed from colptr in one batched
 * scan); item_col: int32 [max_items], the column of each work item; multi_col: int32 [N], the
 * heavy columns in increasing order; slot_item: int32 [max_slots], the work item of each
 * slot. No host read. */
SF_API int sf_backward_plan(const int64_t* colptr, int64_t N, int64_t nnz, int64_t* plan_i64, int32_t* item_col,
                     int32_t* multi_col, int32_t* slot_item, void* stream);

/* Per feature j, over its CSC entries (token m, CSR position e) in increasing m, in work items
 * of at most 256 entries (one wave per item and 512-element slab of D):
 *   g_pre[e]      = (g_xhat[m] . w_dec[j] + g_val[e]) * [values[e] > 0]   (fp32 [nnz], CSR
 *                   order; entries with an index outside [0, N) get 0; g_val [nnz] optional
 *                   dL/df)
 *   d_wdec[j]     = sum values[e] * g_xhat[m]      ([N, D], dt)
 *   d_wenc[:, j]  = sum g_pre[e] * xs[m]           ([D, N] contiguous, dt: dL/dW_enc)
 *   d_benc[j]     = sum g_pre[e]                   (fp32 [N])
 * act'(pre) is 1 exactly where f > 0 for relu, jumprelu and the top-k of relu. fp32
 * accumulation; the dot product is summed per slab, the slabs in order; a heavy column sums
 * fp32 partials (partials: fp32 [max_slots * (2*D + 1)]) in item order; unused columns get
 * zero d_wdec rows, d_wenc columns and d_benc. max_items: item_off[N] (plan_i64[N]) read
 * back, or any bound of it such as sf_backward_bounds's (surplus waves return at once);
 * plan_i64, item_col, multi_col, slot_item and max_slots as given to and bounded for
 * sf_backward_plan. w_dec [N, D] rows of stride sw, xs and g_xhat [M, D] rows of strides sx,
 * sg, all of dtype dt. work: fp32 of at least work_floats of sf_backward_bounds. */
SF_API int sf_backward_columns(const int64_t* colptr, const int32_t* csc_row, const int32_t* csc_pos,
                        const int64_t* plan_i64, const int32_t* item_col, const int32_t* multi_col,
                        const int32_t* slot_item, int64_t max_items, int64_t max_slots, const void* values,
                        int val_dt, const void* g_val, int gval_dt, const void* w_dec, int64_t sw, const void* xs,
                        int64_t sx, const void* g_xhat, int64_t sg, int dt, int64_t N, int64_t M, int64_t D,
                        int64_t nnz, float* g_pre, void* d_wdec, void* d_wenc, float* d_benc,
                        float* partials, float* work, int64_t work_floats, void* stream);

/* dst [C, R] (contiguous) = transpose of src [R, C] (row stride ss), dtype dt. skip_ptr: NULL,
 * or int64 [R+1] offsets (a CSC colptr) under which a source row r with skip_ptr[r+1] ==
 * skip_ptr[r] reads as zeros and is not accessed (rows of unused features). */
SF_API int sf_transpose(const void* src, int64_t R, int64_t C, int64_t ss, int dt, const int64_t* skip_ptr, void* dst,
                 void* stream);

/* out[d] (fp32) = sign * sum_m A[m, d] (+ out[d] when accumulate) for A [M, D] of row stride sa
 * and unit column stride, in a fixed order through min(256, M) partial sums; workspace fp32 of
 * at least min(256, max(M, 1)) * D floats. */
SF_API int sf_column_sums(const void* A, int64_t M, int64_t D, int64_t sa, int dt, float sign, int accumulate,
                   float* out, float* workspace, int64_t workspace_floats, void* stream);

/* out[r] (fp32) = sign * sum_c W[r, c] v[c] (+ out[r] when accumulate) for W [R, C] of strides
 * (swr, swc), v fp32 [C]; partial sums over fixed ranges, added in order. workspace: fp32 of at
 * least R * min(256, max(C, 1)) floats. The encoder's share of db_dec: sum_m dx'[m] =
 * W_enc db_enc. */
SF_API int sf_matvec(const void* W, int64_t R, int64_t C, int64_t swr, int64_t swc, int w_dt, const float* v,
              float sign, int accumulate, float* out, float* workspace, int64_t workspace_floats, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAEFLOW_HIP_H */
