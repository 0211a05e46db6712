/* crbq.h - C ABI of the MI355X-native CRB layer-wise binarization quantizer.
 *
 * Every pointer argument named as "device" is a device pointer owned by the
 * caller (for the Python host: the PyTorch caching allocator).  The library
 * never allocates device memory: scratch space comes in through `ws`
 * (size from the matching *_workspace_size query), or, for
 * crbq_fasterquant_noalloc, is a static device array of the library.  `stream` is a
 * hipStream_t passed as void*; NULL means the default stream.  Every entry
 * point returns a status: 0 = ok, < 0 = error (see crbq_status_string), and
 * never throws across the ABI.  Entry points that must read a device result
 * to continue (the Cholesky retry loop) synchronise `stream`.
 *
 * Reference interface replaced (paths relative to the SDMuhsin/CRB root):
 *   BRAGPTQ.add_batch            bigptq.py:37-53
 *   BRAGPTQ.fasterquant          bigptq.py:56-291
 *   structural_guassian_distribution / structural_searching /
 *   generate_structural_mask     utils/structure.py:8-20,
 *                                utils/autosearch.py:28-83, utils/mask.py:7-18
 *   Binarization.quantize        binary.py:2850-2890 ->
 *                                high_order_residual binary.py:18-39,
 *                                coupled_residual_binarization binary.py:577-687,
 *                                coupled_residual_binarization_stable_v7
 *                                binary.py:1544-1638
 */
#ifndef CRBQ_H
#define CRBQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define CRBQ_OK              0
#define CRBQ_ERR_ARG        -1   /* bad size, stride, enum or alignment */
#define CRBQ_ERR_HIP        -2   /* a HIP runtime call failed */
#define CRBQ_ERR_WORKSPACE  -3   /* workspace pointer NULL or too small */
#define CRBQ_ERR_TOPK       -4   /* block narrower than the salient search limit
                                    (torch.topk k out of range, utils/autosearch.py:42) */
#define CRBQ_ERR_TOO_LARGE  -5   /* problem needs more scratch than the
                                    allocation-free entry point holds */
#define CRBQ_ERR_CAPTURE    -6   /* allocation-free entry point first called on a
                                    device while its stream is capturing: its
                                    one-time set-up copies cannot be captured */

/* ---- enums -------------------------------------------------------------- */
enum crbq_dtype  { CRBQ_F32 = 0, CRBQ_F16 = 1, CRBQ_BF16 = 2 };
/* Binarization methods in scope (binary.py:2875-2890). */
enum crbq_method {
  CRBQ_BRAQ = 0,                 /* high_order_residual                     */
  CRBQ_CRB = 1,                  /* ..._stable_v7                            */
  CRBQ_CRBOG = 2,                /* coupled_residual_binarization            */
  CRBQ_CRB_NOREFINE = 3,         /* v7, skip_refinement=True                 */
  CRBQ_CRB_SYMDAMP = 4,          /* v7, symmetric_damp=True                  */
  CRBQ_CRB_SYMDAMP_NOREFINE = 5  /* v7, both                                 */
};
enum crbq_metric { CRBQ_METRIC_MAGNITUDE = 0, CRBQ_METRIC_HESSIAN = 1 };

/* Quantizer hyper-parameters of one fasterquant call
 * (bigptq.py:56-62, binary.py:2851-2866, run.py:868-873). */
typedef struct crbq_params {
  int32_t method;        /* enum crbq_method                                 */
  int32_t metric;        /* enum crbq_metric (salient_metric)                */
  int32_t blocksize;     /* column block, 1..128 (reference default 128)     */
  int32_t partition;     /* 3 = salient/bell split; 1 = one all-ones mask    */
  int32_t orders[3];     /* binarization order per mask (default 1,1,2)      */
  int32_t up_lim;        /* salient-column search limit (50, bigptq.py:142)  */
  int32_t refine_iters;  /* CRB sign-refinement rounds (reference: 1)        */
  int32_t disable_gptq;  /* 1 = RTN: no error feedback (bigptq.py:149-162)   */
  float   lam;           /* CRB Tikhonov term (1e-5)                          */
  float   corr_damp;     /* CRB correlation damping (0.1)                     */
} crbq_params;

/* Per-block search record (filled when a trace buffer is given).
 * errs_a[i] = summed squared error of salient candidate i (index 0 unused),
 * errs_c[k] = summed squared error of split candidate k, without the
 * constant salient-group term. */
typedef struct crbq_block_trace {
  int32_t i_star;        /* number of salient columns chosen                 */
  int32_t k_star;        /* index of the chosen percentile split             */
  float   split;         /* chosen split value                                */
  float   pvals[81];     /* the 81 float32 percentiles (np.quantile)         */
  double  errs_a[64];
  double  errs_c[81];
} crbq_block_trace;

/* ---- library ------------------------------------------------------------ */
int         crbq_version(void);
const char* crbq_status_string(int status);
/* 0 when the current HIP device is a gfx950 (MI355X), else < 0. */
int         crbq_device_ok(void);
/* The 81 float32 split percentiles, torch.linspace(0.10, 0.90, 81) as the
 * host's torch computes it on the CPU (utils/autosearch.py:65; its last bits
 * depend on the CPU's vector width).  q81: host pointer.  Without this call
 * the library uses torch's scalar formula. */
int         crbq_set_percentiles(const float* q81);

/* ---- Hessian accumulation (BRAGPTQ.add_batch, bigptq.py:37-53) ---------
 * S[i,j] += sum_t X[t,i] * X[t,j] over ntok token rows of X (row stride ldx
 * elements, dtype enum crbq_dtype), for the upper triangle i <= j of the
 * fp32 C x C matrix S (row stride lds).  f16/bf16 products are exact and
 * accumulate in fp32 on MFMA; fp32 inputs use the fp32 MFMA.
 * The reference's running rescale H *= n/(n+b); H += (2/n) X^T X is applied
 * once, in crbq_hessian_finalize, which gives the same H up to rounding.
 * 16-bit inputs with C a multiple of 256, ldx a multiple of 8 and X 16-byte
 * aligned are staged into LDS as they are; ws (optional,
 * crbq_hessian_workspace_size bytes; may be NULL) then holds the per-split
 * partial sums, used when the token range is split across workgroups to
 * fill the GPU (added to S in a fixed order), and a few control words.
 * Other 16-bit inputs: ws also holds a channel-major copy of X (C rounded
 * up to 256 rows of up to 2^21 tokens, at most 8 GiB per pass; longer
 * inputs run in passes), bitwise the same sums; with a workspace too small
 * for it (or NULL) the SYRK transposes X in registers, a slower path with
 * the same result up to summation order.  fp32 inputs use no workspace.
 * The environment variable CRBQ_XT_PASS_TOKENS (read per call) lowers the
 * pass length of the copy. */
size_t crbq_hessian_workspace_size(int64_t ntok, int64_t C);
int crbq_hessian_accum(const void* X, int dtype, int64_t ntok, int64_t ldx,
                       int64_t C, float* S, int64_t lds, void* ws, size_t ws_bytes,
                       void* stream);
/* The same Hessian update from a channel-major copy of the activations that
 * the caller builds (for callers that gather the activations of several
 * forwards before one update: the stack driver's deferred Hessians,
 * run.py:341-374, whose copy of each forward's activations into the store
 * is then the transpose; crbq_hessian_accum on a token-major store gives
 * the same sums).
 *   crbq_hessian_cm_shape: the store's shape for ntok tokens of C channels:
 *     *rows = C rounded up to 256, *ldt = ntok rounded up to 64 (at most
 *     2^21 tokens);
 *   crbq_hessian_transpose: writes ntok token rows of X (16-bit, row stride
 *     ldx) into columns [t0, t0 + ntok rounded up to 64) of the store Xt
 *     (rows x ldt halves, 16-byte aligned; t0 a multiple of 64), zeros in
 *     the padding rows and columns; fill the store in token order so every
 *     column up to ldt is written;
 *   crbq_hessian_accum_cm: S += Xt Xt^T over the first ntok columns
 *     (upper triangle), the same sums as crbq_hessian_accum on the same
 *     tokens; ws holds the per-split partial tiles
 *     (crbq_hessian_cm_workspace_size bytes; with less, fewer splits). */
int crbq_hessian_cm_shape(int64_t ntok, int64_t C, int64_t* rows, int64_t* ldt);
int crbq_hessian_transpose(const void* X, int dtype, int64_t ntok, int64_t ldx, int64_t C,
                           void* Xt, int64_t ldt, int64_t t0, void* stream);
size_t crbq_hessian_cm_workspace_size(int64_t ntok, int64_t C);
int crbq_hessian_accum_cm(const void* Xt, int dtype, int64_t ntok, int64_t ldt, int64_t C,
                          float* S, int64_t lds, void* ws, size_t ws_bytes, void* stream);
/* SYRK launch timing, a profiling aid with no counterpart in the reference.
 * While on != 0, crbq_hessian_accum records a pair of HIP events on its
 * stream right before and right after each SYRK kernel launch (process-wide
 * switch).  crbq_syrk_timing_collect waits for the recorded launches,
 * writes up to max (ms, C) pairs, oldest first, sets *n to the number
 * recorded, and forgets them. */
int crbq_syrk_timing(int on);
int crbq_syrk_timing_collect(float* ms, int64_t* C, int max, int* n);
/* H[i,j] = scale * S[min(i,j), max(i,j)] for all i, j (H may alias S). */
int crbq_hessian_finalize(const float* S, int64_t lds, int64_t C, float scale,
                          float* H, int64_t ldh, void* stream);

/* ---- inverse-Hessian factor (fasterquant prologue, bigptq.py:101-129) ----
 * Dead columns (diag(H) == 0 -> H_ii = 1, W[:, i] = 0), damping
 * H_ii += percdamp * mean(diag H), Cholesky with up to 10 retries adding
 * 1e-3 * mean(diag H) (1e-6 if that is 0), diagonal fallback, and
 * U = upper Cholesky factor of H^-1, written to U (C x C, row stride ldu,
 * zero below the diagonal).  H is modified like the reference's.  U is
 * computed as J L'^-1 J with L' = chol(J H J) (J = index reversal), which is
 * the same matrix in 2C^3/3 flops instead of 4C^3/3.
 * W may be NULL (then dead columns are not cleared).  retries/fallback: host
 * pointers (may be NULL).  Synchronises `stream`. */
size_t crbq_hinv_workspace_size(int64_t C);
int crbq_hinv_upper(float* H, int64_t ldh, int64_t C, float* W, int64_t R,
                    int64_t ldw, float percdamp, float* U, int64_t ldu,
                    void* ws, size_t ws_bytes, int* retries, int* fallback,
                    void* stream);
/* The same in two steps, so several factorizations can run concurrently on
 * different streams: _async enqueues dead-column handling, damping and the
 * first attempt (no synchronisation); _finish synchronises `stream`, checks
 * the outcome and runs any retries / the fallback.  Both calls take the
 * same H, U and workspace. */
int crbq_hinv_upper_async(float* H, int64_t ldh, int64_t C, float* W, int64_t R,
                          int64_t ldw, float percdamp, float* U, int64_t ldu,
                          void* ws, size_t ws_bytes, void* stream);
int crbq_hinv_upper_finish(float* H, int64_t ldh, int64_t C, float* U, int64_t ldu,
                           void* ws, size_t ws_bytes, int* retries, int* fallback,
                           void* stream);

/* ---- block loop (BRAGPTQ.fasterquant, bigptq.py:131-264) -----------------
 * Quantizes W (R x C fp32, row stride ldw) in place, column block by column
 * block: salient/bell mask search, binarization, Err/Loss, and the GPTQ
 * trailing update W[:, ed:] -= Err @ U[st:ed, ed:].  losses (R floats) is
 * accumulated (+= per-row loss sum / 2), like Losses in the reference.
 * masks (optional, R x C uint8, row stride ldm): 1/2/3 = mask1/2/3 member.
 * traces (optional, device array of ceil(C/blocksize) crbq_block_trace). */
size_t crbq_fasterquant_workspace_size(int64_t R, int64_t C,
                                       const crbq_params* p);
int crbq_fasterquant(float* W, int64_t R, int64_t C, int64_t ldw,
                     const float* U, int64_t ldu, const crbq_params* p,
                     float* losses, uint8_t* masks, int64_t ldm,
                     crbq_block_trace* traces, void* ws, size_t ws_bytes,
                     void* stream);

/* crbq_fasterquant over nseg (1..4) sublayers of one shape (R x C, row
 * stride ldw), each with its own inverse factor U[i] (row stride ldu;
 * entries may repeat): q/k/v/out of an attention block, gate/up of a gated
 * MLP.  Replaces nseg consecutive calls of gptq[name].fasterquant(...) in
 * the per-sublayer loop of run.py:286-305 (BRAGPTQ.fasterquant,
 * bigptq.py:56-291).  W, U, losses, masks and traces are HOST arrays of
 * nseg device pointers (masks and traces may be NULL, or arrays whose
 * entries are all NULL); the sublayers' weights, losses, masks and traces
 * must not overlap (the same pointer twice is rejected with CRBQ_ERR_ARG).
 * Every sublayer's results are bit for bit those of its own
 * crbq_fasterquant call with the same params.  The block loop runs
 * once, each search, quantize and update launch covering all nseg
 * sublayers.  Workspace: crbq_fasterquant_batched_workspace_size. */
size_t crbq_fasterquant_batched_workspace_size(int32_t nseg, int64_t R, int64_t C,
                                               const crbq_params* p);
int crbq_fasterquant_batched(int32_t nseg, float* const* W, int64_t R, int64_t C,
                             int64_t ldw, const float* const* U, int64_t ldu,
                             const crbq_params* p, float* const* losses,
                             uint8_t* const* masks, int64_t ldm,
                             crbq_block_trace* const* traces, void* ws,
                             size_t ws_bytes, void* stream);

/* Allocation-free variant of crbq_fasterquant.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as crbq_fasterquant without the
 * workspace: the scratch it needs (crbq_fasterquant_workspace_size(R, C, p)
 * bytes) lives in a static device array of CRBQ_NOALLOC_SCRATCH_BYTES per
 * device, which every GPU the library runs on holds until the process
 * ends; larger problems (for blocksize 128: R above about 18000 rows)
 * return CRBQ_ERR_TOO_LARGE.  It calls no hipMalloc / hipFree.  All calls
 * on one device share that device's scratch, so calls that overlap on one
 * GPU (different streams, or host threads) race: serialize them. */
#define CRBQ_NOALLOC_SCRATCH_BYTES ((size_t)80 << 20)
int crbq_fasterquant_noalloc(float* W, int64_t R, int64_t C, int64_t ldw,
                             const float* U, int64_t ldu, const crbq_params* p,
                             float* losses, uint8_t* masks, int64_t ldm,
                             crbq_block_trace* traces, void* stream);

/* ---- one-block pieces (for tests and the Binarization API) --------------
 * Search of one column block (utils/structure.py:8-20): writes the
 * R x ncols mask codes 1/2/3 (row stride ldm) and, optionally, a trace. */
size_t crbq_block_search_workspace_size(int64_t R, int32_t up_lim);
int crbq_block_search(const float* W, int64_t R, int32_t ncols, int64_t ldw,
                      const float* Ublk, int64_t ldu, int32_t metric,
                      int32_t up_lim, uint8_t* masks, int64_t ldm,
                      crbq_block_trace* trace, void* ws, size_t ws_bytes,
                      void* stream);
/* Binarization.quantize(x, mask, order) (binary.py:2874-2890) on an
 * R x ncols fp32 matrix with a 0/1 uint8 mask; out may alias x.
 * ncols <= 1024. */
int crbq_binarize(const float* x, int64_t R, int32_t ncols, int64_t ldx,
                  const uint8_t* mask, int64_t ldm, int32_t order,
                  int32_t method, float lam, float corr_damp,
                  int32_t refine_iters, float* out, int64_t ldo, void* stream);
/* crbq_binarize that also writes each row's scales to scales[row * lds ..]
 * (fp32; a row of the reference's per-row tensors):
 *   CRB variants (binary.py:1544-1638), and CRBOG at order >= 2
 *   (binary.py:635-687): (mean, mu correction, a1, a2), 4 values: the row
 *   mean (:1599; CRBOG :653), the mean correction of step 7 (:1633-1635;
 *   0 for CRBOG), the two plane scales after the last solve (:1582-1596,
 *   1615-1630; CRBOG :656-679); order 1 gives (mean, 0, a1, 0)
 *   (:1570-1576);
 *   BRAQ (binary.py:18-39), and CRBOG at order 1 (:595-630): (mu_k, alpha_k)
 *   for each residual pass k < order, 2 * order values.
 * lds must hold them (>= 4, >= 2 * order for BRAQ).  Rows are processed
 * one wavefront each; the values written to out are those of crbq_binarize
 * up to summation order. */
int crbq_binarize_scales(const float* x, int64_t R, int32_t ncols, int64_t ldx,
                         const uint8_t* mask, int64_t ldm, int32_t order,
                         int32_t method, float lam, float corr_damp,
                         int32_t refine_iters, float* out, int64_t ldo,
                         float* scales, int64_t lds, void* stream);
/* C = beta*C + alpha*op(A)*op(B), fp32 on MFMA (the trailing update uses
 * alpha = -1, beta = 1, bigptq.py:264).  transa/transb: op(X) = X^T. */
int crbq_sgemm(int transa, int transb, int64_t M, int64_t N, int64_t K,
               float alpha, const float* A, int64_t lda, const float* B,
               int64_t ldb, float beta, float* C, int64_t ldc, void* stream);

/* ---- packed low-bit storage, GEMV and GEMM --------------------------------
 * No counterpart in the reference, which keeps fake-quantized fp16/bf16
 * weights (bigptq.py:278-280); for inference callers that want the
 * quantized layer in about 3 bits per weight.  Within a 128-column block
 * of a row the quantized weights take 2 values per non-salient group
 * (mask 1, mask 2, order 1) and 4 on the salient columns (mask 3, order 2),
 * and the salient columns are the same for every row, except where a
 * binarizer's sign is exactly 0 (torch.sign of an element equal to its
 * group's mean gives the mean itself): such rare elements are kept as
 * exceptions.  With nblk = ceil(C / 128):
 *   codes [R][ldc] bytes, ldc >= nblk * 32 (multiple of 8, 8-byte aligned): 2 bits per
 *     weight, column j of block b at byte b * 32 + j / 4, bits 2 (j % 4);
 *   lut [R][nblk][8] in the weight dtype (16-byte aligned): mask1 two values,
 *     mask2 two, mask3 four, each group's ascending (-0 below +0); a group
 *     keeps its most frequent values (ties to the smaller), chosen among
 *     its 8 smallest distinct values;
 *   sal [nblk][16] bytes (8-byte aligned): bit j % 8 of byte j / 8 marks salient column j;
 *   weight = lut[r][b][4 * salient + code];
 *   exceptions: the other elements, code = their group's first entry, with
 *     ex_idx = r * C + c (int64), ex_val = the exact 16-bit value and
 *     ex_delta = value - lut entry (fp32); list order unspecified.
 * crbq_pack reads the quantized weights Q (fp16/bf16) and the mask codes
 * (1/2/3, as crbq_fasterquant writes them), fills up to ex_cap exceptions,
 * sets the device int *ex_count to their number and *status to 0, or to
 * an OR of 1 (more than ex_cap exceptions), 2 (salient columns differ
 * between rows), 4 (mask code outside 1..3); the caller reads both after
 * the stream.  crbq_unpack writes the weights back bit for bit.
 * crbq_gemv_packed: y[v][r] = sum_c W[r][c] x[v][c] for nvec <= 16 vectors
 * x in the weights' dtype (ldx multiple of 8, 16-byte aligned), fp32 y;
 * the n_ex exceptions are added as delta * x in list order after the
 * packed product. */
int crbq_pack(const void* Q, int dtype, int64_t R, int64_t C, int64_t ldq,
              const uint8_t* masks, int64_t ldm, uint8_t* codes, int64_t ldc,
              void* lut, uint8_t* sal, int64_t* ex_idx, void* ex_val, float* ex_delta,
              int ex_cap, int* ex_count, int* status, void* stream);
int crbq_unpack(const uint8_t* codes, int64_t ldc, const void* lut, const uint8_t* sal,
                const int64_t* ex_idx, const void* ex_val, int64_t n_ex, int dtype,
                int64_t R, int64_t C, void* Q, int64_t ldq, void* stream);
int crbq_gemv_packed(const uint8_t* codes, int64_t ldc, const void* lut,
                     const uint8_t* sal, const int64_t* ex_idx, const float* ex_delta,
                     int64_t n_ex, int dtype, int64_t R, int64_t C, const void* x,
                     int64_t ldx, int nvec, float* y, int64_t ldy, void* stream);
/* crbq_gemm_packed: Y[t][r] = sum_c W[r][c] X[t][c] for ntok tokens (any
 * count; meant for prefill batches above the GEMV's 16), X in the weights'
 * dtype (ldx multiple of 8, 16-byte aligned), fp32 Y [ntok][ldy], the
 * exceptions added as in the GEMV.  Each decoded weight fragment is reused
 * for 64 tokens (128 above 64).  When the shapes give 256 or fewer row x
 * token tiles (128 rows each) the column blocks are split over workgroups
 * (floor(512 / tiles) splits of at least 8 blocks) whose fp32 partials go to
 * the workspace and are summed in split order (deterministic);
 * crbq_gemm_packed_workspace_size(R, C, ntok) bytes (0 when there is no
 * split) depend on the shapes only. */
size_t crbq_gemm_packed_workspace_size(int64_t R, int64_t C, int64_t ntok);
int crbq_gemm_packed(const uint8_t* codes, int64_t ldc, const void* lut,
                     const uint8_t* sal, const int64_t* ex_idx, const float* ex_delta,
                     int64_t n_ex, int dtype, int64_t R, int64_t C, const void* x,
                     int64_t ldx, int64_t ntok, float* y, int64_t ldy, void* ws,
                     size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRBQ_H */
