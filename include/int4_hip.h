/*
 * int4_hip: C-ABI of the MI355X (gfx950) W4A16 quantize + GEMM library.
 *
 * The reference (homomorfism/itmo-final-project, package int4_triton) exposes
 * this path as Python functions that launch Triton kernels; there is no FFI
 * there.  Each entry point below replaces one of those launch sites, named in
 * its comment (file:line in the reference).  A Python host package
 * (itmo-final-project_amd/int4_hip) binds these symbols with ctypes and keeps
 * the reference's Python names, argument meaning and assertions.
 *
 * Conventions (all entry points):
 *  - Plain pointers, sizes and strides; strides are in ELEMENTS.
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *    Work is enqueued on it; nothing synchronises with the host.
 *  - The library never allocates or frees device memory.  Scratch memory
 *    (split-K partial sums) is passed in as `workspace`.
 *  - Half-precision tensors are passed as 16-bit patterns (uint16_t).
 *  - Return 0 on success, a nonzero W4_ERR_* code on failure; the message of
 *    the last failure on the calling thread is returned by w4_last_error().
 *
 * Storage layout (int4_triton/quantize.py:8-12):
 *   qweight int32 [K/8, N] row-major, nibble i of word (k8, n) = row 8*k8+i of
 *   W^T, i.e. bits 4i..4i+3;  scales, zeros fp16 [K/G, N] row-major.
 */
#ifndef INT4_HIP_H
#define INT4_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4_ABI_VERSION 1

/* dtype codes */
#define W4_DTYPE_BF16 0
#define W4_DTYPE_FP16 1
#define W4_DTYPE_FP32 2

/* Every workspace starts with this many bytes of per-tile arrival counters:
 * zero before the first call that uses the workspace, left zero by every call.
 * The rest is scratch (fp32 partial sums). */
#define W4_WORKSPACE_COUNTER_BYTES 65536

/* status codes */
#define W4_OK 0
#define W4_ERR_INVALID 1     /* bad shape, stride, dtype or group size       */
#define W4_ERR_UNSUPPORTED 2 /* valid for the reference, not implemented    */
#define W4_ERR_WORKSPACE 3   /* workspace missing or smaller than required   */
#define W4_ERR_LAUNCH 4      /* HIP launch error (hipGetLastError)           */

/* Library version; lets bindings reject a stale build. */
int w4_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* w4_last_error(void);

/*
 * Group-wise asymmetric RTN int4 quantization of W[N, K] (bf16 or fp16, any
 * strides) into freshly laid-out qweight int32 [K/8, N], scales/zeros fp16
 * [K/G, N] (dense, row-major).  group_size: power of two, multiple of 8,
 * dividing K; -1 means K (per-channel).  Bit-exact with the reference's torch
 * implementation for every finite input.
 * Replaces: int4_triton/quantize.py:67-96 (quantize_int4 and the launch of
 * _quantize_int4_kernel, :21-64); semantics of quantize_int4_ref, :102-117.
 */
int w4_quantize(const void* w, int w_dtype, int64_t N, int64_t K,
                int64_t stride_wn, int64_t stride_wk, int group_size,
                int32_t* qweight, uint16_t* scales, uint16_t* zeros, void* stream);

/*
 * One weight of a grouped quantize call (w4_quantize's arguments).
 */
typedef struct w4_quantize_problem {
  const void* w;
  int32_t* qweight;
  uint16_t* scales;
  uint16_t* zeros;
  int64_t N;
  int64_t K;
  int64_t stride_wn;
  int64_t stride_wk;
  int32_t group_size;
  int32_t reserved;
} w4_quantize_problem;

/*
 * Up to W4_MAX_GROUPED weights quantized as by w4_quantize (same outputs,
 * bit for bit), all of dtype w_dtype: ONE kernel launch when every weight has
 * dense 16-byte-aligned rows and all share one group size <= 512 (the
 * weights of a decoder block), else one w4_quantize per weight, in order.
 * No single counterpart in the reference: it fuses the per-linear
 * quantize_int4 calls that quantize_model_linears issues for the linears of
 * one block (int4_triton/qlinear.py:55-68, quantize.py:67-96).
 */
int w4_quantize_grouped(const w4_quantize_problem* problems, int count, int w_dtype, void* stream);

/*
 * W_hat[N, K] (dense, row-major) = round_once_to_out_dtype((q - z) * s),
 * computed exactly in fp32.  out_dtype: W4_DTYPE_BF16/FP16/FP32.
 * Replaces: int4_triton/quantize.py:128-135 (dequantize_int4_ref) as used by
 * Int4Linear.dequantize (int4_triton/qlinear.py:39-40) and fake mode (:63-64).
 */
int w4_dequantize(const int32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
                  int64_t N, int64_t K, int group_size, int out_dtype, void* out,
                  void* stream);

/*
 * Bytes of workspace w4a16_gemm needs for this problem (0 when the chosen
 * launch writes y directly).  Depends only on (M, N, K, group_size) and the
 * device's compute-unit count, never on timing, so the split-K decomposition
 * (and therefore every output bit) is the same in every process.  The
 * workspace (256-byte aligned) starts with the W4_WORKSPACE_COUNTER_BYTES
 * counter area, so one zero-filled buffer of the largest size needed can be
 * reused by all calls (w4a16_gemm and w4a16_gemm_grouped) issued on one
 * stream.
 * Replaces: the per-call `partials` allocation, int4_triton/gemm.py:268.
 */
size_t w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size);

/*
 * y[M, N] = x[M, K] @ W_hat^T with W_hat the dequantized int4 weight, fp32
 * accumulation, y in x's dtype.  x: bf16/fp16, any strides (stride_xm,
 * stride_xk).  qweight/scales/zeros dense row-major as above.  y: row stride
 * ldy (>= N), unit column stride.  Launch regimes (same boundaries as the
 * reference): M <= 16 (group sizes >= 32) the factored decode kernel in one
 * launch; 17 <= M <= 64 with dense rows (unit column stride, 16-byte aligned,
 * row stride a multiple of 8) the same kernel in one launch, the rows cut
 * into slices of 16 (in both, a long K is split over workgroups whose fp32
 * partial tiles, in `workspace`, are summed in part order by the last one to
 * finish); other M <= 64 problems (and group sizes < 32) split-K with fp32
 * partials in `workspace` and a fixed-order reduce kernel; M > 64 tiled
 * MFMA GEMM, itself split over K when the shape leaves too few tiles to fill
 * the chip: with the same partials-and-reduce scheme, or (two splits of
 * 128 x 256 tiles, and K > 4096 with few tiles) as K ranges in separate
 * workgroups summed in range order by the last one to finish (partial tiles
 * in `workspace`); 65 <= M <= 128 with
 * N <= 4096 and dense rows takes the decode kernel's row slices (up to
 * eight) like 17 <= M <= 64, except that K > 4096 takes that K-range
 * launch.  Every regime is bit-identical run to run.
 * Replaces: int4_triton/gemm.py:303-309 (w4a16_matmul) and its dispatcher
 * _matmul, :234-300 (kernels :74-157, :171-182, :185-220).
 */
int w4a16_gemm(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
               int64_t stride_xm, int64_t stride_xk,
               const int32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
               int group_size, void* y, int64_t ldy,
               void* workspace, size_t workspace_bytes, void* stream);

/*
 * One problem of a grouped decode launch: y_i[M, N_i] = x_i[M, K_i] @ W_hat_i^T.
 * x_i dense row-major [M, K_i]; y_i dense row-major [M, N_i].
 */
typedef struct w4a16_problem {
  const void* x;
  const int32_t* qweight;
  const uint16_t* scales;
  const uint16_t* zeros;
  void* y;
  int64_t N;
  int64_t K;
  int32_t group_size;
  int32_t reserved;
} w4a16_problem;

#define W4_MAX_GROUPED 8

/*
 * Bytes of workspace w4a16_gemm_grouped needs for these problems (0 if none).
 */
size_t w4a16_grouped_workspace_bytes(const w4a16_problem* problems, int count, int64_t M);

/*
 * Up to W4_MAX_GROUPED independent products, all with the same activation
 * dtype and M; x of every problem is dense ([M, K] rows of K elements), y
 * dense [M, N].
 *   1 <= M <= 16: ONE kernel launch for all problems (the factored decode
 *   kernel).  Problems with a long K may be split over several workgroups whose
 *   fp32 partials meet in a fixed order (in `workspace`).
 *   17 <= M <= 64, and up to M = 128 when every problem has N <= 4096: the
 *   same single decode launch, each problem's rows cut into slices of 16
 *   (group sizes >= 32, 16-byte aligned x), long K split the same way.
 *   Otherwise, M > 16: problems that share one activation matrix (same x pointer, K and
 *   group size; at most 4) run as ONE launch of the prefill kernel (no
 *   split-K, the tiles of all problems side by side) when the library's
 *   static cost model puts it below the separate launches; otherwise each
 *   problem is one w4a16_gemm call, in order, on `stream` (sharing
 *   `workspace`).  The choice is a pure function of the shapes.
 * `workspace`: 256-byte aligned, w4a16_grouped_workspace_bytes long, laid out
 * like w4a16_gemm's.  Reusing one workspace for calls that run concurrently
 * (on different streams) is a race.  Results are bit-identical run to run.
 * No single counterpart in the reference: it fuses the per-linear launches of
 * int4_triton/gemm.py:245-264 that a decoder block issues back to back
 * (q/k/v/o/gate/up/down, benchmarks/bench_gemm.py:18-26).
 */
int w4a16_gemm_grouped(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Scratch memory of w4a16_gemm_noalloc, per GPU: the counter area plus 32 MiB
 * of fp32 partial sums. */
#define W4_NOALLOC_SCRATCH_BYTES (W4_WORKSPACE_COUNTER_BYTES + (32u << 20))

/*
 * w4a16_gemm without a workspace argument and without any allocation: the
 * same validation, launch regimes, kernels and output bits as w4a16_gemm, with
 * the split-K scratch taken from a fixed array inside the library (one per
 * GPU, W4_NOALLOC_SCRATCH_BYTES, held until the process ends).  Problems whose
 * w4a16_workspace_bytes exceeds that size are rejected with W4_ERR_WORKSPACE
 * before anything is launched.  It calls no hipMalloc/hipFree and no
 * allocating library routine; it may enqueue one small fill kernel that
 * zeroes the counter area before the product.
 * All calls on one GPU share its scratch array: calls that may overlap in time
 * on one GPU (on different streams, or from several threads without ordering)
 * race on it and must not be issued.  Calls ordered on one stream are safe.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).
 */
int w4a16_gemm_noalloc(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                       int64_t stride_xm, int64_t stride_xk,
                       const int32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
                       int group_size, void* y, int64_t ldy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INT4_HIP_H */
