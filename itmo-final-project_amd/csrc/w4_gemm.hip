// w4a16_gemm: argument validation and regime dispatch (the C-ABI counterpart
// of int4_triton/gemm.py:234-309).
#include <hip/hip_runtime.h>

#include "w4_common.hpp"

using namespace w4host;

size_t w4_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, bool vec4_ok);
bool w4_skinny_vec4_ok(const void* qweight, const void* scales, const void* zeros, int64_t N);
int w4_skinny_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                     int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                     void* y, int64_t ldy, void* ws, size_t ws_bytes, hipStream_t st);
size_t w4_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, int G);
int w4_gemv_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                   const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, void* y, int64_t ldy,
                   unsigned* counters, void* ws, size_t ws_bytes, hipStream_t st);
int w4_gemv_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                           unsigned* counters, void* scratch, size_t scratch_bytes, hipStream_t st);
int64_t w4_gemv_grouped_scratch_bytes(const w4a16_problem* problems, int count, int64_t M);
int w4_prefill_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                      int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                      void* y, int64_t ldy, void* ws, size_t ws_bytes, hipStream_t st);
size_t w4_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K);
int w4_prefill_fast_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                           int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                           void* y, int64_t ldy, void* ws, size_t ws_bytes, hipStream_t st);

// Reference regime boundary: M <= SMALL_M = 64 uses split-K (gemm.py:17, 265).
int w4_prefill_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st);

static constexpr int64_t kSmallM = 64;
// Decode-shaped products (activations staged in LDS) up to this M.
static constexpr int64_t kDecodeM = 16;
// Up to this M, products whose every operand fits the decode kernel's
// 64-column tiles (K <= 4096, group >= 64, aligned, dense activation rows) take
// it too (two 16-row MFMA blocks, no split-K partials); others the split-K path.
static constexpr int64_t kDecode32M = 32;

int w4_decode_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count,
                     int x_dtype, int64_t M, hipStream_t st);

// Every workspace starts with a W4_WORKSPACE_COUNTER_BYTES area of per-tile
// arrival counters (zero before first use, left zero by every call), then
// scratch (fp32 partial sums).
extern "C" size_t w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size) {
  if (M < 1 || N < 1 || K < 8 || group_size < 8) return 0;
  size_t scratch;
  if (M > kSmallM) {
    scratch = w4_prefill_workspace_bytes(M, N, K);
  } else if (M <= kDecodeM) {
    // dense rows take the decode / gemv kernels, strided or unaligned rows the
    // skinny split-K kernel (whose split count may differ): room for either
    const size_t a = w4_gemv_workspace_bytes(M, N, K, group_size);
    const size_t b = w4_skinny_workspace_bytes(M, N, K, (N % 4) == 0);
    const size_t c = w4_skinny_workspace_bytes(M, N, K, false);
    scratch = a > b ? a : b;
    scratch = scratch > c ? scratch : c;
  } else {
    // the pipelined MFMA kernel or, for strided / unaligned / K % 64 != 0
    // operands, the skinny kernel: room for either
    const size_t a = w4_skinny_workspace_bytes(M, N, K, (N % 4) == 0);
    const size_t b = w4_skinny_workspace_bytes(M, N, K, false);
    const size_t c = w4_prefill_workspace_bytes(M, N, K);
    scratch = a > b ? a : b;
    scratch = scratch > c ? scratch : c;
  }
  return scratch > 0 ? W4_WORKSPACE_COUNTER_BYTES + scratch : 0;
}

static void split_workspace(void* ws, size_t ws_bytes, unsigned** counters, void** scratch, size_t* scratch_bytes) {
  if (ws == nullptr || ws_bytes < W4_WORKSPACE_COUNTER_BYTES || ((uintptr_t)ws % 256) != 0) {
    *counters = nullptr;
    *scratch = nullptr;
    *scratch_bytes = 0;
    return;
  }
  *counters = static_cast<unsigned*>(ws);
  *scratch = static_cast<char*>(ws) + W4_WORKSPACE_COUNTER_BYTES;
  *scratch_bytes = ws_bytes - W4_WORKSPACE_COUNTER_BYTES;
}

extern "C" int w4a16_gemm(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                          int64_t stride_xm, int64_t stride_xk, const int32_t* qweight,
                          const uint16_t* scales, const uint16_t* zeros, int group_size, void* y,
                          int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (x_dtype != W4_DTYPE_BF16 && x_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4a16_gemm: x dtype must be bf16 or fp16 (got code %d)", x_dtype);
  if (M < 0 || N < 0 || K < 8 || K % 8 != 0)
    return fail(W4_ERR_INVALID, "w4a16_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  const int64_t G = group_size;
  if (G < 8 || !is_pow2(G) || K % G != 0)
    return fail(W4_ERR_INVALID, "w4a16_gemm: group_size %d must be a power of two >= 8 dividing K=%lld",
                group_size, (long long)K);
  if (ldy < N) return fail(W4_ERR_INVALID, "w4a16_gemm: ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
  if (M == 0 || N == 0) return W4_OK;
  if (!x || !qweight || !scales || !zeros || !y) return fail(W4_ERR_INVALID, "w4a16_gemm: null pointer");
  if (((uintptr_t)x % 2) != 0 || ((uintptr_t)y % 2) != 0)
    return fail(W4_ERR_INVALID, "w4a16_gemm: x and y must be 2-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned* counters;
  void* scratch;
  size_t scratch_bytes;
  split_workspace(workspace, workspace_bytes, &counters, &scratch, &scratch_bytes);
  if (M <= kDecodeM)
    return w4_gemv_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                          counters, scratch, scratch_bytes, st);
  if (M <= kDecode32M && stride_xk == 1) {
    const w4a16_problem q{x, qweight, scales, zeros, y, N, K, (int32_t)G, 0};
    const int rc = w4_decode_launch(&q, &stride_xm, &ldy, 1, x_dtype, M, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
  }
  if (M <= kSmallM) {
    const int rc = w4_prefill_fast_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros,
                                          (int)G, y, ldy, scratch, scratch_bytes, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
    return w4_skinny_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y,
                            ldy, scratch, scratch_bytes, st);
  }
  return w4_prefill_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                           scratch, scratch_bytes, st);
}

static int check_grouped(const w4a16_problem* problems, int count, int64_t M) {
  if (count < 1 || count > W4_MAX_GROUPED)
    return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: count must be in [1, %d]", W4_MAX_GROUPED);
  if (!problems) return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: null problem list");
  if (M < 1) return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: M must be >= 1");
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    if (!q.x || !q.qweight || !q.scales || !q.zeros || !q.y)
      return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: null pointer in problem %d", i);
    const int64_t G = q.group_size;
    if (q.N < 1 || q.K < 8 || q.K % 8 != 0 || G < 8 || !is_pow2(G) || q.K % G != 0)
      return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: bad shape in problem %d (N=%lld K=%lld G=%d)", i,
                  (long long)q.N, (long long)q.K, q.group_size);
  }
  return W4_OK;
}

extern "C" size_t w4a16_grouped_workspace_bytes(const w4a16_problem* problems, int count, int64_t M) {
  clear_error();
  if (check_grouped(problems, count, M) != W4_OK) return 0;
  if (M > kDecodeM) {  // room for the separate launches that may replace the shared one
    size_t most = 0;
    for (int i = 0; i < count; ++i) {
      const size_t b = w4a16_workspace_bytes(M, problems[i].N, problems[i].K, problems[i].group_size);
      most = b > most ? b : most;
    }
    return most;
  }
  const int64_t scratch = w4_gemv_grouped_scratch_bytes(problems, count, M);
  return scratch > 0 ? W4_WORKSPACE_COUNTER_BYTES + (size_t)scratch : 0;
}

extern "C" int w4a16_gemm_grouped(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (x_dtype != W4_DTYPE_BF16 && x_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: x dtype must be bf16 or fp16");
  const int rc = check_grouped(problems, count, M);
  if (rc != W4_OK) return rc;
  if (M > kDecodeM) {
    // up to 32 rows, one decode launch when every problem fits its 64-column
    // tiles; else one launch when the products share their activation matrix,
    // else one w4a16_gemm per problem, in order, on the stream (x rows of K
    // elements)
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M <= kDecode32M) {
      int64_t sxm[W4_MAX_GROUPED];
      for (int i = 0; i < count; ++i) sxm[i] = problems[i].K;
      const int drc = w4_decode_launch(problems, sxm, nullptr, count, x_dtype, M, st);
      if (drc != W4_ERR_UNSUPPORTED) return drc;
    }
    const int grc = w4_prefill_grouped_launch(problems, count, x_dtype, M, st);
    if (grc != W4_ERR_UNSUPPORTED || w4_last_error()[0] != '\0') return grc;
    for (int i = 0; i < count; ++i) {
      const w4a16_problem& q = problems[i];
      const int r = w4a16_gemm(q.x, x_dtype, M, q.N, q.K, q.K, 1, q.qweight, q.scales, q.zeros, q.group_size,
                               q.y, q.N, workspace, workspace_bytes, stream);
      if (r != W4_OK) return r;
    }
    return W4_OK;
  }
  unsigned* counters;
  void* scratch;
  size_t scratch_bytes;
  split_workspace(workspace, workspace_bytes, &counters, &scratch, &scratch_bytes);
  const int lrc = w4_gemv_grouped_launch(problems, count, x_dtype, M, counters, scratch, scratch_bytes,
                                         static_cast<hipStream_t>(stream));
  if (lrc == W4_ERR_UNSUPPORTED && w4_last_error()[0] == '\0')
    return fail(W4_ERR_UNSUPPORTED,
                "w4a16_gemm_grouped: a problem exceeds 2 GiB of packed weights or the column tiles of the "
                "split problems exceed the counter area");
  return lrc;
}

