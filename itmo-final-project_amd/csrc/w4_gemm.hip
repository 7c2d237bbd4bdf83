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
                   void* ws, size_t ws_bytes, hipStream_t st);
int w4_gemv_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st);
int w4_skinny_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st);
int w4_prefill_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                      int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                      void* y, int64_t ldy, hipStream_t st);

// Reference regime boundary: M <= SMALL_M = 64 uses split-K (gemm.py:17, 265).
static constexpr int64_t kSmallM = 64;
// Decode-shaped products (activations staged in LDS) up to this M.
static constexpr int64_t kDecodeM = 16;

extern "C" size_t w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size) {
  if (M < 1 || M > kSmallM || N < 1 || K < 8 || group_size < 8) return 0;
  if (M <= kDecodeM) return w4_gemv_workspace_bytes(M, N, K, group_size);
  // Sized for the 16-byte-aligned layout (the larger of the two plans).
  const size_t a = w4_skinny_workspace_bytes(M, N, K, (N % 4) == 0);
  const size_t b = w4_skinny_workspace_bytes(M, N, K, false);
  return a > b ? a : b;
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
  if (M <= kDecodeM)
    return w4_gemv_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                          workspace, workspace_bytes, st);
  if (M <= kSmallM)
    return w4_skinny_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y,
                            ldy, workspace, workspace_bytes, st);
  return w4_prefill_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                           st);
}

extern "C" int w4a16_gemm_grouped(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                                  void* stream) {
  clear_error();
  if (count < 1 || count > W4_MAX_GROUPED)
    return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: count must be in [1, %d]", W4_MAX_GROUPED);
  if (!problems) return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: null problem list");
  if (x_dtype != W4_DTYPE_BF16 && x_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: x dtype must be bf16 or fp16");
  if (M < 1 || M > kDecodeM) return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: M must be in [1, 16]");
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    if (!q.x || !q.qweight || !q.scales || !q.zeros || !q.y)
      return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: null pointer in problem %d", i);
    const int64_t G = q.group_size;
    if (q.N < 1 || q.K < 8 || q.K % 8 != 0 || G < 8 || !is_pow2(G) || q.K % G != 0)
      return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: bad shape in problem %d (N=%lld K=%lld G=%d)", i,
                  (long long)q.N, (long long)q.K, q.group_size);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rc = w4_gemv_grouped_launch(problems, count, x_dtype, M, st);
  if (rc != W4_ERR_UNSUPPORTED) return rc;
  return w4_skinny_grouped_launch(problems, count, x_dtype, M, st);
}
