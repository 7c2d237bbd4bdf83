// w4a16_gemm: argument validation and regime dispatch (the C-ABI counterpart
// of int4_triton/gemm.py:234-309).
#include <hip/hip_runtime.h>

#include <mutex>

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
                      void* y, int64_t ldy, void* ws, size_t ws_bytes, unsigned* counters, hipStream_t st);
size_t w4_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K);
int w4_prefill_fast_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                           int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                           void* y, int64_t ldy, void* ws, size_t ws_bytes, unsigned* counters, hipStream_t st);
bool w4_prefill_split_route(const void* x, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                            const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, const void* y,
                            int64_t ldy);

int w4_rows_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count, int x_dtype,
                   int64_t M, unsigned* counters, void* scratch, size_t scratch_bytes, hipStream_t st);
size_t w4_rows_workspace_bytes(const w4a16_problem* problems, const int64_t* sxm, int count, int64_t M);

// Reference regime boundary: M <= SMALL_M = 64 uses split-K (gemm.py:17, 265).
int w4_prefill_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st);

static constexpr int64_t kSmallM = 64;
// Decode-shaped products (activations staged in LDS) up to this M.
static constexpr int64_t kDecodeM = 16;
// Up to this M, dense rows run as row slices of kDecodeM in one decode
// launch (four slices at most).
static constexpr int64_t kSliceM = 64;
// A lone product up to this M with N up to kSliceLoneN takes the row slices
// too (eight at most): at M = 128 the prefill kernel's plan for these shapes
// has few tiles and a split-K reduce launch (o_proj 12.5 -> 6.9 us, k_proj
// 8.9 -> 6.4 us, down_proj 19.2 -> 19.1 us), while for N = 8192 (gate_proj)
// it was the faster of the two (19.8 against 20.5 us).  A grouped call above
// kSliceM takes the slices under the same rule, i.e. when every problem has
// N <= kSliceLoneN (q/k/v at M = 128: one launch of 384 workgroups; the 4-call
// block 66.3 -> 59.7 us); with a wider problem (gate/up) it keeps the
// shared-activation prefill launch, which measured faster there (routing
// gate/up through the slices too took the 4-call block to 79.2 us).
static constexpr int64_t kSliceLoneM = 128;
static constexpr int64_t kSliceLoneN = 4096;
static bool sliced_lone(int64_t M, int64_t N) { return M <= kSliceM || (M <= kSliceLoneM && N <= kSliceLoneN); }
static bool sliced_grouped(const w4a16_problem* problems, int count, int64_t M) {
  if (M <= kSliceM) return true;
  if (M > kSliceLoneM) return false;
  for (int i = 0; i < count; ++i)
    if (problems[i].N > kSliceLoneN) return false;
  return true;
}

int w4_decode_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count,
                     int x_dtype, int64_t M, unsigned* counters, void* scratch, size_t scratch_bytes,
                     hipStream_t st, const int64_t* mrows = nullptr);
size_t w4_decode_workspace_bytes(const w4a16_problem* problems, const int64_t* sxm, int count, int64_t M,
                                 const int64_t* mrows = nullptr);
size_t w4_decode_single_workspace_bytes(int64_t M, int64_t N, int64_t K, int G);

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
  if (sliced_lone(M, N)) {
    // the several-row decode kernel's K split (partial tiles)
    const size_t d = w4_decode_single_workspace_bytes(M, N, K, group_size);
    if (d > W4_WORKSPACE_COUNTER_BYTES && d - W4_WORKSPACE_COUNTER_BYTES > scratch)
      scratch = d - W4_WORKSPACE_COUNTER_BYTES;
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

// Argument checks of w4a16_gemm (and w4a16_gemm_noalloc, which runs them
// before it enqueues anything).  Sets *empty for a valid call with nothing to
// compute (M == 0 or N == 0).
static int gemm_validate(const char* who, const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                         const int32_t* qweight, const uint16_t* scales, const uint16_t* zeros, int group_size,
                         const void* y, int64_t ldy, bool* empty) {
  *empty = false;
  if (x_dtype != W4_DTYPE_BF16 && x_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "%s: x dtype must be bf16 or fp16 (got code %d)", who, x_dtype);
  if (M < 0 || N < 0 || K < 8 || K % 8 != 0)
    return fail(W4_ERR_INVALID, "%s: bad shape M=%lld N=%lld K=%lld", who, (long long)M, (long long)N,
                (long long)K);
  const int64_t G = group_size;
  if (G < 8 || !is_pow2(G) || K % G != 0)
    return fail(W4_ERR_INVALID, "%s: group_size %d must be a power of two >= 8 dividing K=%lld", who,
                group_size, (long long)K);
  if (ldy < N) return fail(W4_ERR_INVALID, "%s: ldy (%lld) < N (%lld)", who, (long long)ldy, (long long)N);
  if (M == 0 || N == 0) {
    *empty = true;
    return W4_OK;
  }
  if (!x || !qweight || !scales || !zeros || !y) return fail(W4_ERR_INVALID, "%s: null pointer", who);
  if (((uintptr_t)x % 2) != 0 || ((uintptr_t)y % 2) != 0)
    return fail(W4_ERR_INVALID, "%s: x and y must be 2-byte aligned", who);
  return W4_OK;
}

extern "C" int w4a16_gemm(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                          int64_t stride_xm, int64_t stride_xk, const int32_t* qweight,
                          const uint16_t* scales, const uint16_t* zeros, int group_size, void* y,
                          int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  bool empty;
  const int vrc = gemm_validate("w4a16_gemm", x, x_dtype, M, N, K, qweight, scales, zeros, group_size, y, ldy,
                                &empty);
  if (vrc != W4_OK || empty) return vrc;
  const int64_t G = group_size;
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned* counters;
  void* scratch;
  size_t scratch_bytes;
  split_workspace(workspace, workspace_bytes, &counters, &scratch, &scratch_bytes);
  if (M <= kDecodeM)
    return w4_gemv_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                          counters, scratch, scratch_bytes, st);
  if (sliced_lone(M, N) && stride_xk == 1 &&
      !w4_prefill_split_route(x, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy)) {
    // 17 <= M <= 64 (and up to 128 for N <= 4096): the rows as slices of
    // kDecodeM in one decode launch (the weights are read once per slice, the
    // repeats mostly from L2): no reduce launch.  Rows above 64 with K > 4096
    // that the prefill kernel's K-split launch takes go there instead.
    const w4a16_problem q{x, qweight, scales, zeros, y, N, K, (int32_t)G, 0};
    const int rc = w4_decode_launch(&q, &stride_xm, &ldy, 1, x_dtype, kDecodeM, counters, scratch, scratch_bytes,
                                    st, &M);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
  }
  if (M <= kSmallM) {
    const int rc = w4_prefill_fast_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros,
                                          (int)G, y, ldy, scratch, scratch_bytes, counters, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
    return w4_skinny_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y,
                            ldy, scratch, scratch_bytes, st);
  }
  return w4_prefill_launch(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, (int)G, y, ldy,
                           scratch, scratch_bytes, counters, st);
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
  if (M > kDecodeM) {
    // the decode launch's K split (16-row slices), or room for the separate
    // launches that may replace a shared-activation launch
    size_t most = 0;
    for (int i = 0; i < count; ++i) {
      const size_t b = w4a16_workspace_bytes(M, problems[i].N, problems[i].K, problems[i].group_size);
      most = b > most ? b : most;
    }
    if (sliced_grouped(problems, count, M)) {
      int64_t sxm[W4_MAX_GROUPED], mr[W4_MAX_GROUPED];
      for (int i = 0; i < count; ++i) sxm[i] = problems[i].K, mr[i] = M;
      const size_t d = w4_decode_workspace_bytes(problems, sxm, count, kDecodeM, mr);
      most = d > most ? d : most;
      if (M <= kSmallM) {
        const size_t r = w4_rows_workspace_bytes(problems, sxm, count, M);
        most = r > most ? r : most;
      }
    }
    return most;
  }
  // the decode kernel's K split (counter area only), or the grouped gemv
  // kernel's partials (groups below 32): room for either
  int64_t sxm[W4_MAX_GROUPED];
  for (int i = 0; i < count; ++i) sxm[i] = problems[i].K;
  const int64_t grp = w4_gemv_grouped_scratch_bytes(problems, count, M);
  const size_t dec = w4_decode_workspace_bytes(problems, sxm, count, M);
  const size_t g = grp > 0 ? W4_WORKSPACE_COUNTER_BYTES + (size_t)grp : 0;
  return g > dec ? g : dec;
}

extern "C" int w4a16_gemm_grouped(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (x_dtype != W4_DTYPE_BF16 && x_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4a16_gemm_grouped: x dtype must be bf16 or fp16");
  const int rc = check_grouped(problems, count, M);
  if (rc != W4_OK) return rc;
  if (M > kDecodeM) {
    // up to 64 rows, one decode launch with every problem in 16-row slices
    // (49..64 rows: the several-row kernel where every problem fits it; up to
    // 128 rows when every N <= 4096);
    // else one launch when the products share their activation matrix, else
    // one w4a16_gemm per problem, in order, on the stream (x rows of K
    // elements)
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (sliced_grouped(problems, count, M)) {
      int64_t sxm[W4_MAX_GROUPED], mr[W4_MAX_GROUPED];
      for (int i = 0; i < count; ++i) sxm[i] = problems[i].K, mr[i] = M;
      unsigned* counters;
      void* scratch;
      size_t scratch_bytes;
      split_workspace(workspace, workspace_bytes, &counters, &scratch, &scratch_bytes);
      if (M <= kSmallM) {
        // 49..64 rows: every weight dequantized once for all rows
        const int rrc = w4_rows_launch(problems, sxm, nullptr, count, x_dtype, M, counters, scratch, scratch_bytes, st);
        if (rrc != W4_ERR_UNSUPPORTED) return rrc;
      }
      const int drc = w4_decode_launch(problems, sxm, nullptr, count, x_dtype, kDecodeM, counters, scratch,
                                       scratch_bytes, st, mr);
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

// ------------------------------------------------------------------------
// w4a16_gemm_noalloc: w4a16_gemm with the library's own scratch memory.
//
// The workspace lives in this file-scope device array: one copy per GPU,
// allocated by the runtime when the library's code object is loaded there and
// held until the process ends.  Host code never passes `scratch` itself (on
// the host the name is only a stand-in for the device symbol): its device
// address is looked up once per device with hipGetSymbolAddress and cached.
static __device__ __align__(256) unsigned char scratch[W4_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxNoAllocDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxNoAllocDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call made with that device current).
int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(W4_ERR_LAUNCH, "w4a16_gemm_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxNoAllocDevices)
    return fail(W4_ERR_UNSUPPORTED, "w4a16_gemm_noalloc: device index %d beyond %d", dev, kMaxNoAllocDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(W4_ERR_LAUNCH, "w4a16_gemm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return W4_OK;
}

// Zeroes n32 words (n32 % 4 == 0) with 16-byte vector stores.
__global__ void clear_words_kernel(uint32_t* __restrict__ p, int n32) {
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i < n32) *reinterpret_cast<w4::u32x4*>(p + i) = w4::u32x4{0u, 0u, 0u, 0u};
}

}  // namespace

extern "C" int w4a16_gemm_noalloc(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                                  int64_t stride_xm, int64_t stride_xk, const int32_t* qweight,
                                  const uint16_t* scales, const uint16_t* zeros, int group_size, void* y,
                                  int64_t ldy, void* stream) {
  clear_error();
  // every check of w4a16_gemm, before the scratch size is asked for and before
  // anything is enqueued: a rejected call leaves nothing on the stream
  bool empty;
  const int vrc = gemm_validate("w4a16_gemm_noalloc", x, x_dtype, M, N, K, qweight, scales, zeros, group_size, y,
                                ldy, &empty);
  if (vrc != W4_OK || empty) return vrc;
  const size_t need = w4a16_workspace_bytes(M, N, K, group_size);
  if (need > (size_t)W4_NOALLOC_SCRATCH_BYTES)
    return fail(W4_ERR_WORKSPACE,
                "w4a16_gemm_noalloc: this problem needs %zu bytes of scratch, above the library's fixed %zu "
                "(M=%lld N=%lld K=%lld); use w4a16_gemm with a workspace",
                need, (size_t)W4_NOALLOC_SCRATCH_BYTES, (long long)M, (long long)N, (long long)K);
  void* ws = nullptr;
  int rc = noalloc_scratch(&ws);
  if (rc != W4_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (need > 0) {
    // the arrival counters must start at zero; the previous call on this GPU
    // left them zero, but a fill kernel (not a memset node, so that the call
    // can sit inside a captured graph) makes that hold whatever ran before
    const int n32 = W4_WORKSPACE_COUNTER_BYTES / 4;
    hipLaunchKernelGGL(clear_words_kernel, dim3((unsigned)((n32 / 4 + 255) / 256)), dim3(256), 0, st,
                       static_cast<uint32_t*>(ws), n32);
    rc = check_launch("w4a16_gemm_noalloc (counter clear)");
    if (rc != W4_OK) return rc;
  }
  return w4a16_gemm(x, x_dtype, M, N, K, stride_xm, stride_xk, qweight, scales, zeros, group_size, y, ldy, ws,
                    (size_t)W4_NOALLOC_SCRATCH_BYTES, stream);
}
