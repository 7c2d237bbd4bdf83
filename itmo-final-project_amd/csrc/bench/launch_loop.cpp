// Measurement helper for bench.py, not part of the W4A16 library: issues
// `steps` calls of a grouped-product entry point (w4a16_gemm_grouped of
// libint4_hip.so, passed in as a function pointer) back to back from C, so
// that a timed run of decode steps is bound by the GPU and not by the Python
// interpreter's per-call overhead, with no graph in between.
#include <stddef.h>
#include <stdint.h>

typedef int (*w4bench_grouped_fn)(const void* problems, int count, int x_dtype, int64_t M, void* workspace,
                                  size_t workspace_bytes, void* stream);

// Step i uses the problem list at problems + ((first + i) % nsets) *
// set_stride_bytes (a run that continues the rotation of an earlier one
// passes the number of steps already issued as `first`).  Returns 0, or the
// first nonzero status of the entry point.
extern "C" int w4bench_grouped_steps(void* fn, const void* problems, size_t set_stride_bytes, int count,
                                     int nsets, int first, int steps, int x_dtype, int64_t M, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (fn == nullptr || problems == nullptr || nsets < 1 || first < 0 || steps < 0) return -1;
  const w4bench_grouped_fn f = reinterpret_cast<w4bench_grouped_fn>(fn);
  for (int i = 0; i < steps; ++i) {
    const void* p = static_cast<const char*>(problems) + (size_t)((first + i) % nsets) * set_stride_bytes;
    const int rc = f(p, count, x_dtype, M, workspace, workspace_bytes, stream);
    if (rc != 0) return rc;
  }
  return 0;
}
