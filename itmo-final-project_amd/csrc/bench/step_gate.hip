// Measurement helper for bench.py, not part of the W4A16 library: a gate
// that holds a stream until the host has queued the whole timed region.
//
// A timed run of decode steps is "event, K calls, event" on one stream.  If
// the GPU starts the first call while the host is still queueing the later
// ones, the region also contains the host's latency to issue the first call
// (and its wake-up after the preceding synchronisation), spread over K steps.
// The gate is one single-thread kernel queued before the first event: it polls
// a word of pinned host memory until the host opens the gate (after queueing
// the second event), so the events bracket only the GPU's back-to-back
// execution of the K calls.  The poll is bounded: after `max_ticks` of the
// 100 MHz real-time counter the kernel leaves on its own, and it reports in the
// same word whether it was opened (2) or timed out (3).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

__global__ void gate_kernel(unsigned* flag, unsigned long long max_ticks) {
  if (threadIdx.x != 0) return;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  unsigned state = 3u;
  for (;;) {
    if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 1u) {
      state = 2u;
      break;
    }
    if (__builtin_amdgcn_s_memrealtime() - t0 > max_ticks) break;
    __builtin_amdgcn_s_sleep(8);
  }
  __hip_atomic_store(flag, state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

// One word of pinned host memory for a gate (nullptr on failure).
extern "C" void* w4bench_gate_new() {
  void* p = nullptr;
  if (hipHostMalloc(&p, 64, hipHostMallocCoherent) != hipSuccess) return nullptr;
  __atomic_store_n(static_cast<unsigned*>(p), 0u, __ATOMIC_SEQ_CST);
  return p;
}

extern "C" void w4bench_gate_free(void* flag) {
  if (flag != nullptr) (void)hipHostFree(flag);
}

// Closes the gate and queues its kernel on `stream`: work queued after it
// waits until w4bench_gate_open, or until max_ms have passed.  Returns 0, or
// the HIP error code.
extern "C" int w4bench_gate_close(void* flag, void* stream, double max_ms) {
  if (flag == nullptr) return (int)hipErrorInvalidValue;
  __atomic_store_n(static_cast<unsigned*>(flag), 0u, __ATOMIC_SEQ_CST);
  const unsigned long long ticks = (unsigned long long)(max_ms * 1e5);  // 100 MHz counter
  hipLaunchKernelGGL(gate_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<unsigned*>(flag), ticks);
  return (int)hipGetLastError();
}

extern "C" void w4bench_gate_open(void* flag) {
  __atomic_store_n(static_cast<unsigned*>(flag), 1u, __ATOMIC_SEQ_CST);
}

// After the stream has been synchronised: 2 if the gate was opened by the
// host, 3 if it timed out (the region then includes the host's queueing).
extern "C" int w4bench_gate_state(void* flag) {
  return (int)__atomic_load_n(static_cast<unsigned*>(flag), __ATOMIC_SEQ_CST);
}

// Timing-only events for the same region: created with
// hipEventDisableSystemFence, so recording them does not add the system-scope
// cache write-back and invalidation of a default event to the region (HIP
// documents the flag for events that only measure time).  The caller
// synchronises the device before reading the elapsed time.
extern "C" void* w4bench_event_new() {
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return static_cast<void*>(e);
}

extern "C" int w4bench_event_record(void* ev, void* stream) {
  return (int)hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream));
}

// Milliseconds between two recorded events (negative on error).
extern "C" double w4bench_event_ms(void* e0, void* e1) {
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, static_cast<hipEvent_t>(e0), static_cast<hipEvent_t>(e1)) != hipSuccess) return -1.0;
  return (double)ms;
}

extern "C" void w4bench_event_free(void* ev) {
  if (ev != nullptr) (void)hipEventDestroy(static_cast<hipEvent_t>(ev));
}
