// HIP API stand-in for the CPU sanitizer build of the host-only runtime
// (orcaml_amd/csrc/runtime_host.cpp).  "Device" memory is host memory, copies
// are immediate, and an event reports "not ready" for a configurable number of
// queries so that the staging ring's back-pressure path runs.  Test
// infrastructure only: nothing here is linked into liborca_hip.so.
#pragma once

#include <cstddef>
#include <cstdlib>
#include <cstring>

typedef int hipError_t;
enum : int { hipSuccess = 0, hipErrorOutOfMemory = 2, hipErrorInvalidValue = 1, hipErrorNotReady = 600 };
struct ihipStream_t;
typedef ihipStream_t* hipStream_t;
struct StubEvent {
  int queries_left;  // hipEventQuery answers hipErrorNotReady this many more times
  bool recorded;
};
typedef StubEvent* hipEvent_t;
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2, hipMemcpyDeviceToDevice = 3 };
#define hipHostMallocDefault 0
#define hipEventDisableTiming 2
#define hipEventDisableSystemFence 0x20000000

namespace hip_stub {
inline int& event_delay() { static int v = 0; return v; }        // queries an event stays pending
inline long& device_mallocs() { static long v = 0; return v; }
inline long& stream_waits() { static long v = 0; return v; }
inline long& device_frees() { static long v = 0; return v; }
inline long& stream_syncs() { static long v = 0; return v; }
inline long& event_syncs() { static long v = 0; return v; }
inline size_t& fail_mallocs_above() { static size_t v = 0; return v; }  // 0: never fail
inline int& fail_next_mallocs() { static int v = 0; return v; }
}  // namespace hip_stub

inline const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "stub error"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipMalloc(void** p, size_t n) {
  if (hip_stub::fail_next_mallocs() > 0) {
    --hip_stub::fail_next_mallocs();
    *p = nullptr;
    return hipErrorOutOfMemory;
  }
  *p = std::aligned_alloc(256, (n + 255) / 256 * 256);
  if (!*p) return hipErrorOutOfMemory;
  ++hip_stub::device_mallocs();
  return hipSuccess;
}
inline hipError_t hipFree(void* p) {
  if (p) ++hip_stub::device_frees();
  std::free(p);
  return hipSuccess;
}
inline hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
  *p = std::aligned_alloc(4096, (n + 4095) / 4096 * 4096);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipHostFree(void* p) {
  std::free(p);
  return hipSuccess;
}
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
  std::memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipStreamSynchronize(hipStream_t) {
  ++hip_stub::stream_syncs();
  return hipSuccess;
}
inline hipError_t hipEventCreate(hipEvent_t* e) {
  *e = new StubEvent{0, false};
  return hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { return hipEventCreate(e); }
inline hipError_t hipEventDestroy(hipEvent_t e) {
  delete e;
  return hipSuccess;
}
inline hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
  if (!e) return hipErrorInvalidValue;
  e->recorded = true;
  e->queries_left = hip_stub::event_delay();
  return hipSuccess;
}
inline hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t e, unsigned) {
  ++hip_stub::stream_waits();
  return e && e->recorded ? hipSuccess : hipErrorInvalidValue;
}
inline hipError_t hipEventQuery(hipEvent_t e) {
  if (e->queries_left > 0) {
    --e->queries_left;
    return hipErrorNotReady;
  }
  return hipSuccess;
}
inline hipError_t hipEventSynchronize(hipEvent_t e) {
  ++hip_stub::event_syncs();
  e->queries_left = 0;
  return hipSuccess;
}
inline hipError_t hipEventElapsedTime(float* ms, hipEvent_t, hipEvent_t) {
  *ms = 1.0f;
  return hipSuccess;
}
