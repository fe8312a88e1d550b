// Host-only stand-in for the HIP runtime API, for compiling host code (model::PagedBatchModel)
// with g++ in CPU tests: memory calls use malloc/memset/memcpy on host memory, streams, events
// and graphs are inert handles, and capture is tracked only so that the code's calls are legal.
// Test infrastructure only; the product is built with hipcc against the real runtime.
#ifndef SQ8_TESTS_MOCK_HIP_RUNTIME_H_
#define SQ8_TESTS_MOCK_HIP_RUNTIME_H_
#include <cstddef>
#include <cstdlib>
#include <cstring>

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2 };
struct MockHipStream {
  int capturing;
};
typedef MockHipStream* hipStream_t;
typedef int* hipEvent_t;
typedef int* hipGraph_t;
typedef int* hipGraphExec_t;
typedef int* hipGraphNode_t;
enum hipMemcpyKind {
  hipMemcpyHostToHost = 0,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipMemcpyDeviceToDevice = 3
};
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
enum hipStreamCaptureMode { hipStreamCaptureModeThreadLocal = 1 };
enum { hipStreamNonBlocking = 1, hipEventDisableTiming = 2, hipHostMallocDefault = 0 };

// Every allocation is registered (mock_sq8.cpp) so that logged pointers read as (allocation,
// byte offset) and allocation sizes can be compared.
void mock_register(const void* p, size_t bytes, int owned);
inline const char* hipGetErrorString(hipError_t e) { return e ? "mock error" : "no error"; }
inline hipError_t hipMalloc(void** p, size_t n) {
  *p = std::calloc(n, 1);
  if (*p) mock_register(*p, n, 1);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
  *p = std::calloc(n, 1);
  if (*p) mock_register(*p, n, 0);  // pinned host staging: not a device buffer of the model
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipFree(void* p) {
  std::free(p);
  return hipSuccess;
}
inline hipError_t hipHostFree(void* p) { return hipFree(p); }
inline hipError_t hipMemset(void* p, int v, size_t n) {
  std::memset(p, v, n);
  return hipSuccess;
}
inline hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t s) {
  return s && s->capturing ? hipErrorInvalidValue : hipMemset(p, v, n);  // never in a graph
}
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
  std::memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
  std::memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
inline hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus* c) {
  *c = s && s->capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
  *s = new MockHipStream{0};
  return hipSuccess;
}
inline hipError_t hipStreamDestroy(hipStream_t s) {
  delete s;
  return hipSuccess;
}
inline hipError_t hipStreamSynchronize(hipStream_t s) {
  return s && s->capturing ? hipErrorInvalidValue : hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
  *e = new int(0);
  return hipSuccess;
}
inline hipError_t hipEventDestroy(hipEvent_t e) {
  delete e;
  return hipSuccess;
}
inline hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
  *e = 1;
  return hipSuccess;
}
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
  s->capturing = 1;
  return hipSuccess;
}
inline hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g) {
  s->capturing = 0;
  *g = new int(0);
  return hipSuccess;
}
inline hipError_t hipGraphInstantiate(hipGraphExec_t* x, hipGraph_t, hipGraphNode_t*, char*,
                                      size_t) {
  *x = new int(0);
  return hipSuccess;
}
inline hipError_t hipGraphDestroy(hipGraph_t g) {
  delete g;
  return hipSuccess;
}
inline hipError_t hipGraphExecDestroy(hipGraphExec_t x) {
  delete x;
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t);  // recorded (mock_sq8.cpp)

#endif  // SQ8_TESTS_MOCK_HIP_RUNTIME_H_
