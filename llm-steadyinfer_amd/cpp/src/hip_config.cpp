// HipConfig workspace management.
#include "base/hip_config.h"
#include "base/base.h"

namespace kernel {

void* HipConfig::workspace(size_t bytes) {
  if (bytes == 0) return ws_;
  if (bytes > ws_bytes_) {
    // Growing means hipFree/hipMalloc and a zero fill: none of that may be recorded into a graph
    // being captured on this stream, so refuse (nullptr) and leave the workspace as it is.
    if (stream) {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return nullptr;
    }
    if (ws_) {
      // The old workspace may still be read by queued kernels on this stream.
      if (stream) CHECK(hipStreamSynchronize(stream) == hipSuccess);
      CHECK(hipFree(ws_) == hipSuccess);
      ws_ = nullptr;
      ws_bytes_ = 0;
    }
    CHECK(hipMalloc(&ws_, bytes) == hipSuccess) << "workspace of " << bytes << " bytes";
    // The matmul backend needs a zeroed workspace on first use (its split-K tickets).
    CHECK(hipMemsetAsync(ws_, 0, bytes, stream) == hipSuccess);
    ws_bytes_ = bytes;
  }
  return ws_;
}

HipConfig::~HipConfig() {
  if (ws_) {
    if (stream) (void)hipStreamSynchronize(stream);
    (void)hipFree(ws_);
  }
  if (owns_stream && stream) (void)hipStreamDestroy(stream);
}

}  // namespace kernel
