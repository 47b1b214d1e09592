// Accessors the library's own host modules (round.cpp) use on top of the public C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/mtpx.h"

namespace mtpx {
// Memory the device can read at p: device or managed memory, or host memory mapped for the device
// (pinned or registered).  Plain host memory is refused: a kernel reading it faults the GPU.  (A
// failed query leaves an error the next launch check would report, so it is cleared.)
inline bool device_readable(const void* p) {
  if (!p) return false;
  hipPointerAttribute_t at{};
  if (hipPointerGetAttributes(&at, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged ||
         (at.type == hipMemoryTypeHost && at.devicePointer != nullptr);
}

hipStream_t ctx_stream(mtpx_ctx ctx);
int ctx_device(mtpx_ctx ctx);
// Error text for the next mtpx_last_error() (returns code).
int set_error(int code, const char* msg);
// vocab and multi-stream width (hc * hidden) of a target; hc * hidden of a head.
void target_dims(mtpx_target t, int64_t* vocab, int* width);
int head_width(mtpx_head h);
// Device buffers a target / head frees with itself (the checkpoint loader's copies).
void target_own(mtpx_target t, void* p);
void head_own(mtpx_head h, void* p);
// The drafter's shortlist ids of a head configuration (ascending).
std::vector<int32_t> head_shortlist_ids(const mtpx_head_config* cfg);
}  // namespace mtpx
