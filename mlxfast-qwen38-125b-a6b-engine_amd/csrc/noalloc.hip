// Device scratch of the allocation-free MoE entry point (mtpx_moe_forward_noalloc): a file-scope
// device array, one copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device address): set-up calls
// moe_scratch_address() once per device, with that device current, and every use goes through
// the address it returns.
#include <mutex>

#include "mtpx_kernels.h"

namespace {

constexpr size_t MOE_SCRATCH_BYTES = (size_t)2 << 20;  // 2 MiB: the MoE workspace at M <= 8 of the model's dims

static __device__ __align__(256) uint8_t scratch[MOE_SCRATCH_BYTES];

std::mutex g_mu;
void* g_addr[64] = {nullptr};
const void* g_owner[64] = {nullptr};  // the context that uses this device's array, until it is freed

}  // namespace

namespace mtpx {

size_t moe_scratch_bytes() { return MOE_SCRATCH_BYTES; }

// This device's copy of the scratch array (device must be current).  Looked up once per device.
hipError_t moe_scratch_address(int device, void** ptr) {
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_addr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_addr[device] = p;
  }
  *ptr = g_addr[device];
  return hipSuccess;
}

// One context per device may use the array (the first that asks); another gets false, so two
// contexts on one GPU never share it unknowingly.  The claim ends with moe_scratch_release.
bool moe_scratch_claim(int device, const void* owner) {
  if (device < 0 || device >= 64) return false;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_owner[device]) g_owner[device] = owner;
  return g_owner[device] == owner;
}

void moe_scratch_release(int device, const void* owner) {
  if (device < 0 || device >= 64) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_owner[device] == owner) g_owner[device] = nullptr;
}

}  // namespace mtpx
