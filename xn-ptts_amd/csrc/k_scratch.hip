// The layer step's scratch as a fixed device array of the library, for callers that cannot allocate
// device memory (code under hipGraph capture, serving loops, hosts that forbid hipMalloc):
// xnp_layer_step_static carves its norm output, q/k/v, attention output and FF hidden rows from it
// instead of from a caller's workspace.
//
// The array's name is a host-side stand-in, not a device address.  Its address on each device comes
// from hipGetSymbolAddress, taken once per device with that device current (at pool creation), and
// only that address is handed to kernels.
#include "kernels_common.h"

#include <mutex>

namespace xnp {

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kScratchDevices = 64;
static void *g_scratch_addr[kScratchDevices];
static std::mutex g_scratch_mu;

hipError_t static_scratch_init(int device) {
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_addr[device]) return hipSuccess;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice; // the caller makes the device current first
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!ptr) return hipErrorInvalidSymbol;
    g_scratch_addr[device] = ptr;
    return hipSuccess;
}

void *static_scratch(int device) {
    if (device < 0 || device >= kScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_addr[device];
}

} // namespace xnp
