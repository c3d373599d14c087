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
// The stream of the last call on each device's array and an event recorded behind that call's
// launches: a call on another stream while that work runs would share the array with it.  g_held:
// a call is between its claim and its release (its launches are being issued), so any other call,
// on any stream, would interleave its launches with them.
static hipStream_t g_owner_stream[kScratchDevices];
static hipEvent_t g_owner_done[kScratchDevices];
static bool g_owner_used[kScratchDevices];
static bool g_held[kScratchDevices];
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
    hipEvent_t done = nullptr;
    e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    g_owner_done[device] = done;
    g_scratch_addr[device] = ptr;
    return hipSuccess;
}

ScratchClaim static_scratch_claim(int device, hipStream_t stream, bool capturing) {
    if (device < 0 || device >= kScratchDevices) return ScratchClaim::kError;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[device]) return ScratchClaim::kError;
    if (g_held[device]) return ScratchClaim::kBusy;
    if (!capturing && g_owner_used[device] && g_owner_stream[device] != stream) {
        const hipError_t e = hipEventQuery(g_owner_done[device]);
        if (e == hipErrorNotReady) return ScratchClaim::kBusy;
        if (e != hipSuccess) return ScratchClaim::kError;
    }
    g_held[device] = true;
    return ScratchClaim::kOk;
}

hipError_t static_scratch_release(int device, hipStream_t stream, bool capturing) {
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_held[device] = false;
    if (capturing) return hipSuccess; // a captured call's order is the graph's
    const hipError_t e = hipEventRecord(g_owner_done[device], stream);
    if (e != hipSuccess) return e;
    g_owner_stream[device] = stream;
    g_owner_used[device] = true;
    return hipSuccess;
}

void *static_scratch(int device) {
    if (device < 0 || device >= kScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_addr[device];
}

} // namespace xnp
