// noalloc.hip -- the routed-expert matmul for callers that cannot allocate.
//
// q3x_hip_moe_routed takes a caller-owned workspace.  Some callers cannot
// obtain one: code under hipGraph capture, tight serving loops, harnesses
// that forbid hipMalloc.  q3x_hip_moe_routed_noalloc runs the same kernels
// on a workspace that lives in the library itself: `scratch`, a file-scope
// __device__ array of Q3X_HIP_NOALLOC_SCRATCH_BYTES.  Every device the
// library runs on holds its own copy of the array, at its own address, until
// the process ends.
//
// In host code `scratch` names a host-side stand-in, not a device address.
// The device address comes from hipGetSymbolAddress, taken once per device
// (with that device current) on the entry point's first call there, and only
// that address is ever passed to kernels.  Nothing here calls hipMalloc or
// hipFree or any allocating routine.
//
// The workspace needs no clearing: the grouping kernels write every count,
// base, tile and position before it is read, and the GEMMs read only rows
// of positions they were given.  Every call on a device shares that device's
// array, so calls that overlap on one device (on different streams, or from
// different threads without ordering) race; calls ordered on one stream do
// not.
#include <mutex>

#include "common.h"

namespace q3x {

constexpr size_t kNoAllocScratchBytes = Q3X_HIP_NOALLOC_SCRATCH_BYTES;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Device address of this device's `scratch` (nullptr on a HIP error).
static uint8_t* scratch_address() {
    static std::mutex mutex;
    static uint8_t* address[kNoAllocMaxDevices] = {};
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kNoAllocMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(mutex);
    if (!address[device]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        address[device] = static_cast<uint8_t*>(p);
    }
    return address[device];
}

}  // namespace q3x

extern "C" int q3x_hip_moe_routed_noalloc(const void* gate_up, const void* down, uint32_t type, int experts, int H,
                                          int I, const float* X, int tokens, const int* ids, const float* weights,
                                          int top_k, float* Y, int accumulate, hipStream_t stream) {
    // The workspace this request needs (0 for arguments the sizing rejects;
    // q3x_hip_moe_routed then rejects them too).
    const size_t need = q3x_hip_moe_workspace_bytes(tokens, experts, top_k, H, I);
    if (need > q3x::kNoAllocScratchBytes) return Q3X_HIP_ESCRATCH;
    uint8_t* ws = q3x::scratch_address();
    if (!ws) return Q3X_HIP_ERUNTIME;
    return q3x_hip_moe_routed(gate_up, down, type, experts, H, I, X, tokens, ids, weights, top_k, Y, accumulate, ws,
                              q3x::kNoAllocScratchBytes, stream);
}
