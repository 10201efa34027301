// Fixed device scratch of the allocation-free product entry point (jv_matmul_noalloc).
//
// The array lives in this library's own gfx950 code object; the product kernels (loaded from
// jevons_qmm.hsaco) reach it through the device address that hipGetSymbolAddress returns, passed
// to them as an ordinary pointer argument. Each GPU holds its own copy of the array at its own
// address, so the address is looked up once per device, with that device current, and kept.
// Host code never uses the array's name as a device address: on the host it names a stand-in.

#include <hip/hip_runtime.h>

#include <mutex>

#include "jevons_qmm.h"

namespace {

static __device__ __align__(256) unsigned char scratch[JV_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices];           // device address of `scratch` on each device (null: not set up)
hipError_t g_status[kMaxDevices];   // failure of the set-up on each device

}  // namespace

// Set-up on `device`, which must be current: looks up the array's device address and zeroes its
// first `zero_bytes` (state that must start at zero, such as tile counters). Runs once per
// device; later calls return the kept address. Not for use under graph capture (it synchronizes).
extern "C" hipError_t jv_internal_noalloc_setup(int device, size_t zero_bytes, void **out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) {
        *out = g_ptr[device];
        return hipSuccess;
    }
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e == hipSuccess && zero_bytes) e = hipMemset(ptr, 0, zero_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        g_status[device] = e;
        return e;
    }
    g_ptr[device] = ptr;
    *out = ptr;
    return hipSuccess;
}

// The kept address for `device`, or null when its set-up has not succeeded (with the set-up's
// error in *status).
extern "C" void *jv_internal_noalloc_ptr(int device, hipError_t *status) {
    if (device < 0 || device >= kMaxDevices) {
        *status = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    *status = g_ptr[device] ? hipSuccess : (g_status[device] != hipSuccess ? g_status[device] : hipErrorNotInitialized);
    return g_ptr[device];
}
