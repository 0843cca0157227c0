// ely_host.hpp -- host-side plumbing shared by the C-ABI translation units:
// the thread-local error string, argument checks, per-device properties and
// the pinned upload ring used to hand tensor tables to the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

#include "../../include/ely.h"

namespace ely {

// An error that maps to an ely_status at the C boundary.
struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& msg) : std::runtime_error(msg), status(s) {}
};

void set_last_error(const std::string& msg);

[[noreturn]] inline void fail(int status, const std::string& msg) { throw Error(status, msg); }

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(ELY_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Check the launch that was just made on this thread.
inline void check_launch(const char* kernel) { check_hip(hipGetLastError(), kernel); }

struct DeviceInfo {
    int device = -1;
    int cus = 0;       // compute units (256 on MI355X)
};

// Properties of the current device (cached per device).
const DeviceInfo& device_info();

// True when `p` is pinned host memory the GPU reaches through its mapping
// (a kernel's accesses to it cross PCIe); false for device memory and for
// addresses the runtime does not know.
bool host_resident(const void* p);

// Blocks for a persistent multi-tensor launch: `per_cu` per compute unit,
// capped by ely_set_max_blocks.
int64_t mt_blocks(int per_cu);

// Copy `bytes` of host data to device memory `dst` on `stream` through a
// library-owned pinned ring buffer: returns once the bytes are staged; the
// copy is ordered on `stream` before any later work there.
void upload(void* dst, const void* src, size_t bytes, hipStream_t stream);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Run `body`, translating exceptions into a status and the thread's error
// message.  Nothing escapes across the C boundary.
template <class F>
int guarded(F&& body) {
    try {
        body();
        return ELY_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return ELY_EHIP;
    } catch (...) {
        set_last_error("unknown error");
        return ELY_EHIP;
    }
}

}  // namespace ely
