// runtime.hip -- library identity, error reporting, device properties and
// the pinned host ring that stages tensor tables for the kernels.
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <vector>

#include "ely_host.hpp"

#ifndef ELY_UPLOAD_SLOTS
#define ELY_UPLOAD_SLOTS 8  // pinned upload ring slots per device (two per table AdamW launch)
#endif

namespace ely {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }

static std::mutex g_dev_mu;
static std::map<int, DeviceInfo> g_devices;

const DeviceInfo& device_info() {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_dev_mu);
    auto it = g_devices.find(dev);
    if (it != g_devices.end()) return it->second;
    DeviceInfo info;
    info.device = dev;
    check_hip(hipDeviceGetAttribute(&info.cus, hipDeviceAttributeMultiprocessorCount, dev),
              "hipDeviceGetAttribute(multiProcessorCount)");
    if (info.cus <= 0) info.cus = 1;
    return g_devices.emplace(dev, info).first->second;
}

bool host_resident(const void* p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();  // an unknown address is not an error of the caller's next call
        return false;
    }
    return a.type == hipMemoryTypeHost;
}

static std::atomic<int32_t> g_max_blocks{0};

int64_t mt_blocks(int per_cu) {
    int64_t b = (int64_t)device_info().cus * per_cu;
    const int32_t cap = g_max_blocks.load();
    if (cap > 0 && b > cap) b = cap;
    return b;
}

// A ring of pinned host slots per device.  A slot is refilled only after the
// copy that last read it has completed (its event), so a caller may issue
// many uploads back to back without waiting; the host blocks only when the
// ring wraps onto an upload the GPU has not reached yet, which keeps a
// staged host-moment step at most four chunk launches ahead of its copies.
// Deeper rings (32 and 128 slots) measured slower on that step (C1 staged
// 0.43-0.47 s against 0.40 s; 200M parameters with half the moments
// resident 0.029-0.031 s against 0.019 s): the extra queued table copies
// interleave with the bulk moment copies.
namespace {
struct Slot {
    std::mutex mu;  // held while the slot is waited on and refilled
    void* host = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};
struct Ring {
    static constexpr int kSlots = ELY_UPLOAD_SLOTS;
    Slot slots[kSlots];
    int next = 0;
};
std::mutex g_ring_mu;  // guards the map of rings and each ring's next slot, never held while waiting
std::map<int, Ring> g_rings;
}  // namespace

void upload(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    Slot* slot;
    {
        std::lock_guard<std::mutex> lk(g_ring_mu);
        Ring& ring = g_rings[dev];
        slot = &ring.slots[ring.next];
        ring.next = (ring.next + 1) % Ring::kSlots;
    }
    // Another thread whose ring wrapped onto the same slot waits here, not
    // on the ring: uploads to other slots go on meanwhile.
    Slot& s = *slot;
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.pending) {
        check_hip(hipEventSynchronize(s.done), "hipEventSynchronize(upload slot)");
        s.pending = false;
    }
    if (s.cap < bytes) {
        if (s.host) check_hip(hipHostFree(s.host), "hipHostFree");
        s.host = nullptr;
        s.cap = 0;
        size_t cap = align_up(bytes, 64 * 1024);
        check_hip(hipHostMalloc(&s.host, cap, hipHostMallocDefault), "hipHostMalloc(upload slot)");
        s.cap = cap;
    }
    if (!s.done) check_hip(hipEventCreateWithFlags(&s.done, hipEventDisableTiming), "hipEventCreate");
    memcpy(s.host, src, bytes);
    check_hip(hipMemcpyAsync(dst, s.host, bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(table)");
    check_hip(hipEventRecord(s.done, stream), "hipEventRecord(upload slot)");
    s.pending = true;
}

}  // namespace ely

extern "C" {

int32_t ely_abi_version(void) { return 1; }

const char* ely_last_error(void) { return ely::g_last_error.c_str(); }

int ely_host_device_pointer(const void* host, void** device) {
    return ely::guarded([&] {
        if (!host || !device) ely::fail(ELY_EINVAL, "ely_host_device_pointer: null pointer");
        void* d = nullptr;
        if (hipHostGetDevicePointer(&d, const_cast<void*>(host), 0) != hipSuccess || !d) {
            (void)hipGetLastError();  // the query's error is not sticky state for later calls
            ely::fail(ELY_EINVAL, "ely_host_device_pointer: not pinned, mapped host memory");
        }
        *device = d;
    });
}

int ely_set_max_blocks(int32_t max_blocks) {
    if (max_blocks < 0) {
        ely::set_last_error("ely_set_max_blocks: negative cap");
        return ELY_EINVAL;
    }
    ely::g_max_blocks.store(max_blocks);
    return ELY_OK;
}

}  // extern "C"
