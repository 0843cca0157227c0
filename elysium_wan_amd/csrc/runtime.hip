// runtime.hip -- library identity, error reporting, device properties and
// the pinned host ring that stages tensor tables for the kernels.
#include <string.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <vector>

#include "ely_host.hpp"

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

static std::atomic<int32_t> g_max_blocks{0};

int64_t mt_blocks(int per_cu) {
    int64_t b = (int64_t)device_info().cus * per_cu;
    const int32_t cap = g_max_blocks.load();
    if (cap > 0 && b > cap) b = cap;
    return b;
}

// A ring of pinned host slots per device.  A slot is refilled only after the
// launch that last read it has completed (its event), so a caller may issue
// many uploads back to back without waiting.
//
// The bytes reach the device through a small staging kernel on the caller's
// stream that reads the slot directly (coherent, mapped host memory), not a
// host-to-device copy: a copy engine's hand-off to the compute queue cost
// ~12 us per table, a large share of a small shard's step.
namespace {
struct Slot {
    void* host = nullptr;
    const void* dev = nullptr;  // the slot as the GPU addresses it
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};
struct Ring {
    static constexpr int kSlots = 8;
    Slot slots[kSlots];
    int next = 0;
};
std::mutex g_ring_mu;
std::map<int, Ring> g_rings;
}  // namespace

__global__ __launch_bounds__(256) void stage_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

void upload(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ring_mu);
    Ring& ring = g_rings[dev];
    Slot& s = ring.slots[ring.next];
    ring.next = (ring.next + 1) % Ring::kSlots;
    if (s.pending) {
        check_hip(hipEventSynchronize(s.done), "hipEventSynchronize(upload slot)");
        s.pending = false;
    }
    if (s.cap < bytes) {
        if (s.host) check_hip(hipHostFree(s.host), "hipHostFree");
        s.host = nullptr;
        s.dev = nullptr;
        s.cap = 0;
        size_t cap = align_up(bytes, 64 * 1024);
        check_hip(hipHostMalloc(&s.host, cap, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc(upload slot)");
        void* d = nullptr;
        check_hip(hipHostGetDevicePointer(&d, s.host, 0), "hipHostGetDevicePointer(upload slot)");
        s.dev = d;
        s.cap = cap;
    }
    if (!s.done) check_hip(hipEventCreateWithFlags(&s.done, hipEventDisableTiming), "hipEventCreate");
    memcpy(s.host, src, bytes);
    // 16-byte vectors: the slot holds cap >= bytes rounded up to 16, and every
    // caller's destination region is padded to 256 bytes
    const int64_t n16 = (int64_t)((bytes + 15) / 16);
    const unsigned blocks = (unsigned)std::min<int64_t>((n16 + 255) / 256, 64);
    hipLaunchKernelGGL(stage_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<uint4*>(dst),
                       static_cast<const uint4*>(s.dev), n16);
    check_hip(hipGetLastError(), "stage_kernel launch");
    check_hip(hipEventRecord(s.done, stream), "hipEventRecord(upload slot)");
    s.pending = true;
}

}  // namespace ely

extern "C" {

int32_t ely_abi_version(void) { return 1; }

const char* ely_last_error(void) { return ely::g_last_error.c_str(); }

int ely_set_max_blocks(int32_t max_blocks) {
    if (max_blocks < 0) {
        ely::set_last_error("ely_set_max_blocks: negative cap");
        return ELY_EINVAL;
    }
    ely::g_max_blocks.store(max_blocks);
    return ELY_OK;
}

}  // extern "C"
