// probe.hip -- measurement kernels with the fused AdamW's streams and no
// arithmetic, so that the update can be held against the rate the memory
// system gives its traffic mix in the same physical placement:
//   read  : read p, g, m, v            (14 B per element; bf16 g)
//   write : write p, m, v, copy        (14 B per element; bf16 copy)
//   rw    : read p, g, m, v, write p, m, v, copy (28 B per element; the
//           fp32 streams rotate their values, copy takes g's)
// Each thread moves 4 elements per step (16-byte fp32, 8-byte bf16
// accesses, nontemporal, as the update's), grid-stride over n elements.
// They back bench.py's placement sweeps; nothing on the path calls them.
#include <stdint.h>

#include "ely_device.hpp"
#include "ely_host.hpp"

namespace ely {
namespace {

typedef float pf4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu2 __attribute__((ext_vector_type(2)));
#define ELY_PG __attribute__((address_space(1)))

template <class T>
__device__ __forceinline__ T pld(const T* p) {
    return __builtin_nontemporal_load((const ELY_PG T*)(const void*)p);
}
template <class T>
__device__ __forceinline__ void pst(T* p, T v) {
    __builtin_nontemporal_store(v, (ELY_PG T*)(void*)p);
}

constexpr int kProbeBlock = 256;

__global__ __launch_bounds__(kProbeBlock) void probe_read_kernel(const float* p, const uint16_t* g, const float* m,
                                                                 const float* v, int64_t n, float* sink) {
    float acc = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kProbeBlock * 4;
    for (int64_t i = ((int64_t)blockIdx.x * kProbeBlock + threadIdx.x) * 4; i + 4 <= n; i += stride) {
        const pf4 a = pld((const pf4*)(p + i)), b = pld((const pf4*)(m + i)), c = pld((const pf4*)(v + i));
        const pu2 d = pld((const pu2*)(g + i));
        acc += a.x + b.y + c.z + (float)(d.x & 1u);
    }
    if (acc == -1.0f) sink[0] = acc;  // a store the compiler cannot prove dead keeps every load
}

__global__ __launch_bounds__(kProbeBlock) void probe_write_kernel(float* p, float* m, float* v, uint16_t* c, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kProbeBlock * 4;
    for (int64_t i = ((int64_t)blockIdx.x * kProbeBlock + threadIdx.x) * 4; i + 4 <= n; i += stride) {
        const float f = (float)(i & 1023);
        pst((pf4*)(p + i), pf4{f, f, f, f});
        pst((pf4*)(m + i), pf4{f, f, f, f});
        pst((pf4*)(v + i), pf4{f, f, f, f});
        pst((pu2*)(c + i), pu2{0u, 0u});
    }
}

__global__ __launch_bounds__(kProbeBlock) void probe_rw_kernel(float* p, const uint16_t* g, float* m, float* v,
                                                               uint16_t* c, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kProbeBlock * 4;
    for (int64_t i = ((int64_t)blockIdx.x * kProbeBlock + threadIdx.x) * 4; i + 4 <= n; i += stride) {
        const pf4 a = pld((const pf4*)(p + i)), b = pld((const pf4*)(m + i)), e = pld((const pf4*)(v + i));
        const pu2 d = pld((const pu2*)(g + i));
        // each stream takes another's values: a store of what was just
        // loaded from the same address would be folded away by the compiler
        pst((pf4*)(p + i), b);
        pst((pf4*)(m + i), e);
        pst((pf4*)(v + i), a);
        pst((pu2*)(c + i), d);
    }
}

}  // namespace
}  // namespace ely

using namespace ely;

extern "C" int ely_probe_streams(int32_t which, void* p, void* g, void* m, void* v, void* c, int64_t n,
                                 int32_t blocks, void* sink, void* stream) {
    return guarded([&] {
        if (which < 0 || which > 2) fail(ELY_EINVAL, "ely_probe_streams: which is 0 (read), 1 (write) or 2 (read+write)");
        if (n < 0 || n % 4 != 0) fail(ELY_EINVAL, "ely_probe_streams: n is a non-negative multiple of 4");
        if (blocks <= 0) fail(ELY_EINVAL, "ely_probe_streams: blocks must be positive");
        if (n == 0) return;
        if (!p || !m || !v || (which != 1 && !g) || (which != 0 && !c) || (which == 0 && !sink))
            fail(ELY_EINVAL, "ely_probe_streams: null pointer");
        if (!aligned16(p) || !aligned16(m) || !aligned16(v) || (g && (reinterpret_cast<uintptr_t>(g) & 7u)) ||
            (c && (reinterpret_cast<uintptr_t>(c) & 7u)))
            fail(ELY_EINVAL, "ely_probe_streams: fp32 streams 16-byte aligned, bf16 streams 8-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const dim3 grid((unsigned)blocks), block(kProbeBlock);
        if (which == 0)
            hipLaunchKernelGGL(probe_read_kernel, grid, block, 0, s, static_cast<const float*>(p),
                               static_cast<const uint16_t*>(g), static_cast<const float*>(m),
                               static_cast<const float*>(v), n, static_cast<float*>(sink));
        else if (which == 1)
            hipLaunchKernelGGL(probe_write_kernel, grid, block, 0, s, static_cast<float*>(p), static_cast<float*>(m),
                               static_cast<float*>(v), static_cast<uint16_t*>(c), n);
        else
            hipLaunchKernelGGL(probe_rw_kernel, grid, block, 0, s, static_cast<float*>(p),
                               static_cast<const uint16_t*>(g), static_cast<float*>(m), static_cast<float*>(v),
                               static_cast<uint16_t*>(c), n);
        check_launch("probe kernel");
    });
}
