// elementwise.hip -- the two stand-alone elementwise ops of the sharded
// "pieces" update: the fp32 master -> bf16 working-copy cast
// (pieces.cast_piece, runtime/pieces.py:192-195) and the fp32 fold of a
// microbatch gradient (pieces.fold_add, runtime/pieces.py:206-214).  Both
// are one HBM pass, 16-byte vectors, grid-stride over a persistent grid.
#include <algorithm>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {

constexpr int kEwBlock = 256;

__global__ __launch_bounds__(kEwBlock) void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ out,
                                                             int64_t n, int vec) {
    const int64_t tid = (int64_t)blockIdx.x * kEwBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    int64_t done = 0;
    if (vec) {
        const int64_t nv = n / 8;
        for (int64_t i = tid; i < nv; i += stride) {
            const float4* xp = reinterpret_cast<const float4*>(x + i * 8);
            const float4 a = xp[0], b = xp[1];
            uint4 o;
            o.x = f32_to_bf16(a.x) | (f32_to_bf16(a.y) << 16);
            o.y = f32_to_bf16(a.z) | (f32_to_bf16(a.w) << 16);
            o.z = f32_to_bf16(b.x) | (f32_to_bf16(b.y) << 16);
            o.w = f32_to_bf16(b.z) | (f32_to_bf16(b.w) << 16);
            *reinterpret_cast<uint4*>(out + i * 8) = o;
        }
        done = nv * 8;
    }
    for (int64_t i = done + tid; i < n; i += stride) out[i] = (uint16_t)f32_to_bf16(x[i]);
}

template <bool BF16G>
__global__ __launch_bounds__(kEwBlock) void fold_add_kernel(float* __restrict__ acc, const void* __restrict__ g,
                                                            int64_t n, int vec) {
    const int64_t tid = (int64_t)blockIdx.x * kEwBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    int64_t done = 0;
    if (vec) {
        const int64_t nv = n / 8;
        for (int64_t i = tid; i < nv; i += stride) {
            float4* ap = reinterpret_cast<float4*>(acc + i * 8);
            float4 a = ap[0], b = ap[1];
            float gv[8];
            if (BF16G) {
                const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(g) + i * 8);
                gv[0] = bf16_to_f32(w.x & 0xFFFFu); gv[1] = bf16_to_f32(w.x >> 16);
                gv[2] = bf16_to_f32(w.y & 0xFFFFu); gv[3] = bf16_to_f32(w.y >> 16);
                gv[4] = bf16_to_f32(w.z & 0xFFFFu); gv[5] = bf16_to_f32(w.z >> 16);
                gv[6] = bf16_to_f32(w.w & 0xFFFFu); gv[7] = bf16_to_f32(w.w >> 16);
            } else {
                const float4* gp = reinterpret_cast<const float4*>(static_cast<const float*>(g) + i * 8);
                const float4 c = gp[0], d = gp[1];
                gv[0] = c.x; gv[1] = c.y; gv[2] = c.z; gv[3] = c.w;
                gv[4] = d.x; gv[5] = d.y; gv[6] = d.z; gv[7] = d.w;
            }
            a.x = a.x + gv[0]; a.y = a.y + gv[1]; a.z = a.z + gv[2]; a.w = a.w + gv[3];
            b.x = b.x + gv[4]; b.y = b.y + gv[5]; b.z = b.z + gv[6]; b.w = b.w + gv[7];
            ap[0] = a;
            ap[1] = b;
        }
        done = nv * 8;
    }
    for (int64_t i = done + tid; i < n; i += stride) {
        const float gv = BF16G ? bf16_to_f32(static_cast<const uint16_t*>(g)[i]) : static_cast<const float*>(g)[i];
        acc[i] = acc[i] + gv;
    }
}

// g <- g * coef (coef read from device memory), one fp32 multiply rounded to
// g's dtype: torch's _foreach_mul_(grads, clip_coef) (clip_grad.py:170-177).
template <bool BF16G>
__global__ __launch_bounds__(kEwBlock) void scale_kernel(void* __restrict__ g, int64_t n,
                                                         const float* __restrict__ coef_ptr) {
    const float coef = *coef_ptr;
    const int64_t tid = (int64_t)blockIdx.x * kEwBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    for (int64_t i = tid; i < n; i += stride) {
        if (BF16G) {
            uint16_t* p = static_cast<uint16_t*>(g);
            p[i] = (uint16_t)f32_to_bf16(bf16_to_f32(p[i]) * coef);
        } else {
            float* p = static_cast<float*>(g);
            p[i] = p[i] * coef;
        }
    }
}

static unsigned ew_blocks(int64_t n) {
    const DeviceInfo& dev = device_info();
    const int64_t want = (n + (int64_t)kEwBlock * 8 - 1) / ((int64_t)kEwBlock * 8);
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)dev.cus * 8));
}

}  // namespace ely

using namespace ely;

extern "C" {

int ely_cast_bf16(const float* x, uint16_t* out, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_cast_bf16: negative n");
        if (n == 0) return;
        if (!x || !out) fail(ELY_EINVAL, "ely_cast_bf16: null pointer");
        const int vec = aligned16(x) && aligned16(out);
        hipLaunchKernelGGL(cast_bf16_kernel, dim3(ew_blocks(n)), dim3(kEwBlock), 0, static_cast<hipStream_t>(stream),
                           x, out, n, vec);
        check_launch("cast_bf16_kernel");
    });
}

int ely_fold_add(float* acc, const void* g, int32_t g_dtype, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_fold_add: negative n");
        if (g_dtype != ELY_F32 && g_dtype != ELY_BF16) fail(ELY_EINVAL, "ely_fold_add: g_dtype");
        if (n == 0) return;
        if (!acc || !g) fail(ELY_EINVAL, "ely_fold_add: null pointer");
        const int vec = aligned16(acc) && aligned16(g);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (g_dtype == ELY_BF16)
            hipLaunchKernelGGL(fold_add_kernel<true>, dim3(ew_blocks(n)), dim3(kEwBlock), 0, s, acc, g, n, vec);
        else
            hipLaunchKernelGGL(fold_add_kernel<false>, dim3(ew_blocks(n)), dim3(kEwBlock), 0, s, acc, g, n, vec);
        check_launch("fold_add_kernel");
    });
}

int ely_scale_inplace(const ely_tensor* ts, int32_t n, const float* coef_dev, void* stream) {
    return guarded([&] {
        if (n < 0 || (n > 0 && !ts)) fail(ELY_EINVAL, "ely_scale_inplace: bad tensor list");
        if (!coef_dev) fail(ELY_EINVAL, "ely_scale_inplace: null coefficient");
        hipStream_t s = static_cast<hipStream_t>(stream);
        for (int32_t i = 0; i < n; ++i) {
            const ely_tensor& t = ts[i];
            if (t.numel < 0 || (t.numel > 0 && !t.ptr)) fail(ELY_EINVAL, "ely_scale_inplace: bad tensor");
            if (t.numel == 0) continue;
            if (t.dtype == ELY_BF16)
                hipLaunchKernelGGL(scale_kernel<true>, dim3(ew_blocks(t.numel)), dim3(kEwBlock), 0, s, t.ptr, t.numel,
                                   coef_dev);
            else if (t.dtype == ELY_F32)
                hipLaunchKernelGGL(scale_kernel<false>, dim3(ew_blocks(t.numel)), dim3(kEwBlock), 0, s, t.ptr, t.numel,
                                   coef_dev);
            else
                fail(ELY_EINVAL, "ely_scale_inplace: dtype");
            check_launch("scale_kernel");
        }
    });
}

}  // extern "C"
