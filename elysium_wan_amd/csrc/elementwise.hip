// elementwise.hip -- the stand-alone elementwise ops of the sharded "pieces"
// update: the fp32 master -> bf16 working-copy cast (pieces.cast_piece,
// runtime/pieces.py:192-195), the fp32 fold of a microbatch gradient
// (pieces.fold_add, runtime/pieces.py:206-214; into a bf16 sum for
// OrderedAccumulator, runtime/accumulate.py:101-102).  (The clip's in-place
// scaling of a tensor list is one multi-tensor launch in mta.hip.)  Each is
// one HBM pass over 4-element quads
// (16-byte fp32, 8-byte bf16 vectors, nontemporal) with a per-kernel launch
// shape: quads in flight per thread, threads per block, and a grid that is
// either persistent (a few blocks per CU, striding) or one-shot (a block per
// run of quads, exiting after it).
#include <algorithm>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

// Tunables, per kernel: quads of 4 elements a thread has in flight (_UNROLL),
// the grid's cap in blocks per CU (_BPC; a cap above what the largest
// tensor needs makes the grid one-shot) and threads per block (_BLOCK).
// Each pass below runs one quad per thread on 64-thread blocks, one-shot (a
// block per 256 elements).  Against 256-thread blocks in the same process
// and buffers: at 2^28 elements the fold (bf16 g) 6.78 TB/s against 6.18 at
// 3 blocks per CU, the cast 6.87 against 6.08 at 4 per CU, the widen 6.75
// against 6.44 one-shot; over C1's tensors one launch each, 5.69 against
// 5.50, 5.12 against 4.79 and 4.99 against 4.80.
#ifndef ELY_CAST_UNROLL
#define ELY_CAST_UNROLL 1
#endif
#ifndef ELY_CAST_BPC
#define ELY_CAST_BPC 262144
#endif
#ifndef ELY_CAST_BLOCK
#define ELY_CAST_BLOCK 64
#endif
#ifndef ELY_WIDEN_UNROLL
#define ELY_WIDEN_UNROLL 1
#endif
#ifndef ELY_WIDEN_BPC
#define ELY_WIDEN_BPC 262144
#endif
#ifndef ELY_WIDEN_BLOCK
#define ELY_WIDEN_BLOCK 64
#endif
#ifndef ELY_FOLD_UNROLL
#define ELY_FOLD_UNROLL 1
#endif
#ifndef ELY_FOLD_BPC
#define ELY_FOLD_BPC 262144
#endif
#ifndef ELY_FOLD_BLOCK
#define ELY_FOLD_BLOCK 64
#endif

namespace ely {

// A launch shape: quads in flight per thread, blocks per CU, threads per
// block.
struct EwShape {
    int unroll, bpc, block;
};
constexpr EwShape kCastShape{ELY_CAST_UNROLL, ELY_CAST_BPC, ELY_CAST_BLOCK};
constexpr EwShape kFoldShape{ELY_FOLD_UNROLL, ELY_FOLD_BPC, ELY_FOLD_BLOCK};
constexpr EwShape kWidenShape{ELY_WIDEN_UNROLL, ELY_WIDEN_BPC, ELY_WIDEN_BLOCK};

typedef float ef4 __attribute__((ext_vector_type(4)));
typedef uint32_t eu2 __attribute__((ext_vector_type(2)));
#define EW_G1 __attribute__((address_space(1)))

// Streamed (nontemporal) 16-byte fp32 quads and 8-byte bf16 quads.
__device__ __forceinline__ ef4 ld4(const float* p) { return __builtin_nontemporal_load((const EW_G1 ef4*)p); }
__device__ __forceinline__ void st4(float* p, ef4 v) { __builtin_nontemporal_store(v, (EW_G1 ef4*)p); }
__device__ __forceinline__ eu2 ldh4(const uint16_t* p) { return __builtin_nontemporal_load((const EW_G1 eu2*)p); }
__device__ __forceinline__ void sth4(uint16_t* p, eu2 v) { __builtin_nontemporal_store(v, (EW_G1 eu2*)p); }

__device__ __forceinline__ ef4 widen4(eu2 w) {
    return ef4{bf16_to_f32(w[0] & 0xFFFFu), bf16_to_f32(w[0] >> 16), bf16_to_f32(w[1] & 0xFFFFu), bf16_to_f32(w[1] >> 16)};
}
__device__ __forceinline__ eu2 narrow4(ef4 v) {
    return eu2{f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16), f32_to_bf16(v[2]) | (f32_to_bf16(v[3]) << 16)};
}

// The quad loop shared by the kernels below: thread t of T takes quads
// t, t + T, ..., U of them loaded before the first is computed, so each load
// or store instruction of a wave covers one contiguous run.  load(q) reads
// quad q into registers, store(q, regs) computes and writes it; returns the
// elements covered.
template <int U, int B, class Load, class Store>
__device__ __forceinline__ int64_t quad_loop(int64_t nq, Load load, Store store) {
    const int64_t T = (int64_t)gridDim.x * B;
    const int64_t t = (int64_t)blockIdx.x * B + threadIdx.x;
    for (int64_t base = t; base < nq; base += T * U) {
        decltype(load(0)) r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t q = base + u * T;
            r[u] = load(q < nq ? q : nq - 1);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t q = base + u * T;
            if (q < nq) store(q, r[u]);
        }
    }
    return nq * 4;
}

// pieces.cast_piece: fp32 -> bf16 (RNE, NaN -> 0x7FC0).
__global__ __launch_bounds__(kCastShape.block) void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ out,
                                                             int64_t n, int vec) {
    int64_t done = 0;
    if (vec)
        done = quad_loop<kCastShape.unroll, kCastShape.block>(
            n / 4, [&](int64_t q) { return ld4(x + 4 * q); }, [&](int64_t q, ef4 v) { sth4(out + 4 * q, narrow4(v)); });
    const int64_t T = (int64_t)gridDim.x * kCastShape.block;
    for (int64_t i = done + (int64_t)blockIdx.x * kCastShape.block + threadIdx.x; i < n; i += T) out[i] = (uint16_t)f32_to_bf16(x[i]);
}

// pieces.fold_start: bf16 -> fp32, exact (the 16 bits moved to the top).
__global__ __launch_bounds__(kWidenShape.block) void widen_bf16_kernel(const uint16_t* __restrict__ x, float* __restrict__ out,
                                                              int64_t n, int vec) {
    int64_t done = 0;
    if (vec)
        done = quad_loop<kWidenShape.unroll, kWidenShape.block>(
            n / 4, [&](int64_t q) { return ldh4(x + 4 * q); }, [&](int64_t q, eu2 w) { st4(out + 4 * q, widen4(w)); });
    const int64_t T = (int64_t)gridDim.x * kWidenShape.block;
    for (int64_t i = done + (int64_t)blockIdx.x * kWidenShape.block + threadIdx.x; i < n; i += T) out[i] = bf16_to_f32(x[i]);
}

struct AccG {
    ef4 acc, g;
};

// pieces.fold_add: acc += widen(g), one fp32 rounding per element.
template <bool BF16G>
__global__ __launch_bounds__(kFoldShape.block) void fold_add_kernel(float* __restrict__ acc, const void* __restrict__ g,
                                                            int64_t n, int vec) {
    int64_t done = 0;
    if (vec)
        done = quad_loop<kFoldShape.unroll, kFoldShape.block>(
            n / 4,
            [&](int64_t q) {
                AccG r;
                r.acc = ld4(acc + 4 * q);
                r.g = BF16G ? widen4(ldh4(static_cast<const uint16_t*>(g) + 4 * q)) : ld4(static_cast<const float*>(g) + 4 * q);
                return r;
            },
            [&](int64_t q, AccG r) { st4(acc + 4 * q, ef4{r.acc[0] + r.g[0], r.acc[1] + r.g[1], r.acc[2] + r.g[2], r.acc[3] + r.g[3]}); });
    const int64_t T = (int64_t)gridDim.x * kFoldShape.block;
    for (int64_t i = done + (int64_t)blockIdx.x * kFoldShape.block + threadIdx.x; i < n; i += T) {
        const float gv = BF16G ? bf16_to_f32(static_cast<const uint16_t*>(g)[i]) : static_cast<const float*>(g)[i];
        acc[i] = acc[i] + gv;
    }
}

// OrderedAccumulator's fold into a bf16 sum (runtime/accumulate.py:101-102,
// `acc.add_(t)` on a bf16 tensor): acc = bf16(float(acc) + widen(g)), the
// fp32 add rounded once more to bf16, as torch's in-place add computes it.
template <bool BF16G>
__global__ __launch_bounds__(kFoldShape.block) void fold_add_bf16_kernel(uint16_t* __restrict__ acc, const void* __restrict__ g,
                                                                 int64_t n, int vec) {
    int64_t done = 0;
    if (vec)
        done = quad_loop<kFoldShape.unroll, kFoldShape.block>(
            n / 4,
            [&](int64_t q) {
                AccG r;
                r.acc = widen4(ldh4(acc + 4 * q));
                r.g = BF16G ? widen4(ldh4(static_cast<const uint16_t*>(g) + 4 * q)) : ld4(static_cast<const float*>(g) + 4 * q);
                return r;
            },
            [&](int64_t q, AccG r) {
                sth4(acc + 4 * q, narrow4(ef4{r.acc[0] + r.g[0], r.acc[1] + r.g[1], r.acc[2] + r.g[2], r.acc[3] + r.g[3]}));
            });
    const int64_t T = (int64_t)gridDim.x * kFoldShape.block;
    for (int64_t i = done + (int64_t)blockIdx.x * kFoldShape.block + threadIdx.x; i < n; i += T) {
        const float gv = BF16G ? bf16_to_f32(static_cast<const uint16_t*>(g)[i]) : static_cast<const float*>(g)[i];
        acc[i] = (uint16_t)f32_to_bf16(bf16_to_f32(acc[i]) + gv);
    }
}

// Blocks for n elements: one quad per thread per unrolled slot, capped at
// the shape's blocks per CU.
static unsigned ew_blocks(int64_t n, EwShape sh) {
    const DeviceInfo& dev = device_info();
    const int64_t per_block = (int64_t)sh.block * 4 * sh.unroll;
    const int64_t want = (n + per_block - 1) / per_block;
    // a dispatch counts its work-items in 32 bits: past that the grid strides
    const int64_t cap = std::min<int64_t>((int64_t)dev.cus * sh.bpc, 0xFFFFFFFFLL / sh.block);
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, cap));
}

}  // namespace ely

using namespace ely;

extern "C" {

int ely_cast_bf16(const float* x, uint16_t* out, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_cast_bf16: negative n");
        if (n == 0) return;
        if (!x || !out) fail(ELY_EINVAL, "ely_cast_bf16: null pointer");
        const int vec = aligned16(x) && (reinterpret_cast<uintptr_t>(out) % 8 == 0);
        hipLaunchKernelGGL(cast_bf16_kernel, dim3(ew_blocks(n, kCastShape)), dim3(kCastShape.block), 0, static_cast<hipStream_t>(stream),
                           x, out, n, vec);
        check_launch("cast_bf16_kernel");
    });
}

int ely_widen_bf16(const uint16_t* x, float* out, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_widen_bf16: negative n");
        if (n == 0) return;
        if (!x || !out) fail(ELY_EINVAL, "ely_widen_bf16: null pointer");
        const int vec = aligned16(out) && (reinterpret_cast<uintptr_t>(x) % 8 == 0);
        hipLaunchKernelGGL(widen_bf16_kernel, dim3(ew_blocks(n, kWidenShape)), dim3(kWidenShape.block), 0,
                           static_cast<hipStream_t>(stream), x, out, n, vec);
        check_launch("widen_bf16_kernel");
    });
}

int ely_fold_add(float* acc, const void* g, int32_t g_dtype, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_fold_add: negative n");
        if (g_dtype != ELY_F32 && g_dtype != ELY_BF16) fail(ELY_EINVAL, "ely_fold_add: g_dtype");
        if (n == 0) return;
        if (!acc || !g) fail(ELY_EINVAL, "ely_fold_add: null pointer");
        const int vec = aligned16(acc) && (reinterpret_cast<uintptr_t>(g) % (g_dtype == ELY_BF16 ? 8 : 16) == 0);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (g_dtype == ELY_BF16)
            hipLaunchKernelGGL(fold_add_kernel<true>, dim3(ew_blocks(n, kFoldShape)), dim3(kFoldShape.block), 0, s, acc, g, n, vec);
        else
            hipLaunchKernelGGL(fold_add_kernel<false>, dim3(ew_blocks(n, kFoldShape)), dim3(kFoldShape.block), 0, s, acc, g, n, vec);
        check_launch("fold_add_kernel");
    });
}

int ely_fold_add_bf16(uint16_t* acc, const void* g, int32_t g_dtype, int64_t n, void* stream) {
    return guarded([&] {
        if (n < 0) fail(ELY_EINVAL, "ely_fold_add_bf16: negative n");
        if (g_dtype != ELY_F32 && g_dtype != ELY_BF16) fail(ELY_EINVAL, "ely_fold_add_bf16: g_dtype");
        if (n == 0) return;
        if (!acc || !g) fail(ELY_EINVAL, "ely_fold_add_bf16: null pointer");
        const int vec = (reinterpret_cast<uintptr_t>(acc) % 8 == 0) &&
                        (reinterpret_cast<uintptr_t>(g) % (g_dtype == ELY_BF16 ? 8 : 16) == 0);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (g_dtype == ELY_BF16)
            hipLaunchKernelGGL(fold_add_bf16_kernel<true>, dim3(ew_blocks(n, kFoldShape)), dim3(kFoldShape.block), 0, s, acc, g, n, vec);
        else
            hipLaunchKernelGGL(fold_add_bf16_kernel<false>, dim3(ew_blocks(n, kFoldShape)), dim3(kFoldShape.block), 0, s, acc, g, n, vec);
        check_launch("fold_add_bf16_kernel");
    });
}

}  // extern "C"
