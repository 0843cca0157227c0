// planes.hip -- the byte-level transforms of the lossless boundary wires on
// gfx950, so that only the (host-compressed) planes cross PCIe:
//
//   * byte planes (codec/planes.py:141-190): n elements of esz bytes become
//     esz planes of n bytes, most significant byte first, and back;
//   * e4m3 nibble planes (codec/fp8_planes.py:19-52): the e4m3 code of every
//     element, which must reproduce the element exactly, split into a plane
//     of high nibbles and a plane of low nibbles, two nibbles per byte
//     (element 2i in the high half), and back to fp32.
//
// All four are one HBM pass.  The vector paths move 16 elements per lane per
// step: each plane store is one 16-byte (byte planes) or 8-byte (nibbles)
// vector, contiguous across the wave.  Shapes the vector path cannot take
// (unaligned pointers, n not a multiple of 16) run element-wise.
#include <algorithm>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {

constexpr int kPBlock = 256;

static unsigned grid_for(int64_t work, int per_cu = 8) {
    const int64_t cap = (int64_t)device_info().cus * per_cu;
    const int64_t b = std::max<int64_t>(1, std::min<int64_t>((work + kPBlock - 1) / kPBlock, cap));
    return (unsigned)b;
}

// ------------------------------------------------------------ byte planes

// Byte b (little-endian index within an element) of the 16 elements whose
// bytes are the words w[0 .. 4*ESZ), packed in element order.
template <int ESZ>
__device__ __forceinline__ uint4 gather_byte(const uint32_t (&w)[4 * ESZ], int b) {
    uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int byte = e * ESZ + b;  // byte offset within the 16 elements
        o[e / 4] |= ((w[byte / 4] >> (8 * (byte % 4))) & 0xFFu) << (8 * (e % 4));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int ESZ>
__global__ __launch_bounds__(kPBlock) void split_vec_kernel(const uint4* __restrict__ x, int64_t n16,
                                                            uint8_t* __restrict__ planes, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    for (int64_t c = (int64_t)blockIdx.x * kPBlock + threadIdx.x; c < n16; c += stride) {
        uint32_t w[4 * ESZ];
#pragma unroll
        for (int j = 0; j < ESZ; ++j) {
            const uint4 v = x[c * ESZ + j];
            w[4 * j] = v.x;
            w[4 * j + 1] = v.y;
            w[4 * j + 2] = v.z;
            w[4 * j + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < ESZ; ++j)
            *reinterpret_cast<uint4*>(planes + (int64_t)j * n + c * 16) = gather_byte<ESZ>(w, ESZ - 1 - j);
    }
}

__global__ __launch_bounds__(kPBlock) void split_any_kernel(const uint8_t* __restrict__ x, int64_t n, int esz,
                                                            uint8_t* __restrict__ planes) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    for (int64_t i = (int64_t)blockIdx.x * kPBlock + threadIdx.x; i < n; i += stride)
        for (int j = 0; j < esz; ++j) planes[(int64_t)j * n + i] = x[i * esz + (esz - 1 - j)];
}

template <int ESZ>
__global__ __launch_bounds__(kPBlock) void join_vec_kernel(const uint8_t* __restrict__ planes, int64_t n16, int64_t n,
                                                           uint4* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    for (int64_t c = (int64_t)blockIdx.x * kPBlock + threadIdx.x; c < n16; c += stride) {
        uint32_t pl[ESZ][4];
#pragma unroll
        for (int j = 0; j < ESZ; ++j) {
            const uint4 v = *reinterpret_cast<const uint4*>(planes + (int64_t)j * n + c * 16);
            pl[j][0] = v.x;
            pl[j][1] = v.y;
            pl[j][2] = v.z;
            pl[j][3] = v.w;
        }
        uint32_t words[ESZ * 4];
#pragma unroll
        for (int q = 0; q < ESZ * 4; ++q) words[q] = 0;
#pragma unroll
        for (int j = 0; j < ESZ; ++j) {
            const int b = ESZ - 1 - j;  // the plane's byte within an element
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t byte = (pl[j][e / 4] >> (8 * (e % 4))) & 0xFFu;
                const int off = e * ESZ + b;
                words[off / 4] |= byte << (8 * (off % 4));
            }
        }
#pragma unroll
        for (int j = 0; j < ESZ; ++j)
            out[c * ESZ + j] = make_uint4(words[4 * j], words[4 * j + 1], words[4 * j + 2], words[4 * j + 3]);
    }
}

__global__ __launch_bounds__(kPBlock) void join_any_kernel(const uint8_t* __restrict__ planes, int64_t n, int esz,
                                                           uint8_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    for (int64_t i = (int64_t)blockIdx.x * kPBlock + threadIdx.x; i < n; i += stride)
        for (int j = 0; j < esz; ++j) out[i * esz + (esz - 1 - j)] = planes[(int64_t)j * n + i];
}

// ---------------------------------------------------------- nibble planes

constexpr uint32_t kE4M3MaxBits = 0x43E00000u;  // 448.0f

// e4m3 code of v and whether it reproduces v exactly (fp8_planes.py:22-24:
// torch.equal(f8.to(t.dtype), t): NaN never equal, -0 equal to 0).  On
// |v| <= 448 the conversion instruction is torch's rounding; anything else
// (NaN, Inf, beyond the largest finite e4m3) is not representable.
__device__ __forceinline__ uint32_t e4m3_exact(float v, bool& ok) {
    if (!((__float_as_uint(v) & 0x7FFFFFFFu) <= kE4M3MaxBits)) {
        ok = false;
        return 0u;
    }
    const uint32_t code = cvt_pk_fp8<kE4M3, false>(v, 0.0f, 0u) & 0xFFu;
    float back, unused;
    cvt_pk_f32<kE4M3, false>(code, back, unused);
    ok = back == v;
    return code;
}

template <bool BF16>
__device__ __forceinline__ float load_elem(const void* t, int64_t i) {
    if (BF16) return bf16_to_f32(static_cast<const uint16_t*>(t)[i]);
    return static_cast<const float*>(t)[i];
}

template <bool BF16>
__global__ __launch_bounds__(kPBlock) void nibbles_encode_kernel(const void* __restrict__ t, int64_t n, int vec,
                                                                 uint8_t* __restrict__ hi, uint8_t* __restrict__ lo,
                                                                 unsigned long long* __restrict__ bad) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    const int64_t tid = (int64_t)blockIdx.x * kPBlock + threadIdx.x;
    uint32_t nbad = 0;
    int64_t done = 0;  // elements covered by the vector path
    if (vec) {
        const int64_t n16 = n / 16;
        for (int64_t c = tid; c < n16; c += stride) {
            float f[16];
            if (BF16) {
                const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(t) + c * 16);
                const uint4 a = p[0], b = p[1];
                const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    f[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
                    f[2 * j + 1] = bf16_to_f32(w[j] >> 16);
                }
            } else {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(t) + c * 16);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 a = p[j];
                    f[4 * j] = a.x;
                    f[4 * j + 1] = a.y;
                    f[4 * j + 2] = a.z;
                    f[4 * j + 3] = a.w;
                }
            }
            uint32_t hw[2] = {0u, 0u}, lw[2] = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                bool ok;
                const uint32_t code = e4m3_exact(f[e], ok);
                nbad += ok ? 0u : 1u;
                // element 2i -> high half of byte i; byte i sits at bits 8*(i%4) of word i/4
                const int sh = 8 * ((e / 2) % 4) + ((e & 1) ? 0 : 4);
                hw[e / 8] |= (code >> 4) << sh;
                lw[e / 8] |= (code & 0xFu) << sh;
            }
            *reinterpret_cast<uint2*>(hi + c * 8) = make_uint2(hw[0], hw[1]);
            *reinterpret_cast<uint2*>(lo + c * 8) = make_uint2(lw[0], lw[1]);
        }
        done = n16 * 16;
    }
    // one output byte (two elements) per thread from `done` on
    const int64_t nbytes = (n + 1) / 2;
    for (int64_t b = done / 2 + tid; b < nbytes; b += stride) {
        uint32_t h = 0, l = 0;
        for (int k = 0; k < 2; ++k) {
            const int64_t i = 2 * b + k;
            if (i < n) {
                bool ok;
                const uint32_t code = e4m3_exact(load_elem<BF16>(t, i), ok);
                nbad += ok ? 0u : 1u;
                h |= (code >> 4) << (k ? 0 : 4);
                l |= (code & 0xFu) << (k ? 0 : 4);
            }
        }
        hi[b] = (uint8_t)h;
        lo[b] = (uint8_t)l;
    }
    // one atomic per wave that saw a mismatch
    const uint32_t wave_bad = wave_sum_u32(nbad);
    if ((threadIdx.x & (kWave - 1)) == 0 && wave_bad) atomicAdd(bad, (unsigned long long)wave_bad);
}

__global__ __launch_bounds__(kPBlock) void nibbles_decode_kernel(const uint8_t* __restrict__ hi,
                                                                 const uint8_t* __restrict__ lo, int64_t n, int vec,
                                                                 float* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    const int64_t tid = (int64_t)blockIdx.x * kPBlock + threadIdx.x;
    int64_t done = 0;
    if (vec) {
        const int64_t n16 = n / 16;
        for (int64_t c = tid; c < n16; c += stride) {
            const uint2 h = *reinterpret_cast<const uint2*>(hi + c * 8);
            const uint2 l = *reinterpret_cast<const uint2*>(lo + c * 8);
            const uint32_t hw[2] = {h.x, h.y}, lw[2] = {l.x, l.y};
            float f[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // codes of elements 4q .. 4q+3 packed into one word for the instruction
                uint32_t word = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int e = 4 * q + k;
                    const int sh = 8 * ((e / 2) % 4) + ((e & 1) ? 0 : 4);
                    const uint32_t code = (((hw[e / 8] >> sh) & 0xFu) << 4) | ((lw[e / 8] >> sh) & 0xFu);
                    word |= code << (8 * k);
                }
                cvt_pk_f32<kE4M3, false>(word, f[4 * q], f[4 * q + 1]);
                cvt_pk_f32<kE4M3, true>(word, f[4 * q + 2], f[4 * q + 3]);
            }
            float4* o = reinterpret_cast<float4*>(out + c * 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = make_float4(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
        }
        done = n16 * 16;
    }
    for (int64_t i = done + tid; i < n; i += stride) {
        const int sh = (i & 1) ? 0 : 4;
        const uint32_t code = (((uint32_t)hi[i / 2] >> sh) & 0xFu) << 4 | (((uint32_t)lo[i / 2] >> sh) & 0xFu);
        float a, unused;
        cvt_pk_f32<kE4M3, false>(code, a, unused);
        out[i] = a;
    }
}

static void check_n(int64_t n) {
    if (n < 0) fail(ELY_EINVAL, "negative element count");
}

}  // namespace ely

using namespace ely;

extern "C" {

int ely_byteplanes_split(const void* x, int64_t n, int32_t esz, uint8_t* planes, void* stream) {
    return guarded([&] {
        check_n(n);
        if (esz != 1 && esz != 2 && esz != 4 && esz != 8) fail(ELY_EINVAL, "ely_byteplanes_split: esz must be 1, 2, 4 or 8");
        if (n == 0) return;
        if (!x || !planes) fail(ELY_EINVAL, "ely_byteplanes_split: null pointer");
        if (n > INT64_MAX / 8) fail(ELY_EINVAL, "ely_byteplanes_split: n too large");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (n % 16 == 0 && aligned16(x) && aligned16(planes)) {
            const int64_t n16 = n / 16;
            const unsigned g = grid_for(n16);
            const uint4* xv = static_cast<const uint4*>(x);
            switch (esz) {
                case 1: hipLaunchKernelGGL(split_vec_kernel<1>, dim3(g), dim3(kPBlock), 0, s, xv, n16, planes, n); break;
                case 2: hipLaunchKernelGGL(split_vec_kernel<2>, dim3(g), dim3(kPBlock), 0, s, xv, n16, planes, n); break;
                case 4: hipLaunchKernelGGL(split_vec_kernel<4>, dim3(g), dim3(kPBlock), 0, s, xv, n16, planes, n); break;
                default: hipLaunchKernelGGL(split_vec_kernel<8>, dim3(g), dim3(kPBlock), 0, s, xv, n16, planes, n); break;
            }
            check_launch("split_vec_kernel");
        } else {
            hipLaunchKernelGGL(split_any_kernel, dim3(grid_for(n)), dim3(kPBlock), 0, s, static_cast<const uint8_t*>(x), n,
                               (int)esz, planes);
            check_launch("split_any_kernel");
        }
    });
}

int ely_byteplanes_join(const uint8_t* planes, int64_t n, int32_t esz, void* out, void* stream) {
    return guarded([&] {
        check_n(n);
        if (esz != 1 && esz != 2 && esz != 4 && esz != 8) fail(ELY_EINVAL, "ely_byteplanes_join: esz must be 1, 2, 4 or 8");
        if (n == 0) return;
        if (!out || !planes) fail(ELY_EINVAL, "ely_byteplanes_join: null pointer");
        if (n > INT64_MAX / 8) fail(ELY_EINVAL, "ely_byteplanes_join: n too large");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (n % 16 == 0 && aligned16(out) && aligned16(planes)) {
            const int64_t n16 = n / 16;
            const unsigned g = grid_for(n16);
            uint4* ov = static_cast<uint4*>(out);
            switch (esz) {
                case 1: hipLaunchKernelGGL(join_vec_kernel<1>, dim3(g), dim3(kPBlock), 0, s, planes, n16, n, ov); break;
                case 2: hipLaunchKernelGGL(join_vec_kernel<2>, dim3(g), dim3(kPBlock), 0, s, planes, n16, n, ov); break;
                case 4: hipLaunchKernelGGL(join_vec_kernel<4>, dim3(g), dim3(kPBlock), 0, s, planes, n16, n, ov); break;
                default: hipLaunchKernelGGL(join_vec_kernel<8>, dim3(g), dim3(kPBlock), 0, s, planes, n16, n, ov); break;
            }
            check_launch("join_vec_kernel");
        } else {
            hipLaunchKernelGGL(join_any_kernel, dim3(grid_for(n)), dim3(kPBlock), 0, s, planes, n, (int)esz,
                               static_cast<uint8_t*>(out));
            check_launch("join_any_kernel");
        }
    });
}

int ely_fp8_nibbles_encode(const void* t, int32_t t_dtype, int64_t n, uint8_t* hi, uint8_t* lo,
                           unsigned long long* bad_dev, void* stream) {
    return guarded([&] {
        check_n(n);
        if (t_dtype != ELY_F32 && t_dtype != ELY_BF16) fail(ELY_EINVAL, "ely_fp8_nibbles_encode: t_dtype must be ELY_F32 or ELY_BF16");
        if (n == 0) return;
        if (!t || !hi || !lo || !bad_dev) fail(ELY_EINVAL, "ely_fp8_nibbles_encode: null pointer");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int vec = aligned16(t) && (reinterpret_cast<uintptr_t>(hi) % 8 == 0) && (reinterpret_cast<uintptr_t>(lo) % 8 == 0);
        const unsigned g = grid_for(std::max<int64_t>(n / 16, 1));
        if (t_dtype == ELY_BF16)
            hipLaunchKernelGGL(nibbles_encode_kernel<true>, dim3(g), dim3(kPBlock), 0, s, t, n, vec, hi, lo, bad_dev);
        else
            hipLaunchKernelGGL(nibbles_encode_kernel<false>, dim3(g), dim3(kPBlock), 0, s, t, n, vec, hi, lo, bad_dev);
        check_launch("nibbles_encode_kernel");
    });
}

int ely_fp8_nibbles_decode(const uint8_t* hi, const uint8_t* lo, int64_t n, float* out, void* stream) {
    return guarded([&] {
        check_n(n);
        if (n == 0) return;
        if (!out || !hi || !lo) fail(ELY_EINVAL, "ely_fp8_nibbles_decode: null pointer");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int vec = aligned16(out) && (reinterpret_cast<uintptr_t>(hi) % 8 == 0) && (reinterpret_cast<uintptr_t>(lo) % 8 == 0);
        hipLaunchKernelGGL(nibbles_decode_kernel, dim3(grid_for(std::max<int64_t>(n / 16, 1))), dim3(kPBlock), 0, s, hi, lo,
                           n, vec, out);
        check_launch("nibbles_decode_kernel");
    });
}

}  // extern "C"
