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
// All four are one HBM pass.  The vector paths keep every load and store
// instruction of a wave on one contiguous run (a lane moves one 16-byte
// vector of elements for the byte planes, 4 codes for the nibble decode).
// Shapes the vector path cannot take (unaligned pointers, n not a multiple
// of 16) run element-wise.
#include <algorithm>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {

#ifndef ELY_PLANES_UNROLL
#define ELY_PLANES_UNROLL 1  // byte planes: 16-byte vectors a lane keeps in flight
#endif
#ifndef ELY_PLANES_BPC
#define ELY_PLANES_BPC 262144  // byte planes: grid cap in blocks per compute unit (one-shot)
#endif
#ifndef ELY_NIBBLES_UNROLL
#define ELY_NIBBLES_UNROLL 2  // nibble planes: vectors a lane keeps in flight
#endif
#ifndef ELY_NIB_BALLOT
#define ELY_NIB_BALLOT 1  // nibble encode: count mismatches per wave on the scalar unit
#endif
#ifndef ELY_NIBBLES_BPC
#define ELY_NIBBLES_BPC 262144  // nibble planes: grid cap in blocks per compute unit (one-shot)
#endif

#ifndef ELY_PLANES_BLOCK
// byte planes: threads per block.  64-thread blocks on a one-shot grid,
// against 256-thread blocks at 4 per CU in one process on the same buffers
// (identical planes): 2^28 fp32 split 6.02 TB/s against 5.56, join 5.89
// against 5.23; 2^29 bf16 6.53 and 6.53 against 5.75 and 5.56; C1's
// activation 6.20 and 6.28-6.39 against 5.92 and 5.78-5.88.
#define ELY_PLANES_BLOCK 64
#endif
constexpr int kPBlock = ELY_PLANES_BLOCK;
#ifndef ELY_NIBBLES_BLOCK
// nibble planes: threads per block.  64-thread blocks on a one-shot grid,
// against 256-thread blocks at 8 per CU in one process on the same buffers
// (exact round trips): encode 5.89-6.15 TB/s on C1's activation against
// 5.62-5.76 and 6.48-6.51 on 2^29 elements against 5.68-5.73; decode equal
// on C1 (5.3) and 5.65-5.70 against 5.03-5.05 on 2^29
#define ELY_NIBBLES_BLOCK 64
#endif
constexpr int kNBlock = ELY_NIBBLES_BLOCK;

static unsigned grid_for(int64_t work, int per_cu, int block = kPBlock) {
    // a dispatch counts its work-items in 32 bits: past that the grid strides
    const int64_t cap = std::min<int64_t>((int64_t)device_info().cus * per_cu, 0xFFFFFFFFLL / block);
    const int64_t b = std::max<int64_t>(1, std::min<int64_t>((work + block - 1) / block, cap));
    return (unsigned)b;
}

// ------------------------------------------------------------ byte planes

// The vector paths move one 16-byte vector of elements per lane (EPL =
// 16 / esz elements): a lane's plane share is EPL bytes, so every load and
// every store instruction of a wave covers one contiguous run.  kPUnroll
// vectors per lane are loaded before the first is used; all streams are
// nontemporal.
constexpr int kPUnroll = ELY_PLANES_UNROLL;
constexpr int kNUnroll = ELY_NIBBLES_UNROLL;

typedef uint32_t pv4 __attribute__((ext_vector_type(4)));
typedef uint32_t pv2 __attribute__((ext_vector_type(2)));
#define PL_G1 __attribute__((address_space(1)))

__device__ __forceinline__ pv4 ld16(const void* p) { return __builtin_nontemporal_load((const PL_G1 pv4*)p); }
__device__ __forceinline__ void st16(void* p, pv4 v) { __builtin_nontemporal_store(v, (PL_G1 pv4*)p); }

// EPL bytes (EPL = 16, 8, 4 or 2) packed little-endian in w[0..EPL/4) (or
// the low half of w[0] for 2), stored at p.
template <int EPL>
__device__ __forceinline__ void st_plane(uint8_t* p, const uint32_t (&w)[4]) {
    if (EPL == 16) st16(p, pv4{w[0], w[1], w[2], w[3]});
    else if (EPL == 8) __builtin_nontemporal_store(pv2{w[0], w[1]}, (PL_G1 pv2*)p);
    else if (EPL == 4) __builtin_nontemporal_store(w[0], (PL_G1 uint32_t*)p);
    else __builtin_nontemporal_store((uint16_t)w[0], (PL_G1 uint16_t*)p);
}

template <int EPL>
__device__ __forceinline__ void ld_plane(const uint8_t* p, uint32_t (&w)[4]) {
    w[0] = w[1] = w[2] = w[3] = 0;
    if (EPL == 16) {
        const pv4 v = ld16(p);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    } else if (EPL == 8) {
        const pv2 v = __builtin_nontemporal_load((const PL_G1 pv2*)p);
        w[0] = v[0]; w[1] = v[1];
    } else if (EPL == 4) {
        w[0] = __builtin_nontemporal_load((const PL_G1 uint32_t*)p);
    } else {
        w[0] = __builtin_nontemporal_load((const PL_G1 uint16_t*)p);
    }
}

template <int ESZ>
__global__ __launch_bounds__(kPBlock) void split_vec_kernel(const uint8_t* __restrict__ x, int64_t nvec,
                                                            uint8_t* __restrict__ planes, int64_t n) {
    constexpr int EPL = 16 / ESZ;
    const int64_t T = (int64_t)gridDim.x * kPBlock;
    const int64_t t = (int64_t)blockIdx.x * kPBlock + threadIdx.x;
    for (int64_t base = t; base < nvec; base += T * kPUnroll) {
        pv4 v[kPUnroll];
#pragma unroll
        for (int u = 0; u < kPUnroll; ++u) {
            const int64_t vi = base + u * T;
            v[u] = ld16(x + (vi < nvec ? vi : nvec - 1) * 16);
        }
#pragma unroll
        for (int u = 0; u < kPUnroll; ++u) {
            const int64_t vi = base + u * T;
            if (vi >= nvec) continue;
            const uint32_t in[4] = {v[u][0], v[u][1], v[u][2], v[u][3]};
#pragma unroll
            for (int j = 0; j < ESZ; ++j) {
                const int b = ESZ - 1 - j;  // plane j holds byte esz-1-j of every element
                uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int byte = e * ESZ + b;
                    w[e / 4] |= ((in[byte / 4] >> (8 * (byte % 4))) & 0xFFu) << (8 * (e % 4));
                }
                st_plane<EPL>(planes + (int64_t)j * n + vi * EPL, w);
            }
        }
    }
}

__global__ __launch_bounds__(kPBlock) void split_any_kernel(const uint8_t* __restrict__ x, int64_t n, int esz,
                                                            uint8_t* __restrict__ planes) {
    const int64_t stride = (int64_t)gridDim.x * kPBlock;
    for (int64_t i = (int64_t)blockIdx.x * kPBlock + threadIdx.x; i < n; i += stride)
        for (int j = 0; j < esz; ++j) planes[(int64_t)j * n + i] = x[i * esz + (esz - 1 - j)];
}

template <int ESZ>
__global__ __launch_bounds__(kPBlock) void join_vec_kernel(const uint8_t* __restrict__ planes, int64_t nvec, int64_t n,
                                                           uint8_t* __restrict__ out) {
    constexpr int EPL = 16 / ESZ;
    const int64_t T = (int64_t)gridDim.x * kPBlock;
    const int64_t t = (int64_t)blockIdx.x * kPBlock + threadIdx.x;
    for (int64_t base = t; base < nvec; base += T * kPUnroll) {
        uint32_t pl[kPUnroll][ESZ][4];
#pragma unroll
        for (int u = 0; u < kPUnroll; ++u) {
            const int64_t vi = base + u * T;
            const int64_t vc = vi < nvec ? vi : nvec - 1;
#pragma unroll
            for (int j = 0; j < ESZ; ++j) ld_plane<EPL>(planes + (int64_t)j * n + vc * EPL, pl[u][j]);
        }
#pragma unroll
        for (int u = 0; u < kPUnroll; ++u) {
            const int64_t vi = base + u * T;
            if (vi >= nvec) continue;
            uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < ESZ; ++j) {
                const int b = ESZ - 1 - j;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const uint32_t byte = (pl[u][j][e / 4] >> (8 * (e % 4))) & 0xFFu;
                    const int off = e * ESZ + b;
                    words[off / 4] |= byte << (8 * (off % 4));
                }
            }
            st16(out + vi * 16, pv4{words[0], words[1], words[2], words[3]});
        }
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

// Four codes (element k in byte k of w) -> their nibble pairs as the planes
// hold them, in the low 16 bits: hi byte 0 = c0 >> 4 << 4 | c1 >> 4, byte 1
// the same of c2, c3; lo likewise with the low nibbles.
__device__ __forceinline__ uint32_t hi_pairs(uint32_t w) {
    const uint32_t t = w & 0xF0F0F0F0u;
    const uint32_t u = t | (t >> 12);  // bytes 0 and 2 hold the pairs
    return (u & 0xFFu) | ((u >> 8) & 0xFF00u);
}
__device__ __forceinline__ uint32_t lo_pairs(uint32_t w) {
    const uint32_t t = w & 0x0F0F0F0Fu;
    const uint32_t u = (t << 4) | (t >> 8);  // bytes 0 and 2 hold the pairs
    return (u & 0xFFu) | ((u >> 8) & 0xFF00u);
}

// The inverse: two bytes of each plane (h, l, low 16 bits) -> the four
// codes, element k in byte k.
__device__ __forceinline__ uint32_t join_pairs(uint32_t h, uint32_t l) {
    const uint32_t hx = (h & 0xFFu) | ((h & 0xFF00u) << 8);
    const uint32_t hs = hx | (hx << 8);  // bytes h0, h0, h1, h1
    const uint32_t lx = (l & 0xFFu) | ((l & 0xFF00u) << 8);
    const uint32_t ls = lx | (lx << 8);
    return (hs & 0x00F000F0u) | ((hs << 4) & 0xF000F000u) | ((ls >> 4) & 0x000F000Fu) | (ls & 0x0F000F00u);
}

// e4m3 codes of four floats, element k in byte k, and how many of them do
// not convert back to themselves, added to `bad`: with ELY_NIB_BALLOT the
// count of the whole wave's active lanes (each comparison's lane mask,
// popcounted on the scalar unit), else this lane's.  That test alone decides
// representability: a NaN never equals, and no code decodes to Inf or to a
// value beyond 448, so only the grid values of the instruction's exact
// domain pass (where it is torch's rounding); the codes of the others are
// never used (the encode is refused).
__device__ __forceinline__ uint32_t e4m3_quad(float a, float b, float c, float d, uint32_t& bad) {
    uint32_t w = cvt_pk_fp8<kE4M3, false>(a, b, 0u);
    w = cvt_pk_fp8<kE4M3, true>(c, d, w);
    float ra, rb, rc, rd;
    cvt_pk_f32<kE4M3, false>(w, ra, rb);
    cvt_pk_f32<kE4M3, true>(w, rc, rd);
#if ELY_NIB_BALLOT
    bad += (uint32_t)(__builtin_popcountll(__builtin_amdgcn_ballot_w64(ra != a)) +
                      __builtin_popcountll(__builtin_amdgcn_ballot_w64(rb != b)) +
                      __builtin_popcountll(__builtin_amdgcn_ballot_w64(rc != c)) +
                      __builtin_popcountll(__builtin_amdgcn_ballot_w64(rd != d)));
#else
    bad += (ra != a) + (rb != b) + (rc != c) + (rd != d);
#endif
    return w;
}

// Encode: a lane converts one 16-byte vector of t (8 bf16 or 4 fp32), so its
// share of each nibble plane is EPL/2 bytes (4 or 2) and every load and
// store instruction of a wave covers one contiguous run.
template <bool BF16>
__global__ __launch_bounds__(kNBlock) void nibbles_encode_kernel(const void* __restrict__ t, int64_t n, int vec,
                                                                 uint8_t* __restrict__ hi, uint8_t* __restrict__ lo,
                                                                 unsigned long long* __restrict__ bad) {
    constexpr int EPL = BF16 ? 8 : 4;
    const int64_t T = (int64_t)gridDim.x * kNBlock;
    const int64_t tid = (int64_t)blockIdx.x * kNBlock + threadIdx.x;
    uint32_t nbad = 0;  // this lane's mismatches
    uint32_t qbad = 0;  // the vector path's (the wave's, with ELY_NIB_BALLOT)
    int64_t done = 0;  // elements covered by the vector path
    if (vec) {
        const int64_t nvec = n / 16 * (16 / EPL);  // whole 16-element groups only
        const uint8_t* tb = static_cast<const uint8_t*>(t);
        for (int64_t base = tid; base < nvec; base += T * kNUnroll) {
            pv4 v[kNUnroll];
#pragma unroll
            for (int u = 0; u < kNUnroll; ++u) {
                const int64_t vi = base + u * T;
                v[u] = ld16(tb + (vi < nvec ? vi : nvec - 1) * 16);
            }
#pragma unroll
            for (int u = 0; u < kNUnroll; ++u) {
                const int64_t vi = base + u * T;
                if (vi >= nvec) continue;
                float f[EPL];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (BF16) {
                        f[2 * j] = bf16_to_f32(v[u][j] & 0xFFFFu);
                        f[2 * j + 1] = bf16_to_f32(v[u][j] >> 16);
                    } else {
                        f[j] = __uint_as_float(v[u][j]);
                    }
                }
                uint32_t hw = 0u, lw = 0u;
#pragma unroll
                for (int e = 0; e < EPL; e += 4) {
                    const uint32_t w = e4m3_quad(f[e], f[e + 1], f[e + 2], f[e + 3], qbad);
                    hw |= hi_pairs(w) << (4 * e);
                    lw |= lo_pairs(w) << (4 * e);
                }
                if (BF16) {
                    __builtin_nontemporal_store(hw, (PL_G1 uint32_t*)(hi + vi * 4));
                    __builtin_nontemporal_store(lw, (PL_G1 uint32_t*)(lo + vi * 4));
                } else {
                    __builtin_nontemporal_store((uint16_t)hw, (PL_G1 uint16_t*)(hi + vi * 2));
                    __builtin_nontemporal_store((uint16_t)lw, (PL_G1 uint16_t*)(lo + vi * 2));
                }
            }
        }
        done = nvec * EPL;
    }
    // one output byte (two elements) per thread from `done` on
    const int64_t nbytes = (n + 1) / 2;
    for (int64_t b = done / 2 + tid; b < nbytes; b += T) {
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
    // one atomic per wave that saw a mismatch.  The wave counts of the vector
    // path are complete in lane 0: a lane past the end has no elements, and
    // lane 0 holds the wave's lowest vector, so it is active whenever any
    // lane is; every lane is active again here.
#if ELY_NIB_BALLOT
    const uint32_t wave_bad = __builtin_amdgcn_readfirstlane(qbad) + wave_sum_u32(nbad);
#else
    const uint32_t wave_bad = wave_sum_u32(nbad + qbad);
#endif
    if ((threadIdx.x & (kWave - 1)) == 0 && wave_bad) atomicAdd(bad, (unsigned long long)wave_bad);
}

// Decode: a lane takes 4 codes (2 bytes of each plane) and writes one 16-byte
// fp32 vector, so every store instruction covers one contiguous 1 KB.
__global__ __launch_bounds__(kNBlock) void nibbles_decode_kernel(const uint8_t* __restrict__ hi,
                                                                 const uint8_t* __restrict__ lo, int64_t n, int vec,
                                                                 float* __restrict__ out) {
    const int64_t T = (int64_t)gridDim.x * kNBlock;
    const int64_t tid = (int64_t)blockIdx.x * kNBlock + threadIdx.x;
    int64_t done = 0;
    if (vec) {
        const int64_t nq = n / 4;
        for (int64_t base = tid; base < nq; base += T * kNUnroll) {
            uint32_t h[kNUnroll], l[kNUnroll];
#pragma unroll
            for (int u = 0; u < kNUnroll; ++u) {
                const int64_t q = base + u * T;
                const int64_t qc = q < nq ? q : nq - 1;
                h[u] = __builtin_nontemporal_load((const PL_G1 uint16_t*)(hi + qc * 2));
                l[u] = __builtin_nontemporal_load((const PL_G1 uint16_t*)(lo + qc * 2));
            }
#pragma unroll
            for (int u = 0; u < kNUnroll; ++u) {
                const int64_t q = base + u * T;
                if (q >= nq) continue;
                const uint32_t word = join_pairs(h[u], l[u]);  // codes of elements 4q .. 4q+3, one per byte
                float a, b, c, d;
                cvt_pk_f32<kE4M3, false>(word, a, b);
                cvt_pk_f32<kE4M3, true>(word, c, d);
                st16(out + q * 4, pv4{__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)});
            }
        }
        done = nq * 4;
    }
    for (int64_t i = done + tid; i < n; i += T) {
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
            const int64_t nvec = n * esz / 16;
            const unsigned g = grid_for((nvec + kPUnroll - 1) / kPUnroll, ELY_PLANES_BPC);
            const uint8_t* xb = static_cast<const uint8_t*>(x);
            switch (esz) {
                case 1: hipLaunchKernelGGL(split_vec_kernel<1>, dim3(g), dim3(kPBlock), 0, s, xb, nvec, planes, n); break;
                case 2: hipLaunchKernelGGL(split_vec_kernel<2>, dim3(g), dim3(kPBlock), 0, s, xb, nvec, planes, n); break;
                case 4: hipLaunchKernelGGL(split_vec_kernel<4>, dim3(g), dim3(kPBlock), 0, s, xb, nvec, planes, n); break;
                default: hipLaunchKernelGGL(split_vec_kernel<8>, dim3(g), dim3(kPBlock), 0, s, xb, nvec, planes, n); break;
            }
            check_launch("split_vec_kernel");
        } else {
            hipLaunchKernelGGL(split_any_kernel, dim3(grid_for(n, ELY_PLANES_BPC)), dim3(kPBlock), 0, s, static_cast<const uint8_t*>(x), n,
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
            const int64_t nvec = n * esz / 16;
            const unsigned g = grid_for((nvec + kPUnroll - 1) / kPUnroll, ELY_PLANES_BPC);
            uint8_t* ob = static_cast<uint8_t*>(out);
            switch (esz) {
                case 1: hipLaunchKernelGGL(join_vec_kernel<1>, dim3(g), dim3(kPBlock), 0, s, planes, nvec, n, ob); break;
                case 2: hipLaunchKernelGGL(join_vec_kernel<2>, dim3(g), dim3(kPBlock), 0, s, planes, nvec, n, ob); break;
                case 4: hipLaunchKernelGGL(join_vec_kernel<4>, dim3(g), dim3(kPBlock), 0, s, planes, nvec, n, ob); break;
                default: hipLaunchKernelGGL(join_vec_kernel<8>, dim3(g), dim3(kPBlock), 0, s, planes, nvec, n, ob); break;
            }
            check_launch("join_vec_kernel");
        } else {
            hipLaunchKernelGGL(join_any_kernel, dim3(grid_for(n, ELY_PLANES_BPC)), dim3(kPBlock), 0, s, planes, n, (int)esz,
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
        const int vec = aligned16(t) && (reinterpret_cast<uintptr_t>(hi) % 4 == 0) && (reinterpret_cast<uintptr_t>(lo) % 4 == 0);
        // one lane per kNUnroll 16-byte vectors of the input: 8 bf16 or 4 fp32 elements each
        const int64_t epl = t_dtype == ELY_BF16 ? 8 : 4;
        const unsigned g = grid_for(std::max<int64_t>(n / epl / kNUnroll, 1), ELY_NIBBLES_BPC, kNBlock);
        if (t_dtype == ELY_BF16)
            hipLaunchKernelGGL(nibbles_encode_kernel<true>, dim3(g), dim3(kNBlock), 0, s, t, n, vec, hi, lo, bad_dev);
        else
            hipLaunchKernelGGL(nibbles_encode_kernel<false>, dim3(g), dim3(kNBlock), 0, s, t, n, vec, hi, lo, bad_dev);
        check_launch("nibbles_encode_kernel");
    });
}

int ely_fp8_nibbles_decode(const uint8_t* hi, const uint8_t* lo, int64_t n, float* out, void* stream) {
    return guarded([&] {
        check_n(n);
        if (n == 0) return;
        if (!out || !hi || !lo) fail(ELY_EINVAL, "ely_fp8_nibbles_decode: null pointer");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int vec = aligned16(out) && (reinterpret_cast<uintptr_t>(hi) % 2 == 0) && (reinterpret_cast<uintptr_t>(lo) % 2 == 0);
        hipLaunchKernelGGL(nibbles_decode_kernel, dim3(grid_for(std::max<int64_t>(n / 4 / kNUnroll, 1), ELY_NIBBLES_BPC, kNBlock)), dim3(kNBlock), 0, s,
                           hi, lo, n, vec, out);
        check_launch("nibbles_decode_kernel");
    });
}

}  // extern "C"
