// fp8.hip -- the fp8 boundary codec of model/fp8.py on gfx950.
//
// quantize (fp8.py:28-49): per row, k = frexp(amax|x|).exponent - ebias and
// q = fp8(x * 2^-k).  Three launch shapes:
//   * rows that fit registers (<= 64 lanes x 16 vectors of 16 bytes: 8192
//     bf16 / 4096 fp32 columns, 16-byte aligned): the row is read once into
//     VGPRs, |x|max is a butterfly over the wave, and codes are written from
//     the same registers: one HBM read and one write per element (3 B/elem
//     for bf16 -> fp8).  Rows of up to 6 vectors per lane take one wave;
//     longer ones are shared by a block's 4 waves, whose maxima meet in LDS,
//     so that each wave holds at most 4 vectors and more rows stream at once.
//     Each wave issues its loads one vector per lane at a time: fewer bytes
//     in flight per CU keep the memory latency, and the bandwidth, up.
//   * longer rows (per-tensor scaling is rows = 1): the row is cut into
//     2048-element segments.  A first launch reduces the row's |x|max into
//     at most 2,048 partial maxima (each wave strides over its row's
//     segments; integer max, so order-free), a small second launch folds the
//     partials per row, a third converts one segment per wave.  Two reads
//     of x, no atomics.
//   * any other shape (unaligned, columns not a multiple of the vector):
//     the same two launches with element-wise loads.
// Every row whose exponent keeps 2^-k, 2^k and every product exact
// (|k| <= 110, finite |x|max) converts with the instructions: bf16 words go
// straight into v_cvt_scalef32_pk_{fp8,bf8}_bf16 at scale 2^k (the code of
// x * 2^-k in one instruction per two elements), fp32 through a product and
// v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 (proved equal to torch's rounding on
// that domain by ely_selftest_fp8_scaled and ely_selftest_fp8_cvt); the
// other rows follow the bit-level restatement of torch's arithmetic (pow2
// rounded to the dtype, product rounded to the dtype, software conversion),
// uniformly per row.
//
// dequantize (fp8.py:52-53): out = float(q) * 2^k in the output dtype, the
// codes taken as one flat array (a wave's 1,024 codes may span rows), 8 codes
// per lane per step for bf16 output (4 for fp32) so every store instruction
// covers a contiguous 1 KB; bf16 output decodes with
// v_cvt_scalef32_pk_bf16_{fp8,bf8} at scale 2^k unless the vector holds a
// NaN code; roundtrip (fp8.py:56-63) fuses both.
#include <algorithm>
#include <map>
#include <mutex>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

#ifndef ELY_DEQ_SEG
#define ELY_DEQ_SEG 1024  // dequantize: codes per wave segment
#endif
#ifndef ELY_DEQ_BATCH
#define ELY_DEQ_BATCH 0  // dequantize: vectors per lane per load batch (0: the whole segment at once)
#endif
#ifndef ELY_SPLIT_WAVES
#define ELY_SPLIT_WAVES 2048  // split path: waves of the partial-max launch (at most)
#endif
#ifndef ELY_SPLIT_CACHED_MB
// split path: MB of x the |x|max launch reads last with plain loads instead
// of nontemporal ones.  C4 per-tensor: quantize 0.408 -> 0.403 ms, round
// trip 0.509 -> 0.499 ms (0, 192, 256 and 384 MB measured; a convert launch
// taking the segments last to first, to start on the cached ones, was
// slower)
#define ELY_SPLIT_CACHED_MB 256
#endif
#ifndef ELY_SPLIT_BATCH
#define ELY_SPLIT_BATCH 1  // split path: vectors per lane per load batch of the convert launch (0: all)
#endif
#ifndef ELY_Q_BATCH
#define ELY_Q_BATCH 1  // register paths: vectors per lane per load batch (0: the whole row at once)
#endif
#ifndef ELY_Q_LDS
// wave-per-row quantize: unused dynamic LDS per block, capping it at 16
// blocks (16 waves) per CU.  C1 back to back over 8 inputs, in one process:
// quantize 5.89-5.92 TB/s and round trip 5.92-5.96 against 5.80-5.82 and
// 5.74-5.85 with no cap (256-thread blocks capped at 4 per CU: 5.86-5.88,
// 5.93-5.94)
#define ELY_Q_LDS 10240
#endif
#ifndef ELY_DEQ_LDS
#define ELY_DEQ_LDS 0  // dequantize: unused dynamic LDS per block capping its blocks per CU (caps measured slower)
#endif
#ifndef ELY_RECOVER_KEEP_VPL
#define ELY_RECOVER_KEEP_VPL 16  // longest rows (vectors per lane) whose image reuses the test's codes
#endif
#ifndef ELY_RECOVER_BATCH
#define ELY_RECOVER_BATCH ELY_Q_BATCH  // recover register path: vectors per lane per load batch (0: all)
#endif
#ifndef ELY_RECOVER_WHOLE_VPL
#define ELY_RECOVER_WHOLE_VPL 8  // recover register path: rows of this many vectors per lane or more load at once
#endif

namespace ely {

#ifndef ELY_QBLOCK
// 64: in one process on the same buffers, dequantize 6.55-6.58 TB/s on C4
// and 5.86 on C1 against 6.29-6.46 and 5.68-5.71 on 256-thread blocks;
// the wave-per-row quantize the same (C1 6.0-6.1)
#define ELY_QBLOCK 64
#endif
constexpr int kQBlock = ELY_QBLOCK;            // threads per block; each wave takes its own row or segment
constexpr int kWavesPerBlock = kQBlock / kWave;
constexpr int kRowBlock = 256;                 // the block-row quantize and the row-max reduce: 4 waves share one row
constexpr int kRowWaves = kRowBlock / kWave;
constexpr int64_t kSegElems = 2048;            // split-path segment, elements
constexpr int64_t kDeqSegCodes = ELY_DEQ_SEG;  // dequantize segment, codes
constexpr int kRecoverKeepVpl = ELY_RECOVER_KEEP_VPL;
constexpr int kFastK = 110;                    // |k| bound of the instruction path

// ----------------------------------------------------------- element helpers

#ifndef ELY_FP8_NT
#define ELY_FP8_NT 3  // bit 0: nontemporal codec loads, bit 1: nontemporal stores
#endif

// Stores of streamed data; nontemporal when bit 1 of ELY_FP8_NT is set.
typedef uint32_t ev4u __attribute__((ext_vector_type(4)));
typedef uint32_t ev2u __attribute__((ext_vector_type(2)));
#define ELY_G1 __attribute__((address_space(1)))
__device__ __forceinline__ void st_vec(void* p, uint4 v) {
#if ELY_FP8_NT & 2
    __builtin_nontemporal_store(ev4u{v.x, v.y, v.z, v.w}, (ELY_G1 ev4u*)p);
#else
    *static_cast<uint4*>(p) = v;
#endif
}
__device__ __forceinline__ void st_vec2(void* p, uint2 v) {
#if ELY_FP8_NT & 2
    __builtin_nontemporal_store(ev2u{v.x, v.y}, (ELY_G1 ev2u*)p);
#else
    *static_cast<uint2*>(p) = v;
#endif
}
__device__ __forceinline__ void st_u32(void* p, uint32_t v) {
#if ELY_FP8_NT & 2
    __builtin_nontemporal_store(v, (ELY_G1 uint32_t*)p);
#else
    *static_cast<uint32_t*>(p) = v;
#endif
}

// 8- and 4-byte loads of streamed data.
__device__ __forceinline__ uint2 ld_vec2(const void* p) {
#if ELY_FP8_NT & 1
    const ev2u v = __builtin_nontemporal_load((const ELY_G1 ev2u*)p);
    return make_uint2(v[0], v[1]);
#else
    return *static_cast<const uint2*>(p);
#endif
}
__device__ __forceinline__ uint32_t ld_u32(const void* p) {
#if ELY_FP8_NT & 1
    return __builtin_nontemporal_load((const ELY_G1 uint32_t*)p);
#else
    return *static_cast<const uint32_t*>(p);
#endif
}

// One 16-byte load of streamed data.
template <bool NT = (ELY_FP8_NT & 1) != 0>
__device__ __forceinline__ uint4 ld_vec(const uint4* p) {
    if (NT) {
        typedef uint32_t v4u __attribute__((ext_vector_type(4)));
        const v4u v = __builtin_nontemporal_load((const __attribute__((address_space(1))) v4u*)(const void*)p);
        return make_uint4(v[0], v[1], v[2], v[3]);
    }
    return *p;
}

template <bool BF16>
__device__ __forceinline__ float load_x(const void* x, int64_t i) {
    if (BF16) return bf16_to_f32(static_cast<const uint16_t*>(x)[i]);
    return static_cast<const float*>(x)[i];
}

__device__ __forceinline__ float round_to(float v, bool bf16) { return bf16 ? bf16_to_f32(f32_to_bf16(v)) : v; }

// Exact-arithmetic (slow-path) quantize of one element: fp8.py:49.
template <int FMT, bool BF16>
__device__ __forceinline__ uint32_t quant_sw(float xv, float s_down) {
    return fp8_from_f32_sw<FMT>(round_to(xv * s_down, BF16));
}

// Exact-arithmetic (slow-path) dequantize of one code: fp8.py:53.
template <int FMT, bool BF16OUT>
__device__ __forceinline__ float dequant_sw(uint32_t c, float s_up) {
    float v = round_to(fp8_to_f32_sw<FMT>(c), BF16OUT);
    return round_to(v * s_up, BF16OUT);
}

// A dequantized value from the instruction path as its output dtype's bits.
// In that path the value is exact in bf16, so truncation is the rounding.
__device__ __forceinline__ uint32_t fast_bf16_bits(float v) { return __float_as_uint(v) >> 16; }

struct RowScale {
    int k;
    bool fast;
    float s_down;   // 2^-k in the input dtype
    float s_up;     // 2^k in the output dtype
};

template <int FMT>
__device__ __forceinline__ RowScale row_scale(uint32_t abits, bool bf16_in, bool bf16_out) {
    RowScale r;
    r.k = scale_exp_from_amax<FMT>(abits);
    r.fast = abits < 0x7F800000u && r.k >= -kFastK && r.k <= kFastK;
    if (r.fast) {
        r.s_down = __uint_as_float((uint32_t)(127 - r.k) << 23);
        r.s_up = __uint_as_float((uint32_t)(127 + r.k) << 23);
    } else {
        r.s_down = pow2_dtype(-r.k, bf16_in);
        r.s_up = pow2_dtype(r.k, bf16_out);
    }
    return r;
}

// |x| bits of 8 bf16 packed in a uint4 / 4 fp32 in a uint4, maxed into m.
template <bool BF16>
__device__ __forceinline__ uint32_t vec_absmax(const uint4& w, uint32_t m) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (BF16) {
            const uint32_t lo = ws[j] & 0x7FFFu, hi = (ws[j] >> 16) & 0x7FFFu;
            m = max(m, max(lo, hi));
        } else {
            m = max(m, ws[j] & 0x7FFFFFFFu);
        }
    }
    return m;
}

template <bool BF16>
__device__ __forceinline__ uint32_t to_f32_bits(uint32_t amax) {
    return BF16 ? amax << 16 : amax;
}

// Unpack a uint4 into 8 (bf16) or 4 (fp32) floats.
template <bool BF16>
__device__ __forceinline__ void unpack(const uint4& w, float* f) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (BF16) {
            f[2 * j] = bf16_to_f32(ws[j] & 0xFFFFu);
            f[2 * j + 1] = bf16_to_f32(ws[j] >> 16);
        } else {
            f[j] = __uint_as_float(ws[j]);
        }
    }
}

// Quantize one 16-byte input vector (8 bf16 or 4 fp32) of an instruction-path
// row into codes packed in words[0..1] (bf16: 8 codes) or words[0] (fp32: 4
// codes); with `out`, also write the dequantized values in the input dtype at
// out_vec (exact there, so bf16 truncation is the rounding).
template <int FMT, bool BF16>
__device__ __forceinline__ void quant_vec_fast(const uint4& w, const RowScale& rs, uint32_t* words, void* out_vec) {
    if (BF16) {
        // bf16 words straight into the scaled conversions (scale 2^k), no
        // widening or product; no NaN code arises on this path, so the
        // scaled decode gives the output bits too
        words[0] = cvt_scaled_pk_fp8_bf16<FMT, true>(w.y, rs.s_up, cvt_scaled_pk_fp8_bf16<FMT, false>(w.x, rs.s_up, 0u));
        words[1] = cvt_scaled_pk_fp8_bf16<FMT, true>(w.w, rs.s_up, cvt_scaled_pk_fp8_bf16<FMT, false>(w.z, rs.s_up, 0u));
        if (out_vec)
            st_vec(out_vec, make_uint4(cvt_scaled_pk_bf16<FMT, false>(words[0], rs.s_up),
                                       cvt_scaled_pk_bf16<FMT, true>(words[0], rs.s_up),
                                       cvt_scaled_pk_bf16<FMT, false>(words[1], rs.s_up),
                                       cvt_scaled_pk_bf16<FMT, true>(words[1], rs.s_up)));
        return;
    }
    constexpr int EPV = BF16 ? 8 : 4;
    float f[EPV];
    unpack<BF16>(w, f);
#pragma unroll
    for (int j = 0; j < EPV; j += 4) {
        uint32_t pk = cvt_pk_fp8<FMT, false>(f[j] * rs.s_down, f[j + 1] * rs.s_down, 0u);
        pk = cvt_pk_fp8<FMT, true>(f[j + 2] * rs.s_down, f[j + 3] * rs.s_down, pk);
        words[j / 4] = pk;
    }
    if (out_vec) {
        float o[EPV];
#pragma unroll
        for (int j = 0; j < EPV; j += 4) {
            float a, b, c, d;
            cvt_pk_f32<FMT, false>(words[j / 4], a, b);
            cvt_pk_f32<FMT, true>(words[j / 4], c, d);
            o[j] = a * rs.s_up;
            o[j + 1] = b * rs.s_up;
            o[j + 2] = c * rs.s_up;
            o[j + 3] = d * rs.s_up;
        }
        uint4 r;
        if (BF16) {
            uint32_t b[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) b[j] = fast_bf16_bits(o[j]);
            r = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
        } else {
            r = make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                           __float_as_uint(o[3]));
        }
        st_vec(out_vec, r);
    }
}

// Elements [e0, e1) of a row at `base` through the bit-level restatement of
// torch's arithmetic: the rows the instruction path does not cover (|k| >
// 110 or a non-finite |x|max), one element per lane per step.
template <int FMT, bool BF16>
__device__ __forceinline__ void quant_slow(const void* x, int64_t base, int64_t e0, int64_t e1, const RowScale& rs,
                                        uint8_t* q, void* out, int lane) {
    for (int64_t e = e0 + lane; e < e1; e += kWave) {
        const float xv = load_x<BF16>(x, base + e);
        const uint32_t c = quant_sw<FMT, BF16>(xv, rs.s_down);
        if (q) q[base + e] = (uint8_t)c;
        if (out) {
            const float o = dequant_sw<FMT, BF16>(c, rs.s_up);
            if (BF16) static_cast<uint16_t*>(out)[base + e] = (uint16_t)f32_to_bf16(o);
            else static_cast<float*>(out)[base + e] = o;
        }
    }
}

// ------------------------------------------------- wave-per-row (registers)

template <int FMT, bool BF16, int VPL>
__global__ __launch_bounds__(kQBlock) void quant_rows_kernel(const void* __restrict__ x, int64_t rows, int64_t cols,
                                                             uint8_t* __restrict__ q, int32_t* __restrict__ k,
                                                             void* __restrict__ out) {
    constexpr int EPV = BF16 ? 8 : 4;
    constexpr int ESZ = BF16 ? 2 : 4;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    if (row >= rows) return;  // whole waves leave; the kernel has no block barrier
    const int64_t nvec = cols / EPV;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * cols * ESZ);
    // the row's loads go out in batches of QB vectors per lane, each batch's
    // loads back to back: lanes past the row's end load its last vector (in
    // bounds) and zero it afterwards
    constexpr int QB = (ELY_Q_BATCH <= 0 || ELY_Q_BATCH > VPL) ? VPL : ELY_Q_BATCH;
    uint4 buf[VPL];
    uint32_t amax = 0;
#pragma unroll
    for (int j0 = 0; j0 < VPL; j0 += QB) {
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            buf[j] = ld_vec(xr + (vi < nvec ? vi : nvec - 1));
        }
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nvec) buf[j] = make_uint4(0u, 0u, 0u, 0u);
            amax = vec_absmax<BF16>(buf[j], amax);
        }
        // the next batch is issued only once this one has arrived
        if (QB < VPL) __builtin_amdgcn_sched_barrier(0);
    }
    amax = wave_max_u32(amax);
    const RowScale rs = row_scale<FMT>(to_f32_bits<BF16>(amax), BF16, BF16);
    if (lane == 0 && k) k[row] = rs.k;
    if (!rs.fast) return quant_slow<FMT, BF16>(x, row * cols, 0, cols, rs, q, out, lane);
    uint8_t* qr = q ? q + row * cols : nullptr;
    char* orow = out ? static_cast<char*>(out) + row * cols * ESZ : nullptr;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int64_t vi = lane + (int64_t)kWave * j;
        if (vi < nvec) {
            uint32_t words[2];
            quant_vec_fast<FMT, BF16>(buf[j], rs, words, orow ? orow + vi * 16 : nullptr);
            if (qr) {
                if (BF16) st_vec2(qr + vi * 8, make_uint2(words[0], words[1]));
                else st_u32(qr + vi * 4, words[0]);
            }
        }
    }
}

// Long rows: the block's waves share one row, each wave a contiguous run of
// kWave * VPLW vectors; the waves' |x|max meet in LDS across one barrier.
// The host launches exactly one block per row, so every wave of a block
// reaches the barrier.
template <int FMT, bool BF16, int VPLW>
__global__ __launch_bounds__(kRowBlock) void quant_block_row_kernel(const void* __restrict__ x, int64_t cols,
                                                                  uint8_t* __restrict__ q, int32_t* __restrict__ k,
                                                                  void* __restrict__ out) {
    constexpr int EPV = BF16 ? 8 : 4;
    constexpr int ESZ = BF16 ? 2 : 4;
    constexpr int QB = (ELY_Q_BATCH <= 0 || ELY_Q_BATCH > VPLW) ? VPLW : ELY_Q_BATCH;
    __shared__ uint32_t wmax[kRowWaves];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = wave_uniform(threadIdx.x / kWave);
    const int64_t row = blockIdx.x;
    const int64_t nvec = cols / EPV;
    const int64_t v0 = (int64_t)w * kWave * VPLW;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * cols * ESZ);
    uint4 buf[VPLW];
    uint32_t amax = 0;
#pragma unroll
    for (int j0 = 0; j0 < VPLW; j0 += QB) {
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPLW; ++j) {
            const int64_t vi = v0 + lane + (int64_t)kWave * j;
            buf[j] = ld_vec(xr + (vi < nvec ? vi : nvec - 1));
        }
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPLW; ++j) {
            const int64_t vi = v0 + lane + (int64_t)kWave * j;
            if (vi >= nvec) buf[j] = make_uint4(0u, 0u, 0u, 0u);
            amax = vec_absmax<BF16>(buf[j], amax);
        }
        if (QB < VPLW) __builtin_amdgcn_sched_barrier(0);
    }
    amax = wave_max_u32(amax);
    if (lane == 0) wmax[w] = amax;
    __syncthreads();
    amax = wmax[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; ++i) amax = max(amax, wmax[i]);
    const RowScale rs = row_scale<FMT>(to_f32_bits<BF16>(amax), BF16, BF16);
    if (threadIdx.x == 0 && k) k[row] = rs.k;
    if (!rs.fast) {
        const int64_t e0 = min(v0 * EPV, cols), e1 = min((v0 + (int64_t)kWave * VPLW) * EPV, cols);
        return quant_slow<FMT, BF16>(x, row * cols, e0, e1, rs, q, out, lane);
    }
    uint8_t* qr = q ? q + row * cols : nullptr;
    char* orow = out ? static_cast<char*>(out) + row * cols * ESZ : nullptr;
#pragma unroll
    for (int j = 0; j < VPLW; ++j) {
        const int64_t vi = v0 + lane + (int64_t)kWave * j;
        if (vi < nvec) {
            uint32_t words[2];
            quant_vec_fast<FMT, BF16>(buf[j], rs, words, orow ? orow + vi * 16 : nullptr);
            if (qr) {
                if (BF16) st_vec2(qr + vi * 8, make_uint2(words[0], words[1]));
                else st_u32(qr + vi * 4, words[0]);
            }
        }
    }
}

// ------------------------------------------------------- split long rows

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t value) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = value;
}

// Long rows (and per-tensor scaling, one row) go through segments of
// kSegElems elements.  The row's |x|max is reduced without atomics: wave
// (r, j) of the rowmax_partial_kernel folds segments j, j + wpr, ... of row r
// into partial[r * wpr + j]; rowmax_reduce_kernel folds a row's wpr partials
// (wpr == 1: the partials are the row maxima).  Values are |x| bit patterns
// (fp32 bits for fp32 input, bf16 bits for bf16), so max is an integer max.
constexpr int64_t kSplitWaves = ELY_SPLIT_WAVES;  // waves of the partial-max launch (at most)

static int64_t split_wpr(int64_t rows, int64_t segs) {
    return std::max<int64_t>(1, std::min<int64_t>(segs, kSplitWaves / std::max<int64_t>(rows, 1)));
}

// Vectors of one segment a lane holds: 2048 bf16 = 256 x 16 B -> 4 per lane.
template <bool BF16>
struct Seg {
    static constexpr int EPV = BF16 ? 8 : 4;
    static constexpr int VPL = (int)(kSegElems / EPV / kWave);
};

// |x|max bits of elements [e0, e1) of row `row` (e1 - e0 <= kSegElems).
template <bool BF16, bool NT>
__device__ __forceinline__ uint32_t seg_absmax(const void* x, int64_t row, int64_t cols, int64_t e0, int64_t e1,
                                               int vec, int lane) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    uint32_t amax = 0;
    if (vec) {
        const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + (row * cols + e0) * ESZ);
        const int64_t nv = (e1 - e0) / EPV;
        uint4 buf[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            buf[j] = ld_vec<NT>(xr + (vi < nv ? vi : nv - 1));
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j)
            if (lane + (int64_t)kWave * j < nv) amax = vec_absmax<BF16>(buf[j], amax);
    } else {
        for (int64_t e = e0 + lane; e < e1; e += kWave) {
            uint32_t b = BF16 ? (uint32_t)static_cast<const uint16_t*>(x)[row * cols + e] & 0x7FFFu
                              : __float_as_uint(static_cast<const float*>(x)[row * cols + e]) & 0x7FFFFFFFu;
            amax = max(amax, b);
        }
    }
    return amax;
}

template <bool BF16>
__global__ __launch_bounds__(kQBlock) void rowmax_partial_kernel(const void* __restrict__ x, int64_t rows, int64_t cols,
                                                                 int64_t segs, int64_t wpr, int vec, int64_t cached,
                                                                 uint32_t* __restrict__ partial) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    if (gw >= rows * wpr) return;
    const int64_t row = gw / wpr, j = gw % wpr;
    uint32_t amax = 0;
    // a row's last `cached` segments are read last, with plain loads; two
    // loops in sequence keep the two kinds of loads apart
    const int64_t cut = segs - cached;
    int64_t seg = j;
    for (; seg < cut; seg += wpr) {
        const int64_t e0 = seg * kSegElems;
        amax = max(amax, seg_absmax<BF16, (ELY_FP8_NT & 1) != 0>(x, row, cols, e0, min(e0 + kSegElems, cols), vec, lane));
    }
    for (; seg < segs; seg += wpr) {
        const int64_t e0 = seg * kSegElems;
        amax = max(amax, seg_absmax<BF16, false>(x, row, cols, e0, min(e0 + kSegElems, cols), vec, lane));
    }
    amax = wave_max_u32(amax);
    if (lane == 0) partial[gw] = amax;
}

__global__ __launch_bounds__(kRowBlock) void rowmax_reduce_kernel(const uint32_t* __restrict__ partial, int64_t rows,
                                                                int64_t wpr, uint32_t* __restrict__ rowmax) {
    __shared__ uint32_t red[kRowWaves];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        uint32_t m = 0;
        for (int64_t i = threadIdx.x; i < wpr; i += kRowBlock) m = max(m, partial[r * wpr + i]);
        m = wave_max_u32(m);
        if (lane == 0) red[w] = m;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t t = red[0];
            for (int k = 1; k < kRowWaves; ++k) t = max(t, red[k]);
            rowmax[r] = t;
        }
        __syncthreads();
    }
}

// Segment `seg` of row `row` converted at the row's scale rs (the split
// path's convert launch and the hint path's fixup).
template <int FMT, bool BF16>
__device__ __forceinline__ void quant_segment(const void* x, int64_t row, int64_t cols, int64_t seg, int vec,
                                              const RowScale& rs, uint8_t* q, void* out, int lane) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    const int64_t e0 = seg * kSegElems, e1 = min(e0 + kSegElems, cols);
    const int64_t base = row * cols;
    if (vec && rs.fast) {
        const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + (base + e0) * ESZ);
        const int64_t nv = (e1 - e0) / EPV;
        constexpr int SB = (ELY_SPLIT_BATCH <= 0 || ELY_SPLIT_BATCH > VPL) ? VPL : ELY_SPLIT_BATCH;
        uint4 buf[VPL];
#pragma unroll
        for (int j0 = 0; j0 < VPL; j0 += SB) {
#pragma unroll
            for (int j = j0; j < j0 + SB && j < VPL; ++j) {
                const int64_t vi = lane + (int64_t)kWave * j;
                buf[j] = ld_vec(xr + (vi < nv ? vi : nv - 1));
            }
#pragma unroll
            for (int j = j0; j < j0 + SB && j < VPL; ++j) {
                const int64_t vi = lane + (int64_t)kWave * j;
                if (vi >= nv) continue;
                uint32_t words[2];
                const int64_t e = e0 + vi * EPV;
                quant_vec_fast<FMT, BF16>(buf[j], rs, words, out ? static_cast<char*>(out) + (base + e) * ESZ : nullptr);
                if (q) {
                    if (BF16) st_vec2(q + base + e, make_uint2(words[0], words[1]));
                    else st_u32(q + base + e, words[0]);
                }
            }
            if (SB < VPL) __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        quant_slow<FMT, BF16>(x, base, e0, e1, rs, q, out, lane);
    }
}

template <int FMT, bool BF16>
__global__ __launch_bounds__(kQBlock) void quant_split_kernel(const void* __restrict__ x, int64_t rows, int64_t cols,
                                                              int64_t segs, int vec,
                                                              const uint32_t* __restrict__ rowmax,
                                                              uint8_t* __restrict__ q, int32_t* __restrict__ k,
                                                              void* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t row = gw / segs, seg = gw % segs;
    if (row >= rows) return;
    const RowScale rs = row_scale<FMT>(to_f32_bits<BF16>(rowmax[row]), BF16, BF16);
    if (seg == 0 && lane == 0 && k) k[row] = rs.k;
    quant_segment<FMT, BF16>(x, row, cols, seg, vec, rs, q, out, lane);
}

// ------------------------------------------------- per-tensor, with a hint
//
// Per-tensor scaling needs the whole tensor's |x|max before the first code,
// so the split path reads x twice.  Given the exponent a caller expects (the
// previous step's, say), one pass does both: wave w reads segment w once,
// writes its |x|max to partial[w] and its codes at the hinted scale.  A
// small launch folds the partials to kHintBlocks maxima, and a capped fixup
// launch, whose every wave folds those to the tensor's k, writes k (and
// whether it equals the hint) and exits when it does; on a miss its waves
// convert every segment again at the true scale.  The codes depend on k
// alone, so a hit's codes are the split path's, byte for byte.
constexpr int kHintBlocks = 256;         // maxima the reduce launch leaves (4 per lane of a fixup wave)
#ifndef ELY_HINT_FIXUP_WPC
// fixup grid cap, waves per compute unit.  C4 per-tensor (1.07 GB of bf16):
// a hit 6.25-6.32 TB/s with 8 or 32, 6.1 with 128; a miss 2.5 TB/s with 8,
// 3.1 with 32 or 128
#define ELY_HINT_FIXUP_WPC 32
#endif
constexpr int kHintFixupWavesPerCU = ELY_HINT_FIXUP_WPC;
#ifndef ELY_GUESS_MIN_MB
// per-tensor rows of at least this many MiB of x take the sampled guess.
// Back to back on N(0, 1) bf16 (a right guess), per call: 8 MiB 16.4-18.1 us
// against 12.6-16.5 on the split path, 32 MiB 21.4-21.9 against 17.7-18.8,
// 64 MiB 29.3-29.9 against 28.8-29.5, 128 MiB 45 against 54, 512 MiB 139
// against 201: the guess's four small launches cost what its saved read wins
// back near 64 MiB
#define ELY_GUESS_MIN_MB 64
#endif
#ifndef ELY_GUESS_STRIDE
#define ELY_GUESS_STRIDE 61  // the guess samples every this-many-th segment (a prime)
#endif
constexpr int64_t kGuessStride = ELY_GUESS_STRIDE;

// The hint: k_hint, or *k_hint_dev when that is given (read here, before
// the fixup launch writes k, which may be the same word); with hint_is_amax,
// *k_hint_dev holds fp32 |x|max bits (a sample's, guess_amax_kernel) and
// the hint is their exponent.  Wave 0 keeps the hint it read in hint_copy
// for the fixup.  A hint outside the instruction path's range converts
// nothing here: the call is then a miss.
template <int FMT, bool BF16>
__global__ __launch_bounds__(kQBlock) void quant_hint_kernel(const void* __restrict__ x, int64_t n, int64_t segs,
                                                             int32_t k_hint, const int32_t* k_hint_dev,
                                                             int32_t hint_is_amax, uint8_t* __restrict__ q,
                                                             void* __restrict__ out, uint32_t* __restrict__ partial,
                                                             int32_t* __restrict__ hint_copy) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t seg = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    if (seg >= segs) return;
    int32_t hint = k_hint;
    if (k_hint_dev) {
        hint = __builtin_amdgcn_readfirstlane(*k_hint_dev);
        if (hint_is_amax) hint = scale_exp_from_amax<FMT>((uint32_t)hint);
    }
    if (seg == 0 && lane == 0) hint_copy[0] = hint;
    const bool convert = hint >= -kFastK && hint <= kFastK;
    RowScale hs;
    hs.k = hint;
    hs.fast = true;
    hs.s_down = __uint_as_float((uint32_t)(127 - hint) << 23);
    hs.s_up = __uint_as_float((uint32_t)(127 + hint) << 23);
    const int64_t e0 = seg * kSegElems;
    const int64_t nv = (min(e0 + kSegElems, n) - e0) / EPV;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + e0 * ESZ);
    uint4 buf[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int64_t vi = lane + (int64_t)kWave * j;
        buf[j] = ld_vec(xr + (vi < nv ? vi : nv - 1));
    }
    uint32_t amax = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int64_t vi = lane + (int64_t)kWave * j;
        if (vi >= nv) continue;
        amax = vec_absmax<BF16>(buf[j], amax);
        if (!convert) continue;
        uint32_t words[2];
        const int64_t e = e0 + vi * EPV;
        quant_vec_fast<FMT, BF16>(buf[j], hs, words, out ? static_cast<char*>(out) + e * ESZ : nullptr);
        if (q) {
            if (BF16) st_vec2(q + e, make_uint2(words[0], words[1]));
            else st_u32(q + e, words[0]);
        }
    }
    amax = wave_max_u32(amax);
    if (lane == 0) partial[seg] = amax;
}

// A per-tensor row's exponent guessed from a sample: wave w reads segment
// w * stride (stride a prime, so that the sample does not fall in step with
// a row length or an outlier channel) and writes its |x|max, as fp32 bits,
// to partial[w].  The vector form only (n a whole number of 16-byte
// vectors, aligned x).
template <bool BF16>
__global__ __launch_bounds__(kQBlock) void guess_amax_kernel(const void* __restrict__ x, int64_t n, int64_t stride,
                                                             int64_t samples, uint32_t* __restrict__ partial) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    if (w >= samples) return;
    const int64_t e0 = w * stride * kSegElems;
    const int64_t nv = (min(e0 + kSegElems, n) - e0) / EPV;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + e0 * ESZ);
    uint4 buf[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int64_t vi = lane + (int64_t)kWave * j;
        buf[j] = ld_vec(xr + (vi < nv ? vi : nv - 1));
    }
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
        if (lane + (int64_t)kWave * j < nv) m = vec_absmax<BF16>(buf[j], m);
    m = wave_max_u32(m);
    if (lane == 0) partial[w] = to_f32_bits<BF16>(m);
}

// out[0] = max of partial[0, count): one block (an integer max, order-free;
// one word per sample, so no same-address atomics serialize the guess).
constexpr int kSampleMaxBlock = 1024;
__global__ __launch_bounds__(kSampleMaxBlock) void sample_max_kernel(const uint32_t* __restrict__ partial,
                                                                    int64_t count, uint32_t* __restrict__ out) {
    __shared__ uint32_t red[kSampleMaxBlock / kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    uint32_t m = 0;
#pragma unroll 4
    for (int64_t i = threadIdx.x; i < count; i += kSampleMaxBlock) m = max(m, partial[i]);
    m = wave_max_u32(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = red[0];
        for (int j = 1; j < kSampleMaxBlock / kWave; ++j) r = max(r, red[j]);
        out[0] = r;
    }
}

// partial[0, segs) -> out[b] for b < kHintBlocks (block b folds a contiguous
// share; integer max, so the order does not matter).
__global__ __launch_bounds__(kRowBlock) void hint_reduce_kernel(const uint32_t* __restrict__ partial, int64_t segs,
                                                              uint32_t* __restrict__ out) {
    __shared__ uint32_t red[kRowWaves];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int64_t per = (segs + kHintBlocks - 1) / kHintBlocks;
    const int64_t i0 = (int64_t)blockIdx.x * per, i1 = min(i0 + per, segs);
    uint32_t m = 0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += kRowBlock) m = max(m, partial[i]);
    m = wave_max_u32(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = red[0];
        for (int j = 1; j < kRowWaves; ++j) t = max(t, red[j]);
        out[blockIdx.x] = t;
    }
}

template <int FMT, bool BF16>
__global__ __launch_bounds__(kQBlock) void quant_hint_fixup_kernel(const void* __restrict__ x, int64_t n, int64_t segs,
                                                                   int vec, const int32_t* __restrict__ hint_copy,
                                                                   const uint32_t* __restrict__ block_max,
                                                                   uint8_t* __restrict__ q, int32_t* __restrict__ k,
                                                                   void* __restrict__ out, int32_t* __restrict__ hit) {
    static_assert(kHintBlocks == 4 * kWave, "a fixup lane folds four block maxima");
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t waves = (int64_t)gridDim.x * kWavesPerBlock;
    uint32_t m = max(max(block_max[lane], block_max[lane + kWave]), max(block_max[lane + 2 * kWave], block_max[lane + 3 * kWave]));
    m = wave_max_u32(m);
    const RowScale rs = row_scale<FMT>(to_f32_bits<BF16>(m), BF16, BF16);
    const int32_t k_hint = hint_copy[0];
    const bool same = rs.fast && rs.k == k_hint && k_hint >= -kFastK && k_hint <= kFastK;
    if (gw == 0 && lane == 0) {
        k[0] = rs.k;
        if (hit) hit[0] = same ? 1 : 0;
    }
    if (same) return;
    for (int64_t seg = gw; seg < segs; seg += waves) quant_segment<FMT, BF16>(x, 0, n, seg, vec, rs, q, out, lane);
}

// -------------------------------------------------------------- dequantize

// Codes in rows whose length is a multiple of 16 (and 16-byte aligned
// buffers) are dequantized as one flat array: wave w takes codes
// [S w, S w + S) (S = kDeqSegCodes), which may span rows.  A lane takes CPL
// codes per step (8 for bf16 output, 4 for fp32), so that each store
// instruction of a wave writes one contiguous 1 KB run; every lane issues
// its loads (all of them, or batches of ELY_DEQ_BATCH) before the first is
// used, and each CPL-code vector lies in one row.  Rows at least a segment
// wide give a segment at most two exponents, read once per wave (C1 back to
// back: 5.89-5.94 TB/s against 5.76-5.80 with a division and an exponent
// load per vector); narrower rows look theirs up per vector.  Short
// segments (many short-lived waves) measured fastest.
template <int FMT, bool BF16OUT, bool IDX32>
__global__ __launch_bounds__(kQBlock) void dequant_flat_kernel(const uint8_t* __restrict__ q,
                                                               const int32_t* __restrict__ k, int64_t n,
                                                               int64_t cols, void* __restrict__ out) {
    constexpr int CPL = BF16OUT ? 8 : 4;
    constexpr int VPL = (int)(kDeqSegCodes / CPL / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t e0 = gw * kDeqSegCodes;
    if (e0 >= n) return;
    const int64_t nv = min(kDeqSegCodes, n - e0) / CPL;
    constexpr int DB = (ELY_DEQ_BATCH <= 0 || ELY_DEQ_BATCH > VPL) ? VPL : ELY_DEQ_BATCH;
    // rows at least a segment wide: the segment meets at most two rows, the
    // one holding code e0 and, from code `split` on, the next; the wave reads
    // their two exponents once (uniform loads) instead of one lookup per vector
    const bool two_rows = cols >= kDeqSegCodes;
    int64_t split = 0;
    int k_lo = 0, k_hi = 0;
    uint32_t buf[VPL][CPL / 4];
#pragma unroll
    for (int j0 = 0; j0 < VPL; j0 += DB) {
#pragma unroll
        for (int j = j0; j < j0 + DB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            const uint8_t* src = q + e0 + (vi < nv ? vi : nv - 1) * CPL;
            if (CPL == 8) {
                const uint2 w = ld_vec2(src);
                buf[j][0] = w.x;
                buf[j][CPL / 4 - 1] = w.y;
            } else {
                buf[j][0] = ld_u32(src);
            }
        }
        // the exponents are read once the first codes are requested: a wait
        // for these loads ahead of the code loads would hold those back
        if (j0 == 0 && two_rows) {
            const int64_t row0 = IDX32 ? (int64_t)((uint32_t)e0 / (uint32_t)cols) : e0 / cols;
            split = (row0 + 1) * cols;
            k_lo = k[row0];
            k_hi = k[split < n ? row0 + 1 : row0];
        }
#pragma unroll
        for (int j = j0; j < j0 + DB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nv) continue;
            const int64_t e = e0 + vi * CPL;
            int kk;
            if (two_rows) {
                kk = e < split ? k_lo : k_hi;
            } else {
                const int64_t row = IDX32 ? (int64_t)((uint32_t)e / (uint32_t)cols) : e / cols;
                kk = k[row];
            }
            if (kk >= -kFastK && kk <= kFastK) {
                const float s_up = __uint_as_float((uint32_t)(127 + kk) << 23);
                if (BF16OUT && !(nan_code_bits<FMT>(buf[j][0]) | nan_code_bits<FMT>(buf[j][CPL / 4 - 1]))) {
                    // no NaN code among the eight: the scaled decode writes the bf16 bits
                    st_vec(static_cast<uint16_t*>(out) + e,
                           make_uint4(cvt_scaled_pk_bf16<FMT, false>(buf[j][0], s_up),
                                      cvt_scaled_pk_bf16<FMT, true>(buf[j][0], s_up),
                                      cvt_scaled_pk_bf16<FMT, false>(buf[j][CPL / 4 - 1], s_up),
                                      cvt_scaled_pk_bf16<FMT, true>(buf[j][CPL / 4 - 1], s_up)));
                    continue;
                }
                float o[CPL];
#pragma unroll
                for (int h = 0; h < CPL / 4; ++h) {
                    float a, b, c, d;
                    cvt_pk_f32<FMT, false>(buf[j][h], a, b);
                    cvt_pk_f32<FMT, true>(buf[j][h], c, d);
                    o[4 * h] = a * s_up;
                    o[4 * h + 1] = b * s_up;
                    o[4 * h + 2] = c * s_up;
                    o[4 * h + 3] = d * s_up;
                }
                if (BF16OUT) {
                    uint32_t b[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        // an fp8 NaN is the only non-exact value the instruction path sees
                        const float v = o[t];
                        b[t] = v != v ? 0x7FC0u : fast_bf16_bits(v);
                    }
                    st_vec(static_cast<uint16_t*>(out) + e, make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16),
                                                                       b[4] | (b[5] << 16), b[6] | (b[7] << 16)));
                } else {
                    st_vec(static_cast<float*>(out) + e, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]),
                                                                    __float_as_uint(o[2]), __float_as_uint(o[3])));
                }
            } else {
                // the restatement of torch's arithmetic (|k| > 110), code by code
                const float s_up = pow2_dtype(kk, BF16OUT);
#pragma unroll 1
                for (int t = 0; t < CPL; ++t) {
                    const float o = dequant_sw<FMT, BF16OUT>((buf[j][t / 4] >> (8 * (t % 4))) & 0xFFu, s_up);
                    if (BF16OUT) static_cast<uint16_t*>(out)[e + t] = (uint16_t)f32_to_bf16(o);
                    else static_cast<float*>(out)[e + t] = o;
                }
            }
        }
        // the next batch is issued only once this one has been stored
        if (DB < VPL) __builtin_amdgcn_sched_barrier(0);
    }
}

// Any other shape: one wave per (row, kDeqSegCodes-code segment), element by element.
template <int FMT, bool BF16OUT>
__global__ __launch_bounds__(kQBlock) void dequant_any_kernel(const uint8_t* __restrict__ q,
                                                              const int32_t* __restrict__ k, int64_t rows,
                                                              int64_t cols, int64_t segs, void* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t row = gw / segs, seg = gw % segs;
    if (row >= rows) return;
    const int kk = k[row];
    const bool fast = kk >= -kFastK && kk <= kFastK;
    const float s_up = fast ? __uint_as_float((uint32_t)(127 + kk) << 23) : pow2_dtype(kk, BF16OUT);
    const int64_t e0 = seg * kDeqSegCodes, e1 = min(e0 + kDeqSegCodes, cols);
    const int64_t base = row * cols;
    for (int64_t e = e0 + lane; e < e1; e += kWave) {
        const float o = dequant_sw<FMT, BF16OUT>(q[base + e], s_up);
        if (BF16OUT) static_cast<uint16_t*>(out)[base + e] = (uint16_t)f32_to_bf16(o);
        else static_cast<float*>(out)[base + e] = o;
    }
}

// ------------------------------------------------------- recover_exp / wire

// Bit i of the candidate mask stands for offset kDeltas[i] (fp8.py:25).
__constant__ int kDeltas[5] = {0, -1, 1, -2, 2};

// Is v (a value of the tensor's dtype) exactly fp8(v * 2^-c) * 2^c in that
// dtype's arithmetic (fp8.py:85-86)?  `fast` rows use the conversion
// instructions: every candidate's 2^+-c is a normal power of two there and
// every product exact, so the test is just whether v * 2^-c lies on the fp8
// grid; non-finite elements always take the restatement.
template <int FMT, bool BF16>
__device__ __forceinline__ bool exact_at(float v, int c, bool fast) {
    if (fast && __builtin_isfinite(v)) {
        const float y = v * __uint_as_float((uint32_t)(127 - c) << 23);
        const uint32_t code = cvt_pk_fp8<FMT, false>(y, 0.0f, 0u) & 0xFFu;
        float back, unused;
        cvt_pk_f32<FMT, false>(code, back, unused);
        return back * __uint_as_float((uint32_t)(127 + c) << 23) == v;
    }
    const float y = round_to(v * pow2_dtype(-c, BF16), BF16);
    const uint32_t code = fp8_from_f32_sw<FMT>(y);
    const float back = round_to(round_to(fp8_to_f32_sw<FMT>(code), BF16) * pow2_dtype(c, BF16), BF16);
    return back == v;
}

__device__ __forceinline__ uint32_t wave_and_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v &= (uint32_t)__shfl_xor((int)v, o, kWave);
    return v;
}

// The segment's elements, one callback per element (lanes past the end make
// none): vectorized loads, all issued before the first is used, when `vec`
// (16-byte aligned rows whose length is a multiple of the vector), element
// loads otherwise.
template <bool BF16, class F>
__device__ __forceinline__ void for_seg_elems(const void* t, int64_t row, int64_t cols, int64_t e0, int64_t e1,
                                              int vec, int lane, F f) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    if (vec) {
        const uint4* tr = reinterpret_cast<const uint4*>(static_cast<const char*>(t) + (row * cols + e0) * ESZ);
        const int64_t nv = (e1 - e0) / EPV;
        uint4 buf[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            buf[j] = ld_vec(tr + (vi < nv ? vi : nv - 1));
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (lane + (int64_t)kWave * j >= nv) continue;
            float v[EPV];
            unpack<BF16>(buf[j], v);
#pragma unroll
            for (int e = 0; e < EPV; ++e) f(v[e]);
        }
    } else {
        for (int64_t e = e0 + lane; e < e1; e += kWave) f(load_x<BF16>(t, row * cols + e));
    }
}

// Per (row, segment): the exactness of the candidates over the segment's
// elements, ANDed into rowmask[row] (all candidates set beforehand).  PHASE
// 0 tests the base candidate only; PHASE 1 runs only for rows whose base
// candidate failed somewhere and tests the other four, so a row the base
// exponent recovers (the common case) costs one test per element.
template <int FMT, bool BF16, int PHASE>
__global__ __launch_bounds__(kQBlock) void recover_mask_kernel(const void* __restrict__ t, int64_t rows, int64_t cols,
                                                               int64_t segs, int vec,
                                                               const uint32_t* __restrict__ rowmax,
                                                               uint32_t* __restrict__ rowmask) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t row = gw / segs, seg = gw % segs;
    if (row >= rows) return;
    if (PHASE == 1 && (rowmask[row] & 1u)) return;  // the base candidate holds for the whole row
    const int base = scale_exp_from_amax<FMT>(to_f32_bits<BF16>(rowmax[row]));
    const bool fast = base - 2 >= -kFastK && base + 2 <= kFastK;
    const int64_t e0 = seg * kSegElems, e1 = min(e0 + kSegElems, cols);
    uint32_t mask = PHASE == 0 ? 0x1u : 0x1Eu;
    for_seg_elems<BF16>(t, row, cols, e0, e1, vec, lane, [&](float v) {
#pragma unroll
        for (int i = (PHASE == 0 ? 0 : 1); i < (PHASE == 0 ? 1 : 5); ++i)
            if ((mask >> i) & 1u)
                if (!exact_at<FMT, BF16>(v, base + kDeltas[i], fast)) mask &= ~(1u << i);
    });
    mask = wave_and_u32(mask);
    const uint32_t keep = PHASE == 0 ? ~0x1u : ~0x1Eu;  // the bits this phase does not test
    if (lane == 0 && (mask | keep) != 0xFFFFFFFFu) atomicAnd(rowmask + row, mask | keep);
}

// k = base + the first exact offset; a row with none counts as bad and keeps
// the last candidate, as the reference's `best` does (fp8.py:82-93).
template <int FMT, bool BF16>
__global__ void recover_final_kernel(int64_t rows, const uint32_t* __restrict__ rowmax,
                                     const uint32_t* __restrict__ rowmask, int32_t* __restrict__ k,
                                     unsigned long long* __restrict__ bad) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
        const int base = scale_exp_from_amax<FMT>(to_f32_bits<BF16>(rowmax[r]));
        const uint32_t m = rowmask[r];
        int kk = base + 2;
        if (m == 0u) {
            atomicAdd(bad, 1ull);
        } else {
            kk = base + kDeltas[__builtin_ctz(m)];
        }
        k[r] = kk;
    }
}

// q = fp8(x * 2^-k) with the caller's k per row (planes.py:110-111): the
// wire image of a tensor whose exponents recover_exp found.
template <int FMT, bool BF16>
__global__ __launch_bounds__(kQBlock) void quant_k_kernel(const void* __restrict__ x, int64_t rows, int64_t cols,
                                                          int64_t segs, int vec, const int32_t* __restrict__ kin,
                                                          uint8_t* __restrict__ q) {
    constexpr int EPV = Seg<BF16>::EPV, VPL = Seg<BF16>::VPL, ESZ = BF16 ? 2 : 4;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    const int64_t row = gw / segs, seg = gw % segs;
    if (row >= rows) return;
    const int kk = kin[row];
    const bool fast = kk >= -kFastK && kk <= kFastK;
    const float s_down = fast ? __uint_as_float((uint32_t)(127 - kk) << 23) : pow2_dtype(-kk, BF16);
    const int64_t e0 = seg * kSegElems, e1 = min(e0 + kSegElems, cols);
    const int64_t base = row * cols;
    if (vec && fast) {
        const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + (base + e0) * ESZ);
        const int64_t nv = (e1 - e0) / EPV;
        uint4 buf[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            buf[j] = ld_vec(xr + (vi < nv ? vi : nv - 1));
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nv) continue;
            float f[EPV];
            unpack<BF16>(buf[j], f);
            uint32_t words[2];
#pragma unroll
            for (int h = 0; h < EPV; h += 4) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // non-finite values follow the restatement (NaN, Inf codes)
                    const uint32_t c = __builtin_isfinite(f[h + e])
                                           ? cvt_pk_fp8<FMT, false>(f[h + e] * s_down, 0.0f, 0u) & 0xFFu
                                           : quant_sw<FMT, BF16>(f[h + e], s_down);
                    w |= c << (8 * e);
                }
                words[h / 4] = w;
            }
            const int64_t e = e0 + vi * EPV;
            if (BF16) st_vec2(q + base + e, make_uint2(words[0], words[1]));
            else st_u32(q + base + e, words[0]);
        }
    } else {
        for (int64_t e = e0 + lane; e < e1; e += kWave) {
            const float v = load_x<BF16>(x, base + e);
            uint32_t c;
            if (fast && __builtin_isfinite(v)) c = cvt_pk_fp8<FMT, false>(v * s_down, 0.0f, 0u) & 0xFFu;
            else c = quant_sw<FMT, BF16>(v, s_down);
            q[base + e] = (uint8_t)c;
        }
    }
}

// ---------------------------------------------- recover + image, registers

// The first exact candidate of a row outside the register test (a NaN or Inf
// in the row, or candidates outside the instruction path), element by
// element through the restatement, or -1 (the recover_mask_kernel test).
template <int FMT, bool BF16>
__device__ __forceinline__ int recover_slow_row(const void* t, int64_t row, int64_t cols, int base, int lane) {
#pragma unroll 1
    for (int i = 0; i < 5; ++i) {
        bool ok = true;
#pragma unroll 1
        for (int64_t e = lane; e < cols; e += kWave)
            ok = ok && exact_at<FMT, BF16>(load_x<BF16>(t, row * cols + e), base + kDeltas[i], false);
        if (wave_and_u32(ok ? 1u : 0u)) return i;
    }
    return -1;
}

// One candidate exponent c over a row of finite elements held in registers:
// every element's code at 2^-c (packed four to a word, as quant_vec_fast
// packs them) into `codes`, and whether every element of this lane decodes
// back to itself.
template <int FMT, bool BF16, int VPL>
__device__ __forceinline__ bool recover_candidate(const uint4 (&buf)[VPL], int c, uint32_t (&codes)[VPL][BF16 ? 2 : 1]) {
    constexpr int EPV = BF16 ? 8 : 4;
    const float s_down = __uint_as_float((uint32_t)(127 - c) << 23);
    const float s_up = __uint_as_float((uint32_t)(127 + c) << 23);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        float v[EPV];
        unpack<BF16>(buf[j], v);  // lanes past the end hold zeros: exact at any c
#pragma unroll
        for (int h = 0; h < EPV; h += 4) {
            uint32_t w = cvt_pk_fp8<FMT, false>(v[h] * s_down, v[h + 1] * s_down, 0u);
            w = cvt_pk_fp8<FMT, true>(v[h + 2] * s_down, v[h + 3] * s_down, w);
            codes[j][h / 4] = w;
            float b[4];
            cvt_pk_f32<FMT, false>(w, b[0], b[1]);
            cvt_pk_f32<FMT, true>(w, b[2], b[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ok = ok & (b[e] * s_up == v[h + e]);
            }
        }
    }
    return ok;
}

// One wave per row held in registers (rows of up to kWave * VPL vectors,
// 16-byte aligned): |x|max, the base exponent, the candidates in the
// reference's order, each one wave vote over the registers (the base
// candidate is the only one a recipe round trip usually needs), then, when
// q is given, the row's wire image with the exponent found: one read of t
// and one write of q per element.  A row with no exact candidate counts as
// bad and keeps base + 2 (fp8.py:82-93), the last candidate tested, so in
// either case the codes the last test computed are the image of a row
// without NaN or Inf (the instruction equals the restatement there).
template <int FMT, bool BF16, int VPL>
__global__ __launch_bounds__(kQBlock) void recover_rows_kernel(const void* __restrict__ t, int64_t rows, int64_t cols,
                                                               int32_t* __restrict__ k, uint8_t* __restrict__ q,
                                                               unsigned long long* __restrict__ bad) {
    constexpr int EPV = BF16 ? 8 : 4;
    constexpr int ESZ = BF16 ? 2 : 4;
    // long rows leave few waves per SIMD (registers), so each wave keeps its
    // whole row in flight; short rows batch their loads
    constexpr int QB =
        (VPL >= ELY_RECOVER_WHOLE_VPL || ELY_RECOVER_BATCH <= 0 || ELY_RECOVER_BATCH > VPL) ? VPL : ELY_RECOVER_BATCH;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave_uniform(threadIdx.x / kWave);
    if (row >= rows) return;  // whole waves leave; the kernel has no block barrier
    const int64_t nvec = cols / EPV;
    const uint4* tr = reinterpret_cast<const uint4*>(static_cast<const char*>(t) + row * cols * ESZ);
    uint4 buf[VPL];
    uint32_t amax = 0;
#pragma unroll
    for (int j0 = 0; j0 < VPL; j0 += QB) {
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            buf[j] = ld_vec(tr + (vi < nvec ? vi : nvec - 1));
        }
#pragma unroll
        for (int j = j0; j < j0 + QB && j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nvec) buf[j] = make_uint4(0u, 0u, 0u, 0u);
            amax = vec_absmax<BF16>(buf[j], amax);
        }
        if (QB < VPL) __builtin_amdgcn_sched_barrier(0);
    }
    amax = wave_max_u32(amax);
    const uint32_t amax_bits = to_f32_bits<BF16>(amax);
    const bool finite_row = amax_bits < 0x7F800000u;  // NaN bits sort above Inf's
    const int base = scale_exp_from_amax<FMT>(amax_bits);
    int chosen = -1;
    bool have_codes = false;
    uint32_t codes[VPL][BF16 ? 2 : 1];
    if (finite_row && base - 2 >= -kFastK && base + 2 <= kFastK) {
#pragma unroll 1
        for (int i = 0; i < 5; ++i) {
            if (wave_and_u32(recover_candidate<FMT, BF16, VPL>(buf, base + kDeltas[i], codes) ? 1u : 0u)) {
                chosen = i;
                break;
            }
        }
        have_codes = VPL <= kRecoverKeepVpl;  // a compile-time false drops the codes
    } else {
        // rows holding NaN or Inf, or outside the instruction's exponent range
        chosen = recover_slow_row<FMT, BF16>(t, row, cols, base, lane);
    }
    const int kk = chosen >= 0 ? base + kDeltas[chosen] : base + 2;
    if (lane == 0) {
        k[row] = kk;
        if (chosen < 0) atomicAdd(bad, 1ull);
    }
    if (!q) return;
    // the image with the exponent found, as quant_k_kernel writes it
    uint8_t* qr = q + row * cols;
    if (have_codes) {
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nvec) continue;
            if (BF16) st_vec2(qr + vi * EPV, make_uint2(codes[j][0], codes[j][BF16 ? 1 : 0]));
            else st_u32(qr + vi * EPV, codes[j][0]);
        }
    } else if (kk >= -kFastK && kk <= kFastK) {
        const float s_down = __uint_as_float((uint32_t)(127 - kk) << 23);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t vi = lane + (int64_t)kWave * j;
            if (vi >= nvec) continue;
            float f[EPV];
            unpack<BF16>(buf[j], f);
            uint32_t words[2];
#pragma unroll
            for (int h = 0; h < EPV; h += 4) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t c = __builtin_isfinite(f[h + e])
                                           ? cvt_pk_fp8<FMT, false>(f[h + e] * s_down, 0.0f, 0u) & 0xFFu
                                           : quant_sw<FMT, BF16>(f[h + e], s_down);
                    w |= c << (8 * e);
                }
                words[h / 4] = w;
            }
            if (BF16) st_vec2(qr + vi * EPV, make_uint2(words[0], words[1]));
            else st_u32(qr + vi * EPV, words[0]);
        }
    } else {
        const float s_down = pow2_dtype(-kk, BF16);
#pragma unroll 1
        for (int64_t e = lane; e < cols; e += kWave) qr[e] = (uint8_t)quant_sw<FMT, BF16>(load_x<BF16>(t, row * cols + e), s_down);
    }
}

// --------------------------------------------------------------- self-test

template <int FMT>
__global__ void selftest_cvt_kernel(uint32_t start, uint64_t count, unsigned long long* mism) {
    using F = Fp8Fmt<FMT>;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t u = (uint32_t)(start + i);
        const float x = __uint_as_float(u);
        const uint32_t sw = fp8_from_f32_sw<FMT>(x);
        const uint32_t lo = cvt_pk_fp8<FMT, false>(x, 0.0f, 0u);
        const uint32_t hi = cvt_pk_fp8<FMT, true>(0.0f, x, 0u);
        const uint32_t hw0 = lo & 0xFFu, hw1 = (hi >> 24) & 0xFFu;
        const bool domain = (u & 0x7FFFFFFFu) <= F::kMaxFiniteBits;
        if (hw0 != sw || hw1 != sw) atomicAdd(mism + (domain ? 0 : 1), 1ull);
        if (u - start < 256u && start == 0u) {
            // decode: every code, instruction vs restatement, both halves of the word
            const uint32_t c = u;
            float a, b, c2, d;
            cvt_pk_f32<FMT, false>(c | (c << 8), a, b);
            cvt_pk_f32<FMT, true>((c << 16) | (c << 24), c2, d);
            const float ref = fp8_to_f32_sw<FMT>(c);
            const float got[4] = {a, b, c2, d};
            bool bad = false;
            for (int j = 0; j < 4; ++j) {
                if (ref != ref) bad |= got[j] == got[j];
                else bad |= __float_as_uint(got[j]) != __float_as_uint(ref);
            }
            if (bad) atomicAdd(mism + 2, 1ull);
        }
    }
}

// One thread per (bf16 pattern u, k), |k| <= kFastK.  Quantize: u and its
// negation in the two halves of a word, converted at scale 2^k into both
// halves of the output, against the restatement quant_sw at 2^-k, over the
// pairs the instruction path meets (finite, |x| 2^-k < 2^ebias) -> mism[0].
// Decode (u < 256, the code): the code in all four bytes, both halves
// decoded at 2^k, against dequant_sw rounded to bf16, NaN codes aside (the
// kernels keep them off the scaled decode) -> mism[1].
template <int FMT>
__global__ void selftest_scaled_kernel(unsigned long long* mism) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= 65536u * (2u * kFastK + 1u)) return;
    const uint32_t u = t & 0xFFFFu;
    const int k = (int)(t >> 16) - kFastK;
    const float s_down = __uint_as_float((uint32_t)(127 - k) << 23);
    const float s_up = __uint_as_float((uint32_t)(127 + k) << 23);
    const float x = bf16_to_f32(u);
    const float lim = __uint_as_float((uint32_t)(127 + Fp8Fmt<FMT>::EBIAS) << 23);
    if ((u & 0x7F80u) != 0x7F80u && __builtin_fabsf(x * s_down) < lim) {
        const uint32_t w = u | ((u ^ 0x8000u) << 16);
        const uint32_t want = quant_sw<FMT, true>(x, s_down), want_neg = quant_sw<FMT, true>(-x, s_down);
        const uint32_t lo = cvt_scaled_pk_fp8_bf16<FMT, false>(w, s_up, 0u);
        const uint32_t hi = cvt_scaled_pk_fp8_bf16<FMT, true>(w, s_up, 0u);
        if ((lo & 0xFFu) != want || ((lo >> 8) & 0xFFu) != want_neg || ((hi >> 16) & 0xFFu) != want ||
            (hi >> 24) != want_neg)
            atomicAdd(mism, 1ull);
    }
    if (u < 256u && (nan_code_bits<FMT>(u) == 0u)) {
        const uint32_t want = f32_to_bf16(dequant_sw<FMT, true>(u, s_up));
        const uint32_t w = u * 0x01010101u;
        const uint32_t lo = cvt_scaled_pk_bf16<FMT, false>(w, s_up), hi = cvt_scaled_pk_bf16<FMT, true>(w, s_up);
        if (lo != (want | (want << 16)) || hi != (want | (want << 16))) atomicAdd(mism + 1, 1ull);
    }
}

__global__ void selftest_sqrt_kernel(uint32_t start, uint64_t count, unsigned long long* mism) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t u = (uint32_t)(start + i) & 0x7FFFFFFFu;  // non-negative patterns
        const float x = __uint_as_float(u);
        const float a = __builtin_sqrtf(x);
        const float b = (float)__builtin_sqrt((double)x);
        if (__float_as_uint(a) != __float_as_uint(b) && !(a != a && b != b)) atomicAdd(mism, 1ull);
    }
}

// ------------------------------------------------------------------ launch

static void check_fmt(int32_t fmt) {
    if (fmt != ELY_E4M3 && fmt != ELY_E5M2) fail(ELY_EINVAL, "fp8 format must be ELY_E4M3 or ELY_E5M2");
}

static void check_dtype(int32_t dt, const char* what) {
    if (dt != ELY_F32 && dt != ELY_BF16) fail(ELY_EINVAL, std::string(what) + " must be ELY_F32 or ELY_BF16");
}

static void check_shape(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) fail(ELY_EINVAL, "negative rows or cols");
    if (cols > 0 && rows > INT64_MAX / cols) fail(ELY_EINVAL, "rows * cols overflows");
}

static unsigned blocks_for_waves(int64_t waves) {
    const int64_t b = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    // a dispatch counts its work-items in 32 bits
    if (b > 0xFFFFFFFFLL / kQBlock) fail(ELY_EINVAL, "grid too large: more than 2^32 - 1 threads in one launch");
    return (unsigned)b;
}

// Vectors per lane of the register paths: a wave per row up to kMaxWaveVpl,
// a block of kRowWaves waves per row above (the block's loads in flight
// per row stay the same, and more rows stream at once).
constexpr int kVplChoices[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16};
constexpr int kMaxWaveVpl = 6;

template <int FMT, bool BF16, int VPL>
static void launch_rows(const void* x, int64_t rows, int64_t cols, uint8_t* q, int32_t* k, void* out, hipStream_t s) {
    hipLaunchKernelGGL((quant_rows_kernel<FMT, BF16, VPL>), dim3(blocks_for_waves(rows)), dim3(kQBlock), ELY_Q_LDS, s, x,
                       rows, cols, q, k, out);
    check_launch("quant_rows_kernel");
}

template <int FMT, bool BF16>
static void dispatch_rows(int vpl, const void* x, int64_t rows, int64_t cols, uint8_t* q, int32_t* k, void* out,
                          hipStream_t s) {
    switch (vpl) {
        case 1: return launch_rows<FMT, BF16, 1>(x, rows, cols, q, k, out, s);
        case 2: return launch_rows<FMT, BF16, 2>(x, rows, cols, q, k, out, s);
        case 3: return launch_rows<FMT, BF16, 3>(x, rows, cols, q, k, out, s);
        case 4: return launch_rows<FMT, BF16, 4>(x, rows, cols, q, k, out, s);
        case 5: return launch_rows<FMT, BF16, 5>(x, rows, cols, q, k, out, s);
        case 6: return launch_rows<FMT, BF16, 6>(x, rows, cols, q, k, out, s);
        default: fail(ELY_EINVAL, "internal: no register path for this row length");
    }
}

// Register path's vectors per lane for these columns, or 0 when the row does
// not fit it.
static int rows_vpl(int64_t cols, int32_t dtype, const void* x, const uint8_t* q, const void* out) {
    const int64_t epv = dtype == ELY_BF16 ? 8 : 4;
    if (cols == 0 || cols % epv != 0) return 0;
    if (!aligned16(x) || (out && !aligned16(out))) return 0;
    if (q && (reinterpret_cast<uintptr_t>(q) % (uintptr_t)epv) != 0) return 0;
    const int64_t nvec = cols / epv;
    for (int v : kVplChoices)
        if (nvec <= (int64_t)kWave * v) return v;
    return 0;
}

// Row maxima, then the partial maxima (at most max(rows, kSplitWaves) of them).
static size_t rowmax_bytes(int64_t rows) { return align_up((size_t)std::max<int64_t>(rows, 1) * 4, 256); }
static size_t split_ws_bytes(int64_t rows) {
    return rowmax_bytes(rows) + align_up((size_t)std::max<int64_t>(rows, kSplitWaves) * 4, 256);
}

// rowmax[r] = |x|max bits of row r, through the split path's two launches.
template <bool BF16>
static void split_rowmax(const void* x, int64_t rows, int64_t cols, int vec, void* workspace, uint32_t* rowmax,
                         hipStream_t s) {
    const int64_t segs = (cols + kSegElems - 1) / kSegElems;
    const int64_t wpr = split_wpr(rows, segs);
    if (rows > INT64_MAX / wpr) fail(ELY_EINVAL, "too many rows");
    uint32_t* partial = wpr == 1 ? rowmax : reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + rowmax_bytes(rows));
    const int64_t seg_bytes = kSegElems * (BF16 ? 2 : 4);
    const int64_t cached = std::min<int64_t>(segs, ((int64_t)ELY_SPLIT_CACHED_MB << 20) / (seg_bytes * rows));
    hipLaunchKernelGGL((rowmax_partial_kernel<BF16>), dim3(blocks_for_waves(rows * wpr)), dim3(kQBlock), 0, s, x, rows,
                       cols, segs, wpr, vec, cached, partial);
    check_launch("rowmax_partial_kernel");
    if (wpr > 1) {
        hipLaunchKernelGGL(rowmax_reduce_kernel, dim3((unsigned)std::min<int64_t>(rows, 65536)), dim3(kRowBlock), 0, s,
                           (const uint32_t*)partial, rows, wpr, rowmax);
        check_launch("rowmax_reduce_kernel");
    }
}

static size_t guess_ws_bytes(int64_t n);
template <int FMT, bool BF16>
static void quantize_guess_impl(const void* x, int64_t n, uint8_t* q, int32_t* k, void* out, void* workspace,
                                int64_t ws_bytes, hipStream_t s);

template <int FMT, bool BF16>
static void quantize_impl(const void* x, int64_t rows, int64_t cols, uint8_t* q, int32_t* k, void* out,
                          void* workspace, int64_t ws_bytes, hipStream_t s, bool allow_guess = true) {
    if (rows == 0) return;
    if (cols == 0) {
        // an empty row has |x|max 0, so k = 0 (fp8.py:38)
        if (k) {
            hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)std::min<int64_t>((rows + 255) / 256, 4096)), dim3(256),
                               0, s, reinterpret_cast<uint32_t*>(k), rows, 0u);
            check_launch("fill_u32_kernel");
        }
        return;
    }
    const int32_t dt = BF16 ? ELY_BF16 : ELY_F32;
    const int vpl = rows_vpl(cols, dt, x, q, out);
    if (vpl > kMaxWaveVpl) {
        // one block per row: kRowWaves waves of ceil(vpl / kRowWaves) vectors per lane
        if (rows > 0xFFFFFFFFLL / kRowBlock) fail(ELY_EINVAL, "fp8 quantize: too many rows for one launch");
        switch ((vpl + kRowWaves - 1) / kRowWaves) {
            case 2: hipLaunchKernelGGL((quant_block_row_kernel<FMT, BF16, 2>), dim3((unsigned)rows), dim3(kRowBlock), 0, s, x, cols, q, k, out); break;
            case 3: hipLaunchKernelGGL((quant_block_row_kernel<FMT, BF16, 3>), dim3((unsigned)rows), dim3(kRowBlock), 0, s, x, cols, q, k, out); break;
            case 4: hipLaunchKernelGGL((quant_block_row_kernel<FMT, BF16, 4>), dim3((unsigned)rows), dim3(kRowBlock), 0, s, x, cols, q, k, out); break;
            default: fail(ELY_EINVAL, "internal: no block-row path for this row length");
        }
        check_launch("quant_block_row_kernel");
        return;
    }
    if (vpl) return dispatch_rows<FMT, BF16>(vpl, x, rows, cols, q, k, out, s);
    const int64_t epv = BF16 ? 8 : 4;
    const int vec = (cols % epv == 0) && aligned16(x) && (!out || aligned16(out)) &&
                    (!q || reinterpret_cast<uintptr_t>(q) % (uintptr_t)epv == 0);
    if (allow_guess && rows == 1 && (q || out) && vec && cols >= ((int64_t)ELY_GUESS_MIN_MB << 20) / (BF16 ? 2 : 4) &&
        workspace && ws_bytes >= (int64_t)guess_ws_bytes(cols))
        return quantize_guess_impl<FMT, BF16>(x, cols, q, k, out, workspace, ws_bytes, s);
    if (!workspace || ws_bytes < (int64_t)split_ws_bytes(rows))
        fail(ELY_EWORKSPACE, "fp8 quantize: this shape needs " + std::to_string(split_ws_bytes(rows)) +
                                 " workspace bytes (ely_fp8_workspace_bytes)");
    uint32_t* rowmax = static_cast<uint32_t*>(workspace);
    const int64_t segs = (cols + kSegElems - 1) / kSegElems;
    if (rows > INT64_MAX / segs) fail(ELY_EINVAL, "too many segments");
    split_rowmax<BF16>(x, rows, cols, vec, workspace, rowmax, s);
    const unsigned blocks = blocks_for_waves(rows * segs);
    hipLaunchKernelGGL((quant_split_kernel<FMT, BF16>), dim3(blocks), dim3(kQBlock), 0, s, x, rows, cols, segs, vec,
                       (const uint32_t*)rowmax, q, k, out);
    check_launch("quant_split_kernel");
}

// Workspace of the hint path over n elements: one maximum per segment, the
// reduce launch's kHintBlocks maxima, the hint as read; at least the split
// path's, which a call falls back to when the one-pass form does not apply.
static size_t hint_ws_bytes(int64_t n) {
    const int64_t segs = std::max<int64_t>((n + kSegElems - 1) / kSegElems, 1);
    return std::max(align_up((size_t)segs * 4, 256) + align_up((size_t)kHintBlocks * 4, 256) + 256, split_ws_bytes(1));
}

template <int FMT, bool BF16>
static void quantize_hint_impl(const void* x, int64_t n, int32_t k_hint, const int32_t* k_hint_dev, uint8_t* q,
                               int32_t* k, void* out, int32_t* hit, void* workspace, int64_t ws_bytes,
                               hipStream_t s, bool hint_is_amax = false) {
    if (!workspace || ws_bytes < (int64_t)hint_ws_bytes(n))
        fail(ELY_EWORKSPACE, "ely_fp8_quantize_hint: workspace of " + std::to_string(ws_bytes) + " bytes, need " +
                                 std::to_string(hint_ws_bytes(n)) + " (ely_fp8_hint_workspace_bytes)");
    const int64_t epv = BF16 ? 8 : 4;
    const bool vec = n > 0 && n % epv == 0 && aligned16(x) && (!out || aligned16(out)) &&
                     (!q || reinterpret_cast<uintptr_t>(q) % (uintptr_t)epv == 0);
    if (!vec || (!k_hint_dev && (k_hint < -kFastK || k_hint > kFastK))) {
        // no one-pass form for this tensor or hint: the split path, a miss
        quantize_impl<FMT, BF16>(x, 1, n, q, k, out, workspace, ws_bytes, s, false);
        if (hit) {
            hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<uint32_t*>(hit), (int64_t)1, 0u);
            check_launch("fill_u32_kernel");
        }
        return;
    }
    const int64_t segs = (n + kSegElems - 1) / kSegElems;
    uint32_t* partial = static_cast<uint32_t*>(workspace);
    uint32_t* block_max = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + align_up((size_t)segs * 4, 256));
    int32_t* hint_copy = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(block_max) + align_up((size_t)kHintBlocks * 4, 256));
    hipLaunchKernelGGL((quant_hint_kernel<FMT, BF16>), dim3(blocks_for_waves(segs)), dim3(kQBlock), 0, s, x, n, segs,
                       k_hint, k_hint_dev, hint_is_amax ? 1 : 0, q, out, partial, hint_copy);
    check_launch("quant_hint_kernel");
    hipLaunchKernelGGL(hint_reduce_kernel, dim3(kHintBlocks), dim3(kRowBlock), 0, s, (const uint32_t*)partial, segs,
                       block_max);
    check_launch("hint_reduce_kernel");
    const int64_t waves = std::min<int64_t>(segs, (int64_t)device_info().cus * kHintFixupWavesPerCU);
    hipLaunchKernelGGL((quant_hint_fixup_kernel<FMT, BF16>), dim3(blocks_for_waves(waves)), dim3(kQBlock), 0, s, x, n,
                       segs, 1, (const int32_t*)hint_copy, (const uint32_t*)block_max, q, k, out, hit);
    check_launch("quant_hint_fixup_kernel");
}

// Per-tensor rows of at least ELY_GUESS_MIN_MB MiB (the vector form, a
// workspace of guess_ws_bytes): the exponent is guessed from every
// kGuessStride-th segment's |x|max, and the row goes through the hint path
// at that guess: one read of x when the sample holds the row's maximum
// binade, the hint path's fixup (a second read and write) when it does not.
// Either way the codes and k are the split path's, byte for byte.  C4
// per-tensor (both inputs guess right), kernel time per call: quantize
// 272 us against 404 on the split path, round trip 357 against 488.
static size_t guess_ws_bytes(int64_t n) { return hint_ws_bytes(n) + 256; }

template <int FMT, bool BF16>
static void quantize_guess_impl(const void* x, int64_t n, uint8_t* q, int32_t* k, void* out, void* workspace,
                                int64_t ws_bytes, hipStream_t s) {
    // after the hint path's layout: the sampled |x|max, and k's word when
    // the caller asked for no k (a round trip); the samples' maxima go where
    // the hint path's per-segment maxima go later (samples <= segments)
    uint32_t* amax = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + hint_ws_bytes(n));
    int32_t* kword = k ? k : reinterpret_cast<int32_t*>(amax + 1);
    uint32_t* partial = static_cast<uint32_t*>(workspace);
    const int64_t segs = (n + kSegElems - 1) / kSegElems;
    const int64_t samples = (segs + kGuessStride - 1) / kGuessStride;
    hipLaunchKernelGGL((guess_amax_kernel<BF16>), dim3(blocks_for_waves(samples)), dim3(kQBlock), 0, s, x, n,
                       (int64_t)kGuessStride, samples, partial);
    check_launch("guess_amax_kernel");
    hipLaunchKernelGGL(sample_max_kernel, dim3(1), dim3(kSampleMaxBlock), 0, s, (const uint32_t*)partial, samples, amax);
    check_launch("sample_max_kernel");
    quantize_hint_impl<FMT, BF16>(x, n, 0, reinterpret_cast<const int32_t*>(amax), q, kword, out, nullptr, workspace,
                                  ws_bytes, s, true);
}

template <int FMT, bool BF16OUT>
static void dequantize_impl(const uint8_t* q, const int32_t* k, int64_t rows, int64_t cols, void* out,
                            hipStream_t s) {
    if (rows == 0 || cols == 0) return;
    if ((cols % 16 == 0) && aligned16(q) && aligned16(out)) {
        const int64_t n = rows * cols;
        const unsigned blocks = blocks_for_waves((n + kDeqSegCodes - 1) / kDeqSegCodes);
        if (n < ((int64_t)1 << 32))
            hipLaunchKernelGGL((dequant_flat_kernel<FMT, BF16OUT, true>), dim3(blocks), dim3(kQBlock), ELY_DEQ_LDS, s, q, k, n,
                               cols, out);
        else
            hipLaunchKernelGGL((dequant_flat_kernel<FMT, BF16OUT, false>), dim3(blocks), dim3(kQBlock), ELY_DEQ_LDS, s, q, k, n,
                               cols, out);
        check_launch("dequant_flat_kernel");
        return;
    }
    const int64_t segs = (cols + kDeqSegCodes - 1) / kDeqSegCodes;
    if (rows > INT64_MAX / segs) fail(ELY_EINVAL, "too many segments");
    hipLaunchKernelGGL((dequant_any_kernel<FMT, BF16OUT>), dim3(blocks_for_waves(rows * segs)), dim3(kQBlock), 0, s, q,
                       k, rows, cols, segs, out);
    check_launch("dequant_any_kernel");
}

// Register path of recover_exp / recover_image: vectors per lane (2, 4, 5,
// 6, 8 or 16) for rows of `cols` elements, or 0 when the row does not fit it.
static int recover_vpl(int64_t cols, bool bf16, const void* t, const uint8_t* q) {
    const int64_t epv = bf16 ? 8 : 4;
    if (cols == 0 || cols % epv != 0 || !aligned16(t)) return 0;
    if (q && reinterpret_cast<uintptr_t>(q) % (uintptr_t)epv != 0) return 0;
    const int64_t nvec = cols / epv;
    for (int v : {2, 4, 5, 6, 8, 16})
        if (nvec <= (int64_t)kWave * v) return v;
    return 0;
}

template <int FMT, bool BF16>
static void launch_recover_rows(int vpl, const void* t, int64_t rows, int64_t cols, int32_t* k, uint8_t* q,
                                unsigned long long* bad, hipStream_t s) {
    const dim3 g(blocks_for_waves(rows)), b(kQBlock);
    switch (vpl) {
        case 2: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 2>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        case 4: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 4>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        case 5: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 5>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        case 6: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 6>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        case 8: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 8>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        case 16: hipLaunchKernelGGL((recover_rows_kernel<FMT, BF16, 16>), g, b, 0, s, t, rows, cols, k, q, bad); break;
        default: fail(ELY_EINVAL, "internal: no register path for this row length");
    }
    check_launch("recover_rows_kernel");
}

static void recover_rows(int vpl, const void* t, bool bf16, int64_t rows, int64_t cols, int32_t fmt, int32_t* k,
                         uint8_t* q, unsigned long long* bad, hipStream_t s) {
    if (fmt == ELY_E4M3) {
        if (bf16) launch_recover_rows<kE4M3, true>(vpl, t, rows, cols, k, q, bad, s);
        else launch_recover_rows<kE4M3, false>(vpl, t, rows, cols, k, q, bad, s);
    } else {
        if (bf16) launch_recover_rows<kE5M2, true>(vpl, t, rows, cols, k, q, bad, s);
        else launch_recover_rows<kE5M2, false>(vpl, t, rows, cols, k, q, bad, s);
    }
}

// The multi-launch recovery for any shape: row maxima, the candidates'
// exactness per segment, then k per row.
static void recover_multi(const void* t, bool bf16, int64_t rows, int64_t cols, int32_t fmt, int32_t* k,
                          unsigned long long* bad_rows_dev, void* workspace, hipStream_t s) {
    uint32_t* rowmax = static_cast<uint32_t*>(workspace);
    uint32_t* rowmask = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + split_ws_bytes(rows));
    const unsigned fb = (unsigned)std::min<int64_t>((rows + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(fb), dim3(256), 0, s, rowmask, rows, 0x1Fu);
    check_launch("fill_u32_kernel");
    if (cols == 0) {
        hipLaunchKernelGGL(fill_u32_kernel, dim3(fb), dim3(256), 0, s, rowmax, rows, 0u);
        check_launch("fill_u32_kernel");
    } else {
        const int64_t segs = (cols + kSegElems - 1) / kSegElems;
        if (rows > INT64_MAX / segs) fail(ELY_EINVAL, "too many segments");
        const unsigned blocks = blocks_for_waves(rows * segs);
        const int vec = (cols % (bf16 ? 8 : 4) == 0) && aligned16(t);
        if (bf16) split_rowmax<true>(t, rows, cols, vec, workspace, rowmax, s);
        else split_rowmax<false>(t, rows, cols, vec, workspace, rowmax, s);
#define ELY_RECOVER_MASK(F, B)                                                                                    \
    do {                                                                                                          \
        hipLaunchKernelGGL((recover_mask_kernel<F, B, 0>), dim3(blocks), dim3(kQBlock), 0, s, t, rows, cols, segs, \
                           vec, (const uint32_t*)rowmax, rowmask);                                                \
        hipLaunchKernelGGL((recover_mask_kernel<F, B, 1>), dim3(blocks), dim3(kQBlock), 0, s, t, rows, cols, segs, \
                           vec, (const uint32_t*)rowmax, rowmask);                                                \
    } while (0)
        if (fmt == ELY_E4M3) {
            if (bf16) ELY_RECOVER_MASK(kE4M3, true);
            else ELY_RECOVER_MASK(kE4M3, false);
        } else {
            if (bf16) ELY_RECOVER_MASK(kE5M2, true);
            else ELY_RECOVER_MASK(kE5M2, false);
        }
#undef ELY_RECOVER_MASK
        check_launch("recover_mask_kernel");
    }
#define ELY_RECOVER_FINAL(F, B)                                                                                   \
    hipLaunchKernelGGL((recover_final_kernel<F, B>), dim3(fb), dim3(256), 0, s, rows, (const uint32_t*)rowmax,      \
                       (const uint32_t*)rowmask, k, bad_rows_dev)
    if (fmt == ELY_E4M3) {
        if (bf16) ELY_RECOVER_FINAL(kE4M3, true);
        else ELY_RECOVER_FINAL(kE4M3, false);
    } else {
        if (bf16) ELY_RECOVER_FINAL(kE5M2, true);
        else ELY_RECOVER_FINAL(kE5M2, false);
    }
#undef ELY_RECOVER_FINAL
    check_launch("recover_final_kernel");
}

static void quant_k_launch(const void* x, bool bf16, int64_t rows, int64_t cols, int32_t fmt, const int32_t* k,
                           uint8_t* q, hipStream_t s) {
    const int64_t segs = (cols + kSegElems - 1) / kSegElems;
    if (rows > INT64_MAX / segs) fail(ELY_EINVAL, "too many segments");
    const unsigned blocks = blocks_for_waves(rows * segs);
    const int vec = (cols % (bf16 ? 8 : 4) == 0) && aligned16(x) &&
                    (reinterpret_cast<uintptr_t>(q) % (bf16 ? 8 : 4) == 0);
#define ELY_QK(F, B) \
    hipLaunchKernelGGL((quant_k_kernel<F, B>), dim3(blocks), dim3(kQBlock), 0, s, x, rows, cols, segs, vec, k, q)
    if (fmt == ELY_E4M3) {
        if (bf16) ELY_QK(kE4M3, true);
        else ELY_QK(kE4M3, false);
    } else {
        if (bf16) ELY_QK(kE5M2, true);
        else ELY_QK(kE5M2, false);
    }
#undef ELY_QK
    check_launch("quant_k_kernel");
}

// ------------------------------------------------ quantize without allocation

// Scratch of ely_fp8_quantize_noalloc: the split path's row maxima and
// partial maxima live in this file-scope device array instead of a caller
// workspace, so that entry point allocates nothing.  Each GPU holds its own
// copy at its own address until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns on that device (the
// array's name in host code is a stand-in, not a device address).
constexpr size_t kNoallocScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch_ptr;  // device -> address of `scratch` there

// The current device's address of `scratch`, looked up once per device with
// that device current.
static void* noalloc_scratch() {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_ptr.find(dev);
    if (it != g_scratch_ptr.end()) return it->second;
    void* ptr = nullptr;
    check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) fail(ELY_EHIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr.emplace(dev, ptr);
    return ptr;
}

}  // namespace ely

using namespace ely;

extern "C" {

int64_t ely_fp8_workspace_bytes(int64_t rows, int64_t cols, int32_t x_dtype) {
    if (rows < 0 || cols < 0) return -1;
    // a long per-tensor row also has room for the sampled-guess path
    if (rows == 1 && cols >= ((int64_t)ELY_GUESS_MIN_MB << 20) / (x_dtype == ELY_F32 ? 4 : 2))
        return (int64_t)std::max(split_ws_bytes(1), guess_ws_bytes(cols));
    return (int64_t)split_ws_bytes(rows);
}

int ely_fp8_quantize(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt, uint8_t* q, int32_t* k,
                     void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(x_dtype, "x_dtype");
        check_shape(rows, cols);
        if (rows * cols > 0 && !x) fail(ELY_EINVAL, "ely_fp8_quantize: null x");
        if (rows > 0 && !k) fail(ELY_EINVAL, "ely_fp8_quantize: null k");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (fmt == ELY_E4M3) {
            if (x_dtype == ELY_BF16) quantize_impl<kE4M3, true>(x, rows, cols, q, k, nullptr, workspace, ws_bytes, s);
            else quantize_impl<kE4M3, false>(x, rows, cols, q, k, nullptr, workspace, ws_bytes, s);
        } else {
            if (x_dtype == ELY_BF16) quantize_impl<kE5M2, true>(x, rows, cols, q, k, nullptr, workspace, ws_bytes, s);
            else quantize_impl<kE5M2, false>(x, rows, cols, q, k, nullptr, workspace, ws_bytes, s);
        }
    });
}

int ely_fp8_quantize_noalloc(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt, uint8_t* q,
                             int32_t* k, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(x_dtype, "x_dtype");
        check_shape(rows, cols);
        if (rows * cols > 0 && !x) fail(ELY_EINVAL, "ely_fp8_quantize_noalloc: null x");
        if (rows > 0 && !k) fail(ELY_EINVAL, "ely_fp8_quantize_noalloc: null k");
        // Only the split path (rows that fit no register path) uses scratch;
        // its row maxima and partials must fit the static array.  Every
        // scratch word the split launches read was written by an earlier
        // launch of the same call, so nothing needs clearing between calls.
        const bool split = rows > 0 && cols > 0 && rows_vpl(cols, x_dtype, x, q, nullptr) == 0;
        void* ws = nullptr;
        if (split) {
            const size_t need = split_ws_bytes(rows);
            if (need > kNoallocScratchBytes)
                fail(ELY_EINVAL, "ely_fp8_quantize_noalloc: " + std::to_string(rows) + " rows of " + std::to_string(cols) +
                                     " columns need " + std::to_string(need) + " scratch bytes, above the " +
                                     std::to_string(kNoallocScratchBytes) +
                                     "-byte static scratch; use ely_fp8_quantize with a workspace");
            ws = noalloc_scratch();
        }
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int64_t wsb = split ? (int64_t)kNoallocScratchBytes : 0;
        if (fmt == ELY_E4M3) {
            if (x_dtype == ELY_BF16) quantize_impl<kE4M3, true>(x, rows, cols, q, k, nullptr, ws, wsb, s, false);
            else quantize_impl<kE4M3, false>(x, rows, cols, q, k, nullptr, ws, wsb, s, false);
        } else {
            if (x_dtype == ELY_BF16) quantize_impl<kE5M2, true>(x, rows, cols, q, k, nullptr, ws, wsb, s, false);
            else quantize_impl<kE5M2, false>(x, rows, cols, q, k, nullptr, ws, wsb, s, false);
        }
    });
}

int64_t ely_fp8_hint_workspace_bytes(int64_t n) {
    if (n < 0) return -1;
    return (int64_t)hint_ws_bytes(n);
}

int ely_fp8_quantize_hint(const void* x, int32_t x_dtype, int64_t n, int32_t fmt, int32_t k_hint,
                          const int32_t* k_hint_dev, uint8_t* q, int32_t* k, void* out, int32_t* hit_dev,
                          void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(x_dtype, "x_dtype");
        check_shape(1, n);
        if (!k) fail(ELY_EINVAL, "ely_fp8_quantize_hint: null k");
        if (n > 0 && (!x || (!q && !out))) fail(ELY_EINVAL, "ely_fp8_quantize_hint: null x, or neither q nor out");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (fmt == ELY_E4M3) {
            if (x_dtype == ELY_BF16) quantize_hint_impl<kE4M3, true>(x, n, k_hint, k_hint_dev, q, k, out, hit_dev, workspace, ws_bytes, s);
            else quantize_hint_impl<kE4M3, false>(x, n, k_hint, k_hint_dev, q, k, out, hit_dev, workspace, ws_bytes, s);
        } else {
            if (x_dtype == ELY_BF16) quantize_hint_impl<kE5M2, true>(x, n, k_hint, k_hint_dev, q, k, out, hit_dev, workspace, ws_bytes, s);
            else quantize_hint_impl<kE5M2, false>(x, n, k_hint, k_hint_dev, q, k, out, hit_dev, workspace, ws_bytes, s);
        }
    });
}

int ely_fp8_dequantize(const uint8_t* q, const int32_t* k, int64_t rows, int64_t cols, int32_t fmt, void* out,
                       int32_t out_dtype, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(out_dtype, "out_dtype");
        check_shape(rows, cols);
        if (rows * cols > 0 && (!q || !k || !out)) fail(ELY_EINVAL, "ely_fp8_dequantize: null pointer");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (fmt == ELY_E4M3) {
            if (out_dtype == ELY_BF16) dequantize_impl<kE4M3, true>(q, k, rows, cols, out, s);
            else dequantize_impl<kE4M3, false>(q, k, rows, cols, out, s);
        } else {
            if (out_dtype == ELY_BF16) dequantize_impl<kE5M2, true>(q, k, rows, cols, out, s);
            else dequantize_impl<kE5M2, false>(q, k, rows, cols, out, s);
        }
    });
}

int ely_fp8_roundtrip(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt, void* out, uint8_t* q,
                      int32_t* k, void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(x_dtype, "x_dtype");
        check_shape(rows, cols);
        if (rows * cols > 0 && (!x || !out)) fail(ELY_EINVAL, "ely_fp8_roundtrip: null x or out");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (fmt == ELY_E4M3) {
            if (x_dtype == ELY_BF16) quantize_impl<kE4M3, true>(x, rows, cols, q, k, out, workspace, ws_bytes, s);
            else quantize_impl<kE4M3, false>(x, rows, cols, q, k, out, workspace, ws_bytes, s);
        } else {
            if (x_dtype == ELY_BF16) quantize_impl<kE5M2, true>(x, rows, cols, q, k, out, workspace, ws_bytes, s);
            else quantize_impl<kE5M2, false>(x, rows, cols, q, k, out, workspace, ws_bytes, s);
        }
    });
}

int ely_selftest_fp8_cvt(uint32_t start, uint64_t count, int32_t fmt, unsigned long long* mismatches_dev,
                         void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        if (!mismatches_dev) fail(ELY_EINVAL, "null counters");
        if (count > (1ull << 32) || (uint64_t)start + count > (1ull << 32))
            fail(ELY_EINVAL, "range beyond the 2^32 fp32 patterns");
        if (count == 0) return;
        hipStream_t s = static_cast<hipStream_t>(stream);
        const unsigned blocks = (unsigned)std::min<uint64_t>((count + 255) / 256, 65536);
        if (fmt == ELY_E4M3)
            hipLaunchKernelGGL(selftest_cvt_kernel<kE4M3>, dim3(blocks), dim3(256), 0, s, start, count, mismatches_dev);
        else
            hipLaunchKernelGGL(selftest_cvt_kernel<kE5M2>, dim3(blocks), dim3(256), 0, s, start, count, mismatches_dev);
        check_launch("selftest_cvt_kernel");
    });
}

int ely_selftest_fp8_scaled(int32_t fmt, unsigned long long* mismatches_dev, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        if (!mismatches_dev) fail(ELY_EINVAL, "null counters");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const unsigned blocks = (65536u * (2u * kFastK + 1u) + 255u) / 256u;
        if (fmt == ELY_E4M3)
            hipLaunchKernelGGL(selftest_scaled_kernel<kE4M3>, dim3(blocks), dim3(256), 0, s, mismatches_dev);
        else
            hipLaunchKernelGGL(selftest_scaled_kernel<kE5M2>, dim3(blocks), dim3(256), 0, s, mismatches_dev);
        check_launch("selftest_scaled_kernel");
    });
}

int ely_selftest_sqrt(uint32_t start, uint64_t count, unsigned long long* mismatches_dev, void* stream) {
    return guarded([&] {
        if (!mismatches_dev) fail(ELY_EINVAL, "null counter");
        if (count > (1ull << 32) || (uint64_t)start + count > (1ull << 32))
            fail(ELY_EINVAL, "range beyond the 2^32 fp32 patterns");
        if (count == 0) return;
        hipStream_t s = static_cast<hipStream_t>(stream);
        const unsigned blocks = (unsigned)std::min<uint64_t>((count + 255) / 256, 65536);
        hipLaunchKernelGGL(selftest_sqrt_kernel, dim3(blocks), dim3(256), 0, s, start, count, mismatches_dev);
        check_launch("selftest_sqrt_kernel");
    });
}

int64_t ely_fp8_recover_workspace_bytes(int64_t rows) {
    if (rows < 0) return -1;
    return (int64_t)(split_ws_bytes(rows) + rowmax_bytes(rows));
}

int ely_fp8_recover_exp(const void* t, int32_t t_dtype, int64_t rows, int64_t cols, int32_t fmt, int32_t* k,
                        unsigned long long* bad_rows_dev, void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(t_dtype, "t_dtype");
        check_shape(rows, cols);
        if (rows == 0) return;
        if (!k || !bad_rows_dev || (cols > 0 && !t)) fail(ELY_EINVAL, "ely_fp8_recover_exp: null pointer");
        if (!workspace || ws_bytes < ely_fp8_recover_workspace_bytes(rows))
            fail(ELY_EWORKSPACE, "ely_fp8_recover_exp: workspace smaller than ely_fp8_recover_workspace_bytes");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const bool bf16 = t_dtype == ELY_BF16;
        const int vpl = recover_vpl(cols, bf16, t, nullptr);
        if (vpl) return recover_rows(vpl, t, bf16, rows, cols, fmt, k, nullptr, bad_rows_dev, s);
        recover_multi(t, bf16, rows, cols, fmt, k, bad_rows_dev, workspace, s);
    });
}

int ely_fp8_recover_image(const void* t, int32_t t_dtype, int64_t rows, int64_t cols, int32_t fmt, int32_t* k,
                          uint8_t* q, unsigned long long* bad_rows_dev, void* workspace, int64_t ws_bytes,
                          void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(t_dtype, "t_dtype");
        check_shape(rows, cols);
        if (rows == 0) return;
        if (!k || !bad_rows_dev || (cols > 0 && (!t || !q))) fail(ELY_EINVAL, "ely_fp8_recover_image: null pointer");
        if (!workspace || ws_bytes < ely_fp8_recover_workspace_bytes(rows))
            fail(ELY_EWORKSPACE, "ely_fp8_recover_image: workspace smaller than ely_fp8_recover_workspace_bytes");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const bool bf16 = t_dtype == ELY_BF16;
        const int vpl = recover_vpl(cols, bf16, t, q);
        if (vpl) return recover_rows(vpl, t, bf16, rows, cols, fmt, k, q, bad_rows_dev, s);
        recover_multi(t, bf16, rows, cols, fmt, k, bad_rows_dev, workspace, s);
        if (cols > 0) quant_k_launch(t, bf16, rows, cols, fmt, k, q, s);
    });
}

int ely_fp8_quantize_k(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt, const int32_t* k,
                       uint8_t* q, void* stream) {
    return guarded([&] {
        check_fmt(fmt);
        check_dtype(x_dtype, "x_dtype");
        check_shape(rows, cols);
        if (rows * cols == 0) return;
        if (!x || !k || !q) fail(ELY_EINVAL, "ely_fp8_quantize_k: null pointer");
        quant_k_launch(x, x_dtype == ELY_BF16, rows, cols, fmt, k, q, static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
