// rows.hip -- the row fold of a tied table's step gradient across stages
// (TiedRowFold, runtime/accumulate.py:140-247).  The stock fold is
// acc = g_0, acc += g_i in microbatch order with g_i = h_i + e_i (autograd's
// sum of the table's two uses, e_i = +0 outside the microbatch's rows), one
// rounding per add in the table's dtype.  TiedRowFold reaches the same bits
// without a dense table per microbatch in flight by folding each row as
// soon as its prefix is complete; every fold it makes is one of
//   acc[idx[j]]  = a[rows_a[j]] + 0.0                  (first, free rows)
//   acc[idx[j]] += a[rows_a[j]] + 0.0                  (later, free rows)
//   acc[idx[j]]  = a[j] + e_j       / acc[idx[j]] += a[j] + e_j
//                                                      (held rows resolved)
// over a set of distinct rows, which this kernel runs: one block per row
// (strided), 16-byte vectors across the row when it is aligned.  e_j is the
// embedding row b[b_rows[j]] of a held row the microbatch touched, +0.0 for
// one it did not (b_rows[j] < 0), or b[j] of a compact b.  A second kernel
// takes a whole Head gradient in one pass: its free rows fold, its held
// rows are copied out bit for bit, so that the gradient itself can go.
#include <algorithm>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {
namespace {

constexpr int kRowBlock = 256;
// one block per row up to this many; longer lists stride
constexpr int64_t kRowGrid = 1 << 16;

typedef float rf4 __attribute__((ext_vector_type(4)));
typedef uint32_t ru4 __attribute__((ext_vector_type(4)));

// v = a + b (b = +0.0 when absent) rounded to the dtype, then acc = v or
// acc + v rounded to the dtype: torch's two elementwise adds.
template <bool BF16>
__device__ __forceinline__ float fold1(float acc, float a, float b, bool first) {
    float v = a + b;
    if (BF16) v = bf16_to_f32(f32_to_bf16(v));
    if (first) return v;
    float s = acc + v;
    if (BF16) s = bf16_to_f32(f32_to_bf16(s));
    return s;
}

constexpr int kRowUnroll = 4;  // 16-byte vectors per thread loaded before the first is stored

// One vector of 4 fp32 or 8 bf16 elements: acc (=|+=) x + y, each add rounded
// to the dtype (y = 0 when the row has no b).
template <bool BF16>
__device__ __forceinline__ ru4 fold_vec(ru4 z, ru4 x, ru4 y, int first) {
    ru4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (BF16) {
            const float lo = fold1<true>(bf16_to_f32(z[k] & 0xFFFFu), bf16_to_f32(x[k] & 0xFFFFu), bf16_to_f32(y[k] & 0xFFFFu), first);
            const float hi = fold1<true>(bf16_to_f32(z[k] >> 16), bf16_to_f32(x[k] >> 16), bf16_to_f32(y[k] >> 16), first);
            o[k] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
        } else {
            o[k] = __float_as_uint(fold1<false>(__uint_as_float(z[k]), __uint_as_float(x[k]), __uint_as_float(y[k]), first));
        }
    }
    return o;
}

// One row of d elements: ac (=|+=) av + (bv or +0.0).  Aligned rows move
// 16-byte vectors, kRowUnroll per thread loaded before any is stored, so a
// row's loads are in flight together; others go element by element.
template <bool BF16>
__device__ __forceinline__ void fold_row(void* ac_, const void* av_, const void* bv_, int64_t d, int first, int vec) {
    if (vec) {
        const int64_t nvec = d / (BF16 ? 8 : 4);
        ru4* ac = static_cast<ru4*>(ac_);
        const ru4* av = static_cast<const ru4*>(av_);
        const ru4* bv = static_cast<const ru4*>(bv_);
        for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)kRowBlock * kRowUnroll) {
            ru4 x[kRowUnroll], y[kRowUnroll], z[kRowUnroll];
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int64_t v = v0 + (int64_t)u * kRowBlock;
                const ru4 zero = {0u, 0u, 0u, 0u};
                x[u] = v < nvec ? av[v] : zero;
                y[u] = (v < nvec && bv) ? bv[v] : zero;
                z[u] = (v < nvec && !first) ? ac[v] : zero;
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int64_t v = v0 + (int64_t)u * kRowBlock;
                if (v < nvec) ac[v] = fold_vec<BF16>(z[u], x[u], y[u], first);
            }
        }
    } else if (BF16) {
        uint16_t* ac = static_cast<uint16_t*>(ac_);
        const uint16_t* av = static_cast<const uint16_t*>(av_);
        const uint16_t* bv = static_cast<const uint16_t*>(bv_);
        for (int64_t c = threadIdx.x; c < d; c += kRowBlock) {
            const float z = first ? 0.0f : bf16_to_f32(ac[c]);
            ac[c] = (uint16_t)f32_to_bf16(fold1<true>(z, bf16_to_f32(av[c]), bv ? bf16_to_f32(bv[c]) : 0.0f, first));
        }
    } else {
        float* ac = static_cast<float*>(ac_);
        const float* av = static_cast<const float*>(av_);
        const float* bv = static_cast<const float*>(bv_);
        for (int64_t c = threadIdx.x; c < d; c += kRowBlock) {
            const float z = first ? 0.0f : ac[c];
            ac[c] = fold1<false>(z, av[c], bv ? bv[c] : 0.0f, first);
        }
    }
}

template <bool BF16>
__global__ __launch_bounds__(kRowBlock) void rows_fold_kernel(void* __restrict__ acc, const void* __restrict__ a,
                                                              const int64_t* __restrict__ a_rows,
                                                              const void* __restrict__ b,
                                                              const int64_t* __restrict__ b_rows,
                                                              const int64_t* __restrict__ idx, int64_t n_idx,
                                                              int64_t n_rows, int64_t a_total, int64_t b_total,
                                                              int64_t d, int first, int vec) {
    const int64_t esz = BF16 ? 2 : 4;
    for (int64_t j = blockIdx.x; j < n_idx; j += gridDim.x) {
        const int64_t r = idx[j];
        const int64_t ar = a_rows ? a_rows[j] : j;
        const int64_t br = b ? (b_rows ? b_rows[j] : j) : -1;  // < 0: the row adds +0.0
        // the host checks every index; a row outside the tables is skipped, never touched
        if (r < 0 || r >= n_rows || ar < 0 || ar >= a_total || br >= b_total) continue;
        fold_row<BF16>(static_cast<char*>(acc) + r * d * esz, static_cast<const char*>(a) + ar * d * esz,
                       br >= 0 ? static_cast<const char*>(b) + br * d * esz : nullptr, d, first, vec);
    }
}

// A row of `bytes` bytes copied bit for bit: 16-byte vectors (kRowUnroll per
// thread in flight) when both rows are aligned, bytes otherwise.
__device__ __forceinline__ void copy_row(char* o, const char* x, int64_t bytes, int vec) {
    if (vec) {
        const int64_t nvec = bytes / 16;
        for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)kRowBlock * kRowUnroll) {
            ru4 t[kRowUnroll];
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int64_t v = v0 + (int64_t)u * kRowBlock;
                if (v < nvec) t[u] = reinterpret_cast<const ru4*>(x)[v];
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int64_t v = v0 + (int64_t)u * kRowBlock;
                if (v < nvec) reinterpret_cast<ru4*>(o)[v] = t[u];
            }
        }
    } else {
        for (int64_t c = threadIdx.x; c < bytes; c += kRowBlock) o[c] = x[c];
    }
}

// A Head gradient in one pass, one block per row: a row r with
// slot[r] < 0 is free and takes acc[r] = a[r] + 0.0 (first) or
// acc[r] + (a[r] + 0.0), each add rounded to the dtype; a held row
// (slot[r] >= 0) is copied to held_out[slot[r]] bit for bit and acc[r] is
// left for its resolve.
template <bool BF16>
__global__ __launch_bounds__(kRowBlock) void rows_split_kernel(void* __restrict__ acc, const void* __restrict__ a,
                                                               const int32_t* __restrict__ slot,
                                                               void* __restrict__ held_out, int64_t n_rows,
                                                               int64_t n_held, int64_t d, int first, int vec) {
    const int64_t row_bytes = d * (BF16 ? 2 : 4);
    for (int64_t r = blockIdx.x; r < n_rows; r += gridDim.x) {
        const int64_t s = slot[r];
        const char* x = static_cast<const char*>(a) + r * row_bytes;
        if (s < 0)
            fold_row<BF16>(static_cast<char*>(acc) + r * row_bytes, x, nullptr, d, first, vec);
        else if (s < n_held)  // the host numbers the held rows 0..n_held-1
            copy_row(static_cast<char*>(held_out) + s * row_bytes, x, row_bytes, vec);
    }
}

}  // namespace
}  // namespace ely

using namespace ely;

extern "C" int ely_rows_fold(void* acc, const void* a, const int64_t* a_rows, const void* b, const int64_t* b_rows,
                             const int64_t* idx, int64_t n_idx, int64_t n_rows, int64_t a_total, int64_t b_total,
                             int64_t d, int32_t dtype, int32_t first, void* stream) {
    return guarded([&] {
        if (dtype != ELY_F32 && dtype != ELY_BF16) fail(ELY_EINVAL, "ely_rows_fold: dtype must be ELY_F32 or ELY_BF16");
        if (n_idx < 0 || n_rows < 0 || a_total < 0 || b_total < 0 || d < 0) fail(ELY_EINVAL, "ely_rows_fold: negative size");
        if (n_idx == 0 || d == 0) return;
        if (!acc || !a || !idx) fail(ELY_EINVAL, "ely_rows_fold: null pointer");
        if (!a_rows && a_total < n_idx) fail(ELY_EINVAL, "ely_rows_fold: a compact source holds one row per index");
        if (b_rows && !b) fail(ELY_EINVAL, "ely_rows_fold: b_rows without b");
        if (b && !b_rows && b_total < n_idx) fail(ELY_EINVAL, "ely_rows_fold: a compact b holds one row per index");
        const int64_t esz = dtype == ELY_BF16 ? 2 : 4;
        const int64_t v = 16 / esz;
        const int vec = (d % v == 0) && aligned16(acc) && aligned16(a) && (!b || aligned16(b)) ? 1 : 0;
        const int64_t blocks = std::min<int64_t>(n_idx, kRowGrid);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (dtype == ELY_BF16)
            hipLaunchKernelGGL(rows_fold_kernel<true>, dim3((unsigned)blocks), dim3(kRowBlock), 0, s, acc, a, a_rows, b,
                               b_rows, idx, n_idx, n_rows, a_total, b ? b_total : 0, d, first ? 1 : 0, vec);
        else
            hipLaunchKernelGGL(rows_fold_kernel<false>, dim3((unsigned)blocks), dim3(kRowBlock), 0, s, acc, a, a_rows, b,
                               b_rows, idx, n_idx, n_rows, a_total, b ? b_total : 0, d, first ? 1 : 0, vec);
        check_launch("rows_fold_kernel");
    });
}

extern "C" int ely_rows_split(void* acc, const void* a, const int32_t* slot, void* held_out, int64_t n_rows,
                              int64_t n_held, int64_t d, int32_t dtype, int32_t first, void* stream) {
    return guarded([&] {
        if (dtype != ELY_F32 && dtype != ELY_BF16) fail(ELY_EINVAL, "ely_rows_split: dtype must be ELY_F32 or ELY_BF16");
        if (n_rows < 0 || n_held < 0 || d < 0) fail(ELY_EINVAL, "ely_rows_split: negative size");
        if (n_held > n_rows) fail(ELY_EINVAL, "ely_rows_split: more held rows than rows");
        if (n_rows == 0 || d == 0) return;
        if (!acc || !a || !slot || (n_held && !held_out)) fail(ELY_EINVAL, "ely_rows_split: null pointer");
        const int64_t v = dtype == ELY_BF16 ? 8 : 4;
        const int vec = (d % v == 0) && aligned16(acc) && aligned16(a) && (!n_held || aligned16(held_out)) ? 1 : 0;
        const int64_t blocks = std::min<int64_t>(n_rows, kRowGrid);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (dtype == ELY_BF16)
            hipLaunchKernelGGL(rows_split_kernel<true>, dim3((unsigned)blocks), dim3(kRowBlock), 0, s, acc, a, slot,
                               held_out, n_rows, n_held, d, first ? 1 : 0, vec);
        else
            hipLaunchKernelGGL(rows_split_kernel<false>, dim3((unsigned)blocks), dim3(kRowBlock), 0, s, acc, a, slot,
                               held_out, n_rows, n_held, d, first ? 1 : 0, vec);
        check_launch("rows_split_kernel");
    });
}
