// mta.hip -- multi-tensor kernels over a stage's ragged parameter shard:
//   (a) the deterministic global grad-norm (sum of squares -> norm -> clip
//       coef), and clip_grad_norm_'s in-place scale over the same tile table
//   (b) the fused clip + AdamW step with the bf16 working copy.
//
// Work decomposition.  Every tensor is cut into fixed tiles (kAdamTile /
// the norm tile of the call, kNormTile or, for lists under 2^29 elements,
// kNormSmallTile; a tensor's last tile may be short) numbered
// consecutively across the list, so the ragged list costs one launch.
// AdamW: one 64-lane block per 256-element tile, each block taking its one
// tile and exiting, so the hardware dispatcher keeps every compute unit
// full of short-lived waves streaming one small window of the shard (C1:
// 5.94 ms against 6.64 for the persistent grid of one 256-thread block per
// CU looping over 4,096-element tiles, and 7.5-8.7 ms for persistent grids
// of these small tiles; 5.81-5.87 ms since with buffer instructions and a
// tile -> tensor chunk map).  Norm: wave
// w takes the contiguous tile range [w*T/W, (w+1)*T/W), its last tiles
// (ELY_NORM_CACHED_MB in all) with plain loads, the rest nontemporal.  A
// table of tensor descriptors is staged into the caller's workspace per
// call.
//
// Determinism of (a): a tile's partial sum is a fixed function of its
// elements (lane l owns the 8-element groups l, l+64, ...; each group is
// squared and summed in fp32 by a fixed tree, groups accumulate in fp64 in
// order, lanes combine by a fixed butterfly), and the final kernel combines
// tile partials in a fixed order.  Neither the grid size nor pointer
// alignment changes a bit of the result.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {

// Compile-time tunables (chosen by measurement on MI355X; see the defaults).
#ifndef ELY_ADAM_TILE
// elements per AdamW tile: one block's work (C1, one-shot grids: 256 with
// 64-lane blocks 5.94 ms, 512 with 128 lanes and 1,024 with 256 lanes
// 6.05, 2,048 6.39, 4,096 6.45, 8,192 6.65)
#define ELY_ADAM_TILE 256
#endif
#ifndef ELY_NORM_SCHED
#define ELY_NORM_SCHED 0         // same choice for the grad-norm waves
#endif
#ifndef ELY_NORM_NT
#define ELY_NORM_NT 1            // nontemporal grad-norm loads
#endif
#ifndef ELY_NORM_CACHED_MB
#define ELY_NORM_CACHED_MB 384   // grad-norm bytes read last with plain loads, to stay in the MALL (norm_partials_body)
#endif
#ifndef ELY_NORM_CACHED_LIMIT_MB
#define ELY_NORM_CACHED_LIMIT_MB 3072  // ... for lists of at most this many bytes; larger ones stay nontemporal
#endif
#ifndef ELY_NORM_UNROLL
#define ELY_NORM_UNROLL 8        // 8-element groups a grad-norm lane loads before summing (divides 32)
#endif
#ifndef ELY_NORM_UNROLL_F32
// the same for fp32 gradients (two 16-byte loads a group): on 4 and 8 GB
// lists 1 group reads 10 % faster than 8 (2: 7 %), small lists the same
#define ELY_NORM_UNROLL_F32 1
#endif
#ifndef ELY_ADAM_MAP_CHUNKS
// entries of the tile -> tensor chunk map a table launch looks its first
// tensor up in (one scalar load instead of a binary search of dependent
// loads over the descriptors)
#define ELY_ADAM_MAP_CHUNKS 4096
#endif
#ifndef ELY_ADAM_BPC
#define ELY_ADAM_BPC (1 << 20)   // AdamW grid cap, blocks per compute unit: in practice one block per tile
#endif
#ifndef ELY_ADAM_MAPPED_BPC
// An AdamW launch whose moments live in pinned host memory, read and
// written in place through the GPU's mapping, is bound by PCIe, not HBM:
// a persistent grid of this many blocks per compute unit keeps the link
// busy.  On C1's shard: 64-256 blocks 203 ms a step (99 GB/s each way),
// 1,024 to 65,536 blocks and the one-shot grid 220 ms; the compute units
// left free also take a concurrent forward's work.
#define ELY_ADAM_MAPPED_BPC 1
#endif
#ifndef ELY_NORM_UNROLL_F32_SMALL
#define ELY_NORM_UNROLL_F32_SMALL 1  // the same for the small tile of a list under ELY_NORM_SMALL_LIMIT elements
#endif
#ifndef ELY_NORM_TILE
#define ELY_NORM_TILE 16384      // grad-norm elements per tile (one wave's share; fixes the summation order)
#endif
#ifndef ELY_NORM_BPC
#define ELY_NORM_BPC 24          // grad-norm blocks (of 4 waves) per compute unit
#endif
#ifndef ELY_FINAL_UNROLL
#define ELY_FINAL_UNROLL 8       // tile partials a thread of the final norm kernel loads before adding (16, 32: slower)
#endif
#ifndef ELY_NORM_SMALL_TILE
#define ELY_NORM_SMALL_TILE 4096  // grad-norm tile of a small list (more waves than its large tiles)
#endif
#ifndef ELY_NORM_SMALL_LIMIT
#define ELY_NORM_SMALL_LIMIT (1LL << 29)  // lists of fewer elements take the small tile
#endif

constexpr int64_t kAdamTile = ELY_ADAM_TILE;
constexpr int64_t kNormTile = ELY_NORM_TILE;  // elements per grad-norm tile (one wave): fixes the summation order
constexpr int64_t kNormSmallTile = ELY_NORM_SMALL_TILE;
static_assert(kNormTile % (64 * 8 * ELY_NORM_UNROLL) == 0 && kNormSmallTile % (64 * 8 * ELY_NORM_UNROLL) == 0,
              "a grad-norm tile is whole unrolled rounds of 8-element groups");
constexpr int kNormUnroll = ELY_NORM_UNROLL;
constexpr int kFinalUnroll = ELY_FINAL_UNROLL;
#ifndef ELY_MTA_BLOCK
#define ELY_MTA_BLOCK 256        // threads per block of the grad-norm and clip-scale kernels
#endif
constexpr int kBlock = ELY_MTA_BLOCK;
#ifndef ELY_ADAM_BLOCK
#define ELY_ADAM_BLOCK 64      // AdamW threads per block: one wave
#endif
constexpr int kAdamBlock = ELY_ADAM_BLOCK;
constexpr int kFinalThreads = 1024;

// --------------------------------------------------------------- (a) norm

// Last tensor whose first tile is <= tile (binary search over the table).
template <class Desc>
__device__ __forceinline__ int find_tensor(const Desc* desc, int n, int64_t tile) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (desc[mid].tile_begin <= tile) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}


struct NormDesc {          // 40 bytes
    const void* g;
    const float* acc;      // FOLD: the fp32 fold of the earlier microbatches
    int64_t numel;
    int64_t tile_begin;
    int32_t dtype;         // ELY_F32 | ELY_BF16
    int32_t aligned;       // g (and acc) 16-byte aligned
};

// Sum of squares of 8 values by a fixed fp32 tree.
__device__ __forceinline__ float sq8(const float (&x)[8]) {
    float s0 = x[0] * x[0], s1 = x[1] * x[1], s2 = x[2] * x[2], s3 = x[3] * x[3];
    float s4 = x[4] * x[4], s5 = x[5] * x[5], s6 = x[6] * x[6], s7 = x[7] * x[7];
    return ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
}

// Pointers read from the descriptor table are generic to the compiler; cast
// them to the global address space so accesses are global_load/global_store
// (flat accesses also count against the LDS/scalar counter and serialize).
#define ELY_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ ELY_GLOBAL T* gp(T* p) {
    return (ELY_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ const ELY_GLOBAL T* gp(const T* p) {
    return (const ELY_GLOBAL T*)p;
}

typedef float nf32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nu32x4 __attribute__((ext_vector_type(4)));

template <typename T, bool NT = ELY_NORM_NT != 0>
__device__ __forceinline__ T ld_norm(const ELY_GLOBAL T* p) {
    if (NT) return __builtin_nontemporal_load(p);
    return *p;
}

// The raw 16-byte vectors of one 8-element group: 1 (bf16) or 2 (fp32)
// gradient vectors, plus 2 accumulator vectors with FOLD.
template <bool BF16, bool FOLD>
struct Raw8 {
    nu32x4 g[BF16 ? 1 : 2];
    nf32x4 a[FOLD ? 2 : 1];
};

template <bool BF16, bool FOLD, bool NT>
__device__ __forceinline__ void raw8_load(const NormDesc& d, int64_t i, Raw8<BF16, FOLD>& r) {
    const ELY_GLOBAL nu32x4* p = gp(reinterpret_cast<const nu32x4*>(static_cast<const char*>(d.g) + i * (BF16 ? 2 : 4)));
    r.g[0] = ld_norm<nu32x4, NT>(p);
    if (!BF16) r.g[BF16 ? 0 : 1] = ld_norm<nu32x4, NT>(p + 1);
    if (FOLD) {
        const ELY_GLOBAL nf32x4* q = gp(reinterpret_cast<const nf32x4*>(d.acc + i));
        r.a[0] = ld_norm<nf32x4, NT>(q);
        r.a[FOLD ? 1 : 0] = ld_norm<nf32x4, NT>(q + 1);
    }
}

// The group's values (acc + widen(g) with FOLD), squared and summed by sq8.
template <bool BF16, bool FOLD>
__device__ __forceinline__ float raw8_sumsq(const Raw8<BF16, FOLD>& r) {
    float x[8];
    if (BF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = bf16_to_f32(r.g[0][j] & 0xFFFFu);
            x[2 * j + 1] = bf16_to_f32(r.g[0][j] >> 16);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = __uint_as_float(r.g[0][j]);
            x[4 + j] = __uint_as_float(r.g[BF16 ? 0 : 1][j]);
        }
    }
    if (FOLD) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = r.a[0][j] + x[j];
            x[4 + j] = r.a[FOLD ? 1 : 0][j] + x[4 + j];
        }
    }
    return sq8(x);
}

// Sum of squares of one full, aligned tile: lane l owns the 8-element groups
// j*64 + l, j = 0..TILE/512-1, added in order; kNormUnroll groups' raw vectors are
// loaded before the first of them is summed.
template <bool BF16, bool FOLD, int64_t TILE, bool NT>
__device__ __forceinline__ double tile_sumsq_vec(const NormDesc& d, int64_t e0, int lane) {
    constexpr int G = (int)(TILE / (kWave * 8));
    constexpr int U = BF16 ? kNormUnroll : (TILE == kNormSmallTile ? ELY_NORM_UNROLL_F32_SMALL : ELY_NORM_UNROLL_F32);
    static_assert(G % U == 0, "unroll divides the groups of a tile");
    double acc = 0.0;
    for (int j0 = 0; j0 < G; j0 += U) {
        Raw8<BF16, FOLD> r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) raw8_load<BF16, FOLD, NT>(d, e0 + ((int64_t)(j0 + u) * kWave + lane) * 8, r[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) acc += (double)raw8_sumsq<BF16, FOLD>(r[u]);
    }
    return acc;
}

// The same 8 values element by element (0 past `end`): any alignment.
template <bool FOLD>
__device__ __forceinline__ void load8_any(const NormDesc& d, int64_t i, int64_t end, float (&x)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t e = i + j;
        float v = 0.0f;
        if (e < end) {
            v = d.dtype == ELY_BF16 ? bf16_to_f32(*gp(static_cast<const uint16_t*>(d.g) + e))
                                    : *gp(static_cast<const float*>(d.g) + e);
            if (FOLD) v = *gp(d.acc + e) + v;
        }
        x[j] = v;
    }
}

// DT: the gradients' dtype when one call's are all ELY_F32 or all ELY_BF16
// (the tile loop is then compiled for that dtype only, which keeps the
// kernel's registers, and so its occupancy, to what that dtype needs), or -1
// for a mixed list, dispatched per tile.
// A norm call of at most kNormArgTensors gradients carries its descriptors
// in the kernel arguments (40 bytes each, 1,920 in all), as a short AdamW
// list does: no table copy ahead of the launch.  Longer lists read the
// table uploaded to the workspace.
constexpr int kNormArgTensors = 48;
struct NormArgTable {
    NormDesc d[kNormArgTensors];
};

// One wave's tiles `tile`, tile + tstep, ... below `to`: each tile's
// partial sum of squares, with nontemporal (NT) or plain loads.  Advances
// `tile` and the tensor index `ti`.
template <bool FOLD, int DT, int64_t TILE, bool NT, class Desc>
__device__ __forceinline__ void norm_tiles(const Desc* desc, int32_t n, int64_t& tile, int64_t to, int64_t tstep,
                                           int& ti, int lane, double* partials) {
    for (; tile < to; tile += tstep) {
        while (ti + 1 < n && desc[ti + 1].tile_begin <= tile) ++ti;
        const NormDesc d = desc[ti];
        const int64_t e0 = (tile - d.tile_begin) * TILE;
        const int64_t e1 = min(e0 + TILE, d.numel);
        double acc = 0.0;
        // lane l owns groups j*64 + l of 8 elements, in the same order on both paths
        if (d.aligned && e1 - e0 == TILE) {
            if (DT == ELY_BF16 || (DT < 0 && d.dtype == ELY_BF16)) acc = tile_sumsq_vec<true, FOLD, TILE, NT>(d, e0, lane);
            else acc = tile_sumsq_vec<false, FOLD, TILE, NT>(d, e0, lane);
        } else {
            for (int j = 0; j < (int)(TILE / (kWave * 8)); ++j) {
                float x[8];
                load8_any<FOLD>(d, e0 + ((int64_t)j * kWave + lane) * 8, e1, x);
                acc += (double)sq8(x);
            }
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) partials[tile] = acc;
    }
}

// The last tiles each wave reads, about ELY_NORM_CACHED_MB of the call's
// bytes in all, take plain loads, so that they are still in the MALL when
// the update (or the clip's scale) reads the same gradients next: each
// wave's last cached_q tiles, and one more for the last cached_r waves (the
// last dispatched, when a wave takes one tile).
// The two kinds of tiles run as two loops in sequence (one loop choosing
// per tile let the compiler merge both kinds into plain loads).  The bits
// do not depend on it.
template <bool FOLD, int DT, int64_t TILE, class Desc>
__device__ __forceinline__ void norm_partials_body(const Desc* desc, int32_t n, int64_t total_tiles, int64_t cached_q,
                                                   int64_t cached_r, double* partials) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t waves = (int64_t)gridDim.x * (kBlock / kWave);
    const int64_t w = (int64_t)blockIdx.x * (kBlock / kWave) + wave_uniform(threadIdx.x / kWave);
#if ELY_NORM_SCHED == 0
    const int64_t t0 = w * total_tiles / waves, t1 = (w + 1) * total_tiles / waves, tstep = 1;
#else
    const int64_t t0 = w, t1 = total_tiles, tstep = waves;
#endif
    if (t0 >= t1) return;
    const int64_t cached_from = t1 - (cached_q + (w >= waves - cached_r ? 1 : 0)) * tstep;
    int64_t tile = t0;
    int ti = find_tensor(desc, n, t0);
    norm_tiles<FOLD, DT, TILE, ELY_NORM_NT != 0>(desc, n, tile, cached_from, tstep, ti, lane, partials);
    norm_tiles<FOLD, DT, TILE, false>(desc, n, tile, t1, tstep, ti, lane, partials);
}

template <bool FOLD, int DT, int64_t TILE>
__global__ __launch_bounds__(kBlock) void norm_partials_kernel(const NormDesc* __restrict__ desc, int32_t n,
                                                               int64_t total_tiles, int64_t cached_q, int64_t cached_r,
                                                               double* __restrict__ partials) {
    norm_partials_body<FOLD, DT, TILE>(desc, n, total_tiles, cached_q, cached_r, partials);
}

template <bool FOLD, int DT, int64_t TILE>
__global__ __launch_bounds__(kBlock) void norm_partials_args_kernel(const NormArgTable tab, int32_t n,
                                                                    int64_t total_tiles, int64_t cached_q,
                                                                    int64_t cached_r, double* __restrict__ partials) {
    norm_partials_body<FOLD, DT, TILE>(tab.d, n, total_tiles, cached_q, cached_r, partials);
}

__global__ __launch_bounds__(kFinalThreads) void norm_final_kernel(const double* __restrict__ partials, int64_t tiles,
                                                                   float max_norm, ely_norm_result* out) {
    __shared__ double red[kFinalThreads];
    double s = 0.0;
    int64_t i = threadIdx.x;
    // partials i, i + 1024, ... added in that order; kFinalUnroll loads in flight
    for (; i + (kFinalUnroll - 1) * kFinalThreads < tiles; i += kFinalUnroll * kFinalThreads) {
        double v[kFinalUnroll];
#pragma unroll
        for (int u = 0; u < kFinalUnroll; ++u) v[u] = partials[i + u * kFinalThreads];
#pragma unroll
        for (int u = 0; u < kFinalUnroll; ++u) s += v[u];
    }
    for (; i < tiles; i += kFinalThreads) s += partials[i];
    red[threadIdx.x] = s;
    for (int o = kFinalThreads / 2; o > 0; o >>= 1) {
        __syncthreads();
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    }
    if (threadIdx.x == 0) {
        const double sumsq = red[0];
        const float norm = (float)sqrt(sumsq);
        // clip_grad.py:165-169: max_norm / (norm + 1e-6) is torch's scalar
        // __rdiv__, (norm + 1e-6).reciprocal() * max_norm, then clamp(max=1)
        // keeping NaN; for any max_norm, as torch (0 zeroes the gradients)
        const float denom = norm + 1e-6f;
        const float r = 1.0f / denom;
        float coef = r * max_norm;
        coef = coef > 1.0f ? 1.0f : coef;
        out->sumsq = sumsq;
        out->norm = norm;
        out->coef = coef;
    }
}

#ifndef ELY_CLIP_BPC
#define ELY_CLIP_BPC 65536   // clip scale: blocks (of 4 waves) per compute unit, in practice one wave per tile (C1's
                                     // 192 bf16 gradients 4.93 -> 5.32 TB/s against 4 per CU)
#endif
#ifndef ELY_CLIP_UNROLL
#define ELY_CLIP_UNROLL 2    // clip scale: 16-byte vectors a lane loads before storing
#endif

// g <- g * coef in place, rounded once to g's dtype (torch's
// _foreach_mul_(grads, clip_coef), clip_grad.py:170-177), over the norm's
// own tile table: wave w scales tiles w, w + W, ...  A full, aligned tile
// moves 16-byte vectors, lane l taking vectors l, l + 64, ...; others go
// element by element.  DT as norm_partials_kernel.
template <int DT, int64_t TILE, class Desc>
__device__ __forceinline__ void clip_scale_body(const Desc* desc, int32_t n, int64_t total_tiles, const float* coef_ptr) {
    constexpr int U = ELY_CLIP_UNROLL;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t waves = (int64_t)gridDim.x * (kBlock / kWave);
    const int64_t w = (int64_t)blockIdx.x * (kBlock / kWave) + wave_uniform(threadIdx.x / kWave);
    if (w >= total_tiles) return;
    const float coef = *coef_ptr;
    int ti = find_tensor(desc, n, w);
    for (int64_t tile = w; tile < total_tiles; tile += waves) {
        while (ti + 1 < n && desc[ti + 1].tile_begin <= tile) ++ti;
        const NormDesc d = desc[ti];
        const bool bf16 = DT == ELY_BF16 || (DT < 0 && d.dtype == ELY_BF16);
        const int64_t e0 = (tile - d.tile_begin) * TILE;
        const int64_t e1 = min(e0 + TILE, d.numel);
        if (d.aligned && e1 - e0 == TILE) {
            nu32x4* base = reinterpret_cast<nu32x4*>(static_cast<char*>(const_cast<void*>(d.g)) + e0 * (bf16 ? 2 : 4));
            const int nvec = (int)(TILE * (bf16 ? 2 : 4) / 16);
            for (int j0 = 0; j0 < nvec; j0 += kWave * U) {
                nu32x4 r[U];
#pragma unroll
                for (int u = 0; u < U; ++u) r[u] = ld_norm(gp(base + j0 + u * kWave + lane));
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    nu32x4 o;
                    if (bf16) {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            o[k] = f32_to_bf16(bf16_to_f32(r[u][k] & 0xFFFFu) * coef) |
                                   (f32_to_bf16(bf16_to_f32(r[u][k] >> 16) * coef) << 16);
                    } else {
#pragma unroll
                        for (int k = 0; k < 4; ++k) o[k] = __float_as_uint(__uint_as_float(r[u][k]) * coef);
                    }
                    __builtin_nontemporal_store(o, gp(base + j0 + u * kWave + lane));
                }
            }
        } else if (bf16) {
            uint16_t* g = static_cast<uint16_t*>(const_cast<void*>(d.g));
            for (int64_t e = e0 + lane; e < e1; e += kWave) g[e] = (uint16_t)f32_to_bf16(bf16_to_f32(g[e]) * coef);
        } else {
            float* g = static_cast<float*>(const_cast<void*>(d.g));
            for (int64_t e = e0 + lane; e < e1; e += kWave) g[e] = g[e] * coef;
        }
    }
}

template <int DT, int64_t TILE>
__global__ __launch_bounds__(kBlock) void clip_scale_kernel(const NormDesc* __restrict__ desc, int32_t n,
                                                            int64_t total_tiles, const float* __restrict__ coef_ptr) {
    clip_scale_body<DT, TILE>(desc, n, total_tiles, coef_ptr);
}

template <int DT, int64_t TILE>
__global__ __launch_bounds__(kBlock) void clip_scale_args_kernel(const NormArgTable tab, int32_t n, int64_t total_tiles,
                                                                 const float* __restrict__ coef_ptr) {
    clip_scale_body<DT, TILE>(tab.d, n, total_tiles, coef_ptr);
}

static_assert((kNormSmallTile * 2 / 16) % (64 * ELY_CLIP_UNROLL) == 0,
              "a full clip tile is whole unrolled rounds of 16-byte vectors");

// The tile of one call, a function of the list alone (never of the grid, so
// the result stays bitwise reproducible): lists under ELY_NORM_SMALL_LIMIT
// elements take the small tile, which gives them enough waves to fill the
// chip.
static int64_t norm_tile(const ely_tensor* grads, int32_t n) {
    int64_t total = 0;
    for (int32_t i = 0; i < n; ++i) total += std::max<int64_t>(grads[i].numel, 0);
    return total < ELY_NORM_SMALL_LIMIT ? kNormSmallTile : kNormTile;
}

static int64_t norm_tiles(const ely_tensor* grads, int32_t n, int64_t tile) {
    int64_t t = 0;
    for (int32_t i = 0; i < n; ++i) t += (std::max<int64_t>(grads[i].numel, 0) + tile - 1) / tile;
    return t;
}

static size_t norm_table_bytes(int32_t n) { return align_up((size_t)n * sizeof(NormDesc), 256); }

typedef void (*NormKernel)(const NormDesc*, int32_t, int64_t, int64_t, int64_t, double*);
typedef void (*NormArgsKernel)(const NormArgTable, int32_t, int64_t, int64_t, int64_t, double*);

template <int64_t TILE>
static NormKernel pick_norm(bool fold, int dt) {
    if (fold)
        return dt == ELY_BF16 ? norm_partials_kernel<true, ELY_BF16, TILE>
                              : dt == ELY_F32 ? norm_partials_kernel<true, ELY_F32, TILE> : norm_partials_kernel<true, -1, TILE>;
    return dt == ELY_BF16 ? norm_partials_kernel<false, ELY_BF16, TILE>
                          : dt == ELY_F32 ? norm_partials_kernel<false, ELY_F32, TILE> : norm_partials_kernel<false, -1, TILE>;
}

template <int64_t TILE>
static NormArgsKernel pick_norm_args(bool fold, int dt) {
    if (fold)
        return dt == ELY_BF16 ? norm_partials_args_kernel<true, ELY_BF16, TILE>
                              : dt == ELY_F32 ? norm_partials_args_kernel<true, ELY_F32, TILE>
                                              : norm_partials_args_kernel<true, -1, TILE>;
    return dt == ELY_BF16 ? norm_partials_args_kernel<false, ELY_BF16, TILE>
                          : dt == ELY_F32 ? norm_partials_args_kernel<false, ELY_F32, TILE>
                                          : norm_partials_args_kernel<false, -1, TILE>;
}

// ------------------------------------------------------------- (b) AdamW

struct AdamDesc {          // 64 bytes
    float* p;
    const void* g;
    const float* acc;      // FOLD: the fp32 fold of the earlier microbatches
    float* m;
    float* v;
    uint16_t* copy;        // bf16 working copy or null
    int64_t numel;
    int32_t tile_begin;    // the launch checks that its tiles fit int32
    int32_t aligned;       // every pointer 16-byte aligned
};
static_assert(sizeof(AdamDesc) == 64, "AdamDesc is 64 bytes");

// Where a launch's descriptors and constants live.  A list of many tensors
// (or with per-tensor constants) reads them from a table uploaded to the
// workspace; a short list whose tensors share one set of constants (every
// tensor at the same step) carries them in the kernel arguments, by value, so
// the launch needs no table copy ahead of it: 48 descriptors of 64 bytes and
// one 32-byte constant block, 3,104 bytes, inside the 4 KB of arguments a
// dispatch takes.
struct AdamTableRef {
    const AdamDesc* d;
    const ely_adamw_consts* c;
    const int32_t* map;  // tensor holding the first tile of each 2^shift-tile chunk, or null
    int32_t shift;
    __device__ __forceinline__ const ely_adamw_consts& consts(int i) const { return c[i]; }
    // a tensor at or before the one holding `tile` (the caller walks forward)
    __device__ __forceinline__ int start(int n, int64_t tile) const {
        return map ? map[tile >> shift] : find_tensor(d, n, tile);
    }
};
constexpr int kArgTensors = 48;
struct AdamArgTable {
    AdamDesc d[kArgTensors];
    ely_adamw_consts c;
    __device__ __forceinline__ const ely_adamw_consts& consts(int) const { return c; }
    __device__ __forceinline__ int start(int n, int64_t tile) const { return find_tensor(d, n, tile); }
};

template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
struct AdamOp {
    __device__ __forceinline__ static void moments(float g, float& m, float& v, const ely_adamw_consts& c,
                                                   float coef) {
        if (CLIP) g = g * coef;
        if (ORDER == ELY_ORDER_HOST) adamw_host_moments(g, m, v, *reinterpret_cast<const HostConsts*>(&c));
        else adamw_torch_moments(g, m, v, *reinterpret_cast<const TorchConsts*>(&c));
    }
    __device__ __forceinline__ static void param(float& p, float m, float v, const ely_adamw_consts& c) {
        if (ORDER == ELY_ORDER_HOST) adamw_host_param(p, m, v, *reinterpret_cast<const HostConsts*>(&c), WD);
        else adamw_torch_param(p, m, v, *reinterpret_cast<const TorchConsts*>(&c), WD);
    }
    __device__ __forceinline__ static void elem(float& p, float g, float& m, float& v, const ely_adamw_consts& c,
                                                float coef) {
        moments(g, m, v, c, coef);
        param(p, m, v, c);
    }
};

// The vector path works in block steps of kStep = 4 * kAdamBlock elements:
// lane t owns the quad [4t, 4t+4) of a step, so each load or store
// instruction of the wave covers one contiguous 1 KB (fp32) or 512 B (bf16)
// run, full aligned lines.  Its loads and stores are buffer instructions
// on resources whose base is the range's first element (the descriptor
// words in scalar registers, one 32-bit lane offset per access, accesses
// past the range's bytes dropped by the hardware), all with the
// nontemporal hint: C1's launch ran 1.5-2 % faster than with the same
// accesses as global instructions on 64-bit lane addresses.
constexpr int64_t kStep = (int64_t)kAdamBlock * 4;
static_assert(kAdamTile % kStep == 0, "an AdamW tile is a whole number of block steps");

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
constexpr int kBufNT = 2;  // cache-policy operand of the buffer accesses: nt

// Buffer resource over `bytes` bytes from `base` (raw, stride 0; the third
// word the CDNA3/4 buffer format takes for untyped 32-bit data).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ i32x4 bits4(const float (&x)[4]) {
    return i32x4{__float_as_int(x[0]), __float_as_int(x[1]), __float_as_int(x[2]), __float_as_int(x[3])};
}

// Whole block steps of elements [e0, e0 + steps * kStep) of an aligned tensor.
template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
__device__ __forceinline__ void adam_steps(const AdamDesc& d, const ely_adamw_consts& c, float coef, int64_t e0,
                                           int64_t steps) {
    using Op = AdamOp<BF16G, ORDER, WD, CLIP, FOLD>;
    const int32_t ne = (int32_t)(steps * kStep);  // a tile's range: at most kAdamTile elements
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(d.p + e0, ne * 4), rm = buf_rsrc(d.m + e0, ne * 4),
                                 rv = buf_rsrc(d.v + e0, ne * 4);
    const __amdgpu_buffer_rsrc_t rg = BF16G ? buf_rsrc(static_cast<const uint16_t*>(d.g) + e0, ne * 2)
                                            : buf_rsrc(static_cast<const float*>(d.g) + e0, ne * 4);
    const __amdgpu_buffer_rsrc_t ra = FOLD ? buf_rsrc(d.acc + e0, ne * 4) : rp;
    const __amdgpu_buffer_rsrc_t rc = d.copy ? buf_rsrc(d.copy + e0, ne * 2) : rp;
    for (int64_t s = 0; s < steps; ++s) {
        const int32_t o = (int32_t)(s * kStep) + (int32_t)threadIdx.x * 4;  // the lane's first element
        // g (and the fold's accumulator), m and v are loaded ahead of p: the
        // moments need only those, and m and v are stored before the sqrt
        // and the division that p waits for (C1, alternating fresh
        // processes, against loading p first and storing p, m, v after both
        // halves: faster in 8 of 8 pairs in two sessions, 0.4-0.6 %, and
        // even in a third)
        i32x2 gw = {0, 0};
        i32x4 ga = {0, 0, 0, 0}, A = {0, 0, 0, 0};
        if (BF16G) gw = __builtin_amdgcn_raw_buffer_load_b64(rg, o * 2, 0, kBufNT);
        else ga = __builtin_amdgcn_raw_buffer_load_b128(rg, o * 4, 0, kBufNT);
        if (FOLD) A = __builtin_amdgcn_raw_buffer_load_b128(ra, o * 4, 0, kBufNT);
        const i32x4 M = __builtin_amdgcn_raw_buffer_load_b128(rm, o * 4, 0, kBufNT);
        const i32x4 V = __builtin_amdgcn_raw_buffer_load_b128(rv, o * 4, 0, kBufNT);
        const i32x4 P = __builtin_amdgcn_raw_buffer_load_b128(rp, o * 4, 0, kBufNT);
        float g[4];
        if (BF16G) {
            g[0] = bf16_to_f32((uint32_t)gw[0] & 0xFFFFu);
            g[1] = bf16_to_f32((uint32_t)gw[0] >> 16);
            g[2] = bf16_to_f32((uint32_t)gw[1] & 0xFFFFu);
            g[3] = bf16_to_f32((uint32_t)gw[1] >> 16);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) g[j] = __int_as_float(ga[j]);
        }
        if (FOLD) {
            // the last microbatch folded in: acc + widen(g), one fp32 rounding
#pragma unroll
            for (int j = 0; j < 4; ++j) g[j] = __int_as_float(A[j]) + g[j];
        }
        float p[4], m[4], v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            m[j] = __int_as_float(M[j]);
            v[j] = __int_as_float(V[j]);
            Op::moments(g[j], m[j], v[j], c, coef);
        }
        __builtin_amdgcn_raw_buffer_store_b128(bits4(m), rm, o * 4, 0, kBufNT);
        __builtin_amdgcn_raw_buffer_store_b128(bits4(v), rv, o * 4, 0, kBufNT);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[j] = __int_as_float(P[j]);
            Op::param(p[j], m[j], v[j], c);
        }
        __builtin_amdgcn_raw_buffer_store_b128(bits4(p), rp, o * 4, 0, kBufNT);
        if (d.copy) {
            const i32x2 w = {(int32_t)(f32_to_bf16(p[0]) | (f32_to_bf16(p[1]) << 16)),
                             (int32_t)(f32_to_bf16(p[2]) | (f32_to_bf16(p[3]) << 16))};
            __builtin_amdgcn_raw_buffer_store_b64(w, rc, o * 2, 0, kBufNT);
        }
    }
}

template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
__device__ __forceinline__ void adam_range(const AdamDesc& d, const ely_adamw_consts& c, float coef, int64_t e0,
                                           int64_t e1) {
    using Op = AdamOp<BF16G, ORDER, WD, CLIP, FOLD>;
    int64_t done = e0;
    if (d.aligned) {
        const int64_t steps = (e1 - e0) / kStep;
        if (steps > 0) adam_steps<BF16G, ORDER, WD, CLIP, FOLD>(d, c, coef, e0, steps);
        done = e0 + steps * kStep;
    }
    // Scalar path: unaligned tensors entirely, aligned tensors' last partial step.
    for (int64_t i = done + threadIdx.x; i < e1; i += kAdamBlock) {
        float p = *gp(d.p + i), m = *gp(d.m + i), v = *gp(d.v + i);
        float g = BF16G ? bf16_to_f32(*gp(static_cast<const uint16_t*>(d.g) + i)) : *gp(static_cast<const float*>(d.g) + i);
        if (FOLD) g = *gp(d.acc + i) + g;
        Op::elem(p, g, m, v, c, coef);
        *gp(d.p + i) = p;
        *gp(d.m + i) = m;
        *gp(d.v + i) = v;
        if (d.copy) *gp(d.copy + i) = (uint16_t)f32_to_bf16(p);
    }
}

template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD, class Tab>
__device__ __forceinline__ void adamw_body(const Tab& tab, int32_t n, int64_t total_tiles, const float* coef_ptr) {
    const int64_t G = gridDim.x;
    const int64_t b = blockIdx.x;
    const float coef = CLIP ? *coef_ptr : 1.0f;
    // interleaved: in round r block b takes tile r*G + b, so at any moment the
    // whole grid streams one contiguous window of the shard
    if (b >= total_tiles) return;
    int ti = tab.start(n, b);
    for (int64_t tile = b; tile < total_tiles; tile += G) {
        while (ti + 1 < n && tab.d[ti + 1].tile_begin <= tile) ++ti;
        const AdamDesc d = tab.d[ti];
        const int64_t e0 = (tile - d.tile_begin) * kAdamTile;
        const int64_t e1 = min(e0 + kAdamTile, d.numel);
        const ely_adamw_consts c = tab.consts(ti);
        adam_range<BF16G, ORDER, WD, CLIP, FOLD>(d, c, coef, e0, e1);
    }
}

// The table kernel takes its tables as __restrict__ pointers: the compiler
// then knows the update's stores never touch them and keeps descriptors and
// constants in scalar registers (without it: 150 VGPRs against 125 and a 2 %
// slower C1 launch).  The argument kernel's tables sit in the kernel-argument
// segment, which is constant memory.
template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
__global__ __launch_bounds__(kAdamBlock) void adamw_kernel(const AdamDesc* __restrict__ desc,
                                                       const ely_adamw_consts* __restrict__ consts,
                                                       const int32_t* __restrict__ map, int32_t shift, int32_t n,
                                                       int64_t total_tiles, const float* __restrict__ coef_ptr) {
    adamw_body<BF16G, ORDER, WD, CLIP, FOLD>(AdamTableRef{desc, consts, map, shift}, n, total_tiles, coef_ptr);
}

template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
__global__ __launch_bounds__(kAdamBlock) void adamw_args_kernel(const AdamArgTable tab, int32_t n, int64_t total_tiles,
                                                            const float* __restrict__ coef_ptr) {
    adamw_body<BF16G, ORDER, WD, CLIP, FOLD>(tab, n, total_tiles, coef_ptr);
}

typedef void (*AdamKernel)(const AdamDesc*, const ely_adamw_consts*, const int32_t*, int32_t, int32_t, int64_t,
                           const float*);
typedef void (*AdamArgsKernel)(const AdamArgTable, int32_t, int64_t, const float*);

template <bool BF16G, int ORDER, bool WD, bool CLIP, bool FOLD>
struct AdamKernels {
    static constexpr AdamKernel table = adamw_kernel<BF16G, ORDER, WD, CLIP, FOLD>;
    static constexpr AdamArgsKernel args = adamw_args_kernel<BF16G, ORDER, WD, CLIP, FOLD>;
};

template <bool BF16G, int ORDER, bool FOLD, class K>
static K pick_adam(bool wd, bool clip) {
    constexpr bool A = std::is_same<K, AdamArgsKernel>::value;
    if (wd) {
        if (clip) return A ? (K)AdamKernels<BF16G, ORDER, true, true, FOLD>::args : (K)AdamKernels<BF16G, ORDER, true, true, FOLD>::table;
        return A ? (K)AdamKernels<BF16G, ORDER, true, false, FOLD>::args : (K)AdamKernels<BF16G, ORDER, true, false, FOLD>::table;
    }
    if (clip) return A ? (K)AdamKernels<BF16G, ORDER, false, true, FOLD>::args : (K)AdamKernels<BF16G, ORDER, false, true, FOLD>::table;
    return A ? (K)AdamKernels<BF16G, ORDER, false, false, FOLD>::args : (K)AdamKernels<BF16G, ORDER, false, false, FOLD>::table;
}

constexpr int kMapChunks = ELY_ADAM_MAP_CHUNKS;
static size_t adam_table_bytes(int32_t n) {
    return align_up((size_t)n * sizeof(AdamDesc), 256) + align_up((size_t)n * sizeof(ely_adamw_consts), 256) +
           (size_t)kMapChunks * sizeof(int32_t);
}

static void check_list(const ely_tensor* t, int32_t n, const char* what) {
    if (n < 0) fail(ELY_EINVAL, std::string(what) + ": negative tensor count");
    if (n > 0 && !t) fail(ELY_EINVAL, std::string(what) + ": null tensor list");
    for (int32_t i = 0; i < n; ++i) {
        if (t[i].numel < 0) fail(ELY_EINVAL, std::string(what) + ": negative numel");
        if (t[i].numel > 0 && !t[i].ptr) fail(ELY_EINVAL, std::string(what) + ": null pointer");
        if (t[i].dtype != ELY_F32 && t[i].dtype != ELY_BF16)
            fail(ELY_EINVAL, std::string(what) + ": dtype must be ELY_F32 or ELY_BF16");
    }
}

// Fold accumulators: fp32, one per gradient, of its numel.
static void check_folds(const ely_tensor* accs, const ely_tensor* grads, int32_t n, const char* what) {
    for (int32_t i = 0; i < n; ++i) {
        if (accs[i].dtype != ELY_F32 || accs[i].numel != grads[i].numel)
            fail(ELY_EINVAL, std::string(what) + ": accumulator " + std::to_string(i) + " must be fp32 of the gradient's numel");
        if (accs[i].numel > 0 && !accs[i].ptr) fail(ELY_EINVAL, std::string(what) + ": null accumulator pointer");
    }
}

template <bool FOLD, class K>
static K pick_adam_order(bool bf16g, int32_t order, bool wd, bool clip) {
    if (bf16g)
        return order == ELY_ORDER_HOST ? pick_adam<true, ELY_ORDER_HOST, FOLD, K>(wd, clip)
                                       : pick_adam<true, ELY_ORDER_TORCH, FOLD, K>(wd, clip);
    return order == ELY_ORDER_HOST ? pick_adam<false, ELY_ORDER_HOST, FOLD, K>(wd, clip)
                                   : pick_adam<false, ELY_ORDER_TORCH, FOLD, K>(wd, clip);
}

template <class K>
static K pick_adam_kernel(bool fold, bool bf16g, int32_t order, bool wd, bool clip) {
    return fold ? pick_adam_order<true, K>(bf16g, order, wd, clip) : pick_adam_order<false, K>(bf16g, order, wd, clip);
}

}  // namespace ely

using namespace ely;

// ws query used by the implementations below
extern "C" int64_t ely_grad_norm_workspace_bytes(const ely_tensor* grads, int32_t n);
extern "C" int64_t ely_adamw_workspace_bytes(int32_t n);

namespace ely {

// What a norm call left in the workspace for a clip scale to reuse.
struct NormLaunch {
    const NormDesc* dtable = nullptr;  // the uploaded table, or null when the call's descriptors went by argument
    NormArgTable args;                 // the descriptors themselves for a short list
    int32_t entries = 0;
    int64_t tiles = 0, tile = 0;
    int dt = -1;
};

// The norm of grads (FOLD: of accs[i] + widen(grads[i])): see ely_grad_norm.
static NormLaunch grad_norm_impl(const ely_tensor* accs, const ely_tensor* grads, int32_t n, float max_norm,
                                 ely_norm_result* out_dev, void* workspace, int64_t ws_bytes, void* stream) {
    check_list(grads, n, "ely_grad_norm grads");
    if (accs) check_folds(accs, grads, n, "ely_grad_norm_fold");
    if (!out_dev) fail(ELY_EINVAL, "ely_grad_norm: null result pointer");
    const int64_t need = ely_grad_norm_workspace_bytes(grads, n);
    if (!workspace || ws_bytes < need)
        fail(ELY_EWORKSPACE, "ely_grad_norm: workspace of " + std::to_string(ws_bytes) + " bytes, need " +
                                 std::to_string(need));
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<NormDesc> table;
    table.reserve(n);
    const int64_t tile = norm_tile(grads, n);
    int64_t tiles = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (grads[i].numel == 0) continue;
        NormDesc d;
        d.g = grads[i].ptr;
        d.acc = accs ? static_cast<const float*>(accs[i].ptr) : nullptr;
        d.numel = grads[i].numel;
        d.tile_begin = tiles;
        d.dtype = grads[i].dtype;
        d.aligned = aligned16(grads[i].ptr) && (!accs || aligned16(accs[i].ptr)) ? 1 : 0;
        table.push_back(d);
        tiles += (d.numel + tile - 1) / tile;
    }
    char* ws = static_cast<char*>(workspace);
    NormDesc* dtable = reinterpret_cast<NormDesc*>(ws);
    double* partials = reinterpret_cast<double*>(ws + norm_table_bytes(n));
    NormLaunch out;
    out.entries = (int32_t)table.size();
    out.tiles = tiles;
    out.tile = tile;
    if (tiles > 0) {
        const int64_t waves = std::min<int64_t>(tiles, mt_blocks(ELY_NORM_BPC) * (kBlock / kWave));
        const int64_t blocks = (waves + kBlock / kWave - 1) / (kBlock / kWave);
        int dt = table[0].dtype;
        for (const NormDesc& d : table)
            if (d.dtype != dt) dt = -1;
        out.dt = dt;
        // ~ELY_NORM_CACHED_MB of the last tiles read, spread over the kernel's
        // waves (a list that small is read with plain loads throughout).
        // Measured step (norm + update) against nontemporal loads throughout:
        // C0 (85 MB) -6 %, 256 MB and 1 GB of fp32 gradients -7 % and -3.4 %,
        // C1 (2.5 GB) -0.4 %; 4 and 8 GB lists +0.3 % and 0, so lists past
        // ELY_NORM_CACHED_LIMIT_MB keep nontemporal loads.
        const int64_t tile_bytes = tile * ((dt == ELY_BF16 ? 2 : 4) + (accs ? 4 : 0));
        const int64_t cached = tiles * tile_bytes > ((int64_t)ELY_NORM_CACHED_LIMIT_MB << 20)
                                   ? 0
                                   : ((int64_t)ELY_NORM_CACHED_MB << 20) / tile_bytes;
        const int64_t kwaves = blocks * (kBlock / kWave);
        const int64_t cached_q = cached >= tiles ? tiles : cached / kwaves;
        const int64_t cached_r = cached >= tiles ? 0 : cached % kwaves;
        if (table.size() <= (size_t)kNormArgTensors) {
            memset(&out.args, 0, sizeof out.args);
            memcpy(out.args.d, table.data(), table.size() * sizeof(NormDesc));
            const NormArgsKernel kern = tile == kNormTile ? pick_norm_args<kNormTile>(accs != nullptr, dt)
                                                          : pick_norm_args<kNormSmallTile>(accs != nullptr, dt);
            hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kBlock), 0, s, out.args, (int32_t)table.size(), tiles,
                               cached_q, cached_r, partials);
        } else {
            upload(dtable, table.data(), table.size() * sizeof(NormDesc), s);
            out.dtable = dtable;
            const NormKernel kern = tile == kNormTile ? pick_norm<kNormTile>(accs != nullptr, dt)
                                                      : pick_norm<kNormSmallTile>(accs != nullptr, dt);
            hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kBlock), 0, s, (const NormDesc*)dtable,
                               (int32_t)table.size(), tiles, cached_q, cached_r, partials);
        }
        check_launch("norm_partials_kernel");
    }
    hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(kFinalThreads), 0, s, partials, tiles, max_norm,
                       out_dev);
    check_launch("norm_final_kernel");
    return out;
}

typedef void (*ClipKernel)(const NormDesc*, int32_t, int64_t, const float*);
typedef void (*ClipArgsKernel)(const NormArgTable, int32_t, int64_t, const float*);

template <int64_t TILE>
static ClipKernel pick_clip(int dt) {
    return dt == ELY_BF16 ? clip_scale_kernel<ELY_BF16, TILE>
                          : dt == ELY_F32 ? clip_scale_kernel<ELY_F32, TILE> : clip_scale_kernel<-1, TILE>;
}

template <int64_t TILE>
static ClipArgsKernel pick_clip_args(int dt) {
    return dt == ELY_BF16 ? clip_scale_args_kernel<ELY_BF16, TILE>
                          : dt == ELY_F32 ? clip_scale_args_kernel<ELY_F32, TILE> : clip_scale_args_kernel<-1, TILE>;
}

// Scale every gradient of a finished norm call by its clip coefficient, from
// that call's tile table (uploaded to the workspace, or its descriptors by
// argument again; same stream, so the coefficient is in place when this runs).
static void clip_scale(const NormLaunch& nl, const float* coef_dev, void* stream) {
    if (nl.tiles == 0) return;
    // one wave per tile, in whole blocks; the blocks capped so that the
    // dispatch's work-items stay within 2^32 - 1 (the waves stride past that)
    const int64_t waves = std::min<int64_t>(nl.tiles, mt_blocks(ELY_CLIP_BPC) * (kBlock / kWave));
    const int64_t blocks = std::min<int64_t>((waves + kBlock / kWave - 1) / (kBlock / kWave), 0xFFFFFFFFLL / kBlock);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (nl.dtable) {
        const ClipKernel k = nl.tile == kNormTile ? pick_clip<kNormTile>(nl.dt) : pick_clip<kNormSmallTile>(nl.dt);
        hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kBlock), 0, s, nl.dtable, nl.entries, nl.tiles, coef_dev);
    } else {
        const ClipArgsKernel k = nl.tile == kNormTile ? pick_clip_args<kNormTile>(nl.dt) : pick_clip_args<kNormSmallTile>(nl.dt);
        hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kBlock), 0, s, nl.args, nl.entries, nl.tiles, coef_dev);
    }
    check_launch("clip_scale_kernel");
}

// One fused step (FOLD: the gradient of tensor i is accs[i] + widen(grads[i])).
static void adamw_impl(const ely_tensor* params, const ely_tensor* accs, const ely_tensor* grads,
                       const ely_tensor* exp_avg, const ely_tensor* exp_avg_sq, const ely_tensor* copies, int32_t n,
                       const ely_adamw_consts* consts, int32_t order, int32_t weight_decay_nonzero,
                       const float* coef_dev, void* workspace, int64_t ws_bytes, void* stream) {
    check_list(params, n, "ely_adamw_step params");
    check_list(grads, n, "ely_adamw_step grads");
    if (accs) check_folds(accs, grads, n, "ely_adamw_fold_step");
    check_list(exp_avg, n, "ely_adamw_step exp_avg");
    check_list(exp_avg_sq, n, "ely_adamw_step exp_avg_sq");
    if (order != ELY_ORDER_HOST && order != ELY_ORDER_TORCH)
        fail(ELY_EINVAL, "ely_adamw_step: order must be ELY_ORDER_HOST or ELY_ORDER_TORCH");
    if (n > 0 && !consts) fail(ELY_EINVAL, "ely_adamw_step: null constants");
    const int64_t need = ely_adamw_workspace_bytes(n);
    if (!workspace || ws_bytes < need)
        fail(ELY_EWORKSPACE, "ely_adamw_step: workspace of " + std::to_string(ws_bytes) + " bytes, need " +
                                 std::to_string(need));
    int gdt = -1;
    std::vector<AdamDesc> table;
    std::vector<ely_adamw_consts> cs;
    table.reserve(n);
    cs.reserve(n);
    int64_t tiles = 0;
    for (int32_t i = 0; i < n; ++i) {
        const int64_t ne = params[i].numel;
        if (params[i].dtype != ELY_F32 || exp_avg[i].dtype != ELY_F32 || exp_avg_sq[i].dtype != ELY_F32)
            fail(ELY_EINVAL, "ely_adamw_step: params and moments must be fp32 (tensor " + std::to_string(i) + ")");
        if (grads[i].numel != ne || exp_avg[i].numel != ne || exp_avg_sq[i].numel != ne)
            fail(ELY_EINVAL, "ely_adamw_step: numel mismatch at tensor " + std::to_string(i));
        if (copies && copies[i].ptr) {
            if (copies[i].dtype != ELY_BF16 || copies[i].numel != ne)
                fail(ELY_EINVAL, "ely_adamw_step: working copy " + std::to_string(i) + " must be bf16 of numel " +
                                     std::to_string(ne));
        }
        if (ne == 0) continue;
        if (gdt < 0) gdt = grads[i].dtype;
        else if (gdt != grads[i].dtype)
            fail(ELY_EINVAL, "ely_adamw_step: grads of one call share one dtype");
        AdamDesc d;
        d.p = static_cast<float*>(params[i].ptr);
        d.g = grads[i].ptr;
        d.acc = accs ? static_cast<const float*>(accs[i].ptr) : nullptr;
        d.m = static_cast<float*>(exp_avg[i].ptr);
        d.v = static_cast<float*>(exp_avg_sq[i].ptr);
        d.copy = copies ? static_cast<uint16_t*>(copies[i].ptr) : nullptr;
        d.numel = ne;
        d.tile_begin = (int32_t)tiles;
        d.aligned = aligned16(d.p) && aligned16(d.g) && aligned16(d.m) && aligned16(d.v) &&
                    (!d.copy || aligned16(d.copy)) && (!d.acc || aligned16(d.acc));
        table.push_back(d);
        cs.push_back(consts[i]);
        tiles += (ne + kAdamTile - 1) / kAdamTile;
        if (tiles > INT32_MAX)
            fail(ELY_EINVAL, "ely_adamw_step: more than 2^31 - 1 tiles of " + std::to_string(kAdamTile) +
                                 " elements in one call; split the list");
    }
    if (tiles == 0) return;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool wd = weight_decay_nonzero != 0;
    const bool clip = coef_dev != nullptr;
    // one block per tile, up to the 2^32 - 1 work-items a dispatch counts;
    // a longer list's blocks stride over the rest
    int64_t blocks = std::min<int64_t>({tiles, mt_blocks(ELY_ADAM_BPC), 0xFFFFFFFFLL / kAdamBlock});
    if (ELY_ADAM_MAPPED_BPC > 0 && host_resident(table[0].m))
        blocks = std::min<int64_t>(blocks, (int64_t)device_info().cus * ELY_ADAM_MAPPED_BPC);
    bool shared = true;  // one set of constants for every tensor
    for (const ely_adamw_consts& c : cs) shared = shared && memcmp(&c, &cs[0], sizeof c) == 0;
    if (shared && table.size() <= (size_t)kArgTensors) {
        // a short list at one step: descriptors and constants ride in the kernel arguments
        AdamArgTable at;
        memset(&at, 0, sizeof at);
        memcpy(at.d, table.data(), table.size() * sizeof(AdamDesc));
        at.c = cs[0];
        const AdamArgsKernel k = pick_adam_kernel<AdamArgsKernel>(accs != nullptr, gdt == ELY_BF16, order, wd, clip);
        hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kAdamBlock), 0, s, at, (int32_t)table.size(), tiles, coef_dev);
        check_launch("adamw_kernel");
        return;
    }
    char* ws = static_cast<char*>(workspace);
    AdamDesc* dtable = reinterpret_cast<AdamDesc*>(ws);
    const size_t consts_off = align_up((size_t)n * sizeof(AdamDesc), 256);
    ely_adamw_consts* dconsts = reinterpret_cast<ely_adamw_consts*>(ws + consts_off);
    // One-shot grids (one block per tile) look each block's first tensor up
    // in a chunk map: the tensor holding the first tile of every 2^shift
    // consecutive tiles, at most kMapChunks entries, placed after the
    // constants and uploaded with them (C1: 1.5 % off the launch against a
    // binary search of the descriptors per block).  A capped grid's blocks
    // search the descriptors once each.
    int32_t shift = 0;
    const size_t map_off = align_up(cs.size() * sizeof(ely_adamw_consts), 256);
    std::vector<char> staged(map_off);
    memcpy(staged.data(), cs.data(), cs.size() * sizeof(ely_adamw_consts));
    const bool mapped = blocks == tiles;
    if (mapped) {
        while (((tiles - 1) >> shift) >= kMapChunks) ++shift;
        const int64_t chunks = ((tiles - 1) >> shift) + 1;
        staged.resize(map_off + (size_t)chunks * sizeof(int32_t));
        int32_t* map = reinterpret_cast<int32_t*>(staged.data() + map_off);
        int32_t ti = 0;
        for (int64_t ch = 0; ch < chunks; ++ch) {
            while (ti + 1 < (int32_t)table.size() && table[ti + 1].tile_begin <= (ch << shift)) ++ti;
            map[ch] = ti;
        }
    } else {
        staged.resize(cs.size() * sizeof(ely_adamw_consts));
    }
    // two copies, not one: a single merged copy made the staged host-moment
    // step slower (its small table copies queue behind the moment copies)
    upload(dtable, table.data(), table.size() * sizeof(AdamDesc), s);
    upload(dconsts, staged.data(), staged.size(), s);
    const int32_t* dmap = mapped ? reinterpret_cast<const int32_t*>(ws + consts_off + map_off) : nullptr;
    const AdamKernel k = pick_adam_kernel<AdamKernel>(accs != nullptr, gdt == ELY_BF16, order, wd, clip);
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kAdamBlock), 0, s, (const AdamDesc*)dtable,
                       (const ely_adamw_consts*)dconsts, dmap, shift, (int32_t)table.size(), tiles, coef_dev);
    check_launch("adamw_kernel");
}

}  // namespace ely

extern "C" {

int64_t ely_grad_norm_workspace_bytes(const ely_tensor* grads, int32_t n) {
    if (n < 0 || (n > 0 && !grads)) return -1;
    return (int64_t)(norm_table_bytes(n) +
                     align_up((size_t)std::max<int64_t>(norm_tiles(grads, n, norm_tile(grads, n)), 1) * 8, 256));
}

int ely_grad_norm(const ely_tensor* grads, int32_t n, float max_norm, ely_norm_result* out_dev, void* workspace,
                  int64_t ws_bytes, void* stream) {
    return guarded([&] { grad_norm_impl(nullptr, grads, n, max_norm, out_dev, workspace, ws_bytes, stream); });
}

int ely_grad_norm_clip(const ely_tensor* grads, int32_t n, float max_norm, ely_norm_result* out_dev, void* workspace,
                       int64_t ws_bytes, void* stream) {
    return guarded([&] {
        const NormLaunch nl = grad_norm_impl(nullptr, grads, n, max_norm, out_dev, workspace, ws_bytes, stream);
        clip_scale(nl, &out_dev->coef, stream);
    });
}

int ely_grad_norm_fold(const ely_tensor* accs, const ely_tensor* grads, int32_t n, float max_norm,
                       ely_norm_result* out_dev, void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        if (n > 0 && !accs) fail(ELY_EINVAL, "ely_grad_norm_fold: null accumulator list");
        grad_norm_impl(accs, grads, n, max_norm, out_dev, workspace, ws_bytes, stream);
    });
}

// In-place g <- g * coef over a tensor list: the clip's scale kernel over
// the norm's tiles, with the descriptors in the kernel arguments, one launch
// per kNormArgTensors non-empty tensors (no workspace, no table copy).
int ely_scale_inplace(const ely_tensor* ts, int32_t n, const float* coef_dev, void* stream) {
    return guarded([&] {
        if (n < 0 || (n > 0 && !ts)) fail(ELY_EINVAL, "ely_scale_inplace: bad tensor list");
        if (!coef_dev) fail(ELY_EINVAL, "ely_scale_inplace: null coefficient");
        for (int32_t i = 0; i < n; ++i) {
            if (ts[i].numel < 0 || (ts[i].numel > 0 && !ts[i].ptr)) fail(ELY_EINVAL, "ely_scale_inplace: bad tensor");
            if (ts[i].dtype != ELY_F32 && ts[i].dtype != ELY_BF16) fail(ELY_EINVAL, "ely_scale_inplace: dtype");
        }
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int64_t tile = norm_tile(ts, n);
        NormLaunch nl;
        nl.tile = tile;
        memset(&nl.args, 0, sizeof nl.args);
        auto flush = [&] {
            if (nl.entries == 0) return;
            clip_scale(nl, coef_dev, s);
            nl.entries = 0;
            nl.tiles = 0;
            nl.dt = -2;
            memset(&nl.args, 0, sizeof nl.args);
        };
        nl.dt = -2;  // no tensor yet
        for (int32_t i = 0; i < n; ++i) {
            if (ts[i].numel == 0) continue;
            NormDesc d;
            d.g = ts[i].ptr;
            d.acc = nullptr;
            d.numel = ts[i].numel;
            d.tile_begin = nl.tiles;
            d.dtype = ts[i].dtype;
            d.aligned = aligned16(ts[i].ptr) ? 1 : 0;
            nl.args.d[nl.entries++] = d;
            nl.tiles += (d.numel + tile - 1) / tile;
            nl.dt = nl.dt == -2 ? d.dtype : (nl.dt == d.dtype ? nl.dt : -1);
            if (nl.entries == kNormArgTensors) flush();
        }
        flush();
    });
}

int64_t ely_adamw_workspace_bytes(int32_t n) {
    if (n < 0) return -1;
    return (int64_t)adam_table_bytes(n);
}

int ely_adamw_step(const ely_tensor* params, const ely_tensor* grads, const ely_tensor* exp_avg,
                   const ely_tensor* exp_avg_sq, const ely_tensor* copies, int32_t n, const ely_adamw_consts* consts,
                   int32_t order, int32_t weight_decay_nonzero, const float* coef_dev, void* workspace,
                   int64_t ws_bytes, void* stream) {
    return guarded([&] {
        adamw_impl(params, nullptr, grads, exp_avg, exp_avg_sq, copies, n, consts, order, weight_decay_nonzero, coef_dev,
                   workspace, ws_bytes, stream);
    });
}

int ely_adamw_fold_step(const ely_tensor* params, const ely_tensor* accs, const ely_tensor* grads,
                        const ely_tensor* exp_avg, const ely_tensor* exp_avg_sq, const ely_tensor* copies, int32_t n,
                        const ely_adamw_consts* consts, int32_t order, int32_t weight_decay_nonzero,
                        const float* coef_dev, void* workspace, int64_t ws_bytes, void* stream) {
    return guarded([&] {
        if (n > 0 && !accs) fail(ELY_EINVAL, "ely_adamw_fold_step: null accumulator list");
        adamw_impl(params, accs, grads, exp_avg, exp_avg_sq, copies, n, consts, order, weight_decay_nonzero, coef_dev,
                   workspace, ws_bytes, stream);
    });
}

}  // extern "C"
