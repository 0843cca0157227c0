// mta.hip -- multi-tensor kernels over a stage's ragged parameter shard:
//   (a) the deterministic global grad-norm (sum of squares -> norm -> clip coef)
//   (b) the fused clip + AdamW step with the bf16 working copy.
//
// Work decomposition.  Every tensor is cut into fixed tiles (kAdamTile /
// kNormTile elements; a tensor's last tile may be short) numbered
// consecutively across the list.  A launch gets a persistent grid; block
// (AdamW) or wave (norm) w takes the contiguous tile range
// [w*T/W, (w+1)*T/W), so every worker streams long contiguous runs of one
// or a few tensors and the ragged list costs one launch.  A table of tensor
// descriptors is staged into the caller's workspace per call.
//
// Determinism of (a): a tile's partial sum is a fixed function of its
// elements (lane l owns the 8-element groups l, l+64, ...; each group is
// squared and summed in fp32 by a fixed tree, groups accumulate in fp64 in
// order, lanes combine by a fixed butterfly), and the final kernel combines
// tile partials in a fixed order.  Neither the grid size nor pointer
// alignment changes a bit of the result.
#include <math.h>

#include <algorithm>
#include <vector>

#include "ely_device.hpp"
#include "ely_host.hpp"

#pragma clang fp contract(off)

namespace ely {

constexpr int64_t kAdamTile = 4096;     // elements per AdamW tile
constexpr int64_t kNormTile = 16384;    // elements per grad-norm tile (one wave)
constexpr int kBlock = 256;
constexpr int kFinalThreads = 1024;

// --------------------------------------------------------------- (a) norm

struct NormDesc {          // 32 bytes
    const void* g;
    int64_t numel;
    int64_t tile_begin;
    int32_t dtype;         // ELY_F32 | ELY_BF16
    int32_t aligned;       // g is 16-byte aligned
};

// Sum of squares of 8 values by a fixed fp32 tree.
__device__ __forceinline__ float sq8(const float (&x)[8]) {
    float s0 = x[0] * x[0], s1 = x[1] * x[1], s2 = x[2] * x[2], s3 = x[3] * x[3];
    float s4 = x[4] * x[4], s5 = x[5] * x[5], s6 = x[6] * x[6], s7 = x[7] * x[7];
    return ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
}

__device__ __forceinline__ void load8(const NormDesc& d, int64_t i, int64_t end, float (&x)[8]) {
    if (d.aligned && i + 8 <= end) {
        if (d.dtype == ELY_BF16) {
            uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(d.g) + i);
            uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[2 * j] = bf16_to_f32(ws[j] & 0xFFFFu);
                x[2 * j + 1] = bf16_to_f32(ws[j] >> 16);
            }
        } else {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(d.g) + i);
            float4 a = p[0], b = p[1];
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int64_t e = i + j;
            float v = 0.0f;
            if (e < end) {
                v = d.dtype == ELY_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(d.g)[e])
                                        : static_cast<const float*>(d.g)[e];
            }
            x[j] = v;
        }
    }
}

__global__ __launch_bounds__(kBlock) void norm_partials_kernel(const NormDesc* __restrict__ desc, int32_t n,
                                                               int64_t total_tiles, double* __restrict__ partials) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t waves = (int64_t)gridDim.x * (kBlock / kWave);
    const int64_t w = (int64_t)blockIdx.x * (kBlock / kWave) + wave_uniform(threadIdx.x / kWave);
    const int64_t t0 = w * total_tiles / waves, t1 = (w + 1) * total_tiles / waves;
    if (t0 >= t1) return;
    int lo = 0, hi = n - 1;  // last tensor whose first tile is <= t0
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (desc[mid].tile_begin <= t0) lo = mid;
        else hi = mid - 1;
    }
    int ti = lo;
    for (int64_t tile = t0; tile < t1; ++tile) {
        while (ti + 1 < n && desc[ti + 1].tile_begin <= tile) ++ti;
        const NormDesc d = desc[ti];
        const int64_t e0 = (tile - d.tile_begin) * kNormTile;
        const int64_t e1 = min(e0 + kNormTile, d.numel);
        double acc = 0.0;
#pragma unroll 4
        for (int j = 0; j < (int)(kNormTile / (kWave * 8)); ++j) {
            const int64_t i = e0 + ((int64_t)j * kWave + lane) * 8;
            float x[8];
            load8(d, i, e1, x);
            acc += (double)sq8(x);
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) partials[tile] = acc;
    }
}

__global__ __launch_bounds__(kFinalThreads) void norm_final_kernel(const double* __restrict__ partials, int64_t tiles,
                                                                   float max_norm, ely_norm_result* out) {
    __shared__ double red[kFinalThreads];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < tiles; i += kFinalThreads) s += partials[i];
    red[threadIdx.x] = s;
    for (int o = kFinalThreads / 2; o > 0; o >>= 1) {
        __syncthreads();
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    }
    if (threadIdx.x == 0) {
        const double sumsq = red[0];
        const float norm = (float)sqrt(sumsq);
        float coef = 1.0f;
        if (max_norm > 0.0f) {
            // clip_grad.py:165-169: (norm + 1e-6).reciprocal() * max_norm, clamp(max=1) keeping NaN
            const float denom = norm + 1e-6f;
            const float r = 1.0f / denom;
            coef = r * max_norm;
            coef = coef > 1.0f ? 1.0f : coef;
        }
        out->sumsq = sumsq;
        out->norm = norm;
        out->coef = coef;
    }
}

static int64_t norm_tiles(const ely_tensor* grads, int32_t n) {
    int64_t t = 0;
    for (int32_t i = 0; i < n; ++i) t += (grads[i].numel + kNormTile - 1) / kNormTile;
    return t;
}

static size_t norm_table_bytes(int32_t n) { return align_up((size_t)n * sizeof(NormDesc), 256); }

// ------------------------------------------------------------- (b) AdamW

struct AdamDesc {          // 64 bytes
    float* p;
    const void* g;
    float* m;
    float* v;
    uint16_t* copy;        // bf16 working copy or null
    int64_t numel;
    int64_t tile_begin;
    int32_t aligned;       // every pointer 16-byte aligned
    int32_t pad;
};

template <bool BF16G, int ORDER, bool WD, bool CLIP>
struct AdamOp {
    __device__ __forceinline__ static void elem(float& p, float g, float& m, float& v, const ely_adamw_consts& c,
                                                float coef) {
        if (CLIP) g = g * coef;
        if (ORDER == ELY_ORDER_HOST) {
            adamw_host_elem(p, g, m, v, *reinterpret_cast<const HostConsts*>(&c), WD);
        } else {
            adamw_torch_elem(p, g, m, v, *reinterpret_cast<const TorchConsts*>(&c), WD);
        }
    }
};

template <bool BF16G, int ORDER, bool WD, bool CLIP>
__device__ __forceinline__ void adam_range(const AdamDesc& d, const ely_adamw_consts& c, float coef, int64_t e0,
                                           int64_t e1) {
    using Op = AdamOp<BF16G, ORDER, WD, CLIP>;
    const int64_t vend = e0 + ((e1 - e0) & ~(int64_t)7);
    if (d.aligned) {
        for (int64_t i = e0 + (int64_t)threadIdx.x * 8; i < vend; i += (int64_t)kBlock * 8) {
            float4* pp = reinterpret_cast<float4*>(d.p + i);
            float4* mp = reinterpret_cast<float4*>(d.m + i);
            float4* vp = reinterpret_cast<float4*>(d.v + i);
            float4 p0 = pp[0], p1 = pp[1], m0 = mp[0], m1 = mp[1], v0 = vp[0], v1 = vp[1];
            float g[8];
            if (BF16G) {
                uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(d.g) + i);
                g[0] = bf16_to_f32(w.x & 0xFFFFu); g[1] = bf16_to_f32(w.x >> 16);
                g[2] = bf16_to_f32(w.y & 0xFFFFu); g[3] = bf16_to_f32(w.y >> 16);
                g[4] = bf16_to_f32(w.z & 0xFFFFu); g[5] = bf16_to_f32(w.z >> 16);
                g[6] = bf16_to_f32(w.w & 0xFFFFu); g[7] = bf16_to_f32(w.w >> 16);
            } else {
                const float4* gp = reinterpret_cast<const float4*>(static_cast<const float*>(d.g) + i);
                float4 a = gp[0], b = gp[1];
                g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
                g[4] = b.x; g[5] = b.y; g[6] = b.z; g[7] = b.w;
            }
            float p[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            float m[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) Op::elem(p[j], g[j], m[j], v[j], c, coef);
            pp[0] = make_float4(p[0], p[1], p[2], p[3]);
            pp[1] = make_float4(p[4], p[5], p[6], p[7]);
            mp[0] = make_float4(m[0], m[1], m[2], m[3]);
            mp[1] = make_float4(m[4], m[5], m[6], m[7]);
            vp[0] = make_float4(v[0], v[1], v[2], v[3]);
            vp[1] = make_float4(v[4], v[5], v[6], v[7]);
            if (d.copy) {
                uint4 o;
                o.x = f32_to_bf16(p[0]) | (f32_to_bf16(p[1]) << 16);
                o.y = f32_to_bf16(p[2]) | (f32_to_bf16(p[3]) << 16);
                o.z = f32_to_bf16(p[4]) | (f32_to_bf16(p[5]) << 16);
                o.w = f32_to_bf16(p[6]) | (f32_to_bf16(p[7]) << 16);
                *reinterpret_cast<uint4*>(d.copy + i) = o;
            }
        }
    }
    // Scalar path: unaligned tensors entirely, aligned tensors' last < 8 elements.
    for (int64_t i = (d.aligned ? vend : e0) + threadIdx.x; i < e1; i += kBlock) {
        float p = d.p[i], m = d.m[i], v = d.v[i];
        float g = BF16G ? bf16_to_f32(static_cast<const uint16_t*>(d.g)[i]) : static_cast<const float*>(d.g)[i];
        Op::elem(p, g, m, v, c, coef);
        d.p[i] = p;
        d.m[i] = m;
        d.v[i] = v;
        if (d.copy) d.copy[i] = (uint16_t)f32_to_bf16(p);
    }
}

template <bool BF16G, int ORDER, bool WD, bool CLIP>
__global__ __launch_bounds__(kBlock) void adamw_kernel(const AdamDesc* __restrict__ desc,
                                                       const ely_adamw_consts* __restrict__ consts, int32_t n,
                                                       int64_t total_tiles, const float* __restrict__ coef_ptr) {
    const int64_t G = gridDim.x;
    const int64_t b = blockIdx.x;
    const int64_t t0 = b * total_tiles / G, t1 = (b + 1) * total_tiles / G;
    if (t0 >= t1) return;
    const float coef = CLIP ? *coef_ptr : 1.0f;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (desc[mid].tile_begin <= t0) lo = mid;
        else hi = mid - 1;
    }
    int64_t tile = t0;
    for (int ti = lo; ti < n && tile < t1; ++ti) {
        const AdamDesc d = desc[ti];
        const int64_t ntiles = (d.numel + kAdamTile - 1) / kAdamTile;
        const int64_t tend = min(t1, d.tile_begin + ntiles);
        if (tend <= tile) continue;
        const int64_t e0 = (tile - d.tile_begin) * kAdamTile;
        const int64_t e1 = min((tend - d.tile_begin) * kAdamTile, d.numel);
        const ely_adamw_consts c = consts[ti];
        adam_range<BF16G, ORDER, WD, CLIP>(d, c, coef, e0, e1);
        tile = tend;
    }
}

typedef void (*AdamKernel)(const AdamDesc*, const ely_adamw_consts*, int32_t, int64_t, const float*);

template <bool BF16G, int ORDER>
static AdamKernel pick_adam(bool wd, bool clip) {
    if (wd) return clip ? adamw_kernel<BF16G, ORDER, true, true> : adamw_kernel<BF16G, ORDER, true, false>;
    return clip ? adamw_kernel<BF16G, ORDER, false, true> : adamw_kernel<BF16G, ORDER, false, false>;
}

static size_t adam_table_bytes(int32_t n) {
    return align_up((size_t)n * sizeof(AdamDesc), 256) + align_up((size_t)n * sizeof(ely_adamw_consts), 256);
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

}  // namespace ely

using namespace ely;

extern "C" {

int64_t ely_grad_norm_workspace_bytes(const ely_tensor* grads, int32_t n) {
    if (n < 0 || (n > 0 && !grads)) return -1;
    return (int64_t)(norm_table_bytes(n) + align_up((size_t)std::max<int64_t>(norm_tiles(grads, n), 1) * 8, 256));
}

int ely_grad_norm(const ely_tensor* grads, int32_t n, float max_norm, ely_norm_result* out_dev, void* workspace,
                  int64_t ws_bytes, void* stream) {
    return guarded([&] {
        check_list(grads, n, "ely_grad_norm grads");
        if (!out_dev) fail(ELY_EINVAL, "ely_grad_norm: null result pointer");
        const int64_t need = ely_grad_norm_workspace_bytes(grads, n);
        if (!workspace || ws_bytes < need)
            fail(ELY_EWORKSPACE, "ely_grad_norm: workspace of " + std::to_string(ws_bytes) + " bytes, need " +
                                     std::to_string(need));
        hipStream_t s = static_cast<hipStream_t>(stream);
        std::vector<NormDesc> table;
        table.reserve(n);
        int64_t tiles = 0;
        for (int32_t i = 0; i < n; ++i) {
            if (grads[i].numel == 0) continue;
            NormDesc d;
            d.g = grads[i].ptr;
            d.numel = grads[i].numel;
            d.tile_begin = tiles;
            d.dtype = grads[i].dtype;
            d.aligned = aligned16(grads[i].ptr) ? 1 : 0;
            table.push_back(d);
            tiles += (d.numel + kNormTile - 1) / kNormTile;
        }
        char* ws = static_cast<char*>(workspace);
        NormDesc* dtable = reinterpret_cast<NormDesc*>(ws);
        double* partials = reinterpret_cast<double*>(ws + norm_table_bytes(n));
        if (tiles > 0) {
            upload(dtable, table.data(), table.size() * sizeof(NormDesc), s);
            const int64_t waves = std::min<int64_t>(tiles, mt_blocks(8) * (kBlock / kWave));
            const int64_t blocks = (waves + 3) / 4;
            hipLaunchKernelGGL(norm_partials_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, dtable,
                               (int32_t)table.size(), tiles, partials);
            check_launch("norm_partials_kernel");
        }
        hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(kFinalThreads), 0, s, partials, tiles, max_norm,
                           out_dev);
        check_launch("norm_final_kernel");
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
        check_list(params, n, "ely_adamw_step params");
        check_list(grads, n, "ely_adamw_step grads");
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
            d.m = static_cast<float*>(exp_avg[i].ptr);
            d.v = static_cast<float*>(exp_avg_sq[i].ptr);
            d.copy = copies ? static_cast<uint16_t*>(copies[i].ptr) : nullptr;
            d.numel = ne;
            d.tile_begin = tiles;
            d.aligned = aligned16(d.p) && aligned16(d.g) && aligned16(d.m) && aligned16(d.v) &&
                        (!d.copy || aligned16(d.copy));
            d.pad = 0;
            table.push_back(d);
            cs.push_back(consts[i]);
            tiles += (ne + kAdamTile - 1) / kAdamTile;
        }
        if (tiles == 0) return;
        hipStream_t s = static_cast<hipStream_t>(stream);
        char* ws = static_cast<char*>(workspace);
        AdamDesc* dtable = reinterpret_cast<AdamDesc*>(ws);
        ely_adamw_consts* dconsts = reinterpret_cast<ely_adamw_consts*>(ws + align_up((size_t)n * sizeof(AdamDesc), 256));
        upload(dtable, table.data(), table.size() * sizeof(AdamDesc), s);
        upload(dconsts, cs.data(), cs.size() * sizeof(ely_adamw_consts), s);
        const bool wd = weight_decay_nonzero != 0;
        const bool clip = coef_dev != nullptr;
        AdamKernel k;
        if (gdt == ELY_BF16)
            k = order == ELY_ORDER_HOST ? pick_adam<true, ELY_ORDER_HOST>(wd, clip) : pick_adam<true, ELY_ORDER_TORCH>(wd, clip);
        else
            k = order == ELY_ORDER_HOST ? pick_adam<false, ELY_ORDER_HOST>(wd, clip)
                                        : pick_adam<false, ELY_ORDER_TORCH>(wd, clip);
        const int64_t blocks = std::min<int64_t>(tiles, mt_blocks(8));
        hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kBlock), 0, s, dtable, dconsts, (int32_t)table.size(),
                           tiles, coef_dev);
        check_launch("adamw_kernel");
    });
}

}  // extern "C"
