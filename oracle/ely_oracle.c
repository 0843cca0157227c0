/*
 * ely_oracle.c -- CPU restatement of the reference's per-stage update path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in elysium_wan_amd/csrc.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Every routine is written from the definition of the arithmetic the
 * reference performs (cited file:line, paths relative to the reference repo
 * root, TORCH/ = the installed torch package), not from the reference's code:
 *
 *   fp8 codes          model/fp8.py:17-20 (formats); the conversion itself is
 *                      torch's `.to(float8_e4m3fn | float8_e5m2)`, restated
 *                      here as round-to-nearest-even on the fp8 grid with the
 *                      overflow rule of TORCH/include/torch/headeronly/util/
 *                      Float8_e4m3fn.h:170-232 and Float8_e5m2.h:77-143.
 *   bf16 rounding      TORCH/include/torch/headeronly/util/BFloat16.h:100-114
 *                      (RNE, every NaN -> 0x7FC0); used by pieces.py:192-195.
 *   scale_exp          model/fp8.py:28-38
 *   quantize           model/fp8.py:41-49
 *   dequantize         model/fp8.py:52-53
 *   recover_exp        model/fp8.py:66-93
 *   HostAdamW update   runtime/optim.py:277-298 (_adamw_math), one IEEE fp32
 *                      rounding per operation, sqrt in fp64 rounded once.
 *   torch AdamW        TORCH/optim/adam.py:688-800 (_multi_tensor_adam op
 *                      order; used only for the <=1 ulp contract).
 *   grad sum of squares  TORCH/nn/utils/clip_grad.py:91-108 (the norm the clip
 *                      uses), here in long double as a brute-force bound.
 *   fold_add           runtime/pieces.py:206-214
 *   fold_add_bf16      runtime/accumulate.py:101-102 on a bf16 sum
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).  No
 * FMA contraction: each C operation is one correctly rounded IEEE operation,
 * which is exactly what the reference's one-kernel-per-op torch code does.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define DT_F32 0
#define DT_BF16 1
#define FMT_E4M3 0
#define FMT_E5M2 1

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ bf16 */

/* fp32 -> bf16, round to nearest, ties to even; NaN -> 0x7FC0 (positive). */
uint16_t orc_f32_to_bf16(float f) {
    if (f != f) return 0x7FC0;
    uint32_t u = f2u(f);
    uint32_t lo = u & 0xFFFF0000u;       /* truncation toward zero in magnitude */
    uint32_t rem = u & 0x0000FFFFu;      /* discarded bits */
    uint32_t keep = lo >> 16;
    if (rem > 0x8000u || (rem == 0x8000u && (keep & 1u))) keep += 1; /* carries into the exponent are correct */
    return (uint16_t)keep;
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* ------------------------------------------------------------------- fp8 */

/* fp32 -> fp8 code.  Round to nearest even on the format's grid.  e4m3fn:
 * anything that rounds past 448 (|x| > 464) and NaN/Inf give 0x7F | sign;
 * e5m2: anything that rounds past 57344 (|x| >= 61440) and Inf give
 * 0x7C | sign (Inf), NaN gives 0x7F | sign. */
uint8_t orc_f32_to_fp8(float f, int fmt) {
    const int M = fmt == FMT_E4M3 ? 3 : 2;          /* mantissa bits */
    const int BIAS = fmt == FMT_E4M3 ? 7 : 15;
    const int EMIN = 1 - BIAS;                      /* exponent of the smallest normal */
    uint8_t sign = (f2u(f) >> 31) ? 0x80 : 0x00;
    if (f != f) return (uint8_t)(0x7F | sign);
    double a = fabs((double)f);
    if (fmt == FMT_E4M3) {
        if (a >= 480.0) return (uint8_t)(0x7F | sign);
    } else {
        if (a >= 65536.0) return (uint8_t)(0x7C | sign);
    }
    if (a == 0.0) return sign;
    int E;
    (void)frexp(a, &E);                  /* a = m * 2^E, m in [0.5, 1) */
    E -= 1;                              /* a = m' * 2^E, m' in [1, 2) */
    if (E < EMIN) E = EMIN;              /* subnormal range shares EMIN's quantum */
    double n = ldexp(a, M - E);          /* a / quantum, exact in double */
    double r = nearbyint(n);             /* default rounding mode: ties to even */
    int ri = (int)r;
    if (ri == (2 << M)) {                /* carried into the next binade */
        E += 1;
        ri = 1 << M;
    }
    int code;
    if (ri < (1 << M)) {
        code = ri;                       /* subnormal (E == EMIN) or zero */
    } else {
        code = ((E + BIAS) << M) | (ri - (1 << M));
    }
    return (uint8_t)(code | sign);
}

void orc_fp8_encode_array(const float* x, int64_t n, int fmt, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_fp8(x[i], fmt);
}

/* fp8 code -> fp32 value (exact). */
float orc_fp8_to_f32(uint8_t c, int fmt) {
    const int M = fmt == FMT_E4M3 ? 3 : 2;
    const int BIAS = fmt == FMT_E4M3 ? 7 : 15;
    const int EBITS = fmt == FMT_E4M3 ? 4 : 5;
    int s = c >> 7;
    int e = (c >> M) & ((1 << EBITS) - 1);
    int m = c & ((1 << M) - 1);
    double v;
    if (fmt == FMT_E4M3 && (c & 0x7F) == 0x7F) {
        v = NAN;
    } else if (fmt == FMT_E5M2 && e == 31) {
        v = m == 0 ? INFINITY : NAN;
    } else if (e == 0) {
        v = ldexp((double)m, 1 - BIAS - M);
    } else {
        v = ldexp((double)((1 << M) | m), e - BIAS - M);
    }
    return (float)(s ? -v : v);
}

/* -------------------------------------------------------- element access */

static inline float load_elem(const void* x, int dtype, int64_t i) {
    if (dtype == DT_BF16) return orc_bf16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

/* Round an fp32 value to the tensor's dtype and back (the dtype's own
 * arithmetic: a bf16 op is the fp32 op rounded once to bf16). */
static inline float to_dtype(float v, int dtype) {
    if (dtype == DT_BF16) return orc_bf16_to_f32(orc_f32_to_bf16(v));
    return v;
}

static inline void store_elem(void* x, int dtype, int64_t i, float v) {
    if (dtype == DT_BF16) ((uint16_t*)x)[i] = orc_f32_to_bf16(v);
    else ((float*)x)[i] = v;
}

/* torch.exp2(n.to(dtype)) for an integer n: 2^n rounded once to the dtype
 * (0 below half the smallest subnormal, Inf at or above 2^128). */
float orc_pow2(int n, int dtype) {
    long double v = ldexpl(1.0L, n);
    float f = (float)v;                  /* correctly rounded to fp32 */
    return to_dtype(f, dtype);
}

/* frexp exponent of a non-negative value as torch.frexp reports it
 * (value = m * 2^e, m in [0.5, 1)); Inf and NaN report 0. */
static int frexp_exp(float a) {
    if (a != a || isinf(a)) return 0;
    int e;
    (void)frexpf(a, &e);
    return e;
}

static int ebias_of(int fmt) { return fmt == FMT_E4M3 ? 8 : 15; }

/* fp8.scale_exp (model/fp8.py:28-38) for one row. */
static int32_t row_scale_exp(const void* x, int dtype, int64_t off, int64_t cols, int fmt) {
    float amax = 0.0f;
    int nan = 0;
    for (int64_t j = 0; j < cols; ++j) {
        float a = fabsf(load_elem(x, dtype, off + j));
        if (a != a) nan = 1;
        else if (a > amax) amax = a;
    }
    if (nan) return 0;                   /* amax is NaN: `amax > 0` is false */
    if (!(amax > 0.0f)) return 0;
    return (int32_t)(frexp_exp(amax) - ebias_of(fmt));
}

void orc_scale_exp(const void* x, int dtype, int64_t rows, int64_t cols, int fmt, int32_t* k) {
    for (int64_t r = 0; r < rows; ++r) k[r] = row_scale_exp(x, dtype, r * cols, cols, fmt);
}

/* fp8.quantize (model/fp8.py:45-49): q = fp8(x * 2^-k) with the multiply
 * done in x's dtype. */
void orc_quantize(const void* x, int dtype, int64_t rows, int64_t cols, int fmt,
                  uint8_t* q, int32_t* k) {
    for (int64_t r = 0; r < rows; ++r) {
        int32_t kr = row_scale_exp(x, dtype, r * cols, cols, fmt);
        k[r] = kr;
        float s = orc_pow2(-kr, dtype);
        for (int64_t j = 0; j < cols; ++j) {
            float y = to_dtype(load_elem(x, dtype, r * cols + j) * s, dtype);
            q[r * cols + j] = orc_f32_to_fp8(y, fmt);
        }
    }
}

/* fp8.dequantize (model/fp8.py:52-53): q.to(dtype) * 2^k in dtype. */
void orc_dequantize(const uint8_t* q, const int32_t* k, int64_t rows, int64_t cols, int fmt,
                    void* out, int out_dtype) {
    for (int64_t r = 0; r < rows; ++r) {
        float s = orc_pow2(k[r], out_dtype);
        for (int64_t j = 0; j < cols; ++j) {
            float v = to_dtype(orc_fp8_to_f32(q[r * cols + j], fmt), out_dtype);
            store_elem(out, out_dtype, r * cols + j, v * s);
        }
    }
}

/* fp8.recover_exp (model/fp8.py:66-93): per row, the first k of
 * base + (0, -1, 1, -2, 2) for which every element survives
 * fp8(t * 2^-k) * 2^k == t.  Returns the number of rows with no such k
 * (their k is left at the last candidate tried, as the reference's `best`). */
int64_t orc_recover_exp(const void* t, int dtype, int64_t rows, int64_t cols, int fmt, int32_t* k) {
    static const int deltas[5] = {0, -1, 1, -2, 2};
    int64_t bad = 0;
    for (int64_t r = 0; r < rows; ++r) {
        int32_t base = row_scale_exp(t, dtype, r * cols, cols, fmt);
        int found = 0;
        int32_t best = base;
        for (int di = 0; di < 5 && !found; ++di) {
            int32_t cand = base + deltas[di];
            float sdown = orc_pow2(-cand, dtype);
            float sup = orc_pow2(cand, dtype);
            int ok = 1;
            for (int64_t j = 0; j < cols && ok; ++j) {
                float v = load_elem(t, dtype, r * cols + j);
                float y = to_dtype(v * sdown, dtype);
                float back = to_dtype(orc_fp8_to_f32(orc_f32_to_fp8(y, fmt), fmt), dtype);
                float w = to_dtype(back * sup, dtype);
                if (!(w == v)) ok = 0;
            }
            best = cand;
            found = ok;
        }
        k[r] = best;
        if (!found) ++bad;
    }
    return bad;
}

/* --------------------------------------------------------------- AdamW */

/* Per-step fp32 constants, in the order runtime/optim.py:158-167 names them. */
enum { C_DECAY, C_B1, C_ONE_B1, C_B2, C_ONE_B2, C_INV_BC2_SQRT, C_EPS, C_STEP_SIZE, C_N };

/* HostAdamW's _adamw_math (runtime/optim.py:277-298) over n elements, plus
 * the optional fused clip (g * coef, one fp32 rounding, skipped when
 * coef == 1) and the optional bf16 working copy of the updated parameter
 * (pieces.py:192-195). */
void orc_adamw_host(float* p, const void* g, int gdtype, float* m, float* v, int64_t n,
                    const float* c, int weight_decay_nonzero, float coef, uint16_t* copy) {
    for (int64_t i = 0; i < n; ++i) {
        float gi = load_elem(g, gdtype, i);
        if (coef != 1.0f) gi = gi * coef;
        float pi = p[i], mi = m[i], vi = v[i];
        if (weight_decay_nonzero) pi = pi * c[C_DECAY];
        mi = mi * c[C_B1];
        float t = gi * c[C_ONE_B1];
        mi = mi + t;
        vi = vi * c[C_B2];
        float sq = gi * gi;
        sq = sq * c[C_ONE_B2];
        vi = vi + sq;
        float d = (float)sqrt((double)vi);
        d = d * c[C_INV_BC2_SQRT];
        d = d + c[C_EPS];
        float u = mi / d;
        u = u * c[C_STEP_SIZE];
        pi = pi - u;
        p[i] = pi; m[i] = mi; v[i] = vi;
        if (copy) copy[i] = orc_f32_to_bf16(pi);
    }
}

/* torch.optim.AdamW's GPU foreach op order (TORCH/optim/adam.py:688-800):
 * lerp (ATen/native/Lerp.h, weight < 0.5 branch), addcmul and addcdiv as
 * `a + s * (b op c)`, each written here as an explicit fma, which is how a
 * contracting device compiler emits them.  Constants: decay, w1 = 1-b1,
 * b2, one_b2, bc2_sqrt, eps, neg_step = -(lr / bc1). */
enum { T_DECAY, T_W1, T_B2, T_ONE_B2, T_BC2_SQRT, T_EPS, T_NEG_STEP, T_N };

void orc_adamw_torch(float* p, const void* g, int gdtype, float* m, float* v, int64_t n,
                     const float* c, int weight_decay_nonzero, float coef, uint16_t* copy) {
    for (int64_t i = 0; i < n; ++i) {
        float gi = load_elem(g, gdtype, i);
        if (coef != 1.0f) gi = gi * coef;
        float pi = p[i], mi = m[i], vi = v[i];
        if (weight_decay_nonzero) pi = pi * c[T_DECAY];
        float w = c[T_W1];
        if (fabsf(w) < 0.5f) {
            mi = fmaf(w, gi - mi, mi);
        } else {
            mi = fmaf(-(gi - mi), 1.0f - w, gi);
        }
        vi = vi * c[T_B2];
        vi = fmaf(c[T_ONE_B2], gi * gi, vi);
        float d = (float)sqrt((double)vi);
        d = d / c[T_BC2_SQRT];
        d = d + c[T_EPS];
        pi = fmaf(c[T_NEG_STEP], mi / d, pi);
        p[i] = pi; m[i] = mi; v[i] = vi;
        if (copy) copy[i] = orc_f32_to_bf16(pi);
    }
}

/* ------------------------------------------------------------ grad norm */

/* Sum of squares of one tensor, in long double (64-bit significand), as the
 * brute-force value the device's fp64 tree reduction is held to. */
long double orc_sumsq(const void* g, int dtype, int64_t n) {
    long double s = 0.0L;
    for (int64_t i = 0; i < n; ++i) {
        long double x = (long double)load_elem(g, dtype, i);
        s += x * x;
    }
    return s;
}

double orc_sumsq_d(const void* g, int dtype, int64_t n) { return (double)orc_sumsq(g, dtype, n); }

/* clip_grad_norm_'s coefficient (TORCH/nn/utils/clip_grad.py:165-169) in
 * fp32 tensor arithmetic.  `max_norm / t` on a tensor is t.reciprocal() *
 * max_norm (TORCH/_tensor.py:1119-1122), and clamp(max=1) keeps a NaN. */
float orc_clip_coef(float total_norm, float max_norm) {
    float denom = total_norm + 1e-6f;
    float r = 1.0f / denom;
    float coef = r * max_norm;
    return coef > 1.0f ? 1.0f : coef;
}

/* ----------------------------------------------------------- casts/fold */

/* pieces.cast_piece (runtime/pieces.py:192-195) fp32 -> bf16. */
void orc_cast_bf16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(x[i]);
}

/* pieces.fold_add (runtime/pieces.py:206-214): acc += float(g), one fp32 add. */
void orc_fold_add(float* acc, const void* g, int gdtype, int64_t n) {
    for (int64_t i = 0; i < n; ++i) acc[i] = acc[i] + load_elem(g, gdtype, i);
}

/* OrderedAccumulator's fold into a bf16 sum (runtime/accumulate.py:101-102,
 * `acc.add_(t)` on a bf16 tensor): torch computes the add in fp32 (its
 * opmath type for bf16) and rounds the fp32 sum to bf16. */
void orc_fold_add_bf16(uint16_t* acc, const void* g, int gdtype, int64_t n) {
    for (int64_t i = 0; i < n; ++i) acc[i] = orc_f32_to_bf16(orc_bf16_to_f32(acc[i]) + load_elem(g, gdtype, i));
}
