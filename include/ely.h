/*
 * ely.h -- C ABI of libelyhip.so, the MI355X (gfx950) kernels of the
 * per-stage mixed-precision update path.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, never
 * throws, and returns an ely_status (0 = ok).  On failure ely_last_error()
 * returns a thread-local message.  Device pointers are HIP device memory
 * (e.g. torch's data_ptr()); `stream` is a hipStream_t passed as void*
 * (torch.cuda.current_stream().cuda_stream).  Every launch goes to that
 * stream; nothing synchronizes the device.  The library never allocates or
 * frees caller memory; scratch comes from the caller's `workspace` (sized by
 * the *_workspace_bytes queries) plus a small pinned host ring the library
 * owns for uploading tensor tables.
 *
 * Citations name the reference function each entry point replaces (paths
 * relative to the reference repository root; TORCH/ = the torch package).
 */
#ifndef ELY_H
#define ELY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ely_status {
    ELY_OK = 0,
    ELY_EINVAL = 1,       /* bad argument: shape, dtype, alignment, size (-> ValueError) */
    ELY_EHIP = 2,         /* a HIP runtime call or launch failed (-> RuntimeError) */
    ELY_ENOTREPR = 3,     /* tensor is not scaled-fp8 representable (-> ValueError) */
    ELY_EWORKSPACE = 4    /* workspace smaller than the *_workspace_bytes query */
} ely_status;

enum { ELY_F32 = 0, ELY_BF16 = 1 };          /* element types */
enum { ELY_E4M3 = 0, ELY_E5M2 = 1 };         /* fp8 formats: float8_e4m3fn, float8_e5m2 */
enum { ELY_ORDER_HOST = 0, ELY_ORDER_TORCH = 1 };

/* One tensor of a multi-tensor call: a contiguous range of `numel` elements. */
typedef struct ely_tensor {
    void* ptr;
    int64_t numel;
    int32_t dtype;        /* ELY_F32 | ELY_BF16 */
    int32_t reserved;     /* must be 0 */
} ely_tensor;

/* Result of the grad-norm reduction, written to device memory. */
typedef struct ely_norm_result {
    double sumsq;         /* sum of g^2 over every element, fp64 */
    float norm;           /* (float)sqrt(sumsq) */
    float coef;           /* clip coefficient min(max_norm / (norm + 1e-6), 1), as torch */
} ely_norm_result;

/* AdamW per-step fp32 constants, one block per tensor.
 * ELY_ORDER_HOST uses, in order, the eight scalars runtime/optim.py:158-167
 * computes: decay, b1, one_b1, b2, one_b2, inv_bc2_sqrt, eps, step_size.
 * ELY_ORDER_TORCH uses the first seven slots as the scalars of torch's
 * _multi_tensor_adam (TORCH/optim/adam.py:689-800): decay, 1-b1, b2, 1-b2,
 * bc2_sqrt, eps, -(lr/bc1); the eighth is ignored. */
typedef struct ely_adamw_consts {
    float c[8];
} ely_adamw_consts;

/* Library identity and errors. */
int32_t ely_abi_version(void);
const char* ely_last_error(void);

/* ---------------------------------------------------------------- (a) */

/* Workspace bytes ely_grad_norm needs for these tensors. */
int64_t ely_grad_norm_workspace_bytes(const ely_tensor* grads, int32_t n);

/* Deterministic global L2 norm of a ragged gradient list, and the clip
 * coefficient clip_grad_norm_ derives from it.  Replaces the norm of
 * TORCH/nn/utils/clip_grad.py:50-108 and the coefficient of :160-169 (the
 * reference itself never clips; its optimizer is runtime/optim.py:45-54).
 * Each fixed tile (16,384 elements; 4,096 when the list holds fewer than
 * 2^29 elements) is reduced in a fixed lane order (fp32 squares of at most 8
 * elements, fp64 above), tiles in index order: the result is a function of
 * the list alone, bitwise identical across runs and grid sizes.  coef =
 * min(max_norm * (1/(norm + 1e-6)), 1) in fp32 for any max_norm, as torch
 * computes it (0 gives 0; a NaN norm gives NaN). */
int ely_grad_norm(const ely_tensor* grads, int32_t n, float max_norm,
                  ely_norm_result* out_dev, void* workspace, int64_t ws_bytes, void* stream);

/* torch's clip_grad_norm_ (TORCH/nn/utils/clip_grad.py:50-183) in one call:
 * ely_grad_norm of grads, then every gradient scaled in place by the clip
 * coefficient, g <- g * coef rounded once to g's dtype (the
 * _foreach_mul_(grads, clip_coef) of :170-177), in one launch over the tile
 * table the norm uploaded.  Same workspace as ely_grad_norm.  torch's
 * error_if_nonfinite check needs the norm before the scale: a caller that
 * wants it uses ely_grad_norm and ely_scale_inplace instead. */
int ely_grad_norm_clip(const ely_tensor* grads, int32_t n, float max_norm, ely_norm_result* out_dev,
                       void* workspace, int64_t ws_bytes, void* stream);

/* ely_grad_norm of the folded gradients accs[i] + widen(grads[i]) (each sum
 * rounded once to fp32, pieces.fold_add, runtime/pieces.py:206-214): the
 * norm of the step's gradient when the last microbatch has not been folded
 * into the fp32 accumulators yet.  accs: n fp32 tensors of the grads' numel;
 * nothing is written to them.  Same order and determinism as ely_grad_norm. */
int ely_grad_norm_fold(const ely_tensor* accs, const ely_tensor* grads, int32_t n, float max_norm,
                       ely_norm_result* out_dev, void* workspace, int64_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- (b) */

int64_t ely_adamw_workspace_bytes(int32_t n);

/* One fused AdamW step over a ragged tensor list, one HBM pass per element:
 * read p, g, m, v; write p, m, v and (optionally) the bf16 working copy.
 * Replaces HostAdamW.step/_update/_adamw_math (runtime/optim.py:145-204,
 * 277-298) for ELY_ORDER_HOST, torch.optim.AdamW.step (runtime/optim.py:50-51,
 * TORCH/optim/adam.py:554-800) for ELY_ORDER_TORCH, plus the fp32->bf16 cast
 * of pieces.cast_piece (runtime/pieces.py:192-195) and the bf16 widening of
 * pieces.fold_start (runtime/pieces.py:198-203) when grads are bf16.
 * params/exp_avg/exp_avg_sq: fp32; grads: all ELY_F32 or all ELY_BF16;
 * copies: NULL or n bf16 tensors (a NULL ptr skips that tensor's copy);
 * coef_dev: NULL (no clip) or &ely_norm_result.coef from ely_grad_norm. */
int ely_adamw_step(const ely_tensor* params, const ely_tensor* grads,
                   const ely_tensor* exp_avg, const ely_tensor* exp_avg_sq,
                   const ely_tensor* copies, int32_t n,
                   const ely_adamw_consts* consts, int32_t order, int32_t weight_decay_nonzero,
                   const float* coef_dev, void* workspace, int64_t ws_bytes, void* stream);

/* ely_adamw_step whose gradient is the ordered fold finished inside the
 * update: g = accs[i] + widen(grads[i]), rounded once to fp32 as
 * pieces.fold_add does (runtime/pieces.py:206-214, runtime/accumulate.py:
 * 93-104), then clipped and applied.  The accumulator of the earlier
 * microbatches is read, never written, so the fold costs 4 read bytes per
 * element instead of a 10-byte fold pass plus the update's gradient read.
 * Results equal ely_fold_add followed by ely_adamw_step bit for bit. */
int ely_adamw_fold_step(const ely_tensor* params, const ely_tensor* accs, const ely_tensor* grads,
                        const ely_tensor* exp_avg, const ely_tensor* exp_avg_sq, const ely_tensor* copies, int32_t n,
                        const ely_adamw_consts* consts, int32_t order, int32_t weight_decay_nonzero,
                        const float* coef_dev, void* workspace, int64_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- (c) */

/* Workspace bytes of ely_fp8_quantize / ely_fp8_roundtrip over [rows, cols]
 * of x_dtype: the split path's row maxima and partial maxima; for one row of
 * at least 64 MiB, also room for the sampled guess below (about cols / 512
 * bytes).  -1 for negative sizes. */
int64_t ely_fp8_workspace_bytes(int64_t rows, int64_t cols, int32_t x_dtype);

/* fp8.quantize (model/fp8.py:28-49): per row of `cols` elements,
 * k = frexp(amax(|x|)).exponent - ebias (0 for an all-zero row, ebias 8 for
 * e4m3, 15 for e5m2) and q = fp8(x * 2^-k) with the multiply in x's dtype
 * and torch's round-to-nearest-even conversion.  Per-tensor scaling is
 * rows = 1.  x: [rows, cols] bf16 or fp32; q: [rows, cols] bytes, or NULL to
 * compute k alone (fp8.scale_exp); k: [rows] int32.
 * A row that fits no register path is read twice (its |x|max, then its
 * codes), except one row of at least 64 MiB (16-byte aligned, whole
 * vectors) given the larger workspace: its exponent is guessed from every
 * 61st 2,048-element segment and the codes are made at the guess in the
 * same pass that finds |x|max (as ely_fp8_quantize_hint does), a second
 * pass following only when the guess was wrong.  The bytes are the same
 * either way. */
int ely_fp8_quantize(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt,
                     uint8_t* q, int32_t* k, void* workspace, int64_t ws_bytes, void* stream);

/* No counterpart in the reference: ely_fp8_quantize for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same results; no workspace argument and no
 * allocation of any kind: the split path (rows longer than the register
 * paths take, e.g. per-tensor scaling) keeps its row maxima in a 1 MiB
 * static device array of the library, one per GPU, so it accepts at most
 * ~131,000 such rows and refuses more with ELY_EINVAL.  Calls that overlap
 * on one GPU (different streams, or threads without ordering) share that
 * array and race; calls on one stream are ordered and safe. */
int ely_fp8_quantize_noalloc(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt,
                             uint8_t* q, int32_t* k, void* stream);

/* Per-tensor fp8.quantize / fp8.roundtrip (model/fp8.py:28-63 with rows = 1)
 * given a guess of the exponent; an addition to the reference's interface
 * (fp8.quantize(x, fmt, per_tensor=True, k_hint=...)).  The results are
 * exactly ely_fp8_quantize's / ely_fp8_roundtrip's over one row of n
 * elements: k[0] is the tensor's exponent whatever the hint, and the codes
 * depend on k alone.  When k[0] equals the hint, x is read once (3 B/element
 * for bf16 -> fp8) instead of twice; otherwise the call makes a second pass
 * at the true exponent.  The hint is k_hint, or, when k_hint_dev is not
 * NULL, the device int32 *k_hint_dev, read on the GPU (no host wait); it
 * may be the same word as k, e.g. the last step's exponent updated in
 * place.  *hit_dev (optional, device int32) is 1 when the one pass stood,
 * 0 otherwise (and 0 when the tensor or hint admits no one-pass form:
 * unaligned x, n not a whole number of 16-byte vectors, or a hint outside
 * [-110, 110]).  q: n bytes, or NULL with out given (the round trip without
 * the codes); out: n elements in x's dtype or NULL.  Workspace:
 * ely_fp8_hint_workspace_bytes(n). */
int64_t ely_fp8_hint_workspace_bytes(int64_t n);
int ely_fp8_quantize_hint(const void* x, int32_t x_dtype, int64_t n, int32_t fmt, int32_t k_hint,
                          const int32_t* k_hint_dev, uint8_t* q, int32_t* k, void* out, int32_t* hit_dev,
                          void* workspace, int64_t ws_bytes, void* stream);

/* fp8.dequantize (model/fp8.py:52-53): out = float(q) * 2^k in out_dtype
 * (ELY_F32 is the reference's default; ELY_BF16 is roundtrip's dtype). */
int ely_fp8_dequantize(const uint8_t* q, const int32_t* k, int64_t rows, int64_t cols, int32_t fmt,
                       void* out, int32_t out_dtype, void* stream);

/* fp8.roundtrip (model/fp8.py:56-63) fused: out = dequantize(quantize(x)) in
 * x's dtype, q and k written too when non-NULL. */
int ely_fp8_roundtrip(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt,
                      void* out, uint8_t* q, int32_t* k, void* workspace, int64_t ws_bytes,
                      void* stream);

/* Workspace bytes ely_fp8_recover_exp needs for `rows` rows. */
int64_t ely_fp8_recover_workspace_bytes(int64_t rows);

/* fp8.recover_exp (model/fp8.py:66-93): per row, base = the scale_exp
 * exponent of t's own |t|max, then the first k of base + (0, -1, 1, -2, 2)
 * for which every element satisfies fp8(t * 2^-k) * 2^k == t in t's dtype.
 * k: [rows] int32; a row with no such k keeps base + 2 and adds 1 to
 * *bad_rows_dev (the caller zeroes it; the reference raises ValueError, which
 * the Python layer does when the count is non-zero). */
int ely_fp8_recover_exp(const void* t, int32_t t_dtype, int64_t rows, int64_t cols, int32_t fmt,
                        int32_t* k, unsigned long long* bad_rows_dev, void* workspace, int64_t ws_bytes,
                        void* stream);

/* encode_scaled_fp8's device half (codec/planes.py:85-117): recover_exp's k
 * (model/fp8.py:66-93, as ely_fp8_recover_exp) and the byte image
 * q = fp8(t * 2^-k[row]) (planes.py:110-111, as ely_fp8_quantize_k) in one
 * call; rows that fit registers take one read of t and one write of q.
 * q: [rows * cols] bytes; bad rows as in ely_fp8_recover_exp (their q is not
 * meaningful).  Workspace: ely_fp8_recover_workspace_bytes(rows). */
int ely_fp8_recover_image(const void* t, int32_t t_dtype, int64_t rows, int64_t cols, int32_t fmt,
                          int32_t* k, uint8_t* q, unsigned long long* bad_rows_dev, void* workspace,
                          int64_t ws_bytes, void* stream);

/* q = fp8(x * 2^-k[row]) with the caller's exponents, the multiply in x's
 * dtype: the byte image of the scaled-fp8 wire (codec/planes.py:110-111). */
int ely_fp8_quantize_k(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int32_t fmt,
                       const int32_t* k, uint8_t* q, void* stream);

/* ------------------------------------------------------------ casts/fold */

/* pieces.cast_piece (runtime/pieces.py:192-195): fp32 -> bf16, RNE,
 * every NaN -> 0x7FC0. */
int ely_cast_bf16(const float* x, uint16_t* out, int64_t n, void* stream);

/* The first microbatch's term of the ordered fold, widened to the fp32 sum
 * (runtime/pieces.py:198-203 `fold_start`, `g.to(torch.float32)`; and
 * runtime/accumulate.py:98-100, `t.to(want, copy=True)`): out[i] = x[i] as
 * fp32, exact.  x: n bf16; out: n fp32. */
int ely_widen_bf16(const uint16_t* x, float* out, int64_t n, void* stream);

/* pieces.fold_add (runtime/pieces.py:206-214): acc += float(g), one fp32
 * rounding; g_dtype ELY_F32 or ELY_BF16. */
int ely_fold_add(float* acc, const void* g, int32_t g_dtype, int64_t n, void* stream);

/* OrderedAccumulator._fold into a bf16 sum (runtime/accumulate.py:101-102,
 * `self.acc[i].add_(t)` when the running sum is bf16): acc = bf16(float(acc)
 * + float(g)), the fp32 add rounded to bf16 (RNE, every NaN -> 0x7FC0), as
 * torch's in-place add on a bf16 tensor; g_dtype ELY_F32 or ELY_BF16. */
int ely_fold_add_bf16(uint16_t* acc, const void* g, int32_t g_dtype, int64_t n, void* stream);

/* The row folds of TiedRowFold (runtime/accumulate.py:140-247), the step
 * gradient of a tied table split across stages: for each j < n_idx, with
 * r = idx[j], ar = a_rows ? a_rows[j] : j and e the row b[b_rows[j]]
 * (b_rows[j] >= 0), b[j] (b compact, b_rows NULL), or +0.0 (no b, or
 * b_rows[j] < 0),
 *     v = a[ar] + e                              rounded to dtype,
 *     acc[r] = first ? v : acc[r] + v            rounded to dtype
 * (the reference's `h[fi] + 0.0` folds of a Head gradient's free rows,
 * :210-213, and `hk + e_on` folds of its held rows, :232-235, e_on being
 * the embedding rows where the microbatch has them and +0 elsewhere).
 * acc: [n_rows, d]; a: [a_total, d] rows picked by a_rows, or compact
 * [n_idx, d] when a_rows is NULL; b: NULL, [b_total, d] rows picked by
 * b_rows, or compact [n_idx, d]; idx, a_rows and b_rows are device int64
 * arrays; the rows of idx are distinct.  An index outside its table is
 * skipped (the caller checks them).  dtype ELY_F32 or ELY_BF16. */
int ely_rows_fold(void* acc, const void* a, const int64_t* a_rows, const void* b, const int64_t* b_rows,
                  const int64_t* idx, int64_t n_idx, int64_t n_rows, int64_t a_total, int64_t b_total, int64_t d,
                  int32_t dtype, int32_t first, void* stream);

/* A Head gradient taken in one pass (runtime/accumulate.py:203-221): a row r
 * of [n_rows, d] with slot[r] < 0 is free and takes acc[r] = a[r] + 0.0
 * (first) or acc[r] + (a[r] + 0.0), each add rounded to dtype (the
 * reference's `h[fi] + 0.0` folds, :210-213); a held row, slot[r] >= 0, is
 * copied bit for bit to held_out[slot[r]] (`h[ki].clone()`, :221) and acc[r]
 * is left.  slot: device int32 [n_rows], the held rows numbered
 * 0..n_held-1 (a slot at or past n_held is skipped); held_out: [n_held, d].
 * dtype ELY_F32 or ELY_BF16. */
int ely_rows_split(void* acc, const void* a, const int32_t* slot, void* held_out, int64_t n_rows, int64_t n_held,
                   int64_t d, int32_t dtype, int32_t first, void* stream);

/* In-place g <- g * (*coef_dev) over a tensor list, the product rounded to
 * each tensor's dtype: the scaling step of clip_grad_norm_
 * (TORCH/nn/utils/clip_grad.py:170-183) with the coefficient ely_grad_norm
 * left on the device.  One launch per 48 tensors, no workspace. */
int ely_scale_inplace(const ely_tensor* tensors, int32_t n, const float* coef_dev, void* stream);

/* No counterpart in the reference (its HostAdamW copies m and v through
 * staging buffers, runtime/optim.py:176-204, 301-363): the address under
 * which the GPU reaches pinned, mapped host memory (hipHostGetDevicePointer),
 * so that the fused update reads and writes host-resident moments in place
 * over PCIe.  ELY_EINVAL if `host` is not such memory. */
int ely_host_device_pointer(const void* host, void** device);

/* Cap on the blocks one multi-tensor launch (grad-norm, AdamW) may use; 0
 * restores each kernel's own grid.  For tuning and for the tests
 * that prove results do not depend on the grid.  Process-wide. */
int ely_set_max_blocks(int32_t max_blocks);

/* ---------------------------------------------------------- wire planes */

/* The byte split of codec/planes.py:152-158 (encode's plain-dtype path):
 * n elements of esz bytes (1, 2, 4 or 8; little-endian) at x become esz
 * planes of n bytes at planes[j * n + i], plane j holding byte esz-1-j of
 * every element (most significant first).  esz 1 is a copy. */
int ely_byteplanes_split(const void* x, int64_t n, int32_t esz, uint8_t* planes, void* stream);

/* The byte join of codec/planes.py:174-186 (decode's plain-dtype path): the
 * inverse of ely_byteplanes_split. */
int ely_byteplanes_join(const uint8_t* planes, int64_t n, int32_t esz, void* out, void* stream);

/* codec/fp8_planes.py:19-30: the float8_e4m3fn code of each of the n
 * elements of t (ELY_F32 or ELY_BF16, torch's rounding), written as two
 * nibble planes of (n + 1) / 2 bytes: hi[i] = (code[2i] >> 4) << 4 |
 * code[2i+1] >> 4, lo[i] likewise with the low nibbles, a missing odd
 * element as 0.  Every element whose code does not convert back to it
 * exactly (NaN, Inf, beyond 448, off the e4m3 grid; -0 == 0 as in
 * torch.equal) adds 1 to *bad_dev (the caller zeroes it; the reference
 * asserts, which the Python layer does when the count is non-zero).  The
 * planes' nibbles for such elements are unspecified. */
int ely_fp8_nibbles_encode(const void* t, int32_t t_dtype, int64_t n, uint8_t* hi, uint8_t* lo,
                           unsigned long long* bad_dev, void* stream);

/* codec/fp8_planes.py:35-52: nibble planes -> n fp32 values of the e4m3
 * codes. */
int ely_fp8_nibbles_decode(const uint8_t* hi, const uint8_t* lo, int64_t n, float* out, void* stream);

/* ------------------------------------------------------------ self-test */

/* Device self-check of the gfx950 fp8 conversion instruction against the
 * library's bit-level restatement of torch's conversion, over the fp32 bit
 * patterns [start, start + count).  mismatches_dev: three uint64 counters
 * the caller zeroes: [0] patterns the kernels' instruction path relies on
 * (|x| at most the format's largest finite value) whose code differs,
 * [1] differing patterns outside that domain (NaN, overflow; informational),
 * [2] (only when start == 0) decoded codes that differ from the format's
 * definition, over all 256 codes. */
int ely_selftest_fp8_cvt(uint32_t start, uint64_t count, int32_t fmt,
                         unsigned long long* mismatches_dev, void* stream);

/* Device self-check of the gfx950 scaled conversions the bf16 kernels use
 * (v_cvt_scalef32_pk_{fp8,bf8}_bf16 to quantize, v_cvt_scalef32_pk_bf16_
 * {fp8,bf8} to decode, at scale 2^k) against the library's restatement of
 * torch's arithmetic, over every bf16 pattern and every |k| <= 110.
 * mismatches_dev: two uint64 counters the caller zeroes: [0] quantized
 * (pattern, k) pairs of the instruction path's domain (finite, |x| 2^-k
 * below 2^ebias) whose code differs, in either half of the input word or of
 * the output; [1] (code, k) pairs, NaN codes aside, whose bf16 differs. */
int ely_selftest_fp8_scaled(int32_t fmt, unsigned long long* mismatches_dev, void* stream);

/* Device self-check that the kernels' fp32 sqrt (used by the AdamW update)
 * equals the fp64 sqrt rounded once to fp32 (runtime/optim.py:288-291) on
 * the non-negative fp32 patterns of [start, start + count) (sign bit
 * cleared).  mismatches_dev: one uint64 counter the caller zeroes. */
int ely_selftest_sqrt(uint32_t start, uint64_t count, unsigned long long* mismatches_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ELY_H */
