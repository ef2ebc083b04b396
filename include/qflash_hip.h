/*
 * qflash_hip.h - C ABI of the MI355X (gfx950) integer-only attention forward.
 *
 * The library libqflash_hip.so replaces the two Triton kernels of
 * EfficientCompLab/qflash and their launch ABI:
 *   qflash_kernel[grid](Q, K, V, Out, sm_rscale, exp_M, req_M, l_M, acc_M,
 *                       16 strides, Z, H, N_CTX=, HEAD_DIM=, EXP_USE_SHIFT=,
 *                       L_USE_SHIFT=, ACC_USE_SHIFT=, L_SHIFT=, ACC_SHIFT=)
 *     (qflash/kernel.py:85-104, launched at :319-326)
 *   qflash_masked_kernel[grid](..., attn_bias, ..., 4 more strides, ...)
 *     (qflash/kernel.py:183-203, launched at :339-346)
 *
 * Conventions (all entry points):
 *   - plain C types only; device pointers come from the caller (no
 *     allocation inside any call); strides are in elements, int64, in the
 *     reference's order (z, h, row, col) per tensor; bias strides may be 0
 *     (broadcast);
 *   - the launch is asynchronous on `stream` (a hipStream_t, NULL = the
 *     default stream); the call returns 0 or a negative QFLASH_HIP_E* code
 *     and never throws; qflash_hip_last_error() gives a message for the
 *     last failure on the calling thread;
 *   - reentrant: no mutable global state besides the per-thread message, a
 *     per-thread copy of the last exp2 table formed on the host (a value of
 *     the call's constants), per-process caches filled on first use
 *     (occupancy, device addresses) and the test-hook bits of
 *     qflash_hip_set_test_hooks.
 */
#ifndef QFLASH_HIP_H
#define QFLASH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QFLASH_HIP_OK 0
#define QFLASH_HIP_EINVAL (-1)      /* bad pointer, shape, stride or constant */
#define QFLASH_HIP_EHEADDIM (-2)    /* HEAD_DIM unsupported (D=16 fails BLOCK_N<=HEAD_DIM, kernel.py:105) */
#define QFLASH_HIP_ELAUNCH (-3)     /* the HIP runtime rejected the launch */

/* Element types: floating-point inputs of the quantisation entry points, and
 * outputs of qflash_hip_forward. */
#define QFLASH_HIP_F32 0
#define QFLASH_HIP_F16 1
#define QFLASH_HIP_BF16 2
#define QFLASH_HIP_I8 3 /* output: the int8 codes themselves */
#define QFLASH_HIP_SCALES_WORKSPACE 256

/* Arithmetic-variant switches, kernel.py:30-36 (QFLASH_* environment). */
typedef struct qflash_hip_flags {
    int32_t exp_use_shift; /* QFLASH_EXP_USE_SHIFT, default 1 */
    int32_t l_use_shift;   /* QFLASH_L_USE_SHIFT, default 1 */
    int32_t acc_use_shift; /* QFLASH_ACC_USE_SHIFT, default 1 */
    int32_t l_shift;       /* QFLASH_L_SHIFT, default 30, 1..62 */
    int32_t acc_shift;     /* QFLASH_ACC_SHIFT, default 30, 1..62 */
} qflash_hip_flags;

/*
 * Unmasked integer attention forward: Out[z,h,i,:] = int8 codes of row i.
 * Replaces qflash_kernel (qflash/kernel.py:85-180).
 *   strides[16] = Q(z,h,m,k), K(z,h,n,k), V(z,h,k,n), Out(z,h,m,n),
 *   exactly the order of `*query.stride(), *key.stride(), *value.stride(),
 *   *o.stride()` at kernel.py:322.
 */
int qflash_hip_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out,
                      int32_t sm_rscale, int32_t exp_M, int32_t req_M, int32_t l_M, int32_t acc_M,
                      const int64_t* strides, int32_t Z, int32_t H, int32_t N_CTX, int32_t HEAD_DIM,
                      const qflash_hip_flags* flags, void* stream);

/*
 * Masked integer attention forward with an additive int32 logit bias.
 * Replaces qflash_masked_kernel (qflash/kernel.py:183-272).
 *   strides[20] = the 16 above followed by attn_bias(z,h,m,n) (kernel.py:342);
 *   bias strides may be 0 so a broadcast bias need not be materialised.
 */
int qflash_hip_masked_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out,
                             const int32_t* attn_bias, int32_t sm_rscale, int32_t exp_M, int32_t req_M,
                             int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z, int32_t H,
                             int32_t N_CTX, int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream);

/*
 * Masked forward with a window-periodic bias: batch index z uses
 * attn_bias[z % bias_zmod], i.e. attn_bias has logical shape
 * (bias_zmod, H, N, N) with the 4 bias strides given as for the masked entry.
 * No counterpart in the reference: it serves QWindowAttention
 * (qflash/attention.py:58-75), whose (B_, H, N, N) mask is the relative-position
 * bias plus a shift mask that repeats every nW windows; passing the nW distinct
 * slices gives the same codes as qflash_hip_masked_kernel on the materialised
 * bias without reading or building the B_/nW copies.
 */
int qflash_hip_window_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out,
                             const int32_t* attn_bias, int32_t sm_rscale, int32_t exp_M, int32_t req_M,
                             int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z, int32_t H,
                             int32_t N_CTX, int32_t HEAD_DIM, int32_t bias_zmod, const qflash_hip_flags* flags,
                             void* stream);


/*
 * Per-tensor absmax scales of Q, K and V in their own dtype, replacing
 * `x.abs().amax() / INT8_MAX` and `(q_scale * k_scale)` of qflash_forward
 * (qflash/kernel.py:294-297) with one read of each input:
 *   scales[0..2] = amax(|q|), amax(|k|), amax(|v|) times RN_fp32(1/127), rounded
 *                  to the dtype (torch's division of a device tensor by a host
 *                  scalar), scales[3] = scales[0] * scales[1] rounded to the dtype.
 * shapes_strides: for q, k, v in turn, 4 sizes (Z, H, N, D) then 4 element strides.
 * workspace: at least QFLASH_HIP_SCALES_WORKSPACE device uint32 entries, all
 * ZERO before the first call (partial maxima are kept there); each call
 * leaves them zero again when it completes, so one workspace serves any
 * number of calls in stream order.  Calls that share a workspace must not
 * overlap.  The call allocates nothing.
 */
int qflash_hip_scales(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                      void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream);

/*
 * int8 QKV projection fused with the quantiser: the codes and scales of the
 * q, k, v inputs of the attention straight from the activations, with the
 * projection itself on int8 MFMA.  No counterpart in the reference, which
 * computes the projection in floating point (qflash/attention.py:23-24) and
 * quantises its output (qflash/kernel.py:294-311); this is its int8 variant,
 * for callers that accept an int8 projection (QAttention(int8_proj=True)).
 *   acc[m, c] = sum_k x8[m, k] * w8[c, k]                    (exact int32)
 *   y[m, c]   = RN_fp32(RN_fp32(fp32(acc) * RN_fp32(x_scale * w_scale[c])) + bias[c])
 *               (no bias term when bias is NULL)
 * y's column thirds [0, C), [C, 2C), [2C, 3C) (C = Nc / 3) are q, k, v; scales
 * and codes are what qflash_hip_scales and qflash_hip_quantize (fp32) would
 * write for them: scales[0..2] = amax|q|, amax|k|, amax|v| times RN(1/127),
 * scales[3] = scales[0] * scales[1]; codes[m, c] = clamp(rint(y / scale)).
 * y itself is never stored: one pass reduces its absmax, a second recomputes it
 * and writes the codes.
 * x8: M x K int8 row-major (the activations' codes, x_scale their device fp32
 * scale); w8: Nc x K int8 row-major, w_scale / bias: Nc fp32 (device);
 * scales: 4 fp32 (device); codes: M x Nc int8 row-major (token-major q, k, v:
 * codes + 0, + C, + 2C with row stride Nc).  K a multiple of 32, Nc = 3 C
 * with C a multiple of 32.  workspace: as for qflash_hip_scales (zero before
 * the first call, zero again after each).  Allocates nothing.
 */
int qflash_hip_qkv_int8(const int8_t* x8, const int8_t* w8, const float* w_scale, const float* bias,
                        const float* x_scale, int32_t M, int32_t K, int32_t Nc, float* scales, int8_t* codes,
                        uint32_t* workspace, int64_t workspace_elems, void* stream);

/*
 * qflash_hip_scales without a workspace argument and without any allocation,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The partial maxima live in a static device
 * array of QFLASH_HIP_SCALES_WORKSPACE uint32 entries (1 KiB per GPU, held
 * until the process ends; its size does not depend on the inputs, so no input
 * size is rejected beyond what qflash_hip_scales rejects).  Each call clears it
 * with a fill kernel and then runs qflash_hip_scales on it.  All calls on one
 * GPU share that array: calls that overlap in time on one GPU (different
 * streams, different threads) race and must be serialised by the caller.
 * `stream` must belong to the current device.  Same results as
 * qflash_hip_scales.
 */
int qflash_hip_scales_noalloc(const void* q, const void* k, const void* v, int32_t dtype,
                              const int64_t* shapes_strides, void* scales, void* stream);

/*
 * int8 codes clamp(round(x / scale), -128, 127) of Q, K, V (qflash/kernel.py:
 * 309-311), scale = scales[0..2] as written by qflash_hip_scales (device
 * memory, read on the device: no host synchronisation).  The division is IEEE
 * fp32 (then rounded to the dtype), round half to even.  out_strides: 4 element
 * strides per output, in the order q8, k8, v8.
 */
int qflash_hip_quantize(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                        int8_t* q8, int8_t* k8, int8_t* v8, const int64_t* out_strides, const void* scales,
                        void* stream);

/*
 * int32 logit bias of QWindowAttention's mask, replacing the torch ops that
 * build it: the sum rel + mask of qflash/attention.py:68-74 (on the n_win
 * distinct slices, as qflash_hip_window_kernel reads them) followed by the
 * float-mask conversion of qflash/kernel.py:327-336, in one pass:
 *   x = RN_fp32(rel[h, i, j] + mask[w, i, j])   (mask NULL: x = rel[h, i, j], n_win = 1)
 *   out[w, h, i, j] = -2^20                                          if x < -100
 *                   = (int32) rint(RN_fp32(RN_fp32(x * L) * R))      otherwise,
 * L = RN_fp32(1.44269504), R = RN_fp32(1 / RN_fp32(sm_scale)): torch's
 * arithmetic on the GPU for x * LOG2E / sm_scale with host scalars.
 * rel: (H, N, N), mask: (n_win, N, N), out: (n_win, H, N, N), all contiguous
 * device memory.  Allocates nothing; asynchronous on `stream`.
 */
int qflash_hip_window_bias(const float* rel, const float* mask, int32_t n_win, int32_t H, int32_t N,
                           double sm_scale, int32_t* out, void* stream);

/*
 * The same conversion for a float attn_mask of any shape (qflash/kernel.py:
 * 327-336, the fp32 case of bias_values), element for element over n
 * contiguous fp32 values: one pass instead of the torch ops' eight.
 */
int qflash_hip_mask_bias(const float* mask, int64_t n, double sm_scale, int32_t* out, void* stream);

/*
 * qflash_hip_window_bias / qflash_hip_mask_bias with sm_scale read from a
 * device parameter block (qflash_hip_constants) instead of a host double, so
 * that no host synchronisation precedes them; nothing is written when
 * params[0] != 0.  No counterpart in the reference.
 */
int qflash_hip_window_bias_planned(const float* rel, const float* mask, int32_t n_win, int32_t H, int32_t N,
                                   const int32_t* params, int32_t* out, void* stream);
int qflash_hip_mask_bias_planned(const float* mask, int64_t n, const int32_t* params, int32_t* out, void* stream);

/*
 * One entry point for every case of the forward, used by qflash_forward: the
 * masks of both masked entries (attn_bias NULL = unmasked; bias_zmod 0 = the
 * bias has Z slices, > 0 = window-periodic as in qflash_hip_window_kernel),
 * and the output either as int8 codes (out_dtype QFLASH_HIP_I8, as the
 * reference kernels write them) or dequantised in place of the reference's
 * separate `o * o_scale` (qflash/kernel.py:351): Out[...] = RN_T(code *
 * o_scale) of type out_dtype (F32 / F16 / BF16), o_scale a device scalar of
 * that type, at the element offsets given by the 4 Out strides.  No
 * counterpart in the reference: it fuses the dequantisation pass.
 */
int qflash_hip_forward(const int8_t* Q, const int8_t* K, const int8_t* V, void* Out, int32_t out_dtype,
                       const void* o_scale, const int32_t* attn_bias, int32_t bias_zmod, int32_t sm_rscale,
                       int32_t exp_M, int32_t req_M, int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z,
                       int32_t H, int32_t N_CTX, int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream);

/*
 * The five constants of qflash/kernel.py:297-307 formed on the device, so that
 * a whole forward needs no host synchronisation (and can be captured in a HIP
 * graph); no counterpart in the reference, which forms them on the host after
 * `.item()`.  scales: the device array qflash_hip_scales writes (element 3 =
 * q_scale * k_scale in `dtype`); scale: the host's (scale or 1/sqrt(D)) *
 * 1.44269504 (kernel.py:289-290).  In Python's double arithmetic:
 *   sm_scale = scale * double(scales[3]); sm_rscale = rint(1.0 / sm_scale);
 *   exp_M = rint(-sm_scale * 65536); req_M = rint(sm_scale * 127 * 65536);
 *   l_M = rint(2^l_shift / sm_rscale); acc_M = rint(2^acc_shift / sm_rscale)
 * (rint = round half to even, Python's round).  params (device, 8-byte
 * aligned, QFLASH_HIP_PARAMS_WORDS int32) receives: [0] a status, 0 or one of
 * QFLASH_HIP_STATUS_* -- the first exception the reference's host raises on
 * the same value, in its order of evaluation (then no attention kernel reads
 * the constants and the outputs are left unwritten); [1..5] sm_rscale, exp_M,
 * req_M, l_M, acc_M; [6..12] and [16..18] the fast kernel's plan for N_CTX,
 * HEAD_DIM and masking; [14..15] sm_scale as a double.  Asynchronous on
 * `stream`.
 */
#define QFLASH_HIP_PARAMS_WORDS 20
#define QFLASH_HIP_STATUS_ZERODIV_SCALE 1   /* sm_scale == 0: ZeroDivisionError (1.0 / sm_scale) */
#define QFLASH_HIP_STATUS_NAN 2             /* ValueError: cannot convert float NaN to integer */
#define QFLASH_HIP_STATUS_INF 3             /* OverflowError: cannot convert float infinity to integer */
#define QFLASH_HIP_STATUS_ZERODIV_RSCALE 4  /* sm_rscale == 0 (sm_scale > 2): ZeroDivisionError */
#define QFLASH_HIP_STATUS_RANGE 5           /* a constant outside int32 (the kernels take int32) */
int qflash_hip_constants(const void* scales, int32_t dtype, double scale, int32_t N_CTX, int32_t HEAD_DIM,
                         int32_t masked, const qflash_hip_flags* flags, int32_t* params, void* stream);

/*
 * qflash_hip_scales followed by qflash_hip_constants (qflash/kernel.py:294-307),
 * in two launches instead of three: the absmax pass, then one one-wave kernel
 * that forms the scales and, from scales[3] as stored in `dtype`, the
 * constants and plan.  Arguments, workspace contract and results are those of
 * the two calls.  Allocates nothing.
 */
int qflash_hip_scales_constants(const void* q, const void* k, const void* v, int32_t dtype,
                                const int64_t* shapes_strides, void* scales, uint32_t* workspace,
                                int64_t workspace_elems, double scale, int32_t N_CTX, int32_t HEAD_DIM, int32_t masked,
                                const qflash_hip_flags* flags, int32_t* params, void* stream);

/*
 * qflash_hip_forward with the constants in device memory (`params` from
 * qflash_hip_constants with the same N_CTX, HEAD_DIM, masking and flags)
 * instead of host integers.  No counterpart in the reference.  Nothing is
 * written when params[0] != 0.
 */
int qflash_hip_forward_planned(const int8_t* Q, const int8_t* K, const int8_t* V, void* Out, int32_t out_dtype,
                               const void* o_scale, const int32_t* attn_bias, int32_t bias_zmod,
                               const int32_t* params, const int64_t* strides, int32_t Z, int32_t H, int32_t N_CTX,
                               int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream);

/* Message for the last failing call on this thread ("" if none). */
const char* qflash_hip_last_error(void);

/*
 * Layout self-check of the int8 MFMA used by the kernels (no counterpart in
 * the reference): C(32x32 int32) = A(32x32 int8, row-major) x B(32x32 int8,
 * row-major), all device pointers, computed with the same operand and
 * result register layouts the attention kernels rely on.
 */
int qflash_hip_mfma_layout_check(const int8_t* A, const int8_t* B, int32_t* C, void* stream);

/*
 * Diagnostic, no counterpart in the reference: the bounds of the table that
 * the fast kernel may use for exp2 + requantisation under these constants
 * (shift variant of exp2).  lut_n: entries p(0 .. lut_n-1) with
 * p(u) = int8(requant(exp2(-u))) as in qflash/kernel.py:40-64, the last one 0
 * (0 = no table: the kernel computes p arithmetically); lut_lim: p(u) == 0 for
 * every u in [lut_n-1, lut_lim].  The kernel caps lut_lim at its table size
 * and uses the table for launches large enough to repay filling it.
 * Host-only, needs no GPU.
 */
int qflash_hip_lut_bounds(int32_t sm_rscale, int32_t exp_M, int32_t req_M, int32_t* lut_n, int32_t* lut_lim);

/*
 * Diagnostic, no counterpart in the reference: the range [u_lo, u_hi] of
 * u = m' - s over which the masked fast kernel's table reads one constant
 * p_far = int8(requant(exp2(-u))) (qflash/kernel.py:40-64) for the columns of
 * a step whose biased score is negative (a -2^20 mask, padding), for the
 * constants of a launch that has a table (lut_n > 0).  u_hi < u_lo: no such
 * range.  Host-only, no GPU needed.
 */
int qflash_hip_far_bounds(int32_t sm_rscale, int32_t exp_M, int32_t req_M, int32_t* u_lo, int32_t* u_hi,
                          int32_t* p_far);

/*
 * Test hooks, no counterpart in the reference: each bit forces one of the
 * exact fallbacks of the attention entry points on inputs that would not need
 * it, so that tests can drive every path (the codes never change).  The
 * initial bits come from the environment when the library is loaded
 * (QFLASH_HIP_FORCE_GENERAL, _FORCE_DYNAMIC_BOUND, _FORCE_ROBUST, _NO_LUT,
 * _FORCE_LUT = non-zero); no entry point reads the environment afterwards.
 * Sets the bits for every thread of the process and returns the previous ones.
 */
#define QFLASH_HIP_HOOK_FORCE_GENERAL 1u        /* the general kernel */
#define QFLASH_HIP_HOOK_FORCE_DYNAMIC_BOUND 2u  /* the fast kernel's per-row rescale bound */
#define QFLASH_HIP_HOOK_FORCE_ROBUST 4u         /* the fast kernel's general arithmetic */
#define QFLASH_HIP_HOOK_NO_LUT 8u               /* no exp2 table */
#define QFLASH_HIP_HOOK_FORCE_LUT 16u           /* the exp2 table whatever the launch size */
#define QFLASH_HIP_HOOK_ALL 31u
uint32_t qflash_hip_set_test_hooks(uint32_t bits);

/* Library version string (no counterpart in the reference). */
const char* qflash_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* QFLASH_HIP_H */
