// Integer-only attention forward for MI355X (gfx950 / CDNA4).
//
// Replaces qflash_kernel / qflash_masked_kernel of EfficientCompLab/qflash
// (qflash/kernel.py:85-180, :183-272).  Per query row the result is the
// reference's integer algorithm: int8 Q.K^T into int32, a shift-based
// integer exp2, int8 requantisation of P, fixed-point online-softmax rescale
// of the running sum l and accumulator acc every 32 key columns (in order),
// int8 P.V into int32, one fp32 divide, int8 store.
//
// Work decomposition
//   one workgroup = W waves = 32*W query rows of one (z, h); waves share the
//   K / V^T tiles staged in LDS, 32 keys (one rescale step) per tile.
//   S^T = K . Q^T is one v_mfma_i32_32x32x32_i8 per 32 head-dim columns, so
//   every lane holds 16 scores of ONE query; P (int8) then feeds
//   O = P . V directly as the MFMA A operand, with V^T stored in LDS in the
//   key order that the S^T result layout produces.
//
// Register layouts (v_mfma_i32_32x32x32_i8, wave64)
//   A (32 x 32 int8): lane l holds row l%32, 16 bytes of K-dim half l/32
//   B (32 x 32 int8): lane l holds col l%32, 16 bytes of K-dim half l/32
//   C (32 x 32 int32): lane l, register v holds (row 8*(v/4)+4*(l/32)+v%4,
//                      col l%32)
//   (checked at run time by qflash_hip_mfma_layout_check).
#include "qf_fwd.h"

namespace qf {

__global__ __launch_bounds__(64) void mfma_layout_kernel(const int8_t* A, const int8_t* B, int32_t* C) {
    const int lane = threadIdx.x, lq = lane & 31, g = lane >> 5;
    i32x4 a = *reinterpret_cast<const i32x4*>(A + lq * 32 + g * 16);
    uint32_t w[4] = {0, 0, 0, 0};
    for (int b = 0; b < 16; ++b) w[b >> 2] |= (uint32_t)(uint8_t)B[(g * 16 + b) * 32 + lq] << (8 * (b & 3));
    i32x4 bv = i32x4{(int32_t)w[0], (int32_t)w[1], (int32_t)w[2], (int32_t)w[3]};
    i32x16 c = mfma32(a, bv, i32x16{});
    for (int v = 0; v < 16; ++v) C[crow(v, lane) * 32 + lq] = c[v];
}

// ----------------------------------------------------------------------------
// Host side
using qferr::fail;
using qferr::g_err;

// ---- test and tuning hooks --------------------------------------------------
// Read from the environment once, when the library is loaded, never per
// launch: the test-hook bits (QFLASH_HIP_FORCE_GENERAL, _FORCE_DYNAMIC_BOUND,
// _FORCE_ROBUST, _NO_LUT, _FORCE_LUT set to a non-zero value) and two tuning
// values (QFLASH_HIP_WG_PER_CU: workgroups per CU of the fast kernel, 0 = its
// natural occupancy; QFLASH_HIP_WAVES_PER_WG: 1, 2 or 4).  Tests change the
// bits through qflash_hip_set_test_hooks; launches read them with one relaxed
// atomic load.
static bool env_flag(const char* name) {
    const char* v = getenv(name);
    return v && v[0] && v[0] != '0';
}
static int env_int(const char* name) {
    const char* v = getenv(name);
    return v ? atoi(v) : 0;
}
static uint32_t env_hook_bits() {
    return (env_flag("QFLASH_HIP_FORCE_GENERAL") ? QFLASH_HIP_HOOK_FORCE_GENERAL : 0u) |
           (env_flag("QFLASH_HIP_FORCE_DYNAMIC_BOUND") ? QFLASH_HIP_HOOK_FORCE_DYNAMIC_BOUND : 0u) |
           (env_flag("QFLASH_HIP_FORCE_ROBUST") ? QFLASH_HIP_HOOK_FORCE_ROBUST : 0u) |
           (env_flag("QFLASH_HIP_NO_LUT") ? QFLASH_HIP_HOOK_NO_LUT : 0u) |
           (env_flag("QFLASH_HIP_FORCE_LUT") ? QFLASH_HIP_HOOK_FORCE_LUT : 0u);
}
static std::atomic<uint32_t> g_hook_bits{env_hook_bits()};
static const int g_wg_per_cu = env_int("QFLASH_HIP_WG_PER_CU");
static const int g_waves_per_wg = env_int("QFLASH_HIP_WAVES_PER_WG");
static bool hook(uint32_t bit) { return (g_hook_bits.load(std::memory_order_relaxed) & bit) != 0; }

// Bounds of the fast kernel's exp2 + requantisation table (see lut_pack_vt):
// n entries p(0 .. n - 1), the last one 0, and lim such that p(u) = 0 for
// every u in [n - 1, lim].  From u0 on (q >= bitlen(rs) + 3) the bound of
// lut_pack_vt's comment gives E = 0 up to lim; below u0 the values are
// computed with the kernel's own integer primitives (lut_scan).  n = 0: no
// table.  lut_range returns u0 (or -1: no table) and sets lim.
__host__ __device__ static int64_t lut_range(const Args& a, int64_t* lim_out) {
    const int64_t A = -(int64_t)a.eM, rs = a.rs;
    if (!a.exp_mode || A <= 0 || rs <= 0) return -1;
    const int64_t kap = A * rs - 65536;
    if (kap > 2 * A) return -1;
    int64_t lim = (int64_t)INT32_MAX / A;              // u * |eM| < 2^31: x * eM does not wrap
    if (kap < 0 && rs * 65536 / -kap < lim) lim = rs * 65536 / -kap;  // r >= -2 rs
    int bl = 0;
    while ((1ll << bl) <= rs) ++bl;
    const int64_t u0 = ((bl + 3) * 65536 + A - 1) / A;  // q >= bitlen(rs) + 3 for u >= u0
    // lut_n <= u0 + 1 entries, and the masked kernels' far entry after them
    if (u0 > lim || u0 >= kLutMax - 1) return -1;
    *lim_out = lim;
    return u0;
}

static void lut_bounds(const Args& a, int32_t* n_out, int32_t* lim_out) {
    *n_out = 0;
    *lim_out = 0;
    int64_t lim = 0;
    const int64_t u0 = lut_range(a, &lim);
    if (u0 < 0) return;
    int64_t n = 1;
    for (int64_t u = u0; u >= 0; --u)
        if (requant(exp2_i32((int32_t)-u, a), a) != 0) {
            n = u + 2;
            break;
        }
    *n_out = (int32_t)n;
    *lim_out = (int32_t)lim;
}

// Far columns of the masked table path.  For u = m' - s >= 0 with u*|eM| < 2^31
// (u <= hi) write u*|eM| = 2^16 q + f, 0 <= f < 2^16; then exp2's remainder is
// r = q*rs - u = (u*kappa - rs*f) / 2^16 (kappa = |eM|*rs - 2^16), and for
// q >= 32 (u >= ceil(2^21 / |eM|)) E = ((r >> 1) + rs) >> q is the sign fill
// of (r >> 1) + rs:
//   kappa >= 0: r > -rs, so (r >> 1) + rs >= rs/2 > 0: E = 0, p = 0;
//   kappa <  0: r <= -u*|kappa| / 2^16 < -2 rs once u > 2 rs 2^16 / |kappa|,
//               so (r >> 1) + rs <= -1: E = -1, p = requant(-1).
// Over u in [lo, hi] p is that one constant.  The kernel reads it for every
// column whose biased score s' = s + kScoreBias is negative once a step has
// m' >= far_lo = max(lo - 1, lut_n - 1) (then u = m' - s' >= lo) and
// m' - min s' <= far_hi = min(hi, 2^30) (2^30 also rejects a wrapped s').
// u_lo / u_hi / p_far: the range and the constant (u_hi < u_lo: none).
__host__ __device__ static void far_range(const Args& a, int64_t* u_lo, int64_t* u_hi, int32_t* p_far) {
    *u_lo = 1;
    *u_hi = 0;
    *p_far = 0;
    const int64_t A = -(int64_t)a.eM, rs = a.rs;
    if (!a.exp_mode || A <= 0 || rs <= 0) return;
    const int64_t kap = A * rs - 65536;
    int64_t lo = ((int64_t)32 * 65536 + A - 1) / A;
    if (kap < 0 && 2 * rs * 65536 / -kap + 1 > lo) lo = 2 * rs * 65536 / -kap + 1;
    int64_t hi = (int64_t)INT32_MAX / A;
    if (hi > (1 << 30)) hi = 1 << 30;
    *u_lo = lo;
    *u_hi = hi;
    *p_far = kap < 0 ? requant(-1, a) : 0;
}

// The far-column fields of a masked launch with a table (a.lut_n > 0).
__host__ __device__ static void far_bounds(Args& a) {
    a.far_lo = a.lut_n > 0 ? a.lut_n - 1 : 0;
    a.far_hi = 0;
    a.far_p = 0;
    if (a.lut_n <= 0) return;
    int64_t lo, hi;
    int32_t p;
    far_range(a, &lo, &hi, &p);
    if (lo > hi) return;
    if (lo - 1 > a.far_lo) a.far_lo = (int32_t)(lo - 1);
    a.far_hi = (int32_t)hi;
    a.far_p = p;
}

// Whether the table pays for this launch (test hooks aside): filling it costs
// each workgroup a few hundred VALU operations and every step an LDS round
// trip; it replaces ~80 VALU instructions per 32-key step, and filling it
// costs each wave ~10 per 64 * W entries (measured on MI355X: worth it for
// every N >= 32).
__host__ __device__ static bool lut_wanted(const Args& a, bool no_lut, bool force_lut) {
    if (a.force_robust || no_lut) return false;
    return a.N >= 32 || force_lut;
}

// The table for this call, or none (lut_n = 0).
static void choose_lut(Args& a, bool masked) {
    a.lut_n = 0;
    a.lut_lim = 0;
    a.far_lo = a.far_hi = a.far_p = 0;
    if (!lut_wanted(a, hook(QFLASH_HIP_HOOK_NO_LUT), hook(QFLASH_HIP_HOOK_FORCE_LUT))) return;
    int32_t n, lim;
    lut_bounds(a, &n, &lim);
    if (n - 1 > a.x_safe) return;  // the kernel fills the table with the 24-bit E
    a.lut_n = n;
    a.lut_lim = lim;
    if (masked) far_bounds(a);
}

// Proof obligations of fwd_fast on the constants (see the comment above it).
// Returns true and fills a.x_safe / a.id_ok / a.eps_abs / a.e_acc when the
// fast path computes exactly what the reference does for every possible int8
// input of this shape, given a layout the fast kernel accepts (fast_layout).
__host__ __device__ static bool fast_consts(Args& a, bool masked) {
    if (!a.exp_mode || !a.acc_mode || !a.l_mode) return false;
    if (a.acc_shift < 1 || a.acc_shift > 30 || a.l_shift < 1 || a.l_shift > 30) return false;
    if ((int64_t)a.rs * a.aM >= (1ll << 31) || (int64_t)a.rs * a.lM >= (1ll << 31)) return false;
    const int64_t rs = a.rs, eM = a.eM, rM = a.rM, aem = -(int64_t)a.eM;
    if (eM > 0 || aem >= (1 << 23) || rs <= 0 || rs >= (1 << 15) || rM >= (1 << 23) || rM <= -(1 << 23)) return false;
    if (aem * rs >= (1 << 17)) return false;
    const int64_t lim = (1ll << 31) - (1ll << 17);
    // a = x + (q+2)*rs lies in (|x|*eps/2^16 + rs, |x|*eps/2^16 + 2*rs], eps = |eM|*rs - 2^16
    const int64_t eps = aem * rs - 65536, eabs = eps < 0 ? -eps : eps;
    // |rs - 2^16/|eM|| <= 2 keeps E(x) in [-1, rs] for every x <= 0 with no int32 overflow of x*eM
    if (eabs > 2 * aem) return false;
    a.eps_abs = (int32_t)eabs;
    // masked: the kernel checks |x| <= X per wave and step; unmasked: per wave from ||q||_1
    int64_t X = aem ? lim / aem : (1ll << 22);
    if (X > (1ll << 22)) X = 1ll << 22;
    const int64_t x_amax = eabs ? (((1ll << 22) - 2 * rs - 2) * 65536) / eabs : (1ll << 22);
    if (X > x_amax) X = x_amax;
    if (masked && X < 4096) return false;
    a.x_safe = (int32_t)X;
    // rescale by alpha = rs is the identity while |acc * e| < 2^(As-1); |acc| grows by at
    // most 32*128*128 + 1 per step (x2 for the (1 + |e|/2^As) factors)
    const int64_t T = (a.N + 31) / 32;
    const int64_t e = rs * (int64_t)a.aM - (1ll << a.acc_shift);
    const double bacc = (double)T * ((1 << 19) + 1) * 2.0;
    a.id_ok = (bacc * (double)(e < 0 ? -e : e) < (double)(1ll << (a.acc_shift - 1))) ? 1 : 0;
    a.e_acc = (int32_t)(e < 0 ? -e : e);
    return true;
}

// Layouts the fast kernel accepts (unit column stride, 16-byte rows, buffer
// offsets in 31 bits).
static bool fast_layout(const Args& a, int D, bool vec) {
    if (D > 128) return false;  // D=256 would spill: the general kernel serves it
    if (!vec || a.so[3] != 1) return false;
    // buffer accesses of K, V (loads) and O (stores): rows >= N must fall past
    // (N-1)*stride + D, and the last stage's offsets (keys < N + 128, stages of
    // at most 128 keys) fit 31 bits
    for (int64_t st : {a.sk[2], a.sv[2], a.so[2]})
        if (st < D || (int64_t)(a.N + 128) * st + D > INT32_MAX) return false;
    return true;
}

static bool choose_fast(Args& a, int D, bool masked, bool vec) {
    return fast_layout(a, D, vec) && fast_consts(a, masked);
}

// ---- constants on the device (qflash_hip_constants) --------------------------
// qflash/kernel.py:297-307 in Python's double arithmetic: sm_scale = scale *
// float(q_scale * k_scale), then each constant int(round(...)) (round half to
// even = rint), evaluated in the reference's order so that the first failure
// is the exception Python raises there; then every constant must fit int32.
__device__ static double scale_value_f64(const void* p, int dt) {
    if (dt == QFLASH_HIP_F32) return (double)*reinterpret_cast<const float*>(p);
    const uint32_t h = *reinterpret_cast<const uint16_t*>(p);
    return (double)(dt == QFLASH_HIP_F16 ? __half2float(__ushort_as_half((unsigned short)h)) : __uint_as_float(h << 16));
}

// round() of a finite double as Python's int: status 0, or the exception
__device__ static int py_round(double x, double* r) {
    if (__builtin_isnan(x)) return QFLASH_HIP_STATUS_NAN;
    if (__builtin_isinf(x)) return QFLASH_HIP_STATUS_INF;
    *r = __builtin_rint(x);
    return 0;
}

__device__ static int device_constants(double sm, int l_shift, int acc_shift, int32_t* c) {
    double v[5];
    if (sm == 0.0) return QFLASH_HIP_STATUS_ZERODIV_SCALE;  // 1.0 / sm_scale
    int st = py_round(1.0 / sm, &v[0]);                     // sm_rscale
    if (!st) st = py_round(-sm * 65536.0, &v[1]);           // exp_M
    if (!st) st = py_round(sm * 127.0 * 65536.0, &v[2]);    // req_M (left to right)
    if (st) return st;
    if (v[0] == 0.0) return QFLASH_HIP_STATUS_ZERODIV_RSCALE;  // (1 << shift) / sm_rscale
    // int / int true division: correctly rounded, as IEEE division of the exact
    // operands is while |sm_rscale| < 2^53 (larger ones fail the int32 test anyway)
    v[3] = __builtin_rint(__builtin_ldexp(1.0, l_shift) / v[0]);
    v[4] = __builtin_rint(__builtin_ldexp(1.0, acc_shift) / v[0]);
    for (int i = 0; i < 5; ++i) {
        if (!(v[i] >= -2147483648.0 && v[i] <= 2147483647.0)) return QFLASH_HIP_STATUS_RANGE;
        c[i] = (int32_t)v[i];
    }
    return 0;
}

// One wave: the constants and the plan from sm = scale * float(q_scale *
// k_scale); the table scan of lut_bounds runs over the lanes, lane 0 writes
// the parameter block.
__device__ static void constants_body(double sm, Args a, int32_t masked, uint32_t hooks, int32_t* params) {
    const int lane = threadIdx.x;
    int32_t c[5] = {0, 0, 0, 0, 0};
    const int status = device_constants(sm, a.l_shift, a.acc_shift, c);
    a.rs = c[0]; a.eM = c[1]; a.rM = c[2]; a.lM = c[3]; a.aM = c[4];
    a.id_ok = a.x_safe = a.eps_abs = a.e_acc = a.lut_n = a.lut_lim = 0;
    a.far_lo = a.far_hi = a.far_p = 0;
    bool fast = false;
    if (status == 0) {
        fast = !(hooks & QFLASH_HIP_HOOK_FORCE_GENERAL) && fast_consts(a, masked != 0);
        if (fast && lut_wanted(a, hooks & QFLASH_HIP_HOOK_NO_LUT, hooks & QFLASH_HIP_HOOK_FORCE_LUT)) {
            int64_t lim = 0;
            const int64_t u0 = lut_range(a, &lim);
            // largest u <= u0 (< kLutMax) with p(u) != 0, over the lanes
            int32_t hit = -1;
            for (int32_t u = (int32_t)u0 - lane; u >= 0; u -= 64)
                if (requant(exp2_i32(-u, a), a) != 0) {
                    hit = u;
                    break;
                }
            for (int o = 32; o >= 1; o >>= 1) hit = max(hit, __shfl_xor(hit, o));
            const int64_t n = hit >= 0 ? hit + 2 : 1;
            if (u0 >= 0 && n - 1 <= a.x_safe) {
                a.lut_n = (int32_t)n;
                a.lut_lim = (int32_t)lim;
                if (masked) far_bounds(a);
            }
        }
        if (hooks & QFLASH_HIP_HOOK_FORCE_DYNAMIC_BOUND) a.id_ok = 0;
    }
    if (lane == 0) {
        int32_t w[QFLASH_HIP_PARAMS_WORDS] = {status, a.rs, a.eM, a.rM, a.lM, a.aM, fast ? 1 : 0, a.id_ok, a.x_safe,
                                              a.eps_abs, a.e_acc, a.lut_n, a.lut_lim, 0, 0, 0, a.far_lo, a.far_hi,
                                              a.far_p, 0};
        const uint64_t smb = __double_as_longlong(sm);
        w[kPSmScale] = (int32_t)(uint32_t)smb;
        w[kPSmScale + 1] = (int32_t)(uint32_t)(smb >> 32);
        for (int i = 0; i < QFLASH_HIP_PARAMS_WORDS; ++i) params[i] = w[i];
    }
}

__global__ __launch_bounds__(64) void constants_kernel(const void* scales, int32_t dt, double scale, Args a,
                                                       int32_t masked, uint32_t hooks, int32_t* params) {
    const double sm = scale * scale_value_f64(static_cast<const char*>(scales) + 3 * (dt == QFLASH_HIP_F32 ? 4 : 2),
                                              dt);
    constants_body(sm, a, masked, hooks, params);
}

// The scales kernel of qflash_hip_scales and constants_kernel in one wave:
// the scales from the absmax slots (which it sets back to zero), then the
// constants from their product as stored in T.
template <int DT>
__global__ __launch_bounds__(64) void scales_constants_kernel(uint32_t* ws, void* scales, double scale, Args a,
                                                              int32_t masked, uint32_t hooks, int32_t* params) {
    const float qk = qfs::reduce_scale_slots<DT>(ws, scales);
    constants_body(scale * (double)qk, a, masked, hooks, params);
}

// Checks of qflash_hip_constants' arguments and the Args fields its kernel
// reads; *hooks: the test-hook bits of this call.
static int constants_args(int32_t dtype, int32_t N, int32_t D, const qflash_hip_flags* flags, const int32_t* params,
                          Args* a, uint32_t* hooks) {
    if (!params) return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (dtype != QFLASH_HIP_F32 && dtype != QFLASH_HIP_F16 && dtype != QFLASH_HIP_BF16)
        return fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    if (N <= 0 || D <= 0) return fail(QFLASH_HIP_EINVAL, "bad N_CTX=%d HEAD_DIM=%d", N, D);
    if (((uintptr_t)params & 7u) != 0) return fail(QFLASH_HIP_EINVAL, "params must be 8-byte aligned");
    qflash_hip_flags f = {1, 1, 1, 30, 30};
    if (flags) f = *flags;
    if (f.l_use_shift && (f.l_shift < 1 || f.l_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "l_shift %d outside 1..62", f.l_shift);
    if (f.acc_use_shift && (f.acc_shift < 1 || f.acc_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "acc_shift %d outside 1..62", f.acc_shift);
    a->N = N;
    a->l_shift = f.l_shift;
    a->acc_shift = f.acc_shift;
    a->exp_mode = f.exp_use_shift != 0;
    a->l_mode = f.l_use_shift != 0;
    a->acc_mode = f.acc_use_shift != 0;
    *hooks = g_hook_bits.load(std::memory_order_relaxed);
    a->force_robust = (*hooks & QFLASH_HIP_HOOK_FORCE_ROBUST) ? 1 : 0;
    return 0;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static int forward(const int8_t* Q, const int8_t* K, const int8_t* V, void* O, const int32_t* bias,
                   int32_t rs, int32_t eM, int32_t rM, int32_t lM, int32_t aM, const int64_t* strides,
                   int32_t Z, int32_t H, int32_t N, int32_t D, const qflash_hip_flags* flags, void* stream,
                   int32_t bias_zmod = 0, int32_t out_dt = QFLASH_HIP_I8, const void* o_scale = nullptr,
                   const int32_t* params = nullptr) {
    g_err[0] = 0;
    if (!Q || !K || !V || !O || !strides) return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (out_dt != QFLASH_HIP_I8 && out_dt != QFLASH_HIP_F32 && out_dt != QFLASH_HIP_F16 && out_dt != QFLASH_HIP_BF16)
        return fail(QFLASH_HIP_EINVAL, "unknown output dtype code %d", out_dt);
    if (out_dt != QFLASH_HIP_I8 && !o_scale) return fail(QFLASH_HIP_EINVAL, "o_scale is null");
    if (Z <= 0 || H <= 0 || N <= 0) return fail(QFLASH_HIP_EINVAL, "bad shape Z=%d H=%d N=%d", Z, H, N);
    if (D == 16)
        return fail(QFLASH_HIP_EHEADDIM, "HEAD_DIM=16 < BLOCK_N=32: the reference kernel rejects it "
                                         "(tl.static_assert(BLOCK_N <= HEAD_DIM))");
    if (D != 32 && D != 64 && D != 128 && D != 256)
        return fail(QFLASH_HIP_EHEADDIM, "HEAD_DIM=%d not in {32,64,128,256}", D);
    // rs = round(1/sm_scale) is never 0 at the reference's launch (its host
    // divides by it, kernel.py:306); a negative one (negative `scale`) runs the
    // general kernel, exact for any constants
    if (!params && rs == 0) return fail(QFLASH_HIP_EINVAL, "sm_rscale must not be 0");
    qflash_hip_flags f = {1, 1, 1, 30, 30};
    if (flags) f = *flags;
    if (f.l_use_shift && (f.l_shift < 1 || f.l_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "l_shift %d outside 1..62", f.l_shift);
    if (f.acc_use_shift && (f.acc_shift < 1 || f.acc_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "acc_shift %d outside 1..62", f.acc_shift);
    if ((int64_t)Z * H > (int64_t)INT32_MAX / 64) return fail(QFLASH_HIP_EINVAL, "Z*H too large");
    // the output of one head is written through a buffer resource: byte offsets in 32 bits
    for (int i = 0; i < 4; ++i)
        if (strides[12 + i] < 0) return fail(QFLASH_HIP_EINVAL, "negative output stride");
    if (((int64_t)(N - 1) * strides[14] + (int64_t)(D - 1) * strides[15] + 1) *
            (out_dt == QFLASH_HIP_I8 ? 1 : (out_dt == QFLASH_HIP_F32 ? 4 : 2)) >
        INT32_MAX)
        return fail(QFLASH_HIP_EINVAL, "one head's output spans more than 2 GiB");

    Args a{};
    a.q = Q; a.k = K; a.v = V; a.bias = bias;
    a.o = out_dt == QFLASH_HIP_I8 ? (int8_t*)O : nullptr;
    a.out_t = out_dt == QFLASH_HIP_I8 ? nullptr : O;
    a.out_dt = out_dt;
    a.o_scale = o_scale;
    for (int i = 0; i < 4; ++i) {
        a.sq[i] = strides[i];
        a.sk[i] = strides[4 + i];
        a.sv[i] = strides[8 + i];
        a.so[i] = strides[12 + i];
        a.sb[i] = bias ? strides[16 + i] : 0;
    }
    a.bias_zmod = bias_zmod;
    a.bias_vec = bias && a.sb[3] == 1 && a.sb[0] >= 0 && a.sb[1] >= 0 && a.sb[2] >= 0 &&
                 ((int64_t)(N - 1) * a.sb[2] + N + 64) * 4 <= INT32_MAX;
    a.Z = Z; a.H = H; a.N = N;
    a.rs = rs; a.eM = eM; a.rM = rM; a.lM = lM; a.aM = aM;
    a.l_shift = f.l_shift; a.acc_shift = f.acc_shift;
    a.exp_mode = f.exp_use_shift != 0; a.l_mode = f.l_use_shift != 0; a.acc_mode = f.acc_use_shift != 0;

    // 16-byte vector loads need unit head-dim stride and 16-byte aligned rows.
    bool vec = a.sq[3] == 1 && a.sk[3] == 1 && a.sv[3] == 1 && aligned16(Q) && aligned16(K) && aligned16(V);
    for (int i = 0; i < 3 && vec; ++i)
        vec = (a.sq[i] % 16 == 0) && (a.sk[i] % 16 == 0) && (a.sv[i] % 16 == 0);

    const int blocks32 = (N + 31) / 32;
    int W = blocks32 >= 4 ? 4 : (blocks32 >= 2 ? 2 : 1);
    if (g_waves_per_wg == 1 || g_waves_per_wg == 2 || g_waves_per_wg == 4) W = g_waves_per_wg;  // tuning hook
    a.mblocks = (blocks32 + W - 1) / W;
    const int64_t nwg = (int64_t)Z * H * a.mblocks;
    if (nwg > INT32_MAX) return fail(QFLASH_HIP_EINVAL, "grid too large");
    a.n_wg = (int32_t)nwg;
    const bool masked = bias != nullptr;
    a.id_ok = 0;
    a.x_safe = 0;
    a.eps_abs = 0;
    a.e_acc = 0;
    // Test hooks: FORCE_GENERAL selects the general kernel; FORCE_DYNAMIC_BOUND /
    // FORCE_ROBUST drive the fast kernel's exact fallbacks on inputs that would
    // not need them; NO_LUT / FORCE_LUT turn its table path off / on whatever
    // the shape.
    a.force_robust = hook(QFLASH_HIP_HOOK_FORCE_ROBUST) ? 1 : 0;
    bool fast;
    if (params) {  // the constants and their part of the plan are in device memory
        a.params = params;
        fast = fast_layout(a, D, vec) && !hook(QFLASH_HIP_HOOK_FORCE_GENERAL);
        a.general_only = fast ? 0 : 1;
    } else {
        fast = choose_fast(a, D, masked, vec) && !hook(QFLASH_HIP_HOOK_FORCE_GENERAL);
        if (fast) choose_lut(a, masked);
        if (hook(QFLASH_HIP_HOOK_FORCE_DYNAMIC_BOUND)) a.id_ok = 0;
    }
    dim3 grid((unsigned)nwg);
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
#define QF_CASE(DD)                                                                      \
    case DD:                                                                             \
        e = masked ? launch_d<DD, true>(a, W, vec, fast, g_wg_per_cu, grid, st)          \
                   : launch_d<DD, false>(a, W, vec, fast, g_wg_per_cu, grid, st);        \
        break;
    switch (D) {
        QF_CASE(32)
        QF_CASE(64)
        QF_CASE(128)
        default:
            e = masked ? launch_d<256, true>(a, W, vec, fast, g_wg_per_cu, grid, st)
                       : launch_d<256, false>(a, W, vec, fast, g_wg_per_cu, grid, st);
    }
#undef QF_CASE
    if (e != hipSuccess) return fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return QFLASH_HIP_OK;
}

}  // namespace qf

extern "C" {

int qflash_hip_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out, int32_t sm_rscale,
                      int32_t exp_M, int32_t req_M, int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z,
                      int32_t H, int32_t N_CTX, int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream) {
    return qf::forward(Q, K, V, Out, nullptr, sm_rscale, exp_M, req_M, l_M, acc_M, strides, Z, H, N_CTX, HEAD_DIM,
                       flags, stream);
}

int qflash_hip_masked_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out,
                             const int32_t* attn_bias, int32_t sm_rscale, int32_t exp_M, int32_t req_M,
                             int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z, int32_t H,
                             int32_t N_CTX, int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream) {
    if (!attn_bias) return qf::fail(QFLASH_HIP_EINVAL, "attn_bias is null");
    return qf::forward(Q, K, V, Out, attn_bias, sm_rscale, exp_M, req_M, l_M, acc_M, strides, Z, H, N_CTX,
                       HEAD_DIM, flags, stream);
}

int qflash_hip_window_kernel(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* Out,
                             const int32_t* attn_bias, int32_t sm_rscale, int32_t exp_M, int32_t req_M,
                             int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z, int32_t H,
                             int32_t N_CTX, int32_t HEAD_DIM, int32_t bias_zmod, const qflash_hip_flags* flags,
                             void* stream) {
    if (!attn_bias) return qf::fail(QFLASH_HIP_EINVAL, "attn_bias is null");
    if (bias_zmod < 1) return qf::fail(QFLASH_HIP_EINVAL, "bias_zmod must be >= 1 (got %d)", bias_zmod);
    return qf::forward(Q, K, V, Out, attn_bias, sm_rscale, exp_M, req_M, l_M, acc_M, strides, Z, H, N_CTX,
                       HEAD_DIM, flags, stream, bias_zmod);
}

int qflash_hip_forward(const int8_t* Q, const int8_t* K, const int8_t* V, void* Out, int32_t out_dtype,
                       const void* o_scale, const int32_t* attn_bias, int32_t bias_zmod, int32_t sm_rscale,
                       int32_t exp_M, int32_t req_M, int32_t l_M, int32_t acc_M, const int64_t* strides, int32_t Z,
                       int32_t H, int32_t N_CTX, int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream) {
    if (bias_zmod < 0 || (bias_zmod > 0 && !attn_bias))
        return qf::fail(QFLASH_HIP_EINVAL, "bias_zmod %d needs a bias (>= 0)", bias_zmod);
    return qf::forward(Q, K, V, Out, attn_bias, sm_rscale, exp_M, req_M, l_M, acc_M, strides, Z, H, N_CTX, HEAD_DIM,
                       flags, stream, bias_zmod, out_dtype, o_scale);
}

int qflash_hip_constants(const void* scales, int32_t dtype, double scale, int32_t N_CTX, int32_t HEAD_DIM,
                         int32_t masked, const qflash_hip_flags* flags, int32_t* params, void* stream) {
    qf::g_err[0] = 0;
    if (!scales) return qf::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qf::Args a{};
    uint32_t hooks = 0;
    if (int rc = qf::constants_args(dtype, N_CTX, HEAD_DIM, flags, params, &a, &hooks)) return rc;
    hipLaunchKernelGGL(qf::constants_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, scales, dtype, scale, a,
                       masked ? 1 : 0, hooks, params);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qf::fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return QFLASH_HIP_OK;
}

int qflash_hip_scales_constants(const void* q, const void* k, const void* v, int32_t dtype,
                                const int64_t* shapes_strides, void* scales, uint32_t* workspace,
                                int64_t workspace_elems, double scale, int32_t N_CTX, int32_t HEAD_DIM, int32_t masked,
                                const qflash_hip_flags* flags, int32_t* params, void* stream) {
    qf::g_err[0] = 0;
    if (!scales) return qf::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qf::Args a{};
    uint32_t hooks = 0;
    if (int rc = qf::constants_args(dtype, N_CTX, HEAD_DIM, flags, params, &a, &hooks)) return rc;
    if (int rc = qfq::absmax_pass(q, k, v, dtype, shapes_strides, nullptr, workspace, workspace_elems, stream))
        return rc;
    const hipStream_t st = (hipStream_t)stream;
    const int32_t mk = masked ? 1 : 0;
    switch (dtype) {
        case QFLASH_HIP_F32:
            hipLaunchKernelGGL(qf::scales_constants_kernel<QFLASH_HIP_F32>, dim3(1), dim3(64), 0, st, workspace,
                               scales, scale, a, mk, hooks, params);
            break;
        case QFLASH_HIP_F16:
            hipLaunchKernelGGL(qf::scales_constants_kernel<QFLASH_HIP_F16>, dim3(1), dim3(64), 0, st, workspace,
                               scales, scale, a, mk, hooks, params);
            break;
        default:
            hipLaunchKernelGGL(qf::scales_constants_kernel<QFLASH_HIP_BF16>, dim3(1), dim3(64), 0, st, workspace,
                               scales, scale, a, mk, hooks, params);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qf::fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return QFLASH_HIP_OK;
}

int qflash_hip_forward_planned(const int8_t* Q, const int8_t* K, const int8_t* V, void* Out, int32_t out_dtype,
                               const void* o_scale, const int32_t* attn_bias, int32_t bias_zmod,
                               const int32_t* params, const int64_t* strides, int32_t Z, int32_t H, int32_t N_CTX,
                               int32_t HEAD_DIM, const qflash_hip_flags* flags, void* stream) {
    if (!params) return qf::fail(QFLASH_HIP_EINVAL, "params is null");
    if (bias_zmod < 0 || (bias_zmod > 0 && !attn_bias))
        return qf::fail(QFLASH_HIP_EINVAL, "bias_zmod %d needs a bias (>= 0)", bias_zmod);
    return qf::forward(Q, K, V, Out, attn_bias, 0, 0, 0, 0, 0, strides, Z, H, N_CTX, HEAD_DIM, flags, stream,
                       bias_zmod, out_dtype, o_scale, params);
}

const char* qflash_hip_last_error(void) { return qf::g_err; }

int qflash_hip_mfma_layout_check(const int8_t* A, const int8_t* B, int32_t* C, void* stream) {
    if (!A || !B || !C) return qf::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    hipLaunchKernelGGL(qf::mfma_layout_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, A, B, C);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qf::fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return QFLASH_HIP_OK;
}

int qflash_hip_lut_bounds(int32_t sm_rscale, int32_t exp_M, int32_t req_M, int32_t* lut_n, int32_t* lut_lim) {
    qferr::g_err[0] = 0;
    if (!lut_n || !lut_lim) return qferr::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qf::Args a{};
    a.rs = sm_rscale;
    a.eM = exp_M;
    a.rM = req_M;
    a.exp_mode = 1;
    qf::lut_bounds(a, lut_n, lut_lim);
    return QFLASH_HIP_OK;
}

int qflash_hip_far_bounds(int32_t sm_rscale, int32_t exp_M, int32_t req_M, int32_t* u_lo, int32_t* u_hi,
                          int32_t* p_far) {
    qferr::g_err[0] = 0;
    if (!u_lo || !u_hi || !p_far) return qferr::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qf::Args a{};
    a.rs = sm_rscale;
    a.eM = exp_M;
    a.rM = req_M;
    a.exp_mode = 1;
    int64_t lo, hi;
    qf::far_range(a, &lo, &hi, p_far);
    *u_lo = (int32_t)(lo < INT32_MAX ? lo : INT32_MAX);
    *u_hi = (int32_t)hi;
    return QFLASH_HIP_OK;
}

uint32_t qflash_hip_set_test_hooks(uint32_t bits) {
    return qf::g_hook_bits.exchange(bits & QFLASH_HIP_HOOK_ALL, std::memory_order_relaxed);
}

const char* qflash_hip_version(void) { return "qflash_hip 0.2 (gfx950)"; }

}  // extern "C"
