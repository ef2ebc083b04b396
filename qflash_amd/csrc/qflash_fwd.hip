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
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/qflash_hip.h"

namespace qf {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int32_t kNegInf = -(1 << 20);  // kernel.py:137
constexpr int kBN = 32;                   // kernel.py:27, one rescale step

struct Args {
    const int8_t* q;
    const int8_t* k;
    const int8_t* v;
    int8_t* o;
    const int32_t* bias;
    int64_t sq[4], sk[4], sv[4], so[4], sb[4];
    int32_t Z, H, N;
    int32_t rs, eM, rM, lM, aM;
    int32_t l_shift, acc_shift;
    int32_t exp_mode, l_mode, acc_mode;  // 1 = shift variant, 0 = idiv
    int32_t mblocks;                     // workgroups per (z, h)
};

// ----------------------------------------------------------------------------
// Integer primitives with the reference's (Triton) semantics: int32 wraps,
// `>>` by a count >= 32 (read as unsigned) gives the sign fill, `//`
// truncates.  AMD's 32-bit shifts use only the low 5 bits of the count, so
// the clamp is explicit.
__device__ __forceinline__ int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
__device__ __forceinline__ int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
__device__ __forceinline__ int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__device__ __forceinline__ int32_t sra(int32_t a, int32_t b) {
    return (uint32_t)b > 31u ? (a >> 31) : (a >> b);
}

// exp2_i32: kernel.py:40-59.
__device__ __forceinline__ int32_t exp2_i32(int32_t x, const Args& a) {
    int32_t q = a.exp_mode ? (wmul(x, a.eM) >> 16) : (wsub(0, x) / a.rs);
    int32_t r = wadd(x, wmul(q, a.rs));
    return sra(wadd(r >> 1, a.rs), q);
}

// requantize: kernel.py:62-64 (int8 wrap of the rounded product).
__device__ __forceinline__ int32_t requant(int32_t e, const Args& a) {
    return (int32_t)(int8_t)(wadd(wmul(e, a.rM), 1 << 15) >> 16);
}

// scale_release: kernel.py:67-82.
__device__ __forceinline__ int32_t release(int32_t x, int32_t alpha, int32_t M, int32_t shift, int32_t mode,
                                           int32_t rs) {
    if (mode) {
        uint64_t prod = (uint64_t)((int64_t)x * (int64_t)alpha) * (uint64_t)(int64_t)M;
        prod += 1ull << (shift - 1);
        return (int32_t)(uint32_t)(uint64_t)((int64_t)prod >> shift);
    }
    return wmul(x, alpha) / rs;
}

// fp32 -> int32 as the reference's CPU path does it: truncate, INT_MIN for
// NaN / inf / out of range (v_cvt_i32_f32 would saturate instead).
__device__ __forceinline__ int32_t cvt_x86(float f) {
    return (f >= -2147483648.0f && f < 2147483648.0f) ? (int32_t)f : (int32_t)0x80000000;
}

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Row (within a 32-row block) held by result register v of lane l.
__device__ __forceinline__ int crow(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// 16 bytes from global memory; `vec` = base 16-byte aligned and unit stride.
template <bool VEC>
__device__ __forceinline__ i32x4 load16(const int8_t* p, int64_t sd, bool valid) {
    i32x4 r = {0, 0, 0, 0};
    if (!valid) return r;
    if constexpr (VEC) {
        r = *reinterpret_cast<const i32x4*>(p);
    } else {
        uint32_t w[4] = {0, 0, 0, 0};
        for (int b = 0; b < 16; ++b) w[b >> 2] |= (uint32_t)(uint8_t)p[b * sd] << (8 * (b & 3));
        r = i32x4{(int32_t)w[0], (int32_t)w[1], (int32_t)w[2], (int32_t)w[3]};
    }
    return r;
}

template <bool VEC>
__device__ __forceinline__ uint32_t load4(const int8_t* p, int64_t sd, bool valid) {
    if (!valid) return 0;
    if constexpr (VEC) {
        return *reinterpret_cast<const uint32_t*>(p);
    } else {
        uint32_t w = 0;
        for (int b = 0; b < 4; ++b) w |= (uint32_t)(uint8_t)p[b * sd] << (8 * b);
        return w;
    }
}

// LDS tile geometry.  K: 32 rows of D bytes (+16 pad).  V^T: D rows of 32
// bytes (+16 pad); within a row, byte 16*g + b holds key 8*(b/4)+4*g+b%4,
// the key that S^T's result register b of lane-half g refers to.
template <int D>
struct Tile {
    static constexpr int RK = D + 16;
    static constexpr int RV = 48;
    static constexpr int KBYTES = 32 * RK;
    static constexpr int VBYTES = D * RV;
    static constexpr int BYTES = KBYTES + VBYTES;
};

// Stage keys [kstart, kstart+32) of K and V into LDS (zero past N).
template <int D, int NT, bool VEC>
__device__ __forceinline__ void stage_kv(const Args& a, const int8_t* kb, const int8_t* vb, int kstart,
                                         int8_t* lk, int8_t* lvt, int tid) {
    using T = Tile<D>;
    constexpr int KCH = 32 * (D / 16);
    for (int idx = tid; idx < KCH; idx += NT) {
        int r = idx / (D / 16), c = idx % (D / 16);
        int j = kstart + r;
        i32x4 x = load16<VEC>(kb + (int64_t)j * a.sk[2] + (int64_t)c * 16 * a.sk[3], a.sk[3], j < a.N);
        *reinterpret_cast<i32x4*>(lk + r * T::RK + c * 16) = x;
    }
    constexpr int VBL = 8 * (D / 4);
    for (int idx = tid; idx < VBL; idx += NT) {
        int kg = idx / (D / 4), dg = idx % (D / 4);
        uint32_t r4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int j = kstart + 4 * kg + i;
            r4[i] = load4<VEC>(vb + (int64_t)j * a.sv[2] + (int64_t)dg * 4 * a.sv[3], a.sv[3], j < a.N);
        }
        int off = (kg & 1) * 16 + (kg >> 1) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t c = ((r4[0] >> (8 * i)) & 0xffu) | (((r4[1] >> (8 * i)) & 0xffu) << 8) |
                         (((r4[2] >> (8 * i)) & 0xffu) << 16) | (((r4[3] >> (8 * i)) & 0xffu) << 24);
            *reinterpret_cast<uint32_t*>(lvt + (dg * 4 + i) * T::RV + off) = c;
        }
    }
}

// The reference algorithm with general (wrapping, clamping, 64-bit) integer
// arithmetic on every element: exact for any constants and inputs.
template <int D, int W, bool MASKED, bool VEC>
__global__ __launch_bounds__(64 * W) void fwd_general(Args a) {
    using T = Tile<D>;
    constexpr int NT = 64 * W;
    constexpr int DB = D / 32;  // 32-column blocks of the head dimension
    __shared__ __attribute__((aligned(16))) int8_t smem[T::BYTES];
    int8_t* lk = smem;
    int8_t* lvt = smem + T::KBYTES;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, g = lane >> 5;
    const int zh = blockIdx.x / a.mblocks;
    const int mb = blockIdx.x % a.mblocks;
    const int z = zh / a.H, h = zh % a.H;
    const int q0 = (mb * W + wave) * 32;
    const bool active = q0 < a.N;

    const int8_t* qb = a.q + z * a.sq[0] + h * a.sq[1];
    const int8_t* kb = a.k + z * a.sk[0] + h * a.sk[1];
    const int8_t* vb = a.v + z * a.sv[0] + h * a.sv[1];
    int8_t* ob = a.o + z * a.so[0] + h * a.so[1];

    // Q^T as the B operand: lane holds query q0+lq, head dims 32*db+16*g+[0,16).
    i32x4 qv[DB];
    const int qrow = q0 + lq;
#pragma unroll
    for (int db = 0; db < DB; ++db)
        qv[db] = load16<VEC>(qb + (int64_t)qrow * a.sq[2] + (int64_t)(db * 32 + g * 16) * a.sq[3], a.sq[3],
                             qrow < a.N);

    int32_t m = kNegInf, l = 1;  // kernel.py:138-139 (per query, S layout)
    i32x16 acc[DB];              // kernel.py:140 (O layout)
#pragma unroll
    for (int t = 0; t < DB; ++t) acc[t] = i32x16{};

    for (int kstart = 0; kstart < a.N; kstart += kBN) {  // kernel.py:147
        __syncthreads();
        stage_kv<D, NT, VEC>(a, kb, vb, kstart, lk, lvt, tid);
        __syncthreads();
        if (!active) continue;

        // S^T = K . Q^T  (kernel.py:153); s[v] = S[q0+lq][kstart+crow(v,lane)]
        i32x16 s = {};
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            i32x4 kf = *reinterpret_cast<const i32x4*>(lk + lq * T::RK + db * 32 + g * 16);
            s = mfma32(kf, qv[db], s);
        }
        int32_t mx = INT32_MIN;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            int key = kstart + crow(v, lane);
            int32_t x = s[v];
            if constexpr (MASKED) {  // kernel.py:250-253
                if (key < a.N && qrow < a.N)
                    x = wadd(x, a.bias[z * a.sb[0] + h * a.sb[1] + (int64_t)qrow * a.sb[2] +
                                       (int64_t)key * a.sb[3]]);
            }
            if (key >= a.N) x = kNegInf;  // kernel.py:154-156 (never true when N%32==0)
            s[v] = x;
            mx = max(mx, x);
        }
        mx = max(mx, __shfl_xor(mx, 32));
        const int32_t mn = max(m, mx);  // kernel.py:158
        int32_t lij = 0;
        uint32_t pk[4] = {0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 16; ++v) {  // kernel.py:159-162
            int32_t p = requant(exp2_i32(wsub(s[v], mn), a), a);
            lij += p;
            pk[v >> 2] |= ((uint32_t)p & 0xffu) << (8 * (v & 3));
        }
        lij += __shfl_xor(lij, 32);
        const int32_t alpha = exp2_i32(wsub(m, mn), a);  // kernel.py:163
        l = wadd(release(l, alpha, a.lM, a.l_shift, a.l_mode, a.rs), lij);  // kernel.py:164
        // kernel.py:165 - rescale acc; acc row crow(v,lane) needs that row's alpha
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            int32_t av = __shfl(alpha, crow(v, lane));
#pragma unroll
            for (int t = 0; t < DB; ++t) acc[t][v] = release(acc[t][v], av, a.aM, a.acc_shift, a.acc_mode, a.rs);
        }
        // O += P . V  (kernel.py:171)
        i32x4 pa = i32x4{(int32_t)pk[0], (int32_t)pk[1], (int32_t)pk[2], (int32_t)pk[3]};
#pragma unroll
        for (int t = 0; t < DB; ++t) {
            i32x4 vf = *reinterpret_cast<const i32x4*>(lvt + (t * 32 + lq) * T::RV + g * 16);
            acc[t] = mfma32(pa, vf, acc[t]);
        }
        m = mn;  // kernel.py:172
    }
    if (!active) return;
    // kernel.py:176-180: fp32 divide, fp32->int32, int32->int8, rows < N only.
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = crow(v, lane);
        const int32_t lv = __shfl(l, row);
        const int orow = q0 + row;
        if (orow >= a.N) continue;
        const float lf = (float)lv;
#pragma unroll
        for (int t = 0; t < DB; ++t) {
            int32_t code = cvt_x86(__fdiv_rn((float)acc[t][v], lf));
            ob[(int64_t)orow * a.so[2] + (int64_t)(t * 32 + lq) * a.so[3]] = (int8_t)code;
        }
    }
}

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
static thread_local char g_err[512];

static int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

template <int D, int W, bool MASKED>
static hipError_t launch_dw(const Args& a, bool vec, dim3 grid, hipStream_t st) {
    if (vec)
        hipLaunchKernelGGL((fwd_general<D, W, MASKED, true>), grid, dim3(64 * W), 0, st, a);
    else
        hipLaunchKernelGGL((fwd_general<D, W, MASKED, false>), grid, dim3(64 * W), 0, st, a);
    return hipGetLastError();
}

template <int D, bool MASKED>
static hipError_t launch_d(const Args& a, int W, bool vec, dim3 grid, hipStream_t st) {
    switch (W) {
        case 1: return launch_dw<D, 1, MASKED>(a, vec, grid, st);
        case 2: return launch_dw<D, 2, MASKED>(a, vec, grid, st);
        default: return launch_dw<D, 4, MASKED>(a, vec, grid, st);
    }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static int forward(const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* O, const int32_t* bias,
                   int32_t rs, int32_t eM, int32_t rM, int32_t lM, int32_t aM, const int64_t* strides,
                   int32_t Z, int32_t H, int32_t N, int32_t D, const qflash_hip_flags* flags, void* stream) {
    g_err[0] = 0;
    if (!Q || !K || !V || !O || !strides) return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (Z <= 0 || H <= 0 || N <= 0) return fail(QFLASH_HIP_EINVAL, "bad shape Z=%d H=%d N=%d", Z, H, N);
    if (D == 16)
        return fail(QFLASH_HIP_EHEADDIM, "HEAD_DIM=16 < BLOCK_N=32: the reference kernel rejects it "
                                         "(tl.static_assert(BLOCK_N <= HEAD_DIM))");
    if (D != 32 && D != 64 && D != 128 && D != 256)
        return fail(QFLASH_HIP_EHEADDIM, "HEAD_DIM=%d not in {32,64,128,256}", D);
    if (rs <= 0) return fail(QFLASH_HIP_EINVAL, "sm_rscale must be positive (got %d)", rs);
    qflash_hip_flags f = {1, 1, 1, 30, 30};
    if (flags) f = *flags;
    if (f.l_use_shift && (f.l_shift < 1 || f.l_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "l_shift %d outside 1..62", f.l_shift);
    if (f.acc_use_shift && (f.acc_shift < 1 || f.acc_shift > 62))
        return fail(QFLASH_HIP_EINVAL, "acc_shift %d outside 1..62", f.acc_shift);
    if ((int64_t)Z * H > (int64_t)INT32_MAX / 64) return fail(QFLASH_HIP_EINVAL, "Z*H too large");

    Args a;
    a.q = Q; a.k = K; a.v = V; a.o = O; a.bias = bias;
    for (int i = 0; i < 4; ++i) {
        a.sq[i] = strides[i];
        a.sk[i] = strides[4 + i];
        a.sv[i] = strides[8 + i];
        a.so[i] = strides[12 + i];
        a.sb[i] = bias ? strides[16 + i] : 0;
    }
    a.Z = Z; a.H = H; a.N = N;
    a.rs = rs; a.eM = eM; a.rM = rM; a.lM = lM; a.aM = aM;
    a.l_shift = f.l_shift; a.acc_shift = f.acc_shift;
    a.exp_mode = f.exp_use_shift != 0; a.l_mode = f.l_use_shift != 0; a.acc_mode = f.acc_use_shift != 0;

    // 16-byte vector loads need unit head-dim stride and 16-byte aligned rows.
    bool vec = a.sq[3] == 1 && a.sk[3] == 1 && a.sv[3] == 1 && aligned16(Q) && aligned16(K) && aligned16(V);
    for (int i = 0; i < 3 && vec; ++i)
        vec = (a.sq[i] % 16 == 0) && (a.sk[i] % 16 == 0) && (a.sv[i] % 16 == 0);

    const int blocks32 = (N + 31) / 32;
    const int W = blocks32 >= 4 ? 4 : (blocks32 >= 2 ? 2 : 1);
    a.mblocks = (blocks32 + W - 1) / W;
    const int64_t nwg = (int64_t)Z * H * a.mblocks;
    if (nwg > INT32_MAX) return fail(QFLASH_HIP_EINVAL, "grid too large");
    dim3 grid((unsigned)nwg);
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    const bool masked = bias != nullptr;
#define QF_CASE(DD)                                                                        \
    case DD:                                                                               \
        e = masked ? launch_d<DD, true>(a, W, vec, grid, st) : launch_d<DD, false>(a, W, vec, grid, st); \
        break;
    switch (D) {
        QF_CASE(32)
        QF_CASE(64)
        QF_CASE(128)
        default:
            e = masked ? launch_d<256, true>(a, W, vec, grid, st) : launch_d<256, false>(a, W, vec, grid, st);
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

const char* qflash_hip_last_error(void) { return qf::g_err; }

int qflash_hip_mfma_layout_check(const int8_t* A, const int8_t* B, int32_t* C, void* stream) {
    if (!A || !B || !C) return qf::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    hipLaunchKernelGGL(qf::mfma_layout_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, A, B, C);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return qf::fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return QFLASH_HIP_OK;
}

const char* qflash_hip_version(void) { return "qflash_hip 0.1 (gfx950)"; }

}  // extern "C"
