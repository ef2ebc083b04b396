// Kernels of the integer-only attention forward (gfx950), shared by the
// translation units of libqflash_hip.so: qflash_fwd.hip (host logic and C
// ABI) and qflash_fwd_inst.hip (compiled once per head dim and masking, so
// that the instantiations build in parallel).
//
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
#pragma once
#include <cstring>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <atomic>
#include <utility>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qflash_hip.h"
#include "qf_common.h"

namespace qf {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int32_t kNegInf = -(1 << 20);  // kernel.py:137
#ifndef QF_FAST_WAVES_D64
#define QF_FAST_WAVES_D64 4
#endif
constexpr int kBN = 32;                   // kernel.py:27, one rescale step
constexpr int kLutMax = 4096;             // bytes of LDS for the p(u) table of the fast kernel
// The unmasked fast kernel carries every score (and the running max) plus
// kScoreBias: one extra MFMA of two all-(-128) operands starts each score tile
// at 32 * 128 * 128.  Every difference the algorithm takes is unchanged, and a
// wave whose scores stay above -kScoreBias + kLutMax (128 * ||q_row||_1 below
// that) has all scores and table thresholds positive, so one saturating
// subtraction per score gives its table index.
constexpr int32_t kScoreBias = 32 * 128 * 128;

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
    // fast path (set by the host after proving its guards, see choose_path)
    int32_t id_ok;   // acc rescale by alpha == sm_rscale is the identity (bound on |acc|)
    int32_t x_safe;  // masked: largest |s - m'| the 24-bit exp path accepts
    int32_t eps_abs; // | |eM|*rs - 2^16 |
    int32_t e_acc;   // | rs*acc_M - 2^acc_shift |
    int32_t force_robust;  // test hook: general arithmetic for every score, alpha and l
    int32_t n_wg;    // workgroups in the grid (XCD-aware order)
    int32_t bias_zmod;  // > 0: the bias of batch index z is bias[z % bias_zmod] (window-periodic)
    int32_t bias_vec;   // bias rows have unit key stride and non-negative strides: 16-byte buffer loads
    // exp2 + requantisation by table (see lut_pack_vt): p(u) = p(min(u, lut_n - 1))
    // for u = m' - s in [0, lut_lim], the table holding p(0 .. lut_n - 1) in reverse
    int32_t lut_n;      // table entries (the last one 0), 0 = no table
    int32_t lut_lim;
    // masked table path: columns whose biased score is negative ("far" ones,
    // such as those of a -2^20 mask) read entry lut_n = far_p, which is p(u)
    // for every u in [far_lo + 1, far_hi] (far_bounds); far_hi = 0: no such range
    int32_t far_lo, far_hi, far_p;
    // output: int8 codes at `o` (out_dt == QFLASH_HIP_I8), or RN_T(code * o_scale)
    // of type out_dt at the same element offsets of `out_t` (qflash/kernel.py:351)
    void* out_t;
    int32_t out_dt;
    const void* o_scale;
    // constants and fast-path plan in device memory (qflash_hip_constants), or
    // nullptr: then the fields above hold them
    const int32_t* params;
    int32_t general_only;  // with params: the general kernel runs whatever the plan says (layout)
};

// The p(u) table of a launch on host constants, formed by the host and passed
// with the kernel arguments (fwd_fast_table: the workgroups copy it into LDS
// instead of computing it) when it holds at most 4 kLutArgWords bytes and
// rows have at most 64 keys (two key steps per wave, where the table's
// arithmetic is a large part of a wave: cfg4 -4 % measured on MI355X).
constexpr int kLutArgWords = 256;
struct LutArg {
    uint32_t w[kLutArgWords];
};
__host__ __device__ __forceinline__ bool lut_in_args(const Args& a) {
    return a.lut_n > 0 && a.lut_n < 4 * kLutArgWords && a.N <= 64;
}

// Words of the device parameter block written by qflash_hip_constants.
enum ParamWord : int {
    kPStatus = 0, kPRs, kPEm, kPRm, kPLm, kPAm, kPFast, kPIdOk, kPXSafe, kPEpsAbs, kPEAcc, kPLutN, kPLutLim,
    kPSmScale = 14,  // double, words 14-15
    kPFarLo = 16, kPFarHi, kPFarP
};
static_assert(kPFarP < QFLASH_HIP_PARAMS_WORDS, "parameter block size");

// The constants and plan fields of `a` from its device parameter block.
__device__ __forceinline__ void load_params(Args& a) {
    const int32_t* p = a.params;
    a.rs = p[kPRs];
    a.eM = p[kPEm];
    a.rM = p[kPRm];
    a.lM = p[kPLm];
    a.aM = p[kPAm];
    a.id_ok = p[kPIdOk];
    a.x_safe = p[kPXSafe];
    a.eps_abs = p[kPEpsAbs];
    a.e_acc = p[kPEAcc];
    a.lut_n = p[kPLutN];
    a.lut_lim = p[kPLutLim];
    a.far_lo = p[kPFarLo];
    a.far_hi = p[kPFarHi];
    a.far_p = p[kPFarP];
}

__device__ __forceinline__ int out_esize(int dt) { return dt == QFLASH_HIP_I8 ? 1 : (dt == QFLASH_HIP_F32 ? 4 : 2); }

// o * o_scale in torch's arithmetic: the int8 code and the scale as fp32, one
// rounding to the output type.
__device__ __forceinline__ float scale_value(const Args& a) {
    if (a.out_dt == QFLASH_HIP_F32) return *reinterpret_cast<const float*>(a.o_scale);
    const uint32_t h = *reinterpret_cast<const uint16_t*>(a.o_scale);
    return a.out_dt == QFLASH_HIP_F16 ? __half2float(__ushort_as_half((unsigned short)h)) : __uint_as_float(h << 16);
}

// Stores the output element of `code` at element offset voff + soff of the
// head's output buffer (rsrc covers the head; offsets in elements).
template <int OUT>
__device__ __forceinline__ void put_out(__amdgpu_buffer_rsrc_t rsrc, int32_t code, int32_t voff, int32_t soff,
                                        float os) {
    if constexpr (OUT == QFLASH_HIP_I8) {
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)code, rsrc, voff, soff, 0);
    } else if constexpr (OUT == QFLASH_HIP_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint((float)(int8_t)code * os), rsrc, 4 * voff, 4 * soff, 0);
    } else if constexpr (OUT == QFLASH_HIP_F16) {
        __builtin_amdgcn_raw_buffer_store_b16(__half_as_ushort(__float2half_rn((float)(int8_t)code * os)), rsrc,
                                              2 * voff, 2 * soff, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)qf_bf16_bits((float)(int8_t)code * os), rsrc, 2 * voff,
                                              2 * soff, 0);
    }
}

// Calls f.template operator()<OUT>() for the output type of the launch (one
// uniform branch per wave instead of one per stored element).
template <typename F>
__device__ __forceinline__ void with_out_type(int dt, F&& f) {
    switch (dt) {
        case QFLASH_HIP_I8: f.template operator()<QFLASH_HIP_I8>(); break;
        case QFLASH_HIP_F32: f.template operator()<QFLASH_HIP_F32>(); break;
        case QFLASH_HIP_F16: f.template operator()<QFLASH_HIP_F16>(); break;
        default: f.template operator()<QFLASH_HIP_BF16>();
    }
}

// Buffer over one head's output, ending after row N-1 (element strides so).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(const Args& a, int z, int h, int D) {
    const int es = out_esize(a.out_dt);
    void* base = a.out_dt == QFLASH_HIP_I8 ? (void*)(a.o + z * a.so[0] + h * a.so[1])
                                           : (void*)((char*)a.out_t + (z * a.so[0] + h * a.so[1]) * es);
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, ((a.N - 1) * (int32_t)a.so[2] + (D - 1) * (int32_t)a.so[3] + 1) * es,
                                             0x00020000);
}

// ----------------------------------------------------------------------------
// Integer primitives with the reference's (Triton) semantics: int32 wraps,
// `>>` by a count >= 32 (read as unsigned) gives the sign fill, `//`
// truncates.  AMD's 32-bit shifts use only the low 5 bits of the count, so
// the clamp is explicit.
__host__ __device__ __forceinline__ int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
__host__ __device__ __forceinline__ int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
__host__ __device__ __forceinline__ int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__host__ __device__ __forceinline__ int32_t sra(int32_t a, int32_t b) {
    return (uint32_t)b > 31u ? (a >> 31) : (a >> b);
}

// `//` of two int32 values: truncating, and INT32_MIN // -1 wraps to INT32_MIN
// (numpy's int32 arithmetic, which the Triton interpreter runs).
__host__ __device__ __forceinline__ int32_t tdiv(int32_t a, int32_t b) { return (int32_t)((int64_t)a / b); }

// exp2_i32: kernel.py:40-59.
__host__ __device__ __forceinline__ int32_t exp2_i32(int32_t x, const Args& a) {
    int32_t q = a.exp_mode ? (wmul(x, a.eM) >> 16) : tdiv(wsub(0, x), a.rs);
    int32_t r = wadd(x, wmul(q, a.rs));
    return sra(wadd(r >> 1, a.rs), q);
}

// requantize: kernel.py:62-64 (int8 wrap of the rounded product).
__host__ __device__ __forceinline__ int32_t requant(int32_t e, const Args& a) {
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
    return tdiv(wmul(x, alpha), rs);
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
// Key column kstart + crow(v, lane) lies past N (a padded column of the last
// step) iff 8*(v>>2) + (v&3) >= tcut, tcut = N - kstart - 4*(lane>>5): one
// per-lane value and compile-time constants, instead of 16 column indices.
__device__ __forceinline__ bool padded(int v, int32_t tcut) { return 8 * (v >> 2) + (v & 3) >= tcut; }

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
// Workgroup id -> (head, query block) so that consecutive blocks of one head
// run on the same XCD (workgroups are dealt to the 8 XCDs round-robin).
using qfs::xcd_order;

// One workgroup of the general kernel: row block blk % mblocks of head
// blk / mblocks, with LDS at smem (Tile<D>::BYTES).
template <int D, int W, bool MASKED, bool VEC>
__device__ __forceinline__ void general_block(const Args& a, int blk, int8_t* smem) {
    using T = Tile<D>;
    constexpr int NT = 64 * W;
    constexpr int DB = D / 32;  // 32-column blocks of the head dimension
    int8_t* lk = smem;
    int8_t* lvt = smem + T::KBYTES;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, g = lane >> 5;
    const int zh = blk / a.mblocks;
    const int mb = blk % a.mblocks;
    const int z = zh / a.H, h = zh % a.H;
    const int q0 = (mb * W + wave) * 32;
    const bool active = q0 < a.N;

    const int8_t* qb = a.q + z * a.sq[0] + h * a.sq[1];
    const int8_t* kb = a.k + z * a.sk[0] + h * a.sk[1];
    const int8_t* vb = a.v + z * a.sv[0] + h * a.sv[1];

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
                    x = wadd(x, a.bias[(a.bias_zmod ? z % a.bias_zmod : z) * a.sb[0] + h * a.sb[1] +
                                       (int64_t)qrow * a.sb[2] + (int64_t)key * a.sb[3]]);
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
    const __amdgpu_buffer_rsrc_t orsrc = out_rsrc(a, z, h, D);
    const float os = a.out_dt == QFLASH_HIP_I8 ? 0.f : scale_value(a);
    with_out_type(a.out_dt, [&]<int OUT>() {
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
                put_out<OUT>(orsrc, code, (int32_t)(orow * a.so[2] + (t * 32 + lq) * a.so[3]), 0, os);
            }
        }
    });
}

// Under a plan (constants in device memory: qflash_hip_constants) it runs
// unless they failed or the fast kernel serves them.
template <int D, int W, bool MASKED, bool VEC>
__global__ __launch_bounds__(64 * W) void fwd_general(Args a) {
    __shared__ __attribute__((aligned(16))) int8_t smem[Tile<D>::BYTES];
    if (a.params) {
        if (a.params[kPStatus] != 0 || (!a.general_only && a.params[kPFast])) return;
        load_params(a);
    }
    // consecutive row blocks of a head on one XCD, as in the fast kernel: K and V
    // of the head come from HBM once and then from that XCD's L2
    general_block<D, W, MASKED, VEC>(a, xcd_order(blockIdx.x, a.n_wg), smem);
}

// ----------------------------------------------------------------------------
// Fast exact path.
//
// Valid when the host has proved (choose_path): shift exp variant, shift
// rescale variants with shifts <= 30, eM <= 0, |eM| < 2^23, 0 < rs < 2^15,
// |rM| < 2^23, |eM|*rs < 2^17, and for every real key column
// |x| = |s - m'| <= X with X*|eM| <= 2^31 - 2^17 and the bound on |a| below
// under 2^22 (unmasked: X = 2*D*2^14 from |s| <= D*128*128; masked: checked
// per wave and step, general arithmetic otherwise).  Then q = (x*eM) >> 16 >= 0
// never wraps and, with a = x + (q+2)*rs,
//     E(x) = ((r >> 1) + rs) >> q  =  a >> min(q + 1, 31)        (r = x + q*rs)
// which costs six VALU ops per score with 24-bit multiplies:
//     t  = s*eM + c1          c1 = wrap32(-m'*eM) + 2^16   (t = x*eM + 2^16)
//     q1 = t >> 16            (= q + 1)
//     a  = s + q1*rs + c3     c3 = rs - m'
//     E  = a >> min_u32(q1, 31)
//     y  = E*rM + 2^15        p = int8(bits 16..23 of y)
// Padded key columns (j >= N) use p(NEG_INF - m') evaluated exactly once per
// row.  acc is rescaled only for rows whose running max changed (the rescale
// by alpha = E(0) = rs is the identity while |acc*(rs*acc_M - 2^30)| < 2^29,
// which the host proves from N), a register pair at a time, with one
// 64-bit multiply-add per element.
__device__ __forceinline__ int32_t mad24(int32_t a, int32_t b, int32_t c) { return __mul24(a, b) + c; }
__device__ __forceinline__ int32_t max3(int32_t a, int32_t b, int32_t c) { return max(max(a, b), c); }
__device__ __forceinline__ int32_t min3(int32_t a, int32_t b, int32_t c) { return min(min(a, b), c); }

// K / V stages of 32 * STEPS keys (STEPS rescale steps) per LDS buffer.  Both tiles
// hold rows of D bytes exactly as in HBM, copied there by buffer loads that
// write LDS directly (no registers, no VALU), with the 16-byte chunks of each
// row permuted by an XOR swizzle so that the MFMA operand reads are free of
// bank conflicts:
//   K: chunk c of key k sits at position c ^ kswz(k); lanes 0-7 of a
//      ds_read_b128 read keys 0-7 at one chunk -> 8 distinct 4-bank groups;
//   V: chunk c of key k sits at position c ^ vswz(k); V^T fragments are read
//      with ds_read_b64_tr_b8, whose 16-lane groups read 8 keys x 2 halves of a
//      chunk -> 16 distinct 2-bank groups.
// Keys past N read as zeros (buffer range check), as the reference's
// boundary-checked loads of K and V do.
// Steps per stage: 4 at D = 64 with 4 waves per workgroup (one barrier per 128
// keys; 2.3 % faster than 2 at ViT-B/384, and 36 KiB of LDS per workgroup
// keeps 4 workgroups per CU); 2 otherwise, where the LDS of more, smaller
// workgroups (D = 32 at 6 waves per SIMD, W < 4) or of D = 128 limits it.
#ifdef QF_STAGE_STEPS
template <int D, int W> constexpr int stage_steps() { return QF_STAGE_STEPS; }
#else
template <int D, int W> constexpr int stage_steps() { return D == 64 && W == 4 ? 4 : 2; }
#endif
template <int D, int W = 4>
struct Stage {
    static constexpr int STEPS = stage_steps<D, W>();  // 32-key rescale steps per stage
    static_assert(STEPS >= 1 && STEPS <= 4, "stages of at most 128 keys (host offset check)");
    static constexpr int KEYS = 32 * STEPS;
    static constexpr int CPR = D / 16;       // 16-byte chunks per row
    static constexpr int KBYTES = KEYS * D;  // one tile (K or V)
    static constexpr int BYTES = 2 * KBYTES;
    static constexpr int SLOTS = KEYS * CPR;  // 16-byte slots per tile
    __device__ static int kswz(int k) {
        return D == 32 ? (k >> 2) & 1 : (D == 64 ? (k >> 1) & 3 : k & 7);
    }
    __device__ static int vswz(int k) {
        return D == 32 ? (k >> 3) & 1
                       : (D == 64 ? ((k >> 1) & 1) | (((k >> 3) & 1) << 1) : (k & 3) | (((k >> 3) & 1) << 2));
    }
};

// Per-lane byte offsets of the MFMA fragments inside a tile (keys 0-31 of it;
// the second step of the stage adds 32*D).
//   K (A operand of S^T = K.Q^T): key lq, chunk 2*db + g.
//   V (B operand of O = P.V, read transposed): ds_read_b64_tr_b8 gives lane j
//   of a 16-lane group byte (j & 7) of the 8-byte rows addressed by lanes
//   2b + (j >> 3), b = 0..7.  Lane i = 2b + h of group G therefore addresses
//   key 8(b>>2) + 4g + (b&3) (+16 for the fragment's second 8 bytes) and the
//   8-byte unit 4t + 2(G&1) + h of the row, so that lane n + 32g receives
//   column 32t + n of the 16 keys the P operand's byte order expects
//   (byte 16g + b' <-> key 8(b'>>2) + 4g + (b'&3)).
template <int D>
struct Frag {
    static constexpr int DB = D / 32;
    int32_t k[DB], v[DB];
    __device__ Frag(int lane) {
        using S = Stage<D>;
        const int lq = lane & 31, g = lane >> 5;
        const int i = lane & 15, G = lane >> 4, b = i >> 1, h = i & 1;
        const int kv = 8 * (b >> 2) + 4 * (G >> 1) + (b & 3);
#pragma unroll
        for (int db = 0; db < DB; ++db) k[db] = lq * D + 16 * ((2 * db + g) ^ S::kswz(lq));
#pragma unroll
        for (int t = 0; t < DB; ++t) {
            const int u = 4 * t + 2 * (G & 1) + h;
            v[t] = kv * D + 16 * ((u >> 1) ^ S::vswz(kv)) + 8 * (u & 1);
        }
    }
};

// V^T fragments of one step (B operands of O = P.V): two ds_read_b64_tr_b8
// per 32-column block, the second 16 keys (16*D bytes) further.  Written as
// one asm block with its own lgkmcnt wait: through the builtin, the compiler
// would also wait for the in-flight copy of the NEXT stage (vmcnt(0)) before
// every read, as it cannot tell the two LDS buffers apart.  The tile sits at
// LDS address vbase + VO: the steps of the main loop pass the constant part
// as the immediate VO (vbase is then the LDS array's own address, a
// constant the compiler folds), so their reads need no address arithmetic.
#define QF_TR32                                           \
    "ds_read_b64_tr_b8 %[t0], %[b0] offset:%c[vo]\n\t"    \
    "ds_read_b64_tr_b8 %[t1], %[b0] offset:%c[vo2]\n\t"
#define QF_TR64 QF_TR32                                   \
    "ds_read_b64_tr_b8 %[t2], %[b1] offset:%c[vo]\n\t"    \
    "ds_read_b64_tr_b8 %[t3], %[b1] offset:%c[vo2]\n\t"
#define QF_TR128 QF_TR64                                  \
    "ds_read_b64_tr_b8 %[t4], %[b2] offset:%c[vo]\n\t"    \
    "ds_read_b64_tr_b8 %[t5], %[b2] offset:%c[vo2]\n\t"   \
    "ds_read_b64_tr_b8 %[t6], %[b3] offset:%c[vo]\n\t"    \
    "ds_read_b64_tr_b8 %[t7], %[b3] offset:%c[vo2]\n\t"
#define QF_T32 [t0] "=&v"(t[0]), [t1] "=&v"(t[1])
#define QF_T64 QF_T32, [t2] "=&v"(t[2]), [t3] "=&v"(t[3])
#define QF_T128 QF_T64, [t4] "=&v"(t[4]), [t5] "=&v"(t[5]), [t6] "=&v"(t[6]), [t7] "=&v"(t[7])
#define QF_B32 [b0] "v"(vbase + fr.v[0]), [vo] "i"(VO), [vo2] "i"(VO + 16 * D)
#define QF_B64 QF_B32, [b1] "v"(vbase + fr.v[1])
#define QF_B128 QF_B64, [b2] "v"(vbase + fr.v[2]), [b3] "v"(vbase + fr.v[3])

// LDS address of a shared-memory pointer
__device__ __forceinline__ uint32_t lds_addr(const int8_t* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)p;
}

template <int D, int VO>
__device__ __forceinline__ void read_vt(i32x4* vf, uint32_t vbase, const Frag<D>& fr) {
    static_assert(VO >= 0 && VO + 16 * D < 65536, "offsets must fit the 16-bit LDS immediate");
    typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
    i32x2 t[2 * (D / 32)];
    if constexpr (D == 32)
        asm volatile(QF_TR32 "s_waitcnt lgkmcnt(0)" : QF_T32 : QF_B32);
    else if constexpr (D == 64)
        asm volatile(QF_TR64 "s_waitcnt lgkmcnt(0)" : QF_T64 : QF_B64);
    else
        asm volatile(QF_TR128 "s_waitcnt lgkmcnt(0)" : QF_T128 : QF_B128);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) vf[i] = i32x4{t[2 * i].x, t[2 * i].y, t[2 * i + 1].x, t[2 * i + 1].y};
}

// Direct HBM -> LDS copies of one stage: slot s of a tile (16 bytes at byte
// 16*s) holds chunk (s % CPR) ^ swz(key) of key s / CPR; wave w of the
// workgroup fills slots [r*NT + 64w, r*NT + 64w + 64) in round r.
template <int D, int W>
struct StageDma {
    using S = Stage<D, W>;
    static constexpr int NT = 64 * W;
    static constexpr int R = (S::SLOTS + NT - 1) / NT;
    uint32_t vk[R], vv[R];
    __device__ __forceinline__ StageDma(const Args& a, int wave, int lane) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int slot = r * NT + wave * 64 + lane;
            const int key = slot / S::CPR, pos = slot % S::CPR;
            vk[r] = (uint32_t)(key * (int32_t)a.sk[2] + 16 * (pos ^ S::kswz(key)));
            vv[r] = (uint32_t)(key * (int32_t)a.sv[2] + 16 * (pos ^ S::vswz(key)));
        }
    }
    __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int8_t* buf,
                                          int kstart, const Args& a, int wave) const {
        const uint32_t sk = (uint32_t)(kstart * (int32_t)a.sk[2]), sv = (uint32_t)(kstart * (int32_t)a.sv[2]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r * NT + wave * 64 < S::SLOTS) {
                int8_t* lk = buf + (r * NT + wave * 64) * 16;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)lk, 16, vk[r],
                                                         sk, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rv, (__attribute__((address_space(3))) void*)(lk + S::KBYTES), 16, vv[r], sv, 0, 0);
            }
        }
    }
};

// The copy of a row block's first K / V stage into stage buffer 0 (fast_rows
// builds the same buffers and offsets for the later stages), issued where it
// is called: before the Q loads and the table fill, so their latencies overlap.
template <int D, int W>
__device__ __forceinline__ void first_stage(const Args& a, const int8_t* kb, const int8_t* vb, int8_t* smem,
                                            int wave, int lane) {
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)kb, 0, (a.N - 1) * (int32_t)a.sk[2] + D, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vb, 0, (a.N - 1) * (int32_t)a.sv[2] + D, 0x00020000);
    const StageDma<D, W> dma(a, wave, lane);
    dma.issue(rk, rv, smem, 0, a, wave);
    asm volatile("" ::: "memory");
}

// Completion of this wave's LDS copies (vmcnt), then the workgroup barrier.
__device__ __forceinline__ void stage_sync() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
}


__device__ __forceinline__ int32_t rescale_fast(int32_t x, int32_t A, int64_t half, int32_t sh) {
    const int64_t p = (int64_t)x * (int64_t)A + half;
    return (int32_t)__builtin_amdgcn_alignbit((uint32_t)(p >> 32), (uint32_t)p, (uint32_t)sh);
}

// Value of the other lane-half (lane ^ 32) combined with this lane's: the
// two results of v_permlane32_swap are {this, other} in some order.
__device__ __forceinline__ int32_t half_max(int32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return max((int32_t)r[0], (int32_t)r[1]);
}
// max(v, v of lane ^ 32, c)
__device__ __forceinline__ int32_t half_max3(int32_t v, int32_t c) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return max3((int32_t)r[0], (int32_t)r[1], c);
}
__device__ __forceinline__ int32_t half_sum(int32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int32_t)(r[0] + r[1]);
}
__device__ __forceinline__ int32_t half_min(int32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return min((int32_t)r[0], (int32_t)r[1]);
}
// Keeps the compiler from distributing a per-row constant back into the
// per-element expressions (it would turn one mad into mul + sub + add).
__device__ __forceinline__ int32_t opaque(int32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// E(x) for one x <= 0 inside the fast path's range (see the comment above).
__device__ __forceinline__ int32_t exp2_fast(int32_t x, int32_t eM, int32_t rs) {
    const int32_t t = mad24(x, eM, 1 << 16);
    const int32_t q1 = t >> 16;
    const int32_t av = x + __mul24(q1, rs) + rs;
    return av >> min((uint32_t)q1, 31u);
}

// exp2 + requantisation by table lookup.  For x = s - m' = -u the
// reference's p(x) = int8(requant(exp2(x))) depends on u alone, and past a
// host-computed point it is 0 over a long range: with q = floor(u*|eM| / 2^16)
// (no int32 wrap while u*|eM| < 2^31) and kappa = |eM|*rs - 2^16, the
// remainder r = q*rs - u lies in (u*kappa/2^16 - rs, u*kappa/2^16], so
// E = ((r >> 1) + rs) >> q is 0 once 2^q exceeds rs + max(0, r/2) (true for
// q >= bitlen(rs) + 3 when kappa <= 2|eM|) as long as r >= -2rs (all u when
// kappa >= 0, u <= rs*2^16/|kappa| otherwise); p(E = 0) = 0.  The table holds
// p(u) for u = 0 .. lut_n - 1 (its last entry 0) in reverse order, entry
// j = lut_n - 1 - u, so that the index of every u up to lut_lim is
// max(s - thr, 0) with thr = m' - (lut_n - 1): one saturating subtraction per
// score when scores and thr are positive (kScoreBias), a subtraction and a
// max otherwise.  A step uses the table only when all of its real columns
// have u <= lut_lim.  Clamping also makes the many far-off columns of a step
// read one byte (a broadcast, no LDS bank conflict): with the addresses left
// spread over a table of 8 KB the kernel is slower (measured).  The table
// lives in LDS after the K / V stages, at the compile-time LDS address LUT
// (the kernel's only LDS array starts at address 0; the kernel checks it),
// which the byte loads take as their immediate offset.  Each byte load fills
// bits 0-7 of its own register (the half-register d16 loads are no use here:
// with SRAM ECC on, as on MI355X, they clear the other half), and three
// shift-ors pack four p values into the MFMA A operand's byte order.  The
// step's V^T fragment reads (read_vt) go out in the same asm block, so one
// LDS wait covers both; the compiler's own packing of byte loads would take
// 4.5 instructions per four bytes, and it would wait for the in-flight
// stage copy before every LDS read.
#define QF_L(i) "ds_read_u8 %" #i ", %" #i " offset:%c[lut]\n\t"
#define QF_P(a, b, c, d)                                      \
    "v_lshl_or_b32 %" #a ", %" #b ", 8, %" #a "\n\t"            \
    "v_lshl_or_b32 %" #c ", %" #d ", 8, %" #c "\n\t"            \
    "v_lshl_or_b32 %" #a ", %" #c ", 16, %" #a "\n\t"
#define QF_LOADS4 QF_L(0) QF_L(1) QF_L(2) QF_L(3)
#define QF_LOADS8 QF_LOADS4 QF_L(4) QF_L(5) QF_L(6) QF_L(7)
#define QF_LOADS12 QF_LOADS8 QF_L(8) QF_L(9) QF_L(10) QF_L(11)
#define QF_LOADS16 QF_LOADS12 QF_L(12) QF_L(13) QF_L(14) QF_L(15)
#define QF_PACK4 "s_waitcnt lgkmcnt(0)\n\t" QF_P(0, 1, 2, 3)
#define QF_PACK8 QF_PACK4 QF_P(4, 5, 6, 7)
#define QF_PACK12 QF_PACK8 QF_P(8, 9, 10, 11)
#define QF_PACK16 QF_PACK12 QF_P(12, 13, 14, 15)
#define QF_IDX4 "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3])
#define QF_IDX8 QF_IDX4, "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
#define QF_IDX12 QF_IDX8, "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11])
#define QF_IDX16 QF_IDX12, "+v"(r[12]), "+v"(r[13]), "+v"(r[14]), "+v"(r[15])
#define QF_TV_ASM(LOADS, PACK, IDX)                                                             \
    if constexpr (D == 32)                                                                      \
        asm volatile(LOADS QF_TR32 PACK : IDX, QF_T32 : QF_B32, [lut] "i"(LUT));                \
    else if constexpr (D == 64)                                                                 \
        asm volatile(LOADS QF_TR64 PACK : IDX, QF_T64 : QF_B64, [lut] "i"(LUT));                \
    else                                                                                        \
        asm volatile(LOADS QF_TR128 PACK : IDX, QF_T128 : QF_B128, [lut] "i"(LUT));
// The first TV score registers (TV = 16: all; TV = 4, 8, 12: a partial last
// step of at most 2*TV keys, whose registers TV..15 hold padded columns
// alone): pk[0 .. TV/4 - 1] (the others 0) and the V^T fragments of the tile
// at LDS address vbase + VO (read_vt).
template <int D, int LUT, int TV, int VO>
__device__ __forceinline__ void lut_pack_vt(uint32_t* pk, i32x4* vf, const uint32_t* idx, uint32_t vbase,
                                            const Frag<D>& fr) {
    static_assert(LUT >= 0 && LUT + kLutMax <= 65536, "table offset must fit the 16-bit LDS immediate");
    static_assert(VO >= 0 && VO + 16 * D < 65536, "offsets must fit the 16-bit LDS immediate");
    static_assert(TV == 4 || TV == 8 || TV == 12 || TV == 16, "4, 8, 12 or 16 registers");
    typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
    // each byte load writes its result over its own index register
    uint32_t r[TV];
#pragma unroll
    for (int i = 0; i < TV; ++i) r[i] = idx[i];
    i32x2 t[2 * (D / 32)];
    if constexpr (TV == 4) {
        QF_TV_ASM(QF_LOADS4, QF_PACK4, QF_IDX4)
    } else if constexpr (TV == 8) {
        QF_TV_ASM(QF_LOADS8, QF_PACK8, QF_IDX8)
    } else if constexpr (TV == 12) {
        QF_TV_ASM(QF_LOADS12, QF_PACK12, QF_IDX12)
    } else {
        QF_TV_ASM(QF_LOADS16, QF_PACK16, QF_IDX16)
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) pk[w] = 4 * w < TV ? r[4 * w < TV ? 4 * w : 0] : 0u;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) vf[i] = i32x4{t[2 * i].x, t[2 * i].y, t[2 * i + 1].x, t[2 * i + 1].y};
}
// The full-step table path with the table check of a wave whose rows the host
// bound does not cover (lut_mode 2): the loads go out first, and the check
// (every column of the lane within lut_lim of the row maximum:
// mn - min(s) <= lut_lim, unsigned) runs while they are in flight, instead of
// deciding, before the loads, whether to issue them.  Returns the lanes that
// pass; the caller falls back to the arithmetic unless all do.
#define QF_S16                                                                                            \
    [s0] "v"(s[0]), [s1] "v"(s[1]), [s2] "v"(s[2]), [s3] "v"(s[3]), [s4] "v"(s[4]), [s5] "v"(s[5]),          \
        [s6] "v"(s[6]), [s7] "v"(s[7]), [s8] "v"(s[8]), [s9] "v"(s[9]), [s10] "v"(s[10]), [s11] "v"(s[11]),   \
        [s12] "v"(s[12]), [s13] "v"(s[13]), [s14] "v"(s[14]), [s15] "v"(s[15]), [mn] "v"(mn), [lim] "s"(lim)
#define QF_CHECK                                          \
    "v_min3_i32 %[dm], %[s0], %[s1], %[s2]\n\t"           \
    "v_min3_i32 %[dm], %[dm], %[s3], %[s4]\n\t"           \
    "v_min3_i32 %[dm], %[dm], %[s5], %[s6]\n\t"           \
    "v_min3_i32 %[dm], %[dm], %[s7], %[s8]\n\t"           \
    "v_min3_i32 %[dm], %[dm], %[s9], %[s10]\n\t"          \
    "v_min3_i32 %[dm], %[dm], %[s11], %[s12]\n\t"         \
    "v_min3_i32 %[dm], %[dm], %[s13], %[s14]\n\t"         \
    "v_min_i32 %[dm], %[dm], %[s15]\n\t"                  \
    "v_sub_u32 %[dm], %[mn], %[dm]\n\t"                   \
    "v_cmp_ge_u32_e64 %[ok], %[lim], %[dm]\n\t"
template <int D, int LUT, int VO>
__device__ __forceinline__ uint64_t lut_pack_vt_check(uint32_t* pk, i32x4* vf, const uint32_t* idx, uint32_t vbase,
                                                      const Frag<D>& fr, const i32x16& s, int32_t mn, int32_t lim) {
    static_assert(LUT >= 0 && LUT + kLutMax <= 65536, "table offset must fit the 16-bit LDS immediate");
    static_assert(VO >= 0 && VO + 16 * D < 65536, "offsets must fit the 16-bit LDS immediate");
    typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
    uint32_t r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = idx[i];
    i32x2 t[2 * (D / 32)];
    uint64_t ok;
    int32_t dm;
    if constexpr (D == 32)
        asm volatile(QF_LOADS16 QF_TR32 QF_CHECK QF_PACK16
                     : QF_IDX16, QF_T32, [ok] "=&s"(ok), [dm] "=&v"(dm)
                     : QF_B32, [lut] "i"(LUT), QF_S16);
    else if constexpr (D == 64)
        asm volatile(QF_LOADS16 QF_TR64 QF_CHECK QF_PACK16
                     : QF_IDX16, QF_T64, [ok] "=&s"(ok), [dm] "=&v"(dm)
                     : QF_B64, [lut] "i"(LUT), QF_S16);
    else
        asm volatile(QF_LOADS16 QF_TR128 QF_CHECK QF_PACK16
                     : QF_IDX16, QF_T128, [ok] "=&s"(ok), [dm] "=&v"(dm)
                     : QF_B128, [lut] "i"(LUT), QF_S16);
#pragma unroll
    for (int w = 0; w < 4; ++w) pk[w] = r[4 * w];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) vf[i] = i32x4{t[2 * i].x, t[2 * i].y, t[2 * i + 1].x, t[2 * i + 1].y};
    return ok;
}
#undef QF_S16
#undef QF_CHECK
#undef QF_L
#undef QF_P
#undef QF_LOADS4
#undef QF_LOADS8
#undef QF_LOADS12
#undef QF_LOADS16
#undef QF_PACK4
#undef QF_PACK8
#undef QF_PACK12
#undef QF_PACK16
#undef QF_IDX4
#undef QF_IDX8
#undef QF_IDX12
#undef QF_IDX16
#undef QF_TR32
#undef QF_TR64
#undef QF_TR128
#undef QF_T32
#undef QF_T64
#undef QF_T128
#undef QF_B32
#undef QF_B64
#undef QF_B128
#undef QF_TV_ASM

// Per-wave state of the fast kernel (S layout for m, l, bnd: lane = query;
// O layout for acc).
template <int D>
struct FastState {
    static constexpr int DB = D / 32;
    i32x16 acc[DB];
    int32_t m, l;
    float bnd;  // per-row upper bound on max_d |acc| (dynamic identity proof)
    int wide;   // sticky: an alpha*acc_M left int32 -> every row is rescaled exactly
};

// Bias row of one query (kernel.py:232-236, :253) for the masked fast kernel.
// With unit key stride the 16 values of a lane (keys 8k + 4g + [0, 4) of the
// step) are four 16-byte buffer loads at lane-constant offsets; keys or rows
// past the head's bias extent read as 0 (their scores are replaced anyway).
struct BiasRow {
    __amdgpu_buffer_rsrc_t rsrc;
    int32_t voff;        // bytes: (row * sb2 + 4g) * 4
    const int32_t* row;  // strided fallback (nullptr for rows >= N)
};

template <bool TAIL>
__device__ __forceinline__ void load_bias(int32_t* bias_v, const Args& a, const BiasRow& br, int kstart, int lane) {
    if (a.bias_vec) {
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            const i32x4 b = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(br.rsrc, br.voff + 32 * k4, 4 * kstart, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) bias_v[4 * k4 + e] = b[e];
        }
    } else {
        // (rare layouts) the key of register v is k0 + 8*(v/4) + v%4: offsets from one
        // opaque base, so that the compiler keeps no per-register constants live
        // across the kernel for this path
        const int k0 = opaque(kstart + 4 * (lane >> 5));
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = k0 + 8 * (v >> 2) + (v & 3);
            bias_v[v] = ((!TAIL || key < a.N) && br.row) ? br.row[(int64_t)key * a.sb[3]] : 0;
        }
    }
}

// max / min over the first TV score registers (three-input chains)
template <int TV>
__device__ __forceinline__ int32_t max_first(const i32x16& s) {
    int32_t m = TV == 1 ? s[0] : max(s[0], s[1]);
#pragma unroll
    for (int v = 2; v + 1 < TV; v += 2) m = max3(m, s[v], s[v + 1]);
    if constexpr (TV > 2 && TV % 2) m = max(m, s[TV - 1]);
    return m;
}
template <int TV>
__device__ __forceinline__ int32_t min_first(const i32x16& s) {
    int32_t m = TV == 1 ? s[0] : min(s[0], s[1]);
#pragma unroll
    for (int v = 2; v + 1 < TV; v += 2) m = min3(m, s[v], s[v + 1]);
    if constexpr (TV > 2 && TV % 2) m = min(m, s[TV - 1]);
    return m;
}
template <int TV>
__device__ __forceinline__ uint32_t umin_first(const i32x16& s) {
    uint32_t m = TV == 1 ? (uint32_t)s[0] : min((uint32_t)s[0], (uint32_t)s[1]);
#pragma unroll
    for (int v = 2; v + 1 < TV; v += 2) m = min(min(m, (uint32_t)s[v]), (uint32_t)s[v + 1]);
    if constexpr (TV > 2 && TV % 2) m = min(m, (uint32_t)s[TV - 1]);
    return m;
}

// S^T tile of one step with bias and padding applied (kernel.py:153-156, :250-253);
// returns this lane's maximum over its 16 columns (the row's other 16 are in
// lane ^ 32).
// Every score carries kScoreBias, from an extra MFMA of xb (all bytes -128)
// with itself (int32 arithmetic wraps, so differences are unchanged).
// smin: the minimum over the real columns when MASKED or need_min (else
// INT32_MAX); sminu (MASKED): their minimum as unsigned values, i.e. over the
// columns whose biased score is non-negative (else UINT32_MAX).
// TV < 16 (partial steps of at most 2*TV keys): registers TV..15 hold padded
// columns only and are set to the padding value.
template <int D, bool MASKED, bool TAIL, int TV = 16>
__device__ __forceinline__ int32_t scores(i32x16& s, int32_t& smin, uint32_t& sminu, const Args& a,
                                          const i32x4* qv, const int8_t* lk, const Frag<D>& fr,
                                          const int32_t* bias_v, int kstart, int lane, bool need_min, i32x4 xb) {
    constexpr int DB = D / 32;
    constexpr int32_t PAD = kNegInf + kScoreBias;
    // K fragments first: the bias MFMA runs while they are in flight
    i32x4 kf[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) kf[db] = *reinterpret_cast<const i32x4*>(lk + fr.k[db]);
    if constexpr (MASKED) {
        // the bias enters as the accumulator of the first MFMA (int32 sums wrap)
        i32x16 c;
#pragma unroll
        for (int v = 0; v < 16; ++v) c[v] = bias_v[v];
        s = mfma32(xb, xb, c);
    } else {
        s = mfma32(xb, xb, i32x16{});
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) s = mfma32(kf[db], qv[db], s);
    smin = INT32_MAX;
    sminu = UINT32_MAX;
    const int32_t tcut = a.N - kstart - 4 * (lane >> 5);
    if constexpr (MASKED) {
        if constexpr (!TAIL) {
            smin = min_first<TV>(s);
            sminu = umin_first<TV>(s);
        } else {
#pragma unroll
            for (int v = 0; v < TV; ++v)
                if (!padded(v, tcut)) {
                    smin = min(smin, s[v]);
                    sminu = min(sminu, (uint32_t)s[v]);
                }
        }
    } else if (need_min) {
        // over the raw scores: a padded column's raw score (its K row reads as
        // 0) is the bias alone, which can only lower the minimum, so a check
        // that passes with it passes for the real columns
        smin = min_first<TV>(s);
    }
    if constexpr (TAIL) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
            if (v >= TV || padded(v, tcut)) s[v] = PAD;
    }
    return max_first<TV>(s);
}

// One 32-key step (qflash/kernel.py:147-174) for the 32 query rows of a wave.
// Every branch below is wave-uniform and none of them holds an alternative
// computation of acc (the accumulators keep their registers across steps).
// Scores, m and m' carry the bias SB = kScoreBias: only their differences
// (wrapping, as the reference's int32 arithmetic) enter the arithmetic, and
// the running maximum is the reference's one plus SB as long as no biased
// value wraps (checked for masked steps; unmasked scores are bounded by
// 128 * ||q||_1).  LUT: LDS address of the p table.
// TABM (unmasked waves): 0 = the path of each step is chosen from lut_mode;
// 1 = the table path is proved for every step of the wave (lut_mode 1), so the
// step has no other path; 2 = (lut_mode 2) full steps issue the table loads
// first and check the table's range while they are in flight
// (lut_pack_vt_check), falling back to the arithmetic when it fails.  The
// step's K tile sits at lk, its V tile at LDS address vbase + VO (read_vt).
template <int D, int LUT, bool MASKED, bool TAIL, bool WIDE, bool DYN, bool FIRST, int TABM, int VO, int TV = 16>
__device__ __forceinline__ void fast_step(FastState<D>& st, const Args& a, const i32x4* qv, const int8_t* lk,
                                          uint32_t vbase, const Frag<D>& fr, const BiasRow& brow, int kstart,
                                          int lane, bool wave_fast, int32_t xlim, int lut_mode, i32x4 xb) {
    constexpr int DB = D / 32;
    constexpr int32_t SB = kScoreBias;
    const int g = lane >> 5;
    const int32_t rs = a.rs, eM = a.eM, rM = a.rM;
    // lut_n - 1 as an opaque scalar: the compiler would otherwise form the
    // threshold m' - (lut_n - 1) with two vector operations
    int32_t lut_n1 = a.lut_n - 1;
    asm volatile("" : "+s"(lut_n1));

    // speculative table path of this step (TABM 2)
    constexpr bool SPEC = TABM == 2 && !MASKED && !TAIL;
    int32_t bias_v[16];
    if constexpr (MASKED) load_bias<TAIL>(bias_v, a, brow, kstart, lane);
    i32x16 s;
    int32_t smin;
    uint32_t sminu;
    static_assert(TV == 16 || (TAIL && (TV == 4 || TV == 8 || TV == 12)), "TV < 16: partial steps of <= 2*TV keys");
    const int32_t mxl =
        scores<D, MASKED, TAIL, TV>(s, smin, sminu, a, qv, lk, fr, bias_v, kstart, lane, SPEC ? false : lut_mode == 2,
                                    xb);
    const int32_t m = st.m;
    // opaque: the compiler would otherwise test "row changed" on an
    // intermediate maximum and split the three-input max in two
    int32_t mn = opaque(half_max3(mxl, m));  // kernel.py:158
    constexpr bool first = FIRST;  // kstart == 0

    // Table path.  Unmasked: every real column of the wave has u = m' - s <=
    // lut_lim (lut_mode 1: proved for the whole row block from ||q||_1; the
    // difference is exact as an unsigned 32-bit value since m' >= s).
    // Masked: the columns split by the sign of the biased score s'.  Those with
    // s' >= 0 need u <= lut_lim (checked on their minimum, sminu, or on m'
    // itself when there is none); those with s' < 0 have u = m' - s' >= m' + 1
    // >= far_lo + 1 and need u <= far_hi, where p is the constant far_p
    // (far_bounds); far_lo >= lut_n - 1 keeps thr below non-negative.  The far
    // check runs on min(smin, m): a wrapped biased value (below INT32_MIN + SB,
    // from a reference score >= 2^31 - SB) in this step or in m, the only case
    // in which m' is not the reference's maximum plus SB, fails it (far_hi <=
    // 2^30) and the 24-bit range check below.  A partial step's half with no
    // real column has smin = INT32_MAX, sminu = UINT32_MAX.  The conditions are
    // combined without short-circuit branches.
    bool lut_ok;
    int32_t slo = smin;
    uint32_t pk[4];
    i32x4 vf[DB];
    if constexpr (MASKED) {
        slo = min(smin, m);
        const bool far_ok = (mn >= a.far_lo) & ((uint32_t)(mn - slo) <= (uint32_t)a.far_hi);
        const bool near_ok = (uint32_t)mn - min(sminu, (uint32_t)mn) <= (uint32_t)a.lut_lim;
        lut_ok = lut_mode == 2 && __all(far_ok & near_ok);
    } else if constexpr (SPEC) {
        // the table path's indices (as below); pk and vf are its result when every lane passes
        const int32_t thr = wsub(mn, lut_n1);
        uint32_t idx[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) idx[v] = __builtin_elementwise_sub_sat((uint32_t)s[v], (uint32_t)thr);
        const uint64_t okm = lut_pack_vt_check<D, LUT, VO>(pk, vf, idx, vbase, fr, s, mn, a.lut_lim);
        lut_ok = okm == __builtin_amdgcn_read_exec();
    } else {
        lut_ok = TABM == 1 || lut_mode == 1 || (lut_mode == 2 && __all((uint32_t)(mn - smin) <= (uint32_t)a.lut_lim));
    }
    // 24-bit arithmetic path: masked steps check |x| <= xlim and the 24-bit
    // operand range (then mn - slo < 2^24 is exact in int32), evaluated only
    // when the table path is not taken
    auto vec_ok = [&]() {
        if constexpr (MASKED)
            return wave_fast && __all((slo > -(1 << 23)) & (mn < (1 << 23)) & (wsub(mn, slo) <= xlim));
        else
            return wave_fast;
    };
    if (__builtin_expect(lut_ok, SPEC)) {
        if constexpr (!SPEC) {
        // table index max(s - thr, 0) = lut_n - 1 - min(u, lut_n - 1) with one
        // unsigned saturating subtraction: thr in [0, 2^31) and, for the
        // columns it serves, s in [0, 2^31) (unmasked: s >= SB - 128 * ||q||_1
        // > lut_n - 1, lut_mode != 0 only then)
        const int32_t thr = wsub(mn, lut_n1);
        uint32_t idx[16];
        if constexpr (MASKED) {
            // s' < 0 reads as >= 2^31 > thr + lut_n - 1: clamped to entry lut_n = far_p
#pragma unroll
            for (int v = 0; v < TV; ++v)
                idx[v] = min(__builtin_elementwise_sub_sat((uint32_t)s[v], (uint32_t)thr), (uint32_t)a.lut_n);
        } else {
#pragma unroll
            for (int v = 0; v < TV; ++v) idx[v] = __builtin_elementwise_sub_sat((uint32_t)s[v], (uint32_t)thr);
        }
        if constexpr (TAIL) {  // padded columns read entry 0 (p = 0); l gets their p below
            const int32_t tcut = a.N - kstart - 4 * g;
#pragma unroll
            for (int v = 0; v < TV; ++v)
                if (padded(v, tcut)) idx[v] = 0;
        }
        lut_pack_vt<D, LUT, TV, VO>(pk, vf, idx, vbase, fr);
        }
    } else if (vec_ok()) {
        // kernel.py:159-161 in six ops per score (see the fast-path comment)
        const int32_t c1 = opaque(wadd(wmul(wsub(0, mn), eM), 1 << 16));
        const int32_t c3 = opaque(wsub(rs, mn));
        const int32_t c15 = opaque(1 << 15);
#pragma unroll
        for (int v = 0; v < TV; ++v) {  // registers TV..15 are padded columns (set below)
            const int32_t t = mad24(s[v], eM, c1);
            const int32_t q1 = t >> 16;
            const int32_t av = s[v] + __mul24(q1, rs) + c3;
            const int32_t E = av >> min((uint32_t)q1, 31u);
            s[v] = mad24(E, rM, c15);  // p = bits 16..23
        }
        if constexpr (TAIL) {  // padded key columns: p(NEG_INF - m') exactly, once per row
            const int32_t ppad = (int32_t)((uint32_t)requant(exp2_i32(wsub(kNegInf + SB, mn), a), a) << 16);
            const int32_t tcut = a.N - kstart - 4 * g;
#pragma unroll
            for (int v = 0; v < 16; ++v)
                if (padded(v, tcut)) s[v] = ppad;
        }
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
            const uint32_t lo = __builtin_amdgcn_perm((uint32_t)s[4 * w4 + 1], (uint32_t)s[4 * w4], 0x0c0c0602u);
            const uint32_t hi = __builtin_amdgcn_perm((uint32_t)s[4 * w4 + 3], (uint32_t)s[4 * w4 + 2], 0x0c0c0602u);
            pk[w4] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    } else {  // general exact arithmetic for this step's scores (p in bits 0-7)
        if constexpr (MASKED) {
            // a wrapped biased value: the maximum over the reference's values
            if (__builtin_expect(__any(slo < INT32_MIN + SB), 0)) {
                int32_t r = wsub(s[0], SB);
#pragma unroll
                for (int v = 1; v < 16; ++v) r = max(r, wsub(s[v], SB));
                mn = wadd(max(wsub(m, SB), half_max(r)), SB);
            }
        }
        // One score at a time through a rotating queue: this rare path then holds
        // the temporaries of one evaluation only, not of sixteen interleaved ones.
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
            const int32_t pv = requant(exp2_i32(wsub(s[0], mn), a), a);
#pragma unroll
            for (int v = 0; v < 15; ++v) s[v] = s[v + 1];
            s[15] = pv;
        }
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
            const uint32_t lo = __builtin_amdgcn_perm((uint32_t)s[4 * w4 + 1], (uint32_t)s[4 * w4], 0x0c0c0400u);
            const uint32_t hi = __builtin_amdgcn_perm((uint32_t)s[4 * w4 + 3], (uint32_t)s[4 * w4 + 2], 0x0c0c0400u);
            pk[w4] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    }
    // kernel.py:162
    // the first dot product takes the constant from a scalar register, so that
    // its accumulator can be the inline 0 (no register cleared beforehand)
    int32_t ones, lij;
    asm("s_mov_b32 %0, 0x1010101" : "=s"(ones));
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(lij) : "v"(pk[0]), "s"(ones));
    lij = __builtin_amdgcn_sdot4((int)pk[1], 0x01010101, lij, false);
    lij = __builtin_amdgcn_sdot4((int)pk[2], 0x01010101, lij, false);
    lij = __builtin_amdgcn_sdot4((int)pk[3], 0x01010101, lij, false);
    lij = half_sum(lij);
    if constexpr (TAIL) {
        // Table path of the last, partial step: the padded columns (score
        // NEG_INF) read p = 0; their P.V term is 0 anyway (V rows past N read
        // as 0), so only l needs their exact p.
        if (lut_ok) lij = wadd(lij, (32 - (a.N - kstart)) * requant(exp2_i32(wsub(kNegInf + SB, mn), a), a));
    }

    const int32_t dm = wsub(m, mn);
    // kernel.py:163-165
    int32_t alpha;
    bool wide_step;
    if constexpr (!WIDE) {
        // Unmasked fast waves: past the first step m and m' are maxima of real
        // scores, so |m - m'| <= 2*smax <= X and alpha = E(m - m') is in [-1, rs].
        // The first step's alpha may be anything, but acc is still 0 then.
        alpha = first ? exp2_i32(dm, a) : exp2_fast(dm, eM, rs);
        wide_step = first;
    } else {
        if (!first && wave_fast && __all(-dm <= xlim))
            alpha = exp2_fast(dm, eM, rs);  // in [-1, rs]
        else
            alpha = exp2_i32(dm, a);        // in [-1, rs] unless dm*eM overflows
        // rs*l_M and rs*acc_M < 2^31 (host): alpha in [-rs, rs] keeps both multipliers in int32
        wide_step = !__all(alpha >= -rs && alpha <= rs);
        if (!first && wide_step) st.wide = 1;
    }
    if (!wide_step) {
        const int64_t pl = (int64_t)st.l * (int64_t)wmul(alpha, a.lM) + (1ll << (a.l_shift - 1));
        st.l = wadd((int32_t)__builtin_amdgcn_alignbit((uint32_t)(pl >> 32), (uint32_t)pl, (uint32_t)a.l_shift),
                    lij);
    } else {
        st.l = wadd(release(st.l, alpha, a.lM, a.l_shift, 1, rs), lij);
    }
    const int64_t A64 = (int64_t)alpha * a.aM;
    const int32_t A = (int32_t)A64;
    // high word of A64 once A's sign is extended (zero unless A64 leaves int32)
    const int32_t Ah = (int32_t)(A64 >> 32) + (int32_t)((uint32_t)A >> 31);
    const int32_t as = a.acc_shift;
    if (!first) {  // acc == 0 before the first step: its rescale is 0 for any alpha
        bool need = mn != m;
        if constexpr (DYN) need = need || st.bnd * (float)a.e_acc >= __builtin_ldexpf(0.99f, as - 1);
        uint32_t chg = __builtin_amdgcn_readfirstlane((uint32_t)__ballot(need));
        int wide = 0;
        if constexpr (WIDE) wide = __builtin_amdgcn_readfirstlane(st.wide);
        if (wide) chg = 0xffffffffu;  // the identity proof no longer holds: rescale every row
        if constexpr (DYN)
            if (need || wide)
                st.bnd = __builtin_fmaf(st.bnd * (fabsf((float)alpha) * (float)a.aM * __builtin_ldexpf(1.f, -as)),
                                        1.0000010f, 1.f);
        if (chg) {
            // register pair v = rows rlo (lanes 0-31) and rlo+4 (lanes 32-63) of the O layout;
            // the multiplier of row r sits in lane r of the S layout.  Two lane permutes
            // (one LDS round trip for all pairs) lay the multipliers out as
            //   m1: lane 16j + n holds row n + 4*(j >> 1),   m2: the same rows + 16,
            // and a DPP row broadcast (row_newbcast:n, each 16-lane row takes its lane
            // n) of m1 (rlo < 16) or m2 gives pair v's multipliers: row rlo in lanes
            // 0-31, row rlo + 4 in lanes 32-63.
            // acc*A64 + 2^(as-1) mod 2^64 = acc*sext(A) + 2^(as-1) + (acc*Ah << 32)
            const int64_t ahalf = 1ll << (as - 1);
            const int src = 4 * ((lane & 15) + 4 * g);
            const int32_t m1 = __builtin_amdgcn_ds_bpermute(src, A);
            const int32_t m2 = __builtin_amdgcn_ds_bpermute(src + 64, A);
            int32_t h1 = 0, h2 = 0;
            if constexpr (WIDE)
                if (wide) {
                    h1 = __builtin_amdgcn_ds_bpermute(src, Ah);
                    h2 = __builtin_amdgcn_ds_bpermute(src + 64, Ah);
                }
            // bit rlo: row rlo or rlo + 4 changed (one scalar bit test per pair; most
            // are clear, so the pair's code is laid out off the fall-through path)
            const uint32_t pairs = (chg | (chg >> 4)) & 0x0F0F0F0Fu;
            auto pair = [&]<int V>() {
                constexpr int rlo = 8 * (V >> 2) + (V & 3);
                if (__builtin_expect((pairs >> rlo) & 1u, 0)) {
                    // every lane reads a valid source lane: no old value needed
                    const int32_t av = __builtin_amdgcn_mov_dpp(rlo < 16 ? m1 : m2, 0x150 + (rlo & 15), 0xf, 0xf,
                                                                false);
                    int32_t ah = 0;
                    if constexpr (WIDE)
                        ah = wide ? __builtin_amdgcn_mov_dpp(rlo < 16 ? h1 : h2, 0x150 + (rlo & 15), 0xf, 0xf, false)
                                  : 0;
#pragma unroll
                    for (int t = 0; t < DB; ++t) {
                        const int64_t p = (int64_t)st.acc[t][V] * (int64_t)av + ahalf;
                        uint32_t hi = (uint32_t)(p >> 32);
                        if constexpr (WIDE)
                            if (wide) hi += (uint32_t)wmul(st.acc[t][V], ah);
                        st.acc[t][V] = (int32_t)__builtin_amdgcn_alignbit(hi, (uint32_t)p, (uint32_t)as);
                    }
                }
            };
            [&]<int... V>(std::integer_sequence<int, V...>) { (pair.template operator()<V>(), ...); }(
                std::make_integer_sequence<int, 16>{});
        }
    }
    if constexpr (DYN) {  // |P.V| <= 128 * sum|p|, and sum|p| <= sum of the bytes read as unsigned
        uint32_t sa = __builtin_amdgcn_udot4(pk[0], 0x01010101u, 0u, false);
        sa = __builtin_amdgcn_udot4(pk[1], 0x01010101u, sa, false);
        sa = __builtin_amdgcn_udot4(pk[2], 0x01010101u, sa, false);
        sa = __builtin_amdgcn_udot4(pk[3], 0x01010101u, sa, false);
        sa = (uint32_t)half_sum((int32_t)sa);
        st.bnd = (st.bnd + 128.f * (float)sa) * 1.0000010f;
    }
    // O += P . V (kernel.py:171)
    const i32x4 pa = i32x4{(int32_t)pk[0], (int32_t)pk[1], (int32_t)pk[2], (int32_t)pk[3]};
    if (!SPEC && !lut_ok) read_vt<D, VO>(vf, vbase, fr);  // (SPEC: read with the table)
#pragma unroll
    for (int t = 0; t < DB; ++t) st.acc[t] = mfma32(pa, vf[t], st.acc[t]);
    st.m = mn;  // kernel.py:172
}

// Output codes of the wave's 32 rows (kernel.py:176-180):
// out = int8(cvt_x86(RN_f32(fp32(acc) / fp32(l)))).
// The quotient is taken as RN_f32(a * y) in double precision, y = RN_f64(1/b)
// once per row.  a * y is within 2^-52 (relative) of a/b, while a/b, for
// 24-bit a and b, is never within 2^-49 of a midpoint between two floats (it
// cannot be one: that would need a 25-bit odd significand), so rounding the
// double to float gives exactly the IEEE single division.  For |b| >= 2 the
// quotient is below 2^30 in magnitude, so v_cvt_i32_f32 truncates exactly as
// x86 does; a wave with any row of l in {-1, 0, 1} (quotient +-inf, NaN or
// 2^31: INT_MIN on x86) takes the IEEE division and the x86 conversion.
// Bytes go out with buffer stores: rows >= N fall beyond the buffer's range
// ((N-1)*so2 + D bytes from the head's base, so2 >= D checked by the host)
// and are dropped by the hardware.
template <int D>
__device__ __forceinline__ void fast_store(const FastState<D>& st, const Args& a, int z, int h, int lane, int q0,
                                           double* yslot) {
    constexpr int DB = D / 32;
    const int lq = lane & 31, g = lane >> 5;
    const float b_row = (float)st.l;  // S layout: lane = row
    const bool exact = __any(st.l >= -1 && st.l <= 1);
    const int32_t so2 = (int32_t)a.so[2];
    const __amdgpu_buffer_rsrc_t rsrc = out_rsrc(a, z, h, D);
    const float os = a.out_dt == QFLASH_HIP_I8 ? 0.f : scale_value(a);
    const int32_t voff = (q0 + 4 * g) * so2 + lq;
    if (!exact) {
        // y of the 32 rows to LDS (this wave's 256 bytes, 16-byte aligned), read
        // back two rows at a time in the O layout (registers v and v+1, v even,
        // hold rows r and r+1 of this lane half)
        if (g == 0) yslot[lq] = 1.0 / (double)b_row;
        with_out_type(a.out_dt, [&]<int OUT>() {
#pragma unroll
            for (int v = 0; v < 16; v += 2) {
                typedef double f64x2 __attribute__((ext_vector_type(2)));
                const f64x2 y2 = *reinterpret_cast<const f64x2*>(yslot + crow(v, lane));
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int32_t soff = (8 * ((v + j) >> 2) + ((v + j) & 3)) * so2;
#pragma unroll
                    for (int t = 0; t < DB; ++t) {
                        const float qf = (float)((double)(float)st.acc[t][v + j] * y2[j]);
                        put_out<OUT>(rsrc, (int32_t)qf, voff + t * 32, soff, os);
                    }
                }
            }
        });
    } else {
        with_out_type(a.out_dt, [&]<int OUT>() {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int32_t soff = (8 * (v >> 2) + (v & 3)) * so2;
                const float bf = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * crow(v, lane), __float_as_int(b_row)));
#pragma unroll
                for (int t = 0; t < DB; ++t) {
                    const int32_t code = cvt_x86(__fdiv_rn((float)st.acc[t][v], bf));
                    put_out<OUT>(rsrc, code, voff + t * 32, soff, os);
                }
            }
        });
    }
}

// The 32 query rows of one wave: K / V stages double-buffered in LDS (the
// copy of stage s+1 runs while stage s is consumed), full 32-key steps in the
// loop, a final partial step (N % 32 != 0) after it from the last stage's
// buffer, which no later copy overwrites, then the rows' int8 codes.  Every
// wave of the workgroup issues its share of the copies and passes the same
// barriers, active or not.
template <int D, int W, bool MASKED, bool WIDE, bool DYN, int TABM>
__device__ __forceinline__ void fast_rows(const Args& a, const i32x4* qv, int8_t* smem, const int8_t* kb,
                                          const int8_t* vb, int z, int h, const BiasRow& brow, int wave, int lane,
                                          int q0, bool active, bool wave_fast, int32_t xlim, int lut_mode) {
    using S = Stage<D, W>;
    constexpr int DB = D / 32;
    constexpr int LUT = 2 * S::BYTES;  // LDS address of the p table (smem starts at 0)
    FastState<D> st;
#pragma unroll
    for (int t = 0; t < DB; ++t) st.acc[t] = i32x16{};
    st.m = kNegInf + kScoreBias;  // kernel.py:138
    st.l = 1;                     // kernel.py:139
    st.bnd = 0.f;
    st.wide = 0;
    // all bytes -128; opaque to the compiler each step, so that the bias MFMA
    // is issued per step rather than hoisted into 16 live registers
    i32x4 xb = i32x4{(int32_t)0x80808080, (int32_t)0x80808080, (int32_t)0x80808080, (int32_t)0x80808080};

    // K / V of this head as buffers ending after row N-1: rows >= N read as 0
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)kb, 0, (a.N - 1) * (int32_t)a.sk[2] + D, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vb, 0, (a.N - 1) * (int32_t)a.sv[2] + D, 0x00020000);
    const StageDma<D, W> dma(a, wave, lane);
    const Frag<D> fr(lane);
    const uint32_t lds0 = lds_addr(smem);  // a constant: the kernel's LDS array
    stage_sync();  // the first stage, issued by fast_block

    static_assert(S::BYTES >= W * 256, "epilogue slots of 256 bytes per wave in one stage buffer");
    const int nfull = a.N >> 5;
    const int nstage = (a.N + S::KEYS - 1) / S::KEYS;
    // step 0 (m = NEG_INF, acc = 0) apart from the loop: the loop body then
    // carries no first-step cases
    if (active && nfull > 0)
        fast_step<D, LUT, MASKED, false, WIDE, DYN, true, TABM, S::KBYTES>(st, a, qv, smem, lds0, fr, brow, 0, lane,
                                                                        wave_fast, xlim, lut_mode, xb);
    // One stage in LDS buffer B (compile-time, like the steps within it, so that
    // every K and V^T fragment read takes its tile offset as an immediate).
    auto stage = [&]<int B>(int stg) {
        if (stg + 1 < nstage) dma.issue(rk, rv, smem + (1 - B) * S::BYTES, (stg + 1) * S::KEYS, a, wave);
        if (active) {
            auto one = [&]<int HS>() {
                const int step = stg * S::STEPS + HS;
                if ((B == 0 && HS == 0 && stg == 0) || step >= nfull) return;  // step 0 ran above
                if constexpr (!MASKED) asm volatile("" : "+v"(xb));  // masked: C = bias, not hoistable
                constexpr int KO = B * S::BYTES + HS * 32 * D;
                fast_step<D, LUT, MASKED, false, WIDE, DYN, false, TABM, KO + S::KBYTES>(
                    st, a, qv, smem + KO, lds0, fr, brow, step * 32, lane, wave_fast, xlim, lut_mode, xb);
            };
            [&]<int... HS>(std::integer_sequence<int, HS...>) { (one.template operator()<HS>(), ...); }(
                std::make_integer_sequence<int, S::STEPS>{});
        }
        stage_sync();
    };
    if constexpr (TABM != 0) {
        for (int stg = 0; stg < nstage; stg += 2) {
            stage.template operator()<0>(stg);
            if (stg + 1 < nstage) stage.template operator()<1>(stg + 1);
        }
    } else {
        // the loops with more than the table path: one stage body with the
        // buffer's address in a register (their registers do not fit otherwise)
        for (int stg = 0; stg < nstage; ++stg) {
            const int8_t* buf = smem + (stg & 1) * S::BYTES;
            if (stg + 1 < nstage) dma.issue(rk, rv, smem + ((stg + 1) & 1) * S::BYTES, (stg + 1) * S::KEYS, a, wave);
            if (active) {
#pragma unroll
                for (int half = 0; half < S::STEPS; ++half) {
                    const int step = stg * S::STEPS + half;
                    if (half == 0 && stg == 0) continue;  // step 0 ran above
                    if (step >= nfull) break;
                    if constexpr (!MASKED) asm volatile("" : "+v"(xb));  // masked: C = bias, not hoistable
                    fast_step<D, LUT, MASKED, false, WIDE, DYN, false, TABM, 0>(
                        st, a, qv, buf + half * 32 * D, lds_addr(buf + S::KBYTES + half * 32 * D), fr, brow,
                        step * 32, lane, wave_fast, xlim, lut_mode, xb);
                }
            }
            stage_sync();
        }
    }
    if (active && (a.N & 31)) {
        const int8_t* buf = smem + ((nstage - 1) & 1) * S::BYTES;
        const int th = nfull % S::STEPS;
        const int8_t* lk = buf + th * 32 * D;
        const uint32_t lv = lds_addr(buf + S::KBYTES + th * 32 * D);
        if (nfull == 0)
            fast_step<D, LUT, MASKED, true, WIDE, DYN, true, TABM, 0>(st, a, qv, lk, lv, fr, brow, 0, lane, wave_fast,
                                                                    xlim, lut_mode, xb);
        else if ((a.N & 31) <= 8)  // keys of the first TV score registers only
            fast_step<D, LUT, MASKED, true, WIDE, DYN, false, TABM, 0, 4>(st, a, qv, lk, lv, fr, brow, nfull * 32,
                                                                        lane, wave_fast, xlim, lut_mode, xb);
        else if ((a.N & 31) <= 16)
            fast_step<D, LUT, MASKED, true, WIDE, DYN, false, TABM, 0, 8>(st, a, qv, lk, lv, fr, brow, nfull * 32,
                                                                        lane, wave_fast, xlim, lut_mode, xb);
        else if ((a.N & 31) <= 24)
            fast_step<D, LUT, MASKED, true, WIDE, DYN, false, TABM, 0, 12>(st, a, qv, lk, lv, fr, brow, nfull * 32,
                                                                         lane, wave_fast, xlim, lut_mode, xb);
        else
            fast_step<D, LUT, MASKED, true, WIDE, DYN, false, TABM, 0>(st, a, qv, lk, lv, fr, brow, nfull * 32, lane,
                                                                     wave_fast, xlim, lut_mode, xb);
    }
    if (!active) return;
    // this wave's 256 bytes of the stage buffer that no step reads any more:
    // the last stage used buffer (nstage - 1) & 1 and every wave has passed the
    // barrier after the stage before it
    fast_store<D>(st, a, z, h, lane, q0,
                  reinterpret_cast<double*>(smem + (nstage & 1) * S::BYTES + wave * 256));
}

// Occupancy target (waves per SIMD) by head dim: the register budget of the
// O accumulators (D/32 x 16 VGPRs) and the score / exp temporaries.  D = 32
// runs at 5 (the masked kernel needs 83 VGPRs; at 6, 80 VGPRs, it spills to
// scratch, and measured on Swin windows it is 1.5 % slower).
#ifndef QF_FAST_WAVES_D32
#define QF_FAST_WAVES_D32 5
#endif
template <int D>
constexpr int fast_waves_per_simd() { return D <= 32 ? QF_FAST_WAVES_D32 : (D == 64 ? QF_FAST_WAVES_D64 : 2); }

// The p(u) table at lut, entry lut_n - 1 - u (lut_pack_vt), and for masked
// launches the far columns' constant at entry lut_n (lut_n + 1 <= kLutMax,
// host); visible after fast_rows' first barrier.  Launches of fwd_fast_table
// (lut_in_args: host constants, short rows) pass the bytes with the kernel
// arguments (copy_lut, whole 256-byte chunks, at most 4 kLutArgWords <=
// kLutMax bytes); otherwise the workgroup forms them (fill_lut), exact with
// the 24-bit E since lut_n - 1 <= x_safe (host).  Entries past the table are
// never read.
template <int W, bool MASKED>
__device__ __forceinline__ int lut_dwords(const Args& a) {
    return a.lut_n > 0 ? (a.lut_n + (MASKED ? 4 : 3)) >> 2 : 0;
}

// pre: the host's table, copied to LDS by buffer_load ... lds (wave c
// copies dwords 64 c .. 64 c + 63; those past the table read 0), visible, like
// the first K / V stage, after fast_rows' first wait and barrier.  Issued
// before the stage copy, with no LDS write of its own: an LDS store after an
// LDS-bound load waits for every outstanding load.
template <int W, bool MASKED>
__device__ __forceinline__ void copy_lut(const Args& a, int8_t* lut, const uint32_t* pre, int wave, int lane) {
    const int nd = lut_dwords<W, MASKED>(a);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)pre, 0, nd * 4, 0x00020000);
    for (int c = wave; 64 * c < nd; c += W)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lut + 256 * c), 4,
                                                 256 * c + 4 * lane, 0, 0, 0);
}

// nullptr pre: the workgroup forms the entries (a dword a lane measured slower
// than a byte a lane, cfg1-3 +0.5-1.5 %)
template <int W, bool MASKED>
__device__ __forceinline__ void fill_lut(const Args& a, int8_t* lut) {
    for (int u = threadIdx.x; u < a.lut_n; u += 64 * W)
        lut[a.lut_n - 1 - u] = (int8_t)(mad24(exp2_fast(-u, a.eM, a.rs), a.rM, 1 << 15) >> 16);
    if constexpr (MASKED)
        if (threadIdx.x == 0 && a.lut_n > 0) lut[a.lut_n] = (int8_t)a.far_p;
}

// One workgroup of the single-tile kernel: row block mb (32 * W rows) of head
// zh, in the LDS array smem.  The copy of the first K / V stage, the Q loads
// and the table fill (visible after fast_rows' first barrier) go out before
// any of them is waited for, so that their latencies overlap.
template <int D, int W, bool MASKED, bool DYN>
__device__ __forceinline__ void fast_block(const Args& a, int8_t* smem, int zh, int mb,
                                           const uint32_t* lut_pre = nullptr) {
    constexpr int DB = D / 32;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lq = lane & 31, g = lane >> 5;
    const int z = zh / a.H, h = zh % a.H;
    const int q0 = (mb * W + wave) * 32;
    const bool active = q0 < a.N;
    const int qrow = q0 + lq;

    if (lut_pre) copy_lut<W, MASKED>(a, smem + 2 * Stage<D, W>::BYTES, lut_pre, wave, lane);
    const int8_t* qb = a.q + z * a.sq[0] + h * a.sq[1];
    const int8_t* kb = a.k + z * a.sk[0] + h * a.sk[1];
    const int8_t* vb = a.v + z * a.sv[0] + h * a.sv[1];
    first_stage<D, W>(a, kb, vb, smem, wave, lane);
    BiasRow brow;
    if constexpr (MASKED) {
        const int32_t* bh = a.bias + (a.bias_zmod ? z % a.bias_zmod : z) * a.sb[0] + h * a.sb[1];
        brow.row = qrow < a.N ? bh + (int64_t)qrow * a.sb[2] : nullptr;
        // extent of this head's bias: the last element of row N-1 (strides >= 0 when bias_vec)
        const int32_t nbytes = a.bias_vec ? (int32_t)(((a.N - 1) * a.sb[2] + a.N) * 4) : 0;
        brow.rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)bh, 0, nbytes, 0x00020000);
        brow.voff = (int32_t)((qrow * a.sb[2] + 4 * g) * 4);
    } else {
        brow.row = nullptr;
        brow.voff = 0;
        brow.rsrc = __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0x00020000);
    }

    i32x4 qv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
        qv[db] = qrow < a.N ? *reinterpret_cast<const i32x4*>(qb + (int64_t)qrow * a.sq[2] + db * 32 + g * 16)
                            : i32x4{0, 0, 0, 0};
    if (!lut_pre) fill_lut<W, MASKED>(a, smem + 2 * Stage<D, W>::BYTES);

    // Unmasked: every real key column of this row has |s| <= 128*||q_row||_1, so
    // |x| = |s - m'| <= X_row for the scores and, past the first step, for
    // m - m'; the 24-bit path is exact when X_row*|eM| and the |a| bound stay in
    // range (checked once for the whole wave).  Masked: |x| <= x_safe is checked
    // per step.
    bool wave_fast = !a.force_robust;
    int32_t xlim = a.x_safe;
    // the table sits at LDS address 2 * S::BYTES, the byte loads' immediate offset
    const bool lut_at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem == 0;
    int lut_mode = a.lut_n && lut_at ? 2 : 0;  // 1: u <= lut_lim for every real column, 2: checked per step
    if constexpr (!MASKED) {
        // sum |q|: bytes offset by 128 (xor 0x80) against 0x80 under v_sad_u8
        uint32_t l1u = 0;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int w4 = 0; w4 < 4; ++w4)
                l1u = __builtin_amdgcn_sad_u8((uint32_t)qv[db][w4] ^ 0x80808080u, 0x80808080u, l1u);
        const int32_t l1 = half_sum((int32_t)l1u);
        // real columns: x = s - m' >= -2*smax (padded columns are evaluated exactly apart)
        const int64_t X = 2 * 128ll * l1;
        const int64_t lim = (1ll << 31) - (1ll << 17);
        const bool ok = X * (int64_t)(-(int64_t)a.eM) <= lim &&
                        ((X * a.eps_abs + 65535) >> 16) + 2 * (int64_t)a.rs + 1 < (1 << 22);
        wave_fast = wave_fast && __all(ok);
        xlim = (int32_t)(X < (1 << 30) ? X : (1 << 30));
        // biased scores >= kScoreBias - 128 * ||q||_1 > lut_n - 1: scores and thresholds positive
        if (lut_mode) lut_mode = !__all(X / 2 + kLutMax <= kScoreBias) ? 0 : (__all(X <= a.lut_lim) ? 1 : 2);
    }

    // Unmasked waves whose guard holds run a loop that never meets an alpha
    // outside [-1, rs] after the first step (and, when the table serves every
    // step, a loop with the table path alone); the others (and masked waves)
    // run the loop that also handles it.  All pass the same barriers, and each
    // writes its own rows, so they never merge register state.
    if constexpr (!MASKED) {
        if (wave_fast && lut_mode == 1)
            fast_rows<D, W, false, false, DYN, 1>(a, qv, smem, kb, vb, z, h, brow, wave, lane, q0, active,
                                                  wave_fast, xlim, lut_mode);
        else if (wave_fast && lut_mode == 2)
            fast_rows<D, W, false, false, DYN, 2>(a, qv, smem, kb, vb, z, h, brow, wave, lane, q0, active,
                                                  wave_fast, xlim, lut_mode);
        else if (wave_fast)
            fast_rows<D, W, false, false, DYN, 0>(a, qv, smem, kb, vb, z, h, brow, wave, lane, q0, active,
                                                  wave_fast, xlim, lut_mode);
        else
            fast_rows<D, W, false, true, DYN, 0>(a, qv, smem, kb, vb, z, h, brow, wave, lane, q0, active,
                                                 wave_fast, xlim, lut_mode);
    } else {
        fast_rows<D, W, true, true, DYN, 0>(a, qv, smem, kb, vb, z, h, brow, wave, lane, q0, active, wave_fast,
                                            xlim, lut_mode);
    }
}


template <int D, int W, bool MASKED, bool DYN>
__global__ __launch_bounds__(64 * W, fast_waves_per_simd<D>()) void fwd_fast(Args a) {
    using S = Stage<D, W>;
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * S::BYTES + kLutMax];
    const int wg = xcd_order(blockIdx.x, a.n_wg);
    fast_block<D, W, MASKED, DYN>(a, smem, wg / a.mblocks, wg % a.mblocks);
}

// fwd_fast for short rows (lut_in_args) with the table formed by the host.  A
// kernel of its own: the table's kilobyte of arguments, on every launch of
// fwd_fast, measured slower where the table is computed anyway (cfg3 +3 %).
template <int D, int W, bool MASKED>
__global__ __launch_bounds__(64 * W, fast_waves_per_simd<D>()) void fwd_fast_table(Args a, LutArg) {
    using S = Stage<D, W>;
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * S::BYTES + kLutMax];
    // the table argument, read in place in the kernel-argument segment (where
    // the ABI puts it, right after `a`): indexing the by-value parameter would
    // copy it to scratch memory first
    static_assert(sizeof(Args) % alignof(LutArg) == 0, "LutArg follows Args in the kernel-argument segment");
    const uint32_t* pre =
        reinterpret_cast<const uint32_t*>((const char*)__builtin_amdgcn_kernarg_segment_ptr() + sizeof(Args));
    const int wg = xcd_order(blockIdx.x, a.n_wg);
    fast_block<D, W, MASKED, false>(a, smem, wg / a.mblocks, wg % a.mblocks, pre);
}

// The kernels on constants in device memory (qflash_hip_constants), for
// layouts the fast kernel accepts.  Two launches on the same grid, each
// returning at once unless the plan selects it: fwd_fast_planned runs the fast
// path when the plan proves the rescale by rs the identity (id_ok, the common
// case), fwd_planned_rest every other plan (the per-row bound variant, or the
// general path).  One kernel holding every path keeps the plan's values in
// scalar registers across all of them and spills them to vector lanes in the
// hot loop (cfg3 90.5 us against 82.3 us for the one-path kernel); an empty
// launch costs ~2.5 us.
template <int D, int W, bool MASKED>
__global__ __launch_bounds__(64 * W, fast_waves_per_simd<D>()) void fwd_fast_planned(Args a) {
    using S = Stage<D, W>;
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * S::BYTES + kLutMax];
    if (a.params[kPStatus] != 0 || !a.params[kPFast] || !a.params[kPIdOk]) return;
    load_params(a);
    const int wg = xcd_order(blockIdx.x, a.n_wg);
    fast_block<D, W, MASKED, false>(a, smem, wg / a.mblocks, wg % a.mblocks);
}

template <int D, int W, bool MASKED>
__global__ __launch_bounds__(64 * W, fast_waves_per_simd<D>()) void fwd_planned_rest(Args a) {
    using S = Stage<D, W>;
    static_assert(Tile<D>::BYTES <= 2 * S::BYTES + kLutMax, "the general path's tiles fit the fast path's LDS");
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * S::BYTES + kLutMax];
    if (a.params[kPStatus] != 0 || (a.params[kPFast] && a.params[kPIdOk])) return;
    load_params(a);
    if (!a.params[kPFast]) {
        general_block<D, W, MASKED, true>(a, xcd_order(blockIdx.x, a.n_wg), smem);
        return;
    }
    const int wg = xcd_order(blockIdx.x, a.n_wg);
    fast_block<D, W, MASKED, true>(a, smem, wg / a.mblocks, wg % a.mblocks);
}



// ----------------------------------------------------------------------------
// Host side
using qferr::fail;
using qferr::g_err;

// ---- occupancy ------------------------------------------------------------
// The fast kernel runs at its natural occupancy (as many workgroups per CU as
// its registers allow): measured on MI355X, 4 waves per SIMD beat 3 even where
// 3 would split the grid into whole rounds (cfg3: 142 us vs 198 us).  The
// tuning hook QFLASH_HIP_WG_PER_CU lowers it by padding the workgroup's LDS
// allocation (dynamic shared memory the kernel does not use).

static int device_attr(hipDeviceAttribute_t attr) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, attr, dev) != hipSuccess) return 0;
    return v;
}

// want: the tuning hook's workgroups per CU (0 = natural occupancy)
static inline int pick_wg_per_cu(int kmax, int want) { return want > 0 && want < kmax ? want : kmax; }

// Dynamic LDS bytes that limit `kern` to k workgroups per CU (cached per k).
template <typename Kern>
static size_t lds_pad_for(Kern kern, int block, int k, std::atomic<int>* cache) {
    int c = cache[k].load(std::memory_order_relaxed);
    if (c >= 0) return (size_t)c;
    const int lds_cu = device_attr(hipDeviceAttributeMaxSharedMemoryPerMultiprocessor);
    hipFuncAttributes fa;
    int pad = 0;
    if (lds_cu > 0 && hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kern)) == hipSuccess) {
        const int want = (lds_cu / k) & ~511;
        pad = want > (int)fa.sharedSizeBytes ? want - (int)fa.sharedSizeBytes : 0;
        if (pad > 48 * 1024) pad = 0;
        int n = 0;
        if (pad && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kern), block,
                                                                 (size_t)pad) != hipSuccess || n != k))
            pad = 0;
    }
    cache[k].store(pad, std::memory_order_relaxed);
    return (size_t)pad;
}

// The bytes fill_lut forms (lut_in_args(a)), from the reference's own
// integer primitives: entry lut_n - 1 - u = p(u), then (masked) far_p.  Kept
// per thread for the last constants, which repeat from call to call.
static void lut_table(const Args& a, bool masked, LutArg* tb) {
    struct Key {
        int32_t rs, eM, rM, exp_mode, lut_n, far_p, masked;
    };
    thread_local Key last{};
    thread_local LutArg table;
    thread_local bool have = false;
    const Key k{a.rs, a.eM, a.rM, a.exp_mode, a.lut_n, masked ? a.far_p : 0, masked ? 1 : 0};
    if (!have || memcmp(&k, &last, sizeof k) != 0) {
        uint8_t* b = reinterpret_cast<uint8_t*>(table.w);
        memset(b, 0, sizeof table.w);
        for (int j = 0; j < a.lut_n; ++j) b[j] = (uint8_t)(int8_t)requant(exp2_i32(-(a.lut_n - 1 - j), a), a);
        if (masked) b[a.lut_n] = (uint8_t)(int8_t)a.far_p;
        last = k;
        have = true;
    }
    *tb = table;
}

template <int D, int W, bool MASKED, bool DYN>
static hipError_t launch_fast(const Args& a, int wg_per_cu, dim3 grid, hipStream_t st) {
    static std::atomic<int> kmax_cache{0};
    static std::atomic<int> pad_cache[9] = {-1, -1, -1, -1, -1, -1, -1, -1, -1};
    if constexpr (!DYN) {
        if (lut_in_args(a) && wg_per_cu <= 0) {  // (the occupancy hook pads fwd_fast's LDS)
            LutArg tb;
            lut_table(a, MASKED, &tb);
            hipLaunchKernelGGL((fwd_fast_table<D, W, MASKED>), grid, dim3(64 * W), 0, st, a, tb);
            return hipGetLastError();
        }
    }
    auto kern = fwd_fast<D, W, MASKED, DYN>;
    int kmax = kmax_cache.load(std::memory_order_relaxed);
    if (kmax <= 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&kmax, reinterpret_cast<const void*>(kern), 64 * W, 0) !=
            hipSuccess)
            kmax = 1;
        kmax = kmax < 1 ? 1 : (kmax > 8 ? 8 : kmax);
        kmax_cache.store(kmax, std::memory_order_relaxed);
    }
    const int k = pick_wg_per_cu(kmax, wg_per_cu);
    const size_t pad = k < kmax ? lds_pad_for(kern, 64 * W, k, pad_cache) : 0;
    hipLaunchKernelGGL(kern, grid, dim3(64 * W), pad, st, a);
    return hipGetLastError();
}

template <int D, int W, bool MASKED>
static hipError_t launch_dw(const Args& a, bool vec, bool fast, int wg_per_cu, dim3 grid, hipStream_t st) {
    if (a.params) {
        // constants in device memory: the two planned kernels (the plan selects
        // one of them) when the layout admits the fast kernel, the general
        // kernel otherwise
        if constexpr (D <= 128) {
            if (fast) {
                hipLaunchKernelGGL((fwd_fast_planned<D, W, MASKED>), grid, dim3(64 * W), 0, st, a);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
                hipLaunchKernelGGL((fwd_planned_rest<D, W, MASKED>), grid, dim3(64 * W), 0, st, a);
                return hipGetLastError();
            }
        }
        if (vec)
            hipLaunchKernelGGL((fwd_general<D, W, MASKED, true>), grid, dim3(64 * W), 0, st, a);
        else
            hipLaunchKernelGGL((fwd_general<D, W, MASKED, false>), grid, dim3(64 * W), 0, st, a);
        return hipGetLastError();
    }
    if constexpr (D <= 128) {
        // DYN: the identity of the rescale by alpha = rs is proved per row in-kernel
        if (fast) return a.id_ok ? launch_fast<D, W, MASKED, false>(a, wg_per_cu, grid, st)
                                 : launch_fast<D, W, MASKED, true>(a, wg_per_cu, grid, st);
    }
    if (vec)
        hipLaunchKernelGGL((fwd_general<D, W, MASKED, true>), grid, dim3(64 * W), 0, st, a);
    else
        hipLaunchKernelGGL((fwd_general<D, W, MASKED, false>), grid, dim3(64 * W), 0, st, a);
    return hipGetLastError();
}

// Launch of the kernel chosen for head dim D and masking (defined for every
// (D, MASKED) by qflash_fwd_inst.hip; the other units see it as extern).
template <int D, bool MASKED>
hipError_t launch_d(const Args& a, int W, bool vec, bool fast, int wg_per_cu, dim3 grid, hipStream_t st) {
    switch (W) {
        case 1: return launch_dw<D, 1, MASKED>(a, vec, fast, wg_per_cu, grid, st);
        case 2: return launch_dw<D, 2, MASKED>(a, vec, fast, wg_per_cu, grid, st);
        default: return launch_dw<D, 4, MASKED>(a, vec, fast, wg_per_cu, grid, st);
    }
}

#define QF_LAUNCH_D_EXTERN(D)                                                                                  \
    extern template hipError_t launch_d<D, false>(const Args&, int, bool, bool, int, dim3, hipStream_t);     \
    extern template hipError_t launch_d<D, true>(const Args&, int, bool, bool, int, dim3, hipStream_t);
#ifndef QF_INST_D
QF_LAUNCH_D_EXTERN(32)
QF_LAUNCH_D_EXTERN(64)
QF_LAUNCH_D_EXTERN(128)
QF_LAUNCH_D_EXTERN(256)
#endif
#undef QF_LAUNCH_D_EXTERN

}  // namespace qf
