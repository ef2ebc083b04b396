// Per-tensor absmax scales and int8 quantisation of Q, K, V on the device.
//
// Replaces the host sequence of qflash_forward (qflash/kernel.py:294-296 and
// :309-311), which torch runs as ~12 elementwise / reduction passes over the
// floating-point inputs:
//     x_scale = x.abs().amax() / 127                  (in the input dtype T)
//     qk      = q_scale * k_scale                     (in T; .item() on the host)
//     x_i8    = clamp(round(x / x_scale), -128, 127).to(int8)
// Here: one pass reads each input once for the absmax, a one-wave pass forms
// the scales in T (qflash_hip_scales), and one pass reads each input again and
// writes the int8 codes (qflash_hip_quantize).  The arithmetic is torch's
// on the GPU for T: fp32 natively; fp16 / bf16 as fp32 opmath rounded back to
// T after every operation; a division by the host scalar 127 is a product
// with RN_fp32(1/127); round half to even; clamp; conversion.
//
// Both passes stream each tensor in its memory order: the host sorts the
// dimensions by stride and merges those that are contiguous in memory (a
// token-major (B, N, H, D) view of a dense buffer becomes one run of
// B*N*H*D elements), and the device walks runs of the innermost merged
// dimension in 16-byte chunks, 32 KiB of input per work unit.  Layouts with
// a non-unit innermost stride, or runs that are not 16-byte aligned, are
// walked element by element.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>

#include <atomic>

#include "../../include/qflash_hip.h"
#include "qf_common.h"

namespace qfq {

using qferr::fail;
using qferr::g_err;
using qfs::round_t;
using qfs::store_t;
using qfs::to_float;
using qfs::wave_max;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kSeg = 8 * kThreads;  // 16-byte chunks per work unit
constexpr int kSlots = qfs::kScaleSlots;  // atomic-max slots per tensor (spreads the contention)
constexpr int32_t kNegInfBias = -(1 << 20);  // qflash/kernel.py:288

// One tensor as `rows` runs of L contiguous elements; a run's start is
// sum_i idx_i * in_stride_i over up to 3 outer dimensions (sizes n[], the
// fastest-varying last).  Quantisation writes the same runs of the output.
struct Geo {
    const void* p;
    int8_t* o;
    int64_t L;
    int64_t rows;
    int nout;            // outer dimensions in use
    int64_t n[3], is[3], os[3];
    int vec;             // 16-byte chunks
    // flat: the outer dimensions merged into one of uniform stride (rows runs,
    // run r at r * rs in the input and r * ros in the output); the chunks of
    // all runs are then split into equal contiguous slices, one per block
    int flat;
    int64_t rs, ros;
    float inv_cpr;       // 1 / (16-byte chunks per run), for the chunk -> run split
    // element-wise fallback: the original 4-D sizes and strides
    int64_t n4[4], s4[4], o4[4];
};

// |x| as an unsigned bit pattern: for non-negative floats the order of the
// patterns is the order of the values, NaN above +inf (torch.amax propagates
// NaN, and so does the maximum of the patterns).
template <int DT>
__device__ __forceinline__ uint32_t abs_bits(uint32_t raw) {
    return DT == QFLASH_HIP_F32 ? (raw & 0x7fffffffu) : (raw & 0x7fffu);
}

template <int DT>
constexpr int esize() { return DT == QFLASH_HIP_F32 ? 4 : 2; }

template <int DT>
__device__ __forceinline__ uint32_t load_raw(const void* p, int64_t i) {
    if constexpr (DT == QFLASH_HIP_F32) return reinterpret_cast<const uint32_t*>(p)[i];
    else return reinterpret_cast<const uint16_t*>(p)[i];
}

template <int DT>
__device__ __forceinline__ float load_t(const void* p, int64_t i) {
    return to_float<DT>(load_raw<DT>(p, i));
}

// clamp(round(x / s), -128, 127) -> int8 (kernel.py:309-311); s is a device
// tensor, so the division is a true division in fp32.  NaN stays NaN through
// round and clamp and converts to 0.
template <int DT>
__device__ __forceinline__ int8_t quant1(float x, float s) {
    const float r = rintf(round_t<DT>(__fdiv_rn(x, s)));
    if (r != r) return 0;
    return (int8_t)(int32_t)(r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r));
}

// fp32 quant1 through the reciprocal, for a normal scale s whose r = RN(1/s)
// is normal: q0 = RN(x * r) = (x / s)(1 + d), |d| <= 2^-23 + 2^-48, so while
// |x / s| < 131, q0 is within 2^-16 of x / s and within 2^-15 of RN(x / s)
// (half an ulp, <= 2^-17, apart).  When q0 is farther than 2^-14 from every
// half-integer, rint(q0) = rint(RN(x / s)); when |q0| >= 130, |x / s| > 129.9
// and the clamp gives the bound either way.  The other elements (a fraction of
// about 2^-13, and NaN) take the IEEE division.
__device__ __forceinline__ int8_t quant1_rcp(float x, float s, float r) {
    const float q0 = x * r;
    if (fabsf(q0) >= 130.0f) return q0 > 0.f ? (int8_t)127 : (int8_t)-128;
    const float n = rintf(q0);
    const float h = 0.5f - fabsf(q0 - n);  // distance to the nearest half-integer
    if (h > 0x1p-14f) return (int8_t)(int32_t)(n < -128.0f ? -128.0f : (n > 127.0f ? 127.0f : n));
    return quant1<QFLASH_HIP_F32>(x, s);
}

// quant1_rcp's fast path alone: the code, and in exact whether it equals
// quant1's (false: the element needs the IEEE division, NaN included)
__device__ __forceinline__ int32_t quant1_rcp_try(float x, float r, bool& exact) {
    const float q0 = x * r;
    const float n = rintf(q0);
    const bool big = fabsf(q0) >= 130.0f;
    exact = big || 0.5f - fabsf(q0 - n) > 0x1p-14f;
    const float c = big ? (q0 > 0.f ? 127.0f : -128.0f) : fminf(fmaxf(n, -128.0f), 127.0f);
    return (int32_t)c;
}

struct GeoSet {
    Geo g[3];  // q, k, v
};

// Start offsets (elements) of run r in the input and the output.
__device__ __forceinline__ void run_start(const Geo& g, int64_t r, int64_t& in, int64_t& out) {
    in = 0;
    out = 0;
#pragma unroll
    for (int i = 2; i >= 0; --i) {
        if (i < g.nout) {
            const int64_t idx = r % g.n[i];
            r /= g.n[i];
            in += idx * g.is[i];
            out += idx * g.os[i];
        }
    }
}

// MODE 0: absmax of the patterns into ws[tensor * kSlots + block % kSlots]
// (atomic max; ws is zero on entry).  Blocks are dealt to the 8 XCDs round
// robin, so each slot is updated from one XCD only (its L2); the scales are
// formed by a second kernel, after this one, which sees every slot.  (A
// last-block-done counter in this kernel needs device-scope fences that write
// back the L2 of every block's XCD: measured at twice the pass's time.)
// MODE 1: int8 codes with scale scales[tensor].
template <int DT, int MODE>
__global__ __launch_bounds__(kThreads) void stream_kernel(GeoSet gs, uint32_t* ws, void* scales) {
    const Geo& g = gs.g[blockIdx.y];
    float s = 0.f, rcp = 0.f;
    bool rcp_ok = false;
    if constexpr (MODE == 1) {
        s = load_t<DT>(scales, blockIdx.y);
        rcp = __frcp_rn(s);
        rcp_ok = s >= 0x1p-126f && s < 0x1p126f;  // s and 1/s normal
    }
    uint32_t m = 0;
    if (g.flat) {
        constexpr int EPC = 16 / esize<DT>();
        constexpr int U = 4;  // chunks in flight per thread
        const uint32_t cpr = (uint32_t)(g.L / EPC);
        const uint32_t F = (uint32_t)g.rows * cpr;
        const uint32_t per = (F + gridDim.x - 1) / gridDim.x;
        const uint32_t s0 = blockIdx.x * per, s1 = min(F, s0 + per);
        const uint8_t* src = reinterpret_cast<const uint8_t*>(g.p);
        for (uint32_t base = s0 + threadIdx.x; base < s1; base += kThreads * U) {
            u32x4 v[U];
            int64_t out[U];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const uint32_t f = base + k * kThreads;
                if (f < s1) {
                    // run r = f / cpr from a float estimate, corrected to the exact quotient
                    uint32_t r = 0, c = f;
                    if (g.rows > 1) {
                        r = (uint32_t)((float)f * g.inv_cpr);
                        if (r * cpr > f) --r;
                        else if ((r + 1) * cpr <= f) ++r;
                        c = f - r * cpr;
                    }
                    v[k] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(src + ((int64_t)r * g.rs * esize<DT>() + (int64_t)c * 16)));
                    out[k] = (int64_t)r * g.ros + (int64_t)c * EPC;
                }
            }
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (base + k * kThreads >= s1) break;
                const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
                if constexpr (MODE == 0) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (DT == QFLASH_HIP_F32) {
                            m = max(m, abs_bits<DT>(w[e]));
                        } else {
                            m = max(m, abs_bits<DT>(w[e] & 0xffffu));
                            m = max(m, abs_bits<DT>(w[e] >> 16));
                        }
                    }
                } else {
                    int8_t* dst = g.o + out[k];
                    if constexpr (DT == QFLASH_HIP_F32) {
                        uint32_t packed = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float xe = __uint_as_float(w[e]);
                            const int8_t c = rcp_ok ? quant1_rcp(xe, s, rcp) : quant1<DT>(xe, s);
                            packed |= (uint32_t)(uint8_t)c << (8 * e);
                        }
                        __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(dst));
                    } else {
                        uint32_t lo = 0, hi = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t a = (uint8_t)quant1<DT>(to_float<DT>(w[e] & 0xffffu), s);
                            const uint32_t b = (uint8_t)quant1<DT>(to_float<DT>(w[e] >> 16), s);
                            const uint32_t pair = a | (b << 8);
                            if (e < 2) lo |= pair << (16 * e);
                            else hi |= pair << (16 * (e - 2));
                        }
                        __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(dst));
                    }
                }
            }
        }
    } else if (g.vec) {
        constexpr int EPC = 16 / esize<DT>();  // elements per 16-byte chunk
        const int64_t cpr = g.L / EPC;
        const int64_t segs = (cpr + kSeg - 1) / kSeg;
        for (int64_t u = blockIdx.x; u < g.rows * segs; u += gridDim.x) {
            int64_t in, out;
            run_start(g, u / segs, in, out);
            const int64_t c0 = (u % segs) * kSeg, c1 = min(cpr, c0 + kSeg);
            const uint8_t* src = reinterpret_cast<const uint8_t*>(g.p) + in * esize<DT>();
#pragma unroll 4
            for (int64_t c = c0 + threadIdx.x; c < c1; c += kThreads) {
                const uint4 v = *reinterpret_cast<const uint4*>(src + c * 16);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
                if constexpr (MODE == 0) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (DT == QFLASH_HIP_F32) {
                            m = max(m, abs_bits<DT>(w[e]));
                        } else {
                            m = max(m, abs_bits<DT>(w[e] & 0xffffu));
                            m = max(m, abs_bits<DT>(w[e] >> 16));
                        }
                    }
                } else {
                    int8_t* dst = g.o + out + c * EPC;
                    if constexpr (DT == QFLASH_HIP_F32) {
                        uint32_t packed = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            packed |= (uint32_t)(uint8_t)quant1<DT>(__uint_as_float(w[e]), s) << (8 * e);
                        *reinterpret_cast<uint32_t*>(dst) = packed;
                    } else {
                        uint32_t lo = 0, hi = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t a = (uint8_t)quant1<DT>(to_float<DT>(w[e] & 0xffffu), s);
                            const uint32_t b = (uint8_t)quant1<DT>(to_float<DT>(w[e] >> 16), s);
                            const uint32_t pair = a | (b << 8);
                            if (e < 2) lo |= pair << (16 * e);
                            else hi |= pair << (16 * (e - 2));
                        }
                        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
                    }
                }
            }
        }
    } else {  // element by element over the original 4-D index space
        const int64_t total = g.n4[0] * g.n4[1] * g.n4[2] * g.n4[3];
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
            int64_t r = i, in = 0, out = 0;
#pragma unroll
            for (int d = 3; d >= 0; --d) {
                const int64_t idx = r % g.n4[d];
                r /= g.n4[d];
                in += idx * g.s4[d];
                out += idx * g.o4[d];
            }
            if constexpr (MODE == 0) m = max(m, abs_bits<DT>(load_raw<DT>(g.p, in)));
            else g.o[out] = quant1<DT>(load_t<DT>(g.p, in), s);
        }
    }
    if constexpr (MODE == 0) {
        __shared__ uint32_t red[kThreads / 64];
        m = wave_max(m);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < kThreads / 64; ++w) m = max(m, red[w]);
            atomicMax(ws + blockIdx.y * kSlots + blockIdx.x % kSlots, m);
        }
    }
}

// The scales from the slots of the absmax pass (one wave), which it sets back
// to zero for the next call.
template <int DT>
__global__ __launch_bounds__(64) void scales_kernel(uint32_t* ws, void* scales) {
    qfs::reduce_scale_slots<DT>(ws, scales);
}

// Runs of a tensor in its memory order (see the file comment).  `o` / `os4`
// describe the output of the quantisation (nullptr for the absmax pass).
static int make_geo(Geo& g, const void* p, const int64_t* n4, const int64_t* s4, int8_t* o, const int64_t* os4,
                    int es, int idx) {
    g.p = p;
    g.o = o;
    for (int d = 0; d < 4; ++d) {
        if (n4[d] <= 0) return fail(QFLASH_HIP_EINVAL, "tensor %d has an empty dimension", idx);
        if (s4[d] < 0 || (os4 && os4[d] < 0)) return fail(QFLASH_HIP_EINVAL, "tensor %d has a negative stride", idx);
        g.n4[d] = n4[d];
        g.s4[d] = s4[d];
        g.o4[d] = os4 ? os4[d] : 0;
    }
    // outer dimensions 0..2, slowest first by input stride (stable)
    int ord[3] = {0, 1, 2};
    for (int i = 0; i < 3; ++i)
        for (int j = i + 1; j < 3; ++j)
            if (s4[ord[j]] > s4[ord[i]]) {
                const int t = ord[i];
                ord[i] = ord[j];
                ord[j] = t;
            }
    g.vec = s4[3] == 1 && (!os4 || os4[3] == 1);
    g.L = n4[3];
    int n = 3;
    // merge the fastest outer dimension into the run while it is contiguous with it
    while (n > 0 && g.vec) {
        const int d = ord[n - 1];
        if (s4[d] == g.L && (!os4 || os4[d] == g.L)) {
            g.L *= n4[d];
            --n;
        } else if (n4[d] == 1) {
            --n;
        } else {
            break;
        }
    }
    g.nout = 0;
    g.rows = 1;
    for (int i = 0; i < n; ++i) {
        const int d = ord[i];
        if (n4[d] == 1) continue;
        g.n[g.nout] = n4[d];
        g.is[g.nout] = s4[d];
        g.os[g.nout] = os4 ? os4[d] : 0;
        g.rows *= n4[d];
        ++g.nout;
    }
    const int epc = 16 / es;
    if (g.vec) {
        g.vec = (g.L % epc == 0) && ((uintptr_t)p % 16 == 0) && (!o || (uintptr_t)o % epc == 0);
        for (int i = 0; i < g.nout && g.vec; ++i) g.vec = (g.is[i] % epc == 0) && (!o || g.os[i] % epc == 0);
    }
    // flat: outer dimensions that step uniformly (stride of i = stride of i+1 times
    // size of i+1, in the input and the output) are one dimension of runs
    g.flat = 0;
    if (g.vec) {
        bool uniform = true;
        for (int i = 0; i + 1 < g.nout && uniform; ++i)
            uniform = g.is[i] == g.is[i + 1] * g.n[i + 1] && (!o || g.os[i] == g.os[i + 1] * g.n[i + 1]);
        const int64_t cpr = g.L / epc;
        if (uniform && g.rows * cpr < (1ll << 31) && g.rows < (1ll << 22)) {
            g.flat = 1;
            g.rs = g.nout ? g.is[g.nout - 1] : 0;
            g.ros = g.nout ? g.os[g.nout - 1] : 0;
            g.inv_cpr = 1.0f / (float)cpr;
        }
    }
    return 0;
}

// Blocks per tensor.  flat: `cpt` 16-byte chunks per thread, but at least
// QF_MIN_BLOCKS blocks (measured on MI355X over 10-134 MB per tensor: the
// absmax pass, which ends each block with an atomic, is fastest at
// QF_ABSMAX_CPT, the quantisation pass at QF_QUANT_CPT; small tensors need
// the floor to keep the CUs busy).
#ifndef QF_ABSMAX_CPT
#define QF_ABSMAX_CPT 128
#endif
#ifndef QF_QUANT_CPT
#define QF_QUANT_CPT 2
#endif
#ifndef QF_MIN_BLOCKS
#define QF_MIN_BLOCKS 256
#endif
#ifndef QF_MAX_BLOCKS
#define QF_MAX_BLOCKS 16384
#endif
static unsigned grid_x(const Geo* g, int es, int cpt) {
    int64_t units = 1;
    for (int i = 0; i < 3; ++i) {
        int64_t u;
        if (g[i].flat) {
            const int64_t chunks = g[i].rows * (g[i].L * es / 16);
            u = (chunks + cpt * kThreads - 1) / (cpt * kThreads);
            const int64_t floor_u = chunks < QF_MIN_BLOCKS ? chunks : QF_MIN_BLOCKS;
            u = u > floor_u ? u : floor_u;
        } else {
            u = g[i].vec ? g[i].rows * ((g[i].L * es / 16 + kSeg - 1) / kSeg)
                         : (g[i].n4[0] * g[i].n4[1] * g[i].n4[2] * g[i].n4[3] + kThreads - 1) / kThreads;
        }
        units = units > u ? units : u;
    }
    const int64_t cap = g[0].flat && g[1].flat && g[2].flat ? QF_MAX_BLOCKS : 2048;
    return (unsigned)(units < cap ? units : cap);
}

// The absmax pass; then the scales kernel unless `scales` is null (the
// caller forms the scales itself from the slots).
template <int DT>
static int scales_dt(Geo* g, void* scales, uint32_t* ws, hipStream_t st) {
    const dim3 grid(grid_x(g, esize<DT>(), QF_ABSMAX_CPT), 3);
    const GeoSet gs = {{g[0], g[1], g[2]}};
    hipLaunchKernelGGL((stream_kernel<DT, 0>), grid, dim3(kThreads), 0, st, gs, ws, nullptr);
    if (scales) hipLaunchKernelGGL((scales_kernel<DT>), dim3(1), dim3(64), 0, st, ws, scales);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

template <int DT>
static int quant_dt(Geo* g, const void* scales, hipStream_t st) {
    const dim3 grid(grid_x(g, esize<DT>(), QF_QUANT_CPT), 3);
    const GeoSet gs = {{g[0], g[1], g[2]}};
    hipLaunchKernelGGL((stream_kernel<DT, 1>), grid, dim3(kThreads), 0, st, gs, nullptr, const_cast<void*>(scales));
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

// int32 bias of a window mask (qflash_hip_window_bias): one element per
// thread, the torch ops' fp32 roundings in their order (an add, the compare
// with -100, two products by the host scalars RN(LOG2E) and RN(1/sm_scale) --
// torch multiplies by the reciprocal of a host-scalar divisor -- round half to
// even, conversion).
__device__ __forceinline__ int32_t bias_of(float x, float log2e, float inv_sm) {
    const bool masked = x < -100.0f;
    const float y = __fmul_rn(__fmul_rn(masked ? 0.0f : x, log2e), inv_sm);
    return masked ? kNegInfBias : (int32_t)rintf(y);
}

// RN_fp32(1 / RN_fp32(sm_scale)) from the double at words 14-15 of a device
// parameter block (qflash_hip_constants), as the host forms it.
__device__ __forceinline__ float inv_sm_of(const int32_t* params) {
    const uint64_t b = (uint32_t)params[14] | ((uint64_t)(uint32_t)params[15] << 32);
    return __fdiv_rn(1.0f, (float)__longlong_as_double((long long)b));
}

__global__ __launch_bounds__(256) void window_bias_kernel(const float* rel, const float* mask, int32_t H,
                                                           int32_t nn, int64_t total, float log2e, float inv_sm,
                                                           const int32_t* params, int32_t* out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= total) return;
    if (params) {
        if (params[0] != 0) return;
        inv_sm = inv_sm_of(params);
    }
    const int32_t ij = (int32_t)(e % nn), wh = (int32_t)(e / nn);
    const int32_t h = wh % H, w = wh / H;
    float x = rel[(int64_t)h * nn + ij];
    if (mask) x = __fadd_rn(x, mask[(int64_t)w * nn + ij]);
    out[e] = bias_of(x, log2e, inv_sm);
}

// qflash_hip_mask_bias: four elements per thread, 16-byte loads and stores
// when both buffers are 16-byte aligned.
__global__ __launch_bounds__(256) void mask_bias_kernel(const float* mask, int64_t n, bool vec, float log2e,
                                                         float inv_sm, const int32_t* params, int32_t* out) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (params) {
        if (params[0] != 0) return;
        inv_sm = inv_sm_of(params);
    }
    if (vec && i + 4 <= n) {
        const float4 x = *reinterpret_cast<const float4*>(mask + i);
        *reinterpret_cast<int4*>(out + i) = int4{bias_of(x.x, log2e, inv_sm), bias_of(x.y, log2e, inv_sm),
                                                 bias_of(x.z, log2e, inv_sm), bias_of(x.w, log2e, inv_sm)};
    } else {
        for (int j = 0; j < 4; ++j)
            if (i + j < n) out[i + j] = bias_of(mask[i + j], log2e, inv_sm);
    }
}

// ---- qflash_hip_scales_noalloc: the absmax workspace in static device memory.
// One array per GPU (each device that loads the library holds its own copy,
// kept until the process ends), found through hipGetSymbolAddress once per
// device; host code uses only that address, never the array's name.
__device__ __align__(256) uint32_t scratch[QFLASH_HIP_SCALES_WORKSPACE];
constexpr int kMaxDevices = 64;
static std::atomic<uint32_t*> g_scratch[kMaxDevices];

__global__ __launch_bounds__(256) void clear_kernel(uint32_t* p, int n) {
    for (int i = threadIdx.x; i < n; i += 256) p[i] = 0u;
}

// The device address of `scratch` on device `dev` (the current device), or
// nullptr with the error message set.
static uint32_t* scratch_ptr(int dev) {
    uint32_t* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p) return p;
    void* a = nullptr;
    const hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !a) {
        fail(QFLASH_HIP_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        return nullptr;
    }
    g_scratch[dev].store(static_cast<uint32_t*>(a), std::memory_order_release);
    return static_cast<uint32_t*>(a);
}


// ---- int8 QKV projection fused with the quantiser (qflash_hip_qkv_int8) -----
// acc = x8 . w8^T on int8 MFMA (exact int32), y = RN(RN(fp32(acc) * RN(s_x *
// s_w[c])) + b[c]) per output channel c, and of y's three column thirds (q, k,
// v) the per-tensor scales and int8 codes exactly as qflash_hip_scales /
// qflash_hip_quantize would compute them from a materialised fp32 y.  y is
// never written: pass 0 reduces its absmax into the scales workspace, the
// scales kernel forms the scales, pass 1 recomputes y and stores the codes.
typedef int32_t pi32x4 __attribute__((ext_vector_type(4)));
typedef int32_t pi32x16 __attribute__((ext_vector_type(16)));
#ifndef QF_PROJ_TM
#define QF_PROJ_TM 128
#endif
constexpr int kProjTile = 128;         // columns (output channels) per workgroup
constexpr int kProjTM = QF_PROJ_TM;    // rows (tokens) per workgroup: 128 or 256
constexpr int kProjWaves = kProjTM / 32;  // waves of 64 x 64: kProjTM / 64 row groups x 2 column groups
constexpr int kProjThreads = 64 * kProjWaves;

struct ProjArgs {
    const int8_t* x8;
    const int8_t* w8;
    const float* w_scale;
    const float* bias;
    const float* x_scale;
    int32_t M, K, Nc, C;  // C = Nc / 3, the columns of each of q, k, v
    uint32_t* ws;
    const float* scales;
    int8_t* out;
};


// One workgroup: a 128 x 128 tile of y, four waves of 64 x 64 (2 x 2 blocks of
// v_mfma_i32_32x32x32_i8: lane l holds row l % 32 of x8 and of w8, 16 bytes of
// each 32-byte K block's half l / 32; result register v of lane l is row
// 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32).  Rows >= M and columns >= Nc
// read as 0 (buffer range) and take no part in the results.
// RN(RN(a * b) + c): the product and the sum rounded each (hipcc contracts
// a * b + c into one fused multiply-add unless told not to)
__device__ inline float mul_add_rn(float a, float b, float c) {
#pragma clang fp contract(off)
    return a * b + c;
}

// The workgroup's 128 rows of x8 and 128 rows of w8 go through LDS in stages
// of kProjK bytes of K, double-buffered: each thread copies its 16-byte chunks
// HBM -> LDS with buffer_load ... lds (kProjCopies per operand per stage), so
// the four waves share every load; row r's chunk c sits at r * kProjK + 16 * (c ^ swz(r))
// so that the ds_read_b128 of eight consecutive rows hit distinct banks.
#ifndef QF_PROJ_K
#define QF_PROJ_K 64
#endif
constexpr int kProjK = QF_PROJ_K;                     // bytes of K per stage (64 or 128)
constexpr int kProjCpr = kProjK / 16;                 // 16-byte chunks per row
constexpr int kProjCopiesA = kProjTM * kProjCpr / kProjThreads;    // chunks per thread of x8
constexpr int kProjCopiesB = kProjTile * kProjCpr / kProjThreads;  // and of w8
constexpr int kProjStage = (kProjTM + kProjTile) * kProjK;         // A and B tiles of one stage
static_assert(kProjK == 64 || kProjK == 128, "stages of 64 or 128 bytes of K");
// chunk position of row r: eight consecutive rows at one chunk land in the
// eight 16-byte bank groups
__device__ __forceinline__ int proj_swz(int r) { return kProjCpr == 4 ? (r >> 1) & 3 : r & 7; }

template <int MODE>
__global__ __launch_bounds__(kProjThreads) void proj_kernel(ProjArgs p) {
    __shared__ __attribute__((aligned(16))) int8_t lds[2 * kProjStage];
    constexpr int RG = kProjTM / 64;  // row groups of waves
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, g = lane >> 5;
    // tiles in XCD-aware order: the column tiles of one row tile run on one XCD,
    // so its x8 rows come from HBM once into that XCD's L2
    const int nct = (p.Nc + kProjTile - 1) / kProjTile;
    const int tile = qfs::xcd_order(blockIdx.x, gridDim.x);
    const int mt = (tile / nct) * kProjTM, nt = (tile % nct) * kProjTile;
    const int m0 = mt + (wave % RG) * 64;
    const int n0 = nt + (wave / RG) * 64;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)p.x8, 0, p.M * p.K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.w8, 0, p.Nc * p.K, 0x00020000);
    // this thread's copy slots: slot s = kProjThreads i + tid is row s / kProjCpr,
    // stored chunk s % kProjCpr (A tile first, then the B tile at kProjTM * kProjK)
    int32_t ca[kProjCopiesA], cb[kProjCopiesB];
#pragma unroll
    for (int i = 0; i < kProjCopiesA; ++i) {
        const int sl = kProjThreads * i + tid, r = sl / kProjCpr, c = (sl % kProjCpr) ^ proj_swz(r);
        ca[i] = (mt + r) * p.K + 16 * c;
    }
#pragma unroll
    for (int i = 0; i < kProjCopiesB; ++i) {
        const int sl = kProjThreads * i + tid, r = sl / kProjCpr, c = (sl % kProjCpr) ^ proj_swz(r);
        cb[i] = (nt + r) * p.K + 16 * c;
    }
    auto issue = [&](int8_t* buf, int k0) {
#pragma unroll
        for (int i = 0; i < kProjCopiesA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void*)(buf + (kProjThreads * i + 64 * wave) * 16), 16, ca[i],
                k0, 0, 0);
#pragma unroll
        for (int i = 0; i < kProjCopiesB; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw,
                (__attribute__((address_space(3))) void*)(buf + kProjTM * kProjK + (kProjThreads * i + 64 * wave) * 16),
                16, cb[i], k0, 0, 0);
    };
    // LDS offsets of this lane's fragment rows (chunk 0); the chunk is xor-ed in per K step
    int ra[2], rb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ra[i] = (wave % RG) * 64 + 32 * i + lr;
        rb[i] = (wave / RG) * 64 + 32 * i + lr;
    }
    pi32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = pi32x16{};
    const int nst = (p.K + kProjK - 1) / kProjK;
    issue(lds, 0);
    for (int st = 0; st < nst; ++st) {
        int8_t* buf = lds + (st & 1) * kProjStage;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's copies of stage st
        __syncthreads();                     // every copy of stage st; every read of stage st - 1
        if (st + 1 < nst) issue(lds + ((st + 1) & 1) * kProjStage, (st + 1) * kProjK);
        const int nk = min(kProjK, p.K - st * kProjK) / 32;  // 32-byte MFMA steps in this stage
        for (int kk = 0; kk < nk; ++kk) {
            const int c = 2 * kk + g;
            pi32x4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *reinterpret_cast<const pi32x4*>(buf + ra[i] * kProjK + 16 * (c ^ proj_swz(ra[i])));
                b[i] = *reinterpret_cast<const pi32x4*>(buf + kProjTM * kProjK + rb[i] * kProjK +
                                                        16 * (c ^ proj_swz(rb[i])));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    const float sx = *p.x_scale;
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc((void*)p.out, 0, MODE == 1 ? p.M * p.Nc : 0,
                                                                       0x00020000);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int nb = n0 + 32 * j;  // the column block (32 | C: one of q, k, v)
        if (nb >= p.Nc) break;       // uniform over the wave
        const int n = nb + lr;
        const int t = nb / p.C;
        const float gsc = sx * p.w_scale[n];
        const float bb = p.bias ? p.bias[n] : 0.0f;
        uint32_t mx = 0;
        float s = 0.f, rcp = 0.f;
        bool rcp_ok = false;
        if constexpr (MODE == 1) {
            s = p.scales[t];
            rcp = __frcp_rn(s);
            rcp_ok = s >= 0x1p-126f && s < 0x1p126f;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // y of result register v (row m0 + 32 i + 8 (v / 4) + 4 g + v % 4, column n)
            auto yv = [&](int v) {
                return p.bias ? mul_add_rn((float)acc[i][j][v], gsc, bb) : (float)acc[i][j][v] * gsc;
            };
            if constexpr (MODE == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t ay = __float_as_uint(yv(v)) & 0x7fffffffu;
                    if (m0 + 32 * i + 8 * (v >> 2) + 4 * g + (v & 3) < p.M) mx = max(mx, ay);
                }
            } else {
#pragma unroll
                for (int v4 = 0; v4 < 4; ++v4) {
                    // codes of registers 4 v4 .. 4 v4 + 3 (rows m0 + 32 i + 8 v4 + 4 g + r
                    // of column n, byte r) through the reciprocal with no branch per
                    // element; the few near a half-integer (all of them without a
                    // usable reciprocal) are redone with the IEEE division
                    uint32_t packed = 0, slow = rcp_ok ? 0u : 0xfu;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        bool ok;
                        const int32_t c = quant1_rcp_try(yv(4 * v4 + r), rcp, ok);
                        packed |= (uint32_t)(c & 0xff) << (8 * r);
                        slow |= ok ? 0u : 1u << r;
                    }
                    if (slow) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (slow >> r & 1) {
                                const uint32_t c = (uint8_t)quant1<QFLASH_HIP_F32>(yv(4 * v4 + r), s);
                                packed = (packed & ~(0xffu << (8 * r))) | c << (8 * r);
                            }
                    }
                    // 4 x 4 byte transpose over the lane quad (columns 4a .. 4a + 3): lane
                    // 4a + b then holds row m0 + 32 i + 8 v4 + 4 g + b of those four columns
                    const int b = lr & 3;
                    const uint32_t x = (uint32_t)__builtin_amdgcn_mov_dpp((int)packed, 0xB1, 0xF, 0xF, false);
                    const uint32_t h = __builtin_amdgcn_perm(x, packed, (b & 1) ? 0x03070105u : 0x06020400u);
                    const uint32_t y = (uint32_t)__builtin_amdgcn_mov_dpp((int)h, 0x4E, 0xF, 0xF, false);
                    const uint32_t row = __builtin_amdgcn_perm(y, h, (b & 2) ? 0x03020706u : 0x05040100u);
                    const int m = m0 + 32 * i + 8 * v4 + 4 * g + b;
                    // rows >= M lie past the buffer's end: the store is dropped
                    __builtin_amdgcn_raw_buffer_store_b32(row, ro, m * p.Nc + nb + 4 * (lr >> 2), 0, 0);
                }
            }
        }
        if constexpr (MODE == 0) {
            mx = wave_max(mx);
            if (lane == 0) atomicMax(p.ws + t * kSlots + blockIdx.x % kSlots, mx);
        }
    }
}

static int qkv_int8(const ProjArgs& pa, float* scales, hipStream_t st) {
    const dim3 grid((unsigned)(((pa.M + kProjTM - 1) / kProjTM) * ((pa.Nc + kProjTile - 1) / kProjTile)));
    hipLaunchKernelGGL((proj_kernel<0>), grid, dim3(kProjThreads), 0, st, pa);
    hipLaunchKernelGGL((scales_kernel<QFLASH_HIP_F32>), dim3(1), dim3(64), 0, st, pa.ws, (void*)scales);
    ProjArgs p1 = pa;
    p1.scales = scales;
    hipLaunchKernelGGL((proj_kernel<1>), grid, dim3(kProjThreads), 0, st, p1);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

static int esize_of(int32_t dtype) {
    return dtype == QFLASH_HIP_F32 ? 4 : (dtype == QFLASH_HIP_F16 || dtype == QFLASH_HIP_BF16 ? 2 : 0);
}

// qflash_hip_scales, and without its scales kernel when `scales` is null.
int absmax_pass(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream) {
    if (!q || !k || !v || !shapes_strides || !workspace)
        return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    const int es = esize_of(dtype);
    if (!es) return fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    if (workspace_elems < QFLASH_HIP_SCALES_WORKSPACE)
        return fail(QFLASH_HIP_EINVAL, "workspace holds %lld entries, %d needed", (long long)workspace_elems,
                         QFLASH_HIP_SCALES_WORKSPACE);
    Geo g[3];
    const void* x[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (int rc = make_geo(g[i], x[i], shapes_strides + 8 * i, shapes_strides + 8 * i + 4, nullptr,
                                   nullptr, es, i))
            return rc;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case QFLASH_HIP_F32: return scales_dt<QFLASH_HIP_F32>(g, scales, workspace, st);
        case QFLASH_HIP_F16: return scales_dt<QFLASH_HIP_F16>(g, scales, workspace, st);
        default: return scales_dt<QFLASH_HIP_BF16>(g, scales, workspace, st);
    }
}

}  // namespace qfq

extern "C" {

int qflash_hip_scales(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                      void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream) {
    qfq::g_err[0] = 0;
    if (!scales) return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    return qfq::absmax_pass(q, k, v, dtype, shapes_strides, scales, workspace, workspace_elems, stream);
}

int qflash_hip_qkv_int8(const int8_t* x8, const int8_t* w8, const float* w_scale, const float* bias,
                        const float* x_scale, int32_t M, int32_t K, int32_t Nc, float* scales, int8_t* codes,
                        uint32_t* workspace, int64_t workspace_elems, void* stream) {
    qfq::g_err[0] = 0;
    if (!x8 || !w8 || !w_scale || !x_scale || !scales || !codes || !workspace)
        return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (M < 1 || K < 32 || K % 32 || Nc < 96 || Nc % 96)
        return qfq::fail(QFLASH_HIP_EINVAL, "shape M=%d K=%d Nc=%d: need M >= 1, K a multiple of 32, Nc = 3 C with C a "
                         "multiple of 32", M, K, Nc);
    // byte offsets of the GEMM's loads and stores (rows up to the last tile's end) in 31 bits
    if ((int64_t)(M + 255) * K > INT32_MAX - 64 || (int64_t)(Nc + 127) * K > INT32_MAX - 64 ||
        (int64_t)(M + 255) * Nc > INT32_MAX)
        return qfq::fail(QFLASH_HIP_EINVAL, "operands beyond 2 GiB");
    if (workspace_elems < QFLASH_HIP_SCALES_WORKSPACE)
        return qfq::fail(QFLASH_HIP_EINVAL, "workspace holds %lld entries, %d needed", (long long)workspace_elems,
                         QFLASH_HIP_SCALES_WORKSPACE);
    const qfq::ProjArgs pa = {x8, w8, w_scale, bias, x_scale, M, K, Nc, Nc / 3, workspace, nullptr, codes};
    return qfq::qkv_int8(pa, scales, (hipStream_t)stream);
}

int qflash_hip_scales_noalloc(const void* q, const void* k, const void* v, int32_t dtype,
                              const int64_t* shapes_strides, void* scales, void* stream) {
    qfq::g_err[0] = 0;
    if (!q || !k || !v || !shapes_strides || !scales) return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    int dev = 0, sdev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return qfq::fail(QFLASH_HIP_ELAUNCH, "no current HIP device");
    if (dev < 0 || dev >= qfq::kMaxDevices) return qfq::fail(QFLASH_HIP_EINVAL, "device %d out of range", dev);
    // the static workspace of the stream's device is addressed from this one
    if (stream && hipStreamGetDevice((hipStream_t)stream, &sdev) == hipSuccess && sdev != dev)
        return qfq::fail(QFLASH_HIP_EINVAL, "stream belongs to device %d, current device is %d", sdev, dev);
    uint32_t* ws = qfq::scratch_ptr(dev);
    if (!ws) return QFLASH_HIP_ELAUNCH;
    // every call starts from zeroed slots (a fill kernel, not a memset: the
    // call may be captured into a graph), so a failed earlier call leaves
    // nothing behind
    hipLaunchKernelGGL(qfq::clear_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, ws,
                       (int)QFLASH_HIP_SCALES_WORKSPACE);
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return qfq::fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
    return qflash_hip_scales(q, k, v, dtype, shapes_strides, scales, ws, QFLASH_HIP_SCALES_WORKSPACE, stream);
}

int qflash_hip_quantize(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                        int8_t* q8, int8_t* k8, int8_t* v8, const int64_t* out_strides, const void* scales,
                        void* stream) {
    qfq::g_err[0] = 0;
    if (!q || !k || !v || !shapes_strides || !out_strides || !scales || !q8 || !k8 || !v8)
        return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    const int es = qfq::esize_of(dtype);
    if (!es) return qfq::fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    qfq::Geo g[3];
    const void* x[3] = {q, k, v};
    int8_t* y[3] = {q8, k8, v8};
    for (int i = 0; i < 3; ++i)
        if (int rc = qfq::make_geo(g[i], x[i], shapes_strides + 8 * i, shapes_strides + 8 * i + 4, y[i],
                                   out_strides + 4 * i, es, i))
            return rc;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case QFLASH_HIP_F32: return qfq::quant_dt<QFLASH_HIP_F32>(g, scales, st);
        case QFLASH_HIP_F16: return qfq::quant_dt<QFLASH_HIP_F16>(g, scales, st);
        default: return qfq::quant_dt<QFLASH_HIP_BF16>(g, scales, st);
    }
}

namespace qfq {
static int window_bias(const float* rel, const float* mask, int32_t n_win, int32_t H, int32_t N, double sm_scale,
                       const int32_t* params, int32_t* out, void* stream) {
    g_err[0] = 0;
    if (!rel || !out) return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (H <= 0 || N <= 0 || n_win <= 0 || (!mask && n_win != 1))
        return fail(QFLASH_HIP_EINVAL, "bad window bias shape nW=%d H=%d N=%d%s", n_win, H, N,
                    mask ? "" : " (no mask: nW must be 1)");
    if (!params && (!(sm_scale != 0.0) || !(fabs(sm_scale) < 1e30)))
        return fail(QFLASH_HIP_EINVAL, "bad sm_scale %g", sm_scale);
    const int64_t nn = (int64_t)N * N, total = (int64_t)n_win * H * nn;
    if (total >= ((int64_t)1 << 31)) return fail(QFLASH_HIP_EINVAL, "window bias too large");
    // torch: x * LOG2E and x / sm_scale with host scalars, both taken to fp32
    // (the division as a product with the fp32 reciprocal of the fp32 divisor)
    const float log2e = (float)1.44269504;
    const float inv_sm = params ? 0.0f : 1.0f / (float)sm_scale;
    hipLaunchKernelGGL(window_bias_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       rel, mask, H, (int32_t)nn, total, log2e, inv_sm, params, out);
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
        return fail(QFLASH_HIP_ELAUNCH, "window bias launch: %s", hipGetErrorString(err));
    return 0;
}

static int mask_bias(const float* mask, int64_t n, double sm_scale, const int32_t* params, int32_t* out,
                     void* stream) {
    g_err[0] = 0;
    if (!mask || !out) return fail(QFLASH_HIP_EINVAL, "null pointer argument");
    if (n <= 0 || n >= ((int64_t)1 << 31)) return fail(QFLASH_HIP_EINVAL, "bad mask size %lld", (long long)n);
    if (!params && (!(sm_scale != 0.0) || !(fabs(sm_scale) < 1e30)))
        return fail(QFLASH_HIP_EINVAL, "bad sm_scale %g", sm_scale);
    const float log2e = (float)1.44269504;
    const float inv_sm = params ? 0.0f : 1.0f / (float)sm_scale;
    const bool vec = (((uintptr_t)mask | (uintptr_t)out) & 15u) == 0;
    hipLaunchKernelGGL(mask_bias_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, (hipStream_t)stream, mask,
                       n, vec, log2e, inv_sm, params, out);
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
        return fail(QFLASH_HIP_ELAUNCH, "mask bias launch: %s", hipGetErrorString(err));
    return 0;
}
}  // namespace qfq

int qflash_hip_window_bias(const float* rel, const float* mask, int32_t n_win, int32_t H, int32_t N,
                           double sm_scale, int32_t* out, void* stream) {
    return qfq::window_bias(rel, mask, n_win, H, N, sm_scale, nullptr, out, stream);
}

int qflash_hip_window_bias_planned(const float* rel, const float* mask, int32_t n_win, int32_t H, int32_t N,
                                   const int32_t* params, int32_t* out, void* stream) {
    if (!params) return qfq::fail(QFLASH_HIP_EINVAL, "params is null");
    return qfq::window_bias(rel, mask, n_win, H, N, 0.0, params, out, stream);
}

int qflash_hip_mask_bias(const float* mask, int64_t n, double sm_scale, int32_t* out, void* stream) {
    return qfq::mask_bias(mask, n, sm_scale, nullptr, out, stream);
}

int qflash_hip_mask_bias_planned(const float* mask, int64_t n, const int32_t* params, int32_t* out, void* stream) {
    if (!params) return qfq::fail(QFLASH_HIP_EINVAL, "params is null");
    return qfq::mask_bias(mask, n, 0.0, params, out, stream);
}

}  // extern "C"
