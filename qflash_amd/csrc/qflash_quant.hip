// Per-tensor absmax scales and int8 quantisation of Q, K, V on the device.
//
// Replaces the host sequence of qflash_forward (qflash/kernel.py:294-296 and
// :309-311), which torch runs as ~12 elementwise / reduction passes over the
// floating-point inputs:
//     x_scale = x.abs().amax() / 127                  (in the input dtype T)
//     qk      = q_scale * k_scale                     (in T; .item() on the host)
//     x_i8    = clamp(round(x / x_scale), -128, 127).to(int8)
// Here: one pass reads each input once for the absmax (qflash_hip_scales), a
// one-thread pass forms the scales in T, and one pass reads each input again
// and writes the int8 codes (qflash_hip_quantize).  The arithmetic is torch's
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

#include "../../include/qflash_hip.h"
#include "qf_common.h"

namespace qfq {

using qferr::fail;
using qferr::g_err;

constexpr int kThreads = 256;
constexpr int kSeg = 8 * kThreads;  // 16-byte chunks per work unit
constexpr int kSlots = 64;          // atomic-max slots per tensor (spreads the contention)

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

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
    return v;
}

// T value of a pattern and fp32 -> T rounding (round to nearest even).
template <int DT>
__device__ __forceinline__ float to_float(uint32_t bits) {
    if constexpr (DT == QFLASH_HIP_F32) return __uint_as_float(bits);
    else if constexpr (DT == QFLASH_HIP_F16) return __half2float(__ushort_as_half((unsigned short)bits));
    else return __uint_as_float(bits << 16);
}
template <int DT>
__device__ __forceinline__ float round_t(float f) {
    if constexpr (DT == QFLASH_HIP_F32) return f;
    else if constexpr (DT == QFLASH_HIP_F16) return __half2float(__float2half_rn(f));
    else return __uint_as_float(qf_bf16_bits(f) << 16);
}
template <int DT>
__device__ __forceinline__ void store_t(void* p, int i, float f) {
    if constexpr (DT == QFLASH_HIP_F32) reinterpret_cast<float*>(p)[i] = f;
    else if constexpr (DT == QFLASH_HIP_F16) reinterpret_cast<__half*>(p)[i] = __float2half_rn(f);
    else reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)qf_bf16_bits(f);
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
// (atomic max; ws starts at 0).
// MODE 1: int8 codes with scale scales[tensor].
template <int DT, int MODE>
__global__ __launch_bounds__(kThreads) void stream_kernel(GeoSet gs, uint32_t* ws, const void* scales) {
    const Geo& g = gs.g[blockIdx.y];
    float s = 0.f;
    if constexpr (MODE == 1) s = load_t<DT>(scales, blockIdx.y);
    uint32_t m = 0;
    if (g.vec) {
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

// scales[0..2] = amax / 127 (q, k, v), scales[3] = scales[0] * scales[1], all in T.
// torch divides a GPU tensor by a host scalar as a product with the scalar's
// reciprocal in the opmath type (fp32): amax * RN(1/127).
template <int DT>
__global__ __launch_bounds__(64) void scales_kernel(const uint32_t* ws, void* scales) {
    uint32_t m[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) m[t] = wave_max(ws[t * kSlots + threadIdx.x]);
    if (threadIdx.x != 0) return;
    float s[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        s[t] = round_t<DT>(to_float<DT>(m[t]) * (1.0f / 127.0f));  // kernel.py:294-296
        store_t<DT>(scales, t, s[t]);
    }
    store_t<DT>(scales, 3, round_t<DT>(s[0] * s[1]));  // (q_scale * k_scale), kernel.py:297
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
    return 0;
}

static unsigned grid_x(const Geo* g, int es) {
    int64_t units = 1;
    for (int i = 0; i < 3; ++i) {
        const int64_t u = g[i].vec ? g[i].rows * ((g[i].L * es / 16 + kSeg - 1) / kSeg)
                                   : (g[i].n4[0] * g[i].n4[1] * g[i].n4[2] * g[i].n4[3] + kThreads - 1) / kThreads;
        units = units > u ? units : u;
    }
    return (unsigned)(units < 2048 ? units : 2048);
}

template <int DT>
static int scales_dt(Geo* g, void* scales, uint32_t* ws, hipStream_t st) {
    const dim3 grid(grid_x(g, esize<DT>()), 3);
    const GeoSet gs = {{g[0], g[1], g[2]}};
    hipLaunchKernelGGL((stream_kernel<DT, 0>), grid, dim3(kThreads), 0, st, gs, ws, nullptr);
    hipLaunchKernelGGL((scales_kernel<DT>), dim3(1), dim3(64), 0, st, ws, scales);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

template <int DT>
static int quant_dt(Geo* g, const void* scales, hipStream_t st) {
    const dim3 grid(grid_x(g, esize<DT>()), 3);
    const GeoSet gs = {{g[0], g[1], g[2]}};
    hipLaunchKernelGGL((stream_kernel<DT, 1>), grid, dim3(kThreads), 0, st, gs, nullptr, scales);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

static int esize_of(int32_t dtype) {
    return dtype == QFLASH_HIP_F32 ? 4 : (dtype == QFLASH_HIP_F16 || dtype == QFLASH_HIP_BF16 ? 2 : 0);
}

}  // namespace qfq

extern "C" {

int qflash_hip_scales(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                      void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream) {
    qfq::g_err[0] = 0;
    if (!q || !k || !v || !shapes_strides || !scales || !workspace)
        return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    const int es = qfq::esize_of(dtype);
    if (!es) return qfq::fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    if (workspace_elems < 3 * qfq::kSlots)
        return qfq::fail(QFLASH_HIP_EINVAL, "workspace holds %lld entries, %d needed", (long long)workspace_elems,
                         3 * qfq::kSlots);
    qfq::Geo g[3];
    const void* x[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (int rc = qfq::make_geo(g[i], x[i], shapes_strides + 8 * i, shapes_strides + 8 * i + 4, nullptr,
                                   nullptr, es, i))
            return rc;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case QFLASH_HIP_F32: return qfq::scales_dt<QFLASH_HIP_F32>(g, scales, workspace, st);
        case QFLASH_HIP_F16: return qfq::scales_dt<QFLASH_HIP_F16>(g, scales, workspace, st);
        default: return qfq::scales_dt<QFLASH_HIP_BF16>(g, scales, workspace, st);
    }
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

}  // extern "C"
