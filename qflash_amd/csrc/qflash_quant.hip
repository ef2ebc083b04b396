// Per-tensor absmax scales and int8 quantisation of Q, K, V on the device.
//
// Replaces the host sequence of qflash_forward (qflash/kernel.py:294-296 and
// :309-311), which torch runs as ~12 elementwise / reduction passes over the
// floating-point inputs:
//     x_scale = x.abs().amax() / 127                  (in the input dtype T)
//     qk      = q_scale * k_scale                     (in T; .item() on the host)
//     x_i8    = clamp(round(x / x_scale), -128, 127).to(int8)
// Here: one pass reads each input once for the absmax (qflash_hip_scales), a
// one-block pass forms the scales in T, and one pass reads each input again
// and writes the int8 codes (qflash_hip_quantize).  The arithmetic follows
// torch's for T: fp32 natively; fp16 / bf16 as fp32 opmath rounded back to T
// after every operation (x / s, the product of the scales), round half to
// even, clamp, conversion.
//
// Tensors are 4-D (Z, H, N, D) with element strides; the innermost dimension
// must have unit stride (the module path's token-major views have it).  Rows
// of D elements are read with 16-byte loads when the row bytes and the base
// are 16-byte aligned, element by element otherwise.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <math.h>
#include <stdint.h>

#include "../../include/qflash_hip.h"
#include "qf_error.h"

namespace qfq {

using qferr::fail;
using qferr::g_err;

struct Tensor4 {
    const void* p;
    int64_t n[4];  // sizes Z, H, N, D
    int64_t s[4];  // element strides
};

struct Out4 {
    int8_t* p;
    int64_t s[4];
};

constexpr int kThreads = 256;

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

// One (z, h) head slice of rows per block row: blockIdx.x = (z*H + h) * RB + rb,
// blockIdx.y = tensor.  Each block writes the pattern maximum of its rows.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void absmax_kernel(Tensor4 t0, Tensor4 t1, Tensor4 t2, int rb_per_head,
                                                          uint32_t* partial) {
    const Tensor4 t = blockIdx.y == 0 ? t0 : (blockIdx.y == 1 ? t1 : t2);
    const int64_t zh = blockIdx.x / rb_per_head;
    const int rb = blockIdx.x % rb_per_head;
    const int64_t z = zh / t.n[1], h = zh % t.n[1];
    const int64_t N = t.n[2], D = t.n[3];
    const int64_t rows_per_block = (N + rb_per_head - 1) / rb_per_head;
    const int64_t n0 = rb * rows_per_block, n1 = min(N, n0 + rows_per_block);
    uint32_t m = 0;
    if (z < t.n[0]) {
        const int64_t base = z * t.s[0] + h * t.s[1];
        if constexpr (VEC) {
            constexpr int EPC = 16 / esize<DT>();  // elements per 16-byte chunk
            const int64_t cpr = D / EPC;           // chunks per row
            for (int64_t c = threadIdx.x; c < (n1 - n0) * cpr; c += kThreads) {
                const int64_t n = n0 + c / cpr, col = (c % cpr) * EPC;
                const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(t.p) +
                                                               (base + n * t.s[2] + col) * esize<DT>());
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (DT == QFLASH_HIP_F32) {
                        m = max(m, abs_bits<DT>(w[e]));
                    } else {
                        m = max(m, abs_bits<DT>(w[e] & 0xffffu));
                        m = max(m, abs_bits<DT>(w[e] >> 16));
                    }
                }
            }
        } else {
            for (int64_t c = threadIdx.x; c < (n1 - n0) * D; c += kThreads) {
                const int64_t n = n0 + c / D, d = c % D;
                m = max(m, abs_bits<DT>(load_raw<DT>(t.p, base + n * t.s[2] + d * t.s[3])));
            }
        }
    }
    __shared__ uint32_t red[kThreads / 64];
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) m = max(m, red[w]);
        partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = m;
    }
}

// fp32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
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
    else return __uint_as_float(bf16_bits(f) << 16);
}
template <int DT>
__device__ __forceinline__ void store_t(void* p, int i, float f) {
    if constexpr (DT == QFLASH_HIP_F32) reinterpret_cast<float*>(p)[i] = f;
    else if constexpr (DT == QFLASH_HIP_F16) reinterpret_cast<__half*>(p)[i] = __float2half_rn(f);
    else reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)bf16_bits(f);
}

// scales[0..2] = amax / 127 (q, k, v), scales[3] = scales[0] * scales[1], all in T.
// torch divides a GPU tensor by a host scalar as a product with the scalar's
// reciprocal in the opmath type (fp32): amax * RN(1/127).
template <int DT>
__global__ __launch_bounds__(kThreads) void scales_kernel(const uint32_t* partial, int nblk, void* scales) {
    __shared__ uint32_t red[3][kThreads / 64];
    uint32_t m[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        uint32_t v = 0;
        for (int b = threadIdx.x; b < nblk; b += kThreads) v = max(v, partial[(int64_t)t * nblk + b]);
        v = wave_max(v);
        if ((threadIdx.x & 63) == 0) red[t][threadIdx.x >> 6] = v;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        m[t] = red[t][0];
        for (int w = 1; w < kThreads / 64; ++w) m[t] = max(m[t], red[t][w]);
    }
    float s[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        s[t] = round_t<DT>(to_float<DT>(m[t]) * (1.0f / 127.0f));  // kernel.py:294-296
        store_t<DT>(scales, t, s[t]);
    }
    store_t<DT>(scales, 3, round_t<DT>(s[0] * s[1]));  // (q_scale * k_scale), kernel.py:297
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

template <int DT>
__device__ __forceinline__ float load_t(const void* p, int64_t i) {
    return to_float<DT>(load_raw<DT>(p, i));
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void quant_kernel(Tensor4 t0, Tensor4 t1, Tensor4 t2, Out4 o0, Out4 o1,
                                                         Out4 o2, const void* scales, int rb_per_head) {
    const Tensor4 t = blockIdx.y == 0 ? t0 : (blockIdx.y == 1 ? t1 : t2);
    const Out4 o = blockIdx.y == 0 ? o0 : (blockIdx.y == 1 ? o1 : o2);
    const float s = load_t<DT>(scales, blockIdx.y);
    const int64_t zh = blockIdx.x / rb_per_head;
    const int rb = blockIdx.x % rb_per_head;
    const int64_t z = zh / t.n[1], h = zh % t.n[1];
    if (z >= t.n[0]) return;
    const int64_t N = t.n[2], D = t.n[3];
    const int64_t rows_per_block = (N + rb_per_head - 1) / rb_per_head;
    const int64_t n0 = rb * rows_per_block, n1 = min(N, n0 + rows_per_block);
    const int64_t base = z * t.s[0] + h * t.s[1], obase = z * o.s[0] + h * o.s[1];
    if constexpr (VEC) {
        constexpr int EPC = 16 / esize<DT>();
        const int64_t cpr = D / EPC;
        for (int64_t c = threadIdx.x; c < (n1 - n0) * cpr; c += kThreads) {
            const int64_t n = n0 + c / cpr, col = (c % cpr) * EPC;
            const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(t.p) +
                                                           (base + n * t.s[2] + col) * esize<DT>());
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
            int8_t* dst = o.p + obase + n * o.s[2] + col;
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
    } else {
        for (int64_t c = threadIdx.x; c < (n1 - n0) * D; c += kThreads) {
            const int64_t n = n0 + c / D, d = c % D;
            o.p[obase + n * o.s[2] + d * o.s[3]] = quant1<DT>(load_t<DT>(t.p, base + n * t.s[2] + d * t.s[3]), s);
        }
    }
}

static bool aligned(const void* p, int a) { return ((uintptr_t)p % a) == 0; }

// 16-byte row chunks: unit column stride, rows and base 16-byte aligned, D a
// multiple of the chunk.
static bool vec_ok(const Tensor4& t, int es) {
    if (t.s[3] != 1 || (t.n[3] * es) % 16 || !aligned(t.p, 16)) return false;
    for (int i = 0; i < 3; ++i)
        if ((t.s[i] * es) % 16) return false;
    return true;
}

static int read_tensors(Tensor4* t, const void* const* x, const int64_t* ss) {
    for (int i = 0; i < 3; ++i) {
        if (!x[i]) return fail(QFLASH_HIP_EINVAL, "null tensor pointer");
        t[i].p = x[i];
        for (int j = 0; j < 4; ++j) {
            t[i].n[j] = ss[8 * i + j];
            t[i].s[j] = ss[8 * i + 4 + j];
            if (t[i].n[j] <= 0) return fail(QFLASH_HIP_EINVAL, "tensor %d has an empty dimension", i);
        }
    }
    return 0;
}

// Row blocks per (z, h) head: enough blocks to fill the chip, each a few rows.
static int rows_blocks(const Tensor4* t) {
    int64_t zh = 0;
    for (int i = 0; i < 3; ++i) zh = zh > t[i].n[0] * t[i].n[1] ? zh : t[i].n[0] * t[i].n[1];
    int64_t N = 0;
    for (int i = 0; i < 3; ++i) N = N > t[i].n[2] ? N : t[i].n[2];
    int rb = (int)((4096 + zh - 1) / zh);
    if (rb > N) rb = (int)N;
    return rb < 1 ? 1 : rb;
}

template <int DT>
static int scales_dt(const Tensor4* t, void* scales, uint32_t* ws, int64_t ws_elems, hipStream_t st) {
    const int rb = rows_blocks(t);
    int64_t zh = 0;
    for (int i = 0; i < 3; ++i) zh = zh > t[i].n[0] * t[i].n[1] ? zh : t[i].n[0] * t[i].n[1];
    const int64_t nblk = zh * rb;
    if (nblk > INT32_MAX / 4) return fail(QFLASH_HIP_EINVAL, "too many rows");
    if (ws_elems < 3 * nblk)
        return fail(QFLASH_HIP_EINVAL, "workspace holds %lld entries, %lld needed", (long long)ws_elems,
                    (long long)(3 * nblk));
    const bool vec = vec_ok(t[0], esize<DT>()) && vec_ok(t[1], esize<DT>()) && vec_ok(t[2], esize<DT>());
    const dim3 grid((unsigned)nblk, 3);
    if (vec)
        hipLaunchKernelGGL((absmax_kernel<DT, true>), grid, dim3(kThreads), 0, st, t[0], t[1], t[2], rb, ws);
    else
        hipLaunchKernelGGL((absmax_kernel<DT, false>), grid, dim3(kThreads), 0, st, t[0], t[1], t[2], rb, ws);
    hipLaunchKernelGGL((scales_kernel<DT>), dim3(1), dim3(kThreads), 0, st, ws, (int)nblk, scales);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

template <int DT>
static int quant_dt(const Tensor4* t, const Out4* o, const void* scales, hipStream_t st) {
    const int rb = rows_blocks(t);
    int64_t zh = 0;
    for (int i = 0; i < 3; ++i) zh = zh > t[i].n[0] * t[i].n[1] ? zh : t[i].n[0] * t[i].n[1];
    bool vec = true;
    for (int i = 0; i < 3; ++i) {
        vec = vec && vec_ok(t[i], esize<DT>()) && o[i].s[3] == 1 && aligned(o[i].p, 8);
        for (int j = 0; j < 3; ++j) vec = vec && (o[i].s[j] % 8 == 0);
    }
    const dim3 grid((unsigned)(zh * rb), 3);
    if (vec)
        hipLaunchKernelGGL((quant_kernel<DT, true>), grid, dim3(kThreads), 0, st, t[0], t[1], t[2], o[0], o[1], o[2],
                           scales, rb);
    else
        hipLaunchKernelGGL((quant_kernel<DT, false>), grid, dim3(kThreads), 0, st, t[0], t[1], t[2], o[0], o[1],
                           o[2], scales, rb);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(QFLASH_HIP_ELAUNCH, "launch failed: %s", hipGetErrorString(e));
}

}  // namespace qfq

extern "C" {

int64_t qflash_hip_scales_workspace(const int64_t* shapes_strides) {
    if (!shapes_strides) return -1;
    qfq::Tensor4 t[3];
    const void* dummy[3] = {(const void*)16, (const void*)16, (const void*)16};
    if (qfq::read_tensors(t, dummy, shapes_strides)) return -1;
    int64_t zh = 0;
    for (int i = 0; i < 3; ++i) zh = zh > t[i].n[0] * t[i].n[1] ? zh : t[i].n[0] * t[i].n[1];
    return 3 * zh * qfq::rows_blocks(t);
}

int qflash_hip_scales(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                      void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream) {
    qfq::g_err[0] = 0;
    if (!shapes_strides || !scales || !workspace) return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qfq::Tensor4 t[3];
    const void* x[3] = {q, k, v};
    if (int rc = qfq::read_tensors(t, x, shapes_strides)) return rc;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case QFLASH_HIP_F32: return qfq::scales_dt<QFLASH_HIP_F32>(t, scales, workspace, workspace_elems, st);
        case QFLASH_HIP_F16: return qfq::scales_dt<QFLASH_HIP_F16>(t, scales, workspace, workspace_elems, st);
        case QFLASH_HIP_BF16: return qfq::scales_dt<QFLASH_HIP_BF16>(t, scales, workspace, workspace_elems, st);
        default: return qfq::fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    }
}

int qflash_hip_quantize(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                        int8_t* q8, int8_t* k8, int8_t* v8, const int64_t* out_strides, const void* scales,
                        void* stream) {
    qfq::g_err[0] = 0;
    if (!shapes_strides || !out_strides || !scales || !q8 || !k8 || !v8)
        return qfq::fail(QFLASH_HIP_EINVAL, "null pointer argument");
    qfq::Tensor4 t[3];
    const void* x[3] = {q, k, v};
    if (int rc = qfq::read_tensors(t, x, shapes_strides)) return rc;
    qfq::Out4 o[3];
    int8_t* y[3] = {q8, k8, v8};
    for (int i = 0; i < 3; ++i) {
        o[i].p = y[i];
        for (int j = 0; j < 4; ++j) o[i].s[j] = out_strides[4 * i + j];
    }
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case QFLASH_HIP_F32: return qfq::quant_dt<QFLASH_HIP_F32>(t, o, scales, st);
        case QFLASH_HIP_F16: return qfq::quant_dt<QFLASH_HIP_F16>(t, o, scales, st);
        case QFLASH_HIP_BF16: return qfq::quant_dt<QFLASH_HIP_BF16>(t, o, scales, st);
        default: return qfq::fail(QFLASH_HIP_EINVAL, "unknown dtype code %d", dtype);
    }
}

}  // extern "C"
