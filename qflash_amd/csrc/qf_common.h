// Shared by the translation units of libqflash_hip.so: the per-thread error
// message returned by qflash_hip_last_error, the fp32 -> bf16 rounding, and
// the formation of the per-tensor scales from the absmax pass's slots.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/qflash_hip.h"

namespace qferr {
inline thread_local char g_err[512];

__attribute__((format(printf, 2, 3))) inline int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace qferr

// fp32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t qf_bf16_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

namespace qfs {
// Workgroup id b of a grid of n -> logical id, so that consecutive logical ids
// run on the same XCD (the hardware deals workgroups to the 8 XCDs round
// robin: b runs on XCD b % 8, which gets one contiguous range of ids).
__device__ __forceinline__ int xcd_order(int b, int n) {
    const int per = n >> 3, rem = n & 7, x = b & 7, i = b >> 3;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

constexpr int kScaleSlots = 64;  // absmax slots per tensor in the scales workspace
static_assert(3 * kScaleSlots <= QFLASH_HIP_SCALES_WORKSPACE, "workspace: 3 x kScaleSlots partial maxima");

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

// One wave: the q, k, v scales from the three tensors' absmax slots (lane i
// reads slot i of each and sets it back to zero for the next call), in T:
// torch divides a GPU tensor by a host scalar as a product with the scalar's
// reciprocal in the opmath type (fp32): amax * RN(1/127); scales[3] =
// scales[0] * scales[1].  Returns scales[3] as a float on every lane.
template <int DT>
__device__ float reduce_scale_slots(uint32_t* ws, void* scales) {
    float s[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const uint32_t m = wave_max(ws[t * kScaleSlots + threadIdx.x]);
        ws[t * kScaleSlots + threadIdx.x] = 0;
        s[t] = round_t<DT>(to_float<DT>(m) * (1.0f / 127.0f));  // kernel.py:294-296
    }
    const float qk = round_t<DT>(s[0] * s[1]);  // (q_scale * k_scale), kernel.py:297
    if (threadIdx.x == 0) {
#pragma unroll
        for (int t = 0; t < 3; ++t) store_t<DT>(scales, t, s[t]);
        store_t<DT>(scales, 3, qk);
    }
    return qk;
}
}  // namespace qfs

namespace qfq {
// The absmax pass of qflash_hip_scales (slots of `workspace`), followed by its
// scales kernel unless `scales` is null.
int absmax_pass(const void* q, const void* k, const void* v, int32_t dtype, const int64_t* shapes_strides,
                void* scales, uint32_t* workspace, int64_t workspace_elems, void* stream);
}  // namespace qfq
