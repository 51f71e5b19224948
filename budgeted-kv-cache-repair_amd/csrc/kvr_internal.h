// Internal helpers shared by the kvrepair HIP translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvrepair.h"

namespace kvr {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Storage element types. Kernels move raw bits (uint16_t / uint32_t) and do
// arithmetic in fp32, so every conversion below is explicit.
// ---------------------------------------------------------------------------
struct f32_t {};
struct f16_t {};
struct bf16_t {};

template <typename T> struct elem;
template <> struct elem<f32_t> {
    using bits = uint32_t;
    static constexpr int size = 4;
    __device__ static inline float to_float(bits b) { return __uint_as_float(b); }
    __device__ static inline bits from_float(float f) { return __float_as_uint(f); }
};
template <> struct elem<f16_t> {
    using bits = uint16_t;
    static constexpr int size = 2;
    __device__ static inline float to_float(bits b) {
        _Float16 h = __builtin_bit_cast(_Float16, b);
        return static_cast<float>(h);
    }
    // Round-to-nearest-even conversion (v_cvt_f16_f32 honours the default RNE mode).
    __device__ static inline bits from_float(float f) {
        _Float16 h = static_cast<_Float16>(f);
        return __builtin_bit_cast(uint16_t, h);
    }
};
template <> struct elem<bf16_t> {
    using bits = uint16_t;
    static constexpr int size = 2;
    __device__ static inline float to_float(bits b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
    // Round-to-nearest-even with a canonical quiet NaN (0x7FC0): the rounding
    // that PyTorch's bfloat16 tensor ops apply to their fp32 results.
    __device__ static inline bits from_float(float f) {
        uint32_t u = __float_as_uint(f);
        if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>(0x7fc0u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return static_cast<uint16_t>(u >> 16);
    }
};

// Round an fp32 value through the storage type and back (models one eager op).
template <typename T>
__device__ inline float round_through(float x) {
    return elem<T>::to_float(elem<T>::from_float(x));
}

// SiLU-gated product of one element, as the eager chain computes it:
// dtype(silu(g)) * u in fp32 (the caller rounds the product to dtype).
template <typename T>
__device__ inline float silu_gate(float g, float u) {
#pragma clang fp contract(off)
    const float act = round_through<T>(g / (1.f + expf(-g)));  // silu, rounded to dtype
    return act * u;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_size(int32_t dtype) {
    switch (dtype) {
        case KVR_DTYPE_F32: return 4;
        case KVR_DTYPE_F16: return 2;
        case KVR_DTYPE_BF16: return 2;
        default: return 0;
    }
}

// Launch status: a failed launch is reported, never retried.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? KVR_OK : KVR_E_LAUNCH_FAILED;
}

}  // namespace kvr
