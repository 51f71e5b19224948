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
    // that PyTorch's bfloat16 tensor ops apply to their fp32 results. The
    // conversion is gfx950's v_cvt_pk_bf16_f32 (round to nearest even,
    // denormals kept: the same bits as adding 0x7FFF plus the kept lsb and
    // truncating, for every non-NaN fp32 value); NaN is replaced after it.
    __device__ static inline bits from_float(float f) {
        const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
        return f != f ? static_cast<uint16_t>(0x7fc0u) : b;
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

// Split-K partial tiles left by linear_multi(..., reduce = false): fp32
// [ceil(cols / 64)][splits][64 rows][64 cols]; element (row, col) of the
// projection is the sum over s of tile(col / 64)[s][row][col % 64], added in
// split order and rounded to the dtype -- exactly what the reduce kernel writes.
struct PartialSums {
    const float* base = nullptr;  // nullptr: read the dtype tensor instead
    int32_t splits = 0;
};
constexpr int kPartialTileCols = 64;
constexpr int kPartialTileRows = 64;

int linear_multi(const void* x, int32_t n_weights, const void* const* w, const int32_t* rows, const int64_t* ldw,
                 void* y, int32_t m, int32_t k, int64_t ldx, int64_t ldy, int32_t epilogue, const void* residual,
                 int64_t ldr, void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream, bool reduce,
                 int32_t* splits_out);

// Eight consecutive columns [col, col + 8) of `row` (col % 8 == 0) summed over
// the splits in order, as fp32 (not yet rounded). The loads of up to
// kPartialBatch splits are issued before the adds, so a few splits cost one
// memory round trip, not one per split.
constexpr int kPartialBatch = 8;

__device__ inline void partial_sum8(const PartialSums& p, int64_t row, int64_t col, float out[8]) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const int64_t tile = col / kPartialTileCols;
    const float* at = p.base + (tile * p.splits * kPartialTileRows + row) * kPartialTileCols + col % kPartialTileCols;
    const int64_t step = static_cast<int64_t>(kPartialTileRows) * kPartialTileCols;
    f32x4_t lo = *reinterpret_cast<const f32x4_t*>(at);
    f32x4_t hi = *reinterpret_cast<const f32x4_t*>(at + 4);
    for (int s0 = 1; s0 < p.splits; s0 += kPartialBatch) {
        f32x4_t l[kPartialBatch], h[kPartialBatch];
#pragma unroll
        for (int b = 0; b < kPartialBatch; ++b) {
            if (s0 + b < p.splits) {
                l[b] = *reinterpret_cast<const f32x4_t*>(at + (s0 + b) * step);
                h[b] = *reinterpret_cast<const f32x4_t*>(at + (s0 + b) * step + 4);
            }
        }
#pragma unroll
        for (int b = 0; b < kPartialBatch; ++b) {
            if (s0 + b < p.splits) {
                lo += l[b];
                hi += h[b];
            }
        }
    }
    for (int e = 0; e < 4; ++e) {
        out[e] = lo[e];
        out[4 + e] = hi[e];
    }
}

// One column of `row` summed over the splits in order (fp32, not yet rounded).
__device__ inline float partial_sum1(const PartialSums& p, int64_t row, int64_t col) {
    const int64_t tile = col / kPartialTileCols;
    const float* at = p.base + (tile * p.splits * kPartialTileRows + row) * kPartialTileCols + col % kPartialTileCols;
    const int64_t step = static_cast<int64_t>(kPartialTileRows) * kPartialTileCols;
    float sum = at[0];
    for (int s0 = 1; s0 < p.splits; s0 += kPartialBatch) {
        float v[kPartialBatch];
#pragma unroll
        for (int b = 0; b < kPartialBatch; ++b)
            if (s0 + b < p.splits) v[b] = at[(s0 + b) * step];
#pragma unroll
        for (int b = 0; b < kPartialBatch; ++b)
            if (s0 + b < p.splits) sum += v[b];
    }
    return sum;
}

// kvr_rms_norm with x given as split-K partial sums (rounded to the dtype as the
// reduce kernel rounds them). Only the vector path; rms_norm_partials_ok says
// whether it applies to `hidden` columns of `dtype`.
bool rms_norm_partials_ok(int32_t hidden, int32_t dtype);
int rms_norm_partials(const PartialSums& x, const void* residual, void* residual_out, void* out, const void* weight,
                      int64_t rows, int32_t hidden, const int64_t row_strides[4], float eps, int32_t dtype,
                      void* stream);

// kvr_rope_scatter_kv_norm with q, fresh K and fresh V given as split-K partial
// sums of one concatenated projection (columns part_col[0] + h*head_dim + i for
// query head h, part_col[1] + ... for K, part_col[2] + ... for V). The q /
// fresh-K / fresh-V strides of `strides` are ignored; q_norm / k_norm null: no
// per-head norm.
int rope_scatter_partials(const PartialSums& src, const int64_t part_col[3], void* q_out, void* out_k, void* out_v,
                          const void* cos, const void* sin, const int64_t* positions, int64_t n_sel,
                          int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys, int32_t head_dim,
                          const int64_t strides[18], const int64_t cs_strides[4], int32_t dtype, void* stream,
                          const void* q_norm, const void* k_norm, float eps_q, float eps_k);

// Whether Qwen3's per-head q/k norms can be folded into the fresh-row epilogue
// (kvr_rope_scatter_kv_norm / rope_scatter_partials) for this head dim, dtype,
// norm weights and rotary tables: the fold runs on the epilogue's vector
// kernel only (not fp16; each half row a power-of-two count of 16-byte chunks,
// 16-byte aligned weights and table rows). Given q/k/v rows with unit dim
// stride and 16-byte aligned rows, the epilogue then accepts the norms;
// otherwise callers run kvr_rms_norm on the q and k rows first.
bool rope_norm_fold_ok(int32_t head_dim, int32_t dtype, const void* q_norm, const void* k_norm,
                       const int64_t cs_strides[4], const void* cos, const void* sin);

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
