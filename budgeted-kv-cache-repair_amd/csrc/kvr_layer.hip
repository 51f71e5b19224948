// Per-layer elementwise work of the packed refresh rows, one launch each:
//
//   kvr_rms_norm:  [s = residual + x]  y = weight * dtype(s * rsqrt(mean(s^2) + eps))
//   kvr_silu_mul:  out = dtype(dtype(silu(gate)) * up)
//
// They replace the eager op chains of the native decoder's RMSNorm
// (transformers 5.15.0 models/llama/modeling_llama.py:52-69; Qwen3's per-head
// q/k norm is the same module, models/qwen3/modeling_qwen3.py:50-64), the
// residual add in front of the post-attention norm
// (modeling_llama.py:316-320) and the MLP activation product
// (modeling_llama.py:174-175), which run ~8, 1 and 2 launches per use. Each
// step rounds where the eager ops round: the residual sum, the normalised value
// (`.to(input_dtype)`), the weight product, silu, and the gated product. The
// mean of squares is accumulated in fp32 in a different order than torch's
// reduction kernel, so an output can differ from the eager chain by one unit in
// the last place of the storage type.
#include "kvr_internal.h"

#include <math.h>

namespace kvr {
namespace {

constexpr int kNormThreads = 256;  // 4 waves, one row per wave

struct NormArgs {
    const char* x;
    const char* residual;  // nullptr: no residual add
    char* residual_out;    // s = residual + x (when residual != nullptr)
    char* out;
    const char* weight;
    int64_t rows;
    int64_t x_stride, r_stride, ro_stride, o_stride;  // row strides (elements); dims are unit-stride
    int32_t hidden;
    float eps;
    PartialSums px;        // px.base != nullptr: x comes from split-K partial sums (vector path only)
};

template <typename T>
__device__ inline float load(const char* base, int64_t i) {
    using E = elem<T>;
    return E::to_float(reinterpret_cast<const typename E::bits*>(base)[i]);
}

template <typename T>
__device__ inline void store(char* base, int64_t i, float v) {
    using E = elem<T>;
    reinterpret_cast<typename E::bits*>(base)[i] = E::from_float(v);
}

// Scalar path (any hidden size / alignment): one wave per row, lane l handles
// elements l, l + 64, ... in two passes (sum of squares, then the output).
template <typename T>
__global__ void __launch_bounds__(kNormThreads) rms_norm_kernel(NormArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kNormThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const char* x = a.x + row * a.x_stride * elem<T>::size;
    const char* res = a.residual ? a.residual + row * a.r_stride * elem<T>::size : nullptr;
    char* res_out = a.residual ? a.residual_out + row * a.ro_stride * elem<T>::size : nullptr;
    char* out = a.out + row * a.o_stride * elem<T>::size;

    float ss = 0.f;
    for (int i = lane; i < a.hidden; i += 64) {
        float v = load<T>(x, i);
        if (res) {
            v = round_through<T>(load<T>(res, i) + v);  // residual + hidden_states, rounded to dtype
            store<T>(res_out, i, v);
        }
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    // mean as sum * (1/N), then rsqrt(var + eps), as the eager mean and rsqrt kernels
    const float inv = rsqrtf(ss * (1.f / static_cast<float>(a.hidden)) + a.eps);
    for (int i = lane; i < a.hidden; i += 64) {
        const float v = res ? load<T>(res_out, i) : load<T>(x, i);
        const float y = round_through<T>(v * inv);  // .to(input_dtype)
        store<T>(out, i, load<T>(a.weight, i) * y);
    }
}

// Vector path: 16-byte vectors, TPR (power of two, <= 256) threads per row,
// each holding at most kMaxVec vectors of its row in registers, so the row is
// read once. Rows per block = 256 / TPR; a row wider than a wave reduces its
// partial sums through LDS.
constexpr int kMaxVec = 4;

template <typename T, int NV, int NT>
__global__ void __launch_bounds__(NT) rms_norm_vec_kernel(NormArgs a, int tpr_log2) {
#pragma clang fp contract(off)
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int V = 16 / E::size;  // elements per vector
    __shared__ float partial[NT / 64];
    const int tpr = 1 << tpr_log2;
    const int t = threadIdx.x & (tpr - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT >> tpr_log2) + (threadIdx.x >> tpr_log2);
    const bool live = row < a.rows;
    const int nvec = a.hidden / V;
    const char* x = a.x ? a.x + row * a.x_stride * E::size : nullptr;
    const char* res = a.residual ? a.residual + row * a.r_stride * E::size : nullptr;
    char* res_out = a.residual ? a.residual_out + row * a.ro_stride * E::size : nullptr;
    char* out = a.out + row * a.o_stride * E::size;

    // Every load of the row is issued before any of it is used (weight,
    // residual, x or the fp32 partials), so the block pays one memory round
    // trip; the residual sums are stored after the last load.
    u32x4 wv[NV], rv[NV], xv[NV];
    float xs[NV][V];
    const bool use_partials = V == 8 && a.px.base != nullptr;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int j = t + k * tpr;
        if (!live || j >= nvec) continue;
        wv[k] = *reinterpret_cast<const u32x4*>(a.weight + static_cast<int64_t>(j) * 16);
        if (res) rv[k] = *reinterpret_cast<const u32x4*>(res + static_cast<int64_t>(j) * 16);
        if (!use_partials) xv[k] = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(j) * 16);
    }
    if constexpr (V == 8) {
        if (use_partials) {  // the projection's output elements, rounded as its reduce kernel rounds them
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int j = t + k * tpr;
                if (live && j < nvec) partial_sum8(a.px, row, static_cast<int64_t>(j) * 8, xs[k]);
            }
        }
    }
    float v[NV][V];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int j = t + k * tpr;
        if (!live || j >= nvec) continue;
        bits xb[V];
        if (use_partials) {
#pragma unroll
            for (int e = 0; e < V; ++e) xb[e] = E::from_float(xs[k][e]);
        } else {
            __builtin_memcpy(xb, &xv[k], 16);
        }
        if (res) {
            bits rb[V], sb[V];
            __builtin_memcpy(rb, &rv[k], 16);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                sb[e] = E::from_float(E::to_float(rb[e]) + E::to_float(xb[e]));  // residual + hidden_states
                v[k][e] = E::to_float(sb[e]);
            }
            __builtin_memcpy(&rv[k], sb, 16);  // now the sum, stored below
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) v[k][e] = E::to_float(xb[e]);
        }
#pragma unroll
        for (int e = 0; e < V; ++e) ss += v[k][e] * v[k][e];
    }
    if (res) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int j = t + k * tpr;
            if (live && j < nvec) *reinterpret_cast<u32x4*>(res_out + static_cast<int64_t>(j) * 16) = rv[k];
        }
    }
    const int width = tpr < 64 ? tpr : 64;
    for (int off = width >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off, width);
    if (tpr > 64) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) partial[wave] = ss;
        __syncthreads();
        const int first = (threadIdx.x >> tpr_log2) << (tpr_log2 - 6);  // first wave of this row
        ss = 0.f;
        for (int w = 0; w < (tpr >> 6); ++w) ss += partial[first + w];
    }
    if (!live) return;
    const float inv = rsqrtf(ss * (1.f / static_cast<float>(a.hidden)) + a.eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int j = t + k * tpr;
        if (j >= nvec) continue;
        bits wb[V], ob[V];
        __builtin_memcpy(wb, &wv[k], 16);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const float y = round_through<T>(v[k][e] * inv);  // .to(input_dtype)
            ob[e] = E::from_float(E::to_float(wb[e]) * y);
        }
        u32x4 ov;
        __builtin_memcpy(&ov, ob, 16);
        *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(j) * 16) = ov;
    }
}

constexpr int kEltThreads = 256;

// One element per thread (any alignment) ...
template <typename T>
__global__ void __launch_bounds__(kEltThreads) silu_mul_kernel(const char* gate, const char* up, char* out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kEltThreads + threadIdx.x;
    if (i >= n) return;
    store<T>(out, i, silu_gate<T>(load<T>(gate, i), load<T>(up, i)));
}

// ... or one 16-byte vector per thread.
template <typename T>
__global__ void __launch_bounds__(kEltThreads) silu_mul_vec_kernel(const char* gate, const char* up, char* out,
                                                                   int64_t nvec) {
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int V = 16 / E::size;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kEltThreads + threadIdx.x;
    if (j >= nvec) return;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(gate + j * 16);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(up + j * 16);
    bits gb[V], ub[V], ob[V];
    __builtin_memcpy(gb, &gv, 16);
    __builtin_memcpy(ub, &uv, 16);
#pragma unroll
    for (int e = 0; e < V; ++e) ob[e] = E::from_float(silu_gate<T>(E::to_float(gb[e]), E::to_float(ub[e])));
    u32x4 ov;
    __builtin_memcpy(&ov, ob, 16);
    *reinterpret_cast<u32x4*>(out + j * 16) = ov;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
int launch_norm(const NormArgs& a, hipStream_t s, bool require_vec = false) {
    constexpr int V = 16 / elem<T>::size;
    const int64_t nvec = a.hidden / V;
    bool vec = a.hidden % V == 0 && a.x_stride % V == 0 && a.o_stride % V == 0 && aligned16(a.x) &&
               aligned16(a.out) && aligned16(a.weight) &&
               (!a.residual || (a.r_stride % V == 0 && a.ro_stride % V == 0 && aligned16(a.residual) &&
                                aligned16(a.residual_out)));
    // Rows of at least 512 vectors take a 512-thread block each (twice the
    // loads in flight per row); shorter rows share 256-thread blocks.
    const bool wide = nvec >= 512;
    const int nt = wide ? 512 : kNormThreads;
    int tpr_log2 = 0;
    while ((int64_t(1) << tpr_log2) < nvec && (1 << tpr_log2) < nt) ++tpr_log2;
    const int64_t per_thread = ceil_div(nvec, int64_t(1) << tpr_log2);
    vec = vec && per_thread <= kMaxVec && nvec > 0;
    if (vec) {
        const int64_t blocks = ceil_div(a.rows, nt >> tpr_log2);
        const unsigned g = static_cast<unsigned>(blocks);
        if (wide) {
            switch (per_thread) {
                case 1: rms_norm_vec_kernel<T, 1, 512><<<g, 512, 0, s>>>(a, tpr_log2); break;
                case 2: rms_norm_vec_kernel<T, 2, 512><<<g, 512, 0, s>>>(a, tpr_log2); break;
                case 3: rms_norm_vec_kernel<T, 3, 512><<<g, 512, 0, s>>>(a, tpr_log2); break;
                default: rms_norm_vec_kernel<T, 4, 512><<<g, 512, 0, s>>>(a, tpr_log2); break;
            }
        } else {
            switch (per_thread) {
                case 1: rms_norm_vec_kernel<T, 1, kNormThreads><<<g, kNormThreads, 0, s>>>(a, tpr_log2); break;
                case 2: rms_norm_vec_kernel<T, 2, kNormThreads><<<g, kNormThreads, 0, s>>>(a, tpr_log2); break;
                case 3: rms_norm_vec_kernel<T, 3, kNormThreads><<<g, kNormThreads, 0, s>>>(a, tpr_log2); break;
                default: rms_norm_vec_kernel<T, 4, kNormThreads><<<g, kNormThreads, 0, s>>>(a, tpr_log2); break;
            }
        }
        return launch_status();
    }
    if (require_vec) return KVR_E_UNSUPPORTED_SHAPE;
    const int64_t blocks = ceil_div(a.rows, kNormThreads / 64);
    rms_norm_kernel<T><<<static_cast<unsigned>(blocks), kNormThreads, 0, s>>>(a);
    return launch_status();
}

template <typename T>
int launch_silu(const void* g, const void* u, void* o, int64_t n, hipStream_t s) {
    constexpr int V = 16 / elem<T>::size;
    if (n % V == 0 && aligned16(g) && aligned16(u) && aligned16(o)) {
        const int64_t nvec = n / V;
        silu_mul_vec_kernel<T><<<static_cast<unsigned>(ceil_div(nvec, kEltThreads)), kEltThreads, 0, s>>>(
            static_cast<const char*>(g), static_cast<const char*>(u), static_cast<char*>(o), nvec);
    } else {
        silu_mul_kernel<T><<<static_cast<unsigned>(ceil_div(n, kEltThreads)), kEltThreads, 0, s>>>(
            static_cast<const char*>(g), static_cast<const char*>(u), static_cast<char*>(o), n);
    }
    return launch_status();
}

}  // namespace
}  // namespace kvr

extern "C" int kvr_rms_norm(const void* x, const void* residual, void* residual_out, void* out, const void* weight,
                            int64_t rows, int32_t hidden, const int64_t row_strides[4], float eps, int32_t dtype,
                            void* stream) {
    using namespace kvr;
    if (dtype_size(dtype) == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (rows < 0 || hidden <= 0 || !(eps >= 0.f) || eps == INFINITY) return KVR_E_INVALID_ARGUMENT;
    if (!row_strides) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 4; ++i)
        if (row_strides[i] < 0) return KVR_E_BAD_STRIDE;
    if (rows == 0) return KVR_OK;
    if (!x || !out || !weight || (residual && !residual_out)) return KVR_E_NULL_POINTER;
    if (rows > (int64_t(1) << 40)) return KVR_E_UNSUPPORTED_SHAPE;
    NormArgs a;
    a.x = static_cast<const char*>(x);
    a.residual = static_cast<const char*>(residual);
    a.residual_out = static_cast<char*>(residual_out);
    a.out = static_cast<char*>(out);
    a.weight = static_cast<const char*>(weight);
    a.rows = rows;
    a.x_stride = row_strides[0];
    a.r_stride = row_strides[1];
    a.ro_stride = row_strides[2];
    a.o_stride = row_strides[3];
    a.hidden = hidden;
    a.eps = eps;
    a.px = PartialSums{};
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KVR_DTYPE_F32: return launch_norm<f32_t>(a, s);
        case KVR_DTYPE_F16: return launch_norm<f16_t>(a, s);
        default: return launch_norm<bf16_t>(a, s);
    }
}

namespace kvr {

bool rms_norm_partials_ok(int32_t hidden, int32_t dtype) {
    return (dtype == KVR_DTYPE_BF16 || dtype == KVR_DTYPE_F16) && hidden > 0 && hidden % 8 == 0 &&
           hidden / 8 <= 256 * kMaxVec;
}

int rms_norm_partials(const PartialSums& x, const void* residual, void* residual_out, void* out, const void* weight,
                      int64_t rows, int32_t hidden, const int64_t row_strides[4], float eps, int32_t dtype,
                      void* stream) {
    if (!rms_norm_partials_ok(hidden, dtype)) return KVR_E_UNSUPPORTED_SHAPE;
    if (!x.base || x.splits < 1 || !out || !weight || (residual && !residual_out)) return KVR_E_NULL_POINTER;
    if (rows <= 0 || rows > kPartialTileRows) return KVR_E_UNSUPPORTED_SHAPE;
    NormArgs a;
    a.x = nullptr;
    a.residual = static_cast<const char*>(residual);
    a.residual_out = static_cast<char*>(residual_out);
    a.out = static_cast<char*>(out);
    a.weight = static_cast<const char*>(weight);
    a.rows = rows;
    a.x_stride = hidden;
    a.r_stride = row_strides[1];
    a.ro_stride = row_strides[2];
    a.o_stride = row_strides[3];
    a.hidden = hidden;
    a.eps = eps;
    a.px = x;
    hipStream_t s = as_stream(stream);
    return dtype == KVR_DTYPE_F16 ? launch_norm<f16_t>(a, s, true) : launch_norm<bf16_t>(a, s, true);
}

}  // namespace kvr

extern "C" int kvr_silu_mul(const void* gate, const void* up, void* out, int64_t n, int32_t dtype, void* stream) {
    using namespace kvr;
    if (dtype_size(dtype) == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n < 0) return KVR_E_INVALID_ARGUMENT;
    if (n == 0) return KVR_OK;
    if (!gate || !up || !out) return KVR_E_NULL_POINTER;
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KVR_DTYPE_F32: return launch_silu<f32_t>(gate, up, out, n, s);
        case KVR_DTYPE_F16: return launch_silu<f16_t>(gate, up, out, n, s);
        default: return launch_silu<bf16_t>(gate, up, out, n, s);
    }
}
