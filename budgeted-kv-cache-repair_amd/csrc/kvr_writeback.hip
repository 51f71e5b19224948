// Interval writeback of the interval executors: rows [in_start, in_start + W)
// of two source K/V tensors overwrite rows [out_start, out_start + W) of two
// output tensors, every tensor [batch, heads, tokens, head_dim] with its own
// positive strides. A pure bit copy (NaN payloads, -0 and subnormals kept),
// K and V in one launch, each output element written by one thread.
//
// Reference semantics: src/kv_cache_repair/kernels/writeback.py:18-60 and
// _writeback_triton.py:7-59 (copy_kv_interval_ with absolute source rows;
// scatter_fresh_kv with fresh rows [0, W)).
#include "kvr_internal.h"

namespace kvr {
namespace {

constexpr int kThreads = 256;

struct CopyArgs {
    char* out[2];
    const char* in[2];
    int64_t os[2][4];  // {batch, head, token, dim} element strides of out K/V
    int64_t is[2][4];  // ... of in K/V
    int64_t out_start, in_start;
    int64_t width;
    int32_t heads, head_dim;
    int64_t per_tensor;  // units (vectors or elements) per tensor
};

// Unit u of one tensor -> (b, h, p, c) with c the vector or element index in the row.
__device__ inline void decode(const CopyArgs& a, int64_t u, int64_t units_per_row, int64_t& b, int64_t& h,
                              int64_t& p, int64_t& c) {
    c = u % units_per_row;
    u /= units_per_row;
    p = u % a.width;
    u /= a.width;
    h = u % a.heads;
    b = u / a.heads;
}

// Vector path: unit dim strides, rows and bases 16-byte aligned.
template <int ESIZE>
__global__ void __launch_bounds__(kThreads) copy_interval_vec_kernel(CopyArgs a) {
    constexpr int V = 16 / ESIZE;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= 2 * a.per_tensor) return;
    const int t = g >= a.per_tensor ? 1 : 0;
    int64_t b, h, p, c;
    decode(a, g - t * a.per_tensor, a.head_dim / V, b, h, p, c);
    const int64_t src = b * a.is[t][0] + h * a.is[t][1] + (a.in_start + p) * a.is[t][2] + c * V;
    const int64_t dst = b * a.os[t][0] + h * a.os[t][1] + (a.out_start + p) * a.os[t][2] + c * V;
    *reinterpret_cast<u32x4*>(a.out[t] + dst * ESIZE) = *reinterpret_cast<const u32x4*>(a.in[t] + src * ESIZE);
}

// Scalar path: any strides, one element per thread.
template <typename B>
__global__ void __launch_bounds__(kThreads) copy_interval_kernel(CopyArgs a) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= 2 * a.per_tensor) return;
    const int t = g >= a.per_tensor ? 1 : 0;
    int64_t b, h, p, d;
    decode(a, g - t * a.per_tensor, a.head_dim, b, h, p, d);
    const int64_t src = b * a.is[t][0] + h * a.is[t][1] + (a.in_start + p) * a.is[t][2] + d * a.is[t][3];
    const int64_t dst = b * a.os[t][0] + h * a.os[t][1] + (a.out_start + p) * a.os[t][2] + d * a.os[t][3];
    reinterpret_cast<B*>(a.out[t])[dst] = reinterpret_cast<const B*>(a.in[t])[src];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kvr

extern "C" int kvr_copy_kv_interval(void* out_k, void* out_v, const void* in_k, const void* in_v, int32_t batch,
                                    int32_t heads, int64_t width, int32_t head_dim, int64_t out_start,
                                    int64_t in_start, const int64_t strides[16], int32_t dtype, void* stream) {
    using namespace kvr;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (batch <= 0 || heads <= 0 || head_dim <= 0 || width < 0 || out_start < 0 || in_start < 0)
        return KVR_E_INVALID_ARGUMENT;
    if (!strides) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 16; ++i)
        if (strides[i] <= 0) return KVR_E_BAD_STRIDE;
    if (width == 0) return KVR_OK;
    if (!out_k || !out_v || !in_k || !in_v) return KVR_E_NULL_POINTER;
    const int64_t elems = static_cast<int64_t>(batch) * heads * width * head_dim;
    if (elems > (int64_t(1) << 37)) return KVR_E_UNSUPPORTED_SHAPE;  // grid.x < 2^31

    CopyArgs a;
    a.out[0] = static_cast<char*>(out_k);
    a.out[1] = static_cast<char*>(out_v);
    a.in[0] = static_cast<const char*>(in_k);
    a.in[1] = static_cast<const char*>(in_v);
    for (int i = 0; i < 4; ++i) {
        a.os[0][i] = strides[i];
        a.os[1][i] = strides[4 + i];
        a.is[0][i] = strides[8 + i];
        a.is[1][i] = strides[12 + i];
    }
    a.out_start = out_start;
    a.in_start = in_start;
    a.width = width;
    a.heads = heads;
    a.head_dim = head_dim;

    // Vector path: each row is whole 16-byte vectors at 16-byte aligned addresses.
    bool vec = (static_cast<int64_t>(head_dim) * esize) % 16 == 0 && aligned16(out_k) && aligned16(out_v) &&
               aligned16(in_k) && aligned16(in_v);
    for (int t = 0; t < 4 && vec; ++t) {
        const int64_t* s = strides + 4 * t;
        vec = s[3] == 1 && (s[0] * esize) % 16 == 0 && (s[1] * esize) % 16 == 0 && (s[2] * esize) % 16 == 0;
    }
    hipStream_t s = as_stream(stream);
    if (vec) {
        a.per_tensor = elems / (16 / esize);
        const unsigned grid = static_cast<unsigned>(ceil_div(2 * a.per_tensor, kThreads));
        if (esize == 4) copy_interval_vec_kernel<4><<<grid, kThreads, 0, s>>>(a);
        else copy_interval_vec_kernel<2><<<grid, kThreads, 0, s>>>(a);
    } else {
        a.per_tensor = elems;
        const unsigned grid = static_cast<unsigned>(ceil_div(2 * a.per_tensor, kThreads));
        if (esize == 4) copy_interval_kernel<uint32_t><<<grid, kThreads, 0, s>>>(a);
        else copy_interval_kernel<uint16_t><<<grid, kThreads, 0, s>>>(a);
    }
    return launch_status();
}
