// Indexed K/V scatter: out[:, h, positions[r], :] = fresh[:, h, r, :], bit copy.
//
// Reference semantics: src/kv_cache_repair/kernels/packed_cache.py:189-191
// (index_copy_ along the token axis) and the contract of indexed_kv_scatter_
// (src/kv_cache_repair/kernels/indexed_attention.py:179-204): every other byte
// of the output storage is preserved, payloads are copied as raw bits, and a
// position outside [0, n_keys) writes nothing (_indexed_triton.py:22-27).
#include "kvr_internal.h"

namespace kvr {
namespace {

constexpr int kThreads = 256;

struct ScatterArgs {
    char* out[2];          // K, V
    const char* fresh[2];  // K, V
    int64_t out_stride[2][3];
    int64_t fresh_stride[2][3];
    const int64_t* positions;
    int64_t n_sel;
    int64_t n_keys;
    int32_t n_heads;
    int32_t head_dim;
};

// Vector path: one thread moves one 16-byte chunk. Flat index order is
// (kv, head, row, chunk) so neighbouring lanes touch neighbouring bytes. The
// launch keeps the thread count below 2^31, so the index decode runs in 32
// bits; the cache rows are written with nontemporal stores (streamed).
__global__ void __launch_bounds__(kThreads) scatter_vec_kernel(ScatterArgs a, int esize, int chunks_log2) {
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t n_sel = static_cast<uint32_t>(a.n_sel);
    const uint32_t per_kv = (static_cast<uint32_t>(a.n_heads) * n_sel) << chunks_log2;
    if (idx >= 2 * per_kv) return;
    const int kv = idx >= per_kv ? 1 : 0;
    const uint32_t rem = idx - (kv ? per_kv : 0);
    const int64_t c = rem & ((1u << chunks_log2) - 1);
    const uint32_t hr = rem >> chunks_log2;
    const uint32_t h32 = hr / n_sel;
    const int64_t r = hr - h32 * n_sel;
    const int64_t h = h32;
    const int64_t pos = a.positions[r];
    if (pos < 0 || pos >= a.n_keys) return;
    const int64_t src_off = (h * a.fresh_stride[kv][0] + r * a.fresh_stride[kv][1]) * esize + c * 16;
    const int64_t dst_off = (h * a.out_stride[kv][0] + pos * a.out_stride[kv][1]) * esize + c * 16;
    const u32x4 v = *reinterpret_cast<const u32x4*>(a.fresh[kv] + src_off);
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.out[kv] + dst_off));
}

// Scalar path: one thread per element, arbitrary positive strides.
template <typename bits>
__global__ void __launch_bounds__(kThreads) scatter_scalar_kernel(ScatterArgs a) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t per_kv = static_cast<int64_t>(a.n_heads) * a.n_sel * a.head_dim;
    if (idx >= 2 * per_kv) return;
    const int kv = idx >= per_kv ? 1 : 0;
    const int64_t rem = idx - kv * per_kv;
    const int64_t d = rem % a.head_dim;
    const int64_t hr = rem / a.head_dim;
    const int64_t r = hr % a.n_sel;
    const int64_t h = hr / a.n_sel;
    const int64_t pos = a.positions[r];
    if (pos < 0 || pos >= a.n_keys) return;
    const bits* src = reinterpret_cast<const bits*>(a.fresh[kv]);
    bits* dst = reinterpret_cast<bits*>(a.out[kv]);
    dst[h * a.out_stride[kv][0] + pos * a.out_stride[kv][1] + d * a.out_stride[kv][2]] =
        src[h * a.fresh_stride[kv][0] + r * a.fresh_stride[kv][1] + d * a.fresh_stride[kv][2]];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kvr

extern "C" int kvr_indexed_scatter_kv(void* out_k, void* out_v, const void* fresh_k, const void* fresh_v,
                                      const int64_t* positions, int64_t n_sel, int32_t n_heads, int64_t n_keys,
                                      int32_t head_dim, const int64_t strides[12], int32_t dtype, void* stream) {
    using namespace kvr;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_keys < 0) return KVR_E_INVALID_ARGUMENT;
    if (n_heads <= 0 || head_dim <= 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (!strides) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 12; ++i)
        if (strides[i] <= 0) return KVR_E_BAD_STRIDE;
    if (n_sel == 0) return KVR_OK;
    if (!out_k || !out_v || !fresh_k || !fresh_v || !positions) return KVR_E_NULL_POINTER;

    ScatterArgs a;
    a.out[0] = static_cast<char*>(out_k);
    a.out[1] = static_cast<char*>(out_v);
    a.fresh[0] = static_cast<const char*>(fresh_k);
    a.fresh[1] = static_cast<const char*>(fresh_v);
    for (int i = 0; i < 3; ++i) {
        a.out_stride[0][i] = strides[0 + i];
        a.out_stride[1][i] = strides[3 + i];
        a.fresh_stride[0][i] = strides[6 + i];
        a.fresh_stride[1][i] = strides[9 + i];
    }
    a.positions = positions;
    a.n_sel = n_sel;
    a.n_keys = n_keys;
    a.n_heads = n_heads;
    a.head_dim = head_dim;

    const int64_t row_bytes = static_cast<int64_t>(head_dim) * esize;
    bool vec = row_bytes % 16 == 0;
    int chunks_log2 = 0;
    if (vec) {
        const int64_t chunks = row_bytes / 16;
        while ((int64_t(1) << chunks_log2) < chunks) ++chunks_log2;
        vec = (int64_t(1) << chunks_log2) == chunks;
    }
    for (int t = 0; t < 4 && vec; ++t) {
        const int64_t* s = strides + 3 * t;
        vec = s[2] == 1 && (s[0] * esize) % 16 == 0 && (s[1] * esize) % 16 == 0;
    }
    vec = vec && aligned16(out_k) && aligned16(out_v) && aligned16(fresh_k) && aligned16(fresh_v);

    hipStream_t s = as_stream(stream);
    vec = vec && 2 * static_cast<int64_t>(n_heads) * n_sel * (int64_t(1) << chunks_log2) < (int64_t(1) << 31);
    if (vec) {
        const int64_t total = 2 * static_cast<int64_t>(n_heads) * n_sel * (int64_t(1) << chunks_log2);
        scatter_vec_kernel<<<static_cast<unsigned>(ceil_div(total, kThreads)), kThreads, 0, s>>>(a, esize,
                                                                                                  chunks_log2);
    } else {
        const int64_t total = 2 * static_cast<int64_t>(n_heads) * n_sel * head_dim;
        const unsigned grid = static_cast<unsigned>(ceil_div(total, kThreads));
        if (esize == 4)
            scatter_scalar_kernel<uint32_t><<<grid, kThreads, 0, s>>>(a);
        else
            scatter_scalar_kernel<uint16_t><<<grid, kThreads, 0, s>>>(a);
    }
    return launch_status();
}
