// RoPE delta re-rotation of retained-suffix keys and the fused shift-cache
// build (prefix copy + rotated K tail + copied V tail), all layers per launch.
//
// Reference semantics: src/kv_cache_repair/cache.py:47-77 (shifted_suffix_keys)
// and cache.py:128-139 (per-layer cat of prefix and shifted tail).
//
// Arithmetic is an exact restatement of the eager op sequence
//   c = dtype(cos(inv_freq * shift) * scaling), s = dtype(sin(...) * scaling)
//   out = dtype(dtype(k * c) + dtype(rotate_half(k) * s))
// so the result is bit-identical to the eager chain whenever c and s are.
#include "kvr_internal.h"

#include <string.h>

namespace kvr {
namespace {

constexpr int kMaxLayersPerLaunch = 64;
constexpr int kBlockThreads = 256;
// Rows per thread (each two independent 16-byte loads in flight) is a launch
// parameter: 1 for rotate-only launches (K rows of one tensor per layer), 2 for
// the shift-cache build (K and V). Measured on 8B-shaped bf16 caches of 2k-32k
// tokens: fewer, shorter-lived rows per thread keep every CU busy to the end of
// the grid (rotate-only over an 8k cache 130 -> 120 us, 71 -> 77% of 8 TB/s;
// over a 2k cache 62 -> 69%); 4 or 8 rows per thread were slower for both.

struct LayerTable {
    const void* src[2][kMaxLayersPerLaunch];  // [K=0 / V=1][layer]
    void* dst[2][kMaxLayersPerLaunch];
};

struct RowMap {
    int64_t src_stride[3];  // head, row, dim (elements)
    int64_t dst_stride[3];
    int64_t prefix_rows;     // logical rows [0, prefix) copy row r -> row r
    int64_t src_tail_start;  // logical rows [prefix, prefix+tail) come from src_tail_start + (r - prefix)
    int64_t dst_tail_start;  //   ... and go to dst_tail_start + (r - prefix)
    int64_t tail_rows;
    int32_t n_heads;
    int32_t head_dim;
    int32_t rotary_dim;
    int32_t rotate;      // 0: the tail is copied too (shift == 0)
    float shift_f;       // (float)shift, as HF's position_ids.float()
    float scaling;       // rotary attention_scaling
};

// Logical row -> (src row, dst row, rotated?) for the K (kv==0) or V (kv==1) tensor.
__device__ inline void map_row(const RowMap& m, int kv, int64_t r, int64_t& src_row, int64_t& dst_row, bool& rot) {
    if (r < m.prefix_rows) {
        src_row = r;
        dst_row = r;
        rot = false;
    } else {
        const int64_t t = r - m.prefix_rows;
        src_row = m.src_tail_start + t;
        dst_row = m.dst_tail_start + t;
        rot = (kv == 0) && (m.rotate != 0);
    }
}

// cos/sin of one rotary frequency exactly as the eager path produces them:
// fp32 product inv_freq * position, fp32 cos/sin, fp32 scaling, cast to T.
template <typename T>
__device__ inline void rope_cs(const float* inv_freq, int i, float shift_f, float scaling, float& c, float& s) {
#pragma clang fp contract(off)
    const float freq = inv_freq[i] * shift_f;
    c = round_through<T>(cosf(freq) * scaling);
    s = round_through<T>(sinf(freq) * scaling);
}

// One rotated pair: lo = k[i], hi = k[i + half].
// bf16 pairs through v_cvt_pk_bf16_f32 (round to nearest even, as the
// software rounding of elem<bf16_t> for every non-NaN value): the eager
// sequence of rotate_pair for two elements at once. A NaN stays NaN through
// the intermediate roundings; the final rounding returns torch's canonical
// NaN (0x7FC0) for it.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ inline f32x2 round2_bf16(f32x2 v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    return f32x2{__uint_as_float(b << 16), __uint_as_float(b & 0xffff0000u)};
}

__device__ inline uint32_t pack2_bf16(f32x2 v) {
    const float qnan = __uint_as_float(0x7fc00000u);
    const f32x2 c = {v.x != v.x ? qnan : v.x, v.y != v.y ? qnan : v.y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(c, bf16x2));
}

// Rotated halves of two adjacent elements (e, e + 1): lo/hi hold the first- and
// second-half inputs, c/s their cos/sin; returns the packed bf16 outputs.
__device__ inline void rotate_pair2_bf16(uint32_t lo, uint32_t hi, f32x2 c, f32x2 s, uint32_t& out_lo,
                                         uint32_t& out_hi) {
#pragma clang fp contract(off)
    const f32x2 l = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u)};
    const f32x2 h = {__uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u)};
    const f32x2 a0 = round2_bf16(l * c);
    const f32x2 b0 = round2_bf16((-h) * s);
    const f32x2 a1 = round2_bf16(h * c);
    const f32x2 b1 = round2_bf16(l * s);
    out_lo = pack2_bf16(a0 + b0);
    out_hi = pack2_bf16(a1 + b1);
}

template <typename T>
__device__ inline void rotate_pair(float lo, float hi, float c, float s, float& out_lo, float& out_hi) {
#pragma clang fp contract(off)
    // first half:  k[i]*c + (-k[i+h])*s ; second half: k[i+h]*c + k[i]*s
    const float a0 = round_through<T>(lo * c);
    const float b0 = round_through<T>((-hi) * s);
    const float a1 = round_through<T>(hi * c);
    const float b1 = round_through<T>(lo * s);
    out_lo = round_through<T>(a0 + b0);
    out_hi = round_through<T>(a1 + b1);
}

// ---------------------------------------------------------------------------
// Vector path: rotary_dim == head_dim, unit dim stride, 16-byte aligned rows.
// TPR threads share a row; thread c owns the 16-byte chunk c of the first half
// and its partner chunk c of the second half, so cos/sin are per-thread
// constants computed once. Grid: x = row tiles, y = head*(n_kv) + kv, z = layer.
// ---------------------------------------------------------------------------
template <typename T, int kRowPasses>
__global__ void __launch_bounds__(kBlockThreads)
shift_rows_vec_kernel(LayerTable tab, RowMap m, const float* __restrict__ inv_freq, int n_kv, int tpr_log2) {
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int EPV = 16 / E::size;  // elements per 16-byte vector

    const int layer = blockIdx.z;
    const int kv = (n_kv == 2) ? (blockIdx.y & 1) : 0;
    const int head = (n_kv == 2) ? (blockIdx.y >> 1) : blockIdx.y;
    const int tpr = 1 << tpr_log2;
    const int chunk = threadIdx.x & (tpr - 1);
    const int rows_per_pass = kBlockThreads >> tpr_log2;
    const int64_t total_rows = m.prefix_rows + m.tail_rows;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rows_per_pass * kRowPasses + (threadIdx.x >> tpr_log2);

    const char* src = static_cast<const char*>(tab.src[kv][layer]);
    char* dst = static_cast<char*>(tab.dst[kv][layer]);
    const int half = m.head_dim >> 1;
    const int64_t src_head = static_cast<int64_t>(head) * m.src_stride[0];
    const int64_t dst_head = static_cast<int64_t>(head) * m.dst_stride[0];

    // Loads first (they do not depend on cos/sin), then the cos/sin table.
    u32x4 lo[kRowPasses], hi[kRowPasses];
    int64_t dst_off[kRowPasses];
    bool rot[kRowPasses], live[kRowPasses];
#pragma unroll
    for (int p = 0; p < kRowPasses; ++p) {
        const int64_t r = row0 + static_cast<int64_t>(p) * rows_per_pass;
        live[p] = r < total_rows;
        if (live[p]) {
            int64_t sr, dr;
            bool rr;
            map_row(m, kv, r, sr, dr, rr);
            rot[p] = rr;
            const int64_t so = (src_head + sr * m.src_stride[1]) + static_cast<int64_t>(chunk) * EPV;
            dst_off[p] = (dst_head + dr * m.dst_stride[1]) + static_cast<int64_t>(chunk) * EPV;
            lo[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + so * E::size));
            hi[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (so + half) * E::size));
        }
    }

    // Every rotated row uses the same shift: the block computes the half-row
    // of cos/sin once into LDS (dynamic, 2 * half floats) and each thread reads
    // its chunk's values (the same rope_cs roundings as one thread per value).
    float cs_c[EPV], cs_s[EPV];
    const bool any_rot = (kv == 0) && (m.rotate != 0) && (m.tail_rows > 0);  // block-uniform
    if (any_rot) {
        extern __shared__ float cs_lds[];  // [cos half][sin half]
        for (int i = threadIdx.x; i < half; i += kBlockThreads)
            rope_cs<T>(inv_freq, i, m.shift_f, m.scaling, cs_lds[i], cs_lds[half + i]);
        __syncthreads();
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            cs_c[e] = cs_lds[chunk * EPV + e];
            cs_s[e] = cs_lds[half + chunk * EPV + e];
        }
    }
#pragma unroll
    for (int p = 0; p < kRowPasses; ++p) {
        if (!live[p]) continue;
        u32x4 olo = lo[p], ohi = hi[p];
        if (rot[p]) {
            if constexpr (__is_same(T, bf16_t)) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t rl, rh;
                    rotate_pair2_bf16(lo[p][q], hi[p][q], f32x2{cs_c[2 * q], cs_c[2 * q + 1]},
                                      f32x2{cs_s[2 * q], cs_s[2 * q + 1]}, rl, rh);
                    olo[q] = rl;
                    ohi[q] = rh;
                }
            } else {
                bits lb[EPV], hb[EPV], olb[EPV], ohb[EPV];
                __builtin_memcpy(lb, &lo[p], 16);
                __builtin_memcpy(hb, &hi[p], 16);
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    float a, b;
                    rotate_pair<T>(E::to_float(lb[e]), E::to_float(hb[e]), cs_c[e], cs_s[e], a, b);
                    olb[e] = E::from_float(a);
                    ohb[e] = E::from_float(b);
                }
                __builtin_memcpy(&olo, olb, 16);
                __builtin_memcpy(&ohi, ohb, 16);
            }
        }
        __builtin_nontemporal_store(olo, reinterpret_cast<u32x4*>(dst + dst_off[p] * E::size));
        __builtin_nontemporal_store(ohi, reinterpret_cast<u32x4*>(dst + (dst_off[p] + half) * E::size));
    }
}

// ---------------------------------------------------------------------------
// Scalar path: any strides, partial rotary, any even head_dim. One thread per
// (row, element) of the first rotary half, plus one per passthrough element.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kBlockThreads)
shift_rows_scalar_kernel(LayerTable tab, RowMap m, const float* __restrict__ inv_freq, int n_kv) {
    using E = elem<T>;
    using bits = typename E::bits;
    const int layer = blockIdx.z;
    const int kv = (n_kv == 2) ? (blockIdx.y & 1) : 0;
    const int head = (n_kv == 2) ? (blockIdx.y >> 1) : blockIdx.y;
    const int half = m.rotary_dim >> 1;
    const int lanes_per_row = half + (m.head_dim - m.rotary_dim);
    const int64_t total_rows = m.prefix_rows + m.tail_rows;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlockThreads + threadIdx.x;
    const int64_t r = idx / lanes_per_row;
    const int e = static_cast<int>(idx - r * lanes_per_row);
    if (r >= total_rows) return;
    int64_t sr, dr;
    bool rot;
    map_row(m, kv, r, sr, dr, rot);
    const bits* src = static_cast<const bits*>(tab.src[kv][layer]);
    bits* dst = static_cast<bits*>(tab.dst[kv][layer]);
    const int64_t so = head * m.src_stride[0] + sr * m.src_stride[1];
    const int64_t d0 = head * m.dst_stride[0] + dr * m.dst_stride[1];
    if (e < half) {
        const bits lo = src[so + e * m.src_stride[2]];
        const bits hi = src[so + (e + half) * m.src_stride[2]];
        bits olo = lo, ohi = hi;
        if (rot) {
            float c, s, a, b;
            rope_cs<T>(inv_freq, e, m.shift_f, m.scaling, c, s);
            rotate_pair<T>(E::to_float(lo), E::to_float(hi), c, s, a, b);
            olo = E::from_float(a);
            ohi = E::from_float(b);
        }
        dst[d0 + e * m.dst_stride[2]] = olo;
        dst[d0 + (e + half) * m.dst_stride[2]] = ohi;
    } else {
        const int d = m.rotary_dim + (e - half);
        dst[d0 + d * m.dst_stride[2]] = src[so + d * m.src_stride[2]];
    }
}

template <typename T>
int launch_shift(const LayerTable& tab, const RowMap& m, const float* inv_freq, int n_layers, int n_kv, bool vec,
                 int tpr_log2, hipStream_t stream) {
    const int64_t total_rows = m.prefix_rows + m.tail_rows;
    if (vec) {
        const int passes = n_kv == 1 ? 1 : 2;  // rows per thread (kRowPasses above)
        const int rows_per_block = (kBlockThreads >> tpr_log2) * passes;
        dim3 grid(static_cast<unsigned>(ceil_div(total_rows, rows_per_block)), m.n_heads * n_kv, n_layers);
        const size_t lds = m.rotate ? static_cast<size_t>(m.head_dim) * sizeof(float) : 0;  // cos + sin halves
        if (passes == 1)
            shift_rows_vec_kernel<T, 1><<<grid, kBlockThreads, lds, stream>>>(tab, m, inv_freq, n_kv, tpr_log2);
        else
            shift_rows_vec_kernel<T, 2><<<grid, kBlockThreads, lds, stream>>>(tab, m, inv_freq, n_kv, tpr_log2);
    } else {
        const int lanes_per_row = (m.rotary_dim >> 1) + (m.head_dim - m.rotary_dim);
        dim3 grid(static_cast<unsigned>(ceil_div(total_rows * lanes_per_row, kBlockThreads)), m.n_heads * n_kv,
                  n_layers);
        shift_rows_scalar_kernel<T><<<grid, kBlockThreads, 0, stream>>>(tab, m, inv_freq, n_kv);
    }
    return launch_status();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shared driver for both entry points.
int shift_rows(const void* const* src_k, const void* const* src_v, void* const* dst_k, void* const* dst_v,
               int32_t n_layers, int32_t n_heads, int32_t head_dim, int32_t rotary_dim, const int64_t src_stride[3],
               const int64_t dst_stride[3], int64_t prefix_rows, int64_t src_tail, int64_t dst_tail, int64_t tail_rows,
               int64_t shift, const float* inv_freq, float scaling, int32_t dtype, void* stream) {
    if (n_layers < 0 || n_heads <= 0 || head_dim <= 0 || (head_dim & 1)) return KVR_E_UNSUPPORTED_SHAPE;
    if (rotary_dim <= 0 || (rotary_dim & 1) || rotary_dim > head_dim) return KVR_E_UNSUPPORTED_SHAPE;
    if (prefix_rows < 0 || tail_rows < 0 || src_tail < 0 || dst_tail < 0) return KVR_E_INVALID_ARGUMENT;
    if (n_heads > 65535 / 2 || head_dim > 4096) return KVR_E_UNSUPPORTED_SHAPE;
    if (shift > (int64_t(1) << 24) || shift < -(int64_t(1) << 24)) return KVR_E_INVALID_ARGUMENT;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (!src_stride || !dst_stride || !src_k || !dst_k) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 3; ++i)
        if (src_stride[i] <= 0 || dst_stride[i] <= 0) return KVR_E_BAD_STRIDE;
    const bool rotate = shift != 0 && tail_rows > 0;
    if (rotate && !inv_freq) return KVR_E_NULL_POINTER;
    const int n_kv = src_v ? 2 : 1;
    if (n_kv == 2 && !dst_v) return KVR_E_NULL_POINTER;
    if (n_layers == 0 || prefix_rows + tail_rows == 0) return KVR_OK;
    if (prefix_rows + tail_rows > (int64_t(1) << 40)) return KVR_E_UNSUPPORTED_SHAPE;

    RowMap m;
    for (int i = 0; i < 3; ++i) {
        m.src_stride[i] = src_stride[i];
        m.dst_stride[i] = dst_stride[i];
    }
    m.prefix_rows = prefix_rows;
    m.src_tail_start = src_tail;
    m.dst_tail_start = dst_tail;
    m.tail_rows = tail_rows;
    m.n_heads = n_heads;
    m.head_dim = head_dim;
    m.rotary_dim = rotary_dim;
    m.rotate = rotate ? 1 : 0;
    m.shift_f = static_cast<float>(shift);
    m.scaling = scaling;

    // Vector path eligibility: whole-row rotary, unit dim stride, 16-byte
    // aligned half rows, power-of-two threads per row.
    const int64_t half_bytes = static_cast<int64_t>(head_dim / 2) * esize;
    bool vec = rotary_dim == head_dim && src_stride[2] == 1 && dst_stride[2] == 1 && half_bytes % 16 == 0;
    int tpr_log2 = 0;
    if (vec) {
        const int64_t tpr = half_bytes / 16;
        while ((int64_t(1) << tpr_log2) < tpr) ++tpr_log2;
        vec = (int64_t(1) << tpr_log2) == tpr && tpr <= kBlockThreads;
        for (int i = 0; i < 2 && vec; ++i)
            vec = (src_stride[i] * esize) % 16 == 0 && (dst_stride[i] * esize) % 16 == 0;
    }
    hipStream_t s = as_stream(stream);
    for (int32_t l0 = 0; l0 < n_layers; l0 += kMaxLayersPerLaunch) {
        const int nl = (n_layers - l0) < kMaxLayersPerLaunch ? (n_layers - l0) : kMaxLayersPerLaunch;
        LayerTable tab;
        memset(&tab, 0, sizeof(tab));
        for (int l = 0; l < nl; ++l) {
            tab.src[0][l] = src_k[l0 + l];
            tab.dst[0][l] = dst_k[l0 + l];
            if (!tab.src[0][l] || !tab.dst[0][l]) return KVR_E_NULL_POINTER;
            if (vec && !(aligned16(tab.src[0][l]) && aligned16(tab.dst[0][l]))) vec = false;
            if (n_kv == 2) {
                tab.src[1][l] = src_v[l0 + l];
                tab.dst[1][l] = dst_v[l0 + l];
                if (!tab.src[1][l] || !tab.dst[1][l]) return KVR_E_NULL_POINTER;
                if (vec && !(aligned16(tab.src[1][l]) && aligned16(tab.dst[1][l]))) vec = false;
            }
        }
        int st;
        switch (dtype) {
            case KVR_DTYPE_F32: st = launch_shift<f32_t>(tab, m, inv_freq, nl, n_kv, vec, tpr_log2, s); break;
            case KVR_DTYPE_F16: st = launch_shift<f16_t>(tab, m, inv_freq, nl, n_kv, vec, tpr_log2, s); break;
            default: st = launch_shift<bf16_t>(tab, m, inv_freq, nl, n_kv, vec, tpr_log2, s); break;
        }
        if (st != KVR_OK) return st;
    }
    return KVR_OK;
}

}  // namespace
}  // namespace kvr

extern "C" int kvr_rope_delta_rotate(const void* const* src, void* const* dst, int32_t n_layers, int32_t n_heads,
                                     int64_t rows, int32_t head_dim, int32_t rotary_dim, const int64_t src_stride[3],
                                     const int64_t dst_stride[3], int64_t shift, const float* inv_freq,
                                     float attention_scaling, int32_t dtype, void* stream) {
    if (rows < 0) return KVR_E_INVALID_ARGUMENT;
    return kvr::shift_rows(src, nullptr, dst, nullptr, n_layers, n_heads, head_dim, rotary_dim, src_stride, dst_stride,
                           0, 0, 0, rows, shift, inv_freq, attention_scaling, dtype, stream);
}

extern "C" int kvr_shift_cache_build(const void* const* old_k, const void* const* old_v, void* const* new_k,
                                     void* const* new_v, int32_t n_layers, int32_t n_heads, int32_t head_dim,
                                     int32_t rotary_dim, const int64_t old_stride[3], const int64_t new_stride[3],
                                     int64_t prefix_rows, int64_t old_tail_start, int64_t new_tail_start,
                                     int64_t tail_rows, int64_t shift, const float* inv_freq, float attention_scaling,
                                     int32_t dtype, void* stream) {
    if (!old_v || !new_v) return KVR_E_NULL_POINTER;
    if (new_tail_start < prefix_rows) return KVR_E_INVALID_ARGUMENT;
    return kvr::shift_rows(old_k, old_v, new_k, new_v, n_layers, n_heads, head_dim, rotary_dim, old_stride,
                           new_stride, prefix_rows, old_tail_start, new_tail_start, tail_rows, shift, inv_freq,
                           attention_scaling, dtype, stream);
}
