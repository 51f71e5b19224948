// Fresh-row epilogue of one packed layer in ONE launch:
//   q_out[h, r]              = rope(q[h, r], cos[r], sin[r])        (query heads)
//   out_k[h, positions[r]]   = rope(fresh_k[h, r], cos[r], sin[r])  (KV heads)
//   out_v[h, positions[r]]   = fresh_v[h, r]                        (bit copy)
// where rope(x) = x * cos + rotate_half(x) * sin with split-half pairs.
//
// Reference semantics: the fresh rows' RoPE at absolute positions that the
// native decoder applies before the cache update (transformers 5.15.0
// models/llama/modeling_llama.py:137-160, apply_rotary_pos_emb with the
// cos/sin of the model's rotary_emb), followed by the packed layer's
// index_copy_ writeback (src/kv_cache_repair/kernels/packed_cache.py:189-191).
// Each multiply and the add round to the storage type exactly as the eager
// elementwise ops do, so the outputs are bit-identical to that op sequence.
// A position outside [0, n_keys) writes no K/V row (as the scatter).
//
// With per-head norm weights (Qwen3's q_norm / k_norm, transformers 5.15.0
// models/qwen3/modeling_qwen3.py:252-257 apply them to the projected q and k
// before RoPE) each q / k row is first RMS-normalised over head_dim:
//   x' = w * dtype(x * rsqrt(mean(x^2) + eps))
// with kvr_rms_norm's fp32 summation order (per 16-byte vector, then the
// butterfly over vectors), so the result is bit-identical to kvr_rms_norm
// followed by the plain epilogue.
#include "kvr_internal.h"

#include <type_traits>

namespace kvr {
namespace {

constexpr int kThreads = 64;  // one wave per block: a refresh's few thousand head rows reach ~4x more CUs

struct FreshArgs {
    const char* q;
    char* q_out;
    const char* fresh[2];  // K, V
    char* out[2];          // K, V
    const char* cos;
    const char* sin;
    int64_t qs[3], qos[3], fs[2][3], os[2][3];  // {head,row,dim} element strides
    int64_t cs[2], ss[2];                       // cos/sin {row,dim} element strides
    const int64_t* positions;
    int64_t n_sel;
    int64_t n_keys;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    PartialSums src;      // src.base != nullptr: q / fresh K / fresh V come from split-K partial sums
    int64_t part_col[3];  // their first column in the concatenated projection
    const char* norm_w[2];  // per-head RMSNorm weights [head_dim] of q and k, or null (no norm)
    float norm_eps[2];
};

// One rotated pair with distinct cos/sin for the two halves (the rotary
// embedding's halves are equal by construction, but the values are read as
// given): lo' = lo*c_lo + (-hi)*s_lo ; hi' = hi*c_hi + lo*s_hi.
template <typename T>
__device__ inline void rope_pair(float lo, float hi, float c_lo, float s_lo, float c_hi, float s_hi, float& out_lo,
                                 float& out_hi) {
#pragma clang fp contract(off)
    const float a0 = round_through<T>(lo * c_lo);
    const float b0 = round_through<T>((-hi) * s_lo);
    const float a1 = round_through<T>(hi * c_hi);
    const float b1 = round_through<T>(lo * s_hi);
    out_lo = round_through<T>(a0 + b0);
    out_hi = round_through<T>(a1 + b1);
}

// Rows of the launch: [0, Hq*B) queries, then Hkv*B keys, then Hkv*B values;
// within each part row index = r * heads + h, so the lanes of a wave walk the
// heads of one token (contiguous in the projections' token-major storage).
__device__ inline void decode_row(const FreshArgs& a, int64_t g, int& part, int64_t& h, int64_t& r) {
    const int64_t nq = static_cast<int64_t>(a.n_q_heads) * a.n_sel;
    const int64_t nkv = static_cast<int64_t>(a.n_kv_heads) * a.n_sel;
    if (g < nq) {
        part = 0;
        r = g / a.n_q_heads;
        h = g - r * a.n_q_heads;
    } else {
        g -= nq;
        part = g < nkv ? 1 : 2;
        if (part == 2) g -= nkv;
        r = g / a.n_kv_heads;
        h = g - r * a.n_kv_heads;
    }
}

// RMSNorm of one row held by TPR lanes, lane c holding 16-byte vector c of the
// first half (lo) and vector c of the second half (hi), in place. The sum of
// squares follows kvr_rms_norm, whose lane j holds vector j of 2 TPR: each
// vector's squares summed in order, then a butterfly over the vectors; its
// first step pairs vectors c and c + TPR, i.e. lo + hi here, and the rest of
// the butterfly runs over the TPR lanes.
template <typename T>
__device__ inline void norm_row(u32x4& lo, u32x4& hi, const u32x4& w_lo, const u32x4& w_hi, int tpr, int dim,
                                float eps) {
#pragma clang fp contract(off)
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int EPV = 16 / E::size;
    bits xl[EPV], xh[EPV], wl[EPV], wh[EPV];
    __builtin_memcpy(xl, &lo, 16);
    __builtin_memcpy(xh, &hi, 16);
    __builtin_memcpy(wl, &w_lo, 16);
    __builtin_memcpy(wh, &w_hi, 16);
    float vl[EPV], vh[EPV], s_lo = 0.f, s_hi = 0.f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
        vl[e] = E::to_float(xl[e]);
        vh[e] = E::to_float(xh[e]);
        s_lo += vl[e] * vl[e];
        s_hi += vh[e] * vh[e];
    }
    float ss = s_lo + s_hi;
    for (int off = tpr >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off, tpr);
    const float inv = rsqrtf(ss * (1.f / static_cast<float>(dim)) + eps);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
        xl[e] = E::from_float(E::to_float(wl[e]) * round_through<T>(vl[e] * inv));
        xh[e] = E::from_float(E::to_float(wh[e]) * round_through<T>(vh[e] * inv));
    }
    __builtin_memcpy(&lo, xl, 16);
    __builtin_memcpy(&hi, xh, 16);
}

// Vector path: unit dim strides, 16-byte aligned rows. TPR threads share a
// row; thread c owns the 16-byte chunk c of the first half and chunk c of the
// second half (its rotate_half partner). PARTIALS: q/k/v come from split-K
// partial sums; NORM: per-head RMSNorm weights are given. Each combination is
// its own instantiation, so the plain path keeps its register count (and
// occupancy) free of the partial sums' and the norm's live values. Outputs are
// written with nontemporal stores (streamed, not kept in L2: -20% at c5).
template <typename T, bool PARTIALS, bool NORM>
__global__ void __launch_bounds__(kThreads) fresh_vec_kernel(FreshArgs a, int tpr_log2) {
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int EPV = 16 / E::size;
    const int tpr = 1 << tpr_log2;
    // the launch keeps rows * TPR below 2^31, so the row decode runs in 32 bits
    const uint32_t g = (blockIdx.x * kThreads + threadIdx.x) >> tpr_log2;
    const int c = threadIdx.x & (tpr - 1);
    const uint32_t nq = static_cast<uint32_t>(a.n_q_heads) * static_cast<uint32_t>(a.n_sel);
    const uint32_t nkv = static_cast<uint32_t>(a.n_kv_heads) * static_cast<uint32_t>(a.n_sel);
    if (g >= nq + 2 * nkv) return;
    int part;
    int64_t h, r;
    if (g < nq) {
        part = 0;
        r = g / static_cast<uint32_t>(a.n_q_heads);
        h = g - static_cast<uint32_t>(r) * static_cast<uint32_t>(a.n_q_heads);
    } else {
        const uint32_t k = g - nq;
        part = k < nkv ? 1 : 2;
        const uint32_t kk = part == 2 ? k - nkv : k;
        r = kk / static_cast<uint32_t>(a.n_kv_heads);
        h = kk - static_cast<uint32_t>(r) * static_cast<uint32_t>(a.n_kv_heads);
    }
    const int half = a.head_dim >> 1;
    const int64_t lo_off = static_cast<int64_t>(c) * EPV;
    const int64_t hi_off = lo_off + half;

    // Issue every load first (the row's position, its q/k/v chunks or their
    // fp32 partials, the cos/sin chunks) so the thread waits once; the
    // position is checked only before the store.
    const int64_t pos = part == 0 ? 0 : a.positions[r];
    u32x4 lo, hi, c_lo, c_hi, s_lo, s_hi;
    if constexpr (!PARTIALS) {
        const char* src = part == 0 ? a.q + (h * a.qs[0] + r * a.qs[1]) * E::size
                                    : a.fresh[part - 1] + (h * a.fs[part - 1][0] + r * a.fs[part - 1][1]) * E::size;
        lo = *reinterpret_cast<const u32x4*>(src + lo_off * E::size);
        hi = *reinterpret_cast<const u32x4*>(src + hi_off * E::size);
    }
    if (part != 2) {
        const char* crow = a.cos + r * a.cs[0] * E::size;
        const char* srow = a.sin + r * a.ss[0] * E::size;
        c_lo = *reinterpret_cast<const u32x4*>(crow + lo_off * E::size);
        c_hi = *reinterpret_cast<const u32x4*>(crow + hi_off * E::size);
        s_lo = *reinterpret_cast<const u32x4*>(srow + lo_off * E::size);
        s_hi = *reinterpret_cast<const u32x4*>(srow + hi_off * E::size);
    }
    if constexpr (PARTIALS && EPV == 8) {
        {  // the projection's output, rounded as its reduce kernel rounds it
            const int64_t col = a.part_col[part] + h * a.head_dim;
            float sl8[8], sh8[8];
            partial_sum8(a.src, r, col + lo_off, sl8);
            partial_sum8(a.src, r, col + hi_off, sh8);
            bits b[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) b[e] = E::from_float(sl8[e]);
            __builtin_memcpy(&lo, b, 16);
#pragma unroll
            for (int e = 0; e < EPV; ++e) b[e] = E::from_float(sh8[e]);
            __builtin_memcpy(&hi, b, 16);
        }
    }
    // per-head RMSNorm of a q or k row (uniform over the row's TPR lanes, so
    // the butterfly below runs on whole lane groups)
    if (NORM && part < 2) {
        const char* wrow = a.norm_w[part];
        const u32x4 w_lo = *reinterpret_cast<const u32x4*>(wrow + lo_off * E::size);
        const u32x4 w_hi = *reinterpret_cast<const u32x4*>(wrow + hi_off * E::size);
        norm_row<T>(lo, hi, w_lo, w_hi, tpr, a.head_dim, a.norm_eps[part]);
    }
    char* dst;
    if (part == 0) {
        dst = a.q_out + (h * a.qos[0] + r * a.qos[1]) * E::size;
    } else {
        const int kv = part - 1;
        if (pos < 0 || pos >= a.n_keys) return;
        dst = a.out[kv] + (h * a.os[kv][0] + pos * a.os[kv][1]) * E::size;
    }
    if (part == 2) {  // values: bit copy
        __builtin_nontemporal_store(lo, reinterpret_cast<u32x4*>(dst + lo_off * E::size));
        __builtin_nontemporal_store(hi, reinterpret_cast<u32x4*>(dst + hi_off * E::size));
        return;
    }
    bits xl[EPV], xh[EPV], cl[EPV], ch[EPV], sl[EPV], sh[EPV], ol[EPV], oh[EPV];
    __builtin_memcpy(xl, &lo, 16);
    __builtin_memcpy(xh, &hi, 16);
    __builtin_memcpy(cl, &c_lo, 16);
    __builtin_memcpy(ch, &c_hi, 16);
    __builtin_memcpy(sl, &s_lo, 16);
    __builtin_memcpy(sh, &s_hi, 16);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
        float yl, yh;
        rope_pair<T>(E::to_float(xl[e]), E::to_float(xh[e]), E::to_float(cl[e]), E::to_float(sl[e]),
                     E::to_float(ch[e]), E::to_float(sh[e]), yl, yh);
        ol[e] = E::from_float(yl);
        oh[e] = E::from_float(yh);
    }
    u32x4 out_lo, out_hi;
    __builtin_memcpy(&out_lo, ol, 16);
    __builtin_memcpy(&out_hi, oh, 16);
    __builtin_nontemporal_store(out_lo, reinterpret_cast<u32x4*>(dst + lo_off * E::size));
    __builtin_nontemporal_store(out_hi, reinterpret_cast<u32x4*>(dst + hi_off * E::size));
}

// Scalar path: one thread per (row, pair index i < head_dim/2), any strides.
template <typename T>
__global__ void __launch_bounds__(kThreads) fresh_scalar_kernel(FreshArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    const int half = a.head_dim >> 1;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t rows = (static_cast<int64_t>(a.n_q_heads) + 2 * a.n_kv_heads) * a.n_sel;
    if (idx >= rows * half) return;
    const int64_t g = idx / half;
    const int64_t i = idx - g * half;
    int part;
    int64_t h, r;
    decode_row(a, g, part, h, r);
    const bits* src = nullptr;
    bits* dst;
    int64_t sd = 1, dd;
    if (part == 0) {
        if (!a.src.base) src = reinterpret_cast<const bits*>(a.q) + h * a.qs[0] + r * a.qs[1];
        dst = reinterpret_cast<bits*>(a.q_out) + h * a.qos[0] + r * a.qos[1];
        sd = a.qs[2];
        dd = a.qos[2];
    } else {
        const int kv = part - 1;
        const int64_t pos = a.positions[r];
        if (pos < 0 || pos >= a.n_keys) return;
        if (!a.src.base) src = reinterpret_cast<const bits*>(a.fresh[kv]) + h * a.fs[kv][0] + r * a.fs[kv][1];
        dst = reinterpret_cast<bits*>(a.out[kv]) + h * a.os[kv][0] + pos * a.os[kv][1];
        sd = a.fs[kv][2];
        dd = a.os[kv][2];
    }
    bits lo, hi;
    if (src) {
        lo = src[i * sd];
        hi = src[(i + half) * sd];
    } else {  // the projection's output, rounded as its reduce kernel rounds it
        const int64_t col = a.part_col[part] + h * a.head_dim;
        lo = E::from_float(partial_sum1(a.src, r, col + i));
        hi = E::from_float(partial_sum1(a.src, r, col + i + half));
    }
    if (part == 2) {
        dst[i * dd] = lo;
        dst[(i + half) * dd] = hi;
        return;
    }
    const bits* cr = reinterpret_cast<const bits*>(a.cos) + r * a.cs[0];
    const bits* sr = reinterpret_cast<const bits*>(a.sin) + r * a.ss[0];
    float yl, yh;
    rope_pair<T>(E::to_float(lo), E::to_float(hi), E::to_float(cr[i * a.cs[1]]), E::to_float(sr[i * a.ss[1]]),
                 E::to_float(cr[(i + half) * a.cs[1]]), E::to_float(sr[(i + half) * a.ss[1]]), yl, yh);
    dst[i * dd] = E::from_float(yl);
    dst[(i + half) * dd] = E::from_float(yh);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Head dims the vector kernel serves: each half row splits into a power-of-two
// number (at most 64) of 16-byte chunks; *tpr_log2 = log2(chunks).
bool vec_head_dim(int32_t head_dim, int esize, int* tpr_log2) {
    const int64_t half_bytes = static_cast<int64_t>(head_dim / 2) * esize;
    if (half_bytes <= 0 || half_bytes % 16 != 0) return false;
    const int64_t chunks = half_bytes / 16;
    int t = 0;
    while ((int64_t(1) << t) < chunks) ++t;
    *tpr_log2 = t;
    return (int64_t(1) << t) == chunks && t <= 6;
}

// cos/sin tables the vector kernel reads: unit dim stride, 16-byte rows and bases.
bool vec_tables(const int64_t cs_strides[4], const void* cos, const void* sin, int esize) {
    return cs_strides[1] == 1 && cs_strides[3] == 1 && (cs_strides[0] * esize) % 16 == 0 &&
           (cs_strides[2] * esize) % 16 == 0 && aligned16(cos) && aligned16(sin);
}

template <typename T>
int launch(const FreshArgs& a, bool vec, int tpr_log2, hipStream_t s) {
    const int64_t rows = (static_cast<int64_t>(a.n_q_heads) + 2 * a.n_kv_heads) * a.n_sel;
    // fp16 rows always take the scalar kernel: the vector kernel's fp16
    // instantiation does not compile with packed fp32 instructions disabled.
    if constexpr (!std::is_same<T, f16_t>::value) {
        if (vec && (rows << tpr_log2) < (int64_t(1) << 31)) {
            const unsigned blocks = static_cast<unsigned>(ceil_div(rows << tpr_log2, kThreads));
            const bool partials = a.src.base != nullptr, norm = a.norm_w[0] != nullptr;
            if (partials && norm)
                fresh_vec_kernel<T, true, true><<<blocks, kThreads, 0, s>>>(a, tpr_log2);
            else if (partials)
                fresh_vec_kernel<T, true, false><<<blocks, kThreads, 0, s>>>(a, tpr_log2);
            else if (norm)
                fresh_vec_kernel<T, false, true><<<blocks, kThreads, 0, s>>>(a, tpr_log2);
            else
                fresh_vec_kernel<T, false, false><<<blocks, kThreads, 0, s>>>(a, tpr_log2);
            return launch_status();
        }
    }
    const int64_t threads = rows * (a.head_dim / 2);
    fresh_scalar_kernel<T><<<static_cast<unsigned>(ceil_div(threads, kThreads)), kThreads, 0, s>>>(a);
    return launch_status();
}

}  // namespace
}  // namespace kvr

namespace kvr {
namespace {

int rope_scatter_impl(const void* q, void* q_out, const void* fresh_k, const void* fresh_v, void* out_k, void* out_v,
                      const void* cos, const void* sin, const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                      int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, const int64_t strides[18],
                      const int64_t cs_strides[4], int32_t dtype, void* stream, const PartialSums* partial,
                      const int64_t* part_col, const void* q_norm = nullptr, const void* k_norm = nullptr,
                      float eps_q = 0.f, float eps_k = 0.f) {
    using namespace kvr;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_keys < 0) return KVR_E_INVALID_ARGUMENT;
    if (n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || (head_dim & 1)) return KVR_E_UNSUPPORTED_SHAPE;
    if (!strides || !cs_strides) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 18; ++i)
        if (strides[i] <= 0) return KVR_E_BAD_STRIDE;
    for (int i = 0; i < 4; ++i)
        if (cs_strides[i] < 0 || (i % 2 == 1 && cs_strides[i] == 0)) return KVR_E_BAD_STRIDE;
    if (n_sel == 0) return KVR_OK;
    if (partial) {
        if (!partial->base || partial->splits < 1 || !part_col) return KVR_E_NULL_POINTER;
        if (dtype_size(dtype) != 2 || n_sel > kPartialTileRows) return KVR_E_UNSUPPORTED_SHAPE;
    } else if (!q || !fresh_k || !fresh_v) {
        return KVR_E_NULL_POINTER;
    }
    if (!q_out || !out_k || !out_v || !cos || !sin || !positions) return KVR_E_NULL_POINTER;
    const bool norms = q_norm || k_norm;
    if (norms && (!q_norm || !k_norm)) return KVR_E_NULL_POINTER;
    if (norms && (!(eps_q >= 0.f) || !(eps_k >= 0.f) || eps_q == INFINITY || eps_k == INFINITY))
        return KVR_E_INVALID_ARGUMENT;

    FreshArgs a;
    a.q = static_cast<const char*>(q);
    a.q_out = static_cast<char*>(q_out);
    a.fresh[0] = static_cast<const char*>(fresh_k);
    a.fresh[1] = static_cast<const char*>(fresh_v);
    a.out[0] = static_cast<char*>(out_k);
    a.out[1] = static_cast<char*>(out_v);
    a.cos = static_cast<const char*>(cos);
    a.sin = static_cast<const char*>(sin);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = strides[i];
        a.qos[i] = strides[3 + i];
        a.fs[0][i] = strides[6 + i];
        a.fs[1][i] = strides[9 + i];
        a.os[0][i] = strides[12 + i];
        a.os[1][i] = strides[15 + i];
    }
    a.cs[0] = cs_strides[0];
    a.cs[1] = cs_strides[1];
    a.ss[0] = cs_strides[2];
    a.ss[1] = cs_strides[3];
    a.positions = positions;
    a.n_sel = n_sel;
    a.n_keys = n_keys;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.src = partial ? *partial : PartialSums{};
    for (int i = 0; i < 3; ++i) a.part_col[i] = part_col ? part_col[i] : 0;
    a.norm_w[0] = static_cast<const char*>(q_norm);
    a.norm_w[1] = static_cast<const char*>(k_norm);
    a.norm_eps[0] = eps_q;
    a.norm_eps[1] = eps_k;

    // Vector path: each half splits into a power-of-two number of 16-byte chunks.
    int tpr_log2 = 0;
    bool vec = vec_head_dim(head_dim, esize, &tpr_log2);
    for (int t = 0; t < 6 && vec; ++t) {
        const int64_t* st = strides + 3 * t;
        vec = st[2] == 1 && (st[0] * esize) % 16 == 0 && (st[1] * esize) % 16 == 0;
    }
    vec = vec && vec_tables(cs_strides, cos, sin, esize);
    vec = vec && aligned16(q) && aligned16(q_out) && aligned16(fresh_k) && aligned16(fresh_v) && aligned16(out_k) &&
          aligned16(out_v);
    // the norms run on the vector path only (their butterfly is over its lane
    // groups), which fp16 does not take (see launch); rope_norm_fold_ok is the
    // same condition minus the row layouts
    if (norms && (!vec || dtype == KVR_DTYPE_F16 || !aligned16(q_norm) || !aligned16(k_norm)))
        return KVR_E_UNSUPPORTED_SHAPE;

    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KVR_DTYPE_F32: return launch<f32_t>(a, vec, tpr_log2, s);
        case KVR_DTYPE_F16: return launch<f16_t>(a, vec, tpr_log2, s);
        default: return launch<bf16_t>(a, vec, tpr_log2, s);
    }
}

}  // namespace

bool rope_norm_fold_ok(int32_t head_dim, int32_t dtype, const void* q_norm, const void* k_norm,
                       const int64_t cs_strides[4], const void* cos, const void* sin) {
    const int esize = dtype_size(dtype);
    int tpr_log2 = 0;
    return esize != 0 && dtype != KVR_DTYPE_F16 && vec_head_dim(head_dim, esize, &tpr_log2) &&
           vec_tables(cs_strides, cos, sin, esize) && aligned16(q_norm) && aligned16(k_norm);
}

int rope_scatter_partials(const PartialSums& src, const int64_t part_col[3], void* q_out, void* out_k, void* out_v,
                          const void* cos, const void* sin, const int64_t* positions, int64_t n_sel,
                          int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys, int32_t head_dim,
                          const int64_t strides[18], const int64_t cs_strides[4], int32_t dtype, void* stream,
                          const void* q_norm, const void* k_norm, float eps_q, float eps_k) {
    return rope_scatter_impl(nullptr, q_out, nullptr, nullptr, out_k, out_v, cos, sin, positions, n_sel, n_q_heads,
                             n_kv_heads, n_keys, head_dim, strides, cs_strides, dtype, stream, &src, part_col,
                             q_norm, k_norm, eps_q, eps_k);
}

}  // namespace kvr

extern "C" int kvr_rope_scatter_kv(const void* q, void* q_out, const void* fresh_k, const void* fresh_v, void* out_k,
                                   void* out_v, const void* cos, const void* sin, const int64_t* positions,
                                   int64_t n_sel, int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys,
                                   int32_t head_dim, const int64_t strides[18], const int64_t cs_strides[4],
                                   int32_t dtype, void* stream) {
    return kvr::rope_scatter_impl(q, q_out, fresh_k, fresh_v, out_k, out_v, cos, sin, positions, n_sel, n_q_heads,
                                  n_kv_heads, n_keys, head_dim, strides, cs_strides, dtype, stream, nullptr, nullptr);
}

extern "C" int kvr_rope_scatter_kv_norm(const void* q, void* q_out, const void* fresh_k, const void* fresh_v,
                                        void* out_k, void* out_v, const void* cos, const void* sin,
                                        const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                                        int32_t n_kv_heads, int64_t n_keys, int32_t head_dim,
                                        const int64_t strides[18], const int64_t cs_strides[4], const void* q_norm,
                                        const void* k_norm, float eps_q, float eps_k, int32_t dtype, void* stream) {
    return kvr::rope_scatter_impl(q, q_out, fresh_k, fresh_v, out_k, out_v, cos, sin, positions, n_sel, n_q_heads,
                                  n_kv_heads, n_keys, head_dim, strides, cs_strides, dtype, stream, nullptr, nullptr,
                                  q_norm, k_norm, eps_q, eps_k);
}
