// Packed selected-query causal attention (GQA) for gfx950.
//
// Reference semantics: src/kv_cache_repair/kernels/packed_cache.py:47-67 with the
// boolean mask `key <= position` of packed_cache.py:205-207, i.e.
//   out[h, r] = softmax_{j <= pos[r]}(scale * q[h, r] . k[h / G, j]) @ v[h / G]
// and indexed_causal_attention (indexed_attention.py:207-241).
//
// Work decomposition (host schedule, kvr_attention_schedule):
//   selected rows are cut into row tiles of 16 rows; tile t needs keys
//   [0, pos[last row of t] + 1), cut into chunks of KC keys. One work item is
//   (tile, chunk). The grid is (work item, kv_head * head_groups); the
//   work-item index runs over blockIdx.y so that all blocks of one KV head land
//   on the same XCD (blocks are dealt to the 8 XCDs round-robin by linear id)
//   and that head's K/V stays in one L2.
// Tiles with one chunk write the final output; tiles with several chunks write
// fp32 partials (running max m in the log2 domain, sum l, unnormalised O) and a
// merge kernel combines them.
#include "kvr_internal.h"

#include <math.h>
#include <string.h>

namespace kvr {
namespace {

constexpr int32_t kMagic = 0x4B565253;  // "KVRS"
constexpr int32_t kVersion = 1;
constexpr int kHeader = 16;
constexpr int kRowTile = 16;  // selected rows per tile (MFMA N dimension)

enum Header {
    H_MAGIC = 0,
    H_VERSION,
    H_NSEL,
    H_NTILES,
    H_KC,
    H_NWORK,
    H_QT,
    H_NHG,
    H_HQ,
    H_HKV,
    H_D,
    H_KIND,
    H_NMULTI,
    H_NKEYS,
    H_DTYPE,
    H_RESERVED
};
enum Kind { KIND_GENERIC = 0, KIND_MFMA = 1 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct AttnArgs {
    const char* q;
    const char* k;
    const char* v;
    char* out;
    int64_t qs[3], ks[3], vs[3], os[3];  // {head,row,dim} element strides
    const int64_t* positions;
    const int32_t* sched;  // device schedule
    float* ws_ml;          // [Hq][n_work][16] (m, l)
    float* ws_o;           // [Hq][n_work][16][D]
    int64_t n_sel;
    int64_t n_keys;
    int32_t n_q_heads;
    int32_t group;  // G = Hq / Hkv
    int32_t qt;     // query heads per block
    int32_t n_head_groups;
    int32_t n_tiles;
    int32_t n_work;
    int32_t kc;
    int32_t head_dim;
    float scale_log2;  // scale * log2(e)
};

// Schedule accessors (device or host pointer to the same int32 layout).
__host__ __device__ inline const int32_t* tile_table(const int32_t* s) { return s + kHeader; }
__host__ __device__ inline const int32_t* work_table(const int32_t* s) { return s + kHeader + 2 * s[H_NTILES]; }

// ===========================================================================
// MFMA kernel
// ===========================================================================
template <typename T> struct mma_t;
template <> struct mma_t<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static inline __bf16 cvt(float x) { return static_cast<__bf16>(x); }
    __device__ static inline float back(__bf16 x) { return static_cast<float>(x); }
};
template <> struct mma_t<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __device__ static inline _Float16 cvt(float x) { return static_cast<_Float16>(x); }
    __device__ static inline float back(_Float16 x) { return static_cast<float>(x); }
};

constexpr int kMfmaThreads = 256;  // 4 waves
constexpr int kWaves = 4;
constexpr int kSub = 64;                  // keys per wave per iteration
constexpr int kIterKeys = kWaves * kSub;  // keys staged per iteration
constexpr int kPad = 8;                   // elements of row padding in LDS

template <int D>
struct MfmaSmem {
    static constexpr int ks_stride = D + kPad;          // Ks[key][d]
    static constexpr int vt_stride = kIterKeys + kPad;  // Vt[d][key]
    static constexpr int ks_elems = kIterKeys * ks_stride;
    static constexpr int vt_elems = D * vt_stride;
    static constexpr int stage_bytes = (ks_elems + vt_elems) * 2;
    static constexpr int red_bytes = kWaves * 4 * kRowTile * D * 4 + kWaves * 4 * kRowTile * 2 * 4;
    static constexpr int bytes = stage_bytes > red_bytes ? stage_bytes : red_bytes;
};

// QT query heads (query tiles of 16 rows) per wave; every wave of the block
// owns a different 64-key slice of each 256-key iteration.
template <typename T, int D, int QT, bool PRECISE_P>
__global__ void __launch_bounds__(kMfmaThreads)
attn_mfma_kernel(AttnArgs a) {
    using M = mma_t<T>;
    using v8 = typename M::v8;
    using S = MfmaSmem<D>;
    constexpr int DS = D / 32;  // k-steps of the QK^T MFMA
    constexpr int DT = D / 16;  // d tiles of the PV MFMA
    extern __shared__ __align__(16) char smem[];
    uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
    uint16_t* Vt = Ks + S::ks_elems;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lq = lane & 15;  // query column within the tile
    const int lj = lane >> 4;  // lane group 0..3

    const int32_t* wk = work_table(a.sched);
    const int work = blockIdx.y;
    const int tile = wk[2 * work];
    const int chunk = wk[2 * work + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int32_t* tt = tile_table(a.sched);
    const int n_chunks = tt[2 * tile + 1];

    const int64_t row0 = static_cast<int64_t>(tile) * kRowTile;
    const int64_t last_row = (row0 + kRowTile - 1 < a.n_sel) ? row0 + kRowTile - 1 : a.n_sel - 1;
    const int64_t kmax = a.positions[last_row] + 1;  // keys [0, kmax) needed by the tile
    const int64_t key_begin = static_cast<int64_t>(chunk) * a.kc;
    const int64_t key_end_raw = key_begin + a.kc;
    const int64_t key_end = key_end_raw < kmax ? key_end_raw : kmax;
    const int n_iter = static_cast<int>((key_end - key_begin + kIterKeys - 1) / kIterKeys);

    // Per-lane query row and its causal limit.
    const int64_t my_row = row0 + lq;
    const int64_t my_pos = (my_row < a.n_sel) ? a.positions[my_row] : int64_t(-1);
    const int q_head0 = kv_head * a.group + hg * QT;

    // Q fragments (B operand of S^T = K Q^T): lane holds q[row][32*ds + 8*lj .. +8].
    v8 qf[QT][DS];
#pragma unroll
    for (int h = 0; h < QT; ++h) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (my_row < a.n_sel) {
                const int64_t off = (q_head0 + h) * a.qs[0] + my_row * a.qs[1] + (32 * ds + 8 * lj) * a.qs[2];
                raw = *reinterpret_cast<const u32x4*>(a.q + off * 2);
            }
            qf[h][ds] = __builtin_bit_cast(v8, raw);
        }
    }

    f32x4 o[QT][DT];
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int h = 0; h < QT; ++h) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[h][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const char* kbase = a.k + static_cast<int64_t>(kv_head) * a.ks[0] * 2;
    const char* vbase = a.v + static_cast<int64_t>(kv_head) * a.vs[0] * 2;
    constexpr int C8 = D / 8;  // 16-byte chunks per row

    for (int it = 0; it < n_iter; ++it) {
        const int64_t it_key0 = key_begin + static_cast<int64_t>(it) * kIterKeys;
        // ---- stage K (row-major) and V (transposed) for 256 keys ----
#pragma unroll 4
        for (int cid = tid; cid < kIterKeys * C8; cid += kMfmaThreads) {
            const int kk = cid / C8;
            const int c8 = cid - kk * C8;
            const int64_t key = it_key0 + kk;
            u32x4 kr = {0u, 0u, 0u, 0u}, vr = {0u, 0u, 0u, 0u};
            if (key < key_end) {
                kr = *reinterpret_cast<const u32x4*>(kbase + (key * a.ks[1] + 8 * c8) * 2);
                vr = *reinterpret_cast<const u32x4*>(vbase + (key * a.vs[1] + 8 * c8) * 2);
            }
            *reinterpret_cast<u32x4*>(Ks + kk * S::ks_stride + 8 * c8) = kr;
            uint16_t vv[8];
            __builtin_memcpy(vv, &vr, 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) Vt[(8 * c8 + e) * S::vt_stride + kk] = vv[e];
        }
        __syncthreads();

        const int64_t sub_key0 = it_key0 + wave * kSub;
        if (sub_key0 < key_end) {
            const uint16_t* Kw = Ks + wave * kSub * S::ks_stride;
            // ---- S^T = K Q^T for 4 key tiles of 16 ----
            f32x4 st[QT][4];
#pragma unroll
            for (int h = 0; h < QT; ++h)
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) st[h][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const u32x4 raw =
                        *reinterpret_cast<const u32x4*>(Kw + (16 * kt + lq) * S::ks_stride + 32 * ds + 8 * lj);
                    const v8 kf = __builtin_bit_cast(v8, raw);
#pragma unroll
                    for (int h = 0; h < QT; ++h) st[h][kt] = M::mma(kf, qf[h][ds], st[h][kt]);
                }
            }
            // ---- online softmax (log2 domain), mask key > pos ----
            v8 p_hi[QT][2], p_lo[QT][2];
#pragma unroll
            for (int h = 0; h < QT; ++h) {
                float s[4][4];
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t key = sub_key0 + 16 * kt + 4 * lj + i;
                        const float x = (key <= my_pos) ? st[h][kt][i] * a.scale_log2 : -INFINITY;
                        s[kt][i] = x;
                        mx = fmaxf(mx, x);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const float m_new = fmaxf(m_run[h], mx);
                const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
                const float alpha = exp2f(m_run[h] - m_use);
                m_run[h] = m_new;
                float psum = 0.f;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = exp2f(s[kt][i] - m_use);
                        s[kt][i] = p;
                        psum += p;
                    }
                l_run[h] = l_run[h] * alpha + psum;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[h][dt] *= alpha;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x0 = s[2 * half][i];
                        const float x1 = s[2 * half + 1][i];
                        const auto h0 = M::cvt(x0);
                        const auto h1 = M::cvt(x1);
                        p_hi[h][half][i] = h0;
                        p_hi[h][half][4 + i] = h1;
                        if (PRECISE_P) {
                            p_lo[h][half][i] = M::cvt(x0 - M::back(h0));
                            p_lo[h][half][4 + i] = M::cvt(x1 - M::back(h1));
                        }
                    }
                }
            }
            // ---- O^T += V^T P^T ----
            const uint16_t* Vw = Vt + wave * kSub;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint16_t* vrow = Vw + (16 * dt + lq) * S::vt_stride + 32 * half + 4 * lj;
                    const u32x2 r0 = *reinterpret_cast<const u32x2*>(vrow);
                    const u32x2 r1 = *reinterpret_cast<const u32x2*>(vrow + 16);
                    const u32x4 raw = {r0[0], r0[1], r1[0], r1[1]};
                    const v8 vf = __builtin_bit_cast(v8, raw);
#pragma unroll
                    for (int h = 0; h < QT; ++h) {
                        o[h][dt] = M::mma(vf, p_hi[h][half], o[h][dt]);
                        if (PRECISE_P) o[h][dt] = M::mma(vf, p_lo[h][half], o[h][dt]);
                    }
                }
            }
        }
        __syncthreads();
    }

    // ---- combine the 4 waves of the block through LDS ----
    // lane partial sums -> per-query sums
#pragma unroll
    for (int h = 0; h < QT; ++h) {
        float l = l_run[h];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run[h] = l;
    }
    float* red_o = reinterpret_cast<float*>(smem);                 // [wave][QT][16][D]
    float* red_ml = red_o + kWaves * QT * kRowTile * D;            // [wave][QT][16][2]
    if (lj == 0) {
#pragma unroll
        for (int h = 0; h < QT; ++h) {
            red_ml[((wave * QT + h) * kRowTile + lq) * 2 + 0] = m_run[h];
            red_ml[((wave * QT + h) * kRowTile + lq) * 2 + 1] = l_run[h];
        }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < QT; ++h) {
        float mall = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mall = fmaxf(mall, red_ml[((w * QT + h) * kRowTile + lq) * 2]);
        const float m_use = (mall == -INFINITY) ? 0.f : mall;
        const float sc = exp2f(m_run[h] - m_use);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const f32x4 val = o[h][dt] * sc;
            *reinterpret_cast<f32x4*>(red_o + ((wave * QT + h) * kRowTile + lq) * D + 16 * dt + 4 * lj) = val;
        }
    }
    __syncthreads();

    // ---- final output (single chunk) or fp32 partial ----
    for (int e = tid; e < QT * kRowTile * D; e += kMfmaThreads) {
        const int h = e / (kRowTile * D);
        const int rem = e - h * (kRowTile * D);
        const int r = rem / D;
        const int d = rem - r * D;
        const int64_t row = row0 + r;
        if (row >= a.n_sel) continue;
        float mall = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mall = fmaxf(mall, red_ml[((w * QT + h) * kRowTile + r) * 2]);
        const float m_use = (mall == -INFINITY) ? 0.f : mall;
        float osum = 0.f, lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = red_ml[((w * QT + h) * kRowTile + r) * 2];
            const float lw = red_ml[((w * QT + h) * kRowTile + r) * 2 + 1];
            lsum += lw * exp2f(mw - m_use);
            osum += red_o[((w * QT + h) * kRowTile + r) * D + d];
        }
        const int q_head = q_head0 + h;
        if (n_chunks == 1) {
            const float val = osum / lsum;
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.out);
            dst[q_head * a.os[0] + row * a.os[1] + d * a.os[2]] = elem<T>::from_float(val);
        } else {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kRowTile + r;
            a.ws_o[slot * D + d] = osum;
            if (d == 0) {
                a.ws_ml[slot * 2 + 0] = mall;
                a.ws_ml[slot * 2 + 1] = lsum;
            }
        }
    }
}

// ===========================================================================
// Generic kernel (vector ALU; fp32 / fp16 / bf16, any head_dim <= 256).
// One 64-thread block per (work item, kv head, head group); thread = query
// (head h = tid / 16, row r = tid % 16); K/V staged in LDS as fp32.
// ===========================================================================
constexpr int kGenThreads = 64;
constexpr int kGenSub = 32;

template <typename T, int DMAX>
__global__ void __launch_bounds__(kGenThreads) attn_generic_kernel(AttnArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    extern __shared__ __align__(16) char smem[];
    const int D = a.head_dim;
    float* Kf = reinterpret_cast<float*>(smem);  // [kGenSub][D]
    float* Vf = Kf + kGenSub * D;                // [kGenSub][D]
    float* Sf = Vf + kGenSub * D;                // [kGenSub][kGenThreads] scores

    const int tid = threadIdx.x;
    const int32_t* wk = work_table(a.sched);
    const int work = blockIdx.y;
    const int tile = wk[2 * work];
    const int chunk = wk[2 * work + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int n_chunks = tile_table(a.sched)[2 * tile + 1];

    const int64_t row0 = static_cast<int64_t>(tile) * kRowTile;
    const int64_t last_row = (row0 + kRowTile - 1 < a.n_sel) ? row0 + kRowTile - 1 : a.n_sel - 1;
    const int64_t kmax = a.positions[last_row] + 1;
    const int64_t key_begin = static_cast<int64_t>(chunk) * a.kc;
    const int64_t key_end = (key_begin + a.kc < kmax) ? key_begin + a.kc : kmax;

    const int h = tid / kRowTile;
    const int r = tid - h * kRowTile;
    const bool live = h < a.qt && (row0 + r) < a.n_sel;
    const int64_t row = row0 + r;
    const int64_t pos = live ? a.positions[row] : int64_t(-1);
    const int q_head = kv_head * a.group + hg * a.qt + h;

    const bits* qp = reinterpret_cast<const bits*>(a.q);
    float q[DMAX], acc[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
        q[d] = (live && d < D) ? E::to_float(qp[q_head * a.qs[0] + row * a.qs[1] + d * a.qs[2]]) : 0.f;
        acc[d] = 0.f;
    }
    float m_run = -INFINITY, l_run = 0.f;
    const bits* kp = reinterpret_cast<const bits*>(a.k) + static_cast<int64_t>(kv_head) * a.ks[0];
    const bits* vp = reinterpret_cast<const bits*>(a.v) + static_cast<int64_t>(kv_head) * a.vs[0];

    for (int64_t k0 = key_begin; k0 < key_end; k0 += kGenSub) {
        for (int e = tid; e < kGenSub * D; e += kGenThreads) {
            const int kk = e / D;
            const int d = e - kk * D;
            const int64_t key = k0 + kk;
            float kv = 0.f, vv = 0.f;
            if (key < key_end) {
                kv = E::to_float(kp[key * a.ks[1] + d * a.ks[2]]);
                vv = E::to_float(vp[key * a.vs[1] + d * a.vs[2]]);
            }
            Kf[e] = kv;
            Vf[e] = vv;
        }
        __syncthreads();
        float mx = -INFINITY;
        for (int kk = 0; kk < kGenSub; ++kk) {
            float dot = 0.f;
#pragma unroll
            for (int d = 0; d < DMAX; ++d)
                if (d < D) dot += q[d] * Kf[kk * D + d];
            const int64_t key = k0 + kk;
            const float sv = (key <= pos && key < key_end) ? dot * a.scale_log2 : -INFINITY;
            Sf[kk * kGenThreads + tid] = sv;
            mx = fmaxf(mx, sv);
        }
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = exp2f(m_run - m_use);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DMAX; ++d) acc[d] *= alpha;
        for (int kk = 0; kk < kGenSub; ++kk) {
            const float p = exp2f(Sf[kk * kGenThreads + tid] - m_use);
            l_run += p;
#pragma unroll
            for (int d = 0; d < DMAX; ++d)
                if (d < D) acc[d] += p * Vf[kk * D + d];
        }
        __syncthreads();
    }
    if (!live) return;
    if (n_chunks == 1) {
        bits* op = reinterpret_cast<bits*>(a.out);
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) op[q_head * a.os[0] + row * a.os[1] + d * a.os[2]] = E::from_float(acc[d] / l_run);
    } else {
        const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kRowTile + r;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) a.ws_o[slot * D + d] = acc[d];
        a.ws_ml[slot * 2 + 0] = m_run;
        a.ws_ml[slot * 2 + 1] = l_run;
    }
}

// ===========================================================================
// Merge of multi-chunk tiles: grid (tile, q_head), 256 threads over 16 x D.
// ===========================================================================
template <typename T>
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    const int tile = blockIdx.x;
    const int q_head = blockIdx.y;
    const int32_t* tt = tile_table(a.sched);
    const int base = tt[2 * tile];
    const int n_chunks = tt[2 * tile + 1];
    if (n_chunks <= 1) return;
    const int D = a.head_dim;
    const int64_t row0 = static_cast<int64_t>(tile) * kRowTile;
    for (int e = threadIdx.x; e < kRowTile * D; e += 256) {
        const int r = e / D;
        const int d = e - r * D;
        const int64_t row = row0 + r;
        if (row >= a.n_sel) continue;
        float mall = -INFINITY;
        for (int c = 0; c < n_chunks; ++c) {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + base + c) * kRowTile + r;
            mall = fmaxf(mall, a.ws_ml[slot * 2]);
        }
        const float m_use = (mall == -INFINITY) ? 0.f : mall;
        float osum = 0.f, lsum = 0.f;
        for (int c = 0; c < n_chunks; ++c) {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + base + c) * kRowTile + r;
            const float w = exp2f(a.ws_ml[slot * 2] - m_use);
            lsum += a.ws_ml[slot * 2 + 1] * w;
            osum += a.ws_o[slot * D + d] * w;
        }
        bits* op = reinterpret_cast<bits*>(a.out);
        op[q_head * a.os[0] + row * a.os[1] + d * a.os[2]] = E::from_float(osum / lsum);
    }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
int pick_qt(int group) {
    if (group % 4 == 0) return 4;
    if (group % 2 == 0) return 2;
    return 1;
}

bool mfma_eligible(int32_t dtype, int32_t head_dim) {
    return (dtype == KVR_DTYPE_BF16 || dtype == KVR_DTYPE_F16) && (head_dim == 64 || head_dim == 128);
}

int generic_dmax(int32_t head_dim) {
    if (head_dim <= 32) return 32;
    if (head_dim <= 64) return 64;
    if (head_dim <= 128) return 128;
    if (head_dim <= 256) return 256;
    return 0;
}

// Opt a kernel into more than 64 KiB of dynamic LDS once per process.
template <typename F>
bool allow_lds(F fn, size_t bytes) {
    if (bytes <= 65536) return true;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes)) == hipSuccess;
}

template <typename T, int D, int QT, bool P>
int launch_mfma_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    const size_t smem = MfmaSmem<D>::bytes;
    static const bool ok = allow_lds(attn_mfma_kernel<T, D, QT, P>, smem);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_mfma_kernel<T, D, QT, P><<<grid, kMfmaThreads, smem, s>>>(a);
    return launch_status();
}

// P always enters PV as a hi+lo pair (PRECISE_P = true).
template <typename T, int D>
int launch_mfma(const AttnArgs& a, int qt, dim3 grid, hipStream_t s) {
    if (qt == 4) return launch_mfma_inst<T, D, 4, true>(a, grid, s);
    if (qt == 2) return launch_mfma_inst<T, D, 2, true>(a, grid, s);
    return launch_mfma_inst<T, D, 1, true>(a, grid, s);
}

template <typename T, int DMAX>
int launch_generic_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    const size_t smem = (static_cast<size_t>(2) * kGenSub * DMAX + static_cast<size_t>(kGenSub) * kGenThreads) * sizeof(float);
    static const bool ok = allow_lds(attn_generic_kernel<T, DMAX>, smem);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_generic_kernel<T, DMAX><<<grid, kGenThreads, smem, s>>>(a);
    return launch_status();
}

template <typename T>
int launch_generic(const AttnArgs& a, int dmax, dim3 grid, hipStream_t s) {
    switch (dmax) {
        case 32: return launch_generic_inst<T, 32>(a, grid, s);
        case 64: return launch_generic_inst<T, 64>(a, grid, s);
        case 128: return launch_generic_inst<T, 128>(a, grid, s);
        default: return launch_generic_inst<T, 256>(a, grid, s);
    }
}

template <typename T>
int launch_merge(const AttnArgs& a, hipStream_t s) {
    dim3 grid(a.n_tiles, a.n_q_heads);
    attn_merge_kernel<T><<<grid, 256, 0, s>>>(a);
    return launch_status();
}

}  // namespace
}  // namespace kvr

using namespace kvr;

extern "C" int64_t kvr_attention_schedule(const int64_t* positions, int64_t n_sel, int64_t n_keys, int32_t n_q_heads,
                                          int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t chunk_keys,
                                          int32_t* schedule, int64_t capacity) {
    if (n_sel < 0 || n_keys < 0 || n_sel > n_keys) return KVR_E_INVALID_ARGUMENT;
    if (n_keys >= (int64_t(1) << 31) || n_sel >= (int64_t(1) << 31)) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads) return KVR_E_UNSUPPORTED_SHAPE;
    if (head_dim <= 0 || dtype_size(dtype) == 0) return dtype_size(dtype) ? KVR_E_UNSUPPORTED_SHAPE
                                                                          : KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel > 0 && !positions) return KVR_E_NULL_POINTER;
    for (int64_t i = 0; i < n_sel; ++i) {
        if (positions[i] < 0 || positions[i] >= n_keys) return KVR_E_INVALID_ARGUMENT;
        if (i && positions[i] <= positions[i - 1]) return KVR_E_INVALID_ARGUMENT;
    }
    const bool mfma = mfma_eligible(dtype, head_dim);
    if (!mfma && generic_dmax(head_dim) == 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (chunk_keys < 0 || (chunk_keys > 0 && chunk_keys % (mfma ? kIterKeys : kGenSub) != 0))
        return KVR_E_INVALID_ARGUMENT;
    const int group = n_q_heads / n_kv_heads;
    const int qt = pick_qt(group);
    const int n_head_groups = group / qt;
    const int64_t n_tiles = (n_sel + kRowTile - 1) / kRowTile;

    // Chunk size: the largest multiple of the iteration size that still gives
    // at least `target` blocks; tiles whose key range fits in one chunk need
    // no merge.
    const int unit = mfma ? kIterKeys : kGenSub;
    int64_t kc = chunk_keys;
    if (kc == 0) {
        const int64_t target = 512;
        const int64_t heads = static_cast<int64_t>(n_kv_heads) * n_head_groups;
        int64_t maxk = unit;
        for (int64_t t = 0; t < n_tiles; ++t) {
            const int64_t last = (t + 1) * kRowTile - 1 < n_sel ? (t + 1) * kRowTile - 1 : n_sel - 1;
            maxk = positions[last] + 1 > maxk ? positions[last] + 1 : maxk;
        }
        kc = unit;
        for (int64_t cand = unit; cand <= ((maxk + unit - 1) / unit) * unit; cand *= 2) {
            int64_t blocks = 0;
            for (int64_t t = 0; t < n_tiles; ++t) {
                const int64_t last = (t + 1) * kRowTile - 1 < n_sel ? (t + 1) * kRowTile - 1 : n_sel - 1;
                blocks += (positions[last] + 1 + cand - 1) / cand;
            }
            if (blocks * heads >= target) kc = cand;
        }
        if (kc > (int64_t(1) << 30)) kc = int64_t(1) << 30;
    }
    int64_t n_work = 0, n_multi = 0;
    for (int64_t t = 0; t < n_tiles; ++t) {
        const int64_t last = (t + 1) * kRowTile - 1 < n_sel ? (t + 1) * kRowTile - 1 : n_sel - 1;
        const int64_t c = (positions[last] + 1 + kc - 1) / kc;
        n_work += c;
        n_multi += c > 1;
    }
    if (n_work > 65535) return KVR_E_UNSUPPORTED_SHAPE;  // grid.y limit
    const int64_t need = kHeader + 2 * n_tiles + 2 * n_work;
    if (!schedule) return need;
    if (capacity < need) return KVR_E_CAPACITY;
    int32_t* h = schedule;
    memset(h, 0, sizeof(int32_t) * kHeader);
    h[H_MAGIC] = kMagic;
    h[H_VERSION] = kVersion;
    h[H_NSEL] = static_cast<int32_t>(n_sel);
    h[H_NTILES] = static_cast<int32_t>(n_tiles);
    h[H_KC] = static_cast<int32_t>(kc);
    h[H_NWORK] = static_cast<int32_t>(n_work);
    h[H_QT] = qt;
    h[H_NHG] = n_head_groups;
    h[H_HQ] = n_q_heads;
    h[H_HKV] = n_kv_heads;
    h[H_D] = head_dim;
    h[H_KIND] = mfma ? KIND_MFMA : KIND_GENERIC;
    h[H_NMULTI] = static_cast<int32_t>(n_multi);
    h[H_NKEYS] = static_cast<int32_t>(n_keys);
    h[H_DTYPE] = dtype;
    int32_t* tiles = h + kHeader;
    int32_t* works = tiles + 2 * n_tiles;
    int64_t w = 0;
    for (int64_t t = 0; t < n_tiles; ++t) {
        const int64_t last = (t + 1) * kRowTile - 1 < n_sel ? (t + 1) * kRowTile - 1 : n_sel - 1;
        const int64_t c = (positions[last] + 1 + kc - 1) / kc;
        tiles[2 * t] = static_cast<int32_t>(w);
        tiles[2 * t + 1] = static_cast<int32_t>(c);
        for (int64_t i = 0; i < c; ++i, ++w) {
            works[2 * w] = static_cast<int32_t>(t);
            works[2 * w + 1] = static_cast<int32_t>(i);
        }
    }
    return need;
}

extern "C" int64_t kvr_attention_workspace_bytes(const int32_t* schedule, int64_t schedule_len, int32_t n_q_heads,
                                                 int32_t head_dim) {
    if (!schedule || schedule_len < kHeader || schedule[H_MAGIC] != kMagic || schedule[H_VERSION] != kVersion)
        return KVR_E_BAD_SCHEDULE;
    if (schedule[H_HQ] != n_q_heads || schedule[H_D] != head_dim) return KVR_E_BAD_SCHEDULE;
    if (schedule[H_NMULTI] == 0) return 0;
    return static_cast<int64_t>(n_q_heads) * schedule[H_NWORK] * kRowTile * (head_dim + 2) * 4;
}

extern "C" int kvr_packed_causal_attention(const void* q, const void* k, const void* v, void* out,
                                           const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                                           int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, float scale,
                                           const int64_t strides[12], const int32_t* schedule, int64_t schedule_len,
                                           const int32_t* host_schedule, void* workspace, int64_t workspace_bytes,
                                           int32_t dtype, void* stream) {
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_keys < 0 || n_sel > n_keys) return KVR_E_INVALID_ARGUMENT;
    if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || head_dim <= 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (!strides) return KVR_E_NULL_POINTER;
    for (int i = 0; i < 12; ++i)
        if (strides[i] <= 0) return KVR_E_BAD_STRIDE;
    if (!(scale == scale) || scale == INFINITY || scale == -INFINITY) return KVR_E_INVALID_ARGUMENT;
    if (n_sel == 0) return KVR_OK;
    if (!q || !k || !v || !out || !positions || !schedule || !host_schedule) return KVR_E_NULL_POINTER;
    const int32_t* hs = host_schedule;
    if (schedule_len < kHeader || hs[H_MAGIC] != kMagic || hs[H_VERSION] != kVersion) return KVR_E_BAD_SCHEDULE;
    if (hs[H_NSEL] != n_sel || hs[H_HQ] != n_q_heads || hs[H_HKV] != n_kv_heads || hs[H_D] != head_dim ||
        hs[H_NKEYS] != n_keys || hs[H_DTYPE] != dtype)
        return KVR_E_BAD_SCHEDULE;
    if (schedule_len != kHeader + 2 * static_cast<int64_t>(hs[H_NTILES]) + 2 * static_cast<int64_t>(hs[H_NWORK]))
        return KVR_E_BAD_SCHEDULE;
    const int64_t ws_need = kvr_attention_workspace_bytes(hs, schedule_len, n_q_heads, head_dim);
    if (ws_need < 0) return KVR_E_BAD_SCHEDULE;
    if (workspace_bytes < ws_need || (ws_need > 0 && !workspace)) return KVR_E_WORKSPACE_TOO_SMALL;

    AttnArgs a;
    memset(&a, 0, sizeof(a));
    a.q = static_cast<const char*>(q);
    a.k = static_cast<const char*>(k);
    a.v = static_cast<const char*>(v);
    a.out = static_cast<char*>(out);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = strides[i];
        a.ks[i] = strides[3 + i];
        a.vs[i] = strides[6 + i];
        a.os[i] = strides[9 + i];
    }
    a.positions = positions;
    a.sched = schedule;
    a.n_sel = n_sel;
    a.n_keys = n_keys;
    a.n_q_heads = n_q_heads;
    a.group = n_q_heads / n_kv_heads;
    a.qt = hs[H_QT];
    a.n_head_groups = hs[H_NHG];
    a.n_tiles = hs[H_NTILES];
    a.n_work = hs[H_NWORK];
    a.kc = hs[H_KC];
    a.head_dim = head_dim;
    a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
    if (ws_need > 0) {
        a.ws_ml = static_cast<float*>(workspace);
        a.ws_o = a.ws_ml + static_cast<int64_t>(n_q_heads) * a.n_work * kRowTile * 2;
    }
    if (a.qt * a.n_head_groups != a.group) return KVR_E_BAD_SCHEDULE;

    hipStream_t s = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(n_kv_heads * a.n_head_groups), static_cast<unsigned>(a.n_work));
    // The MFMA kernel reads 16-byte fragments of q/k/v: unit dim strides and
    // 16-byte aligned rows. Other layouts (strided slices, odd offsets) take
    // the generic kernel, whose chunking (multiples of 32 keys) is compatible
    // with every MFMA schedule (multiples of 256 keys).
    bool use_mfma = hs[H_KIND] == KIND_MFMA;
    if (use_mfma && !mfma_eligible(dtype, head_dim)) return KVR_E_BAD_SCHEDULE;
    for (int t = 0; t < 3 && use_mfma; ++t) {
        const int64_t* st3 = strides + 3 * t;
        if (st3[2] != 1 || (st3[0] * esize) % 16 || (st3[1] * esize) % 16) use_mfma = false;
    }
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u)
        use_mfma = false;
    int st;
    if (use_mfma) {
        if (dtype == KVR_DTYPE_BF16)
            st = head_dim == 128 ? launch_mfma<bf16_t, 128>(a, a.qt, grid, s)
                                 : launch_mfma<bf16_t, 64>(a, a.qt, grid, s);
        else
            st = head_dim == 128 ? launch_mfma<f16_t, 128>(a, a.qt, grid, s)
                                 : launch_mfma<f16_t, 64>(a, a.qt, grid, s);
    } else {
        const int dmax = generic_dmax(head_dim);
        if (dmax == 0) return KVR_E_UNSUPPORTED_SHAPE;
        switch (dtype) {
            case KVR_DTYPE_F32: st = launch_generic<f32_t>(a, dmax, grid, s); break;
            case KVR_DTYPE_F16: st = launch_generic<f16_t>(a, dmax, grid, s); break;
            default: st = launch_generic<bf16_t>(a, dmax, grid, s); break;
        }
    }
    if (st != KVR_OK || hs[H_NMULTI] == 0) return st;
    switch (dtype) {
        case KVR_DTYPE_F32: return launch_merge<f32_t>(a, s);
        case KVR_DTYPE_F16: return launch_merge<f16_t>(a, s);
        default: return launch_merge<bf16_t>(a, s);
    }
}
