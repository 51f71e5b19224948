// Packed selected-query causal attention (GQA) for gfx950.
//
// Reference semantics: src/kv_cache_repair/kernels/packed_cache.py:47-67 with the
// boolean mask `key <= position` of packed_cache.py:205-207, i.e.
//   out[h, r] = softmax_{j <= pos[r]}(scale * q[h, r] . k[h / G, j]) @ v[h / G]
// and indexed_causal_attention (indexed_attention.py:207-241).
//
// Work decomposition (host schedule, kvr_attention_schedule):
//   selected rows are cut into groups of 64 (four tiles of 16 rows); group g
//   needs keys [0, pos[last row of g] + 1), cut into chunks of KC keys. One
//   block handles one (KV head, head group, row group, key chunk): it stages
//   the chunk's K/V once in LDS, 64 keys at a time, double-buffered, and each
//   of its four waves attends one row tile (QT query heads x 16 rows) to it.
//   Grid x = KV head x head group, so every block of one KV head lands on the
//   same XCD (blocks are dealt round-robin over the 8 XCDs by linear id) and
//   that head's K/V and partials stay in one L2.
// Groups with one chunk write the final output; groups with several chunks
// write fp32 partials (running max m in the log2 domain, sum l, unnormalised
// O) that a merge kernel combines.
#include "kvr_internal.h"

#include <math.h>
#include <string.h>

#include <utility>

namespace kvr {
namespace {

constexpr int32_t kMagic = 0x4B565253;  // "KVRS"
constexpr int32_t kVersion = 2;
constexpr int kHeader = 16;
constexpr int kRowTile = 16;               // rows per MFMA tile
constexpr int kTilesPerGroup = 4;          // one wave per tile
constexpr int kGroupRows = kRowTile * kTilesPerGroup;
constexpr int kSub = 64;                   // keys per LDS sub-tile
constexpr int kMaxChunksPerGroup = 1024;   // merge weights fit in LDS

enum Header {
    H_MAGIC = 0,
    H_VERSION,
    H_NSEL,
    H_NGROUPS,
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
    H_MAXCHUNKS
};
enum Kind { KIND_GENERIC = 0, KIND_MFMA = 1 };

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const char* q;
    const char* k;
    const char* v;
    char* out;
    int64_t qs[3], ks[3], vs[3], os[3];  // {head,row,dim} element strides
    const int64_t* positions;
    const int32_t* sched;  // device schedule
    float* ws_ml;          // [Hq][n_work][64] (m, l)
    float* ws_o;           // [Hq][n_work][64][D]
    int64_t n_sel;
    int64_t n_keys;
    int32_t n_q_heads;
    int32_t group;  // G = Hq / Hkv
    int32_t qt;     // query heads per wave
    int32_t n_head_groups;
    int32_t n_groups;
    int32_t n_work;
    int32_t kc;
    int32_t head_dim;
    float scale_log2;  // scale * log2(e)
};

// Schedule accessors (device or host pointer to the same int32 layout).
__host__ __device__ inline const int32_t* group_table(const int32_t* s) { return s + kHeader; }
__host__ __device__ inline const int32_t* work_table(const int32_t* s) { return s + kHeader + 2 * s[H_NGROUPS]; }

// Causal key limit (exclusive) of rows [first, first + count) clipped to n_sel.
__device__ inline int64_t rows_kmax(const AttnArgs& a, int64_t first, int64_t count) {
    if (first >= a.n_sel) return 0;
    const int64_t last = (first + count - 1 < a.n_sel) ? first + count - 1 : a.n_sel - 1;
    return a.positions[last] + 1;
}

// ===========================================================================
// MFMA kernel
// ===========================================================================
template <typename T> struct mma_t;
template <> struct mma_t<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    typedef __bf16 scalar;
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static inline scalar cvt(float x) { return static_cast<scalar>(x); }
    __device__ static inline float back(scalar x) { return static_cast<float>(x); }
};
template <> struct mma_t<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    typedef _Float16 scalar;
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __device__ static inline scalar cvt(float x) { return static_cast<scalar>(x); }
    __device__ static inline float back(scalar x) { return static_cast<float>(x); }
};

constexpr int kMfmaThreads = 256;  // 4 waves, one per row tile
constexpr int kPad = 8;            // elements of LDS row padding (16 bytes)

template <int D>
struct MfmaSmem {
    static constexpr int stride = D + kPad;          // elements per staged key row
    static constexpr int tile_elems = kSub * stride;  // one K or V sub-tile
    static constexpr int bytes = 2 /*buffers*/ * 2 /*K,V*/ * tile_elems * 2;
    static constexpr int chunks = kSub * D / 8;              // 16-byte pieces per sub-tile
    static constexpr int per_thread = chunks / kMfmaThreads;  // per tensor
};

// Global -> register prefetch of one 64-key K/V sub-tile (zero beyond `end`).
template <int D>
__device__ inline void load_subtile(const AttnArgs& a, const char* kbase, const char* vbase, int64_t key0,
                                    int64_t end, int tid, u32x4* kr, u32x4* vr) {
    using S = MfmaSmem<D>;
    constexpr int C8 = D / 8;
#pragma unroll
    for (int p = 0; p < S::per_thread; ++p) {
        const int cid = tid + p * kMfmaThreads;
        const int kk = cid / C8;
        const int c8 = cid - kk * C8;
        const int64_t key = key0 + kk;
        kr[p] = u32x4{0u, 0u, 0u, 0u};
        vr[p] = u32x4{0u, 0u, 0u, 0u};
        if (key < end) {
            kr[p] = *reinterpret_cast<const u32x4*>(kbase + (key * a.ks[1] + 8 * c8) * 2);
            vr[p] = *reinterpret_cast<const u32x4*>(vbase + (key * a.vs[1] + 8 * c8) * 2);
        }
    }
}

template <int D>
__device__ inline void store_subtile(uint16_t* Ks, uint16_t* Vs, int tid, const u32x4* kr, const u32x4* vr) {
    using S = MfmaSmem<D>;
    constexpr int C8 = D / 8;
#pragma unroll
    for (int p = 0; p < S::per_thread; ++p) {
        const int cid = tid + p * kMfmaThreads;
        const int kk = cid / C8;
        const int c8 = cid - kk * C8;
        *reinterpret_cast<u32x4*>(Ks + kk * S::stride + 8 * c8) = kr[p];
        *reinterpret_cast<u32x4*>(Vs + kk * S::stride + 8 * c8) = vr[p];
    }
}

// Each wave: QT query heads x the 16 rows of its tile. S^T = K Q^T (keys on the
// MFMA M axis) so each lane holds 4 keys of one query, and the PV MFMA takes
// P^T straight from those registers: O^T += V^T P^T.
template <typename T, int D, int QT>
__global__ void __launch_bounds__(kMfmaThreads)
attn_mfma_kernel(AttnArgs a) {
    using M = mma_t<T>;
    using v8 = typename M::v8;
    using S = MfmaSmem<D>;
    constexpr int DS = D / 32;  // k-steps of the QK^T MFMA
    constexpr int DT = D / 16;  // d tiles of the PV MFMA
    extern __shared__ __align__(16) char smem[];
    uint16_t* lds = reinterpret_cast<uint16_t*>(smem);  // [buf][K|V][64][stride]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lq = lane & 15;  // query row within the tile
    const int lj = lane >> 4;  // lane group 0..3

    const int32_t* wk = work_table(a.sched);
    const int work = blockIdx.y;
    const int grp = wk[2 * work];
    const int chunk = wk[2 * work + 1];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int q_head0 = kv_head * a.group + hg * QT;

    const int64_t group_row0 = static_cast<int64_t>(grp) * kGroupRows;
    const int64_t key_begin = static_cast<int64_t>(chunk) * a.kc;
    const int64_t group_kmax = rows_kmax(a, group_row0, kGroupRows);
    const int64_t key_end = (key_begin + a.kc < group_kmax) ? key_begin + a.kc : group_kmax;
    const int n_sub = static_cast<int>((key_end - key_begin + kSub - 1) / kSub);

    const int64_t tile_row0 = group_row0 + wave * kRowTile;
    const int64_t tile_kmax = rows_kmax(a, tile_row0, kRowTile);  // 0 for an empty tile
    const int64_t my_row = tile_row0 + lq;
    const int64_t my_pos = (my_row < a.n_sel) ? a.positions[my_row] : int64_t(-1);

    // Q fragments (B operand of S^T = K Q^T): lane holds q[row][32*ds + 8*lj .. +8].
    v8 qf[QT][DS];
#pragma unroll
    for (int h = 0; h < QT; ++h)
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (my_row < a.n_sel) {
                const int64_t off = (q_head0 + h) * a.qs[0] + my_row * a.qs[1] + (32 * ds + 8 * lj) * a.qs[2];
                raw = *reinterpret_cast<const u32x4*>(a.q + off * 2);
            }
            qf[h][ds] = __builtin_bit_cast(v8, raw);
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
    u32x4 kr[S::per_thread], vr[S::per_thread];
    if (n_sub > 0) {
        load_subtile<D>(a, kbase, vbase, key_begin, key_end, tid, kr, vr);
        store_subtile<D>(lds, lds + S::tile_elems, tid, kr, vr);
    }

    for (int s = 0; s < n_sub; ++s) {
        const int64_t sub_key0 = key_begin + static_cast<int64_t>(s) * kSub;
        const bool more = s + 1 < n_sub;
        if (more) load_subtile<D>(a, kbase, vbase, sub_key0 + kSub, key_end, tid, kr, vr);
        __syncthreads();  // sub-tile s is staged; buffer (s+1)%2 is free
        const uint16_t* Kb = lds + (s & 1) * 2 * S::tile_elems;
        const uint16_t* Vb = Kb + S::tile_elems;

        if (sub_key0 < tile_kmax) {
            // ---- S^T = K Q^T for 4 key tiles of 16 ----
            f32x4 st[QT][4];
#pragma unroll
            for (int h = 0; h < QT; ++h)
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) st[h][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const u32x4 raw =
                        *reinterpret_cast<const u32x4*>(Kb + (16 * kt + lq) * S::stride + 32 * ds + 8 * lj);
                    const v8 kf = __builtin_bit_cast(v8, raw);
#pragma unroll
                    for (int h = 0; h < QT; ++h) st[h][kt] = M::mma(kf, qf[h][ds], st[h][kt]);
                }
            // ---- online softmax (log2 domain), mask key > pos ----
            v8 p_hi[QT][2], p_lo[QT][2];
#pragma unroll
            for (int h = 0; h < QT; ++h) {
                float sc[4][4];
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t key = sub_key0 + 16 * kt + 4 * lj + i;
                        const float x = (key <= my_pos) ? st[h][kt][i] * a.scale_log2 : -INFINITY;
                        sc[kt][i] = x;
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
                        const float p = exp2f(sc[kt][i] - m_use);
                        sc[kt][i] = p;
                        psum += p;
                    }
                l_run[h] = l_run[h] * alpha + psum;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[h][dt] *= alpha;
#pragma unroll
                for (int half = 0; half < 2; ++half)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x0 = sc[2 * half][i];
                        const float x1 = sc[2 * half + 1][i];
                        const auto h0 = M::cvt(x0);
                        const auto h1 = M::cvt(x1);
                        p_hi[h][half][i] = h0;
                        p_hi[h][half][4 + i] = h1;
                        p_lo[h][half][i] = M::cvt(x0 - M::back(h0));
                        p_lo[h][half][4 + i] = M::cvt(x1 - M::back(h1));
                    }
            }
            // ---- O^T += V^T P^T: A = V^T gathered from the row-major tile ----
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint16_t* col = Vb + (32 * half + 4 * lj) * S::stride + 16 * dt + lq;
                    uint16_t g[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        g[i] = col[i * S::stride];
                        g[4 + i] = col[(16 + i) * S::stride];
                    }
                    v8 vf;
                    __builtin_memcpy(&vf, g, 16);
#pragma unroll
                    for (int h = 0; h < QT; ++h) {
                        o[h][dt] = M::mma(vf, p_hi[h][half], o[h][dt]);
                        o[h][dt] = M::mma(vf, p_lo[h][half], o[h][dt]);
                    }
                }
        }
        if (more) store_subtile<D>(lds + ((s + 1) & 1) * 2 * S::tile_elems,
                                   lds + ((s + 1) & 1) * 2 * S::tile_elems + S::tile_elems, tid, kr, vr);
    }

    // ---- epilogue: per-query sums, then final output or fp32 partial ----
#pragma unroll
    for (int h = 0; h < QT; ++h) {
        float l = l_run[h];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run[h] = l;
    }
    if (my_row >= a.n_sel) return;
    const int r = static_cast<int>(my_row - group_row0);
#pragma unroll
    for (int h = 0; h < QT; ++h) {
        const int q_head = q_head0 + h;
        if (n_chunks == 1) {
            const float inv = 1.f / l_run[h];
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + q_head * a.os[0] + my_row * a.os[1];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    dst[(16 * dt + 4 * lj + i) * a.os[2]] = elem<T>::from_float(o[h][dt][i] * inv);
        } else {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kGroupRows + r;
            float* po = a.ws_o + slot * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * lj) = o[h][dt];
            if (lj == 0) {
                a.ws_ml[slot * 2 + 0] = m_run[h];
                a.ws_ml[slot * 2 + 1] = l_run[h];
            }
        }
    }
}

// ===========================================================================
// Generic kernel (vector ALU; fp32 / fp16 / bf16, any head_dim <= 256).
// Same work items as the MFMA kernel. 256 threads: thread t owns query
// (tile t/64, head (t%64)/16, row t%16); K/V staged in LDS as fp32.
// ===========================================================================
constexpr int kGenThreads = 256;
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
    const int grp = wk[2 * work];
    const int chunk = wk[2 * work + 1];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;

    const int64_t group_row0 = static_cast<int64_t>(grp) * kGroupRows;
    const int64_t key_begin = static_cast<int64_t>(chunk) * a.kc;
    const int64_t group_kmax = rows_kmax(a, group_row0, kGroupRows);
    const int64_t key_end = (key_begin + a.kc < group_kmax) ? key_begin + a.kc : group_kmax;

    const int tile = tid / 64;
    const int h = (tid % 64) / kRowTile;
    const int r = tile * kRowTile + (tid % kRowTile);
    const int64_t row = group_row0 + r;
    const bool live = h < a.qt && row < a.n_sel;
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
        const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kGroupRows + r;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) a.ws_o[slot * D + d] = acc[d];
        a.ws_ml[slot * 2 + 0] = m_run;
        a.ws_ml[slot * 2 + 1] = l_run;
    }
}

// ===========================================================================
// Merge of multi-chunk groups. Grid (q_head, group, row block of 8 rows).
// Phase 1 stages per-(row, chunk) weights exp2(m_c - M) and the total l in
// LDS; phase 2 gives each thread one (row, dim) element to accumulate.
// ===========================================================================
constexpr int kMergeThreads = 256;
constexpr int kMergeRows = 8;

template <typename T>
__global__ void __launch_bounds__(kMergeThreads) attn_merge_kernel(AttnArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    extern __shared__ __align__(16) char smem[];
    const int q_head = blockIdx.x;
    const int grp = blockIdx.y;
    const int32_t* gt = group_table(a.sched);
    const int base = gt[2 * grp];
    const int n_chunks = gt[2 * grp + 1];
    if (n_chunks <= 1) return;
    const int D = a.head_dim;
    const int r0 = blockIdx.z * kMergeRows;  // first row (within the group) of this block
    float* W = reinterpret_cast<float*>(smem);  // [kMergeRows][n_chunks]
    float* Linv = W + kMergeRows * n_chunks;    // [kMergeRows]
    const int64_t slot0 = (static_cast<int64_t>(q_head) * a.n_work + base) * kGroupRows;

    // phase 1: 32 lanes per row reduce over chunks
    const int tr = threadIdx.x / 32;
    const int tl = threadIdx.x % 32;
    {
        const int r = r0 + tr;
        float mx = -INFINITY;
        for (int c = tl; c < n_chunks; c += 32)
            mx = fmaxf(mx, a.ws_ml[(slot0 + static_cast<int64_t>(c) * kGroupRows + r) * 2]);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 32));
        const float m_use = (mx == -INFINITY) ? 0.f : mx;
        float l = 0.f;
        for (int c = tl; c < n_chunks; c += 32) {
            const int64_t s = (slot0 + static_cast<int64_t>(c) * kGroupRows + r) * 2;
            const float w = exp2f(a.ws_ml[s] - m_use);
            W[tr * n_chunks + c] = w;
            l += w * a.ws_ml[s + 1];
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) l += __shfl_xor(l, off, 32);
        if (tl == 0) Linv[tr] = 1.f / l;
    }
    __syncthreads();

    // phase 2: one (row, d) element per thread-iteration
    for (int e = threadIdx.x; e < kMergeRows * D; e += kMergeThreads) {
        const int rr = e / D;
        const int d = e - rr * D;
        const int r = r0 + rr;
        const int64_t row = static_cast<int64_t>(grp) * kGroupRows + r;
        if (row >= a.n_sel) continue;
        const float* po = a.ws_o + (slot0 + r) * D + d;
        const float* w = W + rr * n_chunks;
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        int c = 0;
        for (; c + 4 <= n_chunks; c += 4) {
            acc0 += w[c] * po[static_cast<int64_t>(c) * kGroupRows * D];
            acc1 += w[c + 1] * po[static_cast<int64_t>(c + 1) * kGroupRows * D];
            acc2 += w[c + 2] * po[static_cast<int64_t>(c + 2) * kGroupRows * D];
            acc3 += w[c + 3] * po[static_cast<int64_t>(c + 3) * kGroupRows * D];
        }
        for (; c < n_chunks; ++c) acc0 += w[c] * po[static_cast<int64_t>(c) * kGroupRows * D];
        bits* op = reinterpret_cast<bits*>(a.out);
        op[q_head * a.os[0] + row * a.os[1] + d * a.os[2]] =
            E::from_float(((acc0 + acc1) + (acc2 + acc3)) * Linv[rr]);
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

template <typename T, int D, int QT>
int launch_mfma_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    const size_t smem = MfmaSmem<D>::bytes;
    static const bool ok = allow_lds(attn_mfma_kernel<T, D, QT>, smem);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_mfma_kernel<T, D, QT><<<grid, kMfmaThreads, smem, s>>>(a);
    return launch_status();
}

template <typename T, int D>
int launch_mfma(const AttnArgs& a, int qt, dim3 grid, hipStream_t s) {
    if (qt == 4) return launch_mfma_inst<T, D, 4>(a, grid, s);
    if (qt == 2) return launch_mfma_inst<T, D, 2>(a, grid, s);
    return launch_mfma_inst<T, D, 1>(a, grid, s);
}

template <typename T, int DMAX>
int launch_generic_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    const size_t smem =
        (static_cast<size_t>(2) * kGenSub * DMAX + static_cast<size_t>(kGenSub) * kGenThreads) * sizeof(float);
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
int launch_merge(const AttnArgs& a, int max_chunks, hipStream_t s) {
    const size_t smem = (static_cast<size_t>(kMergeRows) * max_chunks + kMergeRows) * sizeof(float);
    static const bool ok = allow_lds(attn_merge_kernel<T>, static_cast<size_t>(kMergeRows) *
                                                               (kMaxChunksPerGroup + 1) * sizeof(float));
    if (!ok) return KVR_E_LAUNCH_FAILED;
    dim3 grid(a.n_q_heads, a.n_groups, kGroupRows / kMergeRows);
    attn_merge_kernel<T><<<grid, kMergeThreads, smem, s>>>(a);
    return launch_status();
}

int64_t group_kmax_host(const int64_t* positions, int64_t n_sel, int64_t g) {
    const int64_t last = (g + 1) * kGroupRows - 1 < n_sel ? (g + 1) * kGroupRows - 1 : n_sel - 1;
    return positions[last] + 1;
}

}  // namespace
}  // namespace kvr

using namespace kvr;

extern "C" int64_t kvr_attention_schedule(const int64_t* positions, int64_t n_sel, int64_t n_keys, int32_t n_q_heads,
                                          int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t chunk_keys,
                                          int32_t* schedule, int64_t capacity) {
    if (dtype_size(dtype) == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_keys < 0 || n_sel > n_keys) return KVR_E_INVALID_ARGUMENT;
    if (n_keys >= (int64_t(1) << 31) || n_sel >= (int64_t(1) << 31)) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || head_dim <= 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_sel > 0 && !positions) return KVR_E_NULL_POINTER;
    for (int64_t i = 0; i < n_sel; ++i) {
        if (positions[i] < 0 || positions[i] >= n_keys) return KVR_E_INVALID_ARGUMENT;
        if (i && positions[i] <= positions[i - 1]) return KVR_E_INVALID_ARGUMENT;
    }
    const bool mfma = mfma_eligible(dtype, head_dim);
    if (!mfma && generic_dmax(head_dim) == 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (chunk_keys < 0 || (chunk_keys > 0 && chunk_keys % kSub != 0)) return KVR_E_INVALID_ARGUMENT;
    const int group = n_q_heads / n_kv_heads;
    const int qt = pick_qt(group);
    const int n_head_groups = group / qt;
    const int64_t n_groups = (n_sel + kGroupRows - 1) / kGroupRows;
    const int64_t heads = static_cast<int64_t>(n_kv_heads) * n_head_groups;

    int64_t maxk = kSub;
    for (int64_t g = 0; g < n_groups; ++g) {
        const int64_t k = group_kmax_host(positions, n_sel, g);
        maxk = k > maxk ? k : maxk;
    }
    auto chunks_for = [&](int64_t kc) {
        int64_t blocks = 0, worst = 0;
        for (int64_t g = 0; g < n_groups; ++g) {
            const int64_t c = (group_kmax_host(positions, n_sel, g) + kc - 1) / kc;
            blocks += c;
            worst = c > worst ? c : worst;
        }
        return std::pair<int64_t, int64_t>(blocks, worst);
    };
    // Chunk size: the smallest multiple of 64 keys that keeps the grid within
    // one block per CU (256 CUs, one 4-wave block each); when even unsplit
    // groups exceed that, groups are not split. A group whose keys fit one
    // chunk needs no merge.
    int64_t kc = chunk_keys;
    if (kc == 0) {
        const int64_t target = 256;
        const int64_t whole = ((maxk + kSub - 1) / kSub) * kSub;
        kc = whole;
        for (int64_t cand = kSub; cand < whole; cand += kSub) {
            if (chunks_for(cand).first * heads <= target) {
                kc = cand;
                break;
            }
        }
    }
    while (chunks_for(kc).second > kMaxChunksPerGroup) kc += kSub;
    const auto counts = chunks_for(kc);
    const int64_t n_work = counts.first;
    if (n_work > 65535) return KVR_E_UNSUPPORTED_SHAPE;  // grid.y limit
    int64_t n_multi = 0;
    for (int64_t g = 0; g < n_groups; ++g) n_multi += (group_kmax_host(positions, n_sel, g) + kc - 1) / kc > 1;
    const int64_t need = kHeader + 2 * n_groups + 2 * n_work;
    if (!schedule) return need;
    if (capacity < need) return KVR_E_CAPACITY;
    int32_t* h = schedule;
    memset(h, 0, sizeof(int32_t) * kHeader);
    h[H_MAGIC] = kMagic;
    h[H_VERSION] = kVersion;
    h[H_NSEL] = static_cast<int32_t>(n_sel);
    h[H_NGROUPS] = static_cast<int32_t>(n_groups);
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
    h[H_MAXCHUNKS] = static_cast<int32_t>(counts.second);
    int32_t* groups = h + kHeader;
    int32_t* works = groups + 2 * n_groups;
    int64_t w = 0;
    for (int64_t g = 0; g < n_groups; ++g) {
        const int64_t c = (group_kmax_host(positions, n_sel, g) + kc - 1) / kc;
        groups[2 * g] = static_cast<int32_t>(w);
        groups[2 * g + 1] = static_cast<int32_t>(c);
        for (int64_t i = 0; i < c; ++i, ++w) {
            works[2 * w] = static_cast<int32_t>(g);
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
    return static_cast<int64_t>(n_q_heads) * schedule[H_NWORK] * kGroupRows * (head_dim + 2) * 4;
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
    if (schedule_len != kHeader + 2 * static_cast<int64_t>(hs[H_NGROUPS]) + 2 * static_cast<int64_t>(hs[H_NWORK]))
        return KVR_E_BAD_SCHEDULE;
    if (hs[H_MAXCHUNKS] > kMaxChunksPerGroup || hs[H_KC] <= 0 || hs[H_KC] % kSub) return KVR_E_BAD_SCHEDULE;
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
    a.n_groups = hs[H_NGROUPS];
    a.n_work = hs[H_NWORK];
    a.kc = hs[H_KC];
    a.head_dim = head_dim;
    a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
    if (ws_need > 0) {
        a.ws_ml = static_cast<float*>(workspace);
        a.ws_o = a.ws_ml + static_cast<int64_t>(n_q_heads) * a.n_work * kGroupRows * 2;
    }
    if (a.qt * a.n_head_groups != a.group) return KVR_E_BAD_SCHEDULE;

    // The MFMA kernel reads 16-byte fragments of q/k/v: unit dim strides and
    // 16-byte aligned rows. Other layouts (strided slices, odd offsets) take
    // the generic kernel, which accepts every schedule.
    bool use_mfma = hs[H_KIND] == KIND_MFMA;
    if (use_mfma && !mfma_eligible(dtype, head_dim)) return KVR_E_BAD_SCHEDULE;
    for (int t = 0; t < 3 && use_mfma; ++t) {
        const int64_t* st3 = strides + 3 * t;
        if (st3[2] != 1 || (st3[0] * esize) % 16 || (st3[1] * esize) % 16) use_mfma = false;
    }
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u)
        use_mfma = false;

    hipStream_t s = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(n_kv_heads * a.n_head_groups), static_cast<unsigned>(a.n_work));
    int st;
    if (use_mfma) {
        if (dtype == KVR_DTYPE_BF16)
            st = head_dim == 128 ? launch_mfma<bf16_t, 128>(a, a.qt, grid, s) : launch_mfma<bf16_t, 64>(a, a.qt, grid, s);
        else
            st = head_dim == 128 ? launch_mfma<f16_t, 128>(a, a.qt, grid, s) : launch_mfma<f16_t, 64>(a, a.qt, grid, s);
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
        case KVR_DTYPE_F32: return launch_merge<f32_t>(a, hs[H_MAXCHUNKS], s);
        case KVR_DTYPE_F16: return launch_merge<f16_t>(a, hs[H_MAXCHUNKS], s);
        default: return launch_merge<bf16_t>(a, hs[H_MAXCHUNKS], s);
    }
}
