// Packed selected-query causal attention (GQA) for gfx950.
//
// Reference semantics: src/kv_cache_repair/kernels/packed_cache.py:47-67 with the
// boolean mask `key <= position` of packed_cache.py:205-207, i.e.
//   out[h, r] = softmax_{j <= pos[r]}(scale * q[h, r] . k[h / G, j]) @ v[h / G]
// and indexed_causal_attention (indexed_attention.py:207-241).
//
// Work decomposition (host schedule, kvr_attention_schedule):
//   selected rows are cut into groups of 64 (four tiles of 16 rows) -- or, when
//   so few rows would fill under half the grid, into 16-row groups for the
//   split-key tile kernel below; group g needs keys
//   [0, pos[last row of g] + 1). That key range is cut into chunks
//   whose boundaries are multiples of 64 keys, sized so every chunk carries
//   about the same cost (64-key sub-tiles weighted by how many of the group's
//   row tiles still attend to them) and the whole grid is about one block per
//   CU. One block handles one (KV head, head group, row group, chunk): it
//   stages the chunk's K (row-major) and V (transposed) in LDS, 64 keys at a
//   time, double-buffered, and each wave attends the rows of two row tiles
//   for one query head to it. Grid x = KV head x head group, so every block
//   of one KV head lands on the same XCD (blocks are dealt round-robin over
//   the 8 XCDs by linear id) and that head's K/V and partials share one L2.
// Groups with one chunk write the final output; groups with several chunks
// write fp32 partials (running max m in the log2 domain, sum l, unnormalised
// O) only for row tiles that attend into the chunk, and a merge kernel
// combines them.
#include "kvr_internal.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

namespace kvr {
namespace {

constexpr int32_t kMagic = 0x4B565253;  // "KVRS"
constexpr int32_t kVersion = 5;
constexpr int kHeader = 18;
constexpr int kWorkInts = 4;               // (group, chunk, key_begin, key_end)
constexpr int kRowTile = 16;               // rows per MFMA tile
constexpr int kTilesPerGroup = 4;
constexpr int kGroupRows = kRowTile * kTilesPerGroup;  // rows per group of the wide kernels
constexpr int kTileGroupRows = kRowTile;               // rows per group of the split-key tile kernel
constexpr int kSub = 64;                   // keys per LDS sub-tile
constexpr int kMaxChunksPerGroup = 1024;   // merge weights fit in LDS
#ifndef KVR_ATTN_TARGET_BLOCKS
#define KVR_ATTN_TARGET_BLOCKS 256
#endif
#ifndef KVR_ATTN_MAX_QT
#define KVR_ATTN_MAX_QT 4
#endif
#ifndef KVR_ATTN_PAIR
#define KVR_ATTN_PAIR 1
#endif
constexpr int kTargetBlocks = KVR_ATTN_TARGET_BLOCKS;  // one block per CU (MI355X: 256 CUs)
constexpr float kLazyLog2 = 8.f;           // lazy-rescale headroom (log2 units): p <= 256

enum Header {
    H_MAGIC = 0,
    H_VERSION,
    H_NSEL,
    H_NGROUPS,
    H_KC,  // longest chunk in keys
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
    H_MAXCHUNKS,
    H_GROUP_ROWS,
    H_PROB  // 0: probabilities enter PV as a hi + lo pair; 1: rounded to the input dtype (as SDPA rounds them)
};
enum Kind { KIND_GENERIC = 0, KIND_MFMA = 1 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct AttnArgs {
    const char* q;
    const char* k;
    const char* v;
    char* out;
    int64_t qs[3], ks[3], vs[3], os[3];  // {head,row,dim} element strides
    const int64_t* positions;
    const int32_t* sched;  // device schedule
    float* ws_ml;          // [Hq][n_work][group_rows] (m, l)
    float* ws_o;           // [Hq][n_work][group_rows][D]
    int64_t n_sel;
    int64_t n_keys;
    int32_t n_q_heads;
    int32_t group;  // G = Hq / Hkv
    int32_t qt;     // query heads per block
    int32_t n_head_groups;
    int32_t n_groups;
    int32_t n_work;
    int32_t group_rows;  // rows per group: kGroupRows, or kTileGroupRows (tile kernel)
    int32_t head_dim;
    int32_t out_vec;  // output rows take 8-byte stores (unit dim stride, aligned)
    int32_t p_rounded;  // the schedule permits probabilities rounded to the input dtype (H_PROB)
    float scale_log2;  // scale * log2(e)
};

// Schedule accessors (device or host pointer to the same int32 layout).
__host__ __device__ inline const int32_t* group_table(const int32_t* s) { return s + kHeader; }
__host__ __device__ inline const int32_t* work_table(const int32_t* s) { return s + kHeader + 2 * s[H_NGROUPS]; }

// The device schedule's work table, located from the group count the host
// read from the same schedule (one dependent load fewer than reading the
// device header first).
__device__ inline const int32_t* work_table_of(const AttnArgs& a) { return a.sched + kHeader + 2 * a.n_groups; }

// Causal key limit (exclusive) of rows [first, first + count) clipped to n_sel; 0 when empty.
__device__ inline int32_t rows_kmax(const AttnArgs& a, int64_t first, int64_t count) {
    if (first >= a.n_sel) return 0;
    const int64_t last = (first + count - 1 < a.n_sel) ? first + count - 1 : a.n_sel - 1;
    return static_cast<int32_t>(a.positions[last] + 1);
}

// ===========================================================================
// MFMA kernel (bf16 / fp16, head_dim 64 or 128)
// ===========================================================================
// Probabilities enter the PV MFMA as a hi + lo pair of 16-bit values so they
// are not rounded to 16 bits (the reference Triton kernel keeps P in fp32,
// _indexed_triton.py:54-58). split() packs two probabilities: hi holds their
// 16-bit heads, lo the rounded remainders p - head.
template <typename T> struct mma_t;
template <> struct mma_t<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // bf16 head = the upper half of the fp32 bits (truncation); p - head is exact
    // in fp32 and its RNE bf16 rounding leaves an error below 2^-16 |p|.
    // two probabilities rounded to bf16 (RNE), packed
    __device__ static inline uint32_t round2(float p0, float p1) {
        const f32x2 r = {p0, p1};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
    }
    __device__ static inline void split(float p0, float p1, uint32_t& hi, uint32_t& lo) {
        const uint32_t b0 = __float_as_uint(p0), b1 = __float_as_uint(p1);
        hi = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
        const f32x2 r = {p0 - __uint_as_float(b0 & 0xffff0000u), p1 - __uint_as_float(b1 & 0xffff0000u)};
        lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));  // v_cvt_pk_bf16_f32 (RNE)
    }
};
template <> struct mma_t<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __device__ static inline uint32_t round2(float p0, float p1) {
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(p0))) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(p1))) << 16);
    }
    __device__ static inline void split(float p0, float p1, uint32_t& hi, uint32_t& lo) {
        const _Float16 h0 = static_cast<_Float16>(p0), h1 = static_cast<_Float16>(p1);
        const _Float16 l0 = static_cast<_Float16>(p0 - static_cast<float>(h0));
        const _Float16 l1 = static_cast<_Float16>(p1 - static_cast<float>(h1));
        hi = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h0)) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
        lo = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l0)) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
    }
};

// LDS layout of one staged 64-key sub-tile: K row-major [64][D + 8] then V
// transposed [D][64 + 8] (16-bit elements; 16-byte aligned rows). V^T column
// of key k of a sub-tile: k = 32h + 16a + 4j + i sits at 32h + 8j + 4a + i,
// so the 8 keys a lane's PV fragment pairs with P^T (keys 32h + 4j + i and
// 32h + 16 + 4j + i) are one 16-byte read; key pairs stay adjacent for the
// 4-byte transposing V writes.
__device__ inline int vt_pos(int k) { return (k & 32) | ((k & 12) << 1) | ((k & 16) >> 2) | (k & 3); }

template <int D, int QT>
struct MfmaCfg {
    static constexpr int threads = 128 * QT;  // two waves per query head
    static constexpr int kstr = D + 8;
    static constexpr int vstr = kSub + 8;
    static constexpr int k_elems = kSub * kstr;
    static constexpr int v_elems = D * vstr;
    static constexpr int buf_elems = k_elems + v_elems;
    static constexpr int bytes = 2 * buf_elems * 2;  // double-buffered, 2 bytes per element
    static constexpr int c8 = D / 8;                 // 16-byte pieces per row
    static constexpr int k_pieces = kSub * c8;
    static constexpr int v_pieces = (kSub / 2) * c8;  // (key pair, piece)
    static constexpr int kp = (k_pieces + threads - 1) / threads;
    static constexpr int vp = (v_pieces + threads - 1) / threads;
};

template <typename T, int D, int QT>
struct MfmaWave {
    using M = mma_t<T>;
    using v8 = typename M::v8;
    using C = MfmaCfg<D, QT>;
    static constexpr int DS = D / 32;  // k-steps of the QK^T MFMA
    static constexpr int DT = D / 16;  // d tiles of the PV MFMA

    v8 qf[2][DS];
    f32x4 o[2][DT];
    float m_run[2], l_run[2];
    int32_t kmax[2], nomask_end[2], pos[2];

    // One 64-key sub-tile for the wave's active tiles A0 (tile half) / A1 (tile
    // half + 2). MASK: some key of the sub-tile lies beyond some row's position.
    template <bool A0, bool A1, bool MASK>
    __device__ inline void step(const uint16_t* Ks, const uint16_t* Vt, int32_t key0, int lq, int lj,
                                float scale_log2) {
        f32x4 st[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) st[t][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // S^T = K Q^T: keys on the M axis, each lane gets 4 keys of its row.
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const v8 kf = __builtin_bit_cast(
                    v8, *reinterpret_cast<const u32x4*>(Ks + (16 * kt + lq) * C::kstr + 32 * ds + 8 * lj));
                if (A0) st[0][kt] = M::mma(kf, qf[0][ds], st[0][kt]);
                if (A1) st[1][kt] = M::mma(kf, qf[1][ds], st[1][kt]);
            }
        u32x4 phi[2][2], plo[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (!(t == 0 ? A0 : A1)) continue;
            // raw scores; scale_log2 > 0 (the host routes other scales to the
            // generic kernel), so the scaled max is the raw max times the scale
            float x[4][4];
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float s = st[t][kt][i];
                    if (MASK) s = (key0 + 16 * kt + 4 * lj + i <= pos[t]) ? s : -INFINITY;
                    x[kt][i] = s;
                    mx = fmaxf(mx, s);
                }
            mx *= scale_log2;
            // Lazy rescaling: a row's reference max m moves only when its scores
            // exceed m by more than kLazyLog2 (so p <= 2^kLazyLog2 and fp32 o, l
            // cannot overflow). When no lane of the wave sees such a score, the
            // row reduction and the o/l rescale are skipped; o / l is unchanged.
            if (__any(mx > m_run[t] + kLazyLog2)) {
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const float m_new = (mx > m_run[t] + kLazyLog2) ? mx : m_run[t];
                // 1 if unmoved, 0 from -inf; a row with no visible key yet keeps m = -inf
                // and alpha = exp2(-inf - 0) = 0 (never exp2(-inf + inf))
                const float alpha = __builtin_amdgcn_exp2f(m_run[t] - (m_new == -INFINITY ? 0.f : m_new));
                m_run[t] = m_new;
                l_run[t] *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[t][dt] *= alpha;
            }
            const float m_use = (m_run[t] == -INFINITY) ? 0.f : m_run[t];
            float psum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kt][i], scale_log2, -m_use));
                    x[kt][i] = p;
                    psum += p;
                }
            l_run[t] += psum;
            // P^T as the B operand: lane group lj holds keys {4lj+i} of key tiles
            // 2h and 2h+1; V^T below is read in the same key order.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t hv[4], lv[4];
                M::split(x[2 * h][0], x[2 * h][1], hv[0], lv[0]);
                M::split(x[2 * h][2], x[2 * h][3], hv[1], lv[1]);
                M::split(x[2 * h + 1][0], x[2 * h + 1][1], hv[2], lv[2]);
                M::split(x[2 * h + 1][2], x[2 * h + 1][3], hv[3], lv[3]);
                phi[t][h] = u32x4{hv[0], hv[1], hv[2], hv[3]};
                plo[t][h] = u32x4{lv[0], lv[1], lv[2], lv[3]};
            }
        }
        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint16_t* row = Vt + (16 * dt + lq) * C::vstr + 32 * h + 8 * lj;
                const v8 vf = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(row));
                if (A0) {
                    o[0][dt] = M::mma(vf, __builtin_bit_cast(v8, phi[0][h]), o[0][dt]);
                    o[0][dt] = M::mma(vf, __builtin_bit_cast(v8, plo[0][h]), o[0][dt]);
                }
                if (A1) {
                    o[1][dt] = M::mma(vf, __builtin_bit_cast(v8, phi[1][h]), o[1][dt]);
                    o[1][dt] = M::mma(vf, __builtin_bit_cast(v8, plo[1][h]), o[1][dt]);
                }
            }
    }

    template <bool MASK>
    __device__ inline void dispatch(bool a0, bool a1, const uint16_t* Ks, const uint16_t* Vt, int32_t key0,
                                    int lq, int lj, float scale_log2) {
        // Tile half + 2 holds later rows than tile half, so it is active whenever
        // tile half is, unless it has no rows at all (the last, partial group):
        // then it runs fully masked (pos = -1 gives p = 0) and is never written.
        if (a0)
            step<true, true, MASK>(Ks, Vt, key0, lq, lj, scale_log2);
        else if (a1)
            step<false, true, MASK>(Ks, Vt, key0, lq, lj, scale_log2);
    }
};

template <typename T, int D, int QT>
__global__ void __launch_bounds__(128 * QT)
attn_mfma_kernel(AttnArgs a) {
    using C = MfmaCfg<D, QT>;
    using W = MfmaWave<T, D, QT>;
    using v8 = typename W::v8;
    constexpr int NT = C::threads;
    extern __shared__ __align__(16) char smem[];
    uint16_t* lds = reinterpret_cast<uint16_t*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches below
    const int lq = lane & 15;
    const int lj = lane >> 4;

    const int work = blockIdx.y;
    const int32_t* wk = work_table_of(a) + kWorkInts * work;
    const int grp = wk[0];
    const int32_t key_begin = wk[2];
    const int32_t key_end = wk[3];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int hq = wave % QT;
    const int half = wave / QT;
    const int q_head = kv_head * a.group + hg * QT + hq;
    const int64_t group_row0 = static_cast<int64_t>(grp) * kGroupRows;

    const int32_t ks1 = static_cast<int32_t>(a.ks[1]);
    const int32_t vs1 = static_cast<int32_t>(a.vs[1]);
    const char* kbase = a.k + (static_cast<int64_t>(kv_head) * a.ks[0] + static_cast<int64_t>(key_begin) * a.ks[1]) * 2;
    const char* vbase = a.v + (static_cast<int64_t>(kv_head) * a.vs[0] + static_cast<int64_t>(key_begin) * a.vs[1]) * 2;
    const int32_t n_keys_chunk = key_end - key_begin;
    const int n_sub = (n_keys_chunk + kSub - 1) / kSub;

    u32x4 kr[C::kp], vr0[C::vp], vr1[C::vp];
    // Global -> registers: sub-tile s. The loads are unconditional (key rows
    // past the chunk end re-read its last row, in bounds) so the wait for them
    // sits at the LDS store, after the step's compute; store() zeroes those
    // rows. Conditional loads would make the compiler wait for them at once.
    auto load = [&](int s) {
#pragma unroll
        for (int p = 0; p < C::kp; ++p) {
            const int idx = tid + p * NT;
            if (C::k_pieces % NT == 0 || idx < C::k_pieces) {
                const int kk = idx / C::c8;
                const int c8 = idx - kk * C::c8;
                const int32_t key = min(kSub * s + kk, n_keys_chunk - 1);
                kr[p] = *reinterpret_cast<const u32x4*>(kbase + (static_cast<int64_t>(key) * ks1 + 8 * c8) * 2);
            }
        }
#pragma unroll
        for (int p = 0; p < C::vp; ++p) {
            const int idx = tid + p * NT;
            if (C::v_pieces % NT == 0 || idx < C::v_pieces) {
                const int pr = idx & 31;
                const int c8 = idx >> 5;
                const int32_t k0 = min(kSub * s + 2 * pr, n_keys_chunk - 1);
                const int32_t k1 = min(kSub * s + 2 * pr + 1, n_keys_chunk - 1);
                vr0[p] = *reinterpret_cast<const u32x4*>(vbase + (static_cast<int64_t>(k0) * vs1 + 8 * c8) * 2);
                vr1[p] = *reinterpret_cast<const u32x4*>(vbase + (static_cast<int64_t>(k1) * vs1 + 8 * c8) * 2);
            }
        }
    };
    // Registers -> LDS buffer of sub-tile s: K as is, V transposed (key pairs
    // packed per dim); rows past the chunk end are zeroed.
    auto store = [&](uint16_t* buf, int s) {
        uint16_t* Ks = buf;
        uint16_t* Vt = buf + C::k_elems;
        const int32_t left = n_keys_chunk - kSub * s;
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int p = 0; p < C::kp; ++p) {
            const int idx = tid + p * NT;
            if (C::k_pieces % NT == 0 || idx < C::k_pieces) {
                const int kk = idx / C::c8;
                const int c8 = idx - kk * C::c8;
                *reinterpret_cast<u32x4*>(Ks + kk * C::kstr + 8 * c8) = kk < left ? kr[p] : zero;
            }
        }
#pragma unroll
        for (int p = 0; p < C::vp; ++p) {
            const int idx = tid + p * NT;
            if (C::v_pieces % NT == 0 || idx < C::v_pieces) {
                const int pr = idx & 31;
                const int c8 = idx >> 5;
                const u32x4 v0 = 2 * pr < left ? vr0[p] : zero;
                const u32x4 v1 = 2 * pr + 1 < left ? vr1[p] : zero;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t x0 = v0[j], x1 = v1[j];
                    uint16_t* col = Vt + (8 * c8 + 2 * j) * C::vstr + vt_pos(2 * pr);
                    *reinterpret_cast<uint32_t*>(col) = (x0 & 0xffffu) | (x1 << 16);
                    *reinterpret_cast<uint32_t*>(col + C::vstr) = (x0 >> 16) | (x1 & 0xffff0000u);
                }
            }
        }
    };

    W w;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int64_t row0 = group_row0 + kRowTile * (half + 2 * t);
        const int64_t row = row0 + lq;
        w.kmax[t] = rows_kmax(a, row0, kRowTile);
        w.nomask_end[t] = (row0 + kRowTile <= a.n_sel) ? static_cast<int32_t>(a.positions[row0] + 1) : 0;
        w.pos[t] = (row < a.n_sel) ? static_cast<int32_t>(a.positions[row]) : -1;
        w.m_run[t] = -INFINITY;
        w.l_run[t] = 0.f;
#pragma unroll
        for (int dt = 0; dt < W::DT; ++dt) w.o[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < W::DS; ++ds) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row < a.n_sel) {
                const int64_t off = q_head * a.qs[0] + row * a.qs[1] + (32 * ds + 8 * lj);
                raw = *reinterpret_cast<const u32x4*>(a.q + off * 2);
            }
            w.qf[t][ds] = __builtin_bit_cast(v8, raw);
        }
    }

    if (n_sub > 0) {
        load(0);
        store(lds, 0);
    }
    for (int s = 0; s < n_sub; ++s) {
        const bool more = s + 1 < n_sub;
        if (more) load(s + 1);
        __syncthreads();  // sub-tile s is staged; buffer (s+1)&1 is no longer read
        const uint16_t* Ks = lds + (s & 1) * C::buf_elems;
        const uint16_t* Vt = Ks + C::k_elems;
        const int32_t key0 = key_begin + kSub * s;
        const bool a0 = key0 < w.kmax[0];
        const bool a1 = key0 < w.kmax[1];
        // rows of an active tile all see every key of the sub-tile unless the
        // sub-tile reaches past the tile's first (smallest) position
        const int32_t key_stop = key0 + kSub;
        const bool mask = a0 ? (key_stop > w.nomask_end[0] || key_stop > w.nomask_end[1])
                             : key_stop > w.nomask_end[1];
        if (mask)
            w.template dispatch<true>(a0, a1, Ks, Vt, key0, lq, lj, a.scale_log2);
        else
            w.template dispatch<false>(a0, a1, Ks, Vt, key0, lq, lj, a.scale_log2);
        if (more) store(lds + ((s + 1) & 1) * C::buf_elems, s + 1);
    }

    // ---- epilogue: row sums across the 4 lane groups, then output or partial ----
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float l = w.l_run[t];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        w.l_run[t] = l;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int r = kRowTile * (half + 2 * t) + lq;  // row within the group
        const int64_t row = group_row0 + r;
        if (w.kmax[t] <= key_begin || row >= a.n_sel) continue;  // tile does not attend into this chunk
        if (n_chunks == 1) {
            const float inv = 1.f / w.l_run[t];
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + q_head * a.os[0] + row * a.os[1];
#pragma unroll
            for (int dt = 0; dt < W::DT; ++dt) {
                uint16_t e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = elem<T>::from_float(w.o[t][dt][i] * inv);
                if (a.out_vec) {
                    *reinterpret_cast<uint2*>(dst + 16 * dt + 4 * lj) =
                        uint2{e[0] | (static_cast<uint32_t>(e[1]) << 16), e[2] | (static_cast<uint32_t>(e[3]) << 16)};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dst[(16 * dt + 4 * lj + i) * a.os[2]] = e[i];
                }
            }
        } else {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kGroupRows + r;
            float* po = a.ws_o + slot * D;
#pragma unroll
            for (int dt = 0; dt < W::DT; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * lj) = w.o[t][dt];
            if (lj == 0) {
                a.ws_ml[slot * 2 + 0] = w.m_run[t];
                a.ws_ml[slot * 2 + 1] = w.l_run[t];
            }
        }
    }
}

// ===========================================================================
// Split-key tile kernel (bf16 / fp16, head_dim 64 or 128) for schedules of
// 16-row groups (few selected rows). Block = (KV head, head group, one 16-row
// group, chunk); wave w serves query head w % QT over the keys of every other
// 64-key sub-tile (key half w / QT): each iteration stages two sub-tiles (128
// keys, double-buffered) and the two waves of a head attend one each. At the
// end the second wave of each head hands its (m, l, O) to the first through
// LDS, which combines them (rescaling both to the larger reference max) and
// writes the output or the chunk's partial. With a quarter of the rows of the
// wide kernel per block, a group needs a quarter of the chunks for the same
// grid, so the partials (and the merge's reads) shrink 4x; the K/V of a chunk
// is read by up to four groups, all on the XCD of its KV head (grid x).
// ===========================================================================
template <typename T, int D, int QT>
__global__ void __launch_bounds__(128 * QT) attn_tile_kernel(AttnArgs a) {
    using C = MfmaCfg<D, QT>;
    using W = MfmaWave<T, D, QT>;
    using v8 = typename W::v8;
    constexpr int NT = C::threads;
    extern __shared__ __align__(16) char smem[];
    uint16_t* lds = reinterpret_cast<uint16_t*>(smem);  // [stage 2][sub-tile 2][buf_elems]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 15;
    const int lj = lane >> 4;
    const int hq = wave % QT;
    const int kh = wave / QT;  // key half: sub-tiles 2i + kh

    const int work = blockIdx.y;
    const int32_t* wk = work_table_of(a) + kWorkInts * work;
    const int grp = wk[0];
    const int32_t key_begin = wk[2];
    const int32_t key_end = wk[3];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int q_head = kv_head * a.group + hg * QT + hq;
    const int64_t row0 = static_cast<int64_t>(grp) * kTileGroupRows;

    const int32_t ks1 = static_cast<int32_t>(a.ks[1]);
    const int32_t vs1 = static_cast<int32_t>(a.vs[1]);
    const char* kbase = a.k + (static_cast<int64_t>(kv_head) * a.ks[0] + static_cast<int64_t>(key_begin) * a.ks[1]) * 2;
    const char* vbase = a.v + (static_cast<int64_t>(kv_head) * a.vs[0] + static_cast<int64_t>(key_begin) * a.vs[1]) * 2;
    const int32_t n_keys_chunk = key_end - key_begin;
    const int n_sub = (n_keys_chunk + kSub - 1) / kSub;
    const int n_it = (n_sub + 1) / 2;

    u32x4 kr[2][C::kp], vr0[2][C::vp], vr1[2][C::vp];
    // Global -> registers: sub-tiles 2i and 2i + 1, unconditional loads (key
    // rows past the chunk end re-read its last row) so their wait sits at the
    // LDS store after the step's compute; store() zeroes those rows.
    auto load = [&](int i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int s = 2 * i + j;
#pragma unroll
            for (int p = 0; p < C::kp; ++p) {
                const int idx = tid + p * NT;
                if (C::k_pieces % NT == 0 || idx < C::k_pieces) {
                    const int kk = idx / C::c8;
                    const int c8 = idx - kk * C::c8;
                    const int32_t key = min(kSub * s + kk, n_keys_chunk - 1);
                    kr[j][p] = *reinterpret_cast<const u32x4*>(kbase + (static_cast<int64_t>(key) * ks1 + 8 * c8) * 2);
                }
            }
#pragma unroll
            for (int p = 0; p < C::vp; ++p) {
                const int idx = tid + p * NT;
                if (C::v_pieces % NT == 0 || idx < C::v_pieces) {
                    const int pr = idx & 31;
                    const int c8 = idx >> 5;
                    const int32_t k0 = min(kSub * s + 2 * pr, n_keys_chunk - 1);
                    const int32_t k1 = min(kSub * s + 2 * pr + 1, n_keys_chunk - 1);
                    vr0[j][p] = *reinterpret_cast<const u32x4*>(vbase + (static_cast<int64_t>(k0) * vs1 + 8 * c8) * 2);
                    vr1[j][p] = *reinterpret_cast<const u32x4*>(vbase + (static_cast<int64_t>(k1) * vs1 + 8 * c8) * 2);
                }
            }
        }
    };
    // Registers -> LDS stage of step i: per sub-tile K as is, V transposed (key
    // pairs packed per dim); rows past the chunk end are zeroed.
    auto store = [&](uint16_t* stage, int i) {
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint16_t* Ks = stage + j * C::buf_elems;
            uint16_t* Vt = Ks + C::k_elems;
            const int32_t left = n_keys_chunk - kSub * (2 * i + j);
#pragma unroll
            for (int p = 0; p < C::kp; ++p) {
                const int idx = tid + p * NT;
                if (C::k_pieces % NT == 0 || idx < C::k_pieces) {
                    const int kk = idx / C::c8;
                    const int c8 = idx - kk * C::c8;
                    *reinterpret_cast<u32x4*>(Ks + kk * C::kstr + 8 * c8) = kk < left ? kr[j][p] : zero;
                }
            }
#pragma unroll
            for (int p = 0; p < C::vp; ++p) {
                const int idx = tid + p * NT;
                if (C::v_pieces % NT == 0 || idx < C::v_pieces) {
                    const int pr = idx & 31;
                    const int c8 = idx >> 5;
                    const u32x4 v0 = 2 * pr < left ? vr0[j][p] : zero;
                    const u32x4 v1 = 2 * pr + 1 < left ? vr1[j][p] : zero;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t x0 = v0[q], x1 = v1[q];
                        uint16_t* col = Vt + (8 * c8 + 2 * q) * C::vstr + vt_pos(2 * pr);
                        *reinterpret_cast<uint32_t*>(col) = (x0 & 0xffffu) | (x1 << 16);
                        *reinterpret_cast<uint32_t*>(col + C::vstr) = (x0 >> 16) | (x1 & 0xffff0000u);
                    }
                }
            }
        }
    };

    // One row tile per wave (tile slot 0 of MfmaWave; slot 1 stays inactive).
    W w;
    {
        const int64_t row = row0 + lq;
        w.kmax[0] = rows_kmax(a, row0, kRowTile);
        w.nomask_end[0] = (row0 + kRowTile <= a.n_sel) ? static_cast<int32_t>(a.positions[row0] + 1) : 0;
        w.pos[0] = (row < a.n_sel) ? static_cast<int32_t>(a.positions[row]) : -1;
        w.m_run[0] = -INFINITY;
        w.l_run[0] = 0.f;
#pragma unroll
        for (int dt = 0; dt < W::DT; ++dt) w.o[0][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < W::DS; ++ds) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row < a.n_sel) {
                const int64_t off = q_head * a.qs[0] + row * a.qs[1] + (32 * ds + 8 * lj);
                raw = *reinterpret_cast<const u32x4*>(a.q + off * 2);
            }
            w.qf[0][ds] = __builtin_bit_cast(v8, raw);
        }
    }

    if (n_it > 0) {
        load(0);
        store(lds, 0);
    }
    for (int i = 0; i < n_it; ++i) {
        const bool more = i + 1 < n_it;
        if (more) load(i + 1);
        __syncthreads();  // stage i is staged; stage (i + 1) & 1 is no longer read
        const int s = 2 * i + kh;
        const int32_t key0 = key_begin + kSub * s;
        if (s < n_sub && key0 < w.kmax[0]) {
            const uint16_t* Ks = lds + ((i & 1) * 2 + kh) * C::buf_elems;
            const uint16_t* Vt = Ks + C::k_elems;
            if (key0 + kSub > w.nomask_end[0])
                w.template step<true, false, true>(Ks, Vt, key0, lq, lj, a.scale_log2);
            else
                w.template step<true, false, false>(Ks, Vt, key0, lq, lj, a.scale_log2);
        }
        if (more) store(lds + ((i + 1) & 1) * 2 * C::buf_elems, i + 1);
    }

    // ---- combine the two key halves of each head, then output or partial ----
    {
        float l = w.l_run[0];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        w.l_run[0] = l;
    }
    constexpr int kX = W::DT * 4 + 2;  // exchanged floats per lane: O, m, l
    float* xch = reinterpret_cast<float*>(smem) + hq * kX * 64;  // [field][lane] per head
    __syncthreads();  // every wave is done with the K/V stages
    if (kh == 1) {
#pragma unroll
        for (int dt = 0; dt < W::DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) xch[(4 * dt + i) * 64 + lane] = w.o[0][dt][i];
        xch[(kX - 2) * 64 + lane] = w.m_run[0];
        xch[(kX - 1) * 64 + lane] = w.l_run[0];
    }
    __syncthreads();
    if (kh == 1) return;
    {
        const float mb = xch[(kX - 2) * 64 + lane];
        const float lb = xch[(kX - 1) * 64 + lane];
        const float ma = w.m_run[0];
        const float m = fmaxf(ma, mb);
        if (m != -INFINITY) {  // some key of the chunk is visible to this row
            const float fa = __builtin_amdgcn_exp2f(ma - m);  // exp2(-inf) = 0 for an empty half
            const float fb = __builtin_amdgcn_exp2f(mb - m);
#pragma unroll
            for (int dt = 0; dt < W::DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) w.o[0][dt][i] = w.o[0][dt][i] * fa + xch[(4 * dt + i) * 64 + lane] * fb;
            w.l_run[0] = w.l_run[0] * fa + lb * fb;
            w.m_run[0] = m;
        }
    }
    const int r = lq;  // row within the group
    const int64_t row = row0 + r;
    if (w.kmax[0] <= key_begin || row >= a.n_sel) return;  // the row does not attend into this chunk
    if (n_chunks == 1) {
        const float inv = 1.f / w.l_run[0];
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + q_head * a.os[0] + row * a.os[1];
#pragma unroll
        for (int dt = 0; dt < W::DT; ++dt) {
            uint16_t e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = elem<T>::from_float(w.o[0][dt][i] * inv);
            if (a.out_vec) {
                *reinterpret_cast<uint2*>(dst + 16 * dt + 4 * lj) =
                    uint2{e[0] | (static_cast<uint32_t>(e[1]) << 16), e[2] | (static_cast<uint32_t>(e[3]) << 16)};
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[(16 * dt + 4 * lj + i) * a.os[2]] = e[i];
            }
        }
    } else {
        const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * kTileGroupRows + r;
        float* po = a.ws_o + slot * D;
#pragma unroll
        for (int dt = 0; dt < W::DT; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * lj) = w.o[0][dt];
        if (lj == 0) {
            a.ws_ml[slot * 2 + 0] = w.m_run[0];
            a.ws_ml[slot * 2 + 1] = w.l_run[0];
        }
    }
}

// ===========================================================================
// Head-pair kernel (bf16 / fp16, head_dim 64 or 128, four query heads per KV
// head group). Block = (KV head, head group, row group of RT row tiles,
// chunk), 8 waves. A wave owns two query heads of one 16-row tile -- the two
// MFMA column tiles share every K and V fragment it reads from LDS, so one
// fragment read feeds two MFMAs -- and one of X = 8 / (2 RT) key classes.
// Keys are staged 128 per step (four 32-key sub-tiles) by direct global->LDS
// loads (no register staging), double-buffered; the wave of key class x
// attends the step's sub-tiles x, x + X, ... With RT = 1 (16-row groups, few
// selected rows) the four key classes of a head pair take one sub-tile each
// per step and are combined through LDS at the end; with RT = 4 (64-row
// groups) every wave takes all four sub-tiles of a step.
//
// LDS holds K and V row-major, 16-byte pieces XOR-swizzled by row (piece c of
// key row r at c ^ (r mod D/8)), so every fragment read below is free of bank
// conflicts. QK^T reads K fragments with 16-byte reads; the PV operand V^T is
// read with gfx950's transposing ds_read_b64_tr_b16: within each 16-lane
// group, lane i receives element i & 3 of the 8-byte pieces addressed by
// lanes (i >> 2) + 4j, j = 0..3. Pointing lane s of group lj at key row
// 16h + 4 lj + (s >> 2), dims 16 dt + 4 (s & 3) .. + 4 makes lane i receive
// keys 16h + 4 lj .. + 4 of dim 16 dt + i: the V^T fragment whose k order
// matches the score layout of the QK^T MFMA (lane (row, lj) holds keys
// 16 kt + 4 lj + i), so P^T needs no permutation.
// ===========================================================================
constexpr int kPairSub = 32;                 // keys per sub-tile
constexpr int kPairSubs = 4;                 // sub-tiles staged per step
constexpr int kPairStepKeys = kPairSub * kPairSubs;
constexpr int kPairThreads = 512;

template <int D>
struct PairCfg {
    static constexpr int c8 = D / 8;                              // 16-byte pieces per row
    static constexpr int tensor_bytes = kPairStepKeys * D * 2;    // K or V of one step
    static constexpr int stage_bytes = 2 * tensor_bytes;          // K then V
    static constexpr int bytes = 2 * stage_bytes;                 // double-buffered
    static constexpr int pieces_per_wave = tensor_bytes / 16 / 8; // 16-byte pieces one wave loads per tensor
    static constexpr int loads = pieces_per_wave / 64;            // load instructions per wave per tensor
    static_assert(pieces_per_wave % 64 == 0, "whole load instructions");
    // Piece swizzles (XOR on the 16-byte piece index; rows are keys). K: 8
    // consecutive rows at one piece hit 8 distinct bank groups (a 16-byte read
    // serves 8 lanes per cycle). V: the transposing read serves 16 lanes per
    // cycle, 4 consecutive rows x 2 adjacent pieces, which 2 r spreads over 8
    // distinct bank groups.
    __host__ __device__ static constexpr int kswz(int r) { return r & (c8 - 1); }
    __host__ __device__ static constexpr int vswz(int r) { return (2 * r) & (c8 - 1); }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// 16 bytes per lane from `src` (per-lane global address) to LDS at `dst` + 16 *
// lane (`dst` wave-uniform): global_load_lds_dwordx4, the LDS base in M0. Issued
// as inline assembly so the compiler's wait-count pass, which cannot tell these
// LDS writes from the stage being read, adds no vmcnt waits before LDS reads;
// the kernel waits for them itself (vmcnt(0), then a barrier) before reading.
__device__ inline void lds_dma16(const char* src, char* dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)dst)));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}

// The same load from a wave-uniform base (SGPRs) plus a 32-bit per-lane byte
// offset: no per-lane address arithmetic.
__device__ inline void lds_dma16(const char* base, uint32_t off, char* dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)dst)));
    // the base is wave-uniform; reading it from the first lane keeps it in
    // SGPRs even where the compiler cannot prove that (free where it can).
    // readfirstlane returns int: each half goes through uint32_t so the low
    // half is zero-extended, not sign-extended, into the 64-bit address.
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b))));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b >> 32))));
    const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(sb), "s"(m0)
                 : "memory", "m0");
}

// A wave's share of the direct loads of one 128-key step of K or V. Load p of
// wave w fills 1 KB block b = 8 p + w of the staged tile: lane L writes the
// swizzled position (row, c') = divmod(64 b + L, D / 8), i.e. key row
// p * kRows + r0 with r0 = (64 w + L) / (D / 8), and loads piece c' ^ swz(row)
// of that row. kRows is a multiple of D / 8, so the swizzle, and with it the
// lane's byte offset from the load's first row, is the same for every load and
// every step: only wave-uniform bases change.
template <int D>
struct StepLoads {
    using C = PairCfg<D>;
    static constexpr int kRows = 512 / C::c8;  // key rows one load instruction of the 8 waves covers
    static constexpr int kLoads = kPairStepKeys / kRows;
    static_assert(kLoads == C::loads, "one load per 1 KB block");
    int r0;
    int c;

    __device__ inline void init(int wave, int lane) {
        r0 = (64 * wave + lane) / C::c8;
        c = lane % C::c8;
    }
    __device__ inline uint32_t lane_offset(int64_t stride, bool is_v) const {
        const int swz = is_v ? C::vswz(r0) : C::kswz(r0);
        return static_cast<uint32_t>(r0 * stride * 2 + 16 * (c ^ swz));
    }
    // Step `first` (its first key row within the chunk) of a tensor whose
    // chunk starts at `base`; rows past the chunk's n keys re-read its last
    // row (in bounds), only in a chunk's last step.
    __device__ inline void issue(const char* base, int64_t stride, uint32_t lane_off, int32_t first, int32_t n,
                                 char* buf, int wave, bool is_v) const {
        if (first + kPairStepKeys <= n) {
            const char* step = base + static_cast<int64_t>(first) * stride * 2;
#pragma unroll
            for (int p = 0; p < kLoads; ++p)
                lds_dma16(step + static_cast<int64_t>(p * kRows) * stride * 2, lane_off, buf + (8 * p + wave) * 1024);
        } else {
            const int swz = is_v ? C::vswz(r0) : C::kswz(r0);
#pragma unroll
            for (int p = 0; p < kLoads; ++p) {
                const int32_t key = min(first + p * kRows + r0, n - 1);
                lds_dma16(base + (static_cast<int64_t>(key) * stride + 8 * (c ^ swz)) * 2, buf + (8 * p + wave) * 1024);
            }
        }
    }
};

// HILO: probabilities enter PV as a hi + lo pair of 16-bit values (fp32-class,
// the reference Triton kernel's precision); otherwise each is rounded to the
// input dtype before PV, as the SDPA path the packed executor replaces rounds it.
template <typename T, int D, bool HILO>
struct PairWave {
    using M = mma_t<T>;
    using v8 = typename M::v8;
    using C = PairCfg<D>;
    static constexpr int DS = D / 32;  // k-steps of the QK^T MFMA
    static constexpr int DT = D / 16;  // d tiles of the PV MFMA

    v8 qf[2][DS];
    f32x4 o[2][DT];
    f32x4 lsum[2];    // row sums of P as a 17th output tile: row 0 of O^T += ones . P^T
    float m_run[2];
    // kept with m_run, so the per-sub-tile work does not recompute them: the
    // exponent offset -(m_run, or 0 while m_run = -inf) and the lazy-rescale
    // threshold m_run + kLazyLog2
    float m_neg[2], m_thr[2];
    int32_t pos;      // this lane's row position; -1 past the selected rows
    v8 ones;          // A operand of the row-sum tile: row 0 all ones, rows 1..15 zero
    // Per-lane byte offsets of this lane's fragment reads within a staged tile,
    // for sub-tile row 0 (every sub-tile starts at a multiple of 16 rows, so the
    // swizzle of a lane's rows does not depend on the sub-tile or key tile; those
    // add compile-time offsets). K: row lq, piece 4 ds + lj. V (transposing
    // reads): row 4 lj + (lq >> 2), dims 16 dt + 4 (lq & 3).
    int32_t koff[DS];
    int32_t voff[DT];

    // byte offsets of piece c of row r in the swizzled K and V tiles
    __device__ static inline int kpiece(int r, int c) { return (r * C::c8 + (c ^ C::kswz(r))) * 16; }
    __device__ static inline int vpiece(int r, int c) { return (r * C::c8 + (c ^ C::vswz(r))) * 16; }

    __device__ inline void init(int lq, int lj) {
        offsets(lq, lj);
        const uint16_t one = elem<T>::from_float(1.f);
        const uint32_t w = lq == 0 ? (static_cast<uint32_t>(one) | (static_cast<uint32_t>(one) << 16)) : 0u;
        ones = __builtin_bit_cast(v8, u32x4{w, w, w, w});
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            m_run[t] = -INFINITY;
            m_neg[t] = -0.f;
            m_thr[t] = -INFINITY + kLazyLog2;
            lsum[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    __device__ inline void offsets(int lq, int lj) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) koff[ds] = kpiece(lq, 4 * ds + lj);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d0 = 16 * dt + 4 * (lq & 3);
            voff[dt] = vpiece(4 * lj + (lq >> 2), d0 >> 3) + (d0 & 4) * 2;
        }
    }

    // K fragments of the sub-tile: [ds][kt], rows 16 kt + lq, pieces 4 ds + lj.
    __device__ inline void read_k(const char* Ks, v8 (&kf)[DS][2]) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                kf[ds][kt] =
                    __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(Ks + koff[ds] + 16 * kt * D * 2));
    }

    // S^T = K Q_t^T for head t: keys on the M axis, lane (lq, lj) gets keys
    // 16 kt + 4 lj + i of row lq.
    __device__ inline void qk(int t, const v8 (&kf)[DS][2], f32x4 (&st)[2]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) st[kt] = M::mma(kf[ds][kt], qf[t][ds], st[kt]);
    }

    // Scores past a row's position become -inf (the causal mask; only sub-tiles
    // that reach past the tile's first position need it).
    __device__ inline void apply_mask(f32x4 (&st)[2], int32_t key0, int lj) { apply_mask_at(st, key0, lj, pos); }

    // The same with the row's last visible key given (at most its position).
    __device__ static inline void apply_mask_at(f32x4 (&st)[2], int32_t key0, int lj, int32_t last) {
        const int32_t lim = last - key0 - 4 * lj;  // key 16 kt + 4 lj + i is visible iff 16 kt + i <= lim
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) st[kt][i] = (16 * kt + i <= lim) ? st[kt][i] : -INFINITY;
    }

    // Row maximum of head t's scores over this lane's keys, scaled.
    __device__ inline float row_max(const f32x4 (&st)[2], float scale_log2, float (&x)[2][4]) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[kt][i] = st[kt][i];
                mx = fmaxf(mx, x[kt][i]);
            }
        return mx * scale_log2;  // scale_log2 > 0: the scaled maximum is the raw maximum scaled
    }

    // Lazy move of head t's reference maximum: it moves only when a score
    // exceeds it by more than kLazyLog2 (so p <= 2^8 and the fp32 accumulators
    // cannot overflow); O and the row sums are rescaled then (rare).
    __device__ inline void rescale_if(int t, float mx) {
        if (__any(mx > m_thr[t])) {
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = (mx > m_thr[t]) ? mx : m_run[t];
            // 1 if unmoved, 0 from -inf; a row with no visible key keeps m = -inf
            const float alpha = __builtin_amdgcn_exp2f(m_run[t] - (m_new == -INFINITY ? 0.f : m_new));
            m_run[t] = m_new;
            m_neg[t] = -(m_new == -INFINITY ? 0.f : m_new);
            m_thr[t] = m_new + kLazyLog2;
            lsum[t] *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[t][dt] *= alpha;
        }
    }

    // two probabilities as B-operand halves: hi (+ lo) or the rounded pair
    __device__ static inline void pack(float p0, float p1, uint32_t& hi, uint32_t& lo) {
        if (HILO)
            M::split(p0, p1, hi, lo);
        else
            hi = M::round2(p0, p1);
    }

    // P = exp2(scale x - m) of head t as the B operand(s) of the PV MFMA:
    // element 4h + i of lane (lq, lj) is key 16h + 4 lj + i.
    __device__ inline void probs(int t, float (&x)[2][4], float scale_log2, u32x4& phi, u32x4& plo) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[kt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kt][i], scale_log2, m_neg[t]));
        uint32_t hv[4], lv[4] = {0u, 0u, 0u, 0u};
        pack(x[0][0], x[0][1], hv[0], lv[0]);
        pack(x[0][2], x[0][3], hv[1], lv[1]);
        pack(x[1][0], x[1][1], hv[2], lv[2]);
        pack(x[1][2], x[1][3], hv[3], lv[3]);
        phi = u32x4{hv[0], hv[1], hv[2], hv[3]};
        plo = u32x4{lv[0], lv[1], lv[2], lv[3]};
    }

    // V^T fragments of the sub-tile: per d tile two transposing reads give keys
    // 4 lj .. + 4 and 16 + 4 lj .. + 4 of dim 16 dt + lq.
    __device__ inline void read_v(const char* Vs, v8 (&vf)[DT]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vs + voff[dt]));
            const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vs + voff[dt] + 16 * D * 2));
            vf[dt] = __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    }

    // O_t^T += V^T P_t^T and the row sums.
    __device__ inline void pv(int t, const v8 (&vf)[DT], const u32x4& phi, const u32x4& plo) {
        const v8 bh = __builtin_bit_cast(v8, phi), bl = __builtin_bit_cast(v8, plo);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            o[t][dt] = M::mma(vf[dt], bh, o[t][dt]);
            if (HILO) o[t][dt] = M::mma(vf[dt], bl, o[t][dt]);
        }
        lsum[t] = M::mma(ones, bh, lsum[t]);
        if (HILO) lsum[t] = M::mma(ones, bl, lsum[t]);
    }

    // PV(0) with P(1) interleaved in source order: after the two MFMAs of each
    // d tile one probability of head 1 is computed (and, every other tile, a
    // pair is split), so the VALU work issues while the MFMAs execute.
    __device__ inline void pv0_probs1(const v8 (&vf)[DT], const u32x4& h0, const u32x4& l0, float (&x1)[2][4],
                                      float scale_log2, u32x4& h1, u32x4& l1) {
        const v8 bh = __builtin_bit_cast(v8, h0), bl = __builtin_bit_cast(v8, l0);
        float p[8];
        uint32_t hv[4], lv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            o[0][dt] = M::mma(vf[dt], bh, o[0][dt]);
            if (HILO) o[0][dt] = M::mma(vf[dt], bl, o[0][dt]);
            if (dt < 8) {
                p[dt] = __builtin_amdgcn_exp2f(__builtin_fmaf(x1[dt >> 2][dt & 3], scale_log2, m_neg[1]));
                if (dt & 1) pack(p[dt - 1], p[dt], hv[dt >> 1], lv[dt >> 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (DT < 8) {  // head_dim 64: the remaining probabilities
#pragma unroll
            for (int e = DT; e < 8; ++e) {
                p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x1[e >> 2][e & 3], scale_log2, m_neg[1]));
                if (e & 1) pack(p[e - 1], p[e], hv[e >> 1], lv[e >> 1]);
            }
        }
        lsum[0] = M::mma(ones, bh, lsum[0]);
        if (HILO) lsum[0] = M::mma(ones, bl, lsum[0]);
        h1 = u32x4{hv[0], hv[1], hv[2], hv[3]};
        l1 = u32x4{lv[0], lv[1], lv[2], lv[3]};
    }

    // One 32-key sub-tile (Ks / Vs: its first staged K / V row) for both heads,
    // software-pipelined over the two heads so the MFMA work of one overlaps the
    // softmax of the other, each K and V fragment read once for both:
    //   read V, K;  QK(0);  QK(1);  [mask];  max, rescale (0, 1);  P(0);
    //   PV(0) || P(1);  PV(1)
    // MFMAs run asynchronously, so VALU work issued between them overlaps them;
    // the scheduling barriers keep this order.
    // mask: some key may lie beyond some row's position (wave-uniform).
    __device__ inline void step(const char* Ks, const char* Vs, bool mask, int32_t key0, int lj, float scale_log2) {
        v8 vf[DT];
        v8 kf[DS][2];
        read_v(Vs, vf);
        read_k(Ks, kf);
        __builtin_amdgcn_sched_barrier(0);
        compute(kf, vf, mask, key0, lj, scale_log2);
    }

    // The sub-tile's work once its K and V fragments are in registers.
    __device__ inline void compute(const v8 (&kf)[DS][2], const v8 (&vf)[DT], bool mask, int32_t key0, int lj,
                                   float scale_log2) {
        f32x4 s0[2], s1[2];
        float x0[2][4], x1[2][4];
        qk(0, kf, s0);
        qk(1, kf, s1);
        __builtin_amdgcn_sched_barrier(0);
        if (mask) {
            apply_mask(s0, key0, lj);
            apply_mask(s1, key0, lj);
        }
        rescale_if(0, row_max(s0, scale_log2, x0));
        rescale_if(1, row_max(s1, scale_log2, x1));
        finish_subtile(vf, x0, x1, scale_log2);
    }

    // P and PV of both heads from masked, rescaled scores x0 / x1.
    __device__ inline void finish_subtile(const v8 (&vf)[DT], float (&x0)[2][4], float (&x1)[2][4],
                                          float scale_log2) {
        u32x4 h0, l0, h1, l1;
        probs(0, x0, scale_log2, h0, l0);
        __builtin_amdgcn_sched_barrier(0);
        pv0_probs1(vf, h0, l0, x1, scale_log2, h1, l1);
        __builtin_amdgcn_sched_barrier(0);
        pv(1, vf, h1, l1);
    }

    // ---- Software-pipelined stage (one key class: the wave walks every
    // sub-tile of the stage). Sub-tile j's work is split so that the MFMAs of
    // one part issue beside the vector-ALU work of another:
    //   A: P of sub-tile j (both heads)       with the QK MFMAs of sub-tile j + 1
    //   B: PV of sub-tile j (and row sums)    with the row maxima of sub-tile j + 1
    //   C: the lazy rescale for sub-tile j + 1 (rare)
    // Every operation, operand and per-accumulator order is that of step():
    // the results are bit-identical, only independent instructions move.

    // scaled row maximum of one head's scores (the value row_max returns)
    __device__ static inline float scaled_max(const f32x4 (&st)[2], float scale_log2) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[kt][i]);
        return mx * scale_log2;
    }

    // V^T fragment of d tile dt (one tile of read_v).
    __device__ inline v8 read_v_tile(const char* Vs, int dt) {
        const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vs + voff[dt]));
        const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vs + voff[dt] + 16 * D * 2));
        return __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
    }

    // K fragment f of the sub-tile at Ks: k-step f / 2, key tile f % 2 (read_k's kf[f / 2][f % 2]).
    __device__ inline v8 read_k_frag(const char* Ks, int f) {
        return __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(Ks + koff[f >> 1] + 16 * (f & 1) * D * 2));
    }

    // A: probabilities of both heads from scores c0 / c1 (maxima applied), each
    // computed before one QK MFMA of the next sub-tile (K tiles at Ks1) into
    // n0 / n1. The MFMAs go by K fragment, both heads in turn; fragments are
    // read three ahead, each freed after its second MFMA.
    __device__ inline void probs_qk(const f32x4 (&c0)[2], const f32x4 (&c1)[2], const char* Ks1, f32x4 (&n0)[2],
                                    f32x4 (&n1)[2], float scale_log2, u32x4& h0, u32x4& l0, u32x4& h1, u32x4& l1) {
        static_assert(DS == 4, "head_dim 128");
        constexpr int kAhead = 3;
        float p[16];
        uint32_t hv[8], lv[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        v8 kf[2 * DS];
#pragma unroll
        for (int f = 0; f < kAhead; ++f) kf[f] = read_k_frag(Ks1, f);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) n0[kt] = n1[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // probability i: head i / 8, key 16 kt + 4 lj + e with (kt, e) = divmod(i % 8, 4)
            const int e = i & 7;
            const float s = i < 8 ? c0[e >> 2][e & 3] : c1[e >> 2][e & 3];
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s, scale_log2, m_neg[i >> 3]));
            if (i & 1) {
                pack(p[i - 1], p[i], hv[i >> 1], lv[i >> 1]);
                // pinned here: otherwise the compiler sinks the probabilities
                // to their first use in part B, past every QK MFMA (the lo
                // halves only where they exist: a pinned constant 0 costs a move)
                if (HILO)
                    asm volatile("" : "+v"(hv[i >> 1]), "+v"(lv[i >> 1]));
                else
                    asm volatile("" : "+v"(hv[i >> 1]));
            }
            // QK MFMA i: K fragment i / 2 (k-step i / 4, key tile (i / 2) % 2), head i % 2
            // (per accumulator the k-steps go in qk()'s order)
            const int f = i >> 1, ds = i >> 2, kt = f & 1;
            if (i & 1) {
                n1[kt] = M::mma(kf[f], qf[1][ds], n1[kt]);
                if (f + kAhead < 2 * DS) kf[f + kAhead] = read_k_frag(Ks1, f + kAhead);
            } else {
                n0[kt] = M::mma(kf[f], qf[0][ds], n0[kt]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        h0 = u32x4{hv[0], hv[1], hv[2], hv[3]};
        l0 = u32x4{lv[0], lv[1], lv[2], lv[3]};
        h1 = u32x4{hv[4], hv[5], hv[6], hv[7]};
        l1 = u32x4{lv[4], lv[5], lv[6], lv[7]};
    }

    // B: PV of both heads by d tile (V^T fragments read three tiles ahead from
    // Vs, each freed after its two heads' MFMAs), then the row sums; the next
    // sub-tile's scaled row maxima (n0 / n1, masked beforehand where needed)
    // are computed between the MFMAs.
    __device__ inline void pv_max(const char* Vs, const u32x4& h0, const u32x4& l0, const u32x4& h1,
                                  const u32x4& l1, const f32x4 (&n0)[2], const f32x4 (&n1)[2], float scale_log2,
                                  float (&mx)[2]) {
        constexpr int kAhead = 3;
        const v8 b[2][2] = {{__builtin_bit_cast(v8, h0), __builtin_bit_cast(v8, l0)},
                            {__builtin_bit_cast(v8, h1), __builtin_bit_cast(v8, l1)}};
        v8 vf[DT];
#pragma unroll
        for (int dt = 0; dt < kAhead; ++dt) vf[dt] = read_v_tile(Vs, dt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            if (dt + kAhead < DT) vf[dt + kAhead] = read_v_tile(Vs, dt + kAhead);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                o[t][dt] = M::mma(vf[dt], b[t][0], o[t][dt]);
                if (HILO) o[t][dt] = M::mma(vf[dt], b[t][1], o[t][dt]);
            }
            if (dt == 1) {
                mx[0] = scaled_max(n0, scale_log2);
                asm volatile("" : "+v"(mx[0]));  // pinned between the MFMAs
            }
            if (dt == 3) {
                mx[1] = scaled_max(n1, scale_log2);
                asm volatile("" : "+v"(mx[1]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            lsum[t] = M::mma(ones, b[t][0], lsum[t]);
            if (HILO) lsum[t] = M::mma(ones, b[t][1], lsum[t]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // Mask (where a key can lie past a row's last visible key) and lazy rescale
    // of the scores of the sub-tile starting at key0, outside the pipelined parts.
    __device__ inline void mask_rescale(f32x4 (&s0)[2], f32x4 (&s1)[2], bool mask, int32_t key0, int lj,
                                        int32_t last, float scale_log2) {
        if (mask) {
            apply_mask_at(s0, key0, lj, last);
            apply_mask_at(s1, key0, lj, last);
        }
        rescale_if(0, scaled_max(s0, scale_log2));
        rescale_if(1, scaled_max(s1, scale_log2));
    }

    // Sub-tile J of a stage (scores of J in c0 / c1, next scores into n0 / n1).
    template <int J>
    __device__ inline void pipelined_subtile(const char* Ks, const char* Vs, int32_t key0, int32_t mask_from,
                                             int32_t last, int lj, float scale_log2, f32x4 (&c0)[2],
                                             f32x4 (&c1)[2], f32x4 (&n0)[2], f32x4 (&n1)[2]) {
        if (J + 1 < kPairSubs) {
            const int32_t key1 = key0 + kPairSub * (J + 1);
            u32x4 h0, l0, h1, l1;
            probs_qk(c0, c1, Ks + kPairSub * (J + 1) * D * 2, n0, n1, scale_log2, h0, l0, h1, l1);
            if (key1 + kPairSub > mask_from) {
                apply_mask_at(n0, key1, lj, last);
                apply_mask_at(n1, key1, lj, last);
            }
            float mx[2];
            pv_max(Vs + kPairSub * J * D * 2, h0, l0, h1, l1, n0, n1, scale_log2, mx);
            rescale_if(0, mx[0]);
            rescale_if(1, mx[1]);
        } else {
            v8 vf[DT];
            read_v(Vs + kPairSub * J * D * 2, vf);
            __builtin_amdgcn_sched_barrier(0);
            float x0[2][4], x1[2][4];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x0[kt][i] = c0[kt][i];
                    x1[kt][i] = c1[kt][i];
                }
            finish_subtile(vf, x0, x1, scale_log2);
        }
    }

    // All kPairSubs sub-tiles of a staged step, straight-line code (the
    // accumulators stay in their registers): Ks / Vs its K and V tiles, key0
    // the first sub-tile's first key. `last` is this lane's last visible key
    // (its row's position, and before the chunk's end); keys below mask_from
    // are visible to every row of the tile. Sub-tiles past the chunk's end or
    // the tile's causal limit are masked whole: their probabilities are 0 and
    // they add exact zeros (V rows past the chunk's end are zeroed in LDS).
    __device__ inline void stage_pipelined(const char* Ks, const char* Vs, int32_t key0, int32_t mask_from,
                                           int32_t last, int lj, float scale_log2) {
        static_assert(kPairSubs == 4, "four sub-tiles per stage");
        f32x4 sa0[2], sa1[2], sb0[2], sb1[2];
        {
            v8 kf[DS][2];
            read_k(Ks, kf);
            __builtin_amdgcn_sched_barrier(0);
            qk(0, kf, sa0);
            qk(1, kf, sa1);
            __builtin_amdgcn_sched_barrier(0);
        }
        mask_rescale(sa0, sa1, key0 + kPairSub > mask_from, key0, lj, last, scale_log2);
        pipelined_subtile<0>(Ks, Vs, key0, mask_from, last, lj, scale_log2, sa0, sa1, sb0, sb1);
        pipelined_subtile<1>(Ks, Vs, key0, mask_from, last, lj, scale_log2, sb0, sb1, sa0, sa1);
        pipelined_subtile<2>(Ks, Vs, key0, mask_from, last, lj, scale_log2, sa0, sa1, sb0, sb1);
        pipelined_subtile<3>(Ks, Vs, key0, mask_from, last, lj, scale_log2, sb0, sb1, sa0, sa1);
    }
};

template <typename T, int D, int RT, bool HILO>
__device__ inline void pair_finish(const AttnArgs& a, PairWave<T, D, HILO>& w, char* smem, int hp, int rt, int kq,
                                   int lane, int lq, int lj, int work, int n_chunks, int head0, int64_t row0,
                                   int32_t kmax, int32_t key_begin);

template <typename T, int D, int RT, bool HILO>
__global__ void __launch_bounds__(kPairThreads) attn_pair_kernel(AttnArgs a) {
    using C = PairCfg<D>;
    using W = PairWave<T, D, HILO>;
    using v8 = typename W::v8;
    constexpr int X = 8 / (2 * RT);  // key classes per head pair
    constexpr int GR = kRowTile * RT;
    extern __shared__ __align__(16) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 15;
    const int lj = lane >> 4;
    const int hp = wave & 1;              // head pair of the block's four query heads
    const int rt = (wave >> 1) % RT;      // row tile within the group
    const int kq = (wave >> 1) / RT;      // key class

    const int work = blockIdx.y;
    const int32_t* wk = work_table_of(a) + kWorkInts * work;
    const int grp = wk[0];
    const int32_t key_begin = wk[2];
    const int32_t key_end = wk[3];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int head0 = kv_head * a.group + hg * 4 + 2 * hp;
    const int64_t row0 = static_cast<int64_t>(grp) * GR + kRowTile * rt;

    const char* kbase = a.k + (static_cast<int64_t>(kv_head) * a.ks[0] + static_cast<int64_t>(key_begin) * a.ks[1]) * 2;
    const char* vbase = a.v + (static_cast<int64_t>(kv_head) * a.vs[0] + static_cast<int64_t>(key_begin) * a.vs[1]) * 2;
    const int32_t n_keys_chunk = key_end - key_begin;
    const int n_sub = (n_keys_chunk + kPairSub - 1) / kPairSub;
    const int n_it = (n_keys_chunk + kPairStepKeys - 1) / kPairStepKeys;

    // Direct global -> LDS loads of step i into stage buffer `stage`: each load
    // instruction of a wave fills 1 KB of LDS (64 lanes x 16 bytes, lane order);
    // lane L of block b writes swizzled position (row, c') = divmod(64 b + L, D/8)
    // and so loads piece c' ^ (row mod D/8) of that key row. Rows past the chunk
    // end re-read its last row (in bounds); they are masked or zeroed later.
    StepLoads<D> sl;
    sl.init(wave, lane);
    const uint32_t koff = sl.lane_offset(a.ks[1], false);
    const uint32_t voff = sl.lane_offset(a.vs[1], true);
    auto load = [&](int i, char* stage) {
        sl.issue(kbase, a.ks[1], koff, kPairStepKeys * i, n_keys_chunk, stage, wave, false);
        sl.issue(vbase, a.vs[1], voff, kPairStepKeys * i, n_keys_chunk, stage + C::tensor_bytes, wave, true);
    };

    // Prologue, one round trip: the row positions and Q fragments are loaded
    // (unconditionally, from rows clamped into range; n_sel >= 1 whenever a
    // work item exists), then the first stage's K/V loads are issued, then all
    // of them are waited for at once. Consuming the values through the empty
    // asm below keeps the compiler's waits for them here, not inside the loop,
    // where a vmcnt wait would also stall on the next stage's loads.
    W w;
    int32_t kmax, nomask_end;
    {
        const int64_t row = row0 + lq;
        const int64_t last_sel = a.n_sel - 1;
        const int64_t row_c = row < last_sel ? row : last_sel;
        const int64_t tile_last = row0 + kRowTile - 1 < last_sel ? row0 + kRowTile - 1 : last_sel;
        const int64_t tile_first = row0 < last_sel ? row0 : last_sel;
        // positions are below n_keys < 2^31: their low words (little-endian)
        const int32_t* pos32 = reinterpret_cast<const int32_t*>(a.positions);
        int32_t pos_raw = pos32[2 * row_c];
        int32_t kmax_raw = pos32[2 * tile_last];
        int32_t first_raw = pos32[2 * tile_first];
        u32x4 raw[2][W::DS];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ds = 0; ds < W::DS; ++ds) {
                const int64_t off = (head0 + t) * a.qs[0] + row_c * a.qs[1] + (32 * ds + 8 * lj);
                raw[t][ds] = *reinterpret_cast<const u32x4*>(a.q + off * 2);
            }
        if (n_it > 0) load(0, smem);
        asm volatile("" : "+v"(pos_raw), "+v"(kmax_raw), "+v"(first_raw));
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ds = 0; ds < W::DS; ++ds) asm volatile("" : "+v"(raw[t][ds]));
        const bool live_row = row < a.n_sel;
        // the tile's limits are the same in every lane (each lane loaded the
        // same two positions): held in scalar registers, the loop's sub-tile
        // counts and mask tests are scalar branches
        kmax = __builtin_amdgcn_readfirstlane(row0 < a.n_sel ? kmax_raw + 1 : 0);
        nomask_end = __builtin_amdgcn_readfirstlane((row0 + kRowTile <= a.n_sel) ? first_raw + 1 : 0);
        w.pos = live_row ? pos_raw : -1;
        w.init(lq, lj);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ds = 0; ds < W::DS; ++ds)
                w.qf[t][ds] = __builtin_bit_cast(v8, live_row ? raw[t][ds] : u32x4{0u, 0u, 0u, 0u});
    }

    for (int i = 0; i < n_it; ++i) {
        char* stage = smem + (i & 1) * C::stage_bytes;
        // stage i has landed (this wave's loads) and every wave is past step i - 1,
        // so stage (i + 1) & 1 is free for the next loads
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int32_t left = n_keys_chunk - kPairStepKeys * i;
        if (left < kPairStepKeys) {
            // the chunk ends inside this step: zero the V rows past its end (their
            // probabilities are 0, and 0 * V must stay 0 whatever V holds there)
            for (int e = tid; e < (kPairStepKeys - left) * C::c8; e += kPairThreads)
                *reinterpret_cast<u32x4*>(stage + C::tensor_bytes + left * D * 2 + 16 * e) = u32x4{0u, 0u, 0u, 0u};
            __syncthreads();
        }
        if (i + 1 < n_it) load(i + 1, smem + ((i + 1) & 1) * C::stage_bytes);
        const char* Ks = stage;
        const char* Vs = stage + C::tensor_bytes;
        if constexpr (X == 1 && D == 128) {
            // every sub-tile of the step, software-pipelined, when any of them
            // lies inside the chunk and starts below the tile's causal limit
            const int32_t key0 = key_begin + kPairStepKeys * i;
            if (key0 < kmax)
                w.stage_pipelined(Ks, Vs, key0, min(nomask_end, key_end), min(w.pos, key_end - 1), lj,
                                  a.scale_log2);
        } else {
#pragma unroll 1
            for (int j = kq; j < kPairSubs; j += X) {
                const int s = kPairSubs * i + j;
                const int32_t key0 = key_begin + kPairSub * s;
                if (s < n_sub && key0 < kmax)
                    w.step(Ks + kPairSub * j * D * 2, Vs + kPairSub * j * D * 2, key0 + kPairSub > nomask_end, key0,
                           lj, a.scale_log2);
            }
        }
    }
    pair_finish<T, D, RT, HILO>(a, w, smem, hp, rt, kq, lane, lq, lj, work, n_chunks, head0, row0, kmax, key_begin);
}

// LDS bytes of pair_finish's exchange: per (head pair, row tile), class and
// head the D / 16 - D / 16 / X d tiles the class does not own (64 lanes x 16
// bytes each), then (m, l) per class, head and lane.
__host__ __device__ constexpr size_t pair_exchange_bytes(int D, int RT) {
    return RT == 4 ? 0
                   : static_cast<size_t>(2 * RT) * (8 / (2 * RT)) * 2 *
                         ((D / 16 - D / 16 / (8 / (2 * RT))) * 64 * 16 + 64 * 8);
}

// Row sums, the combine of the key classes of each (head pair, row tile)
// through LDS (every wave of the block calls it, after its last step), and the
// output (one chunk) or the chunk's partial (m, l, O). With X key classes,
// wave kq of a (head pair, row tile) combines and writes d tiles
// [SL kq, SL (kq + 1)) of all X classes' O, so the combine's LDS reads and the
// stores are spread over every wave: each wave first puts its (m, l) and the
// d tiles it does not own into LDS (f32x4 per lane and tile).
template <typename T, int D, int RT, bool HILO>
__device__ inline void pair_finish(const AttnArgs& a, PairWave<T, D, HILO>& w, char* smem, int hp, int rt, int kq,
                                   int lane, int lq, int lj, int work, int n_chunks, int head0, int64_t row0,
                                   int32_t kmax, int32_t key_begin) {
    using W = PairWave<T, D, HILO>;
    constexpr int X = 8 / (2 * RT);  // key classes per head pair
    constexpr int GR = kRowTile * RT;
    constexpr int SL = W::DT / X;    // d tiles each wave writes
    static_assert(SL * X == W::DT, "d tiles split evenly over the key classes");
    // ---- row sums: row 0 of the sum tile, i.e. element 0 of lane lq (lj = 0);
    // the other lanes hold zeros, so the sum over the lane groups broadcasts it ----
    float l_run[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float l = w.lsum[t][0];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run[t] = l;
    }
    f32x4 res[2][SL];  // this wave's d tiles [SL kq, SL (kq + 1)) of both heads
    float m_out[2];
    if constexpr (X == 1) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            m_out[t] = w.m_run[t];
#pragma unroll
            for (int j = 0; j < SL; ++j) res[t][j] = w.o[t][j];
        }
    } else {
        // exchange layout (head pair, row tile) -> class c -> head t -> the
        // W::DT - SL d tiles c does not own, in order -> lane; then (m, l)
        constexpr int kTiles = W::DT - SL;
        const int unit = hp * RT + rt;
        f32x4* xo = reinterpret_cast<f32x4*>(smem);
        float2* xml = reinterpret_cast<float2*>(smem + static_cast<size_t>(2 * RT) * X * 2 * kTiles * 64 * 16);
        auto o_at = [&](int c, int t, int dt) {  // dt not owned by class c
            const int k = dt < SL * c ? dt : dt - SL;
            return xo + ((((unit * X + c) * 2 + t) * kTiles + k) * 64 + lane);
        };
        __syncthreads();  // every wave is done with the K/V stages
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int dt = 0; dt < W::DT; ++dt)
                if (dt / SL != kq) *o_at(kq, t, dt) = w.o[t][dt];
            xml[((unit * X + kq) * 2 + t) * 64 + lane] = float2{w.m_run[t], l_run[t]};
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float mc[X], lc[X];
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < X; ++c) {
                const float2 ml = c == kq ? float2{w.m_run[t], l_run[t]} : xml[((unit * X + c) * 2 + t) * 64 + lane];
                mc[c] = ml.x;
                lc[c] = ml.y;
                m = fmaxf(m, mc[c]);
            }
            // a row with no visible key in the chunk keeps O = 0, l = 0, m = -inf
            const float m_use = m == -INFINITY ? 0.f : m;
            float l = 0.f;
#pragma unroll
            for (int j = 0; j < SL; ++j) res[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < X; ++c) {
                const float f = __builtin_amdgcn_exp2f(mc[c] - m_use);  // 0 for an empty class
                l += lc[c] * f;
#pragma unroll
                for (int j = 0; j < SL; ++j) {
                    f32x4 oc;
                    if (c == kq) {
                        // own d tiles: a select over the registers (no dynamic register indexing)
                        oc = w.o[t][j];
#pragma unroll
                        for (int k = 1; k < X; ++k)
                            if (k == kq) oc = w.o[t][SL * k + j];
                    } else {
                        oc = *o_at(c, t, SL * kq + j);
                    }
                    res[t][j] += oc * f;
                }
            }
            m_out[t] = m;
            l_run[t] = l;
        }
    }

    // ---- output (one chunk) or the chunk's partial: d tiles [SL kq, SL (kq + 1)) ----
    const int r = kRowTile * rt + lq;  // row within the group
    const int64_t row = row0 + lq;
    if (kmax <= key_begin || row >= a.n_sel) return;  // the tile does not attend into this chunk
    const int dt0 = X == 1 ? 0 : SL * kq;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int q_head = head0 + t;
        if (n_chunks == 1) {
            const float inv = 1.f / l_run[t];
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + q_head * a.os[0] + row * a.os[1];
#pragma unroll
            for (int j = 0; j < SL; ++j) {
                uint16_t e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = elem<T>::from_float(res[t][j][i] * inv);
                const int d0 = 16 * (dt0 + j) + 4 * lj;
                if (a.out_vec) {
                    *reinterpret_cast<uint2*>(dst + d0) =
                        uint2{e[0] | (static_cast<uint32_t>(e[1]) << 16), e[2] | (static_cast<uint32_t>(e[3]) << 16)};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dst[(d0 + i) * a.os[2]] = e[i];
                }
            }
        } else {
            const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * GR + r;
            float* po = a.ws_o + slot * D;
#pragma unroll
            for (int j = 0; j < SL; ++j) *reinterpret_cast<f32x4*>(po + 16 * (dt0 + j) + 4 * lj) = res[t][j];
            if (kq == 0 && lj == 0) {
                a.ws_ml[slot * 2 + 0] = m_out[t];
                a.ws_ml[slot * 2 + 1] = l_run[t];
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
    const int work = blockIdx.y;
    const int32_t* wk = work_table_of(a) + kWorkInts * work;
    const int grp = wk[0];
    const int64_t key_begin = wk[2];
    const int64_t key_end = wk[3];
    const int n_chunks = group_table(a.sched)[2 * grp + 1];
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;

    const int64_t group_row0 = static_cast<int64_t>(grp) * a.group_rows;
    const int tile = tid / 64;
    const int h = (tid % 64) / kRowTile;
    const int r = tile * kRowTile + (tid % kRowTile);
    const int64_t row = group_row0 + r;
    const bool live = h < a.qt && r < a.group_rows && row < a.n_sel;
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
        const int64_t slot = (static_cast<int64_t>(q_head) * a.n_work + work) * a.group_rows + r;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) a.ws_o[slot * D + d] = acc[d];
        a.ws_ml[slot * 2 + 0] = m_run;
        a.ws_ml[slot * 2 + 1] = l_run;
    }
}

// ===========================================================================
// Merge of multi-chunk groups. Grid x = KV head x head group (as the main
// kernel, so a head's merge blocks run on the XCD whose L2 holds its
// partials), grid y = (group, query head of the head group, block of rows).
// Phase 1 finds, per row, the chunks its tile attended into (a prefix of the
// group's chunks: those starting below the tile's causal limit) and stages
// their weights exp2(m_c - M) and 1 / l in LDS. Phase 2 gives each thread VEC
// dims of one row and one of kSlices interleaved chunk slices, so a thread's
// loads are independent; the slices are summed through LDS.
// ===========================================================================
constexpr int kMergeThreads = 256;
constexpr int kSlices = 4;

__host__ __device__ inline int merge_rows_per_block(int head_dim, int vec) {
    const int per_row = kSlices * (head_dim / vec);
    const int rows = kMergeThreads / per_row;
    return rows < 1 ? 1 : (rows > 8 ? 8 : rows);
}

template <typename T, int VEC>
__global__ void __launch_bounds__(kMergeThreads) attn_merge_kernel(AttnArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    typedef float fvec __attribute__((ext_vector_type(VEC)));
    extern __shared__ __align__(16) char smem[];
    const int D = a.head_dim;
    const int RB = merge_rows_per_block(D, VEC);
    const int GR = a.group_rows;
    const int blocks_per_group = a.qt * ((GR + RB - 1) / RB);
    const int grp = blockIdx.y / blocks_per_group;
    const int rem = blockIdx.y - grp * blocks_per_group;
    const int hq = rem / ((GR + RB - 1) / RB);
    const int r0 = (rem - hq * ((GR + RB - 1) / RB)) * RB;  // first row (within the group)
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int q_head = kv_head * a.group + hg * a.qt + hq;
    const int32_t* gt = group_table(a.sched);
    const int base = gt[2 * grp];
    const int n_chunks = gt[2 * grp + 1];
    if (n_chunks <= 1) return;
    const int32_t* wk = work_table_of(a) + kWorkInts * base;
    float* Red = reinterpret_cast<float*>(smem);          // [RB][kSlices][D] (16-byte aligned)
    float* W = Red + RB * kSlices * D;                     // [RB][n_chunks]
    float* Linv = W + RB * n_chunks;                       // [RB]
    int* NV = reinterpret_cast<int*>(Linv + RB);           // [RB] attended chunks
    const int64_t slot0 = (static_cast<int64_t>(q_head) * a.n_work + base) * GR;
    const int64_t group_row0 = static_cast<int64_t>(grp) * GR;
    const int64_t cstride = static_cast<int64_t>(GR);

    // The partial O of this thread's first (row, slice, VEC dims) item for its
    // first kPre chunks is loaded before phase 1 (every slot of the group is
    // in bounds; slots of chunks a row does not attend hold stale values and
    // are selected away), so the loads of both phases overlap.
    const int dv = D / VEC;
    constexpr int kPre = 4;
    fvec pre[kPre];
    {
        const int e = threadIdx.x;
        const int rr = e / (kSlices * dv);
        const int sl = (e / dv) % kSlices;
        const int d = (e % dv) * VEC;
        const int r = r0 + rr;
        const bool live = e < RB * kSlices * dv && r < GR && group_row0 + r < a.n_sel;
        const float* po = a.ws_o + (slot0 + (live ? r : 0)) * D + (live ? d : 0);
#pragma unroll
        for (int j = 0; j < kPre; ++j) {
            const int c = sl + kSlices * j;
            pre[j] = fvec{};
            if (live && c < n_chunks) pre[j] = *reinterpret_cast<const fvec*>(po + c * cstride * D);
        }
    }

    // phase 1: one wave per row
    const int wave = threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    for (int rr = wave; rr < RB; rr += kMergeThreads / 64) {
        const int r = r0 + rr;
        const int64_t row = group_row0 + r;
        int nv = 0;
        if (r < GR && row < a.n_sel) {
            if (n_chunks <= 64) {
                // one lane per chunk: the chunk start, m and l loads are independent of the row limit
                const bool in = lane < n_chunks;
                const int64_t s = (slot0 + (in ? lane : 0) * cstride + r) * 2;
                const int32_t kb = in ? wk[kWorkInts * lane + 2] : 0;
                const float mc = a.ws_ml[s];
                const float lc = a.ws_ml[s + 1];
                const int32_t tk = rows_kmax(a, group_row0 + (r / kRowTile) * kRowTile, kRowTile);
                // chunk starts increase, so the attended chunks are a prefix
                const bool att = in && kb < tk;
                nv = __popcll(__ballot(att));
                float mx = att ? mc : -INFINITY;
                for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                const float m_use = (mx == -INFINITY) ? 0.f : mx;
                float l = 0.f;
                if (att) {
                    const float w = exp2f(mc - m_use);
                    W[rr * n_chunks + lane] = w;
                    l = w * lc;
                }
                for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
                if (lane == 0) Linv[rr] = 1.f / l;
            } else {
                const int32_t tk = rows_kmax(a, group_row0 + (r / kRowTile) * kRowTile, kRowTile);
                for (int c0 = 0; c0 < n_chunks; c0 += 64) {
                    const int c = c0 + lane;
                    nv += __popcll(__ballot(c < n_chunks && wk[kWorkInts * c + 2] < tk));
                }
                float mx = -INFINITY;
                for (int c = lane; c < nv; c += 64) mx = fmaxf(mx, a.ws_ml[(slot0 + c * cstride + r) * 2]);
                for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                const float m_use = (mx == -INFINITY) ? 0.f : mx;
                float l = 0.f;
                for (int c = lane; c < nv; c += 64) {
                    const int64_t s = (slot0 + c * cstride + r) * 2;
                    const float w = exp2f(a.ws_ml[s] - m_use);
                    W[rr * n_chunks + c] = w;
                    l += w * a.ws_ml[s + 1];
                }
                for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
                if (lane == 0) Linv[rr] = 1.f / l;
            }
        }
        if (lane == 0) NV[rr] = nv;
    }
    __syncthreads();

    // phase 2: (row, slice, VEC dims) per thread-iteration, chunks in slice order
    for (int e = threadIdx.x; e < RB * kSlices * dv; e += kMergeThreads) {
        const int rr = e / (kSlices * dv);
        const int sl = (e / dv) % kSlices;
        const int d = (e % dv) * VEC;
        const int r = r0 + rr;
        fvec acc = {};
        if (r < GR && group_row0 + r < a.n_sel) {
            const int nv = NV[rr];
            const float* po = a.ws_o + (slot0 + r) * D + d;
            const float* w = W + rr * n_chunks;
            int c = sl;
            if (e == static_cast<int>(threadIdx.x)) {
#pragma unroll
                for (int j = 0; j < kPre; ++j, c += kSlices)
                    if (c < nv) acc += w[c] * pre[j];
            }
#pragma unroll 8
            for (; c < nv; c += kSlices)
                acc += w[c] * *reinterpret_cast<const fvec*>(po + c * cstride * D);
        }
        *reinterpret_cast<fvec*>(Red + (rr * kSlices + sl) * D + d) = acc;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < RB * D; e += kMergeThreads) {
        const int rr = e / D;
        const int d = e - rr * D;
        const int r = r0 + rr;
        const int64_t row = group_row0 + r;
        if (r >= GR || row >= a.n_sel) continue;
        float sum = 0.f;
#pragma unroll
        for (int sl = 0; sl < kSlices; ++sl) sum += Red[(rr * kSlices + sl) * D + d];
        bits* op = reinterpret_cast<bits*>(a.out) + q_head * a.os[0] + row * a.os[1];
        op[d * a.os[2]] = E::from_float(sum * Linv[rr]);
    }
}

// ===========================================================================
// Single-pass merge (head_dim 64 / 128): one thread per 4 output dims of one
// (query head, row) -- 32 or 16 threads per row -- combines the row's chunk
// partials online, kBatch chunks at a time with all their (m, l) and O loads
// in flight together: running max M, weights exp2(m_c - M), the sum and O
// rescaled when M grows. No LDS, no barrier, one memory round trip per batch.
// Grid x = KV head x head group (as the main kernel), y = (group, block of
// rows) over multi-chunk groups; blocks of single-chunk groups return.
// ===========================================================================
constexpr int kFlatThreads = 256;

template <typename T, int D>
__global__ void __launch_bounds__(kFlatThreads) attn_merge_flat_kernel(AttnArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int kTpp = D / 4;                    // threads per (query head, row)
    constexpr int kPpb = kFlatThreads / kTpp;      // rows (x heads) per block
    constexpr int kBatch = 8;
    const int GR = a.group_rows;
    const int per_group = a.qt * GR;
    const int blocks_per_group = (per_group + kPpb - 1) / kPpb;
    const int grp = blockIdx.y / blocks_per_group;
    const int item = (blockIdx.y - grp * blocks_per_group) * kPpb + threadIdx.x / kTpp;
    const int d0 = (threadIdx.x % kTpp) * 4;
    const int32_t* gt = group_table(a.sched);
    const int base = gt[2 * grp];
    const int n_chunks = gt[2 * grp + 1];
    if (n_chunks <= 1 || item >= per_group) return;
    const int hq = item / GR;
    const int r = item - hq * GR;
    const int64_t row = static_cast<int64_t>(grp) * GR + r;
    if (row >= a.n_sel) return;
    const int kv_head = blockIdx.x / a.n_head_groups;
    const int hg = blockIdx.x - kv_head * a.n_head_groups;
    const int q_head = kv_head * a.group + hg * a.qt + hq;
    // The chunks this row's tile attended: those starting below its causal
    // limit (a prefix). A one-tile group's key range ends at that limit, so
    // its tile attends every chunk; only groups of several tiles need the
    // (dependent) position and work-table reads.
    int nv = n_chunks;
    if (GR > kRowTile) {
        const int32_t tk = rows_kmax(a, static_cast<int64_t>(grp) * GR + (r / kRowTile) * kRowTile, kRowTile);
        const int32_t* wk = work_table_of(a) + kWorkInts * base;
        nv = 0;
        while (nv < n_chunks && wk[kWorkInts * nv + 2] < tk) ++nv;
    }
    const int64_t slot0 = (static_cast<int64_t>(q_head) * a.n_work + base) * GR + r;
    float m = -INFINITY, l = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nv; c0 += kBatch) {
        f32x2 ml[kBatch];
        f32x4 o[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int64_t slot = slot0 + static_cast<int64_t>(c0 + j < nv ? c0 + j : nv - 1) * GR;
            ml[j] = *reinterpret_cast<const f32x2*>(a.ws_ml + slot * 2);
            o[j] = *reinterpret_cast<const f32x4*>(a.ws_o + slot * D + d0);
        }
        float mb = m;
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (c0 + j < nv) mb = fmaxf(mb, ml[j][0]);
        const float m_use = mb == -INFINITY ? 0.f : mb;
        const float f = __builtin_amdgcn_exp2f(m - m_use);  // 0 while m is -inf
        l *= f;
        acc *= f;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (c0 + j >= nv) continue;
            const float w = __builtin_amdgcn_exp2f(ml[j][0] - m_use);
            l += w * ml[j][1];
            acc += w * o[j];
        }
        m = mb;
    }
    const float inv = 1.f / l;
    bits e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = E::from_float(acc[i] * inv);
    bits* dst = reinterpret_cast<bits*>(a.out) + q_head * a.os[0] + row * a.os[1];
    if (sizeof(bits) == 2 && a.out_vec) {
        uint32_t w0, w1;
        __builtin_memcpy(&w0, e, 4);
        __builtin_memcpy(&w1, e + 2, 4);
        *reinterpret_cast<uint2*>(dst + d0) = uint2{w0, w1};
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(d0 + i) * a.os[2]] = e[i];
    }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
int pick_qt(int group) {
    if (group % 4 == 0 && KVR_ATTN_MAX_QT >= 4) return 4;
    if (group % 2 == 0 && KVR_ATTN_MAX_QT >= 2) return 2;
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
    using C = MfmaCfg<D, QT>;
    static const bool ok = allow_lds(attn_mfma_kernel<T, D, QT>, C::bytes);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_mfma_kernel<T, D, QT><<<grid, C::threads, C::bytes, s>>>(a);
    return launch_status();
}

template <typename T, int D, int QT>
int launch_tile_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    using C = MfmaCfg<D, QT>;
    constexpr size_t bytes = 2 * static_cast<size_t>(C::bytes);  // two sub-tiles per stage
    static_assert(bytes >= static_cast<size_t>(QT) * (D / 16 * 4 + 2) * 64 * 4, "head exchange fits");
    static const bool ok = allow_lds(attn_tile_kernel<T, D, QT>, bytes);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_tile_kernel<T, D, QT><<<grid, C::threads, bytes, s>>>(a);
    return launch_status();
}

template <typename T, int D, int RT, bool HILO>
int launch_pair_inst(const AttnArgs& a, dim3 grid, hipStream_t s) {
    constexpr size_t bytes = PairCfg<D>::bytes;
    static_assert(bytes >= pair_exchange_bytes(D, RT), "key-class exchange fits the stages");
    static const bool ok = allow_lds(attn_pair_kernel<T, D, RT, HILO>, bytes);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    attn_pair_kernel<T, D, RT, HILO><<<grid, kPairThreads, bytes, s>>>(a);
    return launch_status();
}

template <typename T, int D>
int launch_mfma(const AttnArgs& a, int qt, dim3 grid, hipStream_t s) {
    if (qt == 4 && KVR_ATTN_PAIR) {
        if (a.p_rounded) {
            if (a.group_rows == kTileGroupRows) return launch_pair_inst<T, D, 1, false>(a, grid, s);
            return launch_pair_inst<T, D, 4, false>(a, grid, s);
        }
        if (a.group_rows == kTileGroupRows) return launch_pair_inst<T, D, 1, true>(a, grid, s);
        return launch_pair_inst<T, D, 4, true>(a, grid, s);
    }
    if (a.group_rows == kTileGroupRows) {
        if (qt == 4) return launch_tile_inst<T, D, 4>(a, grid, s);
        if (qt == 2) return launch_tile_inst<T, D, 2>(a, grid, s);
        return launch_tile_inst<T, D, 1>(a, grid, s);
    }
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

size_t merge_lds_bytes(int max_chunks, int head_dim, int vec) {
    const int rb = merge_rows_per_block(head_dim, vec);
    return (static_cast<size_t>(rb) * max_chunks + 2 * rb + static_cast<size_t>(rb) * kSlices * head_dim) *
           sizeof(float);
}

template <typename T, int VEC>
int launch_merge_vec(const AttnArgs& a, int max_chunks, hipStream_t s) {
    static const bool ok = allow_lds(attn_merge_kernel<T, VEC>, merge_lds_bytes(kMaxChunksPerGroup, 256, VEC));
    if (!ok) return KVR_E_LAUNCH_FAILED;
    const int rb = merge_rows_per_block(a.head_dim, VEC);
    const unsigned y = static_cast<unsigned>(a.n_groups) * a.qt * ((a.group_rows + rb - 1) / rb);
    if (y > 65535u) return KVR_E_UNSUPPORTED_SHAPE;
    dim3 grid(a.n_q_heads / a.qt, y);
    attn_merge_kernel<T, VEC><<<grid, kMergeThreads, merge_lds_bytes(max_chunks, a.head_dim, VEC), s>>>(a);
    return launch_status();
}

template <typename T, int D>
int launch_merge_flat(const AttnArgs& a, hipStream_t s) {
    constexpr int ppb = kFlatThreads / (D / 4);
    const int64_t blocks_per_group = (static_cast<int64_t>(a.qt) * a.group_rows + ppb - 1) / ppb;
    const int64_t y = static_cast<int64_t>(a.n_groups) * blocks_per_group;
    if (y > 65535) return KVR_E_UNSUPPORTED_SHAPE;
    const dim3 grid(static_cast<unsigned>(a.n_q_heads / a.qt), static_cast<unsigned>(y));
    attn_merge_flat_kernel<T, D><<<grid, kFlatThreads, 0, s>>>(a);
    return launch_status();
}

template <typename T>
int launch_merge(const AttnArgs& a, int max_chunks, hipStream_t s) {
    if (a.head_dim == 128) return launch_merge_flat<T, 128>(a, s);
    if (a.head_dim == 64) return launch_merge_flat<T, 64>(a, s);
    return a.head_dim % 4 == 0 ? launch_merge_vec<T, 4>(a, max_chunks, s) : launch_merge_vec<T, 1>(a, max_chunks, s);
}

// Per-group causal limits on the host: group limit and the limits of its row
// tiles (group_rows / 16 of them; unused entries 0).
struct GroupKeys {
    int64_t kmax;
    int64_t tile_kmax[kTilesPerGroup];
};

GroupKeys group_keys(const int64_t* positions, int64_t n_sel, int64_t g, int group_rows) {
    GroupKeys k;
    const int64_t last = (g + 1) * group_rows - 1 < n_sel ? (g + 1) * group_rows - 1 : n_sel - 1;
    k.kmax = positions[last] + 1;
    for (int t = 0; t < kTilesPerGroup; ++t) {
        const int64_t row0 = g * group_rows + t * kRowTile;
        if (t * kRowTile >= group_rows || row0 >= n_sel) {
            k.tile_kmax[t] = 0;
            continue;
        }
        const int64_t tl = row0 + kRowTile - 1 < n_sel ? row0 + kRowTile - 1 : n_sel - 1;
        k.tile_kmax[t] = positions[tl] + 1;
    }
    return k;
}

// Cost of one 64-key sub-tile: staging it (every sub-tile) plus the MFMA work
// of each row tile that still attends to it.
constexpr int64_t kCostStage = 3;
constexpr int64_t kCostTile = 1;

int64_t subtile_cost(const GroupKeys& k, int64_t s) {
    int64_t c = kCostStage;
    for (int t = 0; t < kTilesPerGroup; ++t) c += (k.tile_kmax[t] > s * kSub) ? kCostTile : 0;
    return c;
}

struct Chunk {
    int32_t group, index, begin, end;
};

// Modelled cost of one block besides its sub-tiles (dispatch, prologue, the
// key-class combine and the partial stores), and of merging one chunk of a split
// group (its partials written and read back), in sub-tile cost units.
constexpr int64_t kCostBlock = 16;
constexpr int64_t kCostMergeChunk = 2;

int64_t chunk_cost(const GroupKeys& k, const Chunk& c) {
    int64_t cost = 0;
    for (int64_t s = c.begin / kSub; s < (c.end + kSub - 1) / kSub; ++s) cost += subtile_cost(k, s);
    return cost;
}

// Longest-first order: whole groups (their chunks stay contiguous and in chunk
// order, as the merge reads them) sorted by their chunks' largest cost, so the
// blocks that take longest are dispatched first and the cheap ones fill in.
void order_longest_first(const std::vector<GroupKeys>& keys, std::vector<Chunk>& chunks) {
    std::vector<int64_t> worst(keys.size(), 0);
    for (const Chunk& c : chunks) worst[c.group] = std::max(worst[c.group], chunk_cost(keys[c.group], c));
    std::stable_sort(chunks.begin(), chunks.end(), [&](const Chunk& a, const Chunk& b) {
        if (a.group == b.group) return a.index < b.index;
        return worst[a.group] > worst[b.group] || (worst[a.group] == worst[b.group] && a.group < b.group);
    });
}

// Modelled span of one head's blocks in dispatch order on the `cus` CUs its
// blocks run on (the blocks of one head land on that head's XCD): each block
// goes to the CU that frees first; split groups add their merge work.
int64_t schedule_span(const std::vector<GroupKeys>& keys, std::vector<Chunk>& chunks, int64_t cus) {
    order_longest_first(keys, chunks);
    std::vector<int64_t> load(static_cast<size_t>(cus > 0 ? cus : 1), 0);
    std::vector<int32_t> count(keys.size(), 0);
    for (const Chunk& c : chunks) {
        auto least = std::min_element(load.begin(), load.end());
        *least += chunk_cost(keys[c.group], c) + kCostBlock;
        ++count[c.group];
    }
    int64_t merge = 0;
    for (int32_t n : count) merge += n > 1 ? n * kCostMergeChunk : 0;
    return *std::max_element(load.begin(), load.end()) + merge;
}

// ---------------------------------------------------------------------------
// Static scratch of kvr_packed_causal_attention_noalloc: the split-K partials
// live in this file-scope device array instead of a caller workspace. Each
// device that runs the library holds its own copy until the process ends. In
// host code the array's name is only a stand-in for the device symbol: the
// device address comes from hipGetSymbolAddress, looked up once per device
// (with that device current) and kept per device.
// ---------------------------------------------------------------------------
// Size in MiB, set at build time with -DKVR_ATTN_SCRATCH_MB=<n> (default 128:
// every c1-c5 schedule fits; the largest, c4, needs 68 MB).
#ifndef KVR_ATTN_SCRATCH_MB
#define KVR_ATTN_SCRATCH_MB 128
#endif
static_assert(KVR_ATTN_SCRATCH_MB >= 1 && KVR_ATTN_SCRATCH_MB <= 4096, "KVR_ATTN_SCRATCH_MB out of range");
constexpr int64_t kScratchBytes = int64_t(KVR_ATTN_SCRATCH_MB) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
// Ordering of the calls that use one device's array: the completion event of
// the last call enqueued outside graph capture, and its stream. A call on
// another stream first waits for that event on the device, so two such calls
// never overlap (no host blocking, no rejection of correctly ordered callers).
hipEvent_t g_scratch_done[kMaxDevices] = {};
hipStream_t g_scratch_last[kMaxDevices] = {};
bool g_scratch_used[kMaxDevices] = {};

// Device address of `scratch` on the device of `stream` (which must be the
// current device), and that device; nullptr when the lookup fails. The first
// call on a device also creates its ordering event (no device allocation).
void* scratch_address(void* stream, int* device) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess || current < 0 || current >= kMaxDevices) return nullptr;
    if (stream) {
        int owner = -1;
        if (hipStreamGetDevice(as_stream(stream), &owner) != hipSuccess || owner != current) return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[current]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        if (!g_scratch_done[current] &&
            hipEventCreateWithFlags(&g_scratch_done[current], hipEventDisableTiming) != hipSuccess) {
            g_scratch_done[current] = nullptr;
            return nullptr;
        }
        g_scratch_ptr[current] = ptr;
    }
    *device = current;
    return g_scratch_ptr[current];
}

// Serialises the calls on one device's scratch array for the duration of an
// enqueue: outside graph capture, a call on a stream other than the previous
// call's waits on the device for the previous call's completion event, and
// records its own when its launches are enqueued. Under capture (where a
// wait on an event recorded outside the graph is not allowed) neither
// happens: replays of captured calls must be ordered by the caller.
class ScratchOrder {
  public:
    ScratchOrder() = default;
    int begin(int device, hipStream_t s) {
        lock_ = std::unique_lock<std::mutex>(g_scratch_mutex);
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return KVR_OK;
        if (g_scratch_used[device] && g_scratch_last[device] != s &&
            hipStreamWaitEvent(s, g_scratch_done[device], 0) != hipSuccess)
            return KVR_E_DEVICE;
        device_ = device;
        stream_ = s;
        return KVR_OK;
    }
    // after the launches (whatever their status): the array is in use until `stream_` gets here
    int end() {
        if (device_ < 0) return KVR_OK;
        if (hipEventRecord(g_scratch_done[device_], stream_) != hipSuccess) return KVR_E_DEVICE;
        g_scratch_last[device_] = stream_;
        g_scratch_used[device_] = true;
        return KVR_OK;
    }

  private:
    std::unique_lock<std::mutex> lock_;
    int device_ = -1;
    hipStream_t stream_ = nullptr;
};

}  // namespace
}  // namespace kvr

using namespace kvr;

extern "C" int64_t kvr_attention_schedule_ex(const int64_t* positions, int64_t n_sel, int64_t n_keys,
                                             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                                             int32_t chunk_keys, int32_t flags, int32_t* schedule, int64_t capacity) {
    if (flags & ~KVR_ATTN_ROUNDED_PROBABILITIES) return KVR_E_INVALID_ARGUMENT;
    const int32_t p_rounded = (flags & KVR_ATTN_ROUNDED_PROBABILITIES) ? 1 : 0;
    if (dtype_size(dtype) == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_keys < 0 || n_sel > n_keys) return KVR_E_INVALID_ARGUMENT;
    if (n_keys >= (int64_t(1) << 31) - kSub || n_sel >= (int64_t(1) << 31)) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || head_dim <= 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_sel > 0 && !positions) return KVR_E_NULL_POINTER;
    for (int64_t i = 0; i < n_sel; ++i) {
        if (positions[i] < 0 || positions[i] >= n_keys) return KVR_E_INVALID_ARGUMENT;
        if (i && positions[i] <= positions[i - 1]) return KVR_E_INVALID_ARGUMENT;
    }
    const bool mfma = mfma_eligible(dtype, head_dim);
    if (!mfma && generic_dmax(head_dim) == 0) return KVR_E_UNSUPPORTED_SHAPE;
    if (chunk_keys < 0) chunk_keys = 0;  // ABI v1: a negative size means "choose from the geometry"
    if (chunk_keys > 0 && chunk_keys % kSub != 0) return KVR_E_INVALID_ARGUMENT;
    const int group = n_q_heads / n_kv_heads;
    const int qt = pick_qt(group);
    const int n_head_groups = group / qt;
    const int64_t heads = static_cast<int64_t>(n_kv_heads) * n_head_groups;
    // Few rows (64-row groups x heads fill under half the grid): 16-row groups
    // for the split-key tile kernel, so a group needs 4x fewer key chunks for
    // the same grid and writes 4x less partial data; the chunk's K/V is then
    // read by up to 4 row groups, from the L2 of the head's XCD.
    const int64_t wide_units = (n_sel + kGroupRows - 1) / kGroupRows * heads;
    const int group_rows = (mfma && 2 * wide_units <= kTargetBlocks) ? kTileGroupRows : kGroupRows;
    const int64_t n_groups = (n_sel + group_rows - 1) / group_rows;
    if (n_groups == 0) {
        // No selected rows: a header-only schedule (no groups, no work).
        const int64_t need = kHeader;
        if (!schedule) return need;
        if (capacity < need) return KVR_E_CAPACITY;
        memset(schedule, 0, sizeof(int32_t) * kHeader);
        schedule[H_MAGIC] = kMagic;
        schedule[H_VERSION] = kVersion;
        schedule[H_QT] = qt;
        schedule[H_NHG] = n_head_groups;
        schedule[H_HQ] = n_q_heads;
        schedule[H_HKV] = n_kv_heads;
        schedule[H_D] = head_dim;
        schedule[H_KIND] = mfma ? KIND_MFMA : KIND_GENERIC;
        schedule[H_NKEYS] = static_cast<int32_t>(n_keys);
        schedule[H_DTYPE] = dtype;
        schedule[H_GROUP_ROWS] = group_rows;
        schedule[H_PROB] = p_rounded;
        return need;
    }

    std::vector<GroupKeys> keys(static_cast<size_t>(n_groups));
    for (int64_t g = 0; g < n_groups; ++g) keys[g] = group_keys(positions, n_sel, g, group_rows);

    std::vector<Chunk> chunks;
    if (chunk_keys > 0) {
        // Fixed chunk length (grown by 64 keys while a group would need more
        // chunks than the merge can weigh).
        int64_t kc = chunk_keys;
        for (;;) {
            int64_t worst = 0;
            for (int64_t g = 0; g < n_groups; ++g) {
                const int64_t c = (keys[g].kmax + kc - 1) / kc;
                worst = c > worst ? c : worst;
            }
            if (worst <= kMaxChunksPerGroup) break;
            kc += kSub;
        }
        for (int64_t g = 0; g < n_groups; ++g) {
            const int64_t c = (keys[g].kmax + kc - 1) / kc;
            for (int64_t i = 0; i < c; ++i) {
                const int64_t end = (i + 1) * kc < keys[g].kmax ? (i + 1) * kc : keys[g].kmax;
                chunks.push_back({static_cast<int32_t>(g), static_cast<int32_t>(i), static_cast<int32_t>(i * kc),
                                  static_cast<int32_t>(end)});
            }
        }
    } else {
        // Cost-balanced chunks: about kTargetBlocks blocks over the whole grid;
        // a group whose cost fits one block's share is not split (no merge).
        int64_t total = 0;
        std::vector<int64_t> group_cost(static_cast<size_t>(n_groups), 0);
        for (int64_t g = 0; g < n_groups; ++g) {
            const int64_t n_sub = (keys[g].kmax + kSub - 1) / kSub;
            for (int64_t s = 0; s < n_sub; ++s) group_cost[g] += subtile_cost(keys[g], s);
            total += group_cost[g];
        }
        const int64_t per_head = kTargetBlocks / heads > 1 ? kTargetBlocks / heads : 1;
        const int64_t max_cost = *std::max_element(group_cost.begin(), group_cost.end());
        // (The head-pair kernel also runs one block per CU in 64-row groups.)
        const bool one_block_per_cu = group_rows == kTileGroupRows || (mfma && qt == 4 && KVR_ATTN_PAIR);
        // The head-pair kernel walks a chunk in steps of two sub-tiles from its
        // first key: a boundary after an odd number of sub-tiles would leave a
        // half-empty step, so inner boundaries close on whole steps.
        const bool pair_steps = mfma && qt == 4 && KVR_ATTN_PAIR && kPairStepKeys == 2 * kSub;
        // Chunks for a share of `share` blocks per head.
        auto build = [&](int64_t share) {
            auto chunks_of = [&](int64_t g, int64_t cap) {
                const int64_t n_sub = (keys[g].kmax + kSub - 1) / kSub;
                int64_t nc = (group_cost[g] + cap - 1) / cap;
                nc = nc < 1 ? 1 : nc;
                nc = nc > n_sub ? n_sub : nc;
                return nc > kMaxChunksPerGroup ? int64_t(kMaxChunksPerGroup) : nc;
            };
            // Per-chunk cost cap: the even share of the total. The tile kernel
            // (one block per CU) raises it to the smallest cap whose rounded-up
            // chunk counts fit the share too (no extra, partial round of
            // blocks), or to the largest group cost (every group one chunk); the
            // count only falls as the cap grows, so a bisection finds it. The
            // wide kernel runs two blocks per CU.
            int64_t cap = (total + share - 1) / share;
            auto fits = [&](int64_t c) {
                int64_t sum = 0;
                for (int64_t g = 0; g < n_groups; ++g) sum += chunks_of(g, c);
                return sum <= share;
            };
            if (one_block_per_cu && cap < max_cost && !fits(cap)) {
                int64_t lo = cap, hi = max_cost;  // lo does not fit; hi fits or is the largest group cost
                while (hi - lo > 1) {
                    const int64_t mid = lo + (hi - lo) / 2;
                    (fits(mid) ? hi : lo) = mid;
                }
                cap = hi;
            }
            std::vector<Chunk> out;
            for (int64_t g = 0; g < n_groups; ++g) {
                const int64_t n_sub = (keys[g].kmax + kSub - 1) / kSub;
                const int64_t nc = chunks_of(g, cap);
                // Boundary i closes the chunk once the running cost reaches i/nc of
                // the group's cost (and the chunk is whole steps long, for the
                // head-pair kernel), leaving at least one sub-tile per later chunk.
                int64_t s = 0, acc = 0;
                for (int64_t i = 0; i < nc; ++i) {
                    const int64_t begin = s;
                    if (i == nc - 1) {
                        s = n_sub;
                    } else {
                        const int64_t goal = group_cost[g] * (i + 1) / nc;
                        do {
                            acc += subtile_cost(keys[g], s);
                            ++s;
                        } while ((acc < goal || (pair_steps && ((s - begin) & 1))) && n_sub - s > nc - 1 - i);
                    }
                    const int64_t end = s * kSub < keys[g].kmax ? s * kSub : keys[g].kmax;
                    out.push_back({static_cast<int32_t>(g), static_cast<int32_t>(i),
                                   static_cast<int32_t>(begin * kSub), static_cast<int32_t>(end)});
                }
            }
            return out;
        };
        chunks = build(per_head);
        if (group_rows == kGroupRows && one_block_per_cu) {
            // 64-row groups (MFMA-bound launches): one block per CU means one round
            // is balanced only as well as the chunk costs are. Two or four rounds
            // of smaller chunks let the dispatcher even the CUs out; keep the
            // share whose modelled span (below) is shortest.
            int64_t best = schedule_span(keys, chunks, per_head);
            for (int64_t rounds : {2, 4}) {
                std::vector<Chunk> more = build(per_head * rounds);
                const int64_t span = schedule_span(keys, more, per_head);
                if (span < best) {
                    best = span;
                    chunks = std::move(more);
                }
            }
        }
    }
    const int64_t n_work = static_cast<int64_t>(chunks.size());
    if (n_work > 65535) return KVR_E_UNSUPPORTED_SHAPE;  // grid.y limit
    int64_t n_multi = 0, max_chunks = 0, longest = 0;
    std::vector<int32_t> first(static_cast<size_t>(n_groups), 0), count(static_cast<size_t>(n_groups), 0);
    for (int64_t w = 0; w < n_work; ++w) {
        const Chunk& c = chunks[w];
        if (count[c.group]++ == 0) first[c.group] = static_cast<int32_t>(w);
        const int64_t len = c.end - c.begin;
        longest = len > longest ? len : longest;
    }
    for (int64_t g = 0; g < n_groups; ++g) {
        n_multi += count[g] > 1;
        max_chunks = count[g] > max_chunks ? count[g] : max_chunks;
    }
    const int64_t need = kHeader + 2 * n_groups + kWorkInts * n_work;
    if (!schedule) return need;
    if (capacity < need) return KVR_E_CAPACITY;
    int32_t* h = schedule;
    memset(h, 0, sizeof(int32_t) * kHeader);
    h[H_MAGIC] = kMagic;
    h[H_VERSION] = kVersion;
    h[H_NSEL] = static_cast<int32_t>(n_sel);
    h[H_NGROUPS] = static_cast<int32_t>(n_groups);
    h[H_KC] = static_cast<int32_t>(longest);
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
    h[H_MAXCHUNKS] = static_cast<int32_t>(max_chunks);
    h[H_GROUP_ROWS] = group_rows;
    h[H_PROB] = p_rounded;
    int32_t* groups = h + kHeader;
    int32_t* works = groups + 2 * n_groups;
    for (int64_t g = 0; g < n_groups; ++g) {
        groups[2 * g] = first[g];
        groups[2 * g + 1] = count[g];
    }
    for (int64_t w = 0; w < n_work; ++w) {
        works[kWorkInts * w + 0] = chunks[w].group;
        works[kWorkInts * w + 1] = chunks[w].index;
        works[kWorkInts * w + 2] = chunks[w].begin;
        works[kWorkInts * w + 3] = chunks[w].end;
    }
    return need;
}

extern "C" int64_t kvr_attention_schedule(const int64_t* positions, int64_t n_sel, int64_t n_keys, int32_t n_q_heads,
                                          int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t chunk_keys,
                                          int32_t* schedule, int64_t capacity) {
    return kvr_attention_schedule_ex(positions, n_sel, n_keys, n_q_heads, n_kv_heads, head_dim, dtype, chunk_keys, 0,
                                     schedule, capacity);
}

extern "C" int64_t kvr_attention_workspace_bytes(const int32_t* schedule, int64_t schedule_len, int32_t n_q_heads,
                                                 int32_t head_dim) {
    if (!schedule || schedule_len < kHeader || schedule[H_MAGIC] != kMagic || schedule[H_VERSION] != kVersion)
        return KVR_E_BAD_SCHEDULE;
    if (schedule[H_HQ] != n_q_heads || schedule[H_D] != head_dim) return KVR_E_BAD_SCHEDULE;
    if (schedule[H_GROUP_ROWS] != kGroupRows && schedule[H_GROUP_ROWS] != kTileGroupRows) return KVR_E_BAD_SCHEDULE;
    if (schedule[H_NMULTI] == 0) return 0;
    return static_cast<int64_t>(n_q_heads) * schedule[H_NWORK] * schedule[H_GROUP_ROWS] * (head_dim + 2) * 4;
}

namespace {

// Argument checks and launches of kvr_packed_causal_attention; `workspace` is
// the caller's buffer, or the library's static scratch array for the
// no-allocation entry point (`scratch_limit` > 0: a request needing more than
// that many bytes is refused before anything is launched).
int attention_call(const void* q, const void* k, const void* v, void* out, const int64_t* positions, int64_t n_sel,
                   int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, float scale,
                   const int64_t strides[12], const int32_t* schedule, int64_t schedule_len,
                   const int32_t* host_schedule, void* workspace, int64_t workspace_bytes, int64_t scratch_limit,
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
    if (schedule_len != kHeader + 2 * static_cast<int64_t>(hs[H_NGROUPS]) + kWorkInts * static_cast<int64_t>(hs[H_NWORK]))
        return KVR_E_BAD_SCHEDULE;
    if (hs[H_MAXCHUNKS] > kMaxChunksPerGroup || hs[H_NWORK] <= 0 || hs[H_NWORK] > 65535) return KVR_E_BAD_SCHEDULE;
    if (hs[H_PROB] != 0 && hs[H_PROB] != 1) return KVR_E_BAD_SCHEDULE;
    const int64_t ws_need = kvr_attention_workspace_bytes(hs, schedule_len, n_q_heads, head_dim);
    if (ws_need < 0) return KVR_E_BAD_SCHEDULE;
    int scratch_device = -1;
    if (scratch_limit > 0) {
        if (ws_need > scratch_limit) return KVR_E_SCRATCH_LIMIT;
        if (ws_need > 0) {
            workspace = scratch_address(stream, &scratch_device);
            if (!workspace) return KVR_E_DEVICE;
            workspace_bytes = scratch_limit;
        }
    }
    if (workspace_bytes < ws_need || (ws_need > 0 && !workspace)) return KVR_E_WORKSPACE_TOO_SMALL;
    // the partials are read and written as 16-byte vectors
    if (ws_need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15u)) return KVR_E_INVALID_ARGUMENT;

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
    a.group_rows = hs[H_GROUP_ROWS];
    a.p_rounded = hs[H_PROB];
    a.head_dim = head_dim;
    a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
    if (ws_need > 0) {
        a.ws_ml = static_cast<float*>(workspace);
        a.ws_o = a.ws_ml + static_cast<int64_t>(n_q_heads) * a.n_work * a.group_rows * 2;
    }
    if (a.qt <= 0 || a.qt * a.n_head_groups != a.group) return KVR_E_BAD_SCHEDULE;

    // The MFMA kernel reads 16-byte fragments of q/k/v (unit dim strides,
    // 16-byte aligned rows) and indexes rows of one 64-key sub-tile in 32 bits.
    // Other layouts (strided slices, odd offsets) take the generic kernel,
    // which accepts every schedule.
    bool use_mfma = hs[H_KIND] == KIND_MFMA;
    if (use_mfma && !mfma_eligible(dtype, head_dim)) return KVR_E_BAD_SCHEDULE;
    for (int t = 0; t < 3 && use_mfma; ++t) {
        const int64_t* st3 = strides + 3 * t;
        if (st3[2] != 1 || (st3[0] * esize) % 16 || (st3[1] * esize) % 16) use_mfma = false;
    }
    if (strides[4] * kSub >= (int64_t(1) << 30) || strides[7] * kSub >= (int64_t(1) << 30)) use_mfma = false;
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u)
        use_mfma = false;
    if (!(scale > 0.f)) use_mfma = false;  // the MFMA softmax takes row maxima of unscaled scores
    a.out_vec = strides[11] == 1 && strides[9] % 4 == 0 && strides[10] % 4 == 0 &&
                (reinterpret_cast<uintptr_t>(out) & 7u) == 0;

    hipStream_t s = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(n_kv_heads * a.n_head_groups), static_cast<unsigned>(a.n_work));
    const int dmax = use_mfma ? 0 : generic_dmax(head_dim);
    if (!use_mfma && dmax == 0) return KVR_E_UNSUPPORTED_SHAPE;
    ScratchOrder order;
    if (scratch_device >= 0) {
        const int ost = order.begin(scratch_device, s);
        if (ost != KVR_OK) return ost;
    }
    int st;
    if (use_mfma) {
        if (dtype == KVR_DTYPE_BF16)
            st = head_dim == 128 ? launch_mfma<bf16_t, 128>(a, a.qt, grid, s) : launch_mfma<bf16_t, 64>(a, a.qt, grid, s);
        else
            st = head_dim == 128 ? launch_mfma<f16_t, 128>(a, a.qt, grid, s) : launch_mfma<f16_t, 64>(a, a.qt, grid, s);
    } else {
        switch (dtype) {
            case KVR_DTYPE_F32: st = launch_generic<f32_t>(a, dmax, grid, s); break;
            case KVR_DTYPE_F16: st = launch_generic<f16_t>(a, dmax, grid, s); break;
            default: st = launch_generic<bf16_t>(a, dmax, grid, s); break;
        }
    }
    if (st == KVR_OK && hs[H_NMULTI] != 0) {
        switch (dtype) {
            case KVR_DTYPE_F32: st = launch_merge<f32_t>(a, hs[H_MAXCHUNKS], s); break;
            case KVR_DTYPE_F16: st = launch_merge<f16_t>(a, hs[H_MAXCHUNKS], s); break;
            default: st = launch_merge<bf16_t>(a, hs[H_MAXCHUNKS], s); break;
        }
    }
    const int ost = order.end();
    return st != KVR_OK ? st : ost;
}

}  // namespace

extern "C" int kvr_packed_causal_attention(const void* q, const void* k, const void* v, void* out,
                                           const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                                           int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, float scale,
                                           const int64_t strides[12], const int32_t* schedule, int64_t schedule_len,
                                           const int32_t* host_schedule, void* workspace, int64_t workspace_bytes,
                                           int32_t dtype, void* stream) {
    return attention_call(q, k, v, out, positions, n_sel, n_q_heads, n_kv_heads, n_keys, head_dim, scale, strides,
                          schedule, schedule_len, host_schedule, workspace, workspace_bytes, 0, dtype, stream);
}

extern "C" int64_t kvr_attention_scratch_limit(void) { return kScratchBytes; }

extern "C" int kvr_packed_causal_attention_noalloc(const void* q, const void* k, const void* v, void* out,
                                                   const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                                                   int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, float scale,
                                                   const int64_t strides[12], const int32_t* schedule,
                                                   int64_t schedule_len, const int32_t* host_schedule, int32_t dtype,
                                                   void* stream) {
    return attention_call(q, k, v, out, positions, n_sel, n_q_heads, n_kv_heads, n_keys, head_dim, scale, strides,
                          schedule, schedule_len, host_schedule, nullptr, 0, kScratchBytes, dtype, stream);
}
