// Frozen-embedding query relevance of every prompt token (the dense scorer
// that ranks suffix tokens for the refresh budget):
//   score[t] = max_j cos(E[ids[t]], E[q_j]) + boost * [ids[t] in {q_j}]
// with cos(a, b) = a.b / (max(|a|, eps) * max(|b|, eps)), eps = 1e-12, in fp32
// (F.normalize of each fp32 embedding row, then their dot product).
//
// Reference semantics: src/kv_cache_repair/scoring.py:11-72
// (dense_query_relevance_scores; chunks of 1024 tokens, embedding lookup,
// F.normalize, fp32 matmul against the normalised query rows, max, plus the
// 0.25 exact-id boost built by a host list comprehension). Here one launch
// covers every token.
//
// Block = 4 waves x 8 tokens. The query rows are staged in LDS in chunks (as
// stored, 16-byte vectors), with their squared norms; each wave walks its
// tokens: the lanes stream the token's row once per query chunk, accumulate
// its squared norm (first chunk) and the dot products with the chunk's rows,
// and a wave reduction gives the cosines. A token id or query id outside
// [0, vocab) yields a NaN score instead of an out-of-bounds read.
#include "kvr_internal.h"

#include <math.h>

namespace kvr {
namespace {

constexpr int kThreads = 256;
constexpr int kTokensPerWave = 8;
constexpr int kTokensPerBlock = kThreads / 64 * kTokensPerWave;
constexpr int kMaxChunkRows = 16;        // query rows per LDS chunk (dot accumulators per lane)
constexpr int kChunkBytes = 64 * 1024 - 256;  // LDS budget of one query chunk (+ norms: <= 64 KiB)
constexpr float kEps = 1e-12f;           // F.normalize's eps
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct ScoreArgs {
    const char* embed;
    int64_t vocab, ld_embed;
    int32_t hidden;
    const char* ids;
    int32_t ids32;
    int64_t n;
    const int64_t* query_ids;
    int32_t n_query;
    int32_t chunk_rows;  // query rows per LDS chunk
    float boost;
    float* scores;
};

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// U elements of the row per load: 16 bytes (VEC) or one element.
template <typename T, bool VEC>
struct Unit {
    using E = elem<T>;
    using bits = typename E::bits;
    static constexpr int U = VEC ? 16 / E::size : 1;
    __device__ static inline void load(const char* row, int u, float out[U]) {
        if constexpr (VEC) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(row + static_cast<int64_t>(u) * 16);
            bits b[U];
            __builtin_memcpy(b, &v, 16);
#pragma unroll
            for (int e = 0; e < U; ++e) out[e] = E::to_float(b[e]);
        } else {
            out[0] = E::to_float(reinterpret_cast<const bits*>(row)[u]);
        }
    }
};

template <typename T, bool VEC>
__global__ void __launch_bounds__(kThreads) query_relevance_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
    using L = Unit<T, VEC>;
    constexpr int U = L::U;
    constexpr int esize = elem<T>::size;
    extern __shared__ __align__(16) char smem[];
    const int row_bytes = a.hidden * esize;
    const int row_stride = (row_bytes + 15) / 16 * 16;  // LDS row stride (16-byte aligned)
    float* qn2 = reinterpret_cast<float*>(smem + a.chunk_rows * row_stride);  // [chunk_rows] squared norms
    int* qok = reinterpret_cast<int*>(qn2 + kMaxChunkRows);                   // [chunk_rows] id in range

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int units = a.hidden / U;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + wave * kTokensPerWave;

    int64_t id[kTokensPerWave];
    bool ok[kTokensPerWave];
#pragma unroll
    for (int i = 0; i < kTokensPerWave; ++i) {
        const int64_t t = t0 + i;
        id[i] = -1;
        if (t < a.n)
            id[i] = a.ids32 ? static_cast<int64_t>(reinterpret_cast<const int32_t*>(a.ids)[t])
                            : reinterpret_cast<const int64_t*>(a.ids)[t];
        ok[i] = id[i] >= 0 && id[i] < a.vocab;
    }
    float best[kTokensPerWave], tn2[kTokensPerWave];
    bool qbad = false;  // some query id out of range
#pragma unroll
    for (int i = 0; i < kTokensPerWave; ++i) {
        best[i] = -INFINITY;
        tn2[i] = 0.f;
    }

    for (int c0 = 0; c0 < a.n_query; c0 += a.chunk_rows) {
        const int qc = min(a.chunk_rows, a.n_query - c0);
        __syncthreads();  // the previous chunk is no longer read
        // stage the chunk's rows (16-byte pieces, or elements) and their squared norms
        for (int j = wave; j < qc; j += kThreads / 64) {
            const int64_t qid = a.query_ids[c0 + j];
            const bool in = qid >= 0 && qid < a.vocab;
            const char* src = a.embed + (in ? qid : 0) * a.ld_embed * esize;
            char* dst = smem + j * row_stride;
            float ss = 0.f;
            for (int u = lane; u < units; u += 64) {
                float x[U];
                L::load(src, u, x);
                if constexpr (VEC) {
                    *reinterpret_cast<u32x4*>(dst + u * 16) = *reinterpret_cast<const u32x4*>(src + u * 16);
                } else {
                    reinterpret_cast<typename elem<T>::bits*>(dst)[u] =
                        reinterpret_cast<const typename elem<T>::bits*>(src)[u];
                }
#pragma unroll
                for (int e = 0; e < U; ++e) ss += x[e] * x[e];
            }
            ss = wave_sum(ss);
            if (lane == 0) {
                qn2[j] = ss;
                qok[j] = in ? 1 : 0;
            }
        }
        __syncthreads();
        for (int j = 0; j < qc; ++j) qbad |= qok[j] == 0;
        const float* qn2c = qn2;
#pragma unroll
        for (int i = 0; i < kTokensPerWave; ++i) {
            if (t0 + i >= a.n) continue;  // wave-uniform
            const char* row = a.embed + (ok[i] ? id[i] : 0) * a.ld_embed * esize;
            float dot[kMaxChunkRows];
#pragma unroll
            for (int j = 0; j < kMaxChunkRows; ++j) dot[j] = 0.f;
            float ss = 0.f;
            for (int u = lane; u < units; u += 64) {
                float x[U];
                L::load(row, u, x);
                if (c0 == 0) {
#pragma unroll
                    for (int e = 0; e < U; ++e) ss += x[e] * x[e];
                }
#pragma unroll
                for (int j = 0; j < kMaxChunkRows; ++j) {
                    if (j < qc) {
                        float y[U];
                        L::load(smem + j * row_stride, u, y);
#pragma unroll
                        for (int e = 0; e < U; ++e) dot[j] += x[e] * y[e];
                    }
                }
            }
            if (c0 == 0) tn2[i] = wave_sum(ss);
            const float tden = fmaxf(sqrtf(tn2[i]), kEps);
#pragma unroll
            for (int j = 0; j < kMaxChunkRows; ++j) {
                if (j < qc) {
                    const float d = wave_sum(dot[j]);
                    best[i] = fmaxf(best[i], d / (tden * fmaxf(sqrtf(qn2c[j]), kEps)));
                }
            }
        }
    }
    if (lane != 0) return;
#pragma unroll
    for (int i = 0; i < kTokensPerWave; ++i) {
        const int64_t t = t0 + i;
        if (t >= a.n) continue;
        bool hit = false;
        for (int j = 0; j < a.n_query; ++j) hit |= a.query_ids[j] == id[i];
        a.scores[t] = (ok[i] && !qbad) ? best[i] + (hit ? a.boost : 0.f) : __builtin_nanf("");
    }
}

// MFMA path (bf16 / fp16 tables, rows of whole 32-element k-steps): the
// dot products are the [tokens x hidden] x [hidden x queries] product on
// v_mfma_f32_16x16x32 (A = 16 gathered token rows, B = 16 query rows, both
// straight from global memory: the query rows stay in L2), fp32 accumulation
// of exact 16-bit products. The squared norms are summed from the same
// fragments. A wave computes 16 tokens over SPLIT-th of the hidden axis: a
// block of max(4, SPLIT) waves covers 16 * waves / SPLIT tokens, and the
// SPLIT waves of one token group add their partial dot products and norms in
// LDS (wave order fixed). SPLIT grows as the prompt shrinks so that a launch
// keeps every CU busy (SPLIT 8: 480 blocks of 8 waves for a 7680-token
// prompt; SPLIT 1: 496 blocks of 4 waves for 31744 tokens). QT x 16 queries
// per pass (QT 1 for up to 16 queries, else 4; more queries take further
// passes over the token rows).
constexpr int kMfmaMinTokens = 16;  // tokens per block at SPLIT 8

template <typename T> struct score_mma;
template <> struct score_mma<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4_t mma(v8 a, v8 b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct score_mma<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4_t mma(v8 a, v8 b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <typename T>
__device__ inline float sumsq8(u32x4 v) {
    typename elem<T>::bits b[8];
    __builtin_memcpy(b, &v, 16);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = elem<T>::to_float(b[e]);
        s += x * x;
    }
    return s;
}

template <typename T, int SPLIT, int QT>
__global__ void __launch_bounds__(64 * (SPLIT > 4 ? SPLIT : 4)) query_relevance_mfma_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
    using M = score_mma<T>;
    using v8 = typename M::v8;
    static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4 || SPLIT == 8, "SPLIT divides the block's waves");
    constexpr int kMfmaWaves = SPLIT > 4 ? SPLIT : 4;
    constexpr int kQTiles = QT;
    constexpr int kParts = 5 * kQTiles + 1;  // per lane: kQTiles x 4 dots, kQTiles query norms, 1 token norm
    __shared__ float part[SPLIT > 1 ? kMfmaWaves : 1][kParts][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hpart = wave % SPLIT;  // this wave's part of the hidden axis
    const int lq = lane & 15;
    const int lj = lane >> 4;
    const int64_t tbase = static_cast<int64_t>(blockIdx.x) * (16 * kMfmaWaves / SPLIT) + (wave / SPLIT) * 16;
    // this lane's A row: token tbase + lq (clamped in bounds; its score is not written)
    const int64_t t = tbase + lq;
    int64_t id = -1;
    if (t < a.n)
        id = a.ids32 ? static_cast<int64_t>(reinterpret_cast<const int32_t*>(a.ids)[t])
                     : reinterpret_cast<const int64_t*>(a.ids)[t];
    const bool ok = id >= 0 && id < a.vocab;
    const char* arow = a.embed + (ok ? id : 0) * a.ld_embed * 2 + 16 * lj;
    // this wave's k-steps: [sbeg, send)
    const int steps = a.hidden / 32;
    const int per = (steps + SPLIT - 1) / SPLIT;
    const int sbeg = min(steps, hpart * per);
    const int send = min(steps, sbeg + per);

    float tn2 = 0.f;  // token lq's squared norm (hidden part 0, lanes (lq, *))
    float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // tokens 4 lj + i (hidden part 0)
    bool qbad = false;
    for (int q0 = 0; q0 < a.n_query; q0 += 16 * kQTiles) {
        const int tiles = min(kQTiles, (a.n_query - q0 + 15) / 16);
        const char* brow[kQTiles];
#pragma unroll
        for (int qt = 0; qt < kQTiles; ++qt) {
            const int j = q0 + 16 * qt + lq;  // this lane's B row: query j
            const int64_t qid = j < a.n_query ? a.query_ids[j] : -1;
            const bool qok = j < a.n_query && qid >= 0 && qid < a.vocab;
            qbad |= j < a.n_query && !qok;
            brow[qt] = a.embed + (qok ? qid : 0) * a.ld_embed * 2 + 16 * lj;
        }
        f32x4_t acc[kQTiles];
        float qn2[kQTiles];
#pragma unroll
        for (int qt = 0; qt < kQTiles; ++qt) {
            acc[qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            qn2[qt] = 0.f;
        }
        float tsum = 0.f;
        for (int s0 = sbeg; s0 < send; s0 += 8) {
            u32x4 av[8];
#pragma unroll
            for (int d = 0; d < 8; ++d)
                av[d] = *reinterpret_cast<const u32x4*>(arow + static_cast<int64_t>(min(s0 + d, send - 1)) * 64);
#pragma unroll
            for (int qt = 0; qt < kQTiles; ++qt) {
                if (qt >= tiles) break;
                u32x4 bv[8];
#pragma unroll
                for (int d = 0; d < 8; ++d)
                    bv[d] = *reinterpret_cast<const u32x4*>(brow[qt] + static_cast<int64_t>(min(s0 + d, send - 1)) * 64);
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    if (s0 + d < send) {
                        acc[qt] = M::mma(__builtin_bit_cast(v8, av[d]), __builtin_bit_cast(v8, bv[d]), acc[qt]);
                        qn2[qt] += sumsq8<T>(bv[d]);
                    }
                }
            }
            if (q0 == 0) {
#pragma unroll
                for (int d = 0; d < 8; ++d)
                    if (s0 + d < send) tsum += sumsq8<T>(av[d]);
            }
        }
        if constexpr (SPLIT > 1) {  // add the token group's partials (hidden parts in order)
#pragma unroll
            for (int qt = 0; qt < kQTiles; ++qt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) part[wave][4 * qt + i][lane] = acc[qt][i];
                part[wave][4 * kQTiles + qt][lane] = qn2[qt];
            }
            part[wave][kParts - 1][lane] = tsum;
            __syncthreads();
            if (hpart == 0) {
#pragma unroll
                for (int w = wave + 1; w < wave + SPLIT; ++w) {
#pragma unroll
                    for (int qt = 0; qt < kQTiles; ++qt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[qt][i] += part[w][4 * qt + i][lane];
                        qn2[qt] += part[w][4 * kQTiles + qt][lane];
                    }
                    tsum += part[w][kParts - 1][lane];
                }
            }
        }
        if (hpart == 0) {
            if (q0 == 0) {
                tn2 = tsum;
                tn2 += __shfl_xor(tn2, 16);
                tn2 += __shfl_xor(tn2, 32);  // lanes (lq, *): token lq's squared norm
            }
            float tden[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) tden[i] = fmaxf(sqrtf(__shfl(tn2, 4 * lj + i)), kEps);
#pragma unroll
            for (int qt = 0; qt < kQTiles; ++qt) {
                if (qt >= tiles) break;
                float n2 = qn2[qt];
                n2 += __shfl_xor(n2, 16);
                n2 += __shfl_xor(n2, 32);  // lanes (lq, *): query q0 + 16 qt + lq
                const float qden = fmaxf(sqrtf(n2), kEps);
                const bool live = q0 + 16 * qt + lq < a.n_query;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // D layout: lane (lq, lj) holds token 4 lj + i x query lq
                    float c = live ? acc[qt][i] / (tden[i] * qden) : -INFINITY;
#pragma unroll
                    for (int off = 8; off > 0; off >>= 1) c = fmaxf(c, __shfl_xor(c, off));  // max over the 16 queries
                    best[i] = fmaxf(best[i], c);
                }
            }
        }
        if constexpr (SPLIT > 1) __syncthreads();  // the next pass rewrites part
    }
    if (hpart != 0) return;
    qbad = __any(qbad);
    int64_t tids[4];  // ids of tokens 4 lj + i (held by lanes 4 lj + i), read while every lane is active
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int src = 4 * lj + i;
        const uint32_t lo = __shfl(static_cast<uint32_t>(static_cast<uint64_t>(id)), src);
        const uint32_t hi = __shfl(static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32), src);
        tids[i] = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    }
    if (lq != 0) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 4 * lj + i;
        const int64_t tt = tbase + tok;
        if (tt >= a.n) continue;
        const int64_t tid = tids[i];
        const bool tok_ok = tid >= 0 && tid < a.vocab;
        bool hit = false;
        for (int j = 0; j < a.n_query; ++j) hit |= a.query_ids[j] == tid;
        a.scores[tt] = (tok_ok && !qbad) ? best[i] + (hit ? a.boost : 0.f) : __builtin_nanf("");
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// SPLIT: the smallest of 1, 2, 4, 8 whose grid still covers the CUs about
// twice (>= 480 blocks of 64 / SPLIT tokens; 8-wave blocks of 16 tokens below).
template <typename T, int QT>
int launch_mfma_split(const ScoreArgs& a, hipStream_t s) {
    const int64_t blocks1 = (a.n + 63) / 64;
    const unsigned b16 = static_cast<unsigned>((a.n + 15) / 16);
    if (blocks1 >= 480) {
        query_relevance_mfma_kernel<T, 1, QT><<<static_cast<unsigned>(blocks1), 256, 0, s>>>(a);
    } else if (blocks1 >= 240) {
        query_relevance_mfma_kernel<T, 2, QT><<<static_cast<unsigned>((a.n + 31) / 32), 256, 0, s>>>(a);
    } else if (blocks1 >= 160) {
        query_relevance_mfma_kernel<T, 4, QT><<<b16, 256, 0, s>>>(a);
    } else {
        query_relevance_mfma_kernel<T, 8, QT><<<b16, 512, 0, s>>>(a);
    }
    return launch_status();
}

template <typename T>
int launch_scores(const ScoreArgs& a, size_t lds, hipStream_t s) {
    const int esize = elem<T>::size;
    if constexpr (!__is_same(T, f32_t)) {
        if (a.hidden % 32 == 0 && (a.ld_embed * esize) % 16 == 0 && aligned16(a.embed)) {
            if (a.n_query <= 16) return launch_mfma_split<T, 1>(a, s);
            return launch_mfma_split<T, 4>(a, s);
        }
    }
    const unsigned grid = static_cast<unsigned>((a.n + kTokensPerBlock - 1) / kTokensPerBlock);
    const bool vec = (static_cast<int64_t>(a.hidden) * esize) % 16 == 0 && (a.ld_embed * esize) % 16 == 0 &&
                     aligned16(a.embed);
    if (vec) query_relevance_kernel<T, true><<<grid, kThreads, lds, s>>>(a);
    else query_relevance_kernel<T, false><<<grid, kThreads, lds, s>>>(a);
    return launch_status();
}

}  // namespace
}  // namespace kvr

extern "C" int kvr_query_relevance(const void* embed, int64_t vocab, int64_t ld_embed, int32_t hidden,
                                   const void* ids, int32_t ids_are_int32, int64_t n, const int64_t* query_ids,
                                   int32_t n_query, float boost, float* scores, int32_t dtype, void* stream) {
    using namespace kvr;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (vocab <= 0 || hidden <= 0 || n < 0 || n_query <= 0 || !(boost == boost)) return KVR_E_INVALID_ARGUMENT;
    if (ld_embed < hidden) return KVR_E_BAD_STRIDE;
    const int64_t row_stride = (static_cast<int64_t>(hidden) * esize + 15) / 16 * 16;
    if (row_stride > kChunkBytes) return KVR_E_UNSUPPORTED_SHAPE;  // one query row must fit a chunk
    if (n == 0) return KVR_OK;
    if (n > int64_t(kMfmaMinTokens) * 0x7fffffff) return KVR_E_UNSUPPORTED_SHAPE;  // grid.x of every path
    if (!embed || !ids || !query_ids || !scores) return KVR_E_NULL_POINTER;
    ScoreArgs a;
    a.embed = static_cast<const char*>(embed);
    a.vocab = vocab;
    a.ld_embed = ld_embed;
    a.hidden = hidden;
    a.ids = static_cast<const char*>(ids);
    a.ids32 = ids_are_int32 ? 1 : 0;
    a.n = n;
    a.query_ids = query_ids;
    a.n_query = n_query;
    const int64_t fit = kChunkBytes / row_stride;
    a.chunk_rows = static_cast<int32_t>(fit < kMaxChunkRows ? fit : kMaxChunkRows);
    a.boost = boost;
    a.scores = scores;
    const size_t lds = static_cast<size_t>(a.chunk_rows) * row_stride + kMaxChunkRows * (sizeof(float) + sizeof(int));
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KVR_DTYPE_F32: return launch_scores<f32_t>(a, lds, s);
        case KVR_DTYPE_F16: return launch_scores<f16_t>(a, lds, s);
        default: return launch_scores<bf16_t>(a, lds, s);
    }
}
