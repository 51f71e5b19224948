// Skinny projection GEMMs of the packed refresh rows (gfx950 MFMA):
//   y[m, r] = sum_k x[m, k] * w[r, k]        m < M <= 64, bf16 / fp16, fp32 accumulation
// i.e. torch.nn.functional.linear(x, w) without bias, the q/k/v/o and MLP
// projections of every decoder layer (transformers 5.15.0
// models/llama/modeling_llama.py:165-175, 243-252). With only the selected
// rows (M = 64 at a 64-token budget) the projections stream the layer's
// weights once and do little arithmetic per byte, so the kernel is built to
// stream W from HBM: every weight byte is read once, straight into MFMA
// registers with a deep prefetch, while the block's rows of x sit in LDS.
//
// One launch can stream up to three weights (their rows concatenated, e.g.
// q/k/v into one [M, nq + nk + nv] output), or a gate/up pair whose epilogue
// applies the SiLU-gated product (the MLP's act_fn(gate) * up) so the two
// projections never reach HBM.
//
// Work split: block = NW waves x 16 streamed weight rows x one K slice, NW = 4,
// or 6 / 7 where that makes the grid exactly one block per CU (q/k/v and the
// gate/up pairs of 8B-shaped models). The slice is walked in chunks of 256 (128
// in launches with more blocks than CUs): x[:, chunk] is staged in one of
// two LDS buffers (the next chunk's global loads are in flight while the
// current one is multiplied) and shared by the waves; the weights stream into
// registers through a ring of 8 loads per lane (one chunk ahead), each load
// instruction covering whole 128-B lines of 8 rows (one memory request per
// line: 16-row x 64-B loads in the MFMA layout reach ~25% less bandwidth),
// and every pair of loads is transposed to MFMA A fragments through a small
// per-wave LDS tile. Split-K slices (S > 1) write fp32 partials to a workspace
// of 64-column tiles and a second launch (or a fused consumer) sums them in
// slice order, so results are deterministic.
#include "kvr_internal.h"

#include <string.h>

namespace kvr {
namespace {

#ifndef KVR_GEMM_CHUNK_STEPS
#define KVR_GEMM_CHUNK_STEPS 8
#endif
#ifndef KVR_GEMM_RING_CHUNKS
#define KVR_GEMM_RING_CHUNKS 1
#endif

// Waves per block (16 streamed weight rows each) is a launch parameter: 4, 6 or
// 7, whichever makes the grid exactly one block per CU (plan_split).
template <int NW>
struct WaveCfg {
    static constexpr int kThreads = 64 * NW;
    static constexpr int kTileN = 16 * NW;      // streamed weight rows per block
    static constexpr int kHalf = kTileN / 2;   // gated: output columns per block (8 per wave)
    static constexpr int kRedStride = kTileN + 4;  // fp32 LDS tile of the gated epilogue
};
constexpr int kRowsMax = 64;                // M <= 64 (four 16-row MFMA tiles)
constexpr int kStep = 32;                   // K per MFMA
constexpr int kSliceChunk = KVR_GEMM_CHUNK_STEPS * kStep;  // split-K slices are whole multiples of this
constexpr int kRingChunks = KVR_GEMM_RING_CHUNKS;  // W ring depth in chunks
static_assert(kRingChunks == 1 || kRingChunks == 2, "chunk buffers alternate with the ring");

// Staged x chunk of CS k-steps (CS = the W ring depth per chunk): 8 for
// launches of at most one block per CU, 4 (half the LDS, chunks turned over
// twice as often) where some CUs run two blocks.
template <int CS, int NW>
struct ChunkCfg {
    static constexpr int kChunkSteps = CS;            // k-steps per staged x chunk = W ring depth
    static constexpr int kChunk = CS * kStep;         // K per chunk
    static constexpr int kXStride = kChunk + 8;       // LDS row stride (elements): 16 B pad, conflict-free B reads
    static constexpr int kXBuf = kRowsMax * kXStride; // one chunk buffer (elements)
    static constexpr int kRing = kRingChunks * CS;    // W fragments in flight per lane (k-steps)
    static constexpr int kGranules = kChunk / 8;      // 16-B x granules per row per chunk
    static constexpr int kXGranules = kRowsMax * kGranules;  // x granules per chunk
    static constexpr int kXLoads = (kXGranules + 64 * NW - 1) / (64 * NW);  // x granules per thread per chunk (at most)
    // two x chunk buffers + the per-wave W transpose tiles (the gated epilogue's fp32 tile reuses them)
    static constexpr size_t kLdsBytes = 2 * static_cast<size_t>(kXBuf) * 2 + NW * 2048;
    static_assert(kRing % 2 == 0 && CS % 2 == 0, "whole-line loads come in pairs");
    static_assert(kSliceChunk % kChunk == 0, "slices are whole chunks");
    static_assert(kLdsBytes >= static_cast<size_t>(kRowsMax) * WaveCfg<NW>::kRedStride * 4, "gated epilogue tile fits");
};
constexpr int kMinSlice = 512;              // K per split at least (bounds the partial traffic)
#ifndef KVR_GEMM_TARGET_BLOCKS
#define KVR_GEMM_TARGET_BLOCKS 256
#endif
constexpr int kTargetBlocks = KVR_GEMM_TARGET_BLOCKS;  // split until the grid covers every CU once
// Split-K partials: fp32 tiles of 64 output columns, [ceil(cols / 64)][S][64 rows][64 cols]
// (the layout kPartialTileCols/kPartialTileRows name for fused consumers), whatever
// the block width; columns are the concatenated rows (gated: gate features, then up).
constexpr int kTile = kPartialTileRows * kPartialTileCols;  // fp32 elements of one partial tile
static_assert(kPartialTileRows == kRowsMax && kPartialTileCols == 64, "partial tile geometry");

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct gemm_t;
template <> struct gemm_t<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct gemm_t<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ static inline f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

struct GemmArgs {
    const char* x;                  // [M][ldx]
    const char* w0;                 // weights: [rows_i][ldw_i]
    const char* w1;
    const char* w2;
    char* y;                        // [M][ldy]
    const char* res;                // residual [M][ldr] added to y (or null)
    float* partial;                 // [ceil(rows / 64)][S][64][64] fp32 (S > 1)
    int64_t ldx, ldy, ldr, ldw0, ldw1, ldw2;
    int32_t end0, end1;             // concatenated row boundaries of w0 | w1 | w2
    int32_t rows;                   // streamed rows in total
    int32_t n_out;                  // output columns (gated: rows / 2)
    int32_t gated;                  // 1: y = silu(x w0^T) * (x w1^T)
    int32_t m, k;
    int32_t slice;                  // K per split (multiple of kStep)
    int32_t splits;                 // S
    int32_t waves;                  // waves per block (4, 6 or 7): 16 streamed rows each
};

// Output value of a concatenated projection: the fp32 sum, or with a residual
// dtype(dtype(sum) + residual) -- `residual + proj(x)` as the eager ops round it.
template <typename T>
__device__ inline float with_residual(const GemmArgs& a, float sum, int m, int col) {
    if (!a.res) return sum;
    const uint16_t r = reinterpret_cast<const uint16_t*>(a.res)[static_cast<int64_t>(m) * a.ldr + col];
    return round_through<T>(sum) + elem<T>::to_float(r);
}

// MFMA roles: A = W (16 streamed rows x 32 k; lane holds w[row lq][k + 8lj ..]),
// B = x^T (32 k x 16 rows of x; lane holds x[m0 + lq][k + 8lj ..]) from LDS;
// D: lane holds the products of x row m0 + lq with streamed rows 4lj + i, i < 4.
//
// Streamed row layout of a block (tile) of NW waves: the rows of wave w are
// tile*kTileN + 16w + 0..15 (concatenated weights); gated: wave w streams gate
// features tile*kHalf + 8w + 0..7 as its rows 0..7 and the same features of up
// as rows 8..15, so lane columns 4lj + i hold gate (lj < 2) or up (lj >= 2) of
// feature 8w + 4(lj & 1) + i, and the SiLU pair meets in one wave.
template <typename T, int MT, int CS, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))  // two blocks per CU
skinny_gemm_kernel(GemmArgs a) {
    using G = gemm_t<T>;
    using E = elem<T>;
    using v8 = typename G::v8;
    using K = ChunkCfg<CS, NW>;
    using WC = WaveCfg<NW>;
    constexpr int kThreads = WC::kThreads;
    constexpr int kTileN = WC::kTileN;
    constexpr int kHalf = WC::kHalf;
    constexpr int kRedStride = WC::kRedStride;
    constexpr int kChunkSteps = K::kChunkSteps;
    constexpr int kChunk = K::kChunk;
    constexpr int kXStride = K::kXStride;
    constexpr int kXBuf = K::kXBuf;
    constexpr int kRing = K::kRing;
    constexpr int kGranules = K::kGranules;
    constexpr int kXLoads = K::kXLoads;
    extern __shared__ __align__(16) char smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);  // two chunk buffers [64][kXStride]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 15;
    const int lj = lane >> 4;
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int k0 = split * a.slice;
    const int klen = (a.k - k0 < a.slice) ? a.k - k0 : a.slice;  // > 0, multiple of 8

    // ---- this lane's streamed weight rows ----
    // Pointer to k0 of row `rw` (0..15) of the wave's 16 streamed rows; rows
    // past the end read row 0 (their outputs are never written).
    auto row_ptr = [&](int rw) __attribute__((always_inline)) -> const char* {
        const char* wb;
        int64_t ldw;
        int local;
        bool row_ok;
        if (a.gated) {
            const bool up = rw >= 8;
            local = tile * kHalf + 8 * wave + (rw & 7);
            row_ok = local < a.n_out;
            wb = up ? a.w1 : a.w0;
            ldw = up ? a.ldw1 : a.ldw0;
        } else {
            const int g = tile * kTileN + 16 * wave + rw;
            row_ok = g < a.rows;
            if (g < a.end0) {
                wb = a.w0; ldw = a.ldw0; local = g;
            } else if (g < a.end1) {
                wb = a.w1; ldw = a.ldw1; local = g - a.end0;
            } else {
                wb = a.w2; ldw = a.ldw2; local = g - a.end1;
            }
        }
        if (!row_ok) local = 0;
        return wb + (static_cast<int64_t>(local) * ldw + k0) * 2;
    };

    // ---- W ring: the load of k-step s lives in wf[s % kRing] ----
    // Loads are unconditional, so the wait before each use covers only the
    // load it consumes; k offsets past the slice are clamped to its last 8
    // elements (in bounds; they meet the zeroed tail of the staged x, so they
    // contribute 0 * w = 0 for finite w).
    //
    // Whole-line loads: one instruction covers 8 rows x 128 B (lane L reads
    // piece L & 7 of row 8h + (L >> 3), h = s & 1, k block s >> 1), every
    // 128-B line in a single request. Each pair of loads (16 rows x 64 k) is
    // transposed to the two MFMA A fragments of k-steps 2u, 2u + 1 through a
    // 2 KB per-wave LDS tile (pieces XOR-swizzled by row: conflict-free).
    const int klast = klen - 8;
    u32x4 wf[kRing];
    const char* wrow[2] = {row_ptr(lane >> 3), row_ptr(8 + (lane >> 3))};
    auto load_w = [&](int s, int h) __attribute__((always_inline)) -> u32x4 {
        const int kk = min((s >> 1) * 64 + 8 * (lane & 7), klast);
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + kk * 2));
    };
    char* wtile = reinterpret_cast<char*>(xs + 2 * kXBuf) + wave * 2048;
    char* const wput = wtile + (lane >> 3) * 128 + (((lane & 7) ^ (lane >> 3)) * 16);
    const char* const wget0 = wtile + (lq >> 3) * 1024 + (lq & 7) * 128 + (((0 + lj) ^ (lq & 7)) * 16);
    const char* const wget1 = wtile + (lq >> 3) * 1024 + (lq & 7) * 128 + (((4 + lj) ^ (lq & 7)) * 16);

    // ---- x chunks: thread t stages granules g = t + threads * i (row g / G, k 8 (g % G)) ----
    const char* xbase = a.x + k0 * 2;
    u32x4 xr[kXLoads];
    auto load_x = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int g0 = tid + kThreads * i;
            const int g = g0 < K::kXGranules ? g0 : 0;  // the last round's spare threads re-read granule 0
            const int r = g / kGranules;
            const int kk = min(c * kChunk + 8 * (g % kGranules), klast);
            xr[i] = *reinterpret_cast<const u32x4*>(xbase + (static_cast<int64_t>(r < a.m ? r : 0) * a.ldx + kk) * 2);
        }
    };
    auto store_x = [&](int c, uint16_t* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int g = tid + kThreads * i;
            if (K::kXGranules % kThreads != 0 && g >= K::kXGranules) continue;
            const int r = g / kGranules;
            const int xcol = 8 * (g % kGranules);
            const bool k_ok = c * kChunk + xcol < klen;  // klen is a multiple of 8
            const u32x4 zero = {0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(buf + r * kXStride + xcol) = (k_ok && r < a.m) ? xr[i] : zero;
        }
    };

    const int chunks = (klen + kChunk - 1) / kChunk;
    load_x(0);
#pragma unroll
    for (int d = 0; d < kRing; ++d) wf[d] = load_w(d, d & 1);
    store_x(0, xs);
    __syncthreads();

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Chunk c: issue chunk c + 1's x loads, multiply chunk c pair by pair
    // (copy the pair's two loads into the transpose tile, refill their slots
    // with the loads kRing steps ahead, read back the two A fragments, run the
    // MFMAs), then store chunk c + 1 into the other buffer. The loop advances kRingChunks chunks at a time so every ring slot
    // index is static; a chunk past the last one multiplies an all-zero x
    // buffer (store_x zeroes k >= klen) and adds nothing. Past the slice the
    // loads repeat in-bounds addresses into the idle buffer or unread slots.
    // sched_barrier pins the loads where they are written: left alone, the
    // scheduler sinks them to the end of the chunk and exposes their latency.
    for (int c = 0; c < chunks; c += kRingChunks) {
#pragma unroll
        for (int r = 0; r < kRingChunks; ++r) {
            const int cc = c + r;
            const uint16_t* cur = xs + (cc & 1) * kXBuf;
            load_x(cc + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int d = 0; d < kChunkSteps; d += 2) {
                const int slot = (r * kChunkSteps + d) % kRing;
                *reinterpret_cast<u32x4*>(wput) = wf[slot];
                *reinterpret_cast<u32x4*>(wput + 1024) = wf[slot + 1];
                wf[slot] = load_w(cc * kChunkSteps + d + kRing, 0);
                wf[slot + 1] = load_w(cc * kChunkSteps + d + 1 + kRing, 1);
                const v8 af0 = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(wget0));
                const v8 af1 = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(wget1));
                u32x4 bf0[MT], bf1[MT];
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    bf0[t] = *reinterpret_cast<const u32x4*>(cur + (16 * t + lq) * kXStride + d * kStep + 8 * lj);
                    bf1[t] = *reinterpret_cast<const u32x4*>(cur + (16 * t + lq) * kXStride + (d + 1) * kStep + 8 * lj);
                }
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[t] = G::mma(af0, __builtin_bit_cast(v8, bf0[t]), acc[t]);
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[t] = G::mma(af1, __builtin_bit_cast(v8, bf1[t]), acc[t]);
                __builtin_amdgcn_sched_barrier(0);
            }
            store_x(cc + 1, xs + ((cc + 1) & 1) * kXBuf);
            __syncthreads();
        }
    }

    uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
    // ---- single split: write y from registers (gated: through an LDS tile) ----
    if (a.splits == 1) {
        if (!a.gated) {
            const int c0 = tile * kTileN + 16 * wave + 4 * lj;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int m = 16 * t + lq;
                if (m >= a.m) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (c0 + i < a.rows)
                        y[static_cast<int64_t>(m) * a.ldy + c0 + i] = E::from_float(with_residual<T>(a, acc[t][i], m, c0 + i));
            }
            return;
        }
        float* red = reinterpret_cast<float*>(smem);  // [64 rows][gate kHalf | up kHalf]
        const int gcol = (lj < 2 ? 0 : kHalf) + 8 * wave + 4 * (lj & 1);
#pragma unroll
        for (int t = 0; t < MT; ++t)
            *reinterpret_cast<f32x4*>(red + (16 * t + lq) * kRedStride + gcol) = acc[t];
        __syncthreads();
        for (int e = tid; e < 16 * MT * kHalf; e += kThreads) {
            const int m = e / kHalf;
            const int c = e % kHalf;
            const int col = tile * kHalf + c;
            if (m < a.m && col < a.n_out) {
                const float g = round_through<T>(red[m * kRedStride + c]);
                const float u = round_through<T>(red[m * kRedStride + kHalf + c]);
                y[static_cast<int64_t>(m) * a.ldy + col] = E::from_float(silu_gate<T>(g, u));
            }
        }
        return;
    }

    // ---- split K: this split's fp32 values in the 64-column partial tiles ----
    auto part_at = [&](int col, int m) -> float* {
        return a.partial + (static_cast<int64_t>(col / kPartialTileCols) * a.splits + split) * kTile +
               m * kPartialTileCols + col % kPartialTileCols;
    };
    if (!a.gated) {
        // 4 columns from a multiple of 4: one 64-column tile; columns past `rows`
        // stay inside the last tile and are never read
        const int col = tile * kTileN + 16 * wave + 4 * lj;
        if (col < a.rows) {
#pragma unroll
            for (int t = 0; t < MT; ++t) *reinterpret_cast<f32x4*>(part_at(col, 16 * t + lq)) = acc[t];
        }
    } else {
        // gate feature f at column f, up feature f at column n_out + f
        const int f0 = tile * kHalf + 8 * wave + 4 * (lj & 1);
        const int base = lj < 2 ? 0 : a.n_out;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (f0 + i < a.n_out) *part_at(base + f0 + i, 16 * t + lq) = acc[t][i];
    }
}

// Split-K reduction (a second launch, so every partial is visible): block
// (64-column tile, 16-row group) sums the S partials of its rows in slice
// order and writes y; non-gated four columns per thread with four slices'
// loads in flight at a time, gated one feature per thread (the SiLU-gated
// product of its gate sum, column f, and up sum, column n_out + f).
constexpr int kReduceThreads = 256;

template <typename T>
__global__ void __launch_bounds__(kReduceThreads) splitk_reduce_kernel(GemmArgs a) {
    using E = elem<T>;
    constexpr int kCols = kPartialTileCols;
    const int tile = blockIdx.x;
    const int group = blockIdx.y;
    uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
    if (!a.gated) {
        const f32x4* base = reinterpret_cast<const f32x4*>(a.partial) + static_cast<int64_t>(tile) * a.splits * (kTile / 4);
        auto sum_splits = [&](int e4) __attribute__((always_inline)) -> f32x4 {
            f32x4 sum = base[e4];
            int sp = 1;
            for (; sp + 4 <= a.splits; sp += 4) {
                const f32x4 p0 = base[(sp + 0) * (kTile / 4) + e4];
                const f32x4 p1 = base[(sp + 1) * (kTile / 4) + e4];
                const f32x4 p2 = base[(sp + 2) * (kTile / 4) + e4];
                const f32x4 p3 = base[(sp + 3) * (kTile / 4) + e4];
                sum += p0;
                sum += p1;
                sum += p2;
                sum += p3;
            }
            for (; sp < a.splits; ++sp) sum += base[sp * (kTile / 4) + e4];
            return sum;
        };
        for (int e = threadIdx.x; e < 16 * kCols / 4; e += kReduceThreads) {
            const int m = 16 * group + e / (kCols / 4);
            const int c = 4 * (e % (kCols / 4));
            if (m >= a.m) continue;
            const f32x4 sum = sum_splits(m * (kCols / 4) + c / 4);
            const int col = tile * kCols + c;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (col + i < a.rows)
                    y[static_cast<int64_t>(m) * a.ldy + col + i] = E::from_float(with_residual<T>(a, sum[i], m, col + i));
        }
    } else {
        auto sum_col = [&](int col, int m) __attribute__((always_inline)) -> float {
            const float* at = a.partial + static_cast<int64_t>(col / kCols) * a.splits * kTile + m * kCols + col % kCols;
            float sum = at[0];
            for (int sp = 1; sp < a.splits; ++sp) sum += at[static_cast<int64_t>(sp) * kTile];
            return sum;
        };
        for (int e = threadIdx.x; e < 16 * kCols; e += kReduceThreads) {
            const int m = 16 * group + e / kCols;
            const int f = tile * kCols + e % kCols;
            if (m >= a.m || f >= a.n_out) continue;
            const float g = sum_col(f, m);
            const float u = sum_col(a.n_out + f, m);
            y[static_cast<int64_t>(m) * a.ldy + f] = E::from_float(silu_gate<T>(round_through<T>(g), round_through<T>(u)));
        }
    }
}

template <typename F>
bool allow_lds(F fn, size_t bytes) {
    if (bytes <= 65536) return true;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes)) == hipSuccess;
}

template <typename T, int MT, int CS, int NW>
int launch_cs(const GemmArgs& a, dim3 grid, hipStream_t s) {
    constexpr size_t lds = ChunkCfg<CS, NW>::kLdsBytes;
    static const bool ok = allow_lds(skinny_gemm_kernel<T, MT, CS, NW>, lds);
    if (!ok) return KVR_E_LAUNCH_FAILED;
    skinny_gemm_kernel<T, MT, CS, NW><<<grid, 64 * NW, lds, s>>>(a);
    return KVR_OK;
}

template <typename T, int MT>
int launch_mt(const GemmArgs& a, hipStream_t s, bool reduce) {
    const dim3 grid(static_cast<unsigned>(ceil_div(a.rows, 16 * a.waves)), static_cast<unsigned>(a.splits));
    int st;
    if (a.waves == 6) {
        st = launch_cs<T, MT, 8, 6>(a, grid, s);
    } else if (a.waves == 7) {
        st = launch_cs<T, MT, 8, 7>(a, grid, s);
    } else {
        // more blocks than CUs (some CUs run two): 4-step chunks; else 8
        st = static_cast<int64_t>(grid.x) * grid.y > kTargetBlocks ? launch_cs<T, MT, 4, 4>(a, grid, s)
                                                                  : launch_cs<T, MT, 8, 4>(a, grid, s);
    }
    if (st != KVR_OK) return st;
    if (a.splits > 1 && reduce) {
        const int64_t cols = a.gated ? a.n_out : a.rows;
        const dim3 rgrid(static_cast<unsigned>(ceil_div(cols, kPartialTileCols)), static_cast<unsigned>(MT));
        splitk_reduce_kernel<T><<<rgrid, kReduceThreads, 0, s>>>(a);
    }
    return launch_status();
}

template <typename T>
int launch(const GemmArgs& a, hipStream_t s, bool reduce) {
    switch ((a.m + 15) / 16) {
        case 1: return launch_mt<T, 1>(a, s, reduce);
        case 2: return launch_mt<T, 2>(a, s, reduce);
        case 3: return launch_mt<T, 3>(a, s, reduce);
        default: return launch_mt<T, 4>(a, s, reduce);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kvr

using namespace kvr;

// K split of a launch of `waves`-wave blocks: the smallest power of two
// giving >= kTargetBlocks blocks, at most k / kMinSlice; slices are whole
// 256-chunks, so the split count is then ceil(k / slice). Blocks have 4 waves
// unless 6 or 7 make the grid exactly one block per CU where 4 do not (q/k/v
// of 8B-shaped models: 6144 rows, 64 x 4 blocks of 6 waves instead of 96 x 4;
// their gate/up pairs: 256 blocks of 7 or 6 waves instead of 448 or 384 of 4):
// a CU running two blocks while others run one makes the launch last as long
// as its slowest CU.
namespace {
struct Split {
    int32_t splits;
    int32_t slice;
    int32_t waves;
};

Split split_for(int32_t rows, int32_t k, int32_t waves) {
    const int64_t tiles = ceil_div(rows, 16 * waves);
    int32_t want = 1;
    while (tiles * want < kTargetBlocks && want < 64) want *= 2;
    const int32_t cap = k / kMinSlice > 1 ? k / kMinSlice : 1;
    const int32_t s = want < cap ? want : cap;
    const int32_t slice = static_cast<int32_t>(ceil_div(ceil_div(k, s), kSliceChunk) * kSliceChunk);
    return Split{static_cast<int32_t>(ceil_div(k, slice)), slice, waves};
}

Split plan_split(int32_t rows, int32_t k) {
    const Split four = split_for(rows, k, 4);
    if (ceil_div(rows, 64) * four.splits == kTargetBlocks) return four;
    for (int32_t waves : {6, 7}) {
        const Split sp = split_for(rows, k, waves);
        if (ceil_div(rows, 16 * waves) * sp.splits == kTargetBlocks) return sp;
    }
    return four;
}
}  // namespace

extern "C" int32_t kvr_linear_splits(int32_t m, int32_t rows, int32_t k) {
    if (m <= 0 || m > kRowsMax || rows <= 0 || k <= 0 || k % 8) return KVR_E_UNSUPPORTED_SHAPE;
    return plan_split(rows, k).splits;
}

extern "C" int64_t kvr_linear_workspace_bytes(int32_t m, int32_t rows, int32_t k) {
    const int32_t splits = kvr_linear_splits(m, rows, k);
    if (splits < 0) return splits;
    if (splits == 1) return 0;
    return ceil_div(rows, kPartialTileCols) * splits * static_cast<int64_t>(kTile) * 4;
}

namespace kvr {

// kvr_linear_multi with an option to stop before the split-K reduction: with
// reduce == false and more than one split, y is left unwritten and the fp32
// partials [ceil(rows / 64)][splits][64][64] stay in `workspace` for a fused
// consumer (*splits_out = splits; 1 means y was written directly).
int linear_multi(const void* x, int32_t n_weights, const void* const* w, const int32_t* rows, const int64_t* ldw,
                 void* y, int32_t m, int32_t k, int64_t ldx, int64_t ldy, int32_t epilogue, const void* residual,
                 int64_t ldr, void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream, bool reduce,
                 int32_t* splits_out) {
    if (dtype != KVR_DTYPE_BF16 && dtype != KVR_DTYPE_F16) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_weights < 1 || n_weights > 3 || !w || !rows || !ldw) return KVR_E_INVALID_ARGUMENT;
    if (epilogue != KVR_LINEAR_CONCAT && epilogue != KVR_LINEAR_SILU_GATE && epilogue != KVR_LINEAR_RESIDUAL)
        return KVR_E_INVALID_ARGUMENT;
    const bool gated = epilogue == KVR_LINEAR_SILU_GATE;
    if (gated && (n_weights != 2 || rows[0] != rows[1])) return KVR_E_UNSUPPORTED_SHAPE;
    int64_t total = 0;
    for (int i = 0; i < n_weights; ++i) {
        if (rows[i] <= 0) return KVR_E_UNSUPPORTED_SHAPE;
        total += rows[i];
    }
    if (total > (1 << 30)) return KVR_E_UNSUPPORTED_SHAPE;
    const int32_t n_out = gated ? rows[0] : static_cast<int32_t>(total);
    const int32_t splits = kvr_linear_splits(m, static_cast<int32_t>(total), k);
    if (splits < 0) return splits;
    if (ldx < k || ldy < n_out || ldx % 8) return KVR_E_BAD_STRIDE;
    if (epilogue == KVR_LINEAR_RESIDUAL && (!residual || ldr < n_out)) return residual ? KVR_E_BAD_STRIDE : KVR_E_NULL_POINTER;
    for (int i = 0; i < n_weights; ++i)
        if (ldw[i] < k || ldw[i] % 8) return KVR_E_BAD_STRIDE;
    if (!x || !y) return KVR_E_NULL_POINTER;
    for (int i = 0; i < n_weights; ++i)
        if (!w[i]) return KVR_E_NULL_POINTER;
    if (!aligned16(x)) return KVR_E_BAD_STRIDE;
    for (int i = 0; i < n_weights; ++i)
        if (!aligned16(w[i])) return KVR_E_BAD_STRIDE;
    const int64_t need = kvr_linear_workspace_bytes(m, static_cast<int32_t>(total), k);
    if (need > 0 && (!workspace || workspace_bytes < need)) return KVR_E_WORKSPACE_TOO_SMALL;
    GemmArgs a;
    memset(&a, 0, sizeof(a));
    a.x = static_cast<const char*>(x);
    a.w0 = static_cast<const char*>(w[0]);
    a.w1 = static_cast<const char*>(n_weights > 1 ? w[1] : w[0]);
    a.w2 = static_cast<const char*>(n_weights > 2 ? w[2] : a.w1);
    a.ldw0 = ldw[0];
    a.ldw1 = n_weights > 1 ? ldw[1] : ldw[0];
    a.ldw2 = n_weights > 2 ? ldw[2] : a.ldw1;
    a.end0 = rows[0];
    a.end1 = n_weights > 1 ? rows[0] + rows[1] : rows[0];
    a.rows = static_cast<int32_t>(total);
    a.n_out = n_out;
    a.gated = gated ? 1 : 0;
    a.y = static_cast<char*>(y);
    a.res = epilogue == KVR_LINEAR_RESIDUAL ? static_cast<const char*>(residual) : nullptr;
    a.ldr = ldr;
    a.partial = static_cast<float*>(workspace);
    a.ldx = ldx;
    a.ldy = ldy;
    a.m = m;
    a.k = k;
    const Split sp = plan_split(static_cast<int32_t>(total), k);
    a.splits = sp.splits;
    a.slice = sp.slice;
    a.waves = sp.waves;
    if (!reduce && (gated || a.res)) return KVR_E_INVALID_ARGUMENT;  // partial consumers take plain sums
    if (splits_out) *splits_out = sp.splits;
    hipStream_t s = as_stream(stream);
    return dtype == KVR_DTYPE_BF16 ? launch<bf16_t>(a, s, reduce) : launch<f16_t>(a, s, reduce);
}

}  // namespace kvr

extern "C" int kvr_linear_multi(const void* x, int32_t n_weights, const void* const* w, const int32_t* rows,
                                const int64_t* ldw, void* y, int32_t m, int32_t k, int64_t ldx, int64_t ldy,
                                int32_t epilogue, const void* residual, int64_t ldr, void* workspace,
                                int64_t workspace_bytes, int32_t dtype, void* stream) {
    return linear_multi(x, n_weights, w, rows, ldw, y, m, k, ldx, ldy, epilogue, residual, ldr, workspace,
                        workspace_bytes, dtype, stream, true, nullptr);
}

extern "C" int kvr_linear(const void* x, const void* w, void* y, int32_t m, int32_t n, int32_t k, int64_t ldx,
                          int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, int32_t dtype,
                          void* stream) {
    const void* ws[1] = {w};
    const int32_t rows[1] = {n};
    const int64_t lds[1] = {ldw};
    return kvr_linear_multi(x, 1, ws, rows, lds, y, m, k, ldx, ldy, KVR_LINEAR_CONCAT, nullptr, 0, workspace,
                            workspace_bytes, dtype, stream);
}
