/*
 * kvrepair.h — C ABI of the MI355X (gfx950) packed refresh executor.
 *
 * Three data-parallel steps of budgeted KV-cache repair run as hand-written
 * HIP kernels behind this header:
 *   1. RoPE delta re-rotation of retained-suffix K rows (and the fused
 *      shift-cache build that also copies the prefix and the V tail),
 *   2. the indexed scatter of refreshed K/V rows into a layer's cache,
 *   3. packed selected-query causal attention with GQA grouping.
 *
 * Conventions shared by every entry point:
 *   - Tensors are rank-4 [batch=1, heads, rows, head_dim] views described by a
 *     base device pointer (the address of element (0,0,0,0)) and three signed
 *     element strides {head, row, dim}. The batch dimension is always 1.
 *   - `dtype` is one of KVR_DTYPE_*; every tensor of a call shares it.
 *   - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream);
 *     NULL means the legacy default stream. Calls only enqueue work on that
 *     stream: no allocation, no free, no host<->device copy, no synchronisation
 *     (the one exception is kvr_upload_async, whose job is a host-to-device
 *     copy from the library's own pinned staging).
 *   - Return value 0 is success; a negative value is a KVR_E_* status whose
 *     text kvr_status_string() gives. Arguments are checked before any launch:
 *     a failed check enqueues nothing.
 *   - Calls are thread-safe and re-entrant; the library keeps no per-request
 *     state.
 */
#ifndef KVREPAIR_H
#define KVREPAIR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVR_ABI_VERSION 1

enum kvr_dtype {
    KVR_DTYPE_F32 = 0,
    KVR_DTYPE_F16 = 1,
    KVR_DTYPE_BF16 = 2,
};

/* Epilogue of kvr_linear_multi. */
enum kvr_linear_epilogue {
    KVR_LINEAR_CONCAT = 0,     /* y[:, off_i + r] = x . w_i[r]; off_i = rows of the weights before i */
    KVR_LINEAR_SILU_GATE = 1,  /* y[:, r] = silu(x . w_0[r]) * (x . w_1[r]), eager rounding */
    KVR_LINEAR_RESIDUAL = 2,   /* as CONCAT, then y = dtype(dtype(y) + residual) (the layer's residual add) */
};

enum kvr_status {
    KVR_OK = 0,
    KVR_E_INVALID_ARGUMENT = -1,
    KVR_E_UNSUPPORTED_DTYPE = -2,
    KVR_E_UNSUPPORTED_SHAPE = -3,
    KVR_E_BAD_STRIDE = -4,
    KVR_E_NULL_POINTER = -5,
    KVR_E_WORKSPACE_TOO_SMALL = -6,
    KVR_E_BAD_SCHEDULE = -7,
    KVR_E_LAUNCH_FAILED = -8,
    KVR_E_CAPACITY = -9,
    KVR_E_SCRATCH_LIMIT = -10,  /* request needs more than the library's static scratch array */
    KVR_E_DEVICE = -11,         /* device query failed (current device, stream device, symbol address) */
};

/* ABI version of the loaded library (KVR_ABI_VERSION at build time). */
int kvr_abi_version(void);

/* Static, NUL-terminated description of a status code. */
const char* kvr_status_string(int status);

/*
 * Asynchronous host-to-device upload of small metadata (a plan's positions and
 * tile bounds, an attention schedule): the `count` host ranges (srcs[i],
 * sizes[i] bytes) are packed back to back into a pinned staging buffer that
 * the library owns, and one copy of the concatenation to `dst` (device memory)
 * is enqueued on `stream`; the call returns without waiting for the device,
 * and the host ranges may be reused as soon as it returns. Each device of a
 * stream has a ring of 8 staging buffers; a buffer is reused only after its
 * previous copy has completed (its event is waited for then). Buffers are
 * pinned with hipHostMalloc on first use and grown when an upload does not fit
 * (at most 256 MiB per upload, else KVR_E_INVALID_ARGUMENT); they are held
 * until the process ends. Refused under stream capture (KVR_E_INVALID_ARGUMENT:
 * a captured copy would read the buffer again at every replay). Thread-safe.
 * No counterpart in the reference, whose plan upload is three
 * torch.tensor(..., device=...) calls (src/kv_cache_repair/kernels/
 * indexed_attention.py:104-107); this one call replaces the chain of host-side
 * tensor operations (pinned staging, packing, copy) of the refresh's set-up.
 */
int kvr_upload_async(void* dst, const void* const* srcs, const int64_t* sizes, int32_t count, void* stream);

/*
 * Host-only token alignment of a context edit (no device access): the
 * reference `token_alignment(old_ids, new_ids)` with `shared_prefix_len` /
 * `shared_suffix_len` (src/kv_cache_repair/alignment.py:6-31). Writes
 * out = {prefix, suffix, old_suffix_start, new_suffix_start,
 * mandatory_changed_tokens, position_shift}. With vocab > 0 every id must lie
 * in [0, vocab) (else KVR_E_INVALID_ARGUMENT; vocab <= 0: ids only nonnegative),
 * the check the shift-cache build makes before any launch that gathers
 * embedding rows by these ids.
 */
int kvr_token_alignment(const int64_t* old_ids, int64_t n_old, const int64_t* new_ids, int64_t n_new,
                        int64_t vocab, int64_t out[6]);

/*
 * RoPE delta re-rotation of retained-suffix keys for every layer in ONE launch.
 *
 * Replaces the per-layer eager chain of the reference
 * `shifted_suffix_keys(model, key, shift)` (src/kv_cache_repair/cache.py:47-77):
 *   cos, sin = rotary_emb(key, full((1, rows), shift))   fp32, cast to dtype
 *   out = key * cos + rotate_half(key) * sin              split-half pairs
 * with each multiply and the add rounded to `dtype` exactly as the eager ops
 * round them. cos/sin are recomputed in fp32 in-kernel from `inv_freq`
 * (the model's rotary_emb.inv_freq as fp32, rotary_dim/2 entries, device
 * memory): freq_i = inv_freq[i] * (float)shift, c = cosf(freq) * scaling.
 * Dims >= rotary_dim pass through unchanged (cache.py:74-77). shift == 0 is an
 * exact bit copy (cache.py:53-54). rows == 0 enqueues nothing.
 *
 * src[l] / dst[l]: per-layer base pointers (host arrays of n_layers device
 * pointers); all layers share the strides. dst must not overlap src.
 */
int kvr_rope_delta_rotate(const void* const* src, void* const* dst, int32_t n_layers, int32_t n_heads,
                          int64_t rows, int32_t head_dim, int32_t rotary_dim, const int64_t src_stride[3],
                          const int64_t dst_stride[3], int64_t shift, const float* inv_freq,
                          float attention_scaling, int32_t dtype, void* stream);

/*
 * Fused shift-cache build: writes a whole shifted cache for every layer in ONE
 * launch (K and V), replacing the per-layer clone/rotate/cat sequence of the
 * reference `build_halo_cache(..., halo_tokens=0)` (cache.py:103-144) when no
 * boundary token needs recomputation:
 *   new_k[:, :, :prefix]           = old_k[:, :, :prefix]            (bit copy)
 *   new_v[:, :, :prefix]           = old_v[:, :, :prefix]            (bit copy)
 *   new_k[:, :, nts:nts+tail_rows] = rotate(old_k[:, :, ots:ots+tail_rows], shift)
 *   new_v[:, :, nts:nts+tail_rows] = old_v[:, :, ots:ots+tail_rows]  (bit copy)
 * with nts = new_tail_start, ots = old_tail_start. Rows of new_* outside those
 * two ranges are not written. The rotation is bit-identical to
 * kvr_rope_delta_rotate.
 */
int kvr_shift_cache_build(const void* const* old_k, const void* const* old_v, void* const* new_k,
                          void* const* new_v, int32_t n_layers, int32_t n_heads, int32_t head_dim,
                          int32_t rotary_dim, const int64_t old_stride[3], const int64_t new_stride[3],
                          int64_t prefix_rows, int64_t old_tail_start, int64_t new_tail_start, int64_t tail_rows,
                          int64_t shift, const float* inv_freq, float attention_scaling, int32_t dtype,
                          void* stream);

/*
 * Indexed K/V scatter (bit copy, NaN payloads included):
 *   out_k[0, h, positions[r], :] = fresh_k[0, h, r, :]   for r < n_sel, h < n_heads
 *   out_v[0, h, positions[r], :] = fresh_v[0, h, r, :]
 * Replaces `_PackedLayer.update`'s index_copy_ pair
 * (src/kv_cache_repair/kernels/packed_cache.py:189-191) and
 * `indexed_kv_scatter_` (src/kv_cache_repair/kernels/indexed_attention.py:179-204).
 * `positions` is a device int64 array; entries outside [0, n_keys) are skipped
 * like the reference Triton kernel's masked store (_indexed_triton.py:22-27).
 * strides: 12 element strides {head,row,dim} for out_k, out_v, fresh_k, fresh_v.
 * n_sel == 0 enqueues nothing.
 */
int kvr_indexed_scatter_kv(void* out_k, void* out_v, const void* fresh_k, const void* fresh_v,
                           const int64_t* positions, int64_t n_sel, int32_t n_heads, int64_t n_keys,
                           int32_t head_dim, const int64_t strides[12], int32_t dtype, void* stream);

/*
 * Input rows of the packed forward in ONE launch: the embedding lookup and the
 * rotary tables that LlamaModel/Qwen3Model.forward computes before its first
 * decoder layer (transformers 5.15.0 models/llama/modeling_llama.py:377-398;
 * default RoPE, LlamaRotaryEmbedding.forward :113-127), for the selected rows:
 *   hidden[r, :] = embed[ids[positions[r]], :]                        (bit copy)
 *   cos[r, d]    = dtype(cosf(float(positions[r]) * inv_freq[d % (D/2)]) * scaling)
 *   sin[r, d]    = dtype(sinf(float(positions[r]) * inv_freq[d % (D/2)]) * scaling)
 * r < n_sel, D = head_dim (even); fp32 product, cos/sin and scaling, one
 * rounding to `dtype`: the rotary module's own operations, bit-identical to its
 * tables on this device. The reference obtains these from the model's modules
 * inside its packed forward (src/kv_cache_repair/kernels/packed_cache.py:
 * 225-298); this entry has no counterpart of its own. ids: n_ids token ids,
 * int32 when ids_are_int32 else int64; positions: n_sel int64 indices into ids.
 * embed: [vocab][ld_embed], hidden: [n_sel][ld_hidden], cos/sin: contiguous
 * [n_sel][head_dim]; inv_freq: head_dim / 2 fp32 values. A position outside
 * [0, n_ids) or a token id outside [0, vocab) writes a quiet-NaN hidden row
 * (nothing is read out of bounds). n_sel == 0 enqueues nothing.
 */
int kvr_refresh_inputs(const void* ids, int32_t ids_are_int32, int64_t n_ids, const int64_t* positions,
                       int64_t n_sel, const void* embed, int64_t vocab, int64_t ld_embed, int32_t hidden_size,
                       void* hidden, int64_t ld_hidden, const float* inv_freq, int32_t head_dim, float scaling,
                       void* cos, void* sin, int32_t dtype, void* stream);

/*
 * Frozen-embedding query relevance of every prompt token in ONE launch (the
 * dense scorer that ranks suffix tokens for the refresh budget,
 * src/kv_cache_repair/scoring.py:11-72, dense_query_relevance_scores):
 *   scores[t] = max_j cos(embed[ids[t]], embed[query_ids[j]]) + boost * [ids[t] in query_ids]
 * cos(a, b) = a.b / (max(|a|, 1e-12) * max(|b|, 1e-12)) in fp32 (F.normalize,
 * then the dot product). embed: [vocab][ld_embed] of `dtype`; ids: n token
 * ids (int32 when ids_are_int32, else int64); query_ids: n_query int64 device
 * ids (n_query > 0); scores: n fp32. One embedding row (padded to 16 bytes)
 * must fit 64 KiB. A token or query id outside [0, vocab) gives NaN scores
 * (nothing is read out of bounds). n == 0 enqueues nothing.
 */
int kvr_query_relevance(const void* embed, int64_t vocab, int64_t ld_embed, int32_t hidden, const void* ids,
                        int32_t ids_are_int32, int64_t n, const int64_t* query_ids, int32_t n_query, float boost,
                        float* scores, int32_t dtype, void* stream);

/*
 * Fresh-row epilogue of one packed layer in ONE launch (RoPE at absolute
 * positions fused with the indexed K/V scatter):
 *   q_out[0, h, r, :]            = rope(q[0, h, r, :], cos[r], sin[r])        h < n_q_heads
 *   out_k[0, h, positions[r], :] = rope(fresh_k[0, h, r, :], cos[r], sin[r])  h < n_kv_heads
 *   out_v[0, h, positions[r], :] = fresh_v[0, h, r, :]                        (bit copy)
 * rope(x) = x * cos + rotate_half(x) * sin (split-half pairs), every multiply
 * and the add rounded to `dtype` as the eager elementwise ops round them, so
 * the result is bit-identical to the native decoder's apply_rotary_pos_emb
 * (transformers 5.15.0 models/llama/modeling_llama.py:137-160) followed by the
 * packed layer's index_copy_ writeback
 * (src/kv_cache_repair/kernels/packed_cache.py:189-191). The reference runs
 * these as separate eager ops; this entry fuses them (no reference
 * counterpart of its own). cos/sin: the rotary embedding's [1, n_sel, head_dim]
 * values in `dtype`; cs_strides = {cos row, cos dim, sin row, sin dim} element
 * strides (row strides may be 0). strides: 18 element strides {head,row,dim}
 * for q, q_out, fresh_k, fresh_v, out_k, out_v. Positions outside [0, n_keys)
 * write no K/V row. head_dim must be even. n_sel == 0 enqueues nothing.
 */
int kvr_rope_scatter_kv(const void* q, void* q_out, const void* fresh_k, const void* fresh_v, void* out_k,
                        void* out_v, const void* cos, const void* sin, const int64_t* positions, int64_t n_sel,
                        int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys, int32_t head_dim,
                        const int64_t strides[18], const int64_t cs_strides[4], int32_t dtype, void* stream);

/*
 * kvr_rope_scatter_kv with Qwen3's per-head RMSNorm of the fresh queries and
 * keys before RoPE (transformers 5.15.0 models/qwen3/modeling_qwen3.py:252-257,
 * q_norm / k_norm of the attention module): each q row uses `q_norm`, each K
 * row `k_norm` ([head_dim] weights in `dtype`, 16-byte aligned), with epsilons
 * eps_q / eps_k; values are not normalised. The norm is HF's
 * w * dtype(x * rsqrt(mean(x^2) + eps)) with kvr_rms_norm's fp32 summation
 * order, so the result is bit-identical to kvr_rms_norm of q and k followed by
 * kvr_rope_scatter_kv. Runs on bf16 / fp32 rows with unit dim strides and
 * 16-byte aligned rows (KVR_E_UNSUPPORTED_SHAPE otherwise: take the two steps
 * separately). Both weights or neither (neither = kvr_rope_scatter_kv). No
 * reference counterpart of its own (the reference runs these as eager ops).
 */
int kvr_rope_scatter_kv_norm(const void* q, void* q_out, const void* fresh_k, const void* fresh_v, void* out_k,
                             void* out_v, const void* cos, const void* sin, const int64_t* positions, int64_t n_sel,
                             int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys, int32_t head_dim,
                             const int64_t strides[18], const int64_t cs_strides[4], const void* q_norm,
                             const void* k_norm, float eps_q, float eps_k, int32_t dtype, void* stream);

/*
 * RMSNorm of `rows` rows of `hidden` elements, with an optional residual add
 * in front (one launch):
 *   s   = residual == NULL ? x : dtype(residual + x)      (s written to residual_out)
 *   out = dtype(weight * dtype(s * rsqrt(mean(s^2) + eps)))
 * Replaces the native decoder's RMSNorm op chain (transformers 5.15.0
 * models/llama/modeling_llama.py:52-69, models/qwen3/modeling_qwen3.py:50-64)
 * and the residual add before the post-attention norm (modeling_llama.py:316-320)
 * for the packed refresh rows; the reference runs them as eager ops (no
 * counterpart of its own). The mean of squares is accumulated in fp32 in this
 * kernel's order, so an element may differ from the eager chain by one unit in
 * the last place of `dtype`. All rows have unit-stride dims; row_strides =
 * {x, residual, residual_out, out} row strides in elements. weight: `hidden`
 * elements of `dtype`. rows == 0 enqueues nothing.
 */
int kvr_rms_norm(const void* x, const void* residual, void* residual_out, void* out, const void* weight,
                 int64_t rows, int32_t hidden, const int64_t row_strides[4], float eps, int32_t dtype,
                 void* stream);

/*
 * Gated activation of the MLP, one launch over n contiguous elements:
 *   out = dtype(dtype(silu(gate)) * up),  silu(g) = g / (1 + exp(-g)) in fp32
 * Replaces act_fn(gate_proj(x)) * up_proj(x) of the native MLP
 * (transformers 5.15.0 models/llama/modeling_llama.py:174-175) for the packed
 * rows (two eager launches; no reference counterpart of its own).
 */
int kvr_silu_mul(const void* gate, const void* up, void* out, int64_t n, int32_t dtype, void* stream);

/*
 * Projection GEMMs of the packed refresh rows (no bias), bf16 / fp16:
 *   y[m, r] = sum_k x[m, k] * w[r, k]     m < M <= 64, fp32 accumulation
 * i.e. torch.nn.functional.linear(x, w) for the few selected rows, replacing
 * the library GEMMs of the native decoder's q/k/v/o and MLP projections
 * (transformers 5.15.0 models/llama/modeling_llama.py:165-175, 243-252; no
 * reference counterpart of its own). Every weight byte is streamed from HBM
 * once. x: row-major [M][ldx]; weights: row-major [rows][ldw] (ldx, ldw
 * multiples of 8 elements, 16-byte aligned bases); y: row-major [M][ldy]; k a
 * multiple of 8. The work is split over K when that fills the GPU better:
 * `workspace` then holds the fp32 partials (kvr_linear_workspace_bytes(m,
 * rows, k) bytes, no initialisation needed) and a second launch on the same
 * stream sums them in slice order. Calls sharing `workspace` must not overlap
 * (one per stream). Results are deterministic (fixed summation order).
 *
 * `rows` of kvr_linear_splits / kvr_linear_workspace_bytes is the number of
 * weight rows one call streams (the sum over its weights).
 */
int32_t kvr_linear_splits(int32_t m, int32_t rows, int32_t k);
int64_t kvr_linear_workspace_bytes(int32_t m, int32_t rows, int32_t k);

/* One weight: y = x w^T (w: [n][ldw]). */
int kvr_linear(const void* x, const void* w, void* y, int32_t m, int32_t n, int32_t k, int64_t ldx, int64_t ldw,
               int64_t ldy, void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream);

/* Up to three weights in one launch. KVR_LINEAR_CONCAT: outputs side by side
 * (the q/k/v projections of one layer into [M][nq + nk + nv]); KVR_LINEAR_RESIDUAL:
 * the same plus `residual` ([M][ldr], may alias y with ldr == ldy) as
 * `residual + down_proj(x)` rounds it (modeling_llama.py:328); `residual`/`ldr`
 * are ignored by the other epilogues;
 * KVR_LINEAR_SILU_GATE: two weights of equal rows (gate_proj, up_proj), y =
 * dtype(dtype(silu(dtype(x gate^T))) * dtype(x up^T)) -- the MLP's
 * act_fn(gate_proj(x)) * up_proj(x) (modeling_llama.py:174) with the
 * rounding of the eager ops, bit-identical to two kvr_linear calls of the
 * same split count followed by kvr_silu_mul. */
int kvr_linear_multi(const void* x, int32_t n_weights, const void* const* w, const int32_t* rows,
                     const int64_t* ldw, void* y, int32_t m, int32_t k, int64_t ldx, int64_t ldy, int32_t epilogue,
                     const void* residual, int64_t ldr, void* workspace, int64_t workspace_bytes, int32_t dtype,
                     void* stream);

/* kvr_linear_multi (KVR_LINEAR_CONCAT) without its split-K reduction, as the
 * packed forward runs the q/k/v, o and down projections whose consumers read
 * the partial sums: with more than one split y is left unwritten and
 * `workspace` holds fp32 partials [ceil(rows / 64)][splits][64 rows][64 cols],
 * element (row, col) of x W^T being the sum over s of
 * tile(col / 64)[s][row][col % 64] in split order (rounded once, that is
 * kvr_linear_multi's y bit for bit); with one split y is written as by
 * kvr_linear_multi. *splits_out receives the split count. No reference
 * counterpart: the reference's projections are nn.Linear calls whose output
 * the next op reads (modeling_llama.py:243-252). */
int kvr_linear_multi_partials(const void* x, int32_t n_weights, const void* const* w, const int32_t* rows,
                              const int64_t* ldw, void* y, int32_t m, int32_t k, int64_t ldx, int64_t ldy,
                              void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream,
                              int32_t* splits_out);

/*
 * One decoder layer of the packed refresh, enqueued by a single call.
 *
 * The packed executor's layer (transformers 5.15.0 modeling_llama.py:301-330 /
 * modeling_qwen3.py:287-316 routed through the packed plugin points of
 * packed_cache.py:85-200 in the reference) as one host call that enqueues its
 * kernels back to back: input RMSNorm -> q/k/v projection (one launch; three for
 * Qwen3, whose per-head q/k RMSNorms follow) -> RoPE of the fresh rows + K/V
 * scatter into this layer's cache -> packed causal attention -> o projection ->
 * residual add + post-attention RMSNorm -> SiLU-gated gate/up projection ->
 * down projection + residual add. Same kernels and arithmetic as the separate
 * entry points, so the result is bit-identical to calling them in that order.
 * `hidden` ([rows][hidden], row-major) is read and overwritten in place with
 * the layer's output. No reference counterpart of its own: it replaces the
 * per-op Python dispatch of the executor's module shells.
 *
 * Split-K projections whose consumer can read the fp32 partials directly skip
 * their reduce launch: the q/k/v sums feed the RoPE + scatter kernel, the o
 * sums the residual add + post-attention norm, the down sums the residual add
 * + the next layer's input norm (`next_norm`; the next call then sets
 * `input_normed`). Those consumers round the sums exactly as the reduce kernel
 * does, so the output stays bit-identical to the separate entry points.
 */
typedef struct kvr_layer_desc {
    const void* input_norm;   /* [hidden] */
    const void* post_norm;    /* [hidden] */
    const void* q_norm;       /* [head_dim] per-head RMSNorm weight (Qwen3) or NULL */
    const void* k_norm;       /* [head_dim] or NULL; both or neither */
    const void* w_q;          /* [q_heads * head_dim][ld_q] */
    const void* w_k;          /* [kv_heads * head_dim][ld_k] */
    const void* w_v;
    const void* w_o;          /* [hidden][ld_o] */
    const void* w_gate;       /* [intermediate][ld_gate] */
    const void* w_up;
    const void* w_down;       /* [hidden][ld_down] */
    int64_t ld_q, ld_k, ld_v, ld_o, ld_gate, ld_up, ld_down;
    float eps_input, eps_post, eps_q, eps_k;
    const void* next_norm;    /* [hidden] input RMSNorm weight of the next layer, or NULL: computed here, */
    float eps_next;           /* fused into the down projection's reduce (its output replaces `hidden`'s */
    int32_t input_normed;     /* norm); nonzero: the previous call already normalised `hidden` this way */
    void* cache_k;            /* this layer's [1, kv_heads, n_keys, head_dim] K and V */
    void* cache_v;
    int64_t cache_strides[6]; /* K {head, row, dim}, V {head, row, dim} in elements */
} kvr_layer_desc;

typedef struct kvr_refresh_desc {
    int32_t rows;             /* selected rows (<= 64) */
    int32_t hidden, q_heads, kv_heads, head_dim, intermediate;
    int64_t n_keys;
    float scale;              /* attention scale */
    int32_t dtype;            /* KVR_DTYPE_BF16 or KVR_DTYPE_F16 */
    const int64_t* positions; /* device, sorted */
    const void* cos;          /* [rows][head_dim] rotary tables at the positions */
    const void* sin;
    int64_t cs_strides[4];    /* cos {row, dim}, sin {row, dim} */
    const int32_t* schedule;  /* kvr_attention_schedule output: device copy, length, host copy */
    int64_t schedule_len;
    const int32_t* host_schedule;
    void* attn_workspace;     /* kvr_attention_workspace_bytes */
    int64_t attn_workspace_bytes;
    void* gemm_workspace;     /* max kvr_linear_workspace_bytes over the layer's projections */
    int64_t gemm_workspace_bytes;
    void* scratch;            /* kvr_decoder_scratch_bytes, 256-byte aligned */
    int64_t scratch_bytes;
} kvr_refresh_desc;

/* Scratch bytes kvr_decoder_layer needs for `d` (negative status if `d` is unsupported). */
int64_t kvr_decoder_scratch_bytes(const kvr_refresh_desc* d);
/* GEMM workspace bytes kvr_decoder_layer needs for `d`. */
int64_t kvr_decoder_gemm_workspace_bytes(const kvr_refresh_desc* d);
int kvr_decoder_layer(const kvr_layer_desc* layer, const kvr_refresh_desc* d, void* hidden, void* stream);
/* kvr_decoder_layer over layers[0 .. n_layers) in order (the packed forward's layer loop). */
int kvr_decoder_forward(const kvr_layer_desc* layers, int32_t n_layers, const kvr_refresh_desc* d, void* hidden,
                        void* stream);
/* sizeof(kvr_layer_desc), sizeof(kvr_refresh_desc): lets bindings check their struct mirrors. */
void kvr_decoder_desc_sizes(int64_t sizes[2]);

/*
 * Interval writeback of the interval executors: rows [in_start, in_start + width)
 * of in_k / in_v overwrite rows [out_start, out_start + width) of out_k / out_v,
 * all [batch][heads][tokens][head_dim] with element strides
 * strides[16] = out_k {b,h,t,d}, out_v {...}, in_k {...}, in_v {...} (all
 * positive). A bit copy, K and V in one launch; outputs must not overlap each
 * other or the inputs (the caller proves it). Replaces copy_kv_interval_
 * (src/kv_cache_repair/kernels/writeback.py:18-60, in_start = out_start) and
 * scatter_fresh_kv (_writeback_triton.py:44-59, in_start = 0).
 */
int kvr_copy_kv_interval(void* out_k, void* out_v, const void* in_k, const void* in_v, int32_t batch,
                         int32_t heads, int64_t width, int32_t head_dim, int64_t out_start, int64_t in_start,
                         const int64_t strides[16], int32_t dtype, void* stream);

/*
 * Host-side work schedule for kvr_packed_causal_attention (no device access).
 * Splits the selected rows into row groups and each group's causal key range
 * [0, positions[last row] + 1) into chunks of `chunk_keys` keys. `positions`
 * is the HOST copy of the strictly increasing selected positions (the
 * reference IndexedPlan.positions, indexed_attention.py:56-83).
 * chunk_keys <= 0 selects a size from the geometry; a positive value must be
 * a multiple of 64. Writes at most `capacity`
 * int32 entries to `schedule` and returns the entry count, or a negative
 * status. With schedule == NULL it returns the required entry count.
 * n_sel == 0 gives a header-only schedule (no work).
 */
int64_t kvr_attention_schedule(const int64_t* positions, int64_t n_sel, int64_t n_keys, int32_t n_q_heads,
                               int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t chunk_keys,
                               int32_t* schedule, int64_t capacity);

/*
 * kvr_attention_schedule with flags. KVR_ATTN_ROUNDED_PROBABILITIES lets the
 * attention round each softmax probability to the input dtype before the PV
 * product, as the SDPA path of the reference packed executor
 * (packed_cache.py:60-67, transformers' sdpa_attention_forward) rounds it; the
 * packed executor builds its schedules this way. Without it (flags 0, what
 * kvr_attention_schedule builds) probabilities enter PV as a hi + lo pair of
 * 16-bit values, the fp32-class precision of the reference Triton operator
 * (_indexed_triton.py:54-58). The flag permits rounding; kernels that do not
 * implement it keep the pair.
 */
#define KVR_ATTN_ROUNDED_PROBABILITIES 1
int64_t kvr_attention_schedule_ex(const int64_t* positions, int64_t n_sel, int64_t n_keys, int32_t n_q_heads,
                                  int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t chunk_keys, int32_t flags,
                                  int32_t* schedule, int64_t capacity);

/* Workspace bytes kvr_packed_causal_attention needs for a schedule (host-only). */
int64_t kvr_attention_workspace_bytes(const int32_t* schedule, int64_t schedule_len, int32_t n_q_heads,
                                      int32_t head_dim);

/*
 * Packed selected-query causal attention, GQA grouped:
 *   out[0, h, r, :] = softmax_{j <= positions[r]}( scale * q[0,h,r,:] . k[0,h/G,j,:] ) @ v[0,h/G,:,:]
 * for h < n_q_heads, r < n_sel, G = n_q_heads / n_kv_heads. Replaces the
 * reference `_packed_attention` SDPA branch (packed_cache.py:47-67, mask
 * key <= position built at :205-207) and `indexed_causal_attention`
 * (indexed_attention.py:207-241). Softmax statistics and accumulation are
 * fp32; QK^T and PV run on bf16/fp16 MFMA (P carried as a hi+lo pair) when
 * dtype is bf16/fp16 and head_dim is 64 or 128, otherwise on the vector ALU.
 * K/V must already hold the fresh selected rows (scatter first, same stream).
 * `positions` (device int64) and `schedule` (device int32, the bytes of
 * kvr_attention_schedule for the same positions/heads) are read-only.
 * strides: 12 element strides {head,row,dim} for q, k, v, out (k and v share
 * n_keys rows). `workspace` holds kvr_attention_workspace_bytes() bytes of
 * scratch, 16-byte aligned (KVR_E_INVALID_ARGUMENT otherwise; no
 * initialisation needed). n_sel == 0 enqueues nothing.
 */
int kvr_packed_causal_attention(const void* q, const void* k, const void* v, void* out, const int64_t* positions,
                                int64_t n_sel, int32_t n_q_heads, int32_t n_kv_heads, int64_t n_keys,
                                int32_t head_dim, float scale, const int64_t strides[12], const int32_t* schedule,
                                int64_t schedule_len, const int32_t* host_schedule, void* workspace,
                                int64_t workspace_bytes, int32_t dtype, void* stream);

/*
 * Allocation-free variant of kvr_packed_causal_attention. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results as
 * kvr_packed_causal_attention, without `workspace`: the split-K partials go to
 * a static device array of kvr_attention_scratch_limit() bytes (128 MiB unless
 * the library is built with -DKVR_ATTN_SCRATCH_MB=<n>) that the library holds
 * on every device where its code object loads, until the process ends. A
 * schedule whose kvr_attention_workspace_bytes exceeds that limit is refused
 * with KVR_E_SCRATCH_LIMIT before anything is launched; use the workspace
 * entry point for it. The call allocates and frees nothing (the first call
 * on a device looks up the array's address and creates one event for the
 * ordering below). `stream` must belong to the current device. All calls on
 * one device share the array (its previous contents are never read: every
 * partial a launch reads is written by the same launch). Calls made outside
 * graph capture are ordered on the device: a call on a stream other than the
 * previous call's first waits (hipStreamWaitEvent, no host blocking) for the
 * previous call to finish, so concurrent streams or threads cannot overlap on
 * the array. Calls captured into a graph are not tracked: replays of captured
 * calls, and eager calls running beside such a replay, must be ordered by the
 * caller (replay on one stream).
 */
int kvr_packed_causal_attention_noalloc(const void* q, const void* k, const void* v, void* out,
                                        const int64_t* positions, int64_t n_sel, int32_t n_q_heads,
                                        int32_t n_kv_heads, int64_t n_keys, int32_t head_dim, float scale,
                                        const int64_t strides[12], const int32_t* schedule, int64_t schedule_len,
                                        const int32_t* host_schedule, int32_t dtype, void* stream);

/* Bytes of the static scratch array behind kvr_packed_causal_attention_noalloc. */
int64_t kvr_attention_scratch_limit(void);

#ifdef __cplusplus
}
#endif

#endif /* KVREPAIR_H */
