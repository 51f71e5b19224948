// One packed-refresh decoder layer enqueued by a single host call.
//
// Host code only: it validates the layer/refresh descriptors once, carves the
// caller's scratch slab into the layer's intermediates and enqueues the
// library's own kernels in the order of the decoder layer (transformers
// 5.15.0 modeling_llama.py:301-330, modeling_qwen3.py:287-316):
//
//   normed = rms_norm(hidden)                                   kvr_rms_norm
//   q|k|v  = normed W_qkv^T    (Qwen3: three launches + per-head q/k norms)
//   q_rot, cache[k, v] = rope(q, k) at the positions, scatter   kvr_rope_scatter_kv
//   attn   = packed causal attention(q_rot, cache)              kvr_packed_causal_attention
//   o      = attn W_o^T                                         kvr_linear
//   hidden2 = hidden + o; normed = rms_norm(hidden2)            kvr_rms_norm (residual)
//   act    = silu(normed W_gate^T) * (normed W_up^T)            kvr_linear_multi (gated)
//   hidden = hidden2 + act W_down^T                             kvr_linear_multi (residual)
//
// Every step is the same kernel the Python shells launch, with the same
// arguments, so the layer output is bit-identical to the step-by-step path;
// what disappears is ~10 Python-level dispatches per layer and three split-K
// reduce launches, whose sums are read straight from the partials by the next
// kernel (RoPE + scatter, residual + post-attention norm, residual + the next
// layer's input norm), with the reduce kernel's summation order and rounding.
#include "kvr_internal.h"

namespace kvr {
namespace {

constexpr int64_t kScratchAlign = 256;

int64_t align_up(int64_t v) { return (v + kScratchAlign - 1) / kScratchAlign * kScratchAlign; }

// Byte offsets of the layer's intermediates inside the scratch slab.
struct ScratchLayout {
    int64_t normed, qkv, qn, kn, q_rot, attn, o_out, hidden2, act, total;
};

ScratchLayout scratch_layout(const kvr_refresh_desc* d) {
    const int64_t rows = d->rows;
    const int64_t qd = static_cast<int64_t>(d->q_heads) * d->head_dim;
    const int64_t kd = static_cast<int64_t>(d->kv_heads) * d->head_dim;
    ScratchLayout s{};
    int64_t off = 0;
    auto take = [&](int64_t cols) {
        const int64_t at = off;
        off = align_up(off + rows * cols * 2);
        return at;
    };
    s.normed = take(d->hidden);
    s.qkv = take(qd + 2 * kd);
    s.qn = take(qd);
    s.kn = take(kd);
    s.q_rot = take(qd);
    s.attn = take(qd);
    s.o_out = take(d->hidden);
    s.hidden2 = take(d->hidden);
    s.act = take(d->intermediate);
    s.total = off;
    return s;
}

int check_refresh(const kvr_refresh_desc* d) {
    if (!d) return KVR_E_NULL_POINTER;
    if (d->dtype != KVR_DTYPE_BF16 && d->dtype != KVR_DTYPE_F16) return KVR_E_UNSUPPORTED_DTYPE;
    if (d->rows <= 0 || d->rows > 64 || d->hidden <= 0 || d->q_heads <= 0 || d->kv_heads <= 0 ||
        d->q_heads % d->kv_heads || d->head_dim <= 0 || d->head_dim % 2 || d->intermediate <= 0 || d->n_keys <= 0)
        return KVR_E_UNSUPPORTED_SHAPE;
    const int64_t qd = static_cast<int64_t>(d->q_heads) * d->head_dim;
    // every projection's k (hidden, q_heads * head_dim, intermediate) must be a multiple of 8
    if (d->hidden % 8 || qd % 8 || d->intermediate % 8 || (d->kv_heads * d->head_dim) % 8)
        return KVR_E_UNSUPPORTED_SHAPE;
    if (!(d->scale > 0.f) && !(d->scale < 0.f)) return KVR_E_INVALID_ARGUMENT;
    return KVR_OK;
}

int64_t max_of(int64_t a, int64_t b) { return a > b ? a : b; }

}  // namespace
}  // namespace kvr

using namespace kvr;

extern "C" int64_t kvr_decoder_scratch_bytes(const kvr_refresh_desc* d) {
    const int st = check_refresh(d);
    if (st < 0) return st;
    return scratch_layout(d).total;
}

extern "C" int64_t kvr_decoder_gemm_workspace_bytes(const kvr_refresh_desc* d) {
    const int st = check_refresh(d);
    if (st < 0) return st;
    const int32_t m = d->rows, h = d->hidden, in = d->intermediate;
    const int32_t qd = d->q_heads * d->head_dim, kd = d->kv_heads * d->head_dim;
    const int64_t sizes[] = {
        kvr_linear_workspace_bytes(m, qd + 2 * kd, h), kvr_linear_workspace_bytes(m, qd, h),
        kvr_linear_workspace_bytes(m, kd, h),          kvr_linear_workspace_bytes(m, h, qd),
        kvr_linear_workspace_bytes(m, 2 * in, h),      kvr_linear_workspace_bytes(m, h, in)};
    int64_t need = 0;
    for (int64_t v : sizes) {
        if (v < 0) return v;
        need = max_of(need, v);
    }
    return need;
}

extern "C" int kvr_decoder_layer(const kvr_layer_desc* L, const kvr_refresh_desc* d, void* hidden, void* stream) {
    int st = check_refresh(d);
    if (st < 0) return st;
    if (!L || !hidden || !d->scratch || !d->positions || !d->cos || !d->sin || !d->schedule || !d->host_schedule)
        return KVR_E_NULL_POINTER;
    if (!L->input_norm || !L->post_norm || !L->w_q || !L->w_k || !L->w_v || !L->w_o || !L->w_gate || !L->w_up ||
        !L->w_down || !L->cache_k || !L->cache_v)
        return KVR_E_NULL_POINTER;
    const bool qk_norm = L->q_norm != nullptr;
    if (qk_norm != (L->k_norm != nullptr)) return KVR_E_INVALID_ARGUMENT;
    const ScratchLayout s = scratch_layout(d);
    if (d->scratch_bytes < s.total || (reinterpret_cast<uintptr_t>(d->scratch) & (kScratchAlign - 1)))
        return KVR_E_WORKSPACE_TOO_SMALL;
    const int64_t gemm_need = kvr_decoder_gemm_workspace_bytes(d);
    if (gemm_need < 0) return static_cast<int>(gemm_need);
    if (gemm_need > 0 && (!d->gemm_workspace || d->gemm_workspace_bytes < gemm_need))
        return KVR_E_WORKSPACE_TOO_SMALL;

    char* base = static_cast<char*>(d->scratch);
    char* normed = base + s.normed;
    char* qkv = base + s.qkv;
    char* q_rot = base + s.q_rot;
    char* attn = base + s.attn;
    char* o_out = base + s.o_out;
    char* hidden2 = base + s.hidden2;
    char* act = base + s.act;
    const int32_t m = d->rows, h = d->hidden, in = d->intermediate, dim = d->head_dim;
    const int32_t qd = d->q_heads * dim, kd = d->kv_heads * dim;
    const int32_t dt = d->dtype;
    void* gws = d->gemm_workspace;
    const int64_t gwb = d->gemm_workspace_bytes;

#define KVR_TRY(call)        \
    do {                     \
        st = (call);         \
        if (st < 0) return st; \
    } while (0)

    // input RMSNorm (already in `normed` when the previous layer fused it into its down projection)
    const int64_t rows_h[4] = {h, h, h, h};
    if (!L->input_normed)
        KVR_TRY(kvr_rms_norm(hidden, nullptr, nullptr, normed, L->input_norm, m, h, rows_h, L->eps_input, dt, stream));
    const PartialSums gemm_partials{static_cast<const float*>(gws), 0};
    const bool norm_partials = rms_norm_partials_ok(h, dt);

    // q/k/v projections (+ Qwen3's per-head norms: inside the fresh-row
    // epilogue where its vector kernel serves them, else two kvr_rms_norm launches)
    const char* qp;
    const char* kp;
    const char* vp;
    int64_t q_ld, k_ld, v_ld;
    int32_t qkv_splits = 1;
    const bool norms_in_epilogue =
        qk_norm && rope_norm_fold_ok(dim, dt, L->q_norm, L->k_norm, d->cs_strides, d->cos, d->sin);
    if (!qk_norm || norms_in_epilogue) {
        const void* w[3] = {L->w_q, L->w_k, L->w_v};
        const int32_t rows[3] = {qd, kd, kd};
        const int64_t ldw[3] = {L->ld_q, L->ld_k, L->ld_v};
        KVR_TRY(linear_multi(normed, 3, w, rows, ldw, qkv, m, h, h, qd + 2 * kd, KVR_LINEAR_CONCAT, nullptr, 0, gws,
                             gwb, dt, stream, /*reduce=*/false, &qkv_splits));
        qp = qkv;
        kp = qkv + static_cast<int64_t>(qd) * 2;
        vp = qkv + static_cast<int64_t>(qd + kd) * 2;
        q_ld = k_ld = v_ld = qd + 2 * kd;
    } else {
        char* qb = qkv;
        char* kb = qkv + static_cast<int64_t>(m) * qd * 2;
        char* vb = kb + static_cast<int64_t>(m) * kd * 2;
        KVR_TRY(kvr_linear(normed, L->w_q, qb, m, qd, h, h, L->ld_q, qd, gws, gwb, dt, stream));
        KVR_TRY(kvr_linear(normed, L->w_k, kb, m, kd, h, h, L->ld_k, kd, gws, gwb, dt, stream));
        KVR_TRY(kvr_linear(normed, L->w_v, vb, m, kd, h, h, L->ld_v, kd, gws, gwb, dt, stream));
        const int64_t rows_d[4] = {dim, dim, dim, dim};
        char* qn = base + s.qn;
        char* kn = base + s.kn;
        KVR_TRY(kvr_rms_norm(qb, nullptr, nullptr, qn, L->q_norm, static_cast<int64_t>(m) * d->q_heads, dim, rows_d,
                             L->eps_q, dt, stream));
        KVR_TRY(kvr_rms_norm(kb, nullptr, nullptr, kn, L->k_norm, static_cast<int64_t>(m) * d->kv_heads, dim, rows_d,
                             L->eps_k, dt, stream));
        qp = qn;
        kp = kn;
        vp = vb;
        q_ld = qd;
        k_ld = kd;
        v_ld = kd;
    }

    // RoPE of the fresh q/k at their positions + K/V scatter into this layer's cache
    const int64_t* ck = L->cache_strides;
    const int64_t* cv = L->cache_strides + 3;
    const int64_t rs[18] = {dim, q_ld, 1, dim, qd, 1, dim, k_ld, 1, dim, v_ld, 1,
                            ck[0], ck[1], ck[2], cv[0], cv[1], cv[2]};
    if (qkv_splits > 1) {  // q/k/v straight from the projection's partials
        const int64_t part_col[3] = {0, qd, qd + kd};
        PartialSums p = gemm_partials;
        p.splits = qkv_splits;
        KVR_TRY(rope_scatter_partials(p, part_col, q_rot, L->cache_k, L->cache_v, d->cos, d->sin, d->positions, m,
                                      d->q_heads, d->kv_heads, d->n_keys, dim, rs, d->cs_strides, dt, stream,
                                      norms_in_epilogue ? L->q_norm : nullptr,
                                      norms_in_epilogue ? L->k_norm : nullptr, L->eps_q, L->eps_k));
    } else if (norms_in_epilogue) {
        KVR_TRY(kvr_rope_scatter_kv_norm(qp, q_rot, kp, vp, L->cache_k, L->cache_v, d->cos, d->sin, d->positions, m,
                                         d->q_heads, d->kv_heads, d->n_keys, dim, rs, d->cs_strides, L->q_norm,
                                         L->k_norm, L->eps_q, L->eps_k, dt, stream));
    } else {
        KVR_TRY(kvr_rope_scatter_kv(qp, q_rot, kp, vp, L->cache_k, L->cache_v, d->cos, d->sin, d->positions, m,
                                    d->q_heads, d->kv_heads, d->n_keys, dim, rs, d->cs_strides, dt, stream));
    }

    // packed causal attention over the whole cache; output in [rows][q_heads * dim]
    const int64_t as[12] = {dim, qd, 1, ck[0], ck[1], ck[2], cv[0], cv[1], cv[2], dim, qd, 1};
    KVR_TRY(kvr_packed_causal_attention(q_rot, L->cache_k, L->cache_v, attn, d->positions, m, d->q_heads,
                                        d->kv_heads, d->n_keys, dim, d->scale, as, d->schedule, d->schedule_len,
                                        d->host_schedule, d->attn_workspace, d->attn_workspace_bytes, dt, stream));

    // o projection, residual add + post-attention RMSNorm (from the partials when split)
    {
        const void* w[1] = {L->w_o};
        const int32_t rows[1] = {h};
        const int64_t ldw[1] = {L->ld_o};
        int32_t splits = 1;
        KVR_TRY(linear_multi(attn, 1, w, rows, ldw, o_out, m, qd, qd, h, KVR_LINEAR_CONCAT, nullptr, 0, gws, gwb, dt,
                             stream, /*reduce=*/!norm_partials, &splits));
        if (norm_partials && splits > 1) {
            PartialSums p = gemm_partials;
            p.splits = splits;
            KVR_TRY(rms_norm_partials(p, hidden, hidden2, normed, L->post_norm, m, h, rows_h, L->eps_post, dt,
                                      stream));
        } else {
            KVR_TRY(kvr_rms_norm(o_out, hidden, hidden2, normed, L->post_norm, m, h, rows_h, L->eps_post, dt,
                                 stream));
        }
    }

    // MLP: SiLU-gated gate/up, then down with the residual add, written over `hidden`
    const void* gw[2] = {L->w_gate, L->w_up};
    const int32_t gr[2] = {in, in};
    const int64_t gl[2] = {L->ld_gate, L->ld_up};
    KVR_TRY(kvr_linear_multi(normed, 2, gw, gr, gl, act, m, h, h, in, KVR_LINEAR_SILU_GATE, nullptr, 0, gws, gwb, dt,
                             stream));
    const void* dw[1] = {L->w_down};
    const int32_t dr[1] = {h};
    const int64_t dl[1] = {L->ld_down};
    if (!L->next_norm) {
        KVR_TRY(kvr_linear_multi(act, 1, dw, dr, dl, hidden, m, in, in, h, KVR_LINEAR_RESIDUAL, hidden2, h, gws, gwb,
                                 dt, stream));
    } else {  // ... and the next layer's input norm into `normed`
        int32_t splits = 1;
        if (norm_partials) {
            KVR_TRY(linear_multi(act, 1, dw, dr, dl, o_out, m, in, in, h, KVR_LINEAR_CONCAT, nullptr, 0, gws, gwb, dt,
                                 stream, /*reduce=*/false, &splits));
        }
        if (norm_partials && splits > 1) {
            PartialSums p = gemm_partials;
            p.splits = splits;
            KVR_TRY(rms_norm_partials(p, hidden2, hidden, normed, L->next_norm, m, h, rows_h, L->eps_next, dt,
                                      stream));
        } else {
            if (!norm_partials)
                KVR_TRY(kvr_linear_multi(act, 1, dw, dr, dl, hidden, m, in, in, h, KVR_LINEAR_RESIDUAL, hidden2, h,
                                         gws, gwb, dt, stream));
            else  // one split: the projection was written to o_out
                KVR_TRY(kvr_rms_norm(o_out, hidden2, hidden, normed, L->next_norm, m, h, rows_h, L->eps_next, dt,
                                     stream));
            if (!norm_partials)
                KVR_TRY(kvr_rms_norm(hidden, nullptr, nullptr, normed, L->next_norm, m, h, rows_h, L->eps_next, dt,
                                     stream));
        }
    }
#undef KVR_TRY
    return KVR_OK;
}

extern "C" int kvr_decoder_forward(const kvr_layer_desc* layers, int32_t n_layers, const kvr_refresh_desc* d,
                                   void* hidden, void* stream) {
    if (n_layers < 0) return KVR_E_INVALID_ARGUMENT;
    if (n_layers > 0 && !layers) return KVR_E_NULL_POINTER;
    for (int32_t i = 0; i < n_layers; ++i) {
        const int st = kvr_decoder_layer(layers + i, d, hidden, stream);
        if (st < 0) return st;
    }
    return KVR_OK;
}

extern "C" int kvr_linear_multi_partials(const void* x, int32_t n_weights, const void* const* w,
                                         const int32_t* rows, const int64_t* ldw, void* y, int32_t m, int32_t k,
                                         int64_t ldx, int64_t ldy, void* workspace, int64_t workspace_bytes,
                                         int32_t dtype, void* stream, int32_t* splits_out) {
    if (!splits_out) return KVR_E_NULL_POINTER;
    return kvr::linear_multi(x, n_weights, w, rows, ldw, y, m, k, ldx, ldy, KVR_LINEAR_CONCAT, nullptr, 0, workspace,
                             workspace_bytes, dtype, stream, /*reduce=*/false, splits_out);
}

extern "C" void kvr_decoder_desc_sizes(int64_t sizes[2]) {
    sizes[0] = static_cast<int64_t>(sizeof(kvr_layer_desc));
    sizes[1] = static_cast<int64_t>(sizeof(kvr_refresh_desc));
}
