/*
 * kvr_oracle.c — CPU restatement of the reference packed-refresh arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests compare
 * the HIP kernels against. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never does.
 *
 * Every function cites the reference file:line (paths under
 * /root/reference/src/kv_cache_repair/) whose behaviour it restates.
 * Plain C99, single-threaded, no dependencies beyond libm.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2

/* ---------------------------------------------------------------------------
 * Scalar conversions. bfloat16 rounding is round-to-nearest-even of the fp32
 * bits with a canonical quiet NaN (0x7FC0), the rounding torch applies when a
 * float result is stored to a bfloat16 tensor. fp16 conversion is IEEE
 * binary16 round-to-nearest-even, written from the format definition.
 * ------------------------------------------------------------------------- */
static float u32_as_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f32_as_u32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float orc_bf16_to_f32(uint16_t b) { return u32_as_f32((uint32_t)b << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f32_as_u32(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24 is exact in fp32 */
        const float mag = (float)man * 5.9604644775390625e-08f;
        return sign ? -mag : mag;
    }
    if (exp == 31) return u32_as_f32(sign | 0x7f800000u | (man << 13));
    return u32_as_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
    const uint32_t u = f32_as_u32(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((au >> 13) & 0x3ffu)); /* NaN stays NaN */
    if (au == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    /* Work in double: |f| * 2^24 is an exact integer+fraction for the subnormal
     * range; the normal range rounds the 23-bit mantissa to 10 bits. */
    const double a = (double)u32_as_f32(au);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (a < 6.103515625e-05) {                           /* below 2^-14: subnormal */
        const double scaled = a * 16777216.0;             /* units of 2^-24 */
        double fl = floor(scaled);
        const double rem = scaled - fl;
        uint32_t m = (uint32_t)fl;
        if (rem > 0.5 || (rem == 0.5 && (m & 1u))) ++m;
        return (uint16_t)(sign | m); /* m == 1024 becomes the smallest normal */
    }
    uint32_t exp = (au >> 23) - 112u;  /* fp16 exponent field */
    uint32_t man = au & 0x7fffffu;
    uint32_t keep = man >> 13;
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) {
        ++keep;
        if (keep == 0x400u) {
            keep = 0;
            ++exp;
        }
    }
    return (uint16_t)(sign | (exp << 10) | keep);
}

static float load_elem(const void* base, int dtype, int64_t idx) {
    switch (dtype) {
        case ORC_F32: return ((const float*)base)[idx];
        case ORC_F16: return orc_f16_to_f32(((const uint16_t*)base)[idx]);
        default: return orc_bf16_to_f32(((const uint16_t*)base)[idx]);
    }
}

static void store_elem(void* base, int dtype, int64_t idx, float v) {
    switch (dtype) {
        case ORC_F32: ((float*)base)[idx] = v; break;
        case ORC_F16: ((uint16_t*)base)[idx] = orc_f32_to_f16(v); break;
        default: ((uint16_t*)base)[idx] = orc_f32_to_bf16(v); break;
    }
}

/* One eager elementwise op stores its fp32 result into the tensor dtype. */
static float round_to(int dtype, float v) {
    switch (dtype) {
        case ORC_F32: return v;
        case ORC_F16: return orc_f16_to_f32(orc_f32_to_f16(v));
        default: return orc_bf16_to_f32(orc_f32_to_bf16(v));
    }
}

static void copy_elem(const void* src, int64_t si, void* dst, int64_t di, int dtype) {
    if (dtype == ORC_F32)
        ((uint32_t*)dst)[di] = ((const uint32_t*)src)[si];
    else
        ((uint16_t*)dst)[di] = ((const uint16_t*)src)[si];
}

/* ---------------------------------------------------------------------------
 * RoPE cos/sin for one shared position (reference cache.py:56-68 calls
 * rotary_emb(key, full((1, rows), shift)); transformers 5.15.0
 * modeling_llama.py:113-127 computes freqs = inv_freq * position in fp32,
 * emb = cat(freqs, freqs), cos = emb.cos() * attention_scaling, cast to dtype).
 * The fp32 cos/sin here are the correctly rounded values (evaluated in double).
 * ------------------------------------------------------------------------- */
void orc_rope_cos_sin(const float* inv_freq, int32_t half, int64_t position, float scaling, float* cos_out,
                      float* sin_out) {
    for (int32_t i = 0; i < half; ++i) {
        const float freq = inv_freq[i] * (float)position; /* one fp32 rounding */
        const float c = (float)cos((double)freq);
        const float s = (float)sin((double)freq);
        cos_out[i] = c * scaling;
        sin_out[i] = s * scaling;
    }
}

/*
 * shifted_suffix_keys (cache.py:47-77) for one layer view [1, heads, rows, head_dim]:
 *   out = key * cos + rotate_half(key) * sin      (rotary_dim == head_dim, :73)
 *   rotated part as above, passthrough dims copied (rotary_dim < head_dim, :74-77)
 *   shift == 0 or rows == 0 -> bit copy (clone, :53-54)
 * rotate_half is split-half: [x1, x2] -> [-x2, x1] (cache.py:25-28).
 * cos/sin are cast to the key dtype before the products (:67-68) and every
 * multiply and the add round to the key dtype (eager elementwise ops).
 * cos_tab/sin_tab: fp32 values of length rotary_dim/2, or NULL to use
 * orc_rope_cos_sin(inv_freq, ...).
 */
int orc_rope_rotate(int dtype, const void* src, void* dst, int64_t heads, int64_t rows, int32_t head_dim,
                    int32_t rotary_dim, const int64_t* src_stride, const int64_t* dst_stride, int64_t shift,
                    const float* inv_freq, float scaling, const float* cos_tab, const float* sin_tab) {
    if (rotary_dim <= 0 || rotary_dim > head_dim || (rotary_dim & 1)) return -1;
    const int32_t half = rotary_dim / 2;
    float cs[2048], sn[2048];
    if (half > 2048) return -1;
    if (shift != 0) {
        if (cos_tab && sin_tab) {
            memcpy(cs, cos_tab, sizeof(float) * half);
            memcpy(sn, sin_tab, sizeof(float) * half);
        } else {
            orc_rope_cos_sin(inv_freq, half, shift, scaling, cs, sn);
        }
        for (int32_t i = 0; i < half; ++i) {
            cs[i] = round_to(dtype, cs[i]);
            sn[i] = round_to(dtype, sn[i]);
        }
    }
    for (int64_t h = 0; h < heads; ++h) {
        for (int64_t r = 0; r < rows; ++r) {
            const int64_t sb = h * src_stride[0] + r * src_stride[1];
            const int64_t db = h * dst_stride[0] + r * dst_stride[1];
            if (shift == 0) {
                for (int32_t d = 0; d < head_dim; ++d)
                    copy_elem(src, sb + d * src_stride[2], dst, db + d * dst_stride[2], dtype);
                continue;
            }
            for (int32_t i = 0; i < half; ++i) {
                const float x1 = load_elem(src, dtype, sb + i * src_stride[2]);
                const float x2 = load_elem(src, dtype, sb + (i + half) * src_stride[2]);
                /* key*cos */
                const float a_lo = round_to(dtype, x1 * cs[i]);
                const float a_hi = round_to(dtype, x2 * cs[i]);
                /* rotate_half(key)*sin: first half gets -x2, second half gets x1 */
                const float b_lo = round_to(dtype, (-x2) * sn[i]);
                const float b_hi = round_to(dtype, x1 * sn[i]);
                store_elem(dst, dtype, db + i * dst_stride[2], a_lo + b_lo);
                store_elem(dst, dtype, db + (i + half) * dst_stride[2], a_hi + b_hi);
            }
            for (int32_t d = rotary_dim; d < head_dim; ++d)
                copy_elem(src, sb + d * src_stride[2], dst, db + d * dst_stride[2], dtype);
        }
    }
    return 0;
}

/*
 * Indexed scatter, the reference's default writeback
 * keys.index_copy_(2, positions, key_states) (kernels/packed_cache.py:189-191),
 * with the masked-store rule of the Triton kernel (_indexed_triton.py:22-27):
 * a position outside [0, n_keys) writes nothing. Raw element bits are copied.
 * One tensor per call (K and V are two calls). strides: {head, row, dim}.
 */
void orc_index_copy(int dtype, void* out, const int64_t* out_stride, int64_t n_keys, const void* fresh,
                    const int64_t* fresh_stride, const int64_t* positions, int64_t n_sel, int64_t heads,
                    int32_t head_dim) {
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t r = 0; r < n_sel; ++r) {
            const int64_t p = positions[r];
            if (p < 0 || p >= n_keys) continue;
            for (int32_t d = 0; d < head_dim; ++d)
                copy_elem(fresh, h * fresh_stride[0] + r * fresh_stride[1] + d * fresh_stride[2], out,
                          h * out_stride[0] + p * out_stride[1] + d * out_stride[2], dtype);
        }
}

/*
 * Interval writeback of the interval executors (kernels/writeback.py:18-60,
 * _writeback_triton.py:7-41): rows [in_start, in_start + width) of `src`
 * overwrite rows [out_start, out_start + width) of `out`, both
 * [batch][heads][tokens][head_dim] with element strides {b, h, t, d}. Raw
 * element bits are copied. One tensor per call (K and V are two calls).
 */
void orc_copy_interval(int dtype, void* out, const int64_t* out_stride, const void* src, const int64_t* src_stride,
                       int64_t batch, int64_t heads, int64_t width, int32_t head_dim, int64_t out_start,
                       int64_t in_start) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t p = 0; p < width; ++p)
                for (int32_t d = 0; d < head_dim; ++d)
                    copy_elem(src,
                              b * src_stride[0] + h * src_stride[1] + (in_start + p) * src_stride[2] +
                                  d * src_stride[3],
                              out,
                              b * out_stride[0] + h * out_stride[1] + (out_start + p) * out_stride[2] +
                                  d * out_stride[3],
                              dtype);
}

/*
 * Dense fp64 absolute-causal GQA attention, the reference's independent oracle
 * (tests/test_indexed_attention.py:106-116): K/V repeated per query group,
 * scores = q . k * scale, keys j > positions[r] masked, softmax, @ V.
 * Equivalent to the SDPA branch of _packed_attention (packed_cache.py:60-67)
 * with the mask of packed_cache.py:205-207. Output is fp64 [q_heads][n_sel][head_dim].
 */
void orc_attention_f64(int dtype, const void* q, const int64_t* q_stride, const void* k, const int64_t* k_stride,
                       const void* v, const int64_t* v_stride, const int64_t* positions, int64_t n_sel,
                       int32_t q_heads, int32_t kv_heads, int64_t n_keys, int32_t head_dim, double scale,
                       double* out) {
    const int32_t group = q_heads / kv_heads;
    for (int32_t h = 0; h < q_heads; ++h) {
        const int32_t kh = h / group;
        for (int64_t r = 0; r < n_sel; ++r) {
            const int64_t limit = positions[r] < n_keys - 1 ? positions[r] : n_keys - 1;
            double mx = -INFINITY;
            for (int64_t j = 0; j <= limit; ++j) {
                double s = 0.0;
                for (int32_t d = 0; d < head_dim; ++d)
                    s += (double)load_elem(q, dtype, h * q_stride[0] + r * q_stride[1] + d * q_stride[2]) *
                         (double)load_elem(k, dtype, kh * k_stride[0] + j * k_stride[1] + d * k_stride[2]);
                s *= scale;
                if (s > mx) mx = s;
            }
            double* o = out + ((int64_t)h * n_sel + r) * head_dim;
            for (int32_t d = 0; d < head_dim; ++d) o[d] = 0.0;
            double z = 0.0;
            for (int64_t j = 0; j <= limit; ++j) {
                double s = 0.0;
                for (int32_t d = 0; d < head_dim; ++d)
                    s += (double)load_elem(q, dtype, h * q_stride[0] + r * q_stride[1] + d * q_stride[2]) *
                         (double)load_elem(k, dtype, kh * k_stride[0] + j * k_stride[1] + d * k_stride[2]);
                const double p = exp(s * scale - mx);
                z += p;
                for (int32_t d = 0; d < head_dim; ++d)
                    o[d] += p * (double)load_elem(v, dtype, kh * v_stride[0] + j * v_stride[1] + d * v_stride[2]);
            }
            for (int32_t d = 0; d < head_dim; ++d) o[d] /= z;
        }
    }
}

/*
 * IndexedPlan tile bounds (kernels/indexed_attention.py:75-79): per block of
 * 16 sorted rows, full = (first + 1) // 64 and total = (last + 64) // 64.
 * Returns the tile count.
 */
int64_t orc_plan_tiles(const int64_t* positions, int64_t n, int64_t* full, int64_t* total) {
    int64_t t = 0;
    for (int64_t row = 0; row < n; row += 16, ++t) {
        const int64_t last = row + 15 < n ? row + 15 : n - 1;
        full[t] = (positions[row] + 1) / 64;
        total[t] = (positions[last] + 64) / 64;
    }
    return t;
}

/*
 * token_alignment (alignment.py:21-31) with shared_prefix_len /
 * shared_suffix_len (alignment.py:6-18). out = {prefix, suffix,
 * old_suffix_start, new_suffix_start, mandatory_changed_tokens, position_shift}.
 */
void orc_token_alignment(const int64_t* old_ids, int64_t n_old, const int64_t* new_ids, int64_t n_new, int64_t* out) {
    int64_t prefix = 0;
    while (prefix < n_old && prefix < n_new && old_ids[prefix] == new_ids[prefix]) ++prefix;
    const int64_t maximum = (n_old - prefix) < (n_new - prefix) ? (n_old - prefix) : (n_new - prefix);
    int64_t suffix = 0;
    while (suffix < maximum && old_ids[n_old - 1 - suffix] == new_ids[n_new - 1 - suffix]) ++suffix;
    out[0] = prefix;
    out[1] = suffix;
    out[2] = n_old - suffix;
    out[3] = n_new - suffix;
    out[4] = n_new - prefix - suffix;
    out[5] = (n_new - suffix) - (n_old - suffix);
}

/*
 * positions_to_intervals (execution.py:14-23): sort, de-duplicate and coalesce
 * into maximal half-open runs. `positions` is sorted in place. Writes pairs to
 * `intervals` (capacity 2*n) and returns the interval count.
 */
int64_t orc_positions_to_intervals(int64_t* positions, int64_t n, int64_t* intervals) {
    /* insertion sort: oracle inputs are small */
    for (int64_t i = 1; i < n; ++i) {
        const int64_t x = positions[i];
        int64_t j = i - 1;
        while (j >= 0 && positions[j] > x) {
            positions[j + 1] = positions[j];
            --j;
        }
        positions[j + 1] = x;
    }
    int64_t count = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t p = positions[i];
        if (count && p < intervals[2 * count - 1]) continue; /* duplicate */
        if (count && p == intervals[2 * count - 1]) {
            intervals[2 * count - 1] = p + 1;
        } else {
            intervals[2 * count] = p;
            intervals[2 * count + 1] = p + 1;
            ++count;
        }
    }
    return count;
}
