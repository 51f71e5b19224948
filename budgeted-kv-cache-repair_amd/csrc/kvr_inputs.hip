// Input rows of the packed forward in one launch: the embedding rows of the
// selected tokens and the rotary cos/sin tables at their absolute positions,
// i.e. what LlamaModel/Qwen3Model.forward computes before its first decoder
// layer (transformers 5.15.0 models/llama/modeling_llama.py:377-398 and the
// default-RoPE LlamaRotaryEmbedding.forward, :113-127) for the packed rows.
//
// The rotary module computes in fp32: freqs = inv_freq * float(position) (a
// K = 1 batched matmul, i.e. one rounded product per element), cos/sin of it,
// times attention_scaling, then one rounding to the model dtype. The same
// operations here use the same device math library (cosf/sinf), so the tables
// are bit-identical to the module's on this device.
//
// Block r owns selected row r: it copies embed[ids[positions[r]]] into
// hidden[r] (16-byte vectors when the rows allow) and writes row r of both
// tables. A token id outside [0, vocab) or a position outside [0, n_ids)
// writes a quiet-NaN hidden row instead of reading out of bounds.
#include "kvr_internal.h"

namespace kvr {
namespace {

constexpr int kThreads = 256;

struct InputArgs {
    const char* ids;
    int32_t ids32;
    int64_t n_ids;
    const int64_t* positions;
    const char* embed;
    int64_t vocab, ld_embed;
    int32_t hidden_size;
    char* hidden;
    int64_t ld_hidden;
    const float* inv_freq;
    int32_t head_dim;
    float scaling;
    char* cos;
    char* sin;
    int32_t vec;  // hidden rows move as 16-byte vectors
};

template <typename T>
__global__ void __launch_bounds__(kThreads) refresh_inputs_kernel(InputArgs a) {
    using E = elem<T>;
    using bits = typename E::bits;
    constexpr int esize = E::size;
    const int64_t r = blockIdx.x;
    const int64_t p = a.positions[r];
    int64_t id = -1;
    if (p >= 0 && p < a.n_ids)
        id = a.ids32 ? static_cast<int64_t>(reinterpret_cast<const int32_t*>(a.ids)[p])
                     : reinterpret_cast<const int64_t*>(a.ids)[p];
    const bool ok = id >= 0 && id < a.vocab;

    // hidden row
    char* dst = a.hidden + r * a.ld_hidden * esize;
    const char* src = a.embed + (ok ? id : 0) * a.ld_embed * esize;
    const bits nan = E::from_float(__builtin_nanf(""));  // the dtype's canonical quiet NaN
    if (a.vec) {
        const uint32_t w = esize == 4 ? static_cast<uint32_t>(nan) : (static_cast<uint32_t>(nan) * 0x10001u);
        const u32x4 nan4 = {w, w, w, w};
        const int n16 = a.hidden_size * esize / 16;
        for (int i = threadIdx.x; i < n16; i += kThreads)
            reinterpret_cast<u32x4*>(dst)[i] = ok ? reinterpret_cast<const u32x4*>(src)[i] : nan4;
    } else {
        for (int i = threadIdx.x; i < a.hidden_size; i += kThreads)
            reinterpret_cast<bits*>(dst)[i] = ok ? reinterpret_cast<const bits*>(src)[i] : nan;
    }

    // rotary tables: column d uses frequency d % (head_dim / 2) (the module's cat(freqs, freqs))
    const int half = a.head_dim / 2;
    const float fp = static_cast<float>(p);
    bits* c = reinterpret_cast<bits*>(a.cos) + r * a.head_dim;
    bits* s = reinterpret_cast<bits*>(a.sin) + r * a.head_dim;
    for (int d = threadIdx.x; d < a.head_dim; d += kThreads) {
#pragma clang fp contract(off)
        const float f = fp * a.inv_freq[d < half ? d : d - half];
        c[d] = E::from_float(cosf(f) * a.scaling);
        s[d] = E::from_float(sinf(f) * a.scaling);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kvr

extern "C" int kvr_refresh_inputs(const void* ids, int32_t ids_are_int32, int64_t n_ids, const int64_t* positions,
                                  int64_t n_sel, const void* embed, int64_t vocab, int64_t ld_embed,
                                  int32_t hidden_size, void* hidden, int64_t ld_hidden, const float* inv_freq,
                                  int32_t head_dim, float scaling, void* cos, void* sin, int32_t dtype,
                                  void* stream) {
    using namespace kvr;
    const int esize = dtype_size(dtype);
    if (esize == 0) return KVR_E_UNSUPPORTED_DTYPE;
    if (n_sel < 0 || n_ids < 0 || vocab <= 0 || hidden_size <= 0 || head_dim <= 0 || head_dim % 2)
        return KVR_E_INVALID_ARGUMENT;
    if (ld_embed < hidden_size || ld_hidden < hidden_size) return KVR_E_BAD_STRIDE;
    if (n_sel > 0x7fffffff) return KVR_E_UNSUPPORTED_SHAPE;
    if (n_sel == 0) return KVR_OK;
    if (!ids || !positions || !embed || !hidden || !inv_freq || !cos || !sin) return KVR_E_NULL_POINTER;
    InputArgs a;
    a.ids = static_cast<const char*>(ids);
    a.ids32 = ids_are_int32 ? 1 : 0;
    a.n_ids = n_ids;
    a.positions = positions;
    a.embed = static_cast<const char*>(embed);
    a.vocab = vocab;
    a.ld_embed = ld_embed;
    a.hidden_size = hidden_size;
    a.hidden = static_cast<char*>(hidden);
    a.ld_hidden = ld_hidden;
    a.inv_freq = inv_freq;
    a.head_dim = head_dim;
    a.scaling = scaling;
    a.cos = static_cast<char*>(cos);
    a.sin = static_cast<char*>(sin);
    a.vec = (static_cast<int64_t>(hidden_size) * esize) % 16 == 0 && (ld_embed * esize) % 16 == 0 &&
            (ld_hidden * esize) % 16 == 0 && aligned16(embed) && aligned16(hidden);
    hipStream_t s = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(n_sel));
    if (dtype == KVR_DTYPE_BF16) refresh_inputs_kernel<bf16_t><<<grid, kThreads, 0, s>>>(a);
    else if (dtype == KVR_DTYPE_F16) refresh_inputs_kernel<f16_t><<<grid, kThreads, 0, s>>>(a);
    else refresh_inputs_kernel<f32_t><<<grid, kThreads, 0, s>>>(a);
    return launch_status();
}
