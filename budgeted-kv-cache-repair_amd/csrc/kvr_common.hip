// Library-wide entry points: ABI version, status strings, and the host-side
// token alignment of a context edit.
#include "kvr_internal.h"

extern "C" int kvr_abi_version(void) { return KVR_ABI_VERSION; }

// Shared prefix, then the shared suffix that does not overlap it
// (src/kv_cache_repair/alignment.py:6-31); ids are range-checked in the same
// pass over the prefix, the suffix and the rows between.
extern "C" int kvr_token_alignment(const int64_t* old_ids, int64_t n_old, const int64_t* new_ids, int64_t n_new,
                                   int64_t vocab, int64_t out[6]) {
    if (n_old < 0 || n_new < 0) return KVR_E_INVALID_ARGUMENT;
    if (!out || (n_old && !old_ids) || (n_new && !new_ids)) return KVR_E_NULL_POINTER;
    const int64_t limit = n_old < n_new ? n_old : n_new;
    int64_t prefix = 0;
    while (prefix < limit && old_ids[prefix] == new_ids[prefix]) ++prefix;
    const int64_t tail = limit - prefix;
    int64_t suffix = 0;
    while (suffix < tail && old_ids[n_old - 1 - suffix] == new_ids[n_new - 1 - suffix]) ++suffix;
    const uint64_t bound = vocab > 0 ? static_cast<uint64_t>(vocab) : ~uint64_t(0) >> 1;
    for (int64_t i = 0; i < n_old; ++i)
        if (static_cast<uint64_t>(old_ids[i]) >= bound) return KVR_E_INVALID_ARGUMENT;
    for (int64_t i = 0; i < n_new; ++i)
        if (static_cast<uint64_t>(new_ids[i]) >= bound) return KVR_E_INVALID_ARGUMENT;
    out[0] = prefix;
    out[1] = suffix;
    out[2] = n_old - suffix;
    out[3] = n_new - suffix;
    out[4] = n_new - prefix - suffix;
    out[5] = (n_new - suffix) - (n_old - suffix);
    return KVR_OK;
}

extern "C" const char* kvr_status_string(int status) {
    switch (status) {
        case KVR_OK: return "ok";
        case KVR_E_INVALID_ARGUMENT: return "invalid argument";
        case KVR_E_UNSUPPORTED_DTYPE: return "unsupported dtype";
        case KVR_E_UNSUPPORTED_SHAPE: return "unsupported shape";
        case KVR_E_BAD_STRIDE: return "unsupported or non-positive stride";
        case KVR_E_NULL_POINTER: return "null pointer";
        case KVR_E_WORKSPACE_TOO_SMALL: return "workspace too small";
        case KVR_E_BAD_SCHEDULE: return "attention schedule does not match the call";
        case KVR_E_LAUNCH_FAILED: return "kernel launch failed";
        case KVR_E_CAPACITY: return "output buffer too small";
        case KVR_E_SCRATCH_LIMIT: return "request needs more scratch than the static scratch array holds";
        case KVR_E_DEVICE: return "device query failed (current device, stream device or symbol address)";
        default: return "unknown status";
    }
}
