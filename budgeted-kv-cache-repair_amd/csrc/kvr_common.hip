// Library-wide entry points: ABI version, status strings, and the host-side
// token alignment of a context edit.
#include "kvr_internal.h"

#include <string.h>

#include <algorithm>
#include <mutex>

extern "C" int kvr_abi_version(void) { return KVR_ABI_VERSION; }

namespace {

// Length of the common run of a[0..n) and b[0..n) from the front (forward) or
// from the back (backward): whole 64-id blocks are compared with memcmp (which
// libc vectorises), the first differing block element by element.
constexpr int64_t kCmpBlock = 64;

int64_t common_front(const int64_t* a, const int64_t* b, int64_t n) {
    int64_t i = 0;
    while (i + kCmpBlock <= n && memcmp(a + i, b + i, kCmpBlock * sizeof(int64_t)) == 0) i += kCmpBlock;
    while (i < n && a[i] == b[i]) ++i;
    return i;
}

// a and b point one past the last element of each run
int64_t common_back(const int64_t* a_end, const int64_t* b_end, int64_t n) {
    int64_t i = 0;
    while (i + kCmpBlock <= n &&
           memcmp(a_end - i - kCmpBlock, b_end - i - kCmpBlock, kCmpBlock * sizeof(int64_t)) == 0)
        i += kCmpBlock;
    while (i < n && a_end[-1 - i] == b_end[-1 - i]) ++i;
    return i;
}

// largest id of the run read unsigned (a negative id reads as >= 2^63)
uint64_t top_id(const int64_t* ids, int64_t n) {
    uint64_t top = 0;
    for (int64_t i = 0; i < n; ++i) top = std::max(top, static_cast<uint64_t>(ids[i]));
    return top;
}

}  // namespace

// Shared prefix, then the shared suffix that does not overlap it
// (src/kv_cache_repair/alignment.py:6-31); then every id of both rows is
// range-checked against the vocabulary (the new row's prefix and suffix equal
// the old row's there, so the old row and the new row's middle cover them all).
extern "C" int kvr_token_alignment(const int64_t* old_ids, int64_t n_old, const int64_t* new_ids, int64_t n_new,
                                   int64_t vocab, int64_t out[6]) {
    if (n_old < 0 || n_new < 0) return KVR_E_INVALID_ARGUMENT;
    if (!out || (n_old && !old_ids) || (n_new && !new_ids)) return KVR_E_NULL_POINTER;
    const int64_t limit = n_old < n_new ? n_old : n_new;
    const int64_t prefix = common_front(old_ids, new_ids, limit);
    const int64_t suffix = limit - prefix ? common_back(old_ids + n_old, new_ids + n_new, limit - prefix) : 0;
    const uint64_t bound = vocab > 0 ? static_cast<uint64_t>(vocab) : ~uint64_t(0) >> 1;
    if (std::max(top_id(old_ids, n_old), top_id(new_ids + prefix, n_new - prefix - suffix)) >= bound)
        return KVR_E_INVALID_ARGUMENT;
    out[0] = prefix;
    out[1] = suffix;
    out[2] = n_old - suffix;
    out[3] = n_new - suffix;
    out[4] = n_new - prefix - suffix;
    out[5] = (n_new - suffix) - (n_old - suffix);
    return KVR_OK;
}

// ---------------------------------------------------------------------------
// Small host-to-device uploads from library-owned pinned staging.
// Each device has a ring of kUploadSlots pinned buffers; an upload takes the
// next slot, waits for that slot's previous copy (recorded event; normally
// long complete), packs the host ranges into it and enqueues one async copy.
// A slot grows (pinned reallocation) only when an upload does not fit it.
namespace {

constexpr int kUploadDevices = 64;
constexpr int kUploadSlots = 8;
constexpr int64_t kUploadMinBytes = 64 << 10;
constexpr int64_t kUploadMaxBytes = int64_t(256) << 20;

struct UploadSlot {
    void* host = nullptr;
    int64_t capacity = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};

struct UploadRing {
    std::mutex mutex;
    UploadSlot slots[kUploadSlots];
    int next = 0;
};

UploadRing g_upload[kUploadDevices];

}  // namespace

extern "C" int kvr_upload_async(void* dst, const void* const* srcs, const int64_t* sizes, int32_t count,
                                void* stream) {
    if (count < 0) return KVR_E_INVALID_ARGUMENT;
    if (count && (!srcs || !sizes)) return KVR_E_NULL_POINTER;
    int64_t total = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (sizes[i] < 0 || sizes[i] > kUploadMaxBytes - total) return KVR_E_INVALID_ARGUMENT;
        if (sizes[i] && !srcs[i]) return KVR_E_NULL_POINTER;
        total += sizes[i];
    }
    if (total == 0) return KVR_OK;  // nothing to copy (an empty destination may be null)
    if (!dst) return KVR_E_NULL_POINTER;
    const hipStream_t s = kvr::as_stream(stream);
    int device = -1;
    if ((s ? hipStreamGetDevice(s, &device) : hipGetDevice(&device)) != hipSuccess || device < 0 ||
        device >= kUploadDevices)
        return KVR_E_DEVICE;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &capture) != hipSuccess) return KVR_E_DEVICE;
    // a captured copy would read the slot again at every replay, after later
    // uploads have refilled it
    if (capture != hipStreamCaptureStatusNone) return KVR_E_INVALID_ARGUMENT;
    UploadRing& ring = g_upload[device];
    std::lock_guard<std::mutex> lock(ring.mutex);
    UploadSlot& slot = ring.slots[ring.next];
    if (slot.pending) {
        if (hipEventSynchronize(slot.done) != hipSuccess) return KVR_E_LAUNCH_FAILED;
        slot.pending = false;
    }
    if (!slot.done && hipEventCreateWithFlags(&slot.done, hipEventDisableTiming) != hipSuccess) {
        slot.done = nullptr;
        return KVR_E_DEVICE;
    }
    if (slot.capacity < total) {
        int64_t capacity = std::max(slot.capacity, kUploadMinBytes);
        while (capacity < total) capacity *= 2;
        void* host = nullptr;
        if (hipHostMalloc(&host, static_cast<size_t>(capacity), hipHostMallocDefault) != hipSuccess || !host)
            return KVR_E_DEVICE;
        if (slot.host) (void)hipHostFree(slot.host);  // no copy from it is pending (waited above)
        slot.host = host;
        slot.capacity = capacity;
    }
    char* staged = static_cast<char*>(slot.host);
    for (int32_t i = 0; i < count; ++i) {
        if (sizes[i]) memcpy(staged, srcs[i], static_cast<size_t>(sizes[i]));
        staged += sizes[i];
    }
    if (hipMemcpyAsync(dst, slot.host, static_cast<size_t>(total), hipMemcpyHostToDevice, s) != hipSuccess)
        return KVR_E_LAUNCH_FAILED;
    if (hipEventRecord(slot.done, s) != hipSuccess) {
        // the copy is enqueued but cannot be tracked: keep this slot out of use
        // until the device has drained
        (void)hipStreamSynchronize(s);
        return KVR_E_LAUNCH_FAILED;
    }
    slot.pending = true;
    ring.next = (ring.next + 1) % kUploadSlots;
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
