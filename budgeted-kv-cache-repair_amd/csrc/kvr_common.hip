// Library-wide entry points: ABI version and status strings.
#include "kvr_internal.h"

extern "C" int kvr_abi_version(void) { return KVR_ABI_VERSION; }

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
