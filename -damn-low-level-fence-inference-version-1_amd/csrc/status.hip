// status.hip -- status strings and version of the C ABI (host only).
#include "common.hpp"

extern "C" const char* fence_status_string(int status) {
    if (status == FENCE_SUCCESS) return "success";
    if (status == FENCE_ERROR_INVALID_VALUE) return "invalid value (shape, null or misaligned pointer)";
    if (status == FENCE_ERROR_NOT_FOUND) return "not found";
    if (status == FENCE_ERROR_OUT_OF_MEMORY) return "out of memory";
    if (status == FENCE_ERROR_BAD_FILE) return "bad or unreadable GGUF file";
    if (status == FENCE_ERROR_TYPE_MISMATCH) return "metadata value has another type";
    if (status == FENCE_ERROR_UNSUPPORTED) return "unsupported model";
    if (status > FENCE_ERROR_HIP_BASE)
        return hipGetErrorString(static_cast<hipError_t>(status - FENCE_ERROR_HIP_BASE));
    return "unknown status";
}

extern "C" const char* fence_version(void) { return "fence-mi355x 0.1.0 (gfx950)"; }

extern "C" int fence_time_next_launch(hipEvent_t start, hipEvent_t stop) {
    fence::timing_hook() = fence::TimingHook{start, stop, 1};
    return FENCE_SUCCESS;
}

extern "C" int fence_time_next_launches(hipEvent_t start, hipEvent_t stop, int count) {
    if (count < 1) return FENCE_ERROR_INVALID_VALUE;
    fence::timing_hook() = fence::TimingHook{start, stop, count};
    return FENCE_SUCCESS;
}
