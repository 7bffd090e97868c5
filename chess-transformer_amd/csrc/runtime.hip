// The library's error reporting and the HIP runtime's address table.
// chess_runtime_addresses replaces engine/cuda_runtime.py:15-49 (CudaRuntime.addresses), the table of
// runtime entry points that the reference's native round loop (engine/selfplay_rs/src/rounds.rs:19-56)
// calls by address: set device, async copy, graph launch, event record/synchronize, stream
// synchronize and the error string, in that order.
#include "chess_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace {
thread_local char last_error[512] = "";
}

int chess_fail(int code, const char* format, ...) {
    va_list arguments;
    va_start(arguments, format);
    vsnprintf(last_error, sizeof last_error, format, arguments);
    va_end(arguments);
    return code;
}

extern "C" const char* chess_last_error(void) { return last_error; }

extern "C" const char* chess_error_string(int code) {
    switch (code) {
        case CHESS_OK: return "no error";
        case CHESS_INVALID_SHAPE: return "invalid shape or argument";
        case CHESS_MISALIGNED: return "misaligned operand";
        case CHESS_UNSUPPORTED: return "unsupported shape";
        default: return hipGetErrorString((hipError_t)code);
    }
}

extern "C" int chess_runtime_addresses(void** table, int count) {
    void* const entries[] = {
        (void*)&hipSetDevice,        (void*)&hipMemcpyAsync,       (void*)&hipGraphLaunch,    (void*)&hipEventRecord,
        (void*)&hipEventSynchronize, (void*)&hipStreamSynchronize, (void*)&hipGetErrorString,
    };
    const int total = (int)(sizeof entries / sizeof entries[0]);
    if (!table || count < total) return chess_fail(CHESS_INVALID_SHAPE, "the runtime table has %d entries, not %d", total, count);
    for (int i = 0; i < total; i++) table[i] = entries[i];
    return CHESS_OK;
}

// The gfx target the library was built for, so a loader can refuse a mismatched device.
extern "C" const char* chess_target(void) { return "gfx950"; }
