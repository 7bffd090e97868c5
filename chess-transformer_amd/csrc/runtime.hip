// The library's error reporting, the HIP runtime's address table, and a graph lane's batch in and out as one call each.
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

namespace {
int lane_step(hipError_t status, const char* step) {
    return status == hipSuccess ? CHESS_OK : chess_fail(status, "%s: hip error %d, %s", step, (int)status, hipGetErrorString(status));
}
}  // namespace

// A lane's batch in, as one call: with the lane's device current, the batch's input bytes copied from pinned host
// memory on the lane's stream, the batch size's recorded graph launched behind the copy, and the lane's event recorded
// behind the graph. The reference makes these four runtime calls one by one from Python (engine/inference.py:183-195).
extern "C" int chess_lane_submit(int device, void* stream, void* input, const void* input_host, size_t bytes, void* graph, void* done) {
    if (!stream || !graph || !done || (bytes && (!input || !input_host)))
        return chess_fail(CHESS_INVALID_SHAPE, "lane_submit: a required handle is null");
    hipStream_t lane = (hipStream_t)stream;
    if (int status = lane_step(hipSetDevice(device), "the lane's device")) return status;
    if (bytes)
        if (int status = lane_step(hipMemcpyAsync(input, input_host, bytes, hipMemcpyHostToDevice, lane), "the boards' copy")) return status;
    if (int status = lane_step(hipGraphLaunch((hipGraphExec_t)graph, lane), "the graph's launch")) return status;
    return lane_step(hipEventRecord((hipEvent_t)done, lane), "the batch's event");
}

// A lane's batch out, as one call: with the lane's device current, (when sleep is set) a wait on the lane's event, which
// sleeps when the event was made blocking, then the answers' bytes copied into pinned host memory on the lane's stream
// and the stream's end awaited (the reference's collect, engine/inference.py:199-214).
extern "C" int chess_lane_fetch(int device, void* stream, void* done, int sleep, void* output_host, const void* output, size_t bytes) {
    if (!stream || (sleep && !done) || (bytes && (!output || !output_host)))
        return chess_fail(CHESS_INVALID_SHAPE, "lane_fetch: a required handle is null");
    hipStream_t lane = (hipStream_t)stream;
    if (int status = lane_step(hipSetDevice(device), "the lane's device")) return status;
    if (sleep)
        if (int status = lane_step(hipEventSynchronize((hipEvent_t)done), "the batch")) return status;
    if (bytes)
        if (int status = lane_step(hipMemcpyAsync(output_host, output, bytes, hipMemcpyDeviceToHost, lane), "the answers' copy")) return status;
    return lane_step(hipStreamSynchronize(lane), "the batch");
}

// The gfx target the library was built for, so a loader can refuse a mismatched device.
extern "C" const char* chess_target(void) { return "gfx950"; }
