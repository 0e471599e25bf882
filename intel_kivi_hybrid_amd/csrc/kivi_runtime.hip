// C-ABI runtime glue: status codes, thread-local last-error text, events and
// stream synchronisation.
//
// Replaces the reference's SYCL queue/event glue
// (src/csrc/include/kivi/common.hpp:26-61, src/csrc/include/kivi/event.hpp:16-31):
// every entry point launches on the caller's HIP stream (torch's current
// stream), so ordering is stream order and no private queue exists.  Errors
// never cross the ABI as exceptions; entry points return a status and keep a
// message for kivi_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {

static thread_local char g_last_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return kOk;
    return set_error(kErrRuntime, "%s: %s", what, hipGetErrorString(err));
}

int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err == hipSuccess) return kOk;
    return set_error(kErrLaunch, "kernel launch failed (%s): %s", what,
                     hipGetErrorString(err));
}

}  // namespace kivi

using namespace kivi;

extern "C" {

const char* kivi_last_error(void) { return g_last_error; }

void kivi_clear_error(void) { g_last_error[0] = '\0'; }

int kivi_abi_version(void) { return KIVI_HIP_ABI_VERSION; }

int kivi_stream_synchronize(void* stream) {
    return check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int kivi_event_record(void* stream, void** event_out) {
    if (event_out == nullptr)
        return set_error(kErrInvalidArgument, "event_out must not be null");
    hipEvent_t ev = nullptr;
    int rc = check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming),
                       "hipEventCreateWithFlags");
    if (rc) return rc;
    rc = check_hip(hipEventRecord(ev, (hipStream_t)stream), "hipEventRecord");
    if (rc) {
        (void)hipEventDestroy(ev);
        return rc;
    }
    *event_out = (void*)ev;
    return kOk;
}

int kivi_event_wait(void* event) {
    if (event == nullptr)
        return set_error(kErrInvalidArgument, "event must not be null");
    return check_hip(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
}

int kivi_event_query(void* event) {
    if (event == nullptr)
        return set_error(kErrInvalidArgument, "event must not be null");
    hipError_t err = hipEventQuery((hipEvent_t)event);
    if (err == hipSuccess) return 1;
    if (err == hipErrorNotReady) return 0;
    return -check_hip(err, "hipEventQuery");
}

int kivi_event_destroy(void* event) {
    if (event == nullptr) return kOk;
    return check_hip(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}

}  // extern "C"
