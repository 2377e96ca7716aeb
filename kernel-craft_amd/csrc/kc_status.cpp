// kc_status.cpp -- per-thread sticky error channel behind the void launchers.
//
// The reference launchers return void and never check for errors
// (quant_int4.cu:205,233; fp8_quant.cu:219,225,252,277).  The ABI keeps the
// void signatures; the error of the last failed call on a thread is kept
// here until kc_get_last_error() reads it.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "kc_common.hpp"

namespace {
thread_local int t_code = KC_SUCCESS;
thread_local char t_msg[512] = "";
}  // namespace

namespace kc {

int set_error(int code, const char* fmt, ...) {
    t_code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_msg, sizeof(t_msg), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(KC_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return KC_SUCCESS;
}

int sync_stream(hipStream_t stream, const char* what) {
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess)
        return set_error(KC_ERR_HIP, "%s: stream sync failed: %s", what, hipGetErrorString(e));
    return KC_SUCCESS;
}

}  // namespace kc

extern "C" int kc_get_last_error(void) {
    int c = t_code;
    t_code = KC_SUCCESS;
    return c;
}

extern "C" int kc_peek_last_error(void) { return t_code; }

extern "C" const char* kc_last_error_string(void) { return t_msg; }

extern "C" const char* kc_version(void) { return "kernel-craft-hip 0.1.0 (gfx950)"; }
