// Host-side helpers shared by the C-ABI translation units: error reporting
// and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/wisp_hip.h"

namespace wisp {

// thread-local message for wisp_last_error()
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

inline int fail_inval(const char* what) {
    set_error("invalid argument: %s", what);
    return WISP_EINVAL;
}

inline int check_launch(const char* kernel) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s launch failed: %s", kernel, hipGetErrorString(e));
        return (int)e;
    }
    return WISP_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Tuning state (process-wide); see wisp_set_tuning.
struct Tuning {
    int gu_rows;   // rows of one expert per wave, kernel 1 (when H/32 == 64)
    int gu_waves;  // waves per workgroup, kernel 1
    int dn_iters;  // row iterations per workgroup, kernel 2
};
Tuning& tuning();

}  // namespace wisp
