// Host-side helpers shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

// Record a failure message for al_last_error() and return `code`.
int al_fail(int code, const char * fmt, ...) __attribute__((format(printf, 2, 3)));
int al_hip_fail(hipError_t e, const char * what);
void al_clear_error();

// Per-device state, created on first use with the device current.
int al_device_cu_count(int * n_cu);
int al_device_lds_per_block(int * bytes);
int al_device_error_flag(int ** flag);   // int[2]: {set, first bad index}
