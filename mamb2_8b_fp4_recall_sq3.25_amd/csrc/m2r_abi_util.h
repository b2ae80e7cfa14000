// Error reporting shared by the C-ABI entry points: a failing entry point
// returns a nonzero status and leaves a message for m2r_last_error().
#pragma once
#include <hip/hip_runtime.h>

int m2r_fail(const char* msg);
int m2r_check(hipError_t e, const char* what);

// Workgroup shape forced for the state-step kernels by m2r_set_step_shape
// (0 = automatic), encoded as waves_per_block * 16 + heads_per_wave.
int m2r_forced_step_shape();
