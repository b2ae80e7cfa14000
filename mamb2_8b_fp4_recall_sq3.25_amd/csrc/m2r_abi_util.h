// Error reporting shared by the C-ABI entry points: a failing entry point
// returns a nonzero status and leaves a message for m2r_last_error().
#pragma once
#include <hip/hip_runtime.h>

int m2r_fail(const char* msg);
int m2r_check(hipError_t e, const char* what);
