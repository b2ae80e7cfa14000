// Instrumented build of the state-step kernels: every wave stamps its phase
// boundaries (M2R_PHASE_TIMELINE in m2r_step.h).  phase_timeline.py compiles
// this file into lib/libm2r_timeline.so, a separate library with the same
// state-step entry points plus m2r_timeline_set; the library proper is built
// from csrc/*.hip only and carries no stamps.
#define M2R_PHASE_TIMELINE 1
#include "../m2r_state.hip"

// Device buffer for the stamps of the next launches (nullptr: none are
// written): one 32-stamp record per wave, 8 bytes per stamp.
extern "C" int m2r_timeline_set(void* stamps) {
  unsigned long long* p = (unsigned long long*)stamps;
  return m2r_check(hipMemcpyToSymbol(HIP_SYMBOL(m2r::g_phase_stamps), &p, sizeof(p)), "timeline buffer");
}
