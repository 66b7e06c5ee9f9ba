// step_m4.hip -- instances of the persistent LLAMA decode step for batch 4
// (step_core.h); one translation unit per batch size so they build in parallel.
#include "step_core.h"

extern "C" void *thvm_step_pick_m4(uint32_t wdt, uint32_t adt, uint32_t hd, uint32_t G) {
  return (void *)step_pick<4>(wdt, adt, hd, G);
}
