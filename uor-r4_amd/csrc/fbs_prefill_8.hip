// fbs_prefill_8.hip - the prefill kernels: decode launches with no generated step (the prompt, its last choice, the state out); one wavefront per sequence, int8 table.
#include "fbs_run.h"

namespace fbs {

FBS_ONE8_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
