// fbs_prefill.hip - the prefill kernels: decode launches with no generated step (the prompt, its last choice, the state out); one wavefront per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_ONE_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
