// fbs_prefill_ham.hip - the prefill kernels: decode launches with no generated step (the prompt, its last choice, the state out); one wavefront per sequence, with the Hamming reads.
#include "fbs_run.h"

namespace fbs {

FBS_HAM_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
