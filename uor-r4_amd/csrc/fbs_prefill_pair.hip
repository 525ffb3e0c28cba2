// fbs_prefill_pair.hip - the prefill kernels: decode launches with no generated step (the prompt, its last choice, the state out); paired blocks, two wavefronts per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
