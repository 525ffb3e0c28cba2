// fbs_prefill_pair8.hip - the prefill kernels: decode launches with no generated step (the prompt, its last choice, the state out); paired blocks, int8 table.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR8_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
