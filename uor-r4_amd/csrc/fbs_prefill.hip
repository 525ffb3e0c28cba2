// fbs_prefill.hip - the prefill kernels: decode launches that generate nothing: the prompt, the choice at its last
// position, and the exported session (the serving prefill).
#include "fbs_run.h"

namespace fbs {

FBS_PHASE_KERNELS(fbs_prefill, kPhasePrefill)

}  // namespace fbs
