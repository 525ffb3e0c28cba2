// fbs_decode.hip - the decode kernels: decode launches that generate: the prompt (often one token), then each greedy choice fed back (the serving decode loop); one wavefront per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_ONE_KERNELS(fbs_decode, kPhaseDecode)

}  // namespace fbs
