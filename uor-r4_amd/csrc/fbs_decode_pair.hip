// fbs_decode_pair.hip - the decode kernels: decode launches that generate: the prompt (often one token), then each greedy choice fed back (the serving decode loop); paired blocks, two wavefronts per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR_KERNELS(fbs_decode, kPhaseDecode)

}  // namespace fbs
