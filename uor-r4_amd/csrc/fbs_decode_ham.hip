// fbs_decode_ham.hip - the decode kernels: decode launches that generate: the prompt (often one token), then each greedy choice fed back (the serving decode loop); one wavefront per sequence, with the Hamming reads.
#include "fbs_run.h"

namespace fbs {

FBS_HAM_KERNELS(fbs_decode, kPhaseDecode)

}  // namespace fbs
