// fbs_decode_pair8.hip - the decode kernels: decode launches that generate: the prompt (often one token), then each greedy choice fed back (the serving decode loop); paired blocks, int8 table.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR8_KERNELS(fbs_decode, kPhaseDecode)

}  // namespace fbs
