// fbs_rows_pair.hip - the teacher-forced kernels: sequences and scoring; paired blocks, two wavefronts per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
