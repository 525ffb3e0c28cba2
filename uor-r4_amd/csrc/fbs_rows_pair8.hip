// fbs_rows_pair8.hip - the teacher-forced kernels: sequences and scoring; paired blocks, int8 table.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR8_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
