// fbs_rows_8.hip - the teacher-forced kernels: sequences and scoring; one wavefront per sequence, int8 table.
#include "fbs_run.h"

namespace fbs {

FBS_ONE8_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
