// fbs_rows.hip - the teacher-forced kernels: sequences and scoring; one wavefront per sequence.
#include "fbs_run.h"

namespace fbs {

FBS_ONE_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
