// fbs_rows_ham.hip - the teacher-forced kernels: sequences and scoring; one wavefront per sequence, with the Hamming reads.
#include "fbs_run.h"

namespace fbs {

FBS_HAM_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
