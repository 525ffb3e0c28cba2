// fbs_rows_pair_ham.hip - the rows phase's paired kernels with the Hamming reads: wave 0 the
// recurrence chain and the reads' even heads, wave 1 the window ring and the odd heads.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR_HAM_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
