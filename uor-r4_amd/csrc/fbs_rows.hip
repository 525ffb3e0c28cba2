// fbs_rows.hip - the rows kernels: the teacher-forced modes: every position of each row, with its choice,
// kept drawers and query (sequences) or the count of next-token matches (score).
#include "fbs_run.h"

namespace fbs {

FBS_PHASE_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
