// fbs_rows_dt.hip - the traced teacher-forced kernels (uor_fbs_decision_sequences): every
// position's decision and Hamming trace record, under the forced replay's buckets and codes;
// one wavefront per sequence, for 16-bit and int8 tables and for models with Hamming reads.
#include "fbs_run.h"

namespace fbs {

FBS_DT_KERNELS(fbs_rows, kPhaseRows)

}  // namespace fbs
