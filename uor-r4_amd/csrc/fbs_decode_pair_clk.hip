// fbs_decode_pair_clk.hip - the paired decode kernels with the part clocks (the phases of each
// step timed in shader-clock cycles, uor_fbs_decode_parts_async), for 16-bit and int8 tables.
#include "fbs_run.h"

namespace fbs {

FBS_PAIR_CLK_KERNELS(fbs_decode, kPhaseDecode)

}  // namespace fbs
