// One (HEAD_DIM, masked) pair of the attention kernels' instantiations:
// compiled once per pair with -DQF_INST_D=<32|64|128|256> -DQF_INST_MASKED=<0|1>
// (qflash_amd/_build.py), so that the pairs build in parallel.
#ifndef QF_INST_D
#error "QF_INST_D (head dim) and QF_INST_MASKED must be defined"
#endif
#include "qf_fwd.h"

namespace qf {
template hipError_t launch_d<QF_INST_D, (QF_INST_MASKED != 0)>(const Args&, int, bool, bool, int, dim3, hipStream_t);
}  // namespace qf
