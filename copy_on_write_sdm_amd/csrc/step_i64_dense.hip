// dense step kernels over int64_t route indices.
#include "step_kernel.h"

template void cowsdm_impl::launch_step_w<int64_t, true>(const cowsdm_impl::StepParams&, int, int,
                                                         hipStream_t);
