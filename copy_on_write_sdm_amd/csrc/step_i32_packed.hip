// packed step kernels over int32_t route indices.
#include "step_kernel.h"

template void cowsdm_impl::launch_step_w<int32_t, false>(const cowsdm_impl::StepParams&, int, int,
                                                         hipStream_t);
