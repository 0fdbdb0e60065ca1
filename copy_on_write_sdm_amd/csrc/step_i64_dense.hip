// dense step kernels (single-step and persistent multi-step) over int64_t
// route indices.
#include "step_kernel.h"
#include "trace_kernel.h"

template void cowsdm_impl::launch_step_w<int64_t, true>(const cowsdm_impl::StepParams&, int,
                                                         int, hipStream_t);
template int32_t cowsdm_impl::launch_trace<int64_t, true>(const cowsdm_impl::StepParams&, int, hipStream_t);
