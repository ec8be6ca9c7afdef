// k_f32.hip -- k_fused<float, false>: batches above SPLIT_MAX_B rows, one workgroup per row.
#include "sampler_kernels.h"

namespace mxs {

template <>
hipError_t launch_fused<float>(const Params& p, hipStream_t s, bool& lds_error)
{
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_fused<float, false>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, KF_LDS_BYTES);
    if (attr != hipSuccess) { lds_error = true; return attr; }
    hipLaunchKernelGGL((k_fused<float, false>), dim3((unsigned)p.B), dim3(NT), KF_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace mxs
