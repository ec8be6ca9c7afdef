// k_f16.hip -- k_fused<__half, false>: batches above SPLIT_MAX_B rows, one workgroup per row.
#include "sampler_kernels.h"

namespace mxs {

template <>
hipError_t launch_fused<__half>(const Params& p, hipStream_t s, bool& lds_error)
{
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_fused<__half, false>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, KF_LDS_BYTES);
    if (attr != hipSuccess) { lds_error = true; return attr; }
    hipLaunchKernelGGL((k_fused<__half, false>), dim3((unsigned)p.B), dim3(NT), KF_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace mxs
