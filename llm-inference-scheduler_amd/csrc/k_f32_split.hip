// k_f32_split.hip -- k_split<float>: batches of up to SPLIT_MAX_B rows, one launch.
#include "sampler_kernels.h"

namespace mxs {

template <>
hipError_t launch_split<float>(const Params& p, hipStream_t s, bool& lds_error)
{
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_split<float>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, KF_LDS_BYTES);
    if (attr != hipSuccess) { lds_error = true; return attr; }
    hipLaunchKernelGGL(k_split<float>, dim3((unsigned)p.G, (unsigned)p.B), dim3(NT), KF_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace mxs
