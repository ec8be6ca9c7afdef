// k_f32_share.hip -- k_fused<float, true>: batches above SPLIT_MAX_B rows whose
// rows with top-k off share their passes with the workgroups that finished
// their own rows (the caller's flag MXS_FLAG_SHARE_ROWS).
#include "sampler_kernels.h"

namespace mxs {

hipError_t launch_fused_share(const Params& p, hipStream_t s, bool& lds_error)
{
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_fused<float, true>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, KF_LDS_BYTES);
    if (attr != hipSuccess) { lds_error = true; return attr; }
    hipLaunchKernelGGL((k_fused<float, true>), dim3((unsigned)p.B), dim3(NT), KF_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace mxs
