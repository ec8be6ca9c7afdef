// k_f32_split.hip -- k_slices<float> then k_fused<float, true>: batches of up to SPLIT_MAX_B rows.
#include "sampler_kernels.h"

namespace mxs {

template <>
hipError_t launch_split<float>(const Params& p, hipStream_t s, bool& lds_error)
{
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_fused<float, true>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, KF_LDS_BYTES);
    if (attr != hipSuccess) { lds_error = true; return attr; }
    hipLaunchKernelGGL(k_slices<float>, dim3((unsigned)p.G, (unsigned)p.B), dim3(NT), 0, s, p,
                       (uint32_t*)p.sl_hdr, (uint32_t*)p.sl_ent);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_fused<float, true>), dim3((unsigned)p.B), dim3(NT), KF_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace mxs
