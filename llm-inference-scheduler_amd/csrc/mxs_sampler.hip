// mxs_sampler.hip -- the C ABI of include/mxs_sampler.h: argument checks,
// the launch parameters, and the choice of kernel instance (k_*.hip).
//
// Reference chain: mini_engine/sampling.py:30-69, one [vocab] row per call;
// here one call samples a whole [B, V] batch.  Batches of more than
// SPLIT_MAX_B rows run k_fused (one workgroup per row); smaller ones run
// k_split, which splits their rows across workgroups.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "mxs_sampler.h"
#include "sampler_params.h"

using namespace mxs;

namespace {

// The workspace: k_fused keeps a row's state in LDS; the workspace holds
// what the slices of k_split hand over for batches of up to SPLIT_MAX_B
// rows, and their per-row counters (the same size for every batch, so that
// a buffer sized once serves every batch).
constexpr size_t WJ_OFF = (SL_WS_BYTES + 255) & ~(size_t)255;   // the shared-row records
constexpr size_t WORKSPACE_BYTES = (WJ_OFF + WJ_BYTES + 255) & ~(size_t)255;

// mxs_sample_noalloc's workspace: a file-scope device array, one copy per
// GPU (each holds it from the library's load to the process's end).  Host
// code never uses the array's name as an address: the first call on a
// device asks the runtime for that device's copy (hipGetSymbolAddress) and
// keeps the pointer, which is what the kernels receive.
constexpr size_t SCRATCH_BYTES = MXS_NOALLOC_SCRATCH_BYTES;
static_assert(WORKSPACE_BYTES <= SCRATCH_BYTES, "every valid shape fits the static scratch");
constexpr int SCRATCH_MAX_DEVICES = 64;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES];

// The current device's copy of `scratch` (looked up once per device).
int scratch_of_current_device(void** out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEVICES) return MXS_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return MXS_ERR_HIP;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MXS_OK;
}

// The current device's compute-unit count (looked up once per device): a
// batch of at most that many rows has every row's workgroup resident from
// the start, the condition for workgroups to wait for shared rows' slices.
int cus_of_current_device()
{
    static std::mutex mu;
    static int cus[SCRATCH_MAX_DEVICES];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEVICES) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cus[dev] = n;
    }
    return cus[dev];
}

// Each call's epoch, which tags its shared-row records (never 0, the value
// of a zero-filled workspace).
std::atomic<unsigned int> g_epoch{0};

}  // namespace

extern "C" {

const char* mxs_version(void) { return "mxs-sampler 0.2.0 gfx950"; }

const char* mxs_status_string(int status)
{
    switch (status) {
    case MXS_OK: return "ok";
    case MXS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MXS_ERR_ALIGNMENT: return "logits not element-aligned or workspace not 256-byte aligned";
    case MXS_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
    case MXS_ERR_VOCAB_TOO_LARGE: return "vocabulary larger than MXS_MAX_VOCAB";
    case MXS_ERR_HIP: return "HIP runtime error";
    case MXS_ERR_LDS_LIMIT: return "could not raise the kernels' LDS limit to the 152 KB they use (hipFuncSetAttribute failed)";
    case MXS_ERR_SCRATCH_LIMIT: return "the batch needs more workspace than mxs_sample_noalloc's static scratch holds";
    default: return "unknown status";
    }
}

size_t mxs_workspace_bytes(int B, int V)
{
    if (B <= 0 || V <= 0 || V > MXS_MAX_VOCAB) return 0;
    return WORKSPACE_BYTES;
}

}  // extern "C"

namespace {

// Both entry points: the history of row r is hist_ids[hbegin[r], hend[r]),
// with hend == NULL meaning CSR (hend[r] = hbegin[r + 1]).
int sample_impl(const void* logits, int dtype, int B, int V, int64_t ld,
                const float* temperature, const int32_t* top_k,
                const float* top_p, const float* penalty,
                const int32_t* hbegin, const int32_t* hend, const int32_t* hist_ids,
                int64_t n_hist_ids, const float* uniforms,
                int64_t* out_tokens, int32_t* out_status, float* out_probs,
                const uint64_t* row_best, void* workspace, size_t workspace_bytes, mxs_stream_t stream)
{
    if (B < 0 || V <= 0) return MXS_ERR_INVALID_ARGUMENT;
    if (V > MXS_MAX_VOCAB) return MXS_ERR_VOCAB_TOO_LARGE;
    const bool share = (dtype & MXS_FLAG_SHARE_ROWS) != 0;
    dtype &= ~MXS_FLAG_SHARE_ROWS;
    if (dtype != MXS_DTYPE_F32 && dtype != MXS_DTYPE_F16) return MXS_ERR_INVALID_ARGUMENT;
    if (B == 0) return MXS_OK;
    if (!logits || !temperature || !top_k || !top_p || !penalty || !out_tokens || !workspace)
        return MXS_ERR_INVALID_ARGUMENT;
    if (hbegin && (!hist_ids || n_hist_ids < 0)) return MXS_ERR_INVALID_ARGUMENT;
    if (ld < V) return MXS_ERR_INVALID_ARGUMENT;
    const uintptr_t esize = dtype == MXS_DTYPE_F32 ? 4u : 2u;
    if (((uintptr_t)logits & (esize - 1u)) || ((uintptr_t)workspace & 255u)) return MXS_ERR_ALIGNMENT;
    if (workspace_bytes < WORKSPACE_BYTES) return MXS_ERR_WORKSPACE_TOO_SMALL;

    Params p;
    p.logits = logits;
    p.B = B;
    p.V = V;
    p.ld = ld;
    p.T = temperature;
    p.K = top_k;
    p.P = top_p;
    p.PEN = penalty;
    p.hoff = hbegin;
    p.hids = hist_ids;
    p.nhids = hbegin ? (long long)n_hist_ids : 0;
    p.hend = hbegin ? hend : nullptr;
    p.U = uniforms;
    p.out_tok = out_tokens;
    p.out_status = out_status;
    p.out_probs = out_probs;

    p.pre_best = (const unsigned long long*)row_best;
    p.sl_hdr = nullptr;
    p.sl_ent = nullptr;
    p.G = 0;
    p.wj = nullptr;
    p.epoch = 0;
    p.help = 0;
    p.wown = (unsigned int*)((unsigned char*)workspace + WJ_OFF + WJ_NJOB * WJ_JOB_BYTES);
    hipStream_t s = (hipStream_t)stream;
    if (B <= SPLIT_MAX_B) {
        p.G = split_slices(B);
        p.sl_hdr = (const uint32_t*)workspace;
        p.sl_ent = (const uint32_t*)((const char*)workspace + SL_HDR_BYTES);
    } else if (share && dtype == MXS_DTYPE_F32) {
        p.wj = (unsigned char*)workspace + WJ_OFF;
        unsigned int e = ++g_epoch;
        if (e == 0) e = ++g_epoch;
        p.epoch = e;
        const int cus = cus_of_current_device();
        p.help = cus > 0 && B <= cus ? 1 : 0;
    }
    bool lds_error = false;
    hipError_t e;
    if (p.sl_hdr) e = dtype == MXS_DTYPE_F32 ? launch_split<float>(p, s, lds_error) : launch_split<__half>(p, s, lds_error);
    else if (p.wj) e = launch_fused_share(p, s, lds_error);
    else e = dtype == MXS_DTYPE_F32 ? launch_fused<float>(p, s, lds_error) : launch_fused<__half>(p, s, lds_error);
    if (e == hipSuccess) return MXS_OK;
    return lds_error ? MXS_ERR_LDS_LIMIT : MXS_ERR_HIP;
}

}  // namespace

extern "C" {

int mxs_sample(const void* logits, int dtype, int B, int V, int64_t ld,
               const float* temperature, const int32_t* top_k,
               const float* top_p, const float* penalty,
               const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
               const float* uniforms,
               int64_t* out_tokens, int32_t* out_status, float* out_probs,
               void* workspace, size_t workspace_bytes, mxs_stream_t stream)
{
    return sample_impl(logits, dtype, B, V, ld, temperature, top_k, top_p, penalty, hist_offsets, nullptr,
                       hist_ids, n_hist_ids, uniforms, out_tokens, out_status, out_probs, nullptr, workspace,
                       workspace_bytes, stream);
}

int mxs_sample_ranges(const void* logits, int dtype, int B, int V, int64_t ld,
                      const float* temperature, const int32_t* top_k,
                      const float* top_p, const float* penalty,
                      const int32_t* hist_begin, const int32_t* hist_end, const int32_t* hist_ids,
                      int64_t n_hist_ids, const float* uniforms,
                      int64_t* out_tokens, int32_t* out_status, float* out_probs,
                      void* workspace, size_t workspace_bytes, mxs_stream_t stream)
{
    if ((hist_begin != nullptr) != (hist_end != nullptr)) return MXS_ERR_INVALID_ARGUMENT;
    return sample_impl(logits, dtype, B, V, ld, temperature, top_k, top_p, penalty, hist_begin, hist_end,
                       hist_ids, n_hist_ids, uniforms, out_tokens, out_status, out_probs, nullptr, workspace,
                       workspace_bytes, stream);
}

int mxs_sample_noalloc(const void* logits, int dtype, int B, int V, int64_t ld,
                       const float* temperature, const int32_t* top_k,
                       const float* top_p, const float* penalty,
                       const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
                       const float* uniforms,
                       int64_t* out_tokens, int32_t* out_status, float* out_probs,
                       mxs_stream_t stream)
{
    if (B == 0) return MXS_OK;
    const size_t need = mxs_workspace_bytes(B, V);
    if (need > SCRATCH_BYTES) return MXS_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (need > 0) {   // (an invalid shape is rejected by sample_impl below)
        const int st = scratch_of_current_device(&ws);
        if (st != MXS_OK) return st;
    }
    return sample_impl(logits, dtype, B, V, ld, temperature, top_k, top_p, penalty, hist_offsets, nullptr,
                       hist_ids, n_hist_ids, uniforms, out_tokens, out_status, out_probs, nullptr,
                       ws, ws ? SCRATCH_BYTES : 0, stream);
}

int mxs_sample_head(const void* logits, int dtype, int B, int V, int64_t ld,
                    const float* temperature, const int32_t* top_k,
                    const float* top_p, const float* penalty,
                    const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
                    const float* uniforms,
                    int64_t* out_tokens, int32_t* out_status, float* out_probs,
                    const uint64_t* row_best, void* workspace, size_t workspace_bytes, mxs_stream_t stream)
{
    return sample_impl(logits, dtype, B, V, ld, temperature, top_k, top_p, penalty, hist_offsets, nullptr,
                       hist_ids, n_hist_ids, uniforms, out_tokens, out_status, out_probs, row_best, workspace,
                       workspace_bytes, stream);
}

int mxs_lm_head(const float* hidden, int B, int D, int64_t ldh, const float* weight, int V, int64_t ldw,
                float* out_logits, int64_t ldl, uint64_t* out_best, mxs_stream_t stream)
{
    if (B < 0 || D <= 0 || V <= 0) return MXS_ERR_INVALID_ARGUMENT;
    if (B == 0) return MXS_OK;
    if (!hidden || !weight || !out_logits || !out_best) return MXS_ERR_INVALID_ARGUMENT;
    if (ldh < D || ldw < D || ldl < V) return MXS_ERR_INVALID_ARGUMENT;
    if (((uintptr_t)hidden & 15u) || ((uintptr_t)weight & 15u) || (ldh & 3) || (ldw & 3) ||
        ((uintptr_t)out_best & 7u) || ((uintptr_t)out_logits & 3u))
        return MXS_ERR_ALIGNMENT;
    const hipError_t e = launch_lm_head(hidden, B, D, (long long)ldh, weight, V, (long long)ldw, out_logits,
                                        (long long)ldl, (unsigned long long*)out_best, (hipStream_t)stream);
    return e == hipSuccess ? MXS_OK : MXS_ERR_HIP;
}

}  // extern "C"
