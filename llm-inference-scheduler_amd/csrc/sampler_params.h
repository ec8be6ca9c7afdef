// sampler_params.h -- what the C-ABI file and the kernel files share: the
// launch parameters of one mxs_sample call, the workspace layout of the
// small-batch hand-over, and the per-instance launchers (each kernel
// instance lives in a file of its own, k_*.hip, so that they compile in
// parallel).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mxs_device.h"
#include "mxs_sampler.h"   // (MXS_MAX_VOCAB)

namespace mxs {

struct Params {
    const void* logits;
    int B, V;
    long long ld;
    const float* T;
    const int32_t* K;
    const float* P;
    const float* PEN;
    const int32_t* hoff;   // row r's history: hids[hoff[r], hend ? hend[r] : hoff[r + 1])
    const int32_t* hids;
    long long nhids;       // ids in hids: every range read lies in [0, nhids)
    const int32_t* hend;
    const float* U;
    int64_t* out_tok;
    int32_t* out_status;
    float* out_probs;
    // candidates handed over by the slices of k_split (NULL: none): G slices per row
    const uint32_t* sl_hdr;
    const uint32_t* sl_ent;
    int G;
    // the rows' packed maxima from the LM head's epilogue (NULL: none):
    // (greedy key << 32) | ~index, the token of a greedy row without a penalty
    const unsigned long long* pre_best;
    // top-k-off rows shared with helpers (k_fused; NULL: none): the job
    // records, this call's epoch (tags them), and whether every row's
    // workgroup is resident from the start (helpers may wait)
    unsigned char* wj;
    unsigned int epoch;
    int help;
    // (every launch) lines of the workspace whose words the passes of
    // finish_wide2 read when no row is shared (WJ_OWN lines of 64 bytes)
    unsigned int* wown;
};

// ---------------------------------------------------------------- small batches
//
// For B <= SPLIT_MAX_B every row that slice_row takes is cut into G slices
// of consecutive logits, one workgroup each (k_split); each slice hands its
// candidates to the row's finish through the workspace: a header of SL_HDR
// words and up to SLICE_CAP (key, id) pairs per slice.
constexpr int SPLIT_MAX_B = 64;
constexpr int SPLIT_SLICES = 256;              // B * G at most
constexpr int SLICE_CAP = FSEG - 64;           // candidates of one slice (a wave segment's room)
constexpr int SL_HDR = 8;                      // header words: n, key max, key min, est, theta, best lo, best hi
constexpr int SL_CNT_WORD = 7;                 // slice 0's last header word: the row's count of finished slices
constexpr uint32_t SL_NONE = 0xFFFFFFFFu;      // n of a slice that hands over nothing
constexpr size_t SL_HDR_BYTES = (size_t)SPLIT_SLICES * SL_HDR * 4;
constexpr size_t SL_WS_BYTES = SL_HDR_BYTES + (size_t)SPLIT_SLICES * SLICE_CAP * 8;

__host__ __device__ __forceinline__ int split_slices(int B) { return B <= 4 ? 64 : SPLIT_SLICES / B; }
static_assert(SPLIT_MAX_B * (SPLIT_SLICES / SPLIT_MAX_B) <= SPLIT_SLICES && 4 * 64 <= SPLIT_SLICES &&
              SPLIT_SLICES / 5 <= 64, "B * G <= SPLIT_SLICES and G <= 64 (one header per lane)");

// ---------------------------------------------------------------- rows shared with helpers
//
// In k_fused (more than SPLIT_MAX_B rows), a row with top-k off reads its
// logits twice (finish_wide2), about four times as long as a top-k row.  Its
// workgroup (the owner) opens each pass as at most WJ_S slices of whole
// tiles; workgroups that have finished their own rows take slices from the
// back while the owner streams from the front, and hand their results over
// through the workspace, the owner merges them with its own.  The records:
// WJ_NJOB jobs, each a header of WJ_HDR bytes, the helpers' bin counts
// (2048 u32), per slice up to WJ_TOPS top-list entries and WJ_WINS elements
// of each of the two windows (u64), the slices' counts of these (3 x WJ_S
// u32), the row's history bitmap (WJ_BMW u32, written once by the owner)
// and the slices' pass-2 sums (3 x WJ_S u64).  Every record carries the call's epoch, so a call needs no reset
// of the previous call's state.
constexpr int WJ_NJOB = 16;
constexpr int WJ_S = 32;
constexpr int WJ_TOPS = 64;
constexpr int WJ_WINS = 128;
constexpr int WJ_BMW = MXS_MAX_VOCAB / 32;
constexpr size_t WJ_HDR = 256;
constexpr size_t WJ_JOB_BYTES = WJ_HDR + 4 * 2048 + 8 * (size_t)WJ_S * WJ_TOPS + 2 * 8 * (size_t)WJ_S * WJ_WINS +
                                4 * 3 * (size_t)WJ_S + 4 * (size_t)WJ_BMW + 8 * 3 * (size_t)WJ_S;
constexpr int WJ_OWN = 512;   // then a 64-byte line per row (rows r mod WJ_OWN), Params::wown
constexpr size_t WJ_BYTES = WJ_NJOB * WJ_JOB_BYTES + 64 * (size_t)WJ_OWN;

// The launchers of the kernel instances (k_f32.hip, k_f16.hip,
// k_f32_split.hip, k_f16_split.hip).  Each returns the first HIP error of
// its launches, or hipErrorInvalidConfiguration-class errors from raising
// the kernels' LDS limit (lds_error is then set).
template <typename TIn>
hipError_t launch_fused(const Params& p, hipStream_t s, bool& lds_error);
// k_fused with shared top-k-off rows (fp32; k_f32_share.hip)
hipError_t launch_fused_share(const Params& p, hipStream_t s, bool& lds_error);
template <typename TIn>
hipError_t launch_split(const Params& p, hipStream_t s, bool& lds_error);

// k_lmhead.hip: logits = hidden . weight^T and the rows' packed maxima
hipError_t launch_lm_head(const float* H, int B, int D, long long ldh, const float* W, int V, long long ldw,
                          float* C, long long ldc, unsigned long long* best, hipStream_t s);

}  // namespace mxs
