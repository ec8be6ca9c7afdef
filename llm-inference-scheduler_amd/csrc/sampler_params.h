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

// The launchers of the kernel instances (k_f32.hip, k_f16.hip,
// k_f32_split.hip, k_f16_split.hip).  Each returns the first HIP error of
// its launches, or hipErrorInvalidConfiguration-class errors from raising
// the kernels' LDS limit (lds_error is then set).
template <typename TIn>
hipError_t launch_fused(const Params& p, hipStream_t s, bool& lds_error);
template <typename TIn>
hipError_t launch_split(const Params& p, hipStream_t s, bool& lds_error);

// k_lmhead.hip: logits = hidden . weight^T and the rows' packed maxima
hipError_t launch_lm_head(const float* H, int B, int D, long long ldh, const float* W, int V, long long ldw,
                          float* C, long long ldc, unsigned long long* best, hipStream_t s);

}  // namespace mxs
