/*
 * mxs_sampler.h -- C ABI of the MI355X (gfx950) sampler chain.
 *
 * One call samples a whole batch of logits rows on the GPU:
 *   repetition penalty -> greedy (T == 0) -> temperature -> top-k -> top-p
 *   -> softmax -> draw,
 * the chain of mini_engine/sampling.py:30-69, with per-row parameters passed
 * as device arrays.  Plain pointers and sizes only; every buffer belongs to
 * the caller and the library allocates nothing.  A call enqueues one kernel
 * on `stream` and returns; two calls may run concurrently only with
 * distinct workspaces.
 *
 * Results per row (token ids, post-filter probabilities) are defined by the
 * exact arithmetic described in the oracle that the tests check against:
 * integer softmax masses floor(exp(l - m) * 2^44), exact top-p and draw
 * thresholds, ties in value broken by the lowest index, and an inverse-CDF
 * draw (in sorted order) from one uniform per row in place of
 * torch.multinomial's exponential race.
 */
#ifndef MXS_SAMPLER_H
#define MXS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* HIP stream handle; identical to hipStream_t from <hip/hip_runtime_api.h>. */
typedef struct ihipStream_t* mxs_stream_t;

/* Logits element types (sampling.py:36 upcasts fp16 rows to fp32). */
enum mxs_dtype {
    MXS_DTYPE_F32 = 0,
    MXS_DTYPE_F16 = 1
};

/*
 * Or'ed into the dtype argument of the sampling calls: the batch may mix
 * rows with top-k off (top_k <= 0 or >= V, temperature not 0) with other
 * rows.  For fp32 batches of more than 64 rows, the first 16 such rows then
 * share their two reads of the logits with the workgroups that finished
 * their own rows (the caller knows each row's parameters when it builds
 * them; sample_requests sets the flag for such batches).  Results are the
 * same with and without it; without it, a launch carries none of the
 * sharing code, which costs the other rows about a microsecond.
 */
#define MXS_FLAG_SHARE_ROWS 0x100

/* Return codes of the calls below. */
enum mxs_status {
    MXS_OK = 0,
    MXS_ERR_INVALID_ARGUMENT = 1,  /* bad shape, dtype or null pointer */
    MXS_ERR_ALIGNMENT = 2,         /* logits not element-aligned or workspace not 256-byte aligned */
    MXS_ERR_WORKSPACE_TOO_SMALL = 3,
    MXS_ERR_VOCAB_TOO_LARGE = 4,   /* V > MXS_MAX_VOCAB */
    MXS_ERR_HIP = 5,               /* a HIP runtime call failed */
    MXS_ERR_LDS_LIMIT = 6,         /* the kernels' LDS limit could not be raised (hipFuncSetAttribute) */
    MXS_ERR_SCRATCH_LIMIT = 7      /* mxs_sample_noalloc: the batch needs more than its static scratch */
};

/* Per-row outcome written to out_status (out_tokens holds -1 unless OK). */
enum mxs_row_status {
    MXS_ROW_OK = 0,
    MXS_ROW_BAD_HISTORY = 1,    /* a history id is outside [0, V) (torch: IndexError), or the
                                   row's history range lies outside hist_ids */
    MXS_ROW_BAD_PARAM = 2,      /* temperature is NaN */
    MXS_ROW_NONFINITE = 3,      /* a tempered logit is NaN or the max is infinite (torch: multinomial error) */
    MXS_ROW_EMPTY_NUCLEUS = 4   /* top_p <= 0 removes every token (torch: multinomial error) */
};

#define MXS_MAX_VOCAB 262144

/* Library version string, e.g. "mxs-sampler 0.1.0 gfx950". */
const char* mxs_version(void);

/* Human-readable text for an mxs_status value. */
const char* mxs_status_string(int status);

/*
 * Workspace size in bytes for a batch of B rows of V logits (the same for
 * every valid shape, about 4.8 MiB): batches of up to 64 rows split each row
 * across several workgroups, which hand their candidates over in the
 * workspace and count themselves done on a per-row counter kept there;
 * larger batches keep every row's state on chip, and a row with top-k off
 * hands slices of its passes to workgroups that finished their own rows
 * through job records kept there (tagged with the call, so never reset).
 * It must be 256-byte
 * aligned and zero-filled before its first use (every call returns the
 * counters to zero, so a workspace is zero-filled once, not per call); its
 * other contents need not survive between calls.  Returns 0 for an invalid
 * shape.
 */
size_t mxs_workspace_bytes(int B, int V);

/*
 * Sample one token per row.  Replaces the per-row Python call
 * sample(logits[i], params, generated_ids, generator) of
 * mini_engine/sampling.py:30-69 as called from mini_engine/scheduler.py:268-275.
 *
 *   logits        [B, ld] device array of dtype `dtype`; row r uses the first V
 *                 elements.  Rows that start on a 16-byte boundary are read
 *                 with 128-bit loads, other rows element by element.
 *   temperature   f32[B]  0 => greedy argmax (sampling.py:25-27, 47-48)
 *   top_k         i32[B]  <= 0 => off (sampling.py:52)
 *   top_p         f32[B]  >= 1 or NaN => off (sampling.py:56)
 *   penalty       f32[B]  1 => off (sampling.py:38)
 *   hist_offsets  i32[B+1] CSR offsets into hist_ids, or NULL for no history
 *   hist_ids      i32[n_hist_ids] generated token ids (any order, repeats ok)
 *   n_hist_ids    number of ids in hist_ids (>= 0).  A row's history is read
 *                 only when its penalty is not 1 (sampling.py:38); then
 *                 offsets outside [0, n_hist_ids], or hist_offsets[r + 1] <
 *                 hist_offsets[r], make the row MXS_ROW_BAD_HISTORY, and no id
 *                 outside hist_ids is read.
 *   uniforms      f32[B]  one u in [0,1) per row (clamped into it), or NULL for u = 0
 *   out_tokens    i64[B]  sampled ids; -1 for rows whose status is not MXS_ROW_OK
 *   out_status    i32[B]  mxs_row_status per row, or NULL
 *   out_probs     f32[B, V] post-filter probabilities (sampling.py:68), or NULL.
 *                 Greedy rows get a one-hot row.
 *   workspace     device buffer of at least mxs_workspace_bytes(B, V) bytes,
 *                 zero-filled before its first use (see mxs_workspace_bytes)
 */
int mxs_sample(const void* logits, int dtype, int B, int V, int64_t ld,
               const float* temperature, const int32_t* top_k,
               const float* top_p, const float* penalty,
               const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
               const float* uniforms,
               int64_t* out_tokens, int32_t* out_status, float* out_probs,
               void* workspace, size_t workspace_bytes, mxs_stream_t stream);

/*
 * mxs_sample with each row's history given as a range of a caller-owned id
 * buffer: row r's generated ids are hist_ids[hist_begin[r], hist_end[r])
 * (an empty range when hist_end[r] <= hist_begin[r]).  Ranges may overlap
 * and need not be in row order, so a buffer that holds every request's
 * generated ids at fixed places on the device serves any subset of the
 * requests without repacking.  It replaces the per-step rebuild of each
 * request's history from req.output_ids (mini_engine/scheduler.py:43, 275-276,
 * consumed at mini_engine/sampling.py:38-45).  hist_begin and hist_end are
 * both i32[B] device arrays, or both NULL for no history; a non-empty range
 * that leaves [0, n_hist_ids) makes its row MXS_ROW_BAD_HISTORY (when the
 * row's penalty is not 1).  Everything else is as for mxs_sample.
 */
int mxs_sample_ranges(const void* logits, int dtype, int B, int V, int64_t ld,
                      const float* temperature, const int32_t* top_k,
                      const float* top_p, const float* penalty,
                      const int32_t* hist_begin, const int32_t* hist_end, const int32_t* hist_ids,
                      int64_t n_hist_ids, const float* uniforms,
                      int64_t* out_tokens, int32_t* out_status, float* out_probs,
                      void* workspace, size_t workspace_bytes, mxs_stream_t stream);

/*
 * The model's LM head, with the sampler's greedy statistic in its epilogue.
 * Replaces F.linear(h[last_idx], self.lm_head) of
 * mini_engine/model/qwen2.py:176-183 (the tied embedding of :92-96, fp32):
 *
 *   out_logits[r, v] = sum_k hidden[r, k] * weight[v, k]   (fp32; MFMA)
 *   out_best[r]      = max over v of (key(out_logits[r, v]) << 32) | ~v
 *
 * with key the order-preserving key of the value (NaN above every value,
 * -0 equal to +0), so the low word of out_best[r] is the bitwise complement
 * of the row's first maximal index.  hidden is [B, ldh] and weight [V, ldw]
 * (rows 16-byte aligned, ld a multiple of 4), out_logits [B, ldl] with
 * ldl >= V, out_best [B] (8-byte aligned); all device memory.  The sums are
 * fp32 in an order of the kernel's own, so a logit differs from another
 * fp32 summation by rounding (at most D * 2^-23 * sum_k |hidden[r, k]
 * weight[v, k]|).  Asynchronous on `stream`.
 */
int mxs_lm_head(const float* hidden, int B, int D, int64_t ldh, const float* weight, int V, int64_t ldw,
                float* out_logits, int64_t ldl, uint64_t* out_best, mxs_stream_t stream);

/*
 * mxs_sample for logits that mxs_lm_head wrote, with its out_best as
 * row_best (or NULL: then exactly mxs_sample).  A greedy row (temperature
 * 0) without a penalty (penalty 1, or no history) takes its token from
 * row_best and its logits are not read again; every other row is sampled
 * from the logits as by mxs_sample.  row_best must come from the same
 * logits.
 */
int mxs_sample_head(const void* logits, int dtype, int B, int V, int64_t ld,
                    const float* temperature, const int32_t* top_k,
                    const float* top_p, const float* penalty,
                    const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
                    const float* uniforms,
                    int64_t* out_tokens, int32_t* out_status, float* out_probs,
                    const uint64_t* row_best, void* workspace, size_t workspace_bytes, mxs_stream_t stream);

/*
 * mxs_sample without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops and harnesses
 * that forbid allocation).  It has no counterpart in the reference, whose
 * sampler (mini_engine/sampling.py:30-69) allocates freely through torch.
 *
 * It allocates nothing: the workspace is a static device array inside the
 * library, MXS_NOALLOC_SCRATCH_BYTES bytes on each GPU, held from the
 * library's load until the process ends; the first call on a device looks
 * up that device's copy.  It serves every shape mxs_workspace_bytes() sizes
 * at most MXS_NOALLOC_SCRATCH_BYTES (every valid shape of this version) and
 * returns MXS_ERR_SCRATCH_LIMIT for any other.  The scratch of the current
 * device (hipGetDevice) is used, so `stream` must belong to that device.
 * All calls on one GPU share its scratch: calls that may overlap on one
 * GPU (different streams, or different threads) race and must be
 * serialized by the caller.  Arguments and results are as for mxs_sample.
 */
#define MXS_NOALLOC_SCRATCH_BYTES 5044224
int mxs_sample_noalloc(const void* logits, int dtype, int B, int V, int64_t ld,
                       const float* temperature, const int32_t* top_k,
                       const float* top_p, const float* penalty,
                       const int32_t* hist_offsets, const int32_t* hist_ids, int64_t n_hist_ids,
                       const float* uniforms,
                       int64_t* out_tokens, int32_t* out_status, float* out_probs,
                       mxs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MXS_SAMPLER_H */
