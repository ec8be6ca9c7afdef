// sampler_ext.cpp -- thin PyTorch-ROCm extension over the C ABI (mxs_sampler.h).
//
// It checks tensor dtypes, shapes, devices and contiguity, takes torch's
// current HIP stream for the logits' device and forwards raw pointers to
// the C ABI (mxs_sample, mxs_sample_ranges, mxs_sample_head, mxs_lm_head).
// No compute happens here and nothing is allocated: the Python layer
// (mi355x_sampler.batch, mi355x_sampler.head) owns outputs and the workspace.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <optional>
#include <sstream>
#include <string>

#include "mxs_sampler.h"

namespace {

void check_dev(const torch::Tensor& t, const torch::Tensor& ref, const char* name,
               c10::ScalarType dt, int64_t numel)
{
    TORCH_CHECK(t.device() == ref.device(), name, " must be on ", ref.device(), ", got ", t.device());
    TORCH_CHECK(t.scalar_type() == dt, name, " must be ", c10::toString(dt), ", got ", t.scalar_type());
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
    if (numel >= 0) TORCH_CHECK(t.numel() == numel, name, " must have ", numel, " elements, got ", t.numel());
}

const void* opt_ptr(const std::optional<torch::Tensor>& t) { return t ? t->data_ptr() : nullptr; }

void raise_status(int st, const char* what)
{
    if (st == MXS_OK) return;
    std::ostringstream os;
    os << what << " failed: " << mxs_status_string(st) << " (status " << st << ")";
    if (st == MXS_ERR_INVALID_ARGUMENT || st == MXS_ERR_VOCAB_TOO_LARGE || st == MXS_ERR_ALIGNMENT)
        throw std::invalid_argument(os.str());
    throw std::runtime_error(os.str());
}

}  // namespace

int64_t workspace_bytes(int64_t B, int64_t V)
{
    return (int64_t)mxs_workspace_bytes((int)B, (int)V);
}

// mxs_sample, or mxs_sample_head when row_best is given
void sample_common(torch::Tensor logits, torch::Tensor temperature, torch::Tensor top_k,
                   torch::Tensor top_p, torch::Tensor penalty,
                   std::optional<torch::Tensor> hist_offsets, std::optional<torch::Tensor> hist_ids,
                   std::optional<torch::Tensor> uniforms, torch::Tensor out_tokens,
                   std::optional<torch::Tensor> out_status, std::optional<torch::Tensor> out_probs,
                   const std::optional<torch::Tensor>& row_best, torch::Tensor workspace, int64_t flags)
{
    TORCH_CHECK(logits.is_cuda(), "logits must be on a GPU device");
    TORCH_CHECK(logits.dim() == 2, "logits must be [B, V]");
    TORCH_CHECK(logits.stride(1) == 1, "logits rows must be contiguous");
    const int64_t B = logits.size(0), V = logits.size(1);
    int dtype;
    if (logits.scalar_type() == torch::kFloat32) dtype = MXS_DTYPE_F32;
    else if (logits.scalar_type() == torch::kFloat16) dtype = MXS_DTYPE_F16;
    else TORCH_CHECK(false, "logits must be float32 or float16, got ", logits.scalar_type());
    TORCH_CHECK((flags & ~(int64_t)MXS_FLAG_SHARE_ROWS) == 0, "unknown flags ", flags);
    dtype |= (int)flags;

    check_dev(temperature, logits, "temperature", torch::kFloat32, B);
    check_dev(top_k, logits, "top_k", torch::kInt32, B);
    check_dev(top_p, logits, "top_p", torch::kFloat32, B);
    check_dev(penalty, logits, "penalty", torch::kFloat32, B);
    TORCH_CHECK(hist_offsets.has_value() == hist_ids.has_value(),
                "hist_offsets and hist_ids go together");
    if (hist_offsets) {
        check_dev(*hist_offsets, logits, "hist_offsets", torch::kInt32, B + 1);
        check_dev(*hist_ids, logits, "hist_ids", torch::kInt32, -1);
    }
    if (uniforms) check_dev(*uniforms, logits, "uniforms", torch::kFloat32, B);
    check_dev(out_tokens, logits, "out_tokens", torch::kInt64, B);
    if (out_status) check_dev(*out_status, logits, "out_status", torch::kInt32, B);
    if (out_probs) check_dev(*out_probs, logits, "out_probs", torch::kFloat32, B * V);
    TORCH_CHECK(workspace.device() == logits.device() && workspace.is_contiguous() &&
                workspace.scalar_type() == torch::kUInt8, "workspace must be a uint8 tensor on the logits device");

    const c10::DeviceGuard guard(logits.device());
    auto stream = c10::hip::getCurrentHIPStream();
    const int32_t* hoff = hist_offsets ? hist_offsets->data_ptr<int32_t>() : nullptr;
    // An empty id list may have no storage; any valid pointer will do since
    // the offsets then select no ids.
    const int32_t* hids = nullptr;
    if (hist_ids) hids = hist_ids->numel() ? hist_ids->data_ptr<int32_t>() : hoff;
    const int64_t nids = hist_ids ? hist_ids->numel() : 0;
    int st;
    if (row_best) {
        st = mxs_sample_head(logits.data_ptr(), dtype, (int)B, (int)V, logits.stride(0),
                             temperature.data_ptr<float>(), top_k.data_ptr<int32_t>(),
                             top_p.data_ptr<float>(), penalty.data_ptr<float>(), hoff, hids, nids,
                             (const float*)opt_ptr(uniforms), out_tokens.data_ptr<int64_t>(),
                             out_status ? out_status->data_ptr<int32_t>() : nullptr,
                             out_probs ? out_probs->data_ptr<float>() : nullptr,
                             (const uint64_t*)row_best->data_ptr(), workspace.data_ptr(),
                             (size_t)workspace.numel(), (mxs_stream_t)stream.stream());
        raise_status(st, "mxs_sample_head");
        return;
    }
    st = mxs_sample(logits.data_ptr(), dtype, (int)B, (int)V, logits.stride(0),
                    temperature.data_ptr<float>(), top_k.data_ptr<int32_t>(),
                    top_p.data_ptr<float>(), penalty.data_ptr<float>(), hoff, hids, nids,
                    (const float*)opt_ptr(uniforms), out_tokens.data_ptr<int64_t>(),
                    out_status ? out_status->data_ptr<int32_t>() : nullptr,
                    out_probs ? out_probs->data_ptr<float>() : nullptr,
                    workspace.data_ptr(), (size_t)workspace.numel(),
                    (mxs_stream_t)stream.stream());
    raise_status(st, "mxs_sample");
}

void sample(torch::Tensor logits, torch::Tensor temperature, torch::Tensor top_k,
            torch::Tensor top_p, torch::Tensor penalty,
            std::optional<torch::Tensor> hist_offsets, std::optional<torch::Tensor> hist_ids,
            std::optional<torch::Tensor> uniforms, torch::Tensor out_tokens,
            std::optional<torch::Tensor> out_status, std::optional<torch::Tensor> out_probs,
            torch::Tensor workspace, int64_t flags)
{
    sample_common(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids, uniforms, out_tokens,
                  out_status, out_probs, std::nullopt, workspace, flags);
}

// mxs_sample_head: greedy rows without a penalty take their token from
// row_best, the maxima lm_head wrote for these logits
void sample_head(torch::Tensor logits, torch::Tensor temperature, torch::Tensor top_k,
                 torch::Tensor top_p, torch::Tensor penalty,
                 std::optional<torch::Tensor> hist_offsets, std::optional<torch::Tensor> hist_ids,
                 std::optional<torch::Tensor> uniforms, torch::Tensor out_tokens,
                 std::optional<torch::Tensor> out_status, std::optional<torch::Tensor> out_probs,
                 torch::Tensor row_best, torch::Tensor workspace, int64_t flags)
{
    check_dev(row_best, logits, "row_best", torch::kInt64, logits.dim() == 2 ? logits.size(0) : -1);
    sample_common(logits, temperature, top_k, top_p, penalty, hist_offsets, hist_ids, uniforms, out_tokens,
                  out_status, out_probs, row_best, workspace, flags);
}

// logits = hidden . weight^T and the rows' packed maxima (mxs_lm_head)
void lm_head(torch::Tensor hidden, torch::Tensor weight, torch::Tensor out_logits, torch::Tensor out_best)
{
    TORCH_CHECK(hidden.is_cuda(), "hidden must be on a GPU device");
    TORCH_CHECK(hidden.dim() == 2 && weight.dim() == 2 && out_logits.dim() == 2,
                "hidden [B, D], weight [V, D] and out_logits [B, V] are matrices");
    const int64_t B = hidden.size(0), D = hidden.size(1), V = weight.size(0);
    TORCH_CHECK(weight.size(1) == D, "weight must be [V, ", D, "], got ", weight.sizes());
    TORCH_CHECK(out_logits.size(0) == B && out_logits.size(1) == V, "out_logits must be [", B, ", ", V, "]");
    for (const auto* t : {&hidden, &weight, &out_logits}) {
        TORCH_CHECK(t->device() == hidden.device(), "all tensors must be on ", hidden.device());
        TORCH_CHECK(t->scalar_type() == torch::kFloat32, "hidden, weight and out_logits must be float32");
        TORCH_CHECK(t->stride(1) == 1, "rows must be contiguous");
    }
    check_dev(out_best, hidden, "out_best", torch::kInt64, B);
    TORCH_CHECK(B <= INT32_MAX && D <= INT32_MAX && V <= INT32_MAX, "sizes must fit in int32");
    const c10::DeviceGuard guard(hidden.device());
    auto stream = c10::hip::getCurrentHIPStream();
    int st = mxs_lm_head(hidden.data_ptr<float>(), (int)B, (int)D, hidden.stride(0), weight.data_ptr<float>(),
                         (int)V, weight.stride(0), out_logits.data_ptr<float>(), out_logits.stride(0),
                         (uint64_t*)out_best.data_ptr(), (mxs_stream_t)stream.stream());
    raise_status(st, "mxs_lm_head");
}

// The same launch with row r's history at hist_ids[hist_begin[r], hist_end[r])
// (mxs_sample_ranges): hist_ids may be a buffer that stays on the device.
void sample_ranges(torch::Tensor logits, torch::Tensor temperature, torch::Tensor top_k,
                   torch::Tensor top_p, torch::Tensor penalty,
                   torch::Tensor hist_begin, torch::Tensor hist_end, torch::Tensor hist_ids,
                   std::optional<torch::Tensor> uniforms, torch::Tensor out_tokens,
                   std::optional<torch::Tensor> out_status, std::optional<torch::Tensor> out_probs,
                   torch::Tensor workspace, int64_t flags)
{
    TORCH_CHECK(logits.is_cuda(), "logits must be on a GPU device");
    TORCH_CHECK(logits.dim() == 2, "logits must be [B, V]");
    TORCH_CHECK(logits.stride(1) == 1, "logits rows must be contiguous");
    const int64_t B = logits.size(0), V = logits.size(1);
    int dtype;
    if (logits.scalar_type() == torch::kFloat32) dtype = MXS_DTYPE_F32;
    else if (logits.scalar_type() == torch::kFloat16) dtype = MXS_DTYPE_F16;
    else TORCH_CHECK(false, "logits must be float32 or float16, got ", logits.scalar_type());
    TORCH_CHECK((flags & ~(int64_t)MXS_FLAG_SHARE_ROWS) == 0, "unknown flags ", flags);
    dtype |= (int)flags;

    check_dev(temperature, logits, "temperature", torch::kFloat32, B);
    check_dev(top_k, logits, "top_k", torch::kInt32, B);
    check_dev(top_p, logits, "top_p", torch::kFloat32, B);
    check_dev(penalty, logits, "penalty", torch::kFloat32, B);
    check_dev(hist_begin, logits, "hist_begin", torch::kInt32, B);
    check_dev(hist_end, logits, "hist_end", torch::kInt32, B);
    check_dev(hist_ids, logits, "hist_ids", torch::kInt32, -1);
    TORCH_CHECK(hist_ids.numel() > 0, "hist_ids must not be empty");
    if (uniforms) check_dev(*uniforms, logits, "uniforms", torch::kFloat32, B);
    check_dev(out_tokens, logits, "out_tokens", torch::kInt64, B);
    if (out_status) check_dev(*out_status, logits, "out_status", torch::kInt32, B);
    if (out_probs) check_dev(*out_probs, logits, "out_probs", torch::kFloat32, B * V);
    TORCH_CHECK(workspace.device() == logits.device() && workspace.is_contiguous() &&
                workspace.scalar_type() == torch::kUInt8, "workspace must be a uint8 tensor on the logits device");

    const c10::DeviceGuard guard(logits.device());
    auto stream = c10::hip::getCurrentHIPStream();
    int st = mxs_sample_ranges(logits.data_ptr(), dtype, (int)B, (int)V, logits.stride(0),
                               temperature.data_ptr<float>(), top_k.data_ptr<int32_t>(),
                               top_p.data_ptr<float>(), penalty.data_ptr<float>(),
                               hist_begin.data_ptr<int32_t>(), hist_end.data_ptr<int32_t>(),
                               hist_ids.data_ptr<int32_t>(), hist_ids.numel(),
                               (const float*)opt_ptr(uniforms), out_tokens.data_ptr<int64_t>(),
                               out_status ? out_status->data_ptr<int32_t>() : nullptr,
                               out_probs ? out_probs->data_ptr<float>() : nullptr,
                               workspace.data_ptr(), (size_t)workspace.numel(),
                               (mxs_stream_t)stream.stream());
    raise_status(st, "mxs_sample_ranges");
}

std::string version() { return mxs_version(); }

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m)
{
    m.doc() = "MI355X sampler chain: torch front end of the mxs_sampler C ABI";
    m.def("version", &version);
    m.def("workspace_bytes", &workspace_bytes, "workspace size for a [B, V] batch");
    m.def("sample", &sample, "sample one token per row (see mxs_sampler.h)",
          py::arg("logits"), py::arg("temperature"), py::arg("top_k"), py::arg("top_p"),
          py::arg("penalty"), py::arg("hist_offsets"), py::arg("hist_ids"), py::arg("uniforms"),
          py::arg("out_tokens"), py::arg("out_status"), py::arg("out_probs"), py::arg("workspace"),
          py::arg("flags") = 0);
    m.def("sample_head", &sample_head,
          "sample with the LM head's row maxima (see mxs_sample_head)",
          py::arg("logits"), py::arg("temperature"), py::arg("top_k"), py::arg("top_p"),
          py::arg("penalty"), py::arg("hist_offsets"), py::arg("hist_ids"), py::arg("uniforms"),
          py::arg("out_tokens"), py::arg("out_status"), py::arg("out_probs"), py::arg("row_best"),
          py::arg("workspace"), py::arg("flags") = 0);
    m.def("lm_head", &lm_head, "logits = hidden . weight^T with the rows' packed maxima (mxs_lm_head)",
          py::arg("hidden"), py::arg("weight"), py::arg("out_logits"), py::arg("out_best"));
    m.def("sample_ranges", &sample_ranges,
          "sample one token per row, histories as [begin, end) ranges of a device id buffer",
          py::arg("logits"), py::arg("temperature"), py::arg("top_k"), py::arg("top_p"),
          py::arg("penalty"), py::arg("hist_begin"), py::arg("hist_end"), py::arg("hist_ids"),
          py::arg("uniforms"), py::arg("out_tokens"), py::arg("out_status"), py::arg("out_probs"),
          py::arg("workspace"), py::arg("flags") = 0);
    m.attr("FLAG_SHARE_ROWS") = (int)MXS_FLAG_SHARE_ROWS;
}
