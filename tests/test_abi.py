"""The C-ABI library (libmxs_sampler.so) loads without a GPU, exports every
function include/mxs_sampler.h declares, and rejects bad arguments with the
header's status codes before touching the device.  No call here launches a
kernel: the invalid-argument paths return before any HIP call, and the
pointers passed are never dereferenced on the host.
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "mxs_sampler.h")
LIB = os.path.join(ROOT, "llm-inference-scheduler_amd", "mi355x_sampler", "_lib", "libmxs_sampler.so")

OK, INVALID, ALIGN, SMALL_WS, VOCAB, HIP, LDS_LIMIT, SCRATCH_LIMIT = range(8)
MAX_VOCAB = 262144


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(mxs_\w+)\s*\(", text, flags=re.M)))


def header_constants():
    text = open(HEADER).read()
    consts = {k: int(v) for k, v in re.findall(r"\b(MXS_\w+)\s*=\s*(\d+)", text)}
    consts.update({k: int(v, 0) for k, v in re.findall(r"#define\s+(MXS_\w+)\s+(0x[0-9a-fA-F]+|\d+)", text)})
    return consts


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run python __graft_entry__.py")
    L = ctypes.CDLL(LIB)
    L.mxs_version.restype = ctypes.c_char_p
    L.mxs_status_string.restype = ctypes.c_char_p
    L.mxs_status_string.argtypes = [ctypes.c_int]
    L.mxs_workspace_bytes.restype = ctypes.c_size_t
    L.mxs_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    p = ctypes.c_void_p
    L.mxs_sample.restype = ctypes.c_int
    L.mxs_sample.argtypes = [p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                             p, p, p, p, p, p, ctypes.c_int64, p, p, p, p, p, ctypes.c_size_t, p]
    L.mxs_sample_ranges.restype = ctypes.c_int
    L.mxs_sample_ranges.argtypes = [p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                    p, p, p, p, p, p, p, ctypes.c_int64, p, p, p, p, p,
                                    ctypes.c_size_t, p]
    L.mxs_sample_head.restype = ctypes.c_int
    L.mxs_sample_head.argtypes = [p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                  p, p, p, p, p, p, ctypes.c_int64, p, p, p, p, p, p, ctypes.c_size_t, p]
    L.mxs_lm_head.restype = ctypes.c_int
    L.mxs_lm_head.argtypes = [p, ctypes.c_int, ctypes.c_int, ctypes.c_int64, p, ctypes.c_int, ctypes.c_int64,
                              p, ctypes.c_int64, p, p]
    return L


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == ["mxs_lm_head", "mxs_sample", "mxs_sample_head", "mxs_sample_noalloc",
                                    "mxs_sample_ranges", "mxs_status_string", "mxs_version",
                                    "mxs_workspace_bytes"]


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_header_constants_match_the_python_layer():
    from mi355x_sampler import batch
    c = header_constants()
    assert c["MXS_OK"] == OK and c["MXS_ERR_INVALID_ARGUMENT"] == INVALID
    assert c["MXS_ERR_ALIGNMENT"] == ALIGN and c["MXS_ERR_WORKSPACE_TOO_SMALL"] == SMALL_WS
    assert c["MXS_ERR_VOCAB_TOO_LARGE"] == VOCAB and c["MXS_ERR_HIP"] == HIP
    assert c["MXS_ERR_LDS_LIMIT"] == LDS_LIMIT and c["MXS_ERR_SCRATCH_LIMIT"] == SCRATCH_LIMIT
    assert c["MXS_DTYPE_F32"] == 0 and c["MXS_DTYPE_F16"] == 1
    assert c["MXS_FLAG_SHARE_ROWS"] == 0x100
    assert c["MXS_MAX_VOCAB"] == MAX_VOCAB == batch.MAX_VOCAB
    assert (c["MXS_ROW_OK"], c["MXS_ROW_BAD_HISTORY"], c["MXS_ROW_BAD_PARAM"],
            c["MXS_ROW_NONFINITE"], c["MXS_ROW_EMPTY_NUCLEUS"]) == \
        (batch.ROW_OK, batch.ROW_BAD_HISTORY, batch.ROW_BAD_PARAM, batch.ROW_NONFINITE,
         batch.ROW_EMPTY_NUCLEUS)


def test_version_and_status_strings(lib):
    assert lib.mxs_version().decode().startswith("mxs-sampler")
    assert "gfx950" in lib.mxs_version().decode()
    texts = [lib.mxs_status_string(s).decode() for s in range(8)]
    assert len(set(texts)) == 8 and all(texts)
    assert lib.mxs_status_string(99).decode()


def test_noalloc_scratch_covers_every_valid_shape(lib):
    scratch = header_constants()["MXS_NOALLOC_SCRATCH_BYTES"]
    for B in (1, 2, 64, 65, 256, 1024, 4096):
        for V in (1, 1000, 151936, MAX_VOCAB):
            assert 0 < lib.mxs_workspace_bytes(B, V) <= scratch


def test_workspace_bytes(lib):
    assert lib.mxs_workspace_bytes(0, 100) == 0
    assert lib.mxs_workspace_bytes(-1, 100) == 0
    assert lib.mxs_workspace_bytes(4, 0) == 0
    assert lib.mxs_workspace_bytes(4, MAX_VOCAB + 1) == 0
    sizes = [lib.mxs_workspace_bytes(B, 151936) for B in (1, 2, 64, 256, 1024)]
    assert all(s > 0 and s % 256 == 0 for s in sizes)
    assert sizes == sorted(sizes)
    assert lib.mxs_workspace_bytes(1, MAX_VOCAB) > 0


# fake, never-dereferenced device addresses
A = 0x7F0000000000          # 256-aligned
P = ctypes.c_void_p


def call(lib, logits=A, dtype=0, B=4, V=1000, ld=1000, temperature=A, top_k=A, top_p=A,
         penalty=A, hist_offsets=None, hist_ids=None, n_hist_ids=0, uniforms=A, out_tokens=A,
         out_status=A, out_probs=None, workspace=A, workspace_bytes=None):
    if workspace_bytes is None:
        workspace_bytes = 0 if B <= 0 or V <= 0 or V > MAX_VOCAB else lib.mxs_workspace_bytes(B, V)
    return lib.mxs_sample(P(logits), dtype, B, V, ld, P(temperature), P(top_k), P(top_p),
                          P(penalty), P(hist_offsets), P(hist_ids), n_hist_ids, P(uniforms), P(out_tokens),
                          P(out_status), P(out_probs), P(workspace), workspace_bytes, None)


def test_sample_rejects_bad_arguments_before_launching(lib):
    assert call(lib, B=-1) == INVALID
    assert call(lib, V=0) == INVALID
    assert call(lib, V=MAX_VOCAB + 1, ld=MAX_VOCAB + 1) == VOCAB
    assert call(lib, dtype=2) == INVALID
    assert call(lib, dtype=0x100 | 2) == INVALID      # the sharing flag on an unknown dtype
    assert call(lib, dtype=0x200) == INVALID          # an unknown flag
    assert call(lib, logits=None) == INVALID
    assert call(lib, temperature=None) == INVALID
    assert call(lib, top_k=None) == INVALID
    assert call(lib, top_p=None) == INVALID
    assert call(lib, penalty=None) == INVALID
    assert call(lib, out_tokens=None) == INVALID
    assert call(lib, workspace=None) == INVALID
    assert call(lib, hist_offsets=A, hist_ids=None) == INVALID
    assert call(lib, hist_offsets=A, hist_ids=A, n_hist_ids=-1) == INVALID
    assert call(lib, ld=999) == INVALID
    assert call(lib, logits=A + 2) == ALIGN                  # f32 rows need 4-byte alignment
    assert call(lib, workspace=A + 64) == ALIGN
    assert call(lib, workspace_bytes=lib.mxs_workspace_bytes(4, 1000) - 1) == SMALL_WS


def call_ranges(lib, logits=A, dtype=0, B=4, V=1000, ld=1000, hist_begin=A, hist_end=A,
                hist_ids=A, n_hist_ids=16, out_tokens=A, workspace=A):
    ws = 0 if B <= 0 or V <= 0 or V > MAX_VOCAB else lib.mxs_workspace_bytes(B, V)
    return lib.mxs_sample_ranges(P(logits), dtype, B, V, ld, P(A), P(A), P(A), P(A),
                                 P(hist_begin), P(hist_end), P(hist_ids), n_hist_ids, P(A), P(out_tokens),
                                 P(A), P(None), P(workspace), ws, None)


def test_sample_ranges_rejects_bad_arguments_before_launching(lib):
    assert call_ranges(lib, hist_begin=A, hist_end=None) == INVALID   # begin and end go together
    assert call_ranges(lib, hist_begin=None, hist_end=A) == INVALID
    assert call_ranges(lib, hist_ids=None) == INVALID                 # ranges need an id buffer
    assert call_ranges(lib, n_hist_ids=-3) == INVALID
    assert call_ranges(lib, B=-1) == INVALID
    assert call_ranges(lib, V=MAX_VOCAB + 1, ld=MAX_VOCAB + 1) == VOCAB
    assert call_ranges(lib, logits=A + 2) == ALIGN
    assert call_ranges(lib, out_tokens=None) == INVALID
    assert call_ranges(lib, B=0, logits=None, out_tokens=None, workspace=None) == OK


def call_head(lib, hidden=A, B=4, D=896, ldh=896, weight=A, V=1000, ldw=896, logits=A, ldl=1000, best=A):
    return lib.mxs_lm_head(P(hidden), B, D, ldh, P(weight), V, ldw, P(logits), ldl, P(best), None)


def test_lm_head_rejects_bad_arguments_before_launching(lib):
    assert call_head(lib, B=-1) == INVALID
    assert call_head(lib, D=0) == INVALID
    assert call_head(lib, V=0) == INVALID
    assert call_head(lib, hidden=None) == INVALID
    assert call_head(lib, weight=None) == INVALID
    assert call_head(lib, logits=None) == INVALID
    assert call_head(lib, best=None) == INVALID
    assert call_head(lib, ldh=895) == INVALID         # strides cover a row
    assert call_head(lib, ldw=100) == INVALID
    assert call_head(lib, ldl=999) == INVALID
    assert call_head(lib, hidden=A + 4) == ALIGN        # rows are read as 16-byte vectors
    assert call_head(lib, weight=A + 8) == ALIGN
    assert call_head(lib, D=897, ldh=897, ldw=900) == ALIGN
    assert call_head(lib, D=897, ldh=900, ldw=898) == ALIGN
    assert call_head(lib, best=A + 4) == ALIGN
    assert call_head(lib, logits=A + 2) == ALIGN
    assert call_head(lib, B=0, hidden=None, weight=None, logits=None, best=None) == OK


def test_sample_head_checks_as_sample_does(lib):
    def ch(**kw):
        a = dict(logits=A, B=4, V=1000, ld=1000, out_tokens=A, workspace=A)
        a.update(kw)
        ws = lib.mxs_workspace_bytes(4, 1000)
        return lib.mxs_sample_head(P(a["logits"]), 0, a["B"], a["V"], a["ld"], P(A), P(A), P(A), P(A),
                                   P(None), P(None), 0, P(A), P(a["out_tokens"]), P(A), P(None), P(A),
                                   P(a["workspace"]), ws, None)
    assert ch(B=-1) == INVALID
    assert ch(ld=999) == INVALID
    assert ch(logits=A + 2) == ALIGN
    assert ch(out_tokens=None) == INVALID
    assert ch(workspace=None) == INVALID
    assert ch(B=0, logits=None, out_tokens=None, workspace=None) == OK


def test_empty_batch_is_a_no_op(lib):
    # B == 0 returns before looking at any pointer
    assert call(lib, B=0, logits=None, temperature=None, out_tokens=None, workspace=None) == OK


def test_torch_extension_loads_and_agrees(lib):
    from mi355x_sampler import _native
    ext = _native.extension()
    assert ext.version() == lib.mxs_version().decode()
    for B, V in [(1, 151936), (256, 151936), (1024, 151936), (3, 4099)]:
        assert ext.workspace_bytes(B, V) == lib.mxs_workspace_bytes(B, V)
