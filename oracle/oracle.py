"""ctypes front end of the CPU oracle (sampler_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, as the checker.  The product never imports it.

The oracle restates mini_engine/sampling.py:30-69 row by row with exact,
order-independent arithmetic (integer softmax masses, exact top-p and draw
thresholds); see the header of sampler_oracle.c for the definition.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmxs_oracle.so")

ROW_OK = 0
ROW_BAD_HISTORY = 1
ROW_BAD_PARAM = 2
ROW_NONFINITE = 3
ROW_EMPTY_NUCLEUS = 4
MASS_BITS = 44
MAX_V = 1 << 19


class OrcInfo(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int32),
        ("n_topk", ctypes.c_int32),
        ("n_kept", ctypes.c_int32),
        ("draw_pos", ctypes.c_int32),
        ("W", ctypes.c_uint64),
        ("W_kept", ctypes.c_uint64),
        ("T_mass", ctypes.c_uint64),
        ("D_mass", ctypes.c_uint64),
        ("m", ctypes.c_float),
        ("kth", ctypes.c_float),
        ("p_margin", ctypes.c_double),
        ("u_margin", ctypes.c_double),
    ]


INFO_DTYPE = np.dtype(
    [
        ("status", np.int32), ("n_topk", np.int32), ("n_kept", np.int32),
        ("draw_pos", np.int32), ("W", np.uint64), ("W_kept", np.uint64),
        ("T_mass", np.uint64), ("D_mass", np.uint64), ("m", np.float32),
        ("kth", np.float32), ("p_margin", np.float64), ("u_margin", np.float64),
    ]
)
assert INFO_DTYPE.itemsize == ctypes.sizeof(OrcInfo)

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        L.orc_sample.argtypes = [p, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                 p, p, p, p, p, p, p, p, p, p, p]
        L.orc_sample.restype = ctypes.c_int
        L.orc_mass.argtypes = [ctypes.c_float]
        L.orc_mass.restype = ctypes.c_uint64
        L.orc_ceil_mul.argtypes = [ctypes.c_float, ctypes.c_uint64]
        L.orc_ceil_mul.restype = ctypes.c_uint64
        L.orc_floor_mul.argtypes = [ctypes.c_float, ctypes.c_uint64]
        L.orc_floor_mul.restype = ctypes.c_uint64
        L.orc_vkey.argtypes = [ctypes.c_float]
        L.orc_vkey.restype = ctypes.c_uint32
        L.orc_clamp_uniform.argtypes = [ctypes.c_float]
        L.orc_clamp_uniform.restype = ctypes.c_float
        _lib = L
    return _lib


def mass(d: float) -> int:
    return int(lib().orc_mass(float(np.float32(d))))


def ceil_mul(p: float, W: int) -> int:
    return int(lib().orc_ceil_mul(float(np.float32(p)), int(W)))


def floor_mul(u: float, W: int) -> int:
    return int(lib().orc_floor_mul(float(np.float32(u)), int(W)))


def vkey(f: float) -> int:
    return int(lib().orc_vkey(float(np.float32(f))))


@dataclass
class OracleResult:
    tokens: np.ndarray        # int64[B], -1 on error rows
    status: np.ndarray        # int32[B]
    info: np.ndarray          # INFO_DTYPE[B]
    probs: np.ndarray | None  # float32[B, V] post-filter probabilities


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sample_rows(logits: np.ndarray, temperature, top_k, top_p, penalty,
                hist_offsets, hist_ids, uniforms, want_probs: bool = False) -> OracleResult:
    """Run the oracle over a [B, V] batch (float32 or float16 logits).

    History is CSR: row r owns hist_ids[hist_offsets[r]:hist_offsets[r+1]].
    """
    x = np.asarray(logits)
    if x.ndim != 2:
        raise ValueError("logits must be [B, V]")
    if x.dtype == np.float16:
        x = x.astype(np.float32)          # exact upcast (sampling.py:36)
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, V = x.shape
    T = np.ascontiguousarray(temperature, dtype=np.float32).reshape(B)
    K = np.ascontiguousarray(top_k, dtype=np.int32).reshape(B)
    P = np.ascontiguousarray(top_p, dtype=np.float32).reshape(B)
    R = np.ascontiguousarray(penalty, dtype=np.float32).reshape(B)
    off = np.ascontiguousarray(hist_offsets, dtype=np.int32).reshape(B + 1)
    ids = np.ascontiguousarray(hist_ids, dtype=np.int32).reshape(-1)
    if ids.size == 0:
        ids = np.zeros(1, dtype=np.int32)
    U = np.ascontiguousarray(uniforms, dtype=np.float32).reshape(B)
    tok = np.empty(B, dtype=np.int64)
    st = np.empty(B, dtype=np.int32)
    info = np.zeros(B, dtype=INFO_DTYPE)
    probs = np.empty((B, V), dtype=np.float32) if want_probs else None
    rc = lib().orc_sample(_ptr(x), B, V, V, _ptr(T), _ptr(K), _ptr(P), _ptr(R),
                          _ptr(off), _ptr(ids), _ptr(U), _ptr(tok), _ptr(probs),
                          _ptr(st), _ptr(info))
    if rc < 0:
        raise ValueError("oracle rejected the batch shape")
    return OracleResult(tok, st, info, probs)
