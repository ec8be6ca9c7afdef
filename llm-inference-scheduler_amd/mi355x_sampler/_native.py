"""Loads the in-tree native parts: the torch extension and the C-ABI library.

There is no CPU fallback: if the extension has not been built, or no GPU is
visible, the sampler raises instead of computing anything elsewhere.
"""

from __future__ import annotations

import glob
import importlib.machinery
import importlib.util
import os

import torch

LIBDIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(LIBDIR, "libmxs_sampler.so")

_ext = None


def extension():
    """The `_mxs_ext` torch extension (built by __graft_entry__.build())."""
    global _ext
    if _ext is None:
        found = sorted(glob.glob(os.path.join(LIBDIR, "_mxs_ext*.so")))
        if not found:
            raise ImportError(
                f"mi355x_sampler native extension not built (looked in {LIBDIR}); "
                "run `python __graft_entry__.py` or llm-inference-scheduler_amd/build.py")
        loader = importlib.machinery.ExtensionFileLoader("_mxs_ext", found[0])
        spec = importlib.util.spec_from_file_location("_mxs_ext", found[0], loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _ext = mod
    return _ext


def require_gpu(device: torch.device) -> None:
    if device.type != "cuda":
        raise RuntimeError(f"mi355x_sampler runs on a HIP device; got a tensor on {device}")
    if not torch.cuda.is_available():
        raise RuntimeError("mi355x_sampler needs a visible HIP GPU")


_workspaces: dict = {}


def workspace(device: torch.device, B: int, V: int) -> torch.Tensor:
    """A ready workspace for a [B, V] call on `device` and its current stream.

    Kernels leave the control area (per-row counters at the front) zeroed after
    each call, so consecutive calls with the same B reuse the workspace as is.
    A call with another B stores candidate lists where this B's counters lie,
    so the control area is zeroed again whenever B changes.  One workspace per
    (device, stream) keeps calls on different streams apart.
    """
    ext = extension()
    need = int(ext.workspace_bytes(B, V))
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ent = _workspaces.get(key)
    if ent is None or ent[0].numel() < need:
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=device)
        ext.workspace_init(ws)
        ent = [ws, B]
        _workspaces[key] = ent
    elif ent[1] != B:
        ext.workspace_init(ent[0][: int(ext.control_bytes(B))])
        ent[1] = B
    return ent[0]


def reset_workspaces() -> None:
    """Forget cached workspaces (e.g. after a failed launch left one dirty)."""
    _workspaces.clear()
