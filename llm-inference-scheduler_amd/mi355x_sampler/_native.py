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
    """A workspace of at least mxs_workspace_bytes(B, V) bytes for `device`
    and its current stream (one per (device, stream), grown on demand),
    zero-filled when allocated: the small-batch launch keeps one counter per
    row in it, which every call returns to zero."""
    need = int(extension().workspace_bytes(B, V))
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws
