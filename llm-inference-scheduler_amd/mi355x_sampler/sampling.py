"""Drop-in for mini_engine/sampling.py: logits -> token on an MI355X.

Same names, fields, defaults and call signature as the reference
(mini_engine/sampling.py:15-35), so mini_engine/generate.py:71 and
mini_engine/scheduler.py:275 can call it unchanged.  The chain runs as one
launch of the gfx950 kernels behind the mxs_sampler C ABI.

Documented differences from the reference:
  * the draw is an inverse CDF over the kept tokens (in sorted order) from one
    uniform u = torch.rand((), generator=generator), not torch.multinomial's
    exponential race over V draws; the distribution is the same, the realized
    token for a given seed is not, and the generator advances by one draw;
  * ties in the top-p sort go to the lowest index (the reference's torch.sort
    is unstable); the top-p cut and softmax use exact integer masses;
  * the caller's fp32 logits are not modified (the reference writes the
    penalized values back into them, sampling.py:36/45; nothing reads them
    afterwards at either call site).
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native
from .batch import ROW_OK, _normalize_history, device_temperature, raise_row_status


@dataclass
class SamplingParams:
    temperature: float = 0.7
    top_k: int = 0          # 0 = disabled
    top_p: float = 1.0      # 1.0 = disabled
    repetition_penalty: float = 1.0
    max_new_tokens: int = 256
    stop_token_ids: set = field(default_factory=set)
    seed: int | None = None

    @property
    def greedy(self) -> bool:
        return self.temperature == 0.0


class _RowBuffers:
    """Per-device buffers of the one-row call, made once: a pinned host
    block and its device copy (parameters, CSR offsets and the history ids),
    the device outputs and a pinned block they come back to, and the
    tensor views the extension takes (so a call makes no new tensors)."""

    def __init__(self, device: torch.device, n: int):
        self.n = n
        self.lock = threading.Lock()   # (one call at a time uses the blocks)
        self.pin_in = torch.empty(8 + n, dtype=torch.int32, pin_memory=True)
        self.host = self.pin_in.numpy()
        self.host_f = self.host.view(np.float32)
        self.dev_in = torch.empty(8 + n, dtype=torch.int32, device=device)
        f = self.dev_in.view(torch.float32)
        self.T, self.K, self.P, self.PEN, self.U = f[0:1], self.dev_in[1:2], f[2:3], f[3:4], f[4:5]
        self.off, self.ids = self.dev_in[5:7], self.dev_in[8:]
        self.dev_out = torch.empty(2, dtype=torch.int64, device=device)   # token, then the status word
        self.tokens = self.dev_out[0:1]
        self.status = self.dev_out[1:2].view(torch.int32)[0:1]
        self.pin_out = torch.empty(2, dtype=torch.int64, pin_memory=True)
        self.out = self.pin_out.numpy()


_row_buffers: dict = {}
_row_buffers_lock = threading.Lock()


def _buffers(device: torch.device, H: int) -> _RowBuffers:
    with _row_buffers_lock:
        b = _row_buffers.get(device.index)
        if b is None or b.n < max(H, 1):
            b = _RowBuffers(device, max(H, 1024))
            _row_buffers[device.index] = b
        return b


def sample(
    logits: torch.Tensor,  # [vocab]
    params: SamplingParams,
    generated_ids: list[int],
    generator: torch.Generator | None = None,
) -> int:
    """One token from a [vocab] row (mini_engine/sampling.py:30-69).

    Logits on the CPU are copied to the current GPU first (the copy crosses
    PCIe; keep logits on the device to avoid it).  float32 and float16 rows
    are read as they are; other dtypes are upcast to float32 first, as
    `logits.float()` does at sampling.py:36.  The parameters and history go
    over in one asynchronous copy from a pinned block, and the token and
    status come back in one: the call synchronizes once, as `.item()` does
    at sampling.py:69.
    """
    if logits.dim() != 1:
        raise ValueError(f"sample() takes one [vocab] row, got shape {tuple(logits.shape)}")
    x = logits
    if x.device.type != "cuda":
        x = x.to(torch.device("cuda", torch.cuda.current_device()))
    _native.require_gpu(x.device)
    if x.dtype not in (torch.float32, torch.float16):
        x = x.float()
    x = x.contiguous()
    V = x.shape[0]
    ext = _native.extension()

    hist = []
    if params.repetition_penalty != 1.0 and generated_ids:
        hist = _normalize_history(generated_ids, V)
    u = 0.0
    if not params.greedy:
        u = float(torch.rand((), generator=generator))

    H = len(hist)
    b = _buffers(x.device, H)
    with b.lock:
        return _sample_row(ext, x, b, params, hist, u)


def _sample_row(ext, x, b: _RowBuffers, params: SamplingParams, hist: list, u: float) -> int:
    H = len(hist)
    V = x.shape[0]
    h, hf = b.host, b.host_f
    hf[0] = device_temperature(params.temperature)
    tk = int(params.top_k)
    h[1] = tk if -2**31 <= tk < 2**31 else 2**31 - 1
    hf[2] = float(params.top_p)
    hf[3] = float(params.repetition_penalty)
    hf[4] = u
    h[5] = 0
    h[6] = H
    if H:
        h[8:8 + H] = hist
    stream = torch.cuda.current_stream(x.device)
    try:
        b.dev_in[:8 + H].copy_(b.pin_in[:8 + H], non_blocking=True)
        ws = _native.workspace(x.device, 1, V)
        ext.sample(x.unsqueeze(0), b.T, b.K, b.P, b.PEN, b.off, b.ids, b.U, b.tokens, b.status, None, ws)
        b.pin_out.copy_(b.dev_out, non_blocking=True)
    finally:
        stream.synchronize()   # (also before the pinned blocks may be written again)
    tok = int(b.out[0])
    st = int(b.out[1] & 0xFFFFFFFF)
    if st != ROW_OK:
        raise_row_status(st)
    return tok
