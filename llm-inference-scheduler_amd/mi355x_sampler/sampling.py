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

from dataclasses import dataclass, field

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
    `logits.float()` does at sampling.py:36.
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
    buf = torch.empty(8 + max(H, 1), dtype=torch.int32)
    f = buf.view(torch.float32)
    f[0] = device_temperature(params.temperature)
    tk = int(params.top_k)
    buf[1] = tk if -2**31 <= tk < 2**31 else 2**31 - 1
    f[2] = float(params.top_p)
    f[3] = float(params.repetition_penalty)
    f[4] = u
    buf[5] = 0
    buf[6] = H
    if H:
        buf[8:8 + H] = torch.tensor(hist, dtype=torch.int32)
    d = buf.to(x.device)
    df = d.view(torch.float32)
    tokens = torch.empty(1, dtype=torch.int64, device=x.device)
    status = torch.empty(1, dtype=torch.int32, device=x.device)
    ws = _native.workspace(x.device, 1, V)
    ext.sample(x.unsqueeze(0), df[0:1], d[1:2], df[2:3], df[3:4],
               d[5:7], d[8:8 + H], df[4:5], tokens, status, None, ws)
    tok, st = torch.cat([tokens, status.to(torch.int64)]).tolist()   # one sync, as .item() at :69
    if st != ROW_OK:
        raise_row_status(st)
    return tok
