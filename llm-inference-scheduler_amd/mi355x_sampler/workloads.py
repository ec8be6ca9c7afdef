"""Seeded synthetic sampler workloads (the five benchmark shapes).

Every row draws from its own numpy PCG64 stream, ``default_rng([seed, row])``,
so row r of a batch does not depend on the batch size: the first rows of the
B=256 Zipf batch equal a B=8 batch built with the same seed.  Within a row the
draw order is fixed: per-row parameters, the uniform, the history ids, then the
logits.

Shapes (vocabulary V = 151,936, mini_engine/model/config.py:13):

  "single"  B=1, fp32 3*N(0,1); T=0.8, top_k=50, top_p=0.9, penalty=1.1 over
            64 history ids ~ U[0, V)
  "greedy"  B=256, fp32 3*N(0,1); temperature 0 (argmax), no penalty/history
  "peaked"  B=64, fp32 N(0,1) plus 12 at 5 distinct indices; T=0.7, top_k=50,
            top_p=0.9, penalty=1.1 over 512 ids (256 from the 5 peaked ids,
            256 ~ U[0, V), shuffled)
  "zipf"    B=256, fp32 -1.1*ln(rank) + 0.1*N(0,1) under a random permutation
            per row (computed in fp64, rounded to fp32); per row T ~ U[0.3,1.5],
            top_k ~ U{0..1000} (0 = off), top_p ~ U[0.5, 1.0),
            penalty ~ U[1.0, 1.3] over 1024 ids ~ U[0, V)
  "flat16"  B=1024, fp16 N(0,1); T=0.7, top_k=0, top_p=0.95, penalty=1.05
            over 2048 ids ~ U[0, V)
  "default" B=256, fp32 Zipf-shaped rows as "zipf", with the reference's
            default SamplingParams (mini_engine/sampling.py:16-19,
            server/worker.py:56-59): T=0.7, top_k=0 (off), top_p=1.0 (off),
            penalty 1.0, no history
  "zipf_k0" the "zipf" batch (same seed, rows and parameters) with top_k = 0
            (off) on every 32nd row, as the draw top_k ~ U{0..1000} gives
            some batches
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

VOCAB = 151936

# name -> (seed, default batch, logits dtype, history length)
SHAPES = {
    "single": (1001, 1, np.float32, 64),
    "greedy": (1002, 256, np.float32, 0),
    "peaked": (1003, 64, np.float32, 512),
    "zipf": (1004, 256, np.float32, 1024),
    "flat16": (1005, 1024, np.float16, 2048),
    "default": (1006, 256, np.float32, 0),
    "zipf_k0": (1004, 256, np.float32, 1024),
}


@dataclass
class Workload:
    name: str
    logits: np.ndarray            # [B, V] float32 or float16
    temperature: np.ndarray       # float32[B]
    top_k: np.ndarray             # int32[B]
    top_p: np.ndarray             # float32[B]
    penalty: np.ndarray           # float32[B]
    hist_offsets: np.ndarray      # int32[B+1]
    hist_ids: np.ndarray          # int32[N]
    uniforms: np.ndarray          # float32[B]
    meta: dict = field(default_factory=dict)

    @property
    def B(self) -> int:
        return self.logits.shape[0]

    @property
    def V(self) -> int:
        return self.logits.shape[1]

    def algorithmic_bytes(self) -> int:
        """Bytes one pass must move: logits once, history, 16 B of parameters,
        the uniform on stochastic rows and the int64 token out."""
        stochastic = int((self.temperature != 0).sum())
        return (self.logits.nbytes + 4 * self.hist_ids.size + 16 * self.B
                + 4 * stochastic + 8 * self.B)

    def take(self, rows) -> "Workload":
        """The given rows as a workload of their own (histories rebased)."""
        rows = np.asarray(rows, dtype=np.int64)
        hists = [self.hist_ids[self.hist_offsets[r]:self.hist_offsets[r + 1]] for r in rows]
        off = np.zeros(rows.size + 1, np.int32)
        off[1:] = np.cumsum([h.size for h in hists])
        ids = np.concatenate(hists).astype(np.int32) if hists else np.zeros(0, np.int32)
        return Workload(self.name, np.ascontiguousarray(self.logits[rows]), self.temperature[rows],
                        self.top_k[rows], self.top_p[rows], self.penalty[rows], off, ids,
                        self.uniforms[rows], dict(self.meta))

    def to_device(self, device):
        """Device tensors in sample_batch argument order."""
        import torch
        d = torch.device(device)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(d)
        ids = self.hist_ids if self.hist_ids.size else np.zeros(0, np.int32)
        return dict(logits=t(self.logits), temperature=t(self.temperature),
                    top_k=t(self.top_k), top_p=t(self.top_p), penalty=t(self.penalty),
                    hist_offsets=t(self.hist_offsets), hist_ids=t(ids),
                    uniforms=t(self.uniforms))


def _row(name, seed, r, V, H):
    rng = np.random.default_rng([seed, r])
    if name in ("zipf", "zipf_k0"):
        T = rng.uniform(0.3, 1.5)
        k = int(rng.integers(0, 1001))
        p = rng.uniform(0.5, 1.0)
        pen = rng.uniform(1.0, 1.3)
    elif name == "single":
        T, k, p, pen = 0.8, 50, 0.9, 1.1
    elif name == "greedy":
        T, k, p, pen = 0.0, 0, 1.0, 1.0
    elif name == "peaked":
        T, k, p, pen = 0.7, 50, 0.9, 1.1
    elif name == "flat16":
        T, k, p, pen = 0.7, 0, 0.95, 1.05
    elif name == "default":
        T, k, p, pen = 0.7, 0, 1.0, 1.0
    else:
        raise KeyError(name)
    if name == "zipf_k0" and r % 32 == 0:
        k = 0
    u = rng.random(dtype=np.float32) if T != 0.0 else np.float32(0.0)

    if name == "peaked":
        peaks = rng.choice(V, size=5, replace=False)
        hist = np.concatenate([rng.choice(peaks, size=H // 2),
                               rng.integers(0, V, size=H - H // 2)])
        rng.shuffle(hist)
        x = rng.standard_normal(V)
        x[peaks] += 12.0
        x = x.astype(np.float32)
    else:
        hist = rng.integers(0, V, size=H)
        if name in ("single", "greedy"):
            x = (3.0 * rng.standard_normal(V)).astype(np.float32)
        elif name in ("zipf", "zipf_k0", "default"):
            rank = rng.permutation(V) + 1
            x = (-1.1 * np.log(rank) + 0.1 * rng.standard_normal(V)).astype(np.float32)
        else:  # flat16
            x = rng.standard_normal(V).astype(np.float16)
    return x, np.float32(T), k, np.float32(p), np.float32(pen), np.float32(u), hist.astype(np.int32)


def make_workload(name: str, B: int | None = None, V: int = VOCAB) -> Workload:
    """Build a seeded workload; B defaults to the shape's benchmark batch."""
    seed, B0, dtype, H = SHAPES[name]
    B = B0 if B is None else B
    H = min(H, V)
    logits = np.empty((B, V), dtype=dtype)
    T = np.empty(B, np.float32)
    K = np.empty(B, np.int32)
    P = np.empty(B, np.float32)
    R = np.empty(B, np.float32)
    U = np.empty(B, np.float32)
    hists = []
    for r in range(B):
        x, T[r], K[r], P[r], R[r], U[r], h = _row(name, seed, r, V, H)
        logits[r] = x
        hists.append(h)
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum([h.size for h in hists])
    ids = np.concatenate(hists).astype(np.int32) if hists else np.zeros(0, np.int32)
    return Workload(name, logits, T, K, P, R, off, ids, U,
                    meta={"seed": seed, "history": H, "dtype": np.dtype(dtype).name})
