"""MI355X-native sampler chain (repetition penalty, greedy, temperature,
top-k, top-p, softmax, draw) for the reference engine's
mini_engine/sampling.py, on hand-written gfx950 HIP kernels.

  SamplingParams, sample     drop-in for mini_engine/sampling.py:15-69
  sample_batch               one launch for a [B, V] batch, per-row device params
  sample_requests            batch from per-request SamplingParams / histories
  HistoryStore               requests' generated ids kept on the device across steps
  sample_requests_resident   sample_requests reading the histories from a HistoryStore
  params_from_request        SamplingParams from a request body, checked (check_params)
  lm_head                    the model's LM head with the rows' maxima (greedy rows' tokens)
"""

from .batch import (MAX_VOCAB, ROW_BAD_HISTORY, ROW_BAD_PARAM, ROW_EMPTY_NUCLEUS,
                    ROW_NONFINITE, ROW_OK, HistoryStore, Sampler, pack_requests, pack_resident,
                    sample_batch, sample_batch_ranges, sample_requests, sample_requests_resident,
                    shares_rows)
from .head import best_token, lm_head
from .params import check_params, params_from_request
from .sampling import SamplingParams, sample

__all__ = [
    "SamplingParams", "sample", "sample_batch", "Sampler", "sample_requests", "pack_requests",
    "HistoryStore", "sample_batch_ranges", "sample_requests_resident", "pack_resident",
    "params_from_request", "check_params", "lm_head", "best_token", "shares_rows",
    "MAX_VOCAB", "ROW_OK", "ROW_BAD_HISTORY", "ROW_BAD_PARAM", "ROW_NONFINITE",
    "ROW_EMPTY_NUCLEUS",
]
