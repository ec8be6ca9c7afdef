"""The device-resident history (HistoryStore) and its packing, on the CPU:
slot layout, appends, capacity and index rules, and that pack_resident hands
the kernel the same rows and the same uniforms as pack_requests does from the
requests' Python lists (mini_engine/scheduler.py:43, 275-276).
"""

import pytest
import torch

from mi355x_sampler import SamplingParams
from mi355x_sampler.batch import HistoryStore, pack_requests, pack_resident


def test_slots_own_fixed_ranges():
    s = HistoryStore(slots=3, max_len=5, device="cpu")
    assert s.ranges([0, 1, 2]) == ([0, 5, 10], [0, 5, 10])
    s.reset(1, [4, 7])
    s.append([2, 1], torch.tensor([9, 8]))
    s.append([1], [6])
    assert s.history(1) == [4, 7, 8, 6] and s.history(2) == [9] and s.history(0) == []
    assert s.ranges([2, 1]) == ([10, 5], [11, 9])
    assert s.ids.dtype == torch.int32


def test_reset_normalizes_like_the_reference_and_clears():
    s = HistoryStore(2, 4, "cpu")
    s.reset(0, [1, -1], V=10)          # sampling.py:39-40 indexing rules
    assert s.history(0) == [1, 9]
    with pytest.raises(IndexError):
        s.reset(0, [10], V=10)
    s.reset(0)
    assert s.history(0) == [] and s.ranges([0]) == ([0], [0])


def test_capacity_and_argument_errors():
    s = HistoryStore(2, 2, "cpu")
    s.append([0], [1])
    s.append([0], [2])
    with pytest.raises(ValueError):
        s.append([0], [3])             # full
    with pytest.raises(ValueError):
        s.append([1, 1], [3, 4])       # a slot twice in one step
    with pytest.raises(ValueError):
        s.append([1], [3, 4])          # token count
    with pytest.raises(IndexError):
        s.append([2], [3])
    with pytest.raises(ValueError):
        s.reset(1, [1, 2, 3])
    with pytest.raises(ValueError):
        HistoryStore(0, 4, "cpu")
    assert s.history(1) == []          # failed appends change nothing


def test_pack_resident_matches_pack_requests():
    V = 1000
    params = [SamplingParams(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1),
              SamplingParams(temperature=0.0),
              SamplingParams(temperature=1.2, top_k=0, top_p=0.5, repetition_penalty=1.3)]
    hists = [[5, 6, 5], [1], [999, 0]]
    slots = [2, 0, 1]
    s = HistoryStore(3, 8, "cpu")
    for slot, h in zip(slots, hists):
        s.reset(slot, h)
    g1 = [torch.Generator().manual_seed(7 + i) for i in range(3)]
    g2 = [torch.Generator().manual_seed(7 + i) for i in range(3)]
    a = pack_requests(params, hists, V, "cpu", g1)
    b = pack_resident(params, s, slots, "cpu", g2)
    for k in ("temperature", "top_k", "top_p", "penalty", "uniforms"):
        assert torch.equal(a[k], b[k]), k
    off = a["hist_offsets"].tolist()
    for r in range(3):
        want = a["hist_ids"][off[r]:off[r + 1]].tolist()
        got = s.ids[int(b["hist_begin"][r]):int(b["hist_end"][r])].tolist()
        if params[r].repetition_penalty != 1.0:
            assert got == want
        else:
            assert want == []          # pack_requests drops a history the penalty ignores
    with pytest.raises(ValueError):
        pack_resident(params, s, [0, 1], "cpu")
