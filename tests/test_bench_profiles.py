"""bench.py's roofline.traffic comes from the committed rocprofv3 summaries
in profiles/: the HBM byte counters and, from the trace summary of the same
build, the kernel's average duration, against which the bench judges the
counters stale (live kernel time more than 10 % away)."""

import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("workload,B", [("zipf", 256), ("zipf_k0", 256), ("default", 256), ("flat16", 1024),
                                        ("greedy", 256)])
def test_committed_profiles_parse(workload, B):
    traffic, prof_us = load_bench().load_traffic(workload, B)
    assert traffic is not None and traffic > 100_000_000
    assert prof_us is not None and 5.0 < prof_us < 1000.0


def test_missing_profile():
    assert load_bench().load_traffic("no_such_workload", 3) == (None, None)
