"""bench.py's measurement plumbing that needs no GPU: the stage kernels it prices against the committed rocprofv3
summaries must be the kernels those summaries name (a renamed kernel template would otherwise turn the bench line's
`traffic` and counter fields into null without an error)."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def stage_kernels(bench, scatter, bits=4):
    stages = {**bench.STAGE_KERNELS, **bench.DOWN_STAGE_KERNELS[scatter]}
    return {st: [k.format(bits=bits) for k in ks] for st, ks in stages.items()}


@pytest.mark.parametrize("scatter", ["combine", "atomic"])
def test_stage_kernels_are_in_the_traffic_summary(bench, scatter):
    per = bench.profile_json("grouped_prefill_headline_traffic")["bytes_per_launch"]
    for st, ks in stage_kernels(bench, scatter).items():
        for k in ks:
            assert k in per, (st, k)
        assert bench.traffic_from_profiles("headline", ks) > 0


@pytest.mark.parametrize("scatter", ["combine", "atomic"])
def test_gemm_stage_kernels_are_in_the_counter_summary(bench, scatter):
    kernels = bench.profile_json("grouped_prefill_headline_sq_counters")["kernels"]
    for st, ks in stage_kernels(bench, scatter).items():
        if not st.startswith("gemm"):
            continue
        for k in ks:
            assert k in kernels, (st, k)
        busy = bench.mfma_busy_from_profiles("headline", ks)
        assert busy is not None and 0 < busy["mfma_busy"] < 1 and 0 < busy["valu_busy"] < 1.5


def test_stage_kernels_are_in_the_kernel_trace(bench):
    kernels = bench.profile_json("grouped_prefill_headline_ktrace")["kernels"]
    for st, ks in stage_kernels(bench, "combine").items():
        for k in ks:
            assert k in kernels, (st, k)
