"""The benchmark's contract on the CPU: it refuses more than one GPU before
touching any device, and the profile figures it reports beside its own
timing (the rocprofv3 average and the PMC traffic of the dominant decode
kernel) parse from the committed summaries and agree with the kernel's
algorithmic bytes."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "5"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stdout + r.stderr


def test_bench_reads_the_committed_profile_figures():
    import bench
    from tinyminigo_amd import workloads as W

    wl = W.ONE_B
    # the gate/up GEMV's algorithmic bytes per launch: 2 * intermediate rows
    # of hidden BF16 weights, the activation and norm weights (f32) and the
    # SwiGLU output (f32)
    alg = 2 * wl.intermediate_size * wl.hidden_size * 2 + wl.hidden_size * 8 + wl.intermediate_size * 4
    assert alg == 50372608
    traffic, tree = bench.pmc_traffic("gemv_gateup_swiglu")
    assert tree and traffic is not None
    assert 1.0 <= traffic / alg < 1.05  # the weights read once
    us, tree = bench.rocprof_avg("gemv_gateup_swiglu")
    assert tree and us is not None
    # a launch cannot stream its bytes faster than the 8 TB/s peak
    assert alg / (us * 1e-6) / 1e9 < bench.HBM_PEAK_GBS
    assert bench.pmc_traffic("no_such_kernel") == (None, None)
    assert bench.rocprof_avg("no_such_kernel") == (None, None)


@pytest.mark.parametrize("weights", ["bf16", "i8"])
def test_traffic_summaries_exist(weights):
    import bench
    assert os.path.exists(bench.TRAFFIC_FILES[weights])
