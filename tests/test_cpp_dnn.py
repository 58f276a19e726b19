"""The C++ drop-in (libdfdnn.so, namespace dnn) through its test runner
tests/cpp/dnn_tests, whose cases mirror the reference's GTest suites
tests/core/cuda_test.cu, tests/core/tensor_test.cu and
tests/layers/fully_connected_layer_test.cu, with fp8 expected values from
the CPU oracle."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
RUNNER = os.path.join(HERE, "cpp", "dnn_tests")

SUITES = ("HipTest", "TensorTest", "Fp8TensorTest", "FullyConnectedLayerTest", "AdamOptimizerTest",
          "ClipGradNormTest", "LayerNormLayerTest")


def _runner():
    if not os.path.exists(RUNNER):
        pytest.fail("tests/cpp/dnn_tests is not built (run __graft_entry__.build())")
    return RUNNER


def test_runner_lists_every_suite():
    out = subprocess.run([_runner(), "--list"], capture_output=True, text=True, timeout=60, check=True).stdout
    names = out.split()
    for suite in SUITES:
        assert any(n.startswith(suite + ".") for n in names), suite
    assert "FullyConnectedLayerTest.BackwardPass" in names


@pytest.mark.gpu
def test_cpp_suites():
    """All suites in one process of the runner; every case must pass."""
    print("running tests/cpp/dnn_tests (all suites)", flush=True)
    res = subprocess.run([_runner()], capture_output=True, text=True, timeout=110)
    print(res.stdout[-6000:])
    print(res.stderr[-2000:])
    assert res.returncode == 0, f"dnn_tests exit {res.returncode}"
    for suite in SUITES:
        assert f"[       OK ] {suite}." in res.stdout, suite
