"""Host check of the grouped backward schedule (csrc/gemm_sched.hpp):
tests/cpp/test_gemm_sched.cpp, built with g++ and run here (no GPU)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_schedule_partitions_units(tmp_path):
    exe = str(tmp_path / "test_gemm_sched")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-I", os.path.join(ROOT, "deepfuse_amd", "csrc"),
                    os.path.join(HERE, "cpp", "test_gemm_sched.cpp"), "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 failures" in res.stdout
