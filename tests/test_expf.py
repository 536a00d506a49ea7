"""hg_expf (the device exp of the exact paths) equals the host C library's expf on all
2^32 binary32 inputs.  Rust's f32::exp calls that expf, so this pins the exp used by the
reference's softmax (ops.rs:121), sigmoid (ops.rs:76) and silu (ops.rs:81)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.slow
def test_expf_matches_libm_exhaustively(tmp_path):
    exe = tmp_path / "expf_exhaustive"
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c++20",
                    "-I", os.path.join(ROOT, "hobbylm_amd", "csrc"),
                    os.path.join(ROOT, "tests", "expf_exhaustive.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["2", "0"], out
