"""The oracle and the product's host-side GGUF reader under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only): the oracle rebuilt with the sanitizers runs every entry
the tests use (tests/sanitize/oracle_check.py), and the GGUF reader, config and Q8 packing
(hobbylm_amd/csrc/hg_gguf.cpp, built for the host alone) read valid and malformed files
(tests/sanitize/gguf_check.cpp).  Any sanitizer report fails the test."""
import os
import shutil
import struct
import subprocess
import sys

import pytest

from hobbylm_amd import gguf_synth as gs

ROOT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _runtime():
    p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _malformed(tmp_path):
    good = open(gs.synth_path("tiny", 11, norm_jitter=0.1), "rb").read()
    files = {
        "magic": b"XXXX" + good[4:],
        "version": good[:4] + struct.pack("<I", 2) + good[8:],
        "truncated": good[:100],
        "truncated_data": good[: len(good) // 2],
        "empty": b"",
        "missing_key": good.replace(b"hobbylm.block_count", b"hobbylm.block_counX", 1),
        "bad_string_len": good[:24] + struct.pack("<Q", 1 << 60) + good[32:],
    }
    out = []
    for k, v in files.items():
        p = tmp_path / f"{k}.gguf"
        p.write_bytes(v)
        out.append(str(p))
    return out


def _check(r):
    text = r.stdout + r.stderr
    assert "AddressSanitizer" not in text and "runtime error" not in text, text[-4000:]
    assert r.returncode == 0, text[-4000:]


@pytest.mark.skipif(shutil.which("gcc") is None or _runtime() is None, reason="gcc with libasan")
def test_oracle_under_sanitizers(tmp_path):
    lib = tmp_path / "liboracle_san.so"
    src = os.path.join(ROOT, "oracle", "oracle.c")
    subprocess.run(["gcc", "-mavx2", "-mfma", "-mf16c", "-fno-fast-math", "-ffp-contract=off", "-fopenmp", "-fPIC",
                    "-std=gnu11", *SAN, "-shared", "-o", str(lib), src, "-lm"], check=True)
    env = dict(os.environ, ORACLE_LIB=str(lib), LD_PRELOAD=_runtime(), OMP_NUM_THREADS="4", **ENV)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "sanitize", "oracle_check.py"),
                        *_malformed(tmp_path)], capture_output=True, text=True, env=env, timeout=600)
    _check(r)
    assert r.stdout.strip().endswith("OK")


CLANG = "/opt/rocm/llvm/bin/clang++"   # (host C++ only: hg_gguf.cpp uses _Float16, which this g++ lacks)


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang++")
def test_gguf_reader_under_sanitizers(tmp_path):
    exe = tmp_path / "gguf_check"
    csrc = os.path.join(ROOT, "hobbylm_amd", "csrc")
    subprocess.run([CLANG, "-std=c++20", *SAN, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    os.path.join(ROOT, "tests", "sanitize", "gguf_check.cpp"), os.path.join(csrc, "hg_gguf.cpp"),
                    "-o", str(exe), "-lpthread"], check=True)
    files = [gs.synth_path("tiny", 11, norm_jitter=0.1), gs.synth_path("tiny", 31, norm_jitter=0.1, qtype="kquant"),
             *_malformed(tmp_path)]
    r = subprocess.run([str(exe), *files], capture_output=True, text=True, env=dict(os.environ, **ENV), timeout=600)
    _check(r)
    lines = r.stdout.strip().splitlines()
    assert len(lines) == len(files)
    rcs = [(int(l.split()[2]), int(l.split()[4]), int(l.split()[6])) for l in lines]
    assert rcs[0] == (0, 0, 0) and rcs[1] == (0, 0, 0)          # the valid files load whole
    assert all(rc != (0, 0, 0) for rc in rcs[2:]), lines        # every malformed one reports an error
