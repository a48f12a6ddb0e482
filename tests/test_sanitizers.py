"""The host C code under AddressSanitizer and UndefinedBehaviorSanitizer.

Builds the sanitized variants of the three native libraries -- the C oracle
(oracle/Makefile, target san), the synthetic-input generator and the host pass
of every csrc/*.hip file (the argument validation, error recording, workspace
table and launch selection of the C ABI) -- and runs the CPU tests that drive
them in a child process with clang's ASan runtime preloaded.  Any out-of-bounds
access, use after free or undefined operation (signed overflow, bad shift,
misaligned load, ...) aborts the child and fails this test.  CPU only: skipped
where a GPU is visible (the GPU tests cover the device side).
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# the CPU tests that exercise the three libraries
SUITES = ["tests/test_oracle_reference.py", "tests/test_oracle_math.py", "tests/test_oracle_q6k.py",
          "tests/test_oracle_pad64.py", "tests/test_oracle_llama.py", "tests/test_abi_host.py", "tests/test_gguf.py"]


def _gpu_visible():
    import torch
    return torch.cuda.device_count() > 0


@pytest.mark.skipif(not os.path.exists("/opt/rocm/llvm/bin/clang"), reason="needs ROCm's clang for the sanitizer runtime")
def test_host_code_under_asan_and_ubsan(tmp_path):
    if _gpu_visible():
        pytest.skip("the sanitized host build runs in the CPU suite, not next to a GPU")
    from bpd_substrate_amd import build as b
    hip, synth = b.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "san"], check=True)
    oracle = os.path.join(ROOT, "oracle", "_san", "liboracle.so")
    rt = b.asan_runtime()
    assert os.path.exists(rt), rt
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": rt,
        # the interpreter's own allocations are not this code's leaks
        "ASAN_OPTIONS": f"detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86:log_path={tmp_path}/asan",
        "UBSAN_OPTIONS": f"halt_on_error=1:print_stacktrace=1:exitcode=87:log_path={tmp_path}/ubsan",
        "BPDQ_HIP_LIB": hip, "BPDQ_SYNTH_LIB": synth, "BPDQ_ORACLE_LIB": oracle,
    })
    # the child must load exactly these builds
    probe = ("import ctypes; from bpd_substrate_amd import _native; from oracle import oracle as O; "
             "_native.load_hip(); _native.load_synth(); O.lib(); "
             "maps = open('/proc/self/maps').read(); "
             f"assert {hip!r} in maps and {synth!r} in maps and {oracle!r} in maps, 'sanitized builds not loaded'")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider", *SUITES],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    # each report: its first lines (the error and the innermost frames)
    reports = "".join("\n".join(open(os.path.join(tmp_path, f)).read().splitlines()[:24]) + "\n"
                      for f in sorted(os.listdir(tmp_path)) if f.startswith(("asan", "ubsan")))
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, f"sanitized run failed (exit {r.returncode}):\n{reports[-8000:]}\n{tail}"
    assert not reports, reports[-8000:]
    assert " passed" in r.stdout, tail
