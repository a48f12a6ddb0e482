"""Build the native libraries in-tree.

    python -m bpd_substrate_amd.build             # libbpdq_hip.so + libbpdq_synth.so
    python -m bpd_substrate_amd.build --sanitize  # _san/: host code under ASan + UBSan

libbpdq_hip.so   hipcc --offload-arch=gfx950, one object per csrc/*.hip, then -shared
libbpdq_synth.so gcc, the deterministic input generator (csrc/synth.c)

The sanitized variants (_san/libbpdq_hip.so, _san/libbpdq_synth.so) are for the
CPU test suite: the host pass of every HIP source is compiled with Address-
Sanitizer and UndefinedBehaviorSanitizer (the device code is the usual one and
is not instrumented), and synth.c with clang under the same runtime, so one
process can load both next to the sanitized oracle (oracle/Makefile, target
san).

The built files stay next to this module so that they travel with the source
tree to the GPU host; nothing is installed.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_obj")
HIP_LIB = os.path.join(PKG, "libbpdq_hip.so")
SYNTH_LIB = os.path.join(PKG, "libbpdq_synth.so")

ARCH = os.environ.get("BPDQ_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the parity kernels must execute the fp32 operations as
# written (HIP clang contracts a*b+c into FMA by default).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in generated code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the prefill epilogue reads every one with the VALU
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # kernel arguments preloaded into SGPRs at wave launch (gfx950), so a wave's first
    # loads do not wait for scalar loads of its arguments (the code object keeps a
    # prologue that loads them for firmware without preloading).  Measured on the metric
    # GEMV: 6.93 -> 6.68 us per launch, same bits.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def hip_sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_hip(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    srcs = hip_sources()
    objs = [os.path.join(OBJ, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]
        for f in futs:
            out = f.result()
            if verbose and out.strip():
                print(out)
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_synth():
    tmp = SYNTH_LIB + ".tmp"
    _run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-Wall", "-o", tmp,
          os.path.join(CSRC, "synth.c"), "-lm", "-lpthread"])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


SAN_DIR = os.path.join(PKG, "_san")
CLANG = os.environ.get("BPDQ_CLANG", "/opt/rocm/llvm/bin/clang")
# each -fsanitize option goes to the host pass only
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
SAN_C = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-shared-libsan"]


def asan_runtime():
    """The clang ASan runtime the sanitized libraries need preloaded (LD_PRELOAD)."""
    return _run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"]).strip()


def build_sanitized():
    """_san/libbpdq_hip.so (the host pass of every csrc/*.hip under ASan + UBSan)
    and _san/libbpdq_synth.so, with clang's shared sanitizer runtime."""
    obj = os.path.join(SAN_DIR, "obj")
    os.makedirs(obj, exist_ok=True)
    srcs = hip_sources()
    objs = [os.path.join(obj, os.path.basename(s)[:-4] + ".o") for s in srcs]
    base = [HIPCC, *HIP_FLAGS, *SAN_HOST, "-g"]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))) as ex:
        for f in [ex.submit(_run, [*base, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]:
            f.result()
    hip = os.path.join(SAN_DIR, "libbpdq_hip.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *SAN_HOST, "-Xarch_host", "-shared-libsan",
          "-o", hip, *objs])
    synth = os.path.join(SAN_DIR, "libbpdq_synth.so")
    _run([CLANG, "-O1", "-g", "-ffp-contract=off", "-fPIC", "-shared", *SAN_C, "-o", synth,
          os.path.join(CSRC, "synth.c"), "-lm", "-lpthread"])
    return hip, synth


def build_all(verbose=False):
    build_synth()
    build_hip(verbose=verbose)


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(*build_sanitized(), sep="\n")
    else:
        build_all(verbose="-v" in sys.argv)
        print(HIP_LIB)
        print(SYNTH_LIB)
