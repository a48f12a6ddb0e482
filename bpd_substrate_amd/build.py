"""Build the native libraries in-tree.

    python -m bpd_substrate_amd.build          # libbpdq_hip.so + libbpdq_synth.so

libbpdq_hip.so   hipcc --offload-arch=gfx950, one object per csrc/*.hip, then -shared
libbpdq_synth.so gcc, the deterministic input generator (csrc/synth.c)

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


def build_all(verbose=False):
    build_synth()
    build_hip(verbose=verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(HIP_LIB)
    print(SYNTH_LIB)
