"""bpd_qmatmul_q8_0_llamafile_noalloc_gpu: the llamafile entry with its Q8_0
activation rows in the library's fixed device scratch array instead of an
allocated workspace.  Called through the C ABI; its output must equal the
allocating entry point's bit for bit, on two calls in a row (the second with a
smaller input, so stale scratch contents from the first would show), and it
must refuse a size beyond the scratch array without launching anything."""
import numpy as np
import pytest

from bpd_substrate_amd import gpu, synth
from helpers import assert_bits_equal, to_np


def _run(name, W, X, mw, mt, K, dev):
    import torch

    out = torch.full((mt * mw,), float("nan"), device=dev)
    gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
    gpu.call(name, W, X, out, mw, mt, K)
    torch.cuda.synchronize()
    return to_np(out)


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [((300, 64, 4096), (77, 5, 1024)), ((14336, 4, 4096), (4096, 1, 14336))])
def test_noalloc_matches_allocating_entry_twice(dev, first, second):
    import torch

    for i, (mw, mt, K) in enumerate((first, second)):
        W = torch.from_numpy(synth.q8_0(mw, K, synth.key(60 + i, mw))).to(dev)
        X = torch.from_numpy(synth.normal_f32(mt * K, synth.key(61 + i, mt))).to(dev)
        want = _run("bpd_qmatmul_q8_0_llamafile_gpu", W, X, mw, mt, K, dev)
        got = _run("bpd_qmatmul_q8_0_llamafile_noalloc_gpu", W, X, mw, mt, K, dev)
        assert not np.isnan(want).any()
        assert_bits_equal(got, want, f"no-allocation llamafile call {i + 1} ({mw}x{mt}x{K})")


@pytest.mark.gpu
def test_noalloc_refuses_beyond_the_scratch_array(dev):
    import torch

    mw, K = 8, 4096
    mt = (8 << 20) // (K // 32 * 34) + 1          # one token more than 8 MiB of Q8_0 rows hold
    W = torch.zeros(mw * K // 32 * 34, dtype=torch.uint8, device=dev)
    X = torch.zeros(mt * K, dtype=torch.float32, device=dev)
    out = torch.full((mt * mw,), 7.0, device=dev)
    with pytest.raises(gpu.BpdqError) as e:
        gpu.call("bpd_qmatmul_q8_0_llamafile_noalloc_gpu", W, X, out, mw, mt, K)
    assert e.value.code == 7
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())                # nothing was launched


def test_noalloc_refusal_needs_no_gpu_call():
    # the size limit is checked before any HIP call: fake pointers, nothing launched
    L = gpu.lib()
    L.bpd_gpu_last_error()
    mt = (8 << 20) // (4096 // 32 * 34) + 1
    L.bpd_qmatmul_q8_0_llamafile_noalloc_gpu(0x1000, 0x2000, 0x3000, 8, mt, 4096)
    assert L.bpd_gpu_last_error() == 7
    assert "scratch" in L.bpd_gpu_last_error_message().decode()


@pytest.mark.gpu
def test_noalloc_inside_graph_capture(dev):
    """The entry exists for callers that cannot allocate.  Called eagerly on a stream
    the library has never seen (after one torch launch there, which sets up the
    runtime's own per-stream resources), it leaves the device's free memory
    unchanged (the allocating entry would create that stream's workspace); captured in a HIP graph,
    every replay, with eager work and synchronizations between them, gives the eager
    bits."""
    import torch

    mw, mt, K = 1000, 8, 4096
    W = torch.from_numpy(synth.q8_0(mw, K, synth.key(62, 1))).to(dev)
    X = torch.from_numpy(synth.normal_f32(mt * K, synth.key(62, 2))).to(dev)
    want = _run("bpd_qmatmul_q8_0_llamafile_gpu", W, X, mw, mt, K, dev)
    out = torch.zeros(mt * mw, device=dev)
    s0 = torch.cuda.Stream()
    with torch.cuda.stream(s0):
        out.add_(0.0)                  # the runtime's own resources for a new stream's first launch
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(dev)[0]
    gpu.lib().bpd_gpu_set_stream(s0.cuda_stream)
    gpu.call("bpd_qmatmul_q8_0_llamafile_noalloc_gpu", W, X, out, mw, mt, K)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free_before, "the no-allocation call changed the free device memory"
    assert_bits_equal(to_np(out), want, "eager call on a new stream")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gpu.lib().bpd_gpu_set_stream(s.cuda_stream)
        gpu.call("bpd_qmatmul_q8_0_llamafile_noalloc_gpu", W, X, out, mw, mt, K)
    gpu.lib().bpd_gpu_set_stream(None)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bits_equal(to_np(out), want, f"replay {rep}")


_FIRST_CALL_IN_CAPTURE = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from bpd_substrate_amd import gpu, synth
dev = torch.device("cuda:0")
mw, mt, K = 64, 2, 1024
W = torch.from_numpy(synth.q8_0(mw, K, synth.key(63, 1))).to(dev)
X = torch.from_numpy(synth.normal_f32(mt * K, synth.key(63, 2))).to(dev)
out = torch.zeros(mt * mw, device=dev)
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
torch.cuda.synchronize()
with torch.cuda.graph(g, stream=s):          # the library's first call in this process
    gpu.lib().bpd_gpu_set_stream(s.cuda_stream)
    gpu.call("bpd_qmatmul_q8_0_llamafile_noalloc_gpu", W, X, out, mw, mt, K)
gpu.lib().bpd_gpu_set_stream(None)
g.replay()
torch.cuda.synchronize()
got = out.cpu().numpy().view(np.uint32).copy()
ref = torch.zeros(mt * mw, device=dev)
gpu.call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, ref, mw, mt, K)
torch.cuda.synchronize()
assert np.array_equal(got, ref.cpu().numpy().view(np.uint32)), "replay differs from the eager call"
print("first call inside capture: ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_inside_capture():
    """In a fresh process whose first library call is made under graph capture, the
    per-device lookup of the scratch array's address happens inside the capture and
    must be accepted there."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root], capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
