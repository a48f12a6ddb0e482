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
