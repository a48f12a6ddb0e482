"""GGUF bytes straight into the GPU ABI: tensors written to a GGUF file, located
by bpd_substrate_amd.gguf, copied to the device unchanged and consumed by the
entry points; outputs compared with the oracle on the bytes read back from the
file."""
import numpy as np
import pytest

from bpd_substrate_amd import gguf, gpu, synth
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_gguf_tensors_feed_the_abi(dev, tmp_path):
    import torch

    M, K, V, E = 1024, 4096, 512, 256
    w = synth.q4k(M, K, synth.key(61, 1))
    emb = synth.q8_0(V, E, synth.key(61, 2))
    p = str(tmp_path / "model.gguf")
    gguf.write_gguf(p, [("general.architecture", gguf.T_STR, "llama"), ("llama.rope.freq_base", gguf.T_F32, 1e4),
                        ("general.quantization_version", gguf.T_U32, 3)],
                    [("token_embd.weight", (E, V), gguf.Q8_0, emb.tobytes()),
                     ("blk.0.ffn_gate.weight", (K, M), gguf.Q4_K, w.tobytes())])
    g = gguf.open_gguf(p)
    assert all(ok for _, ok, _ in gguf.report(p))
    t = g.tensor("blk.0.ffn_gate.weight")
    assert (t.row_len, t.n_rows) == (K, M)
    host_w = np.frombuffer(g.tensor_bytes(t.name), np.uint8).copy()
    wd = g.to_device(t.name, dev)
    x = synth.normal_f32(K, synth.key(61, 3))
    y = gpu.qmatmul_q4k_q8k_fused(wd, torch.from_numpy(x).to(dev), M, K)
    assert_bits_equal(to_np(y), O.qmatmul_q4k_q8k(host_w, O.quant_q8_k(x), M, K, 0, nthreads=8), "gguf Q4_K GEMV")
    deq = gpu.dequant_q4k(wd[: 64 * 144])
    assert_bits_equal(to_np(deq), O.dequant_q4k(host_w[: 64 * 144]), "gguf Q4_K dequant")

    e = g.tensor("token_embd.weight")
    ed = g.to_device(e.name, dev)
    ids = torch.tensor([0, 7, V - 1, 7], dtype=torch.int32, device=dev)
    out = gpu.embed_lookup_q8_0(ed, ids, E)
    host_e = np.frombuffer(g.tensor_bytes(e.name), np.uint8).copy()
    want = O.embed_lookup_q8_0(host_e, np.array([0, 7, V - 1, 7], np.int32), E)
    assert_bits_equal(to_np(out).ravel(), want.ravel(), "gguf Q8_0 embedding rows")
