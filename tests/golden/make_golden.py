#!/usr/bin/env python3
"""Write the golden vectors of tests/golden/ from the reference's own C code.

The reference functions are compiled unchanged from /root/reference/bench/*.c
into oracle/_ref/ (oracle/Makefile, target `ref`) and called here through
ctypes on seeded synthetic inputs.  Outputs:

  q4k.npz      bpd_dequant_q4k / bpd_qmatmul_q4k / bpd_qmm_q4k (bench/bpd_quant.c)
  q8_0.npz     bpd_quant_q8_0_cpu, bpd_dequant_q8_0_cpu, bpd_embed_lookup_q8_0_cpu,
               bpd_qdot_q8_0_q8_0_cpu, bpd_qmatmul_q8_0_cpu,
               bpd_qmatmul_q8_0_dispatch_cpu, bpd_qmatmul_q8_0_llamafile_cpu
               (bench/bpd_cpu.c, bench/bpd_gemm_q8_0_cpu.c), scalar (-O2) and
               AVX1 (-O2 -mavx -mssse3) builds
  hashes.json  SHA-256 of full-size synthetic inputs and of the reference's
               outputs at the BASELINE config sizes

Run from the repository root after `make -C oracle ref`:
    python tests/golden/make_golden.py
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from bpd_substrate_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
P, I = ctypes.c_void_p, ctypes.c_int


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bind(lib, name, args, res=None):
    f = getattr(lib, name)
    f.argtypes, f.restype = args, res
    return f


def refs():
    q, s, a = O.ref("quant"), O.ref("scalar"), O.ref("avx")
    if q is None or s is None or a is None:
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref` with /root/reference mounted")
    return q, s, a


def q8_0_blocks_random(n_blocks, key):
    """Q8_0 blocks with finite f16 scales and int8 values over the full [-128, 127]."""
    raw = synth.random_bytes(n_blocks * 34, key).reshape(n_blocks, 34)
    d = synth.q8_0(n_blocks, 32, key ^ 0x55)[np.arange(n_blocks)[:, None] * 34 + np.arange(2)]
    raw[:, 0:2] = d
    return raw.reshape(-1).copy()


def main():
    RQ, RS, RA = refs()
    deq = bind(RQ, "bpd_dequant_q4k", [P, P, I])
    mv = bind(RQ, "bpd_qmatmul_q4k", [P, P, P, I, I])
    qmm = bind(RQ, "bpd_qmm_q4k", [P, P, P, I, I, I])

    def r_deq(q):
        out = np.empty(q.size // 144 * 256, np.float32)
        deq(q.ctypes.data, out.ctypes.data, q.size // 144)
        return out

    # ---------------------------------------------------------------- Q4_K
    g = {}
    g["synth_q"] = synth.q4k(32, 256, synth.key(42, 0))
    g["synth_deq"] = r_deq(g["synth_q"])
    g["rand_q"] = synth.random_bytes(32 * 144, synth.key(7, 0))
    g["rand_deq"] = r_deq(g["rand_q"])
    M, K = 8, 512
    g["mm_w"] = synth.q4k(M, K, synth.key(42, 20))
    g["mm_x"] = synth.normal_f32(K, synth.key(42, 21))
    g["mm_y"] = np.empty(M, np.float32)
    mv(g["mm_w"].ctypes.data, g["mm_x"].ctypes.data, g["mm_y"].ctypes.data, M, K)
    g["qmm_A"] = synth.q4k(3, 256, synth.key(42, 22))
    g["qmm_B"] = synth.normal_f32(256 * 5, synth.key(42, 23))
    g["qmm_C"] = np.empty(15, np.float32)
    qmm(g["qmm_A"].ctypes.data, g["qmm_B"].ctypes.data, g["qmm_C"].ctypes.data, 3, 5, 256)
    np.savez_compressed(os.path.join(OUT, "q4k.npz"), **g)

    # ---------------------------------------------------------------- Q8_0
    h = {}
    quant = {k: bind(L, "bpd_quant_q8_0_cpu", [P, P, I]) for k, L in (("s", RS), ("a", RA))}
    x = synth.normal_f32(10 * 32, synth.key(42, 30))
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5      # x*id ties
    x[64:96] = 6.0e-5 * (np.arange(32) - 16)                # subnormal f16 scale
    x[96:128] = 9.0e6                                       # scale overflows f16 -> Inf
    x[128:160] = 0.0                                        # amax = 0
    x[160:192] = -0.0
    h["quant_x"] = x
    for k in ("s", "a"):
        y = np.empty(10 * 34, np.uint8)
        quant[k](x.ctypes.data, y.ctypes.data, x.size)
        h[f"quant_y_{k}"] = y
    h["deq_raw"] = q8_0_blocks_random(12, synth.key(42, 31))
    dq8 = bind(RS, "bpd_dequant_q8_0_cpu", [P, P, I])
    h["deq_out"] = np.empty(12 * 32, np.float32)
    dq8(h["deq_raw"].ctypes.data, h["deq_out"].ctypes.data, 12)
    emb = bind(RS, "bpd_embed_lookup_q8_0_cpu", [P, P, P, I, I])
    h["emb_table"] = q8_0_blocks_random(10 * 2, synth.key(42, 32))
    h["emb_ids"] = np.array([9, 0, 4, 4], np.int32)
    h["emb_out"] = np.empty(4 * 64, np.float32)
    emb(h["emb_table"].ctypes.data, h["emb_ids"].ctypes.data, h["emb_out"].ctypes.data, 4, 64)
    # one row-row dot with an odd block count (pair loop + tail)
    h["dot_w"] = q8_0_blocks_random(7, synth.key(42, 33))
    h["dot_act"] = q8_0_blocks_random(7, synth.key(42, 34))
    for k, L in (("s", RS), ("a", RA)):
        f = bind(L, "bpd_qdot_q8_0_q8_0_cpu", [P, P, I], ctypes.c_float)
        h[f"dot_{k}"] = np.array([f(h["dot_w"].ctypes.data, h["dot_act"].ctypes.data, 7)], np.float32)
    # dispatcher: 9 weight rows x 7 token rows, K = 128 (tiles 4+4+1 x 4+2+1)
    mw, mt, Kd = 9, 7, 128
    h["disp_W"] = q8_0_blocks_random(mw * Kd // 32, synth.key(42, 35))
    h["disp_X"] = q8_0_blocks_random(mt * Kd // 32, synth.key(42, 36))
    for k, L in (("s", RS), ("a", RA)):
        f = bind(L, "bpd_qmatmul_q8_0_dispatch_cpu", [P, P, P, I, I, I])
        out = np.empty(mw * mt, np.float32)
        f(h["disp_W"].ctypes.data, h["disp_X"].ctypes.data, out.ctypes.data, mw, mt, Kd)
        h[f"disp_{k}"] = out
    # llamafile entry (fp32 X) and bpd_qmatmul_q8_0_cpu
    mw2, mt2, K2 = 6, 3, 96
    h["lf_W"] = synth.q8_0(mw2, K2, synth.key(42, 37))
    h["lf_X"] = synth.normal_f32(mt2 * K2, synth.key(42, 38))
    for k, L in (("s", RS), ("a", RA)):
        f = bind(L, "bpd_qmatmul_q8_0_llamafile_cpu", [P, P, P, I, I, I])
        out = np.empty(mw2 * mt2, np.float32)
        f(h["lf_W"].ctypes.data, h["lf_X"].ctypes.data, out.ctypes.data, mw2, mt2, K2)
        h[f"lf_{k}"] = out
        f = bind(L, "bpd_qmatmul_q8_0_cpu", [P, P, P, I, I, I])
        out = np.empty(mt2 * mw2, np.float32)
        f(h["lf_W"].ctypes.data, h["lf_X"].ctypes.data, out.ctypes.data, mt2, mw2, K2)
        h[f"qm_{k}"] = out
    np.savez_compressed(os.path.join(OUT, "q8_0.npz"), **h)

    # ---------------------------------------------------------------- hashes
    H = {}
    w0 = synth.q4k(4096, 4096, synth.key(42, synth.STREAM["cfg0_w"]))
    H["input cfg0_w q4k 4096x4096"] = sha(w0)
    H["ref bpd_dequant_q4k cfg0"] = sha(r_deq(w0))
    x1 = synth.normal_f32(4096, synth.key(42, synth.STREAM["cfg1_x"]))
    H["input cfg1_x f32[4096]"] = sha(x1)
    y = np.empty(4096, np.float32)
    mv(w0.ctypes.data, x1.ctypes.data, y.ctypes.data, 4096, 4096)
    H["ref bpd_qmatmul_q4k cfg0_w . cfg1_x"] = sha(y)
    wm = synth.q4k(14336, 4096, synth.key(42, synth.STREAM["metric_w"]))
    H["input metric_w q4k 14336x4096"] = sha(wm)
    xm = synth.normal_f32(4096, synth.key(42, synth.STREAM["metric_x"]))
    H["input metric_x f32[4096]"] = sha(xm)
    for name, (rows, k, sw, sx) in {"up": (14336, 4096, "cfg2_up", "cfg2_x_up"),
                                    "down": (4096, 14336, "cfg2_down", "cfg2_x_down")}.items():
        W = synth.q8_0(rows, k, synth.key(42, synth.STREAM[sw]))
        X = synth.normal_f32(k, synth.key(42, synth.STREAM[sx]))
        H[f"input cfg2_{name} q8_0 {rows}x{k}"] = sha(W)
        H[f"input cfg2_x_{name} f32[{k}]"] = sha(X)
        Xq = np.empty(k // 32 * 34, np.uint8)
        quant["a"](X.ctypes.data, Xq.ctypes.data, k)
        H[f"ref bpd_quant_q8_0_cpu cfg2_x_{name}"] = sha(Xq)
        f = bind(RA, "bpd_qmatmul_q8_0_dispatch_cpu", [P, P, P, I, I, I])
        out = np.empty(rows, np.float32)
        f(W.ctypes.data, Xq.ctypes.data, out.ctypes.data, rows, 1, k)
        H[f"ref avx dispatch cfg2_{name}"] = sha(out)
    # cfg4: prefill, W as cfg2 up (14336 x 4096), X 512 x 4096 -> Q8_0, scalar build (order S);
    # the reference dispatcher is run on token ranges in parallel (rows of out are independent)
    import threading

    W = synth.q8_0(14336, 4096, synth.key(42, synth.STREAM["cfg2_up"]))
    X = synth.normal_f32(512 * 4096, synth.key(42, synth.STREAM["cfg4_x"]))
    H["input cfg4_x f32[512x4096]"] = sha(X)
    qs = bind(RS, "bpd_quant_q8_0_cpu", [P, P, I])
    Xq = np.empty(512 * 128 * 34, np.uint8)
    qs(X.ctypes.data, Xq.ctypes.data, X.size)
    H["ref bpd_quant_q8_0_cpu cfg4_x"] = sha(Xq)
    f = bind(RS, "bpd_qmatmul_q8_0_dispatch_cpu", [P, P, P, I, I, I])
    out = np.empty(512 * 14336, np.float32)
    nt = 16

    def part(i):
        t0, t1 = 512 * i // nt, 512 * (i + 1) // nt
        f(W.ctypes.data, Xq.ctypes.data + t0 * 128 * 34, out.ctypes.data + t0 * 14336 * 4, 14336, t1 - t0, 4096)

    ths = [threading.Thread(target=part, args=(i,)) for i in range(nt)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    H["ref scalar dispatch cfg4 512x14336x4096"] = sha(out)
    with open(os.path.join(OUT, "hashes.json"), "w") as fh:
        json.dump(H, fh, indent=1, sort_keys=True)
    print("wrote", os.listdir(OUT))


if __name__ == "__main__":
    main()
