#!/usr/bin/env python3
"""Benchmark of the MI355X quantized path at the headline metric shape (Q4_K x Q8_K, 14336x4096).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one Q4_K x Q8_K GEMV at M=14336, K=4096 (the metric workload) with
the weight, the Q8_K activation and the output already resident in HBM.  The
weight rotates over distinct copies so the 256 MB MALL cannot serve it: at
least 16 (> 512 MB), and for eager regions K + 8, so that the K timed launches
read K different copies and the 8 untimed warm-up launches before them read 8
others (264 MB, which also push the previous region's copies out).  The K timed
launches go back to back on one stream behind a GPU spin (so the host has
queued them before the start event runs): as eager launches after the warm-up
launches for K <= 64 (the driver's --steps 20), as one HIP graph for longer
regions.  HIP events on that stream
bracket the K launches, so the host's launch rate cannot hide or inflate
kernel time; the median over 7 timed regions is kept.  `value` and
`roofline.achieved` are the algorithmic bytes of one GEMV divided by that
median / K.  The same method times, on the same rotating copies, a plain
streaming read of the weight's bytes (the single-launch HBM read floor of this
size on this device), the cfg0 dequant, the cfg1 GEMV and the cfg2 Q8_0 GEMVs.
Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
M, K = 14336, 4096
W_BYTES = M * (K // 256) * 144                    # 33,030,144
X_BYTES = (K // 256) * 292                        # 4,672
Y_BYTES = M * 4                                   # 57,344
ALG_BYTES = W_BYTES + X_BYTES + Y_BYTES           # 33,092,160 per GEMV
DQ_BLOCKS = 4096 * 4096 // 256                    # cfg0: 65,536 Q4_K blocks
DQ_BYTES = DQ_BLOCKS * 144 + DQ_BLOCKS * 256 * 4  # 76,546,048 per dequant
Q80_SHAPES = {"up": (14336, 4096), "down": (4096, 14336)}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="metric GEMV and its read floor only")
    ap.add_argument("--cpu-runs", type=int, default=10)
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 32-layer, 512-token prefill forward (for profiling); prints its JSON")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Timer:
    """Time K back-to-back library launches on one stream.

    Short regions (K <= EAGER_MAX, as the driver's --steps 20) are timed as eager
    launches: a GPU spin and a few untimed warm-up launches go first on the same
    stream, so the host has queued all K launches before the start event runs and the
    GPU goes straight from warm-up into the timed launches.  Longer regions are one
    HIP graph of the K launches, replayed after the same spin (a graph replay carries
    a fixed ~8 us of its own on this GPU, which a 20-launch region would count as
    0.4 us per launch; eager launches carry a smaller per-launch gap instead).  HIP
    events on the stream bracket the K launches; the median over `repeats` timed
    regions is kept."""

    SPIN_CYCLES = 1_000_000  # ~0.4 ms at the MI355X shader clock: covers the host's queueing
    EAGER_MAX = 64

    def __init__(self, torch, lib, stream):
        self.torch, self.lib, self.stream = torch, lib, stream
        try:
            with torch.cuda.stream(stream):
                torch.cuda._sleep(1000)
            torch.cuda.synchronize()
            self.spin = True
        except Exception:  # no spin kernel in this torch build: time without the pre-roll
            self.spin = False

    def _region(self, pre, body):
        torch = self.torch
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            self.lib.bpd_gpu_set_stream(self.stream.cuda_stream)
            if self.spin:
                torch.cuda._sleep(self.SPIN_CYCLES)
            pre()
            s.record(self.stream)
            body()
            e.record(self.stream)
        e.synchronize()
        return s.elapsed_time(e)

    def us_per_launch(self, launches, repeats=7, graph=None, warm=None):
        """graph: None picks by K; True always captures (for "launches" that are whole
        decode steps of hundreds of kernels, which the host could not queue ahead).
        warm: the eager regions' untimed warm-up launches (default: the last 4 timed
        ones).  Launches that rotate weight copies pass launches of copies that the
        first timed launches do not read, so that no timed launch finds its weights
        in the MALL from the warm-up."""
        torch = self.torch
        if not graph and len(launches) <= self.EAGER_MAX:
            warm = warm if warm is not None else launches[-min(4, len(launches)):]

            def run_all(fs):
                for fn in fs:
                    fn()

            self._region(lambda: None, lambda: run_all(launches))  # first use: warms caches and clocks
            times = [self._region(lambda: run_all(warm), lambda: run_all(launches)) for _ in range(repeats)]
            return float(np.median(times)) * 1e3 / len(launches)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            with torch.cuda.graph(g, stream=self.stream):
                self.lib.bpd_gpu_set_stream(self.stream.cuda_stream)
                for fn in launches:
                    fn()
            self.lib.bpd_gpu_set_stream(self.stream.cuda_stream)
        self._region(lambda: None, g.replay)  # the first replay warms the graph
        times = [self._region(lambda: None, g.replay) for _ in range(repeats)]
        del g
        return float(np.median(times)) * 1e3 / len(launches)


# ---------------------------------------------------------------- CPU baseline

def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _pinned_parallel(n_items, nthreads, work):
    """Run work(i0, i1) over nthreads disjoint ranges of [0, n_items), each thread pinned
    to one CPU of this process's affinity set (ctypes releases the GIL during the C call)."""
    import threading

    cpus = sorted(os.sched_getaffinity(0))
    per = -(-n_items // nthreads)

    def part(t):
        try:
            os.sched_setaffinity(0, {cpus[t % len(cpus)]})  # this thread only (Linux)
        except OSError:
            pass
        i0, i1 = t * per, min(n_items, (t + 1) * per)
        if i1 > i0:
            work(i0, i1)

    if nthreads == 1:
        part(0)
        return
    ths = [threading.Thread(target=part, args=(t,)) for t in range(nthreads)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()


def _median_ms(run, runs):
    run()  # warm
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e3


def cpu_baseline(w_host, x_host, runs=10):
    """The CPU baseline: the reference C of the path on this host's cores, 1 core
    and all cores (a pinned thread per core over disjoint rows / blocks, which leaves
    every output's bits unchanged), median of `runs` runs per leg, full config sizes.
    Legs: cfg0 bpd_dequant_q4k and the metric-shape bpd_qmatmul_q4k (bench/bpd_quant.c,
    -O2); cfg2 bpd_quant_q8_0_cpu + bpd_qmatmul_q8_0_dispatch_cpu (bench/bpd_cpu.c +
    bench/bpd_gemm_q8_0_cpu.c, -O2 -mavx -mssse3); and this build's own Q4_K x Q8_K C
    oracle at the metric shape (no reference C exists for it).  Returns the result
    object (its value: the metric-shape bpd_qmatmul_q4k on all cores) and that leg's
    output for the GPU parity check."""
    import ctypes

    from bpd_substrate_amd import synth
    from oracle import oracle as O

    P, I = ctypes.c_void_p, ctypes.c_int
    allc = max(1, min(16, len(os.sched_getaffinity(0))))  # the GPU box's CPU share is 16
    RQ, RA = O.ref("quant"), O.ref("avx")
    kind = "reference" if RQ is not None else "port"
    if RQ is not None:
        dq, mm = RQ.bpd_dequant_q4k, RQ.bpd_qmatmul_q4k
        dq.argtypes, mm.argtypes = [P, P, I], [P, P, P, I, I]
    else:  # the in-repo restatement, pinned bit-identical to it
        dq, mm = O.lib().bpdq_o_dequant_q4k, O.lib().bpdq_o_qmatmul_q4k
    legs = {}

    def leg(name, run_1, run_n, work_bytes, extra):
        r = {"1_core_ms": round(_median_ms(run_1, runs), 3), f"{allc}_cores_ms": round(_median_ms(run_n, runs), 3)}
        r.update({"1_core_gb_s": round(work_bytes / r["1_core_ms"] / 1e6, 3),
                  f"{allc}_cores_gb_s": round(work_bytes / r[f"{allc}_cores_ms"] / 1e6, 3)})
        r.update(extra)
        legs[name] = r
        return r

    # metric shape, reference order, fp32 x
    y = np.empty(M, np.float32)
    row_b = (K // 256) * 144
    mm_work = lambda r0, r1: mm(w_host.ctypes.data + r0 * row_b, x_host.ctypes.data, y.ctypes.data + 4 * r0,
                                r1 - r0, K)
    m = leg("metric_bpd_qmatmul_q4k_14336x4096", lambda: mm_work(0, M),
            lambda: _pinned_parallel(M, allc, mm_work), W_BYTES + K * 4 + Y_BYTES,
            {"ref": "bench/bpd_quant.c:88-109", "flags": "-O2", "bytes": "W 33,030,144 + fp32 x + y"})
    # cfg0 dequant
    q0 = synth.q4k(DQ_BLOCKS, 256, synth.key(42, synth.STREAM["cfg0_w"]))
    o0 = np.empty(DQ_BLOCKS * 256, np.float32)
    dq_work = lambda b0, b1: dq(q0.ctypes.data + b0 * 144, o0.ctypes.data + b0 * 1024, b1 - b0)
    r = leg("cfg0_bpd_dequant_q4k_4096x4096", lambda: dq_work(0, DQ_BLOCKS),
            lambda: _pinned_parallel(DQ_BLOCKS, allc, dq_work), DQ_BYTES,
            {"ref": "bench/bpd_quant.c:41-81", "flags": "-O2", "bytes": "76,546,048 (144 B in + 1 KiB out per block)"})
    for c in ("1_core", f"{allc}_cores"):
        r[f"{c}_gelem_s"] = round(DQ_BLOCKS * 256 / r[f"{c}_ms"] / 1e6, 3)
    del q0, o0
    # cfg2: quantize x, then the AVX1 build's dispatcher (tile order T)
    if RA is not None:
        qz, dp = RA.bpd_quant_q8_0_cpu, RA.bpd_qmatmul_q8_0_dispatch_cpu
        qz.argtypes, dp.argtypes = [P, P, I], [P, P, P, I, I, I]
        for name, (rows, k) in Q80_SHAPES.items():
            W = synth.q8_0(rows, k, synth.key(42, synth.STREAM[f"cfg2_{name}"]))
            X = synth.normal_f32(k, synth.key(42, synth.STREAM[f"cfg2_x_{name}"]))
            Xq = np.empty(k // 32 * 34, np.uint8)
            out = np.empty(rows, np.float32)
            bpr = k // 32 * 34
            d_work = lambda r0, r1, W=W, Xq=Xq, out=out, k=k, bpr=bpr: dp(
                W.ctypes.data + r0 * bpr, Xq.ctypes.data, out.ctypes.data + 4 * r0, r1 - r0, 1, k)
            run1 = lambda X=X, Xq=Xq, k=k, rows=rows, d_work=d_work: (qz(X.ctypes.data, Xq.ctypes.data, k),
                                                                       d_work(0, rows))
            runn = lambda X=X, Xq=Xq, k=k, rows=rows, d_work=d_work: (qz(X.ctypes.data, Xq.ctypes.data, k),
                                                                       _pinned_parallel(rows, allc, d_work))
            leg(f"cfg2_{name}_quant_q8_0+dispatch_{rows}x{k}", run1, runn, W.nbytes + k * 4 + rows * 4,
                {"ref": "bench/bpd_cpu.c:4106-4136 + bench/bpd_gemm_q8_0_cpu.c:159-207",
                 "flags": "-O2 -mavx -mssse3 (tile order T)"})
            del W
    # the build's Q4_K x Q8_K order (no reference C exists), metric shape
    xq = O.quant_q8_k(x_host)
    leg("metric_q4k_q8k_oracle_14336x4096", lambda: O.qmatmul_q4k_q8k(w_host, xq, M, K, 0, 1),
        lambda: O.qmatmul_q4k_q8k(w_host, xq, M, K, 0, allc), ALG_BYTES,
        {"ref": "none: no reference C exists for Q4_K x Q8_K; this build's C oracle", "flags": "-O2 -ffp-contract=off",
         "threads": "unpinned pthreads over rows"})
    mm_work(0, M)  # the output of the parity check below
    res = {"value": m[f"{allc}_cores_gb_s"], "unit": "GB/s", "cores": allc, "kind": kind,
           "sample": f"bpd_qmatmul_q4k (reference C, -O2) at the full 14336x4096 metric shape with fp32 x, rows "
                     f"split over {allc} pinned threads, median of {runs} runs: {m[f'{allc}_cores_ms']} ms per "
                     f"GEMV; bytes counted as for the GPU metric with fp32 x",
           "cpu_model": _cpu_model(), "cpus_available": len(os.sched_getaffinity(0)), "runs_per_leg": runs,
           "legs": legs}
    return res, y


def cfg3_layers(torch, dev, synth, n_layers=32):
    """Q4_K weights of a 32-layer Mistral-7B-shaped model (each tensor its own
    seed) and N(0,1) activations for the GEMV chain."""
    from bpd_substrate_amd import decode

    log(f"cfg3: generating {n_layers} layers of Q4_K weights")
    d = decode.Dims()
    e, kv, ff = d.n_embd, d.n_kv, d.ff
    layers, acts = [], []
    for i in range(n_layers):
        k = lambda t: synth.key(42, 1000 + 8 * i + t)
        shapes = dict(q=(e, e), k=(kv, e), v=(kv, e), o=(e, e), gate=(ff, e), up=(ff, e), down=(e, ff))
        layers.append(decode.LayerWeights(**{n: torch.from_numpy(synth.q4k(m, kk, k(t))).to(dev)
                                             for t, (n, (m, kk)) in enumerate(shapes.items())}))
        acts.append([torch.from_numpy(synth.normal_f32(n, synth.key(43, 10 * i + j))).to(dev)
                     for j, n in enumerate((e, e, e, ff))])
    return layers, acts


def decode_chain(torch, L, T, dev, gpu, layers, acts, tokens=10):
    """cfg3: the GEMV portion of a 32-layer Mistral-7B-shaped decode step,
    Q4_K weights, activations N(0,1) -> Q8_K."""
    from bpd_substrate_amd import decode

    d = decode.Dims()
    n_layers = len(layers)
    out = {}
    for fused in (True, False):
        chain = decode.GemvChain(layers, d, dev, fused=fused)
        torch.cuda.synchronize()
        L.bpd_gpu_set_stream(T.stream.cuda_stream)
        chain.step(acts)
        torch.cuda.synchronize()
        gpu.check()
        us = T.us_per_launch([lambda: chain.step(acts)] * tokens, graph=True)  # us per token
        wb = chain.weight_bytes()
        gpu.check()
        r = {"us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1), "weight_bytes": wb,
             "gb_s": round(wb / us / 1e3, 1), "frac_hbm": round(wb / us / 1e3 / HBM_PEAK_GBS, 4),
             "launches_per_token": (4 if fused else 8) * n_layers,
             "roofline_us_per_token": round(wb / HBM_PEAK_GBS / 1e3, 1)}
        if fused:
            out = r
            out["quantization"] = "Q8_K of each activation inside its GEMV kernel"
        else:
            out["separate_quant_launches"] = {k: r[k] for k in ("us_per_token", "tokens_per_s", "launches_per_token")}
        del chain
    return out


def decode_step(torch, L, T, dev, gpu, synth, layers, tokens=10, max_seq=4096, vocab=32000):
    """cfg3 as a whole decode step (bpd_llama_step_gpu): the chain's
    Q4_K weights plus RMSNorm, RoPE, the fp32 K/V cache, GQA attention,
    SwiGLU, a Q4_K head of `vocab` rows and argmax, one token at a time.
    Timed at short context (positions 0..tokens-1) and after 2048 cached rows."""
    from bpd_substrate_amd import llama

    E, H, HKV, D, F = 4096, 32, 8, 128, 14336
    cfg = dict(n_layers=len(layers), n_embd=E, n_head=H, n_head_kv=HKV, head_dim=D, ff_dim=F, vocab_size=vocab,
               max_seq=max_seq, eps=1e-5, rope_theta=1e6)
    norm = lambda t: torch.from_numpy(1.0 + 0.1 * synth.normal_f32(E, synth.key(44, t))).to(dev)
    dl = [dict(attn_norm=norm(2 * i), ffn_norm=norm(2 * i + 1), **{n: getattr(lw, n) for n in llama.MATRICES})
          for i, lw in enumerate(layers)]
    lm = torch.from_numpy(synth.q4k(vocab, E, synth.key(44, 999))).to(dev)
    m = llama.DecodeModel(cfg, dl, norm(998), lm_head=lm, fmt=llama.W_Q4K, device=dev)
    embs = [torch.from_numpy(synth.normal_f32(E, synth.key(45, t))).to(dev) for t in range(tokens)]
    with torch.cuda.stream(T.stream):
        m.step(embs[0], 0)  # allocates the step workspace before any capture
    torch.cuda.synchronize()
    gpu.check()
    wb = sum(t.numel() for lw in layers for t in (getattr(lw, n) for n in llama.MATRICES)) + lm.numel()
    out = {"weight_bytes": wb, "vocab": vocab, "max_seq": max_seq}
    for pos0 in (0, 2048):
        us = T.us_per_launch([(lambda t=t: m.enqueue(embs[t], pos0 + t)) for t in range(tokens)], graph=True)
        gpu.check()
        # the RMSNorms fold into the GEMVs at this shape: per layer Q/K/V (with the
        # attention norm), attention (1 kernel up to 64 rows, else 2), O, the FFN
        # norm's Q8_K, gate/up, down; layer 0's attention norm, the final norm, the
        # head and argmax on top
        attn = 1 if pos0 + tokens <= 64 else 2
        out[f"pos{pos0}"] = {"launches_per_token": len(layers) * (5 + attn) + 4,
                             "us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1),
                             "weight_gb_s": round(wb / us / 1e3, 1),
                             "frac_hbm": round(wb / us / 1e3 / HBM_PEAK_GBS, 4)}
    # the reference driver's pattern: one synchronous generate-style call per token, no graph
    with torch.cuda.stream(T.stream):
        t0 = time.perf_counter()
        for t in range(tokens):
            m.step(embs[t], t)
        eager = (time.perf_counter() - t0) / tokens * 1e6
    out["eager_sync_us_per_token"] = round(eager, 1)
    out["roofline_us_per_token"] = round(wb / HBM_PEAK_GBS / 1e3, 1)
    del m, dl, lm
    return out


def prefill_forward(torch, dev, gpu, synth, n_layers=32, tokens=512, vocab=32000, sets=4, runs=3):
    """The reference CPU library's forward (bpd_llama_forward_s_gpu: order S, the
    cfg4 int8-MFMA GEMM for every projection) over a 32-layer Mistral-7B-shaped
    Q8_0 model with binary16 caches, one prefill of `tokens` tokens from an empty
    cache; `sets` distinct weight copies rotate over the layers (0.93 GB, beyond
    the MALL).  Eager calls: the forward uploads its host token and position
    arrays and waits for that copy, as the reference's CPU call reads them."""
    from bpd_substrate_amd import llama

    E, H, HKV, D, F = 4096, 32, 8, 128, 14336
    cfg = dict(n_layers=n_layers, n_heads=H, n_kv_heads=HKV, head_dim=D, embed_dim=E, ffn_dim=F, vocab_size=vocab,
               max_seq_len=tokens, rms_eps=1e-5, rope_base=1e6, rope_dim=D, kv_cache_f16=1)
    shapes = {"w_q": (H * D, E), "w_k": (HKV * D, E), "w_v": (HKV * D, E), "w_o": (E, H * D),
              "w_gate": (F, E), "w_up": (F, E), "w_down": (E, F)}
    base = {n: torch.from_numpy(synth.q8_0(r, k, synth.key(46, i), d_sigma=0.002)).to(dev)
            for i, (n, (r, k)) in enumerate(shapes.items())}
    norm = lambda t: torch.from_numpy((1.0 + 0.1 * synth.normal_f32(E, synth.key(47, t))).astype(np.float32)).to(dev)
    wsets = [base] + [{n: t.clone() for n, t in base.items()} for _ in range(sets - 1)]
    layers = [dict(attn_norm_w=norm(2 * l), ffn_norm_w=norm(2 * l + 1), **wsets[l % sets]) for l in range(n_layers)]
    embd = torch.from_numpy(synth.q8_0(vocab, E, synth.key(46, 90), d_sigma=0.02)).to(dev)
    out_w = torch.from_numpy(synth.q8_0(vocab, E, synth.key(46, 91), d_sigma=0.002)).to(dev)
    f = llama.Forward(cfg, layers, embd, norm(999), out_w, device=dev)
    ids = (np.arange(tokens, dtype=np.int64) * 7919 % vocab).astype(np.int32)
    pos = np.arange(tokens, dtype=np.int32)
    f.forward(ids, pos, 0, order="S")
    torch.cuda.synchronize()
    gpu.check()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        f.forward(ids, pos, 0, order="S")
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    gpu.check()
    ms = float(np.median(times)) * 1e3
    gemm_ops = 2.0 * tokens * n_layers * sum(r * k for r, k in shapes.values())
    out = {"ms_per_prefill": round(ms, 2), "tokens_per_s": round(tokens / ms * 1e3, 1),
           "projection_tops": round(gemm_ops / ms / 1e9, 1), "tokens": tokens, "n_layers": n_layers,
           "weights": "Q8_0", "kv_cache": "binary16",
           "note": "bpd_llama_forward_s_gpu, host wall clock per call (launches, the token/position upload and "
                   "the logits of every token included); projections on k_q8_0_gemm_SH"}
    del f, layers, wsets, base, embd, out_w
    return out


def load_traffic():
    p = os.path.join(ROOT, "profiles", "q4k_q8k_gemv_14336x4096_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              f"the row-sharded multi-GPU design is documented but not run", file=sys.stderr)
        sys.exit(2)
    import torch

    from bpd_substrate_amd import gpu, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = gpu.lib()
    if a.prefill_only:
        log("prefill forward only (reference CPU library ABI, 32 layers, 512 tokens)")
        res = prefill_forward(torch, dev, gpu, synth)
        # a read of known size (the metric's weight bytes), the reference for FETCH_SIZE
        buf = torch.zeros(W_BYTES, dtype=torch.uint8, device=dev)
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        for _ in range(5):
            L.bpdq_stream_read_gpu(buf.data_ptr(), W_BYTES // 16, sink.data_ptr())
        torch.cuda.synchronize()
        gpu.check()
        print(json.dumps({"prefill_forward_32_layers_512_tokens": res}))
        return
    stream = torch.cuda.Stream()
    T = Timer(torch, L, stream)

    log("generating the 14336x4096 Q4_K weight and x")
    w_host = synth.q4k(M, K, synth.key(42, synth.STREAM["metric_w"]))
    x_host = synth.normal_f32(K, synth.key(42, synth.STREAM["metric_x"]))
    w0 = torch.from_numpy(w_host).to(dev)
    # eager regions (--steps <= 64) read `steps` distinct copies, and their warm-up 8 more, so
    # that no timed launch reads a copy that the warm-up or the previous region left in the
    # 256 MB MALL; graph regions cycle >= 512 MiB of copies
    copies = max(a.copies, -(-512 * 2**20 // W_BYTES), a.steps + 8 if a.steps <= Timer.EAGER_MAX else 0)
    ws = [w0] + [w0.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(x_host).to(dev)
    xq = torch.empty(X_BYTES, dtype=torch.uint8, device=dev)
    y = torch.empty(M, dtype=torch.float32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    L.bpd_gpu_set_stream(stream.cuda_stream)
    with torch.cuda.stream(stream):
        gpu.call("bpd_quant_q8_k_gpu", x, xq, K)
    torch.cuda.synchronize()
    wp = [t.data_ptr() for t in ws]

    def gemv(i):
        return lambda: L.bpd_qmatmul_q4k_q8k_gpu(wp[i % copies], xq.data_ptr(), y.data_ptr(), M, K)

    for i in range(a.warmup):
        gemv(i)()
    torch.cuda.synchronize()
    gpu.check()

    log(f"timing {a.steps} GEMVs over {copies} weight copies ({copies * W_BYTES / 2**20:.0f} MiB)")
    # eager warm-up on the 8 copies after the timed ones (264 MB): the first timed launches'
    # copies were last read a whole region earlier
    cold_warm = range(copies - 8, copies)
    us = T.us_per_launch([gemv(i) for i in range(a.steps)], warm=[gemv(i) for i in cold_warm])
    gpu.check()
    ms_per_step = us * 1e-3
    value = ALG_BYTES / (us * 1e-6) / 1e9

    # single-launch streaming-read floor for the same bytes, same copies
    def read(i):
        return lambda: L.bpdq_stream_read_gpu(wp[i % copies], W_BYTES // 16, sink.data_ptr())

    rd_us = T.us_per_launch([read(i) for i in range(a.steps)], warm=[read(i) for i in cold_warm])
    rd_gbs = W_BYTES / (rd_us * 1e-6) / 1e9
    # warm: one weight copy for every launch, so the 33 MB stay in the 256 MB MALL (not the
    # metric; skipped with --no-extra, so that a kernel trace of that run holds only the
    # metric's own launches of this kernel and grid)
    warm_us = None if a.no_extra else T.us_per_launch([gemv(0) for _ in range(a.steps)])
    gpu.check()


    result = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak) at 14336x4096; dequant Gelem/s; ULP vs ref",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot4 / fp32 (Q4_K x Q8_K)",
        "data": "synthetic (seeded splitmix64 Q4_K blocks per benchmark config; x ~ N(0,1) -> Q8_K)",
        "config": {"workload": "Q4_K x Q8_K GEMV, M=14336, K=4096, batch 1 (the headline metric shape)",
                   "weight_copies": copies,
                   "timing": ("eager" if a.steps <= Timer.EAGER_MAX else "HIP graph of") +
                             " `steps` back-to-back launches behind a GPU spin, events on their stream, median of 7"},
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
                     "kernel": "k_q4k_q8k_gemv_span", "alg_bytes_per_launch": ALG_BYTES,
                     "launch_us": round(us, 3),
                     "stream_read_floor": {"us": round(rd_us, 3), "gb_s": round(rd_gbs, 1),
                                           "frac_of_floor": round(rd_us / us, 4)}},
    }
    if warm_us is not None:
        result["metric_warm_mall"] = {"us": round(warm_us, 3), "gb_s": round(ALG_BYTES / warm_us / 1e3, 1),
                                      "note": "one weight copy for every launch (resident in the MALL): not the "
                                              f"metric, which rotates {copies} copies beyond it"}

    if not a.no_extra:
        # the same kernel family with the launch cost shared: two 14336x4096 matrices of one
        # Q8_K x in one multi-matrix launch (the decode step's gate + up), same rotating copies
        import ctypes
        y2 = torch.empty(M, dtype=torch.float32, device=dev)
        y_arr = (ctypes.c_void_p * 2)(y.data_ptr(), y2.data_ptr())
        m_arr = (ctypes.c_int * 2)(M, M)
        w_arrs = [(ctypes.c_void_p * 2)(wp[i % copies], wp[(i + 1) % copies]) for i in range(copies)]
        def pair(i):
            return lambda: L.bpd_qmatmul_q4k_q8k_multi_gpu(ctypes.addressof(w_arrs[(2 * i) % copies]),
                                                           ctypes.addressof(y_arr), ctypes.addressof(m_arr), 2,
                                                           xq.data_ptr(), K)

        # warm-up on the copies after the timed ones (the pairs of cold_warm)
        pair_us = T.us_per_launch([pair(i) for i in range(a.steps // 2)],
                                  warm=[pair(i) for i in range((copies - 8) // 2, copies // 2)])
        gpu.check()
        pair_bytes = 2 * W_BYTES + X_BYTES + 2 * Y_BYTES
        result["two_matrix_launch_2x14336x4096"] = {
            "us": round(pair_us, 3), "gb_s": round(pair_bytes / pair_us / 1e3, 1),
            "frac_hbm": round(pair_bytes / pair_us / 1e3 / HBM_PEAK_GBS, 4),
            "note": "not the metric: two GEMVs of one x per launch, as the decode step's gate + up"}
        log("dequant 4096x4096 (cfg0) and Q8_0 GEMVs (cfg2)")
        dq_in = torch.from_numpy(synth.q4k(DQ_BLOCKS, 256, synth.key(42, synth.STREAM["cfg0_w"]))).to(dev)
        dq_q = [dq_in] + [dq_in.clone() for _ in range(7)]
        dq_o = [torch.empty(DQ_BLOCKS * 256, dtype=torch.float32, device=dev) for _ in range(8)]
        dq_us = T.us_per_launch([(lambda i=i: L.bpd_dequant_q4k_gpu(dq_q[i % 8].data_ptr(), dq_o[i % 8].data_ptr(),
                                                                   DQ_BLOCKS)) for i in range(400)])
        # the write floor of one launch of the dequant's output size (67 MB), same buffers
        wr_us = T.us_per_launch([(lambda i=i: L.bpdq_stream_write_gpu(dq_o[i % 8].data_ptr(), DQ_BLOCKS * 64, i))
                                 for i in range(400)])
        gpu.check()
        result["dequant_cfg0"] = {"us": round(dq_us, 3), "gelem_s": round(DQ_BLOCKS * 256 / dq_us / 1e3, 1),
                                  "gb_s": round(DQ_BYTES / dq_us / 1e3, 1),
                                  "frac_hbm": round(DQ_BYTES / dq_us / 1e3 / HBM_PEAK_GBS, 4),
                                  "stream_write_floor_67MB": {
                                      "us": round(wr_us, 3), "gb_s": round(DQ_BLOCKS * 1024 / wr_us / 1e3, 1),
                                      "note": "k_stream_write of the output bytes alone; the dequant also reads 9.4 MB"}}
        del dq_q, dq_o, dq_in
        q_us = T.us_per_launch([(lambda: L.bpd_quant_q8_k_gpu(x.data_ptr(), xq.data_ptr(), K))] * 200)
        result["quant_q8_k_4096_us"] = round(q_us, 3)
        # cfg1: the cfg0 weight as a 4096x4096 GEMV against x -> Q8_K (rows of 16 blocks)
        w1 = torch.from_numpy(synth.q4k(4096, 4096, synth.key(42, synth.STREAM["cfg0_w"]))).to(dev)
        g1 = [w1] + [w1.clone() for _ in range(-(-512 * 2**20 // w1.numel()) - 1)]
        y1 = torch.empty(4096, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        c1_us = T.us_per_launch([(lambda i=i: L.bpd_qmatmul_q4k_q8k_gpu(g1[i % len(g1)].data_ptr(), xq.data_ptr(),
                                                                       y1.data_ptr(), 4096, 4096))
                                 for i in range(1000)])
        # its single-launch read floor: k_stream_read of the same weight bytes, same copies
        c1_rd = T.us_per_launch([(lambda i=i: L.bpdq_stream_read_gpu(g1[i % len(g1)].data_ptr(), w1.numel() // 16,
                                                                    sink.data_ptr())) for i in range(1000)])
        gpu.check()
        c1_bytes = 4096 * 16 * 144 + X_BYTES + 4096 * 4
        result["q4k_q8k_gemv_cfg1_4096x4096"] = {"us": round(c1_us, 3), "gb_s": round(c1_bytes / c1_us / 1e3, 1),
                                                 "frac_hbm": round(c1_bytes / c1_us / 1e3 / HBM_PEAK_GBS, 4),
                                                 "copies": len(g1),
                                                 "stream_read_floor": {"us": round(c1_rd, 3),
                                                                       "frac_of_floor": round(c1_rd / c1_us, 4)}}
        del g1, w1, y1
        # Q6_K x Q8_K (GGUF element map) at the 32,000 x 4096 head of a Q4_K_M model: random
        # quant bytes with a finite f16 scale per block (seeded)
        nq6 = 32000 * 16
        q6 = synth.random_bytes(nq6 * 210, synth.key(42, 700)).reshape(nq6, 210)
        q6[:, 208:210] = (np.abs(synth.normal_f32(nq6, synth.key(42, 701))) * 0.02).astype(np.float16) \
            .view(np.uint8).reshape(nq6, 2)
        w6 = torch.from_numpy(q6.reshape(-1)).to(dev)
        g6 = [w6] + [w6.clone() for _ in range(-(-512 * 2**20 // w6.numel()) - 1)]
        y6 = torch.empty(32000, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        q6_us = T.us_per_launch([(lambda i=i: L.bpd_qmatmul_q6k_q8k_gguf_gpu(g6[i % len(g6)].data_ptr(), xq.data_ptr(),
                                                                            y6.data_ptr(), 32000, 4096))
                                 for i in range(400)])
        q6_bytes = nq6 * 210 + X_BYTES + 32000 * 4
        result["q6k_q8k_gemv_gguf_32000x4096"] = {"us": round(q6_us, 3), "gb_s": round(q6_bytes / q6_us / 1e3, 1),
                                                  "frac_hbm": round(q6_bytes / q6_us / 1e3 / HBM_PEAK_GBS, 4),
                                                  "copies": len(g6)}
        del g6, w6, y6, q6
        for name, (rows, k) in Q80_SHAPES.items():
            W = torch.from_numpy(synth.q8_0(rows, k, synth.key(42, synth.STREAM[f"cfg2_{name}"]))).to(dev)
            n_c = max(16, -(-512 * 2**20 // W.numel()))
            Ws = [W] + [W.clone() for _ in range(n_c - 1)]
            X = torch.from_numpy(synth.normal_f32(k, synth.key(42, synth.STREAM[f"cfg2_x_{name}"]))).to(dev)
            Xq = gpu.quant_q8_0(X)
            out = torch.empty(rows, dtype=torch.float32, device=dev)
            torch.cuda.synchronize()
            u = T.us_per_launch([(lambda i=i: L.bpd_qmatmul_q8_0_dispatch_gpu(Ws[i % n_c].data_ptr(), Xq.data_ptr(),
                                                                             out.data_ptr(), rows, 1, k))
                                 for i in range(400)])
            rd = T.us_per_launch([(lambda i=i: L.bpdq_stream_read_gpu(Ws[i % n_c].data_ptr(), W.numel() // 16,
                                                                      sink.data_ptr())) for i in range(400)])
            gpu.check()
            alg = W.numel() + Xq.numel() + rows * 4
            result[f"q8_0_gemv_{rows}x{k}"] = {"us": round(u, 3), "gb_s": round(alg / u / 1e3, 1),
                                              "frac_hbm": round(alg / u / 1e3 / HBM_PEAK_GBS, 4),
                                              "order": "llamafile tile (T), bit-exact",
                                              "stream_read_floor": {"us": round(rd, 3),
                                                                    "frac_of_floor": round(rd / u, 4)}}
            del Ws, W
        # the reference-order fp32-x GEMV (bpd_qmatmul_q4k_gpu, bit-identical to the CPU
        # reference) at the metric shape, same rotating weight copies
        y_c = torch.empty(M, dtype=torch.float32, device=dev)
        rc_us = T.us_per_launch([(lambda i=i: L.bpd_qmatmul_q4k_gpu(wp[i % copies], x.data_ptr(), y_c.data_ptr(), M, K))
                                 for i in range(100)])
        gpu.check()
        rc_bytes = W_BYTES + K * 4 + Y_BYTES
        result["reference_order_gemv_14336x4096"] = {
            "us": round(rc_us, 3), "gb_s": round(rc_bytes / rc_us / 1e3, 1),
            "frac_hbm": round(rc_bytes / rc_us / 1e3 / HBM_PEAK_GBS, 4),
            "order": "bpd_qmatmul_q4k's sequential fp32 chain per row (bench/bpd_quant.c:88-109), bit-exact"}
        del y_c
        # cfg4: batched prefill, 512 tokens x 4096 x 14336 rows, order S on int8 MFMA
        W = torch.from_numpy(synth.q8_0(14336, 4096, synth.key(42, synth.STREAM["cfg2_up"]))).to(dev)
        X = torch.from_numpy(synth.normal_f32(512 * 4096, synth.key(42, synth.STREAM["cfg4_x"]))).to(dev)
        Xq = gpu.quant_q8_0(X)
        out = torch.empty(512 * 14336, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        u = T.us_per_launch([(lambda: L.bpd_qmatmul_q8_0_dispatch_s_gpu(W.data_ptr(), Xq.data_ptr(), out.data_ptr(),
                                                                         14336, 512, 4096))] * 50)
        ops = 2.0 * 512 * 4096 * 14336
        # the device's int8 MFMA rate: register-only v_mfma_i32_32x32x32_i8 rounds, 8 waves per CU
        probe_waves, probe_iters = 2048, 4096
        sink = torch.zeros(4, dtype=torch.int32, device=dev)
        pu = T.us_per_launch([(lambda: L.bpdq_mfma_i8_probe_gpu(probe_waves, probe_iters, sink.data_ptr()))] * 5)
        gpu.check()
        probe_tops = probe_waves * probe_iters * 4 * 32 * 32 * 32 * 2 / pu / 1e6
        result["int8_mfma_probe"] = {"tops": round(probe_tops, 1), "frac_of_peak": round(probe_tops / 5000.0, 4),
                                     "us": round(pu, 2),
                                     "kernel": "k_mfma_i8_probe: 2048 waves x 4096 rounds of 4 register-only "
                                               "v_mfma_i32_32x32x32_i8"}
        result["prefill_q8_0_cfg4"] = {"us": round(u, 2), "tops": round(ops / u / 1e6, 1),
                                       "frac_int8_mfma": round(ops / u / 1e6 / 5000.0, 4),
                                       "frac_of_probe": round(ops / u / 1e6 / probe_tops, 4),
                                       "order": "scalar S, bit-exact vs the -O2 reference build"}
        del W, X, Xq, out
        gpu.check()
        layers, acts = cfg3_layers(torch, dev, synth)
        result["decode_cfg3"] = decode_chain(torch, L, T, dev, gpu, layers, acts)
        result["decode_cfg3"]["full_step"] = decode_step(torch, L, T, dev, gpu, synth, layers)
        del layers, acts
        log("prefill forward (reference CPU library ABI, 32 layers, 512 tokens)")
        result["prefill_forward_32_layers_512_tokens"] = prefill_forward(torch, dev, gpu, synth)

    if not a.no_cpu:
        log("CPU baseline (reference C, 1 core and all cores)")
        cb, y_cpu = cpu_baseline(w_host, x_host, a.cpu_runs)
        for name, gpu_us in (("metric_bpd_qmatmul_q4k_14336x4096", result.get("reference_order_gemv_14336x4096", {}).get("us")),
                             ("metric_q4k_q8k_oracle_14336x4096", us),
                             ("cfg0_bpd_dequant_q4k_4096x4096", result.get("dequant_cfg0", {}).get("us"))):
            if gpu_us and name in cb["legs"]:
                c = cb["legs"][name]
                c["gpu_speedup_vs_all_cores"] = round(c[f"{cb['cores']}_cores_ms"] * 1e3 / gpu_us, 1)
        result["cpu_baseline"] = cb
        # the GPU reference-order entry point reproduces the CPU reference bit for bit
        y_chain = torch.empty(M, dtype=torch.float32, device=dev)
        with torch.cuda.stream(stream):
            gpu.call("bpd_qmatmul_q4k_gpu", w0, x, y_chain, M, K)
        torch.cuda.synchronize()
        diff = int(np.count_nonzero(y_chain.cpu().numpy().view(np.uint32) != y_cpu.view(np.uint32)))
        result["ulp_vs_ref"] = {"bpd_qmatmul_q4k_gpu_rows_differing_from_reference_C": diff, "of_rows": M}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
