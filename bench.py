#!/usr/bin/env python3
"""Benchmark of the MLX-affine Q4 matrix-product path on one MI355X.

Headline workload (one "step"): the per-token MLP + lm_head work of
marlin-mlx's decode loop at M = 1 (src/core/engine.cpp:79-94 ->
src/model/marlin.cpp:110-145, 161-169 -> src/sampling/sampler.cpp:14-16):
    for each of 24 layers:  x = x + down(swiglu(gate n, up n)),  n = rms_norm_l(x)
    token = argmax(lm_head(rms_norm(x)))
with MLX affine Q4 group-64 weights (gate/up 6144x2048, down 2048x6144, tied
lm_head 248320x2048), bf16 activations, fp32 accumulation.  rms_norm is the
reference's (1 + w) RMSNorm (src/model/marlin.cpp:12-16, 141, 145); without it
the 24-layer residual chain grows quadratically and overflows bf16.  Weights
are synthetic N(0, 0.02) bf16 from the counter-based generator, quantized on
the GPU by this library's pack kernel.  The timed path is the one-launch
decode step (mq4_decode_step), launched back to back; it is checked against
the 49-kernel chain of the separate entry points (same token and hidden
state) before timing.

Output: one JSON line on stdout.  `value` is the step's algorithmic HBM
bandwidth, Q4 weight bytes per step (795,672,576 B) / step time; inputs are
resident in HBM before the timed region and the 796 MB weight stream is larger
than the 256 MB last-level cache, so every step reads the weights from HBM.
`configs` holds the other benchmark configurations, each with its own
roofline: the single gate GEMV cold and warm (config 1), the 24-layer MLP
chain (2), lm_head + argmax (3), the prefill GEMM (4), batched decode (5a)
and the pack of the full weight set (5b).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import statistics
import sys
import time
import traceback

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4 GEMV HBM GB/s (% of 8 TB/s peak); µs per decode-step MLP+lm_head"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0          # MI355X dense bf16 MFMA
LAYERS, HID, INTER, VOCAB = 24, 2048, 6144, 248320
EPS = 1e-6


def q4_bytes(N: int, K: int) -> int:
    """Packed nibbles + bf16 scales + bf16 biases of an [N, K] g64 matrix."""
    return N * K // 2 + 2 * 2 * (N * K // 64)


W_MLP = 3 * q4_bytes(INTER, HID)                  # 21,233,664
W_LM = q4_bytes(VOCAB, HID)                       # 286,064,640
STEP_BYTES = LAYERS * W_MLP + W_LM               # 795,672,576
KERNEL_BYTES = {                                  # algorithmic bytes per launch
    "norm_gate_up_silu": 2 * q4_bytes(INTER, HID) + 2 * 2 * HID + 2 * INTER,
    "down_residual": q4_bytes(HID, INTER) + 2 * INTER + 2 * 2 * HID,
    "norm_lm_head_argmax": W_LM + 2 * 2 * HID + 4,
    # weights + norm weights + x in, token out (activation exchange stays in L2)
    "decode_step": STEP_BYTES + (LAYERS + 1) * 2 * HID + 2 * HID + 4,
}
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_step_m1_hbm_traffic.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--kernel-steps", type=int, default=10,
                   help="eager steps with per-kernel HIP events (separate kernels)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-configs", action="store_true", help="headline only")
    p.add_argument("--only", default=None,
                   help="comma-separated config names to run (e.g. config5a_batched); default all")
    p.add_argument("--cpu-reps", type=int, default=3)
    p.add_argument("--profile-kernel", default=None,
                   choices=["decode_step", "copy", "gemv_gate", "lm_head", "prefill", "batched", "pack"],
                   help="counter-collection mode: run only that workload (warmup + steps launches) "
                        "and print no JSON line; 'copy' calibrates FETCH_SIZE/WRITE_SIZE with a "
                        "plain device copy of --copy-mib MiB per launch")
    p.add_argument("--copy-mib", type=int, default=256)
    p.add_argument("--prefill-m", type=int, default=2048)
    p.add_argument("--batched-m", type=int, default=16)
    return p.parse_args()


def measured_traffic():
    """HBM bytes per decode-step launch from the committed rocprofv3 summary
    (FETCH_SIZE and WRITE_SIZE runs, calibrated on a device copy)."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9,]+)", text)
    return int(m.group(1).replace(",", "")) if m else None


class Q4:
    """Device-resident MLX-layout Q4 matrix."""

    def __init__(self, wq, s, b, N, K):
        self.wq, self.s, self.b, self.N, self.K = wq, s, b, N, K

    def ptrs(self):
        return (ctypes.c_void_p(self.wq.data_ptr()), ctypes.c_void_p(self.s.data_ptr()),
                ctypes.c_void_p(self.b.data_ptr()))


class Env:
    """Library, device, stream helpers and the synthetic model."""

    def __init__(self, torch, mq4, dev):
        self.torch, self.mq4, self.dev = torch, mq4, dev
        self.L = mq4.lib()
        self.P = ctypes.c_void_p
        self.pack_us = 0.0
        self.pack_bytes = 0
        self.pack_set = []          # (shape, stream id) of every matrix quantized in the setup
        self.ev = lambda: torch.cuda.Event(enable_timing=True)

    def st(self):
        return self.P(self.torch.cuda.current_stream().cuda_stream)

    def make_q4(self, shape, stream_id, timed=True):
        torch, P, L = self.torch, self.P, self.L
        N, K = shape
        w = self.mq4.fill_normal_bf16(shape, stream_id, 0.0, 0.02, device=self.dev)
        wq = torch.empty((N, K // 8), dtype=torch.int32, device=self.dev)
        s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=self.dev)
        b = torch.empty_like(s)
        e0, e1 = self.ev(), self.ev()
        e0.record()
        self.mq4._check(L.mq4_quantize(P(w.data_ptr()), N, K, 64, 4, P(wq.data_ptr()), P(s.data_ptr()),
                                       P(b.data_ptr()), self.st()))
        e1.record()
        torch.cuda.synchronize()
        if timed:
            self.pack_us += e0.elapsed_time(e1) * 1e3
            self.pack_bytes += 2 * N * K + q4_bytes(N, K)
            self.pack_set.append((shape, stream_id))
        del w
        return Q4(wq, s, b, N, K)

    def per_launch(self, fn, n, warm=1):
        """Statistics of fn() timed one launch at a time: a HIP event pair on the
        launch stream around each of n calls (the events add a marker packet
        between launches, so these are per-launch durations, not throughput)."""
        for _ in range(warm):
            fn()
        self.torch.cuda.synchronize()
        evs = [(self.ev(), self.ev()) for _ in range(n)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        self.torch.cuda.synchronize()
        return launch_stats([a.elapsed_time(b) * 1e3 for a, b in evs])

    def timed(self, fn, n, warm=1):
        """Mean microseconds of fn() launched n times back to back, HIP events on
        the launch stream around the batch."""
        for _ in range(warm):
            fn()
        self.torch.cuda.synchronize()
        e0, e1 = self.ev(), self.ev()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        self.torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n


def launch_stats(us):
    """median / p10 / p90 / min / max / mean of per-launch microseconds."""
    v = sorted(us)
    q = lambda f: v[min(len(v) - 1, max(0, int(round(f * (len(v) - 1)))))]
    return {"n": len(v), "median": round(q(0.5), 2), "p10": round(q(0.1), 2), "p90": round(q(0.9), 2),
            "min": round(v[0], 2), "max": round(v[-1], 2), "mean": round(sum(v) / len(v), 2)}


def hbm_roofline(nbytes, us):
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def mfma_roofline(flops, us):
    tf = flops / (us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4)}


def load_oracle():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mq4_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    O = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(O)
    return O


def host_q4(torch, q):
    import numpy as np
    return (q.wq.cpu().numpy().view(np.uint32), q.s.cpu().view(torch.int16).numpy().view(np.uint16),
            q.b.cpu().view(torch.int16).numpy().view(np.uint16))


def host_bf16(torch, t):
    import numpy as np
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU mode).", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    mq4 = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    E = Env(torch, mq4, dev)
    L, P = E.L, E.P

    if args.profile_kernel == "copy":
        n = args.copy_mib * (1 << 20)
        src = torch.ones(n // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy: {args.warmup + args.steps} launches of {n} bytes read + {n} bytes written")
        return

    # ---------------------------------------------------------------- setup
    log(f"[bench] device {torch.cuda.get_device_name(dev)}; generating + packing "
        f"{LAYERS}x3 MLP matrices and the {VOCAB}x{HID} lm_head")
    layers = []
    for l in range(LAYERS):
        layers.append((E.make_q4((INTER, HID), mq4.stream_id_layer(l, 0)),
                       E.make_q4((INTER, HID), mq4.stream_id_layer(l, 1)),
                       E.make_q4((HID, INTER), mq4.stream_id_layer(l, 2))))
    lm = E.make_q4((VOCAB, HID), mq4.STREAM_LM_HEAD)
    norm_w = mq4.fill_normal_bf16((HID,), mq4.STREAM_NORM_WEIGHT, 0.1, 0.02, device=dev)
    layer_norms = [mq4.fill_normal_bf16((HID,), mq4.stream_id_layer_norm(l), 0.1, 0.02, device=dev)
                   for l in range(LAYERS)]
    x0 = mq4.fill_normal_bf16((1, HID), mq4.stream_id_decode_row(0), 0.0, 1.0, device=dev)
    torch.cuda.synchronize()
    log(f"[bench] pack: {E.pack_bytes} B in {E.pack_us:.1f} us ({E.pack_bytes / E.pack_us / 1e3:.1f} GB/s)")

    qt = lambda q: mq4.QuantizedTensor(q.wq, q.s, q.b)
    dec_layers = [mq4.DecoderLayer(layer_norms[l], mq4.MLPWeights(qt(g), qt(u), qt(d)))
                  for l, (g, u, d) in enumerate(layers)]
    dstep = mq4.DecodeStep(dec_layers, norm_w, qt(lm), EPS)
    idx_p = torch.zeros((1,), dtype=torch.int32, device=dev)
    dargs = lambda st, idx=idx_p, xo=None: (
        P(x0.data_ptr()), HID, INTER, LAYERS, ctypes.cast(dstep._arr, P), P(norm_w.data_ptr()), EPS,
        *lm.ptrs(), VOCAB, P(idx.data_ptr()), P(xo.data_ptr()) if xo is not None else None,
        P(dstep.workspace.data_ptr()), dstep.ws_bytes, st)

    if args.profile_kernel is not None:
        profile_mode(args, E, layers, lm, norm_w, layer_norms, x0, dstep, dargs)
        return

    # -------------------------------- separate kernels (the reference chain)
    x = torch.empty((1, HID), dtype=torch.bfloat16, device=dev)
    hbuf = torch.empty((1, INTER), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((1,), dtype=torch.int32, device=dev)
    ws_bytes = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)

    def launches():
        out = []
        xp, hp = P(x.data_ptr()), P(hbuf.data_ptr())
        for l, (g, u, d) in enumerate(layers):
            xin = P(x0.data_ptr()) if l == 0 else xp
            nw = P(layer_norms[l].data_ptr())
            out.append(("norm_gate_up_silu",
                        lambda st, xin=xin, nw=nw, g=g, u=u: L.mq4_rmsnorm_gate_up_silu(
                            xin, 1, HID, nw, EPS, *g.ptrs(), *u.ptrs(), INTER, hp, st)))
            out.append(("down_residual",
                        lambda st, xin=xin, d=d: L.mq4_qmm_residual(hp, 1, INTER, *d.ptrs(), HID, xin, xp, st)))
        out.append(("norm_lm_head_argmax", lambda st: L.mq4_rmsnorm_lm_head_argmax(
            xp, 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB, P(idx.data_ptr()), None,
            P(ws.data_ptr()), ws_bytes, st)))
        return out

    steps = launches()

    def run_step(st):
        for _, fn in steps:
            rc = fn(st)
            if rc != 0:
                mq4._check(rc)

    run_step(E.st())
    torch.cuda.synchronize()
    tok_eager = int(idx.item())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_step(P(side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step(E.st())
    torch.cuda.synchronize()
    us_sep = E.timed(graph.replay, max(args.steps // 4, 5), warm=args.warmup)
    if int(idx.item()) != tok_eager:
        raise RuntimeError("separate-kernel graph replay token differs from the eager token")
    log(f"[bench] separate kernels (HIP graph of 49 launches): {us_sep:.1f} us per step")

    kernels = {}
    st = E.st()
    kinds = []
    for kind, _ in steps:
        if kind not in kinds:
            kinds.append(kind)
    for kind in kinds:
        fns = [fn for k, fn in steps if k == kind]
        nk = args.kernel_steps
        us = E.timed(lambda: [fn(st) for fn in fns], nk) / len(fns)
        kernels[kind] = {"mean_us": round(us, 3), "launches_per_step": len(fns),
                         "us_per_step": round(us * len(fns), 2), "bytes_per_launch": KERNEL_BYTES[kind],
                         "GBps": round(KERNEL_BYTES[kind] / (us * 1e-6) / 1e9, 1)}
        log(f"[bench] kernel {kind}: {kernels[kind]}")

    # ------------------------------------------------ headline: one launch
    x_p = torch.empty((HID,), dtype=torch.bfloat16, device=dev)
    run_step(E.st())
    mq4._check(L.mq4_decode_step(*dargs(E.st(), idx_p, x_p)))
    torch.cuda.synchronize()
    tok_p = int(idx_p.item())
    if tok_p != tok_eager or not torch.equal(x_p.view(torch.int16), x.reshape(-1).view(torch.int16)):
        raise RuntimeError(f"one-launch decode step disagrees with the separate kernels "
                           f"(token {tok_p} vs {tok_eager})")
    log(f"[bench] one-launch step = separate kernels: token {tok_p}, hidden state bit-identical")
    st = E.st()
    for _ in range(args.warmup):
        L.mq4_decode_step(*dargs(st))
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.warmup} launches); timing {args.steps} steps")
    t0, t1 = E.ev(), E.ev()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        L.mq4_decode_step(*dargs(st))
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    if int(idx_p.item()) != tok_eager:
        raise RuntimeError("one-launch decode step: token changed across launches")
    gbps = STEP_BYTES / (ms_step * 1e-3) / 1e9
    log(f"[bench] step {ms_step * 1e3:.1f} us, {gbps:.0f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of 8 TB/s)")
    # the same launches one at a time, each between its own pair of events
    step_stats = E.per_launch(lambda: L.mq4_decode_step(*dargs(st)), args.steps, warm=2)
    log(f"[bench] per-launch step durations: {step_stats}")
    # the same kernel replayed from a HIP graph (for callers that capture)
    pgraph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dstep(x0, None, idx_p)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(pgraph):
        dstep(x0, None, idx_p)
    us_graph = E.timed(pgraph.replay, max(args.steps // 4, 5), warm=3)
    kernels["decode_step"] = {"mean_us": round(ms_step * 1e3, 3), "launches_per_step": 1,
                              "us_per_step": round(ms_step * 1e3, 2),
                              "bytes_per_launch": KERNEL_BYTES["decode_step"],
                              "GBps": round(KERNEL_BYTES["decode_step"] / (ms_step * 1e-3) / 1e9, 1),
                              "graph_replay_us": round(us_graph, 2), "per_launch_us": step_stats}
    roofline = {"kernel": "decode_step", **hbm_roofline(KERNEL_BYTES["decode_step"], ms_step * 1e3),
                "traffic": measured_traffic()}

    # ------------------------------------------------------ other configs
    configs = {}
    if not args.no_configs:
        for name, fn in (("config1_gemv_gate", lambda: bench_gemv_gate(E, layers, x0)),
                         ("config2_mlp_chain", lambda: bench_mlp_chain(E, dec_layers, lm, norm_w, x0)),
                         ("config3_lm_head_argmax", lambda: bench_lm_head(E, lm, norm_w, x0, dstep)),
                         ("integration_per_layer", lambda: bench_per_layer(E, dstep, layers, lm, norm_w, layer_norms,
                                                                           x0, tok_p)),
                         ("config4_prefill", lambda: bench_prefill(E, layers, args, layer_norms)),
                         ("config5a_batched", lambda: bench_batched(E, layers, lm, norm_w, layer_norms)),
                         ("config5b_pack", lambda: bench_pack(E, layers, lm)),
                         ("next_q4_projections", lambda: bench_projections(E, x0)),
                         ("next_sampling", lambda: bench_sampling(E, lm, norm_w, x0))):
            if args.only and name not in args.only.split(","):
                continue
            try:
                configs[name] = fn()
                log(f"[bench] {name}: {json.dumps(configs[name])}")
            except Exception as e:                      # reported, never hidden
                traceback.print_exc()
                configs[name] = {"error": f"{type(e).__name__}: {e}"}

    # ------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(torch, layers, lm, x0, norm_w, layer_norms, args.cpu_reps, tok_eager, configs)

    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode step M=1: 24 x [RMSNorm(1+w) -> Q4 SwiGLU MLP (gate/up 6144x2048, "
                        "down 2048x6144, group 64) -> residual add], RMSNorm(1+w) -> Q4 lm_head "
                        "248320x2048 -> greedy argmax",
            "M": 1,
            "weight_bytes_per_step": STEP_BYTES,
            "us_per_step": round(ms_step * 1e3, 2),
            "us_per_launch_median_p10_p90": [step_stats["median"], step_stats["p10"], step_stats["p90"]],
            "pct_of_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "separate_kernels": {"us_per_step": round(us_sep, 2),
                             "GBps": round(STEP_BYTES / (us_sep * 1e-6) / 1e9, 1),
                             "note": "the same step as 49 separate kernels (24 x [norm+gate/up+SiLU, "
                                     "down+residual], norm+lm_head+argmax, argmax finalize) replayed "
                                     "from one HIP graph"},
        "path": "one-launch decode step (mq4_decode_step), launched back to back",
        "configs": configs,
        "token": tok_p,
    }
    print(json.dumps(line), flush=True)


# ------------------------------------------------------------------ configs

def bench_gemv_gate(E, layers, x0):
    """Config 1: one gate GEMV, M=1, 6144x2048 (mq4_qmm).  Cold: rotating over
    80 distinct gate-shaped matrices (566 MB, more than twice the 256 MB
    last-level cache); warm: one matrix repeated (it stays in that cache)."""
    torch, L, P = E.torch, E.L, E.P
    mats = [g for g, u, d in layers] + [u for g, u, d in layers]
    extra = [E.make_q4((INTER, HID), 5000 + i, timed=False) for i in range(80 - len(mats))]
    mats = mats + extra
    y = torch.empty((1, INTER), dtype=torch.bfloat16, device=E.dev)
    st = E.st()
    xp, yp = P(x0.data_ptr()), P(y.data_ptr())
    nbytes = q4_bytes(INTER, HID) + 2 * HID + 2 * INTER
    cold = E.timed(lambda: [L.mq4_qmm(xp, 1, HID, *m.ptrs(), INTER, 1, 64, 4, yp, st) for m in mats], 3,
                   warm=1) / len(mats)
    m0 = mats[0]
    warm = E.timed(lambda: L.mq4_qmm(xp, 1, HID, *m0.ptrs(), INTER, 1, 64, 4, yp, st), 200, warm=20)

    # the same launches replayed from HIP graphs: no host launch gaps, only the
    # device's own dispatch gap between consecutive kernels
    def graph_per_launch(fns, reps):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for f in fns:
                f(P(side.cuda_stream))
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_):
            for f in fns:
                f(E.st())
        us_ = E.timed(g_.replay, reps, warm=2) / len(fns)
        del g_
        return us_

    qmm = lambda m: (lambda s_: L.mq4_qmm(xp, 1, HID, *m.ptrs(), INTER, 1, 64, 4, yp, s_))
    cold_g = graph_per_launch([qmm(m) for m in mats], 10)
    warm_g = graph_per_launch([qmm(m0)] * len(mats), 10)
    del extra
    return {"shape": "M=1, N=6144, K=2048 (gate_proj)", "bytes_per_launch": nbytes,
            "cold_us": round(cold_g, 3), "warm_us": round(warm_g, 3),
            "roofline_cold": hbm_roofline(nbytes, cold_g), "roofline_warm": hbm_roofline(nbytes, warm_g),
            "cold_back_to_back_us": round(cold, 3), "warm_back_to_back_us": round(warm, 3),
            "note": "cold_us / warm_us: HIP graph of 80 launches replayed, time per launch (the device's "
                    "dispatch gap between kernels included, no host launch gaps; the rooflines use it); "
                    "back_to_back: the same launches issued from the host one after another; cold rotates "
                    "over 80 distinct matrices (566 MB > 2 x 256 MB last-level cache), warm repeats one "
                    "(served from that cache, so its rate exceeds HBM)"}


def bench_mlp_chain(E, dec_layers, lm, norm_w, x0):
    """Config 2: the 24 SwiGLU MLP layers with the residual chain, M=1 (the
    one-launch decode step with a 1-row lm_head, so the step is all MLP)."""
    torch, L, P, mq4 = E.torch, E.L, E.P, E.mq4
    lm1 = mq4.QuantizedTensor(lm.wq[:1].contiguous(), lm.s[:1].contiguous(), lm.b[:1].contiguous())
    step = mq4.DecodeStep(dec_layers, norm_w, lm1, EPS)
    idx = torch.zeros((1,), dtype=torch.int32, device=E.dev)
    st = E.st()
    a = (P(x0.data_ptr()), HID, INTER, LAYERS, ctypes.cast(step._arr, P), P(norm_w.data_ptr()), EPS,
         P(lm1.weight.data_ptr()), P(lm1.scales.data_ptr()), P(lm1.biases.data_ptr()), 1, P(idx.data_ptr()),
         None, P(step.workspace.data_ptr()), step.ws_bytes, st)
    us = E.timed(lambda: L.mq4_decode_step(*a), 50, warm=5)
    nbytes = LAYERS * W_MLP
    return {"shape": "24 x [RMSNorm, gate/up 6144x2048 + SwiGLU, down 2048x6144 + residual], M=1",
            "weight_bytes": nbytes, "us": round(us, 2), "roofline": hbm_roofline(nbytes, us),
            "note": "mq4_decode_step with a 1-row lm_head (the final norm and one 1 KB lm_head row "
                    "are the only extra work)"}


def bench_per_layer(E, dstep, layers, lm, norm_w, layer_norms, x0, tok):
    """The headline step as the reference's layer loop can call it (its
    attention / SSM half runs between the MLP halves, src/model/marlin.cpp:
    110-143): 24 separate calls of one MLP half each, then the final norm +
    lm_head + argmax, replayed from a HIP graph (as a serving loop would
    capture it).  Two call structures: the one-launch MLP half
    (mq4_decode_step with one layer and vocab 0; one-launch lm_head:
    mq4_decode_step with no layers) and mq4_mlp_residual at M = 1 (two
    kernels per layer) + mq4_rmsnorm_lm_head_argmax.  Both must give the
    headline token."""
    torch, L, P = E.torch, E.L, E.P
    a = torch.empty((HID,), dtype=torch.bfloat16, device=E.dev)
    b = torch.empty_like(a)
    idx = torch.zeros((1,), dtype=torch.int32, device=E.dev)
    sz = ctypes.sizeof(type(dstep._arr[0]))
    base = ctypes.addressof(dstep._arr)
    mwsb = L.mq4_mlp_workspace_size(1, HID, INTER)
    mws = torch.empty(mwsb, dtype=torch.uint8, device=E.dev)
    lwsb = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
    lws = torch.zeros(lwsb, dtype=torch.uint8, device=E.dev)

    def one_launch(st):
        src = P(x0.data_ptr())
        for l in range(LAYERS):
            dst = a if l % 2 == 0 else b
            E.mq4._check(L.mq4_decode_step(src, HID, INTER, 1, P(base + l * sz), None, EPS, None, None, None, 0,
                                           None, P(dst.data_ptr()), P(dstep.workspace.data_ptr()), dstep.ws_bytes,
                                           st))
            src = P(dst.data_ptr())
        E.mq4._check(L.mq4_decode_step(src, HID, INTER, 0, None, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                       P(idx.data_ptr()), None, P(dstep.workspace.data_ptr()), dstep.ws_bytes, st))

    def two_kernel(st):
        src = P(x0.data_ptr())
        for l, (g, u, d) in enumerate(layers):
            dst = a if l % 2 == 0 else b
            E.mq4._check(L.mq4_mlp_residual(src, 1, HID, P(layer_norms[l].data_ptr()), EPS, *g.ptrs(), *u.ptrs(),
                                            *d.ptrs(), INTER, P(mws.data_ptr()), mwsb, P(dst.data_ptr()), st))
            src = P(dst.data_ptr())
        E.mq4._check(L.mq4_rmsnorm_lm_head_argmax(src, 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                                  P(idx.data_ptr()), None, P(lws.data_ptr()), lwsb, st))

    def graph_us(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(P(side.cuda_stream))
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        if int(idx.item()) != tok:
            raise RuntimeError(f"integration_per_layer: token {int(idx.item())} differs from the step's {tok}")
        g_ = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_):
            fn(E.st())
        us_ = E.timed(g_.replay, 20, warm=3)
        idx.fill_(-1)
        g_.replay()
        torch.cuda.synchronize()
        if int(idx.item()) != tok:
            raise RuntimeError("integration_per_layer: graph replay token differs")
        del g_
        return us_

    us_one = graph_us(one_launch)
    us_two = graph_us(two_kernel)
    # one MLP half alone (the per-layer call), per launch
    st = E.st()
    half = E.per_launch(lambda: L.mq4_decode_step(P(x0.data_ptr()), HID, INTER, 1, P(base), None, EPS, None, None,
                                                  None, 0, None, P(a.data_ptr()), P(dstep.workspace.data_ptr()),
                                                  dstep.ws_bytes, st), 100, warm=5)
    return {"workload": "24 x one-call MLP half (M=1) + final norm + lm_head 248320 + argmax, each call "
                        "separate (the reference loop runs attention / SSM between them), HIP graph replay",
            "one_launch_mlp_half_us_per_step": round(us_one, 1),
            "one_launch_roofline": hbm_roofline(STEP_BYTES, us_one),
            "mlp_residual_two_kernels_us_per_step": round(us_two, 1),
            "mlp_residual_roofline": hbm_roofline(STEP_BYTES, us_two),
            "one_launch_mlp_half_per_launch_us": half, "token": tok,
            "note": "one-launch MLP half = mq4_decode_step(n_layers=1, vocab=0), the whole MLP half of a "
                    "layer in one persistent launch; the lm_head there is mq4_decode_step(n_layers=0)"}


def bench_lm_head(E, lm, norm_w, x0, dstep):
    """Config 3: final RMSNorm + lm_head 248320x2048 + greedy argmax, M=1, two
    ways: mq4_rmsnorm_lm_head_argmax (GEMV with per-block argmax keys, then a
    finalize launch; its workspace needs no initialisation) and the one-launch
    decode step with no layers (its lm_head phase, keys reduced inside the
    launch through tagged words; workspace zero-filled once).  Both must give
    the same token; `us` is the faster."""
    torch, L, P = E.torch, E.L, E.P
    idx = torch.zeros((1,), dtype=torch.int32, device=E.dev)
    idx1 = torch.zeros((1,), dtype=torch.int32, device=E.dev)
    wsb = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=E.dev)
    st = E.st()
    f = lambda: L.mq4_rmsnorm_lm_head_argmax(P(x0.data_ptr()), 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(),
                                             VOCAB, P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st)
    g = lambda: L.mq4_decode_step(P(x0.data_ptr()), HID, INTER, 0, None, P(norm_w.data_ptr()), EPS, *lm.ptrs(),
                                  VOCAB, P(idx1.data_ptr()), None, P(dstep.workspace.data_ptr()), dstep.ws_bytes, st)
    us_two = E.timed(f, 50, warm=5)
    us_one = E.timed(g, 50, warm=5)
    if int(idx.item()) != int(idx1.item()):
        raise RuntimeError(f"config3: one-launch token {int(idx1.item())} != two-launch token {int(idx.item())}")
    one_stats = E.per_launch(g, 50, warm=2)
    nbytes = KERNEL_BYTES["norm_lm_head_argmax"]
    us = min(us_one, us_two)
    return {"shape": "M=1, N=248320, K=2048 (+ (1+w) RMSNorm, greedy argmax)", "bytes_per_call": nbytes,
            "us": round(us, 2), "roofline": hbm_roofline(nbytes, us), "token": int(idx.item()),
            "one_launch_us": round(us_one, 2), "one_launch_per_launch_us": one_stats,
            "two_launch_us": round(us_two, 2),
            "note": "us is the faster of: one launch (mq4_decode_step with no layers: norm, lm_head GEMV and "
                    "the argmax reduced in the launch) and mq4_rmsnorm_lm_head_argmax (GEMV with per-block "
                    "argmax keys + a 4 us finalize launch); the 286 MB weight stream exceeds the last-level "
                    "cache"}


def bench_prefill(E, layers, args, layer_norms):
    """Config 4: prefill Q4 GEMM (MFMA), M tokens through gate/up + SwiGLU
    (6144x2048 x2) and down + residual (2048x6144), M in {1960, 2048, 8192}:
    the two entries separately, and the block's whole MLP half (RMSNorm +
    gate/up + SwiGLU + down + residual) as one mq4_mlp_residual call."""
    torch, L, P, mq4 = E.torch, E.L, E.P, E.mq4
    g, u, d = layers[0]
    st = E.st()
    out = {}
    for M in (1960, 2048, 8192):
        x = mq4.fill_normal_bf16((M, HID), mq4.STREAM_PREFILL, 0.0, 1.0, device=E.dev)
        h = torch.empty((M, INTER), dtype=torch.bfloat16, device=E.dev)
        y = torch.empty((M, HID), dtype=torch.bfloat16, device=E.dev)
        wsb = L.mq4_mlp_workspace_size(M, HID, INTER)
        ws = torch.empty(wsb, dtype=torch.uint8, device=E.dev)
        reps = 3 if M == 8192 else 10
        us_gu = E.timed(lambda: L.mq4_mlp_gate_up_silu(P(x.data_ptr()), M, HID, *g.ptrs(), *u.ptrs(), INTER,
                                                       P(h.data_ptr()), st), reps, warm=2)
        us_dn = E.timed(lambda: L.mq4_qmm_residual(P(h.data_ptr()), M, INTER, *d.ptrs(), HID, P(x.data_ptr()),
                                                   P(y.data_ptr()), st), reps, warm=2)
        us_one = E.timed(lambda: L.mq4_mlp_residual(P(x.data_ptr()), M, HID, P(layer_norms[0].data_ptr()), 1e-6,
                                                    *g.ptrs(), *u.ptrs(), *d.ptrs(), INTER, P(ws.data_ptr()), wsb,
                                                    P(y.data_ptr()), st), reps, warm=2)
        f_gu, f_dn = 2 * 2.0 * M * INTER * HID, 2.0 * M * HID * INTER
        out[str(M)] = {"gate_up_silu_us": round(us_gu, 1), "gate_up_silu": mfma_roofline(f_gu, us_gu),
                       "down_residual_us": round(us_dn, 1), "down_residual": mfma_roofline(f_dn, us_dn),
                       "mlp_us": round(us_gu + us_dn, 1), "mlp": mfma_roofline(f_gu + f_dn, us_gu + us_dn),
                       "mlp_residual_one_call_us": round(us_one, 1),
                       "mlp_residual_one_call": mfma_roofline(f_gu + f_dn, us_one)}
        del x, h, y, ws
    return {"shapes": "M x 2048 @ gate/up 6144x2048 (fused SwiGLU), M x 6144 @ down 2048x6144 (+ residual)",
            "flops": "2*M*N*K per matrix (algorithmic, bf16 MFMA peak 2.5 PFLOP/s dense)",
            "mlp_residual_one_call": "mq4_mlp_residual: RMSNorm(1+w) + gate/up + SwiGLU + down + residual in one "
                                     "call (pre-pass of the normalized x in the MFMA operand order, h written so by "
                                     "the SwiGLU epilogue; the norm's work counted in the time, not the flops)",
            "M": out}


def bench_batched(E, layers, lm, norm_w, layer_norms):
    """Config 5a: M concurrent token rows through the 24 MLPs (fused norm +
    gate/up + SwiGLU, down + residual) and norm + lm_head + argmax: one decode
    step of M streams, the separate entry points replayed from a HIP graph."""
    torch, L, P, mq4 = E.torch, E.L, E.P, E.mq4
    out = {}
    for M in (4, 16, 32):
        x = mq4.fill_normal_bf16((M, HID), 3000, 0.0, 1.0, device=E.dev)
        xb = torch.empty_like(x)
        h = torch.empty((M, INTER), dtype=torch.bfloat16, device=E.dev)
        idx = torch.empty((M,), dtype=torch.int32, device=E.dev)
        wsb = L.mq4_lm_head_argmax_workspace_size(M, VOCAB)
        ws = torch.zeros(wsb, dtype=torch.uint8, device=E.dev)

        def step(st):
            xin = P(x.data_ptr())
            for l, (g, u, d) in enumerate(layers):
                mq4._check(L.mq4_rmsnorm_gate_up_silu(xin, M, HID, P(layer_norms[l].data_ptr()), EPS, *g.ptrs(),
                                                      *u.ptrs(), INTER, P(h.data_ptr()), st))
                mq4._check(L.mq4_qmm_residual(P(h.data_ptr()), M, INTER, *d.ptrs(), HID, xin, P(xb.data_ptr()), st))
                xin = P(xb.data_ptr())
            mq4._check(L.mq4_rmsnorm_lm_head_argmax(xin, M, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                                    P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st))

        mwsb = L.mq4_mlp_workspace_size(M, HID, INTER)
        mws = torch.empty(mwsb, dtype=torch.uint8, device=E.dev)

        def step_one_call(st):
            # the MLP half of each layer as one mq4_mlp_residual call (from 5
            # rows its down product runs as two K parts per tile + a combine)
            xin = P(x.data_ptr())
            for l, (g, u, d) in enumerate(layers):
                mq4._check(L.mq4_mlp_residual(xin, M, HID, P(layer_norms[l].data_ptr()), EPS, *g.ptrs(), *u.ptrs(),
                                              *d.ptrs(), INTER, P(mws.data_ptr()), mwsb, P(xb.data_ptr()), st))
                xin = P(xb.data_ptr())
            mq4._check(L.mq4_rmsnorm_lm_head_argmax(xin, M, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                                    P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st))

        # the MLP halves of the 24 layers through mq4_mlp_layers: one launch
        # per layer (XCD-split gate/up and down products with in-kernel
        # exchanges), the hidden state ping-ponging in its workspace
        arr = (mq4._MlpLayerC * LAYERS)()
        for l, (g, u, d) in enumerate(layers):
            arr[l] = mq4._MlpLayerC(layer_norms[l].data_ptr(), *[q.value for q in (*g.ptrs(), *u.ptrs(), *d.ptrs())])
        lwsb = L.mq4_mlp_layers_workspace_size(M, HID, INTER)
        lws = torch.zeros(lwsb, dtype=torch.uint8, device=E.dev)

        def step_layers(st):
            mq4._check(L.mq4_mlp_layers(P(x.data_ptr()), M, HID, INTER, LAYERS, ctypes.cast(arr, P), EPS,
                                        P(xb.data_ptr()), P(lws.data_ptr()), lwsb, st))
            mq4._check(L.mq4_rmsnorm_lm_head_argmax(P(xb.data_ptr()), M, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(),
                                                    VOCAB, P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st))

        def graph_us(fn):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                fn(P(side.cuda_stream))
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g_ = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g_):
                fn(E.st())
            us_ = E.timed(g_.replay, 10, warm=3)
            del g_
            return us_

        us_sep = graph_us(step)
        tok_sep = idx.clone()
        us_one = graph_us(step_one_call)
        if not torch.equal(idx, tok_sep):
            raise RuntimeError(f"config5a M={M}: one-call MLP tokens differ from the separate entries'")
        us_lay = graph_us(step_layers)
        # same per-element arithmetic, fp32 sums grouped differently: the
        # tokens agree except on near-ties
        agree = float((idx == tok_sep).float().mean().item())
        us = min(us_sep, us_one, us_lay)
        nbytes = STEP_BYTES + M * (LAYERS * (2 * HID * 2 + INTER * 2) + 2 * HID)
        out[str(M)] = {"us_per_step": round(us, 1), "bytes_per_step": nbytes, "roofline": hbm_roofline(nbytes, us),
                       "separate_entries_us": round(us_sep, 1), "one_call_mlp_us": round(us_one, 1),
                       "one_launch_mlp_us": round(us_lay, 1), "one_launch_tokens_agree": round(agree, 3)}
    return {"workload": "M rows x [24 x (RMSNorm + gate/up 6144x2048 + SwiGLU, down 2048x6144 + residual), "
                        "RMSNorm + lm_head 248320x2048 + argmax]; MLP halves: MFMA GEMV (M >= 5) / dot2 GEMV "
                        "(M <= 4) or mq4_mlp_layers; lm_head + argmax: weight-ring kernel (M >= 3)",
            "note": "us_per_step is the fastest of three call structures, all HIP graphs of the same "
                    "per-element arithmetic: separate entries (mq4_rmsnorm_gate_up_silu + mq4_qmm_residual per "
                    "layer), one mq4_mlp_residual call per layer (the greedy tokens of these two must agree), "
                    "and mq4_mlp_layers (one launch per layer's MLP half, fp32 sums grouped differently; "
                    "one_launch_tokens_agree is its token agreement with the separate entries)",
            "M": out}


def bench_projections(E, x0):
    """The model's other projections quantized to Q4 (SSM in_proj_qkv 6144x2048,
    in_proj_z / out_proj 2048x2048; attention q_proj 4096x2048, k/v_proj
    512x2048, o_proj 2048x2048), one M=1 GEMV each, rotating over enough
    distinct copies that the set exceeds the 256 MB last-level cache."""
    torch, L, P = E.torch, E.L, E.P
    st = E.st()
    out = {}
    for name, (N, K) in (("in_proj_qkv", (6144, 2048)), ("q_proj", (4096, 2048)),
                         ("o_proj / out_proj / in_proj_z", (2048, 2048)), ("k_proj / v_proj", (512, 2048))):
        nb = q4_bytes(N, K)
        copies = max(4, (600 << 20) // nb)
        mats = [E.make_q4((N, K), 6000 + 97 * i + N, timed=False) for i in range(copies)]
        y = torch.empty((1, N), dtype=torch.bfloat16, device=E.dev)
        us = E.timed(lambda: [L.mq4_qmm(P(x0.data_ptr()), 1, K, *m.ptrs(), N, 1, 64, 4, P(y.data_ptr()), st)
                              for m in mats], 2, warm=1) / len(mats)
        out[name] = {"N": N, "K": K, "us": round(us, 3), "copies": copies,
                     "roofline": hbm_roofline(nb + 2 * K + 2 * N, us)}
        del mats
    return {"workload": "M=1 GEMV per projection shape, rotating over > 600 MB of distinct copies", "shapes": out}


_SAMPLING_LOGITS = []            # the logits bench_sampling used, for the CPU baseline
SAMPLING_CASES = (("temperature 0.7", (0.7, 0, 1.0)), ("temperature 0.7, top_k 50", (0.7, 50, 1.0)),
                  ("temperature 0.7, top_p 0.9", (0.7, 0, 0.9)),
                  ("temperature 0.7, top_k 50, top_p 0.9", (0.7, 50, 0.9)))


def bench_sampling(E, lm, norm_w, x0):
    """sample_token after the lm_head (src/sampling/sampler.cpp:18-39) on the
    248320 logits of one decode row, M=1 (mq4_sample_bf16 with its workspace:
    the chunked multi-workgroup path).  A short chain of small kernels, so the
    figure is latency; the bytes that bound it (one read of the logits) are
    given for scale."""
    torch, L, P = E.torch, E.L, E.P
    st = E.st()
    logits = torch.empty((1, VOCAB), dtype=torch.bfloat16, device=E.dev)
    idx = torch.zeros((1,), dtype=torch.int32, device=E.dev)
    wsb = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=E.dev)
    rc = L.mq4_rmsnorm_lm_head_argmax(P(x0.data_ptr()), 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                      P(idx.data_ptr()), P(logits.data_ptr()), P(ws.data_ptr()), wsb, st)
    assert rc == 0
    swb = L.mq4_sample_workspace_size(1, VOCAB)
    sws = torch.empty(swb, dtype=torch.uint8, device=E.dev)
    out = {}
    for name, (t, k, p) in SAMPLING_CASES:
        def f(t=t, k=k, p=p):
            L.mq4_sample_bf16(P(logits.data_ptr()), 1, VOCAB, ctypes.c_float(t), k, ctypes.c_float(p), 7,
                              P(idx.data_ptr()), None, P(sws.data_ptr()), swb, st)
        out[name] = {"us": round(E.timed(f, 200, warm=10), 2)}
    _SAMPLING_LOGITS[:] = [logits]
    return {"workload": "sample_token over 248320 bf16 logits, M=1", "logit_bytes": 2 * VOCAB, "cases": out,
            "note": "stream-ordered chain: chunk stats, top-k select, top-p mass passes, Gumbel-max "
                    "draw, final reduce (only the stages a case needs); HIP events around 200 back-to-back calls"}


def bench_pack(E, layers, lm):
    """Config 5b: quantize/pack of the full weight set (72 MLP matrices + the
    lm_head).  The bf16 weights are generated again (the same streams as the
    setup) and packed by mq4_quantize_batch (the loader's whole loop in three
    launches of at most 32 matrices), 5 passes back to back between one pair
    of HIP events (mean per pass, median of 3 such batches); the same 73
    matrices as 73 mq4_quantize calls are timed beside it the same way.  Both outputs must equal the setup's bit for bit.  The
    setup's per-matrix timings (an event pair and a synchronize around each
    call) are reported too."""
    torch, L, P, mq4 = E.torch, E.L, E.P, E.mq4
    srcs = [(mq4.fill_normal_bf16(shape, sid, 0.0, 0.02, device=E.dev), shape) for shape, sid in E.pack_set]

    def fresh():
        return [(torch.empty((N, K // 8), dtype=torch.int32, device=E.dev),
                 torch.empty((N, K // 64), dtype=torch.bfloat16, device=E.dev),
                 torch.empty((N, K // 64), dtype=torch.bfloat16, device=E.dev)) for _, (N, K) in srcs]

    st = E.st()
    ref = [q for lay in layers for q in lay] + [lm]

    def same_as_setup(outs):
        return all(torch.equal(o[0], r.wq) and torch.equal(o[1], r.s) and torch.equal(o[2], r.b)
                   for o, r in zip(outs, ref))

    outs = fresh()

    def pack_separate():
        for (w, (N, K)), (wq, s, b) in zip(srcs, outs):
            L.mq4_quantize(P(w.data_ptr()), N, K, 64, 4, P(wq.data_ptr()), P(s.data_ptr()), P(b.data_ptr()), st)

    us_sep = statistics.median([E.timed(pack_separate, 5, warm=1 if i == 0 else 0) for i in range(3)])
    same_sep = same_as_setup(outs)

    outs_b = fresh()
    jobs = (mq4._QuantJobC * len(srcs))()
    for i, ((w, (N, K)), (wq, s, b)) in enumerate(zip(srcs, outs_b)):
        jobs[i] = mq4._QuantJobC(w.data_ptr(), N, K, wq.data_ptr(), s.data_ptr(), b.data_ptr())
    jobs_p = ctypes.cast(jobs, ctypes.c_void_p)

    def pack_batch():
        mq4._check(L.mq4_quantize_batch(jobs_p, len(srcs), 64, 4, st))

    us = statistics.median([E.timed(pack_batch, 5, warm=1 if i == 0 else 0) for i in range(3)])
    same = same_as_setup(outs_b)
    del srcs, outs, outs_b
    return {"bytes": E.pack_bytes, "us": round(us, 1), "roofline": hbm_roofline(E.pack_bytes, us),
            "bit_identical_to_setup": bool(same and same_sep),
            "separate_calls_us": round(us_sep, 1),
            "separate_calls_roofline": hbm_roofline(E.pack_bytes, us_sep),
            "per_matrix_sum_us": round(E.pack_us, 1),
            "note": "read 2 B per bf16 weight + write 0.5625 B per weight (words, scales, biases); "
                    "mq4_quantize_batch over the 73 matrices (3 launches), 5 passes back to back between one "
                    "event pair (mean per pass, median of 3); separate_calls_us: the same 73 matrices as "
                    "73 mq4_quantize calls, timed the same way"}


# ----------------------------------------------------------- profile modes

def profile_mode(args, E, layers, lm, norm_w, layer_norms, x0, dstep, dargs):
    """Run one workload warmup + steps times for rocprofv3 (no JSON line)."""
    torch, L, P, mq4 = E.torch, E.L, E.P, E.mq4
    n = args.warmup + args.steps
    st = E.st()
    k = args.profile_kernel
    if k == "decode_step":
        for _ in range(n):
            L.mq4_decode_step(*dargs(st))
    elif k == "gemv_gate":
        y = torch.empty((1, INTER), dtype=torch.bfloat16, device=E.dev)
        mats = [g for g, u, d in layers] + [u for g, u, d in layers]
        for i in range(n):
            L.mq4_qmm(P(x0.data_ptr()), 1, HID, *mats[i % len(mats)].ptrs(), INTER, 1, 64, 4, P(y.data_ptr()), st)
    elif k == "lm_head":
        idx = torch.zeros((1,), dtype=torch.int32, device=E.dev)
        wsb = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
        ws = torch.zeros(wsb, dtype=torch.uint8, device=E.dev)
        for _ in range(n):
            L.mq4_rmsnorm_lm_head_argmax(P(x0.data_ptr()), 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                         P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st)
    elif k == "prefill":
        M = args.prefill_m
        g, u, d = layers[0]
        x = mq4.fill_normal_bf16((M, HID), mq4.STREAM_PREFILL, 0.0, 1.0, device=E.dev)
        h = torch.empty((M, INTER), dtype=torch.bfloat16, device=E.dev)
        y = torch.empty((M, HID), dtype=torch.bfloat16, device=E.dev)
        wsb = L.mq4_mlp_workspace_size(M, HID, INTER)
        ws = torch.empty(wsb, dtype=torch.uint8, device=E.dev)
        for _ in range(n):
            L.mq4_mlp_gate_up_silu(P(x.data_ptr()), M, HID, *g.ptrs(), *u.ptrs(), INTER, P(h.data_ptr()), st)
            L.mq4_qmm_residual(P(h.data_ptr()), M, INTER, *d.ptrs(), HID, P(x.data_ptr()), P(y.data_ptr()), st)
            # the same MLP half as one call (norm pre-pass, paired operands)
            L.mq4_mlp_residual(P(x.data_ptr()), M, HID, P(layer_norms[0].data_ptr()), 1e-6, *g.ptrs(), *u.ptrs(),
                               *d.ptrs(), INTER, P(ws.data_ptr()), wsb, P(y.data_ptr()), st)
    elif k == "batched":
        M = args.batched_m
        x = mq4.fill_normal_bf16((M, HID), 3000, 0.0, 1.0, device=E.dev)
        h = torch.empty((M, INTER), dtype=torch.bfloat16, device=E.dev)
        idx = torch.empty((M,), dtype=torch.int32, device=E.dev)
        wsb = L.mq4_lm_head_argmax_workspace_size(M, VOCAB)
        ws = torch.zeros(wsb, dtype=torch.uint8, device=E.dev)
        for _ in range(n):
            for l, (g, u, d) in enumerate(layers):
                L.mq4_rmsnorm_gate_up_silu(P(x.data_ptr()), M, HID, P(layer_norms[l].data_ptr()), EPS, *g.ptrs(),
                                           *u.ptrs(), INTER, P(h.data_ptr()), st)
                L.mq4_qmm_residual(P(h.data_ptr()), M, INTER, *d.ptrs(), HID, P(x.data_ptr()), P(x.data_ptr()), st)
            L.mq4_rmsnorm_lm_head_argmax(P(x.data_ptr()), M, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB,
                                         P(idx.data_ptr()), None, P(ws.data_ptr()), wsb, st)
    elif k == "pack":
        # the setup above packed the full weight set matrix by matrix; here the
        # same set goes through mq4_quantize_batch warmup + steps times
        srcs = [(mq4.fill_normal_bf16(shape, sid, 0.0, 0.02, device=E.dev), shape) for shape, sid in E.pack_set]
        jobs = (mq4._QuantJobC * len(srcs))()
        keep = []
        for i, (w, (N, K)) in enumerate(srcs):
            o = (torch.empty((N, K // 8), dtype=torch.int32, device=E.dev),
                 torch.empty((N, K // 64), dtype=torch.bfloat16, device=E.dev),
                 torch.empty((N, K // 64), dtype=torch.bfloat16, device=E.dev))
            keep.append(o)
            jobs[i] = mq4._QuantJobC(w.data_ptr(), N, K, o[0].data_ptr(), o[1].data_ptr(), o[2].data_ptr())
        for _ in range(n):
            mq4._check(L.mq4_quantize_batch(ctypes.cast(jobs, ctypes.c_void_p), len(srcs), 64, 4, st))
    torch.cuda.synchronize()
    log(f"[bench] profile {k}: {n} iterations")


# ------------------------------------------------------------ CPU baseline

def cpu_baseline(torch, layers, lm, x0, norm_w, layer_norms, reps, tok_gpu, configs):
    """The oracle's fp32-accumulating GEMV (OpenMP over rows) running the same
    decode step on the host cores, plus the literal MLX bf16 loop order on one
    thread over a one-layer sample; also CPU figures for the other configs
    (bounded samples), filed under each config's cpu_baseline."""
    import numpy as np
    O = load_oracle()
    log("[bench] cpu baseline: copying Q4 weights to host")
    hl = [tuple(host_q4(torch, q) for q in lay) for lay in layers]
    hlm = host_q4(torch, lm)
    xh = host_bf16(torch, x0)
    nw = host_bf16(torch, norm_w)
    lnw = [host_bf16(torch, t) for t in layer_norms]
    threads = O.omp_threads()

    def step():
        x = xh
        for (g, u, d), w in zip(hl, lnw):
            n = O.rmsnorm_1pw(x, w, EPS)
            h = O.swiglu_bf16(O.qmm_f32(n, *g), O.qmm_f32(n, *u))
            x = O.add_bf16(x, O.qmm_f32(h, *d))
        hn = O.rmsnorm_1pw(x, nw, EPS)
        return int(O.argmax_bf16(O.qmm_f32(hn, *hlm))[0])

    times = []
    tok = None
    for _ in range(reps):
        t = time.perf_counter()
        tok = step()
        times.append(time.perf_counter() - t)
    sec = statistics.median(times)
    # one-thread MLX-order sample: layer 0's three products
    g, u, d = hl[0]
    t = time.perf_counter()
    gm = O.qmm_mlx_bf16(xh, *g)
    um = O.qmm_mlx_bf16(xh, *u)
    O.qmm_mlx_bf16(O.swiglu_bf16(gm, um), *d)
    s1 = time.perf_counter() - t
    mlx_order_step_s = s1 * STEP_BYTES / W_MLP
    log(f"[bench] cpu fp32/OpenMP step {sec * 1e3:.1f} ms on {threads} threads (token {tok} vs GPU {tok_gpu}); "
        f"MLX-order 1-thread sample {s1 * 1e3:.0f} ms -> {mlx_order_step_s:.2f} s/step")

    def med(fn, r=3):
        ts = []
        for _ in range(r):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    extra = {}
    try:
        # config 1: one gate GEMV
        s_g = med(lambda: O.qmm_f32(xh, *hl[0][0]), 5)
        extra["config1_gemv_gate"] = {"value": round(q4_bytes(INTER, HID) / s_g / 1e9, 2), "unit": "GB/s",
                                      "us": round(s_g * 1e6, 1), "cores": threads, "kind": "port",
                                      "sample": "the oracle's fp32 GEMV, gate 6144x2048, M=1, median of 5"}
        # config 2 / 3: the MLP chain and the lm_head alone
        def mlp_only():
            x = xh
            for (g_, u_, d_), w in zip(hl, lnw):
                n = O.rmsnorm_1pw(x, w, EPS)
                x = O.add_bf16(x, O.qmm_f32(O.swiglu_bf16(O.qmm_f32(n, *g_), O.qmm_f32(n, *u_)), *d_))
        s_mlp = med(mlp_only, 3)
        extra["config2_mlp_chain"] = {"value": round(LAYERS * W_MLP / s_mlp / 1e9, 2), "unit": "GB/s",
                                      "us": round(s_mlp * 1e6, 1), "cores": threads, "kind": "port",
                                      "sample": "24 layers of the oracle's chain, median of 3"}
        s_lm = med(lambda: O.argmax_bf16(O.qmm_f32(O.rmsnorm_1pw(xh, nw, EPS), *hlm)), 3)
        extra["config3_lm_head_argmax"] = {"value": round(W_LM / s_lm / 1e9, 2), "unit": "GB/s",
                                           "us": round(s_lm * 1e6, 1), "cores": threads, "kind": "port",
                                           "sample": "norm + lm_head 248320x2048 + argmax, median of 3"}
        # config 4: prefill, a 64-row sample of M=2048 scaled
        xs = O.gen_normal_bf16(4000, 64 * HID).reshape(64, HID)
        s_p = med(lambda: O.qmm_f32(xs, *hl[0][0]), 2)
        tf = 2.0 * 64 * INTER * HID / s_p / 1e12
        extra["config4_prefill"] = {"value": round(tf, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
                                    "sample": "the oracle's fp32 product of 64 prefill rows with gate 6144x2048 "
                                              "(rate per matrix; the GEMM's rate does not depend on M here)"}
        # config 5a: batched M=16, one layer's MLP scaled to the step
        x16 = O.gen_normal_bf16(3000, 16 * HID).reshape(16, HID)
        s_b = med(lambda: O.qmm_f32(O.swiglu_bf16(O.qmm_f32(x16, *hl[0][0]), O.qmm_f32(x16, *hl[0][1])),
                                    *hl[0][2]), 2)
        extra["config5a_batched"] = {"value": round(W_MLP / s_b / 1e9, 2), "unit": "GB/s", "cores": threads,
                                     "kind": "port", "sample": "M=16 through layer 0's MLP (oracle fp32), "
                                                               "weight bytes / time"}
        # config 5b: pack, 4 MLP matrices of bf16 weights
        ws_ = [O.gen_normal_bf16(1000 + i, INTER * HID, 0.0, 0.02).reshape(INTER, HID) for i in range(4)]
        s_q = med(lambda: [O.quantize(w) for w in ws_], 2)
        nb = 4 * (2 * INTER * HID + q4_bytes(INTER, HID))
        extra["config5b_pack"] = {"value": round(nb / s_q / 1e9, 2), "unit": "GB/s", "cores": threads,
                                  "kind": "port", "sample": "the oracle's quantize of 4 gate-shaped matrices "
                                                            "(bytes read + written / time)"}
        # sampling: the oracle's masks (numpy sort-based, as the reference computes them)
        if "next_sampling" in configs and _SAMPLING_LOGITS:
            import importlib.util
            spec = importlib.util.spec_from_file_location("mq4_oracle_sampler",
                                                          os.path.join(ROOT, "oracle", "sampler.py"))
            Smp = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(Smp)
            lg = host_bf16(torch, _SAMPLING_LOGITS[0])
            s_s = med(lambda: Smp.keep_mask(lg, 0.7, 50, 0.9), 3)
            extra["next_sampling"] = {"value": round(s_s * 1e6, 1), "unit": "us", "cores": 1, "kind": "port",
                                      "sample": "oracle/sampler.py keep_mask (temperature 0.7, top_k 50, "
                                                "top_p 0.9) over the same 248320 logits, numpy, median of 3 "
                                                "(masks only, no draw)"}
    except Exception as e:
        traceback.print_exc()
        extra["error"] = f"{type(e).__name__}: {e}"
    for k, v in extra.items():
        if k in configs and isinstance(configs[k], dict):
            configs[k]["cpu_baseline"] = v
    return {
        "value": round(STEP_BYTES / sec / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "ms_per_step": round(sec * 1e3, 2),
        "sample": f"the full decode step (24 x [RMSNorm + MLP + residual], RMSNorm, lm_head, argmax), "
                  f"oracle fp32 accumulation with OpenMP over rows, median of {reps}",
        "token": tok,
        "mlx_order_1thread": {
            "value": round(STEP_BYTES / mlx_order_step_s / 1e9, 3), "unit": "GB/s", "cores": 1,
            "sample": "layer 0 gate+up+down in MLX's bf16-accumulating scalar loop order, "
                      "scaled by step bytes / layer bytes"},
    }


if __name__ == "__main__":
    main()
