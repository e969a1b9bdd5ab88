#!/usr/bin/env python3
"""Benchmark of the MLX-affine Q4 decode path on one MI355X.

Workload (one "step"): the per-token MLP + lm_head work of marlin-mlx's decode
loop at M = 1 (src/core/engine.cpp:79-94 -> src/model/marlin.cpp:110-145,
161-169 -> src/sampling/sampler.cpp:14-16):
    for each of 24 layers:  x = x + down(swiglu(gate n, up n)),  n = rms_norm_l(x)
    token = argmax(lm_head(rms_norm(x)))
with MLX affine Q4 group-64 weights (gate/up 6144x2048, down 2048x6144, tied
lm_head 248320x2048), bf16 activations, fp32 accumulation.  rms_norm is the
reference's (1 + w) RMSNorm (src/model/marlin.cpp:12-16, 141, 145), fused into
the gate/up and lm_head kernels; without it the 24-layer residual chain grows
quadratically and overflows bf16.  Weights are
synthetic N(0, 0.02) bf16 from the counter-based generator, quantized on the
GPU by this library's pack kernel (timed as well: the quantize/pack of the
full weight set).  The step is captured once in a HIP graph and replayed.

Output: one JSON line on stdout.  `value` is the step's algorithmic HBM
bandwidth, Q4 weight bytes per step (795,672,576 B) / step time.  Inputs are
resident in HBM before the timed region; the 796 MB weight stream is larger
than the 256 MB last-level cache, so every step reads the weights from HBM.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4 GEMV HBM GB/s (% of 8 TB/s peak); µs per decode-step MLP+lm_head"
HBM_PEAK_GBPS = 8000.0
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


# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (separate runs of
# `bench.py --profile-kernel decode_step`), each scaled by the same counter's reading for a
# 256 MiB device copy (FETCH x 1.99982, WRITE x 1.0); see profiles/decode_step_m1_hbm_traffic.md.
MEASURED_TRAFFIC = {"decode_step": 803_470_292 + 6_299_750}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--kernel-steps", type=int, default=10,
                   help="eager steps with per-kernel HIP events (roofline)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-reps", type=int, default=3)
    p.add_argument("--profile-kernel", choices=["decode_step", "copy"], default=None,
                   help="counter-collection mode: run only the one-launch decode step (warmup + steps "
                        "launches) or, to calibrate FETCH_SIZE/WRITE_SIZE, a plain device copy of "
                        "--copy-mib MiB per launch; prints no JSON line")
    p.add_argument("--copy-mib", type=int, default=256)
    return p.parse_args()


class Q4:
    """Device-resident MLX-layout Q4 matrix."""

    def __init__(self, wq, s, b, N, K):
        self.wq, self.s, self.b, self.N, self.K = wq, s, b, N, K

    def ptrs(self):
        return (ctypes.c_void_p(self.wq.data_ptr()), ctypes.c_void_p(self.s.data_ptr()),
                ctypes.c_void_p(self.b.data_ptr()))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU mode).", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    mq4 = __graft_entry__.load_package()
    L = mq4.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    P = ctypes.c_void_p

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
    pack_ms = 0.0
    pack_bytes = 0
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def make_q4(shape, stream_id):
        nonlocal pack_ms, pack_bytes
        N, K = shape
        w = mq4.fill_normal_bf16(shape, stream_id, 0.0, 0.02, device=dev)
        wq = torch.empty((N, K // 8), dtype=torch.int32, device=dev)
        s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=dev)
        b = torch.empty_like(s)
        st = P(torch.cuda.current_stream().cuda_stream)
        ev_a.record()
        mq4._check(L.mq4_quantize(P(w.data_ptr()), N, K, 64, 4, P(wq.data_ptr()), P(s.data_ptr()),
                                  P(b.data_ptr()), st))
        ev_b.record()
        torch.cuda.synchronize()
        pack_ms += ev_a.elapsed_time(ev_b)
        pack_bytes += 2 * N * K + q4_bytes(N, K)
        del w
        return Q4(wq, s, b, N, K)

    layers = []
    for l in range(LAYERS):
        layers.append((make_q4((INTER, HID), mq4.stream_id_layer(l, 0)),
                       make_q4((INTER, HID), mq4.stream_id_layer(l, 1)),
                       make_q4((HID, INTER), mq4.stream_id_layer(l, 2))))
    lm = make_q4((VOCAB, HID), mq4.STREAM_LM_HEAD)
    norm_w = mq4.fill_normal_bf16((HID,), mq4.STREAM_NORM_WEIGHT, 0.1, 0.02, device=dev)
    layer_norms = [mq4.fill_normal_bf16((HID,), mq4.stream_id_layer_norm(l), 0.1, 0.02, device=dev)
                   for l in range(LAYERS)]
    x0 = mq4.fill_normal_bf16((1, HID), mq4.stream_id_decode_row(0), 0.0, 1.0, device=dev)
    torch.cuda.synchronize()
    log(f"[bench] pack: {pack_bytes} B in {pack_ms * 1e3:.1f} us "
        f"({pack_bytes / pack_ms / 1e6:.1f} GB/s)")

    x = torch.empty((1, HID), dtype=torch.bfloat16, device=dev)
    hbuf = torch.empty((1, INTER), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((1,), dtype=torch.int32, device=dev)
    ws_bytes = L.mq4_lm_head_argmax_workspace_size(1, VOCAB)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)     # zero once (arrival counters)

    # Launch list of one step: (kind, callable(stream)).
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
                        lambda st, xin=xin, d=d: L.mq4_qmm_residual(
                            hp, 1, INTER, *d.ptrs(), HID, xin, xp, st)))
        out.append(("norm_lm_head_argmax", lambda st: L.mq4_rmsnorm_lm_head_argmax(
            xp, 1, HID, P(norm_w.data_ptr()), EPS, *lm.ptrs(), VOCAB, P(idx.data_ptr()), None,
            P(ws.data_ptr()), ws_bytes, st)))
        return out

    steps = launches()

    if args.profile_kernel == "decode_step":
        qt = lambda q: mq4.QuantizedTensor(q.wq, q.s, q.b)
        dec_layers = [mq4.DecoderLayer(layer_norms[l], mq4.MLPWeights(qt(g), qt(u), qt(d)))
                      for l, (g, u, d) in enumerate(layers)]
        dstep = mq4.DecodeStep(dec_layers, norm_w, qt(lm), EPS)
        idx_p = torch.zeros((1,), dtype=torch.int32, device=dev)
        for _ in range(args.warmup + args.steps):
            dstep(x0, None, idx_p)
        torch.cuda.synchronize()
        log(f"[bench] decode_step: {args.warmup + args.steps} launches, token {int(idx_p.item())}")
        return

    def run_step(st):
        for _, fn in steps:
            rc = fn(st)
            if rc != 0:
                mq4._check(rc)

    # ------------------------------------------------ eager check + graph
    run_step(P(torch.cuda.current_stream().cuda_stream))
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
        run_step(P(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.warmup} graph replays); timing {args.steps} steps")
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    tok_graph = int(idx.item())
    if tok_graph != tok_eager:
        raise RuntimeError(f"graph replay token {tok_graph} != eager token {tok_eager}")
    gbps = STEP_BYTES / (ms_step * 1e-3) / 1e9
    log(f"[bench] step {ms_step * 1e3:.1f} us, {gbps:.0f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of "
        f"8 TB/s), token {tok_graph}")

    # ---------------------------------------- per-kernel HIP-event timing
    # Each kernel kind is launched back to back (its launches from the step in
    # order, `--kernel-steps` times over, so weights rotate through all layers
    # and stay cold) between one pair of HIP events on the stream the kernels
    # run on; the mean is the batch time over the launch count.  Event pairs
    # around single launches would add several microseconds of event overhead
    # per launch.
    st = P(torch.cuda.current_stream().cuda_stream)
    nk = args.kernel_steps
    kinds = []
    for kind, _ in steps:
        if kind not in kinds:
            kinds.append(kind)
    kernels = {}
    for kind in kinds:
        fns = [fn for k, fn in steps if k == kind]
        for fn in fns:                     # warm the launch path
            fn(st)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(nk):
            for fn in fns:
                fn(st)
        e1.record()
        torch.cuda.synchronize()
        n = nk * len(fns)
        mean_us = e0.elapsed_time(e1) * 1e3 / n
        kernels[kind] = {
            "mean_us": round(mean_us, 3),
            "launches_per_step": len(fns),
            "us_per_step": round(mean_us * len(fns), 2),
            "bytes_per_launch": KERNEL_BYTES[kind],
            "GBps": round(KERNEL_BYTES[kind] / (mean_us * 1e-6) / 1e9, 1),
        }
    dom = max(kernels, key=lambda k: kernels[k]["us_per_step"])
    for k, v in kernels.items():
        log(f"[bench] kernel {k}: {v}")
    dk = kernels[dom]
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": dk["GBps"],
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(dk["GBps"] / HBM_PEAK_GBPS, 4),
        "traffic": MEASURED_TRAFFIC.get(dom),
    }

    # ------------------------------------ the whole step in one launch
    # DecodeStep runs the same step as one persistent kernel (same arithmetic,
    # so the same token and hidden state as the separate kernels above).
    qt = lambda q: mq4.QuantizedTensor(q.wq, q.s, q.b)
    dec_layers = [mq4.DecoderLayer(layer_norms[l], mq4.MLPWeights(qt(g), qt(u), qt(d)))
                  for l, (g, u, d) in enumerate(layers)]
    dstep = mq4.DecodeStep(dec_layers, norm_w, qt(lm), EPS)
    idx_p = torch.zeros((1,), dtype=torch.int32, device=dev)
    x_p = torch.empty((HID,), dtype=torch.bfloat16, device=dev)
    run_step(P(torch.cuda.current_stream().cuda_stream))   # x, idx: the separate kernels' result
    dstep(x0, x_p, idx_p)
    torch.cuda.synchronize()
    tok_p = int(idx_p.item())
    if tok_p != tok_eager or not torch.equal(x_p.view(torch.int16), x.reshape(-1).view(torch.int16)):
        raise RuntimeError(f"one-launch decode step disagrees with the separate kernels "
                           f"(token {tok_p} vs {tok_eager})")
    pgraph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dstep(x0, None, idx_p)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(pgraph):
        dstep(x0, None, idx_p)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        pgraph.replay()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        pgraph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_step_p = t0.elapsed_time(t1) / args.steps
    if int(idx_p.item()) != tok_eager:
        raise RuntimeError("one-launch decode step: graph replay token differs")
    log(f"[bench] one-launch step {ms_step_p * 1e3:.1f} us, "
        f"{STEP_BYTES / (ms_step_p * 1e-3) / 1e9:.0f} GB/s")
    # kernel duration: back-to-back launches between HIP events on the launch stream
    st = P(torch.cuda.current_stream().cuda_stream)
    lay_c = dstep._arr
    dargs = (P(x0.data_ptr()), HID, INTER, LAYERS, ctypes.cast(lay_c, P), P(norm_w.data_ptr()), EPS,
             *lm.ptrs(), VOCAB, P(idx_p.data_ptr()), None, P(dstep.workspace.data_ptr()), dstep.ws_bytes, st)
    mq4._check(L.mq4_decode_step(*dargs))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(args.kernel_steps * 5, 10)
    e0.record()
    for _ in range(n):
        L.mq4_decode_step(*dargs)
    e1.record()
    torch.cuda.synchronize()
    mean_us = e0.elapsed_time(e1) * 1e3 / n
    kernels["decode_step"] = {
        "mean_us": round(mean_us, 3),
        "launches_per_step": 1,
        "us_per_step": round(mean_us, 2),
        "bytes_per_launch": KERNEL_BYTES["decode_step"],
        "GBps": round(KERNEL_BYTES["decode_step"] / (mean_us * 1e-6) / 1e9, 1),
    }
    log(f"[bench] kernel decode_step: {kernels['decode_step']}")
    sep = {"us_per_step": round(ms_step * 1e3, 2), "GBps": round(gbps, 1),
           "note": "the same step as 49 separate kernels (24 x [norm+gate/up+SiLU, down+residual], "
                   "norm+lm_head+argmax, argmax finalize) replayed from one HIP graph"}
    if ms_step_p < ms_step:
        ms_step, gbps = ms_step_p, STEP_BYTES / (ms_step_p * 1e-3) / 1e9
        dom = "decode_step"
    dk = kernels[dom]
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": dk["GBps"],
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(dk["GBps"] / HBM_PEAK_GBPS, 4),
        "traffic": MEASURED_TRAFFIC.get(dom),
    }

    # ------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(torch, layers, lm, x0, norm_w, layer_norms, args.cpu_reps, tok_eager)

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
            "pct_of_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "separate_kernels": sep,
        "path": "one-launch decode step" if dom == "decode_step" else "separate kernels",
        "pack": {"bytes": pack_bytes, "us": round(pack_ms * 1e3, 1),
                 "GBps": round(pack_bytes / pack_ms / 1e6, 1),
                 "frac": round(pack_bytes / pack_ms / 1e6 / HBM_PEAK_GBPS, 4),
                 "note": "quantize/pack of the full weight set (72 MLP matrices + lm_head), "
                         "sum of per-matrix HIP-event times"},
        "token": tok_graph,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(torch, layers, lm, x0, norm_w, layer_norms, reps, tok_gpu):
    """The oracle's fp32-accumulating GEMV (OpenMP over rows) running the same
    decode step on the host cores, plus the literal MLX bf16 loop order on one
    thread over a one-layer sample."""
    import numpy as np
    import importlib.util
    spec = importlib.util.spec_from_file_location("mq4_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    O = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(O)

    def host(q):
        return (q.wq.cpu().numpy().view(np.uint32), q.s.cpu().view(torch.int16).numpy().view(np.uint16),
                q.b.cpu().view(torch.int16).numpy().view(np.uint16))

    log("[bench] cpu baseline: copying Q4 weights to host")
    hl = [tuple(host(q) for q in lay) for lay in layers]
    hlm = host(lm)
    xh = x0.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    nw = norm_w.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    lnw = [t.cpu().view(torch.int16).numpy().view(np.uint16).copy() for t in layer_norms]

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
    threads = O.omp_threads()
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
