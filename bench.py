#!/usr/bin/env python3
"""Benchmark of the MI355X KDA operator path (one GPU).

Default workload: one KDA layer forward+backward in bf16 with f32
state and gates, B=2, T=4096, H=3, K=V=128, chunk 64, seed 42; q,k L2-normalised from
N(0,1), v ~ N(0,1), beta logits ~ N(0,1), g = -exp(A_log) softplus(N(0,1) + dt_bias) with
A_log ~ U(-1,1), dt_bias = 0, upstream gradient ~ N(0,1) bf16.  All inputs are resident
in HBM before the timed region.  A "step" is one forward+backward of the operator,
captured once as a HIP graph and replayed (ms_per_step_eager: the same step issued from
Python autograd, which depends on the host's speed).

Prints ONE JSON line: value = algorithmic TFLOP/s of the KDA core (13.388 GFLOP per layer
forward+backward), ms_per_step = ms per layer forward+backward, plus the forward-only
time, the K3-gate variant, per-kernel times, the roofline of the dominant kernel and the
CPU baseline (the reference's eager f32 path restated, timed on the host).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

# Algorithmic FLOPs per (64-token chunk, head) at K = V = 128 (C = 64):
#   forward = 11,621,717;  backward := 2 x forward.
FWD_FLOP_PER_TILE = 11_621_717
# per-kernel algorithmic FLOPs per tile (sum of the products each kernel owns)
KERNEL_FLOP_PER_TILE = {
    "fwd_intra": 3 * 1_048_576 + 1_048_576 + 87_381,   # A, M', W (2C^2K), U (2C^2V), solve C^3/3
    "fwd_scan": 2 * 2_097_152,                         # W S, Kd^T delta (2CKV)
    "fwd_output": 2_097_152 + 1_048_576,               # Qg S (2CKV), A delta (2C^2V)
    "bwd_scan": 3 * 2_097_152 + 1_048_576,             # Kd dS', Qg^T dO, W^T dDelta, A^T dO
    "bwd_dense": 3 * 2_097_152 + 5 * 1_048_576 + 4 * 262_144,  # dQg dKd dW; dA dT(2) dVb dKb; Y dM
    "bwd_decay": 4 * 1_048_576,                        # row/column terms of A and M'
}
# the staged backward launches the dense and decay roles as one kernel
KERNEL_FLOP_PER_TILE["bwd_dense_decay"] = KERNEL_FLOP_PER_TILE["bwd_dense"] + KERNEL_FLOP_PER_TILE["bwd_decay"]
# the whole backward (one call) is one fused launch of scan members and dense+decay tiles
KERNEL_FLOP_PER_TILE["bwd_fused"] = KERNEL_FLOP_PER_TILE["bwd_scan"] + KERNEL_FLOP_PER_TILE["bwd_dense_decay"]
# kernels one fwd+bwd step launches (the other entries time one stage alone)
STEP_KERNELS = ("fwd_intra", "fwd_scan", "fwd_output", "bwd_fused")
STAGES = {"fwd_intra": 1, "fwd_scan": 2, "fwd_output": 3, "bwd_scan": 10, "bwd_dense": 11, "bwd_decay": 12,
          "bwd_dense_decay": 14, "bwd_fused": None}
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
# the backward's compulsory HBM I/O at config 2 with the precomputed gate: q, k, v, dO bf16,
# g f32 and beta bf16 in; dq, dk, dv bf16, dg f32 and dbeta bf16 out (the secondary bytes
# figure of the dominant kernel)
BWD_COMPULSORY_BYTES = 4 * 6_291_456 + 12_582_912 + 49_152 + 3 * 6_291_456 + 12_582_912 + 49_152


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true", help="skip the 6-layer training throughput")
    ap.add_argument("--train-only", action="store_true",
                    help="print only the 6-layer training throughput (3 graphed updates) and exit")
    ap.add_argument("--hbm-sweep", action="store_true",
                    help="print the HBM-peak fraction of conv / norm-gate / copy over batch sizes and exit")
    ap.add_argument("--hbm-kernels", action="store_true",
                    help="print only the conv / norm-gate / decode HBM figures and exit")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="print the bf16 MFMA rate kda_mfma_probe sustains on this device and exit")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run each kernel once (plus a 64 MiB calibration copy) for rocprofv3 --pmc; no timing")
    ap.add_argument("--cpu-sample-len", type=int, default=1024,
                    help="T of the CPU baseline sample (extrapolated linearly to T=4096)")
    return ap.parse_args()


def make_inputs(torch, B=2, T=4096, H=3, K=128, V=128, seed=42, gate="precomputed"):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    v = torch.randn(B, T, H, V, generator=g)
    z = torch.randn(B, T, H, K, generator=g)
    beta = torch.randn(B, T, H, generator=g)
    A_log = torch.rand(H, generator=g) * 2 - 1
    dt_bias = torch.zeros(H * K)
    do = torch.randn(B, T, H, V, generator=g)
    if gate == "precomputed":
        gv = (-A_log.exp().view(1, 1, H, 1) * torch.nn.functional.softplus(z + dt_bias.view(1, 1, H, K))).float()
    else:  # reference Level-1 inputs: K3 gate, raw ~ N(0,1), A_log = dt_bias = 0
        gv = z.bfloat16()
        A_log = torch.zeros(H)
    dev = "cuda"
    t = dict(q=q.bfloat16(), k=k.bfloat16(), v=v.bfloat16(), g=gv, beta=beta.bfloat16(),
             A_log=A_log.float(), dt_bias=dt_bias.float())
    t = {n: x.to(dev).requires_grad_(True) for n, x in t.items()}
    return t, do.bfloat16().to(dev)


def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_graph_steps(torch, fn, steps, warmup):
    """Per-step time (ms) of fn captured once in a HIP graph and replayed: the same kernels
    as the eager step, issued by one host call per step, so the figure does not depend on
    the box's host speed.  Warm-up runs on a side stream before capture, as capture needs."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return time_steps(torch, graph.replay, steps, warmup)


def kernel_times(torch, t, do, gate, reps=20):
    """Average duration (ms) of each chunk kernel, launched alone on the current stream
    between HIP events, after a full forward+backward has prepared its buffers."""
    from experiment_swa_kda_amd import _lib, ops
    from experiment_swa_kda_amd._lib import ptr

    d = {n: x.detach() for n, x in t.items()}
    K = d["q"].shape[-1]
    out, fin, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                     None, False, -5.0, K ** -0.5, gate=gate)
    p = ops._problem(d["q"], d["v"], None, ops.GATE_MODES[gate], -5.0, K ** -0.5)
    lib = _lib.load()
    scratch = torch.empty(lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p)), dtype=torch.uint8, device="cuda")
    grads = [torch.empty_like(d[n]) for n in ("q", "k", "v", "g", "beta")]
    dA = torch.empty_like(d["A_log"])
    ddt = torch.empty_like(d["dt_bias"])
    stream = torch.cuda.current_stream().cuda_stream
    fargs = (ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(d["g"]), ptr(d["beta"]), ptr(d["A_log"]),
             ptr(d["dt_bias"]), None, ptr(out), None, ptr(ws), stream)
    bargs = (ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(d["g"]), ptr(d["beta"]), ptr(d["A_log"]),
             ptr(d["dt_bias"]), None, ptr(ws), ptr(do), None, *[ptr(x) for x in grads], ptr(dA), ptr(ddt),
             None, ptr(scratch), stream)
    _lib.check(lib.kda_chunk_backward(ctypes.byref(p), *bargs), "chunk_backward")
    res = {}
    for name, stage in STAGES.items():
        if stage is None:  # the full backward: the scheduling launch + the fused launch
            call = lambda: lib.kda_chunk_backward(ctypes.byref(p), *bargs)  # noqa: E731
        elif stage < 10:
            call = lambda: lib.kda_chunk_forward_stage(stage, ctypes.byref(p), *fargs)  # noqa: E731
        else:
            call = lambda: lib.kda_chunk_backward_stage(stage, ctypes.byref(p), *bargs)  # noqa: E731
        _lib.check(call(), name)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            call()
        e.record()
        torch.cuda.synchronize()
        res[name] = s.elapsed_time(e) / reps
    return res


def mfma_probe(torch, shape=0, iters=20000, per_cu=8):
    """bf16 MFMA rate that kda_mfma_probe sustains (shape 0: 16x16x32, the chunk kernels'
    shape; 1: 32x32x16), best of three launches timed between HIP events on the launch
    stream, with the sustained shader clock and cycles per MFMA from workgroup 0's counters."""
    from experiment_swa_kda_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs = per_cu * cus
    sink = torch.zeros(wgs + 2, device=dev)
    flop = ctypes.c_double()
    stream = torch.cuda.current_stream()
    for _ in range(2):
        _lib.check(lib.kda_mfma_probe(shape, wgs, iters, sink.data_ptr(), ctypes.byref(flop), stream.cuda_stream),
                   "kda_mfma_probe")
    best = 0.0
    for _ in range(3):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        lib.kda_mfma_probe(shape, wgs, iters, sink.data_ptr(), ctypes.byref(flop), stream.cuda_stream)
        end.record(stream)
        end.synchronize()
        best = max(best, flop.value / (start.elapsed_time(end) * 1e-3) / 1e12)
    cyc, ticks = sink[:2].tolist()
    clock_ghz = cyc / ticks * 0.1 if ticks > 0 else None
    return {"tflops": round(best, 1), "shape": "16x16x32" if shape == 0 else "32x32x16",
            "workgroups": wgs, "waves_per_simd": per_cu,
            "wg0_clock_ghz": None if clock_ghz is None else round(clock_ghz, 3)}


def mfma_peak_measured(torch):
    """The measured bf16 MFMA peak (TFLOP/s): the larger of the two probe shapes' rates
    (32x32x16 sustains more than 16x16x32, the chunk kernels' shape), so the fraction
    against it is the conservative one; both rates are returned."""
    r = {s: mfma_probe(torch, s, per_cu=4)["tflops"] for s in (0, 1)}
    return max(r.values()), r


def train_throughput(torch, updates=5, warmup=2, accum=4, seed=42, graphed=True):
    """6-layer all-KDA decoder, d_model 384, H3 D128, vocab 32768,
    B2 T4096, 4 gradient-accumulation microsteps per update (32,768 tokens), uniform
    random token ids, AdamW update.  Returns tokens/s as the median over the timed
    updates (the reference scores the median of steps 2-6, docs/BENCHMARK.md:33-36).
    graphed: the whole update (4 x forward + backward, optimizer step) is one HIP graph
    replay (model.GraphedUpdate); otherwise every op is dispatched eagerly."""
    from experiment_swa_kda_amd.model import GPT, GPTConfig, GraphedUpdate, make_optimizer, use_tuned_gemms

    tuned = use_tuned_gemms()  # recorded library-GEMM solutions for the trainer's shapes
    torch.manual_seed(seed)
    cfg = GPTConfig(sequence_len=4096, vocab_size=32768, n_layer=6, n_head=3, n_embd=384)
    model = GPT(cfg).cuda()
    model.init_weights()
    opt = make_optimizer(model, capturable=graphed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, T = 2, 4096
    data = [torch.randint(0, cfg.vocab_size, (B, T + 1), device="cuda", generator=g) for _ in range(accum)]

    if graphed:
        step = GraphedUpdate(model, opt, data, warmup=warmup)
        update = step
        warmup = 1
    else:
        def update():
            for mb in data:
                loss = model(mb[:, :-1], mb[:, 1:]) / accum
                loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            return loss * accum

    times = []
    for i in range(warmup + updates):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loss = update()
        torch.cuda.synchronize()
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    return {"tok_per_s": round(B * T * accum / (ms * 1e-3), 1), "ms_per_update": round(ms, 3),
            "tokens_per_update": B * T * accum, "updates_timed": updates,
            "loss": round(float(loss.detach()), 4), "optimizer": "AdamW",
            "execution": "hip_graph" if graphed else "eager",
            "gemm_selection": "tuned" if tuned else "library default", "reference_gb10_tok_per_s": 44942}


def load_mfma_busy():
    """MFMA-busy fraction per chunk kernel from the committed rocprofv3 --pmc summary
    (SQ_VALU_MFMA_BUSY_CYCLES over dispatch cycles x 1024 SIMDs), or {}."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mfma_util_config2.txt")
    out = {}
    if os.path.exists(path):
        for line in open(path):
            if line.startswith("#") or not line.strip():
                continue
            f = line.split()
            out[f[0]] = float(f[-1])
    return out


def load_traffic():
    """HBM bytes per dispatch from the committed rocprofv3 --pmc summary, or {}."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_config2.txt")
    out = {}
    if os.path.exists(path):
        for line in open(path):
            if line.startswith("#") or not line.strip():
                continue
            name, fb, wb = line.split()[:3]
            out[name] = int(fb) + int(wb)
    return out


def graph_time_us(torch, fn, n=50, reps=5):
    """Per-call GPU time of fn (microseconds): n calls captured in one HIP graph, replayed
    between events, so host launch overhead is excluded."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(n):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (n * reps)


def hbm_kernels(torch):
    """Conv+SiLU, RMSNorm*gate (config 2 shapes) and the decode step (config 3): per-call
    time, compulsory HBM bytes and the fraction of the 8 TB/s HBM peak."""
    from experiment_swa_kda_amd import ops

    g = torch.Generator(device="cuda").manual_seed(42)
    out = {}

    def rec(name, us, nbytes, n_copy=50):
        gbs = nbytes / (us * 1e-6) / 1e9
        # a plain device copy moving the same bytes (half read, half written), timed the same way
        src = torch.empty(nbytes // 2 // 16 * 16, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        cus = graph_time_us(torch, lambda: dst.copy_(src), n=n_copy)
        copy_gbs = 2 * src.numel() / (cus * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "bytes": int(nbytes), "GB_per_s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                     "copy_same_bytes_frac_hbm_peak": round(copy_gbs / PEAK_HBM_GBS, 4),
                     "ratio_to_copy": round(gbs / copy_gbs, 3)}

    B, T, C, W = 2, 4096, 384, 4
    x = torch.randn(B, T, C, device="cuda", generator=g).bfloat16()
    w = torch.randn(C, W, device="cuda", generator=g).bfloat16()
    dy = torch.randn(B, T, C, device="cuda", generator=g).bfloat16()
    rec("conv_fwd", graph_time_us(torch, lambda: ops.causal_conv_forward(x, w, None, False)), 2 * x.numel() * 2)
    rec("conv_bwd", graph_time_us(torch, lambda: ops.causal_conv_backward(x, w, None, dy, None)), 3 * x.numel() * 2)
    # the trainer's launch: the three projections' 1,152 channels read in place from the
    # packed projection output (row stride 2312 columns) and dx written back into its columns
    ld = 2312
    packed = torch.randn(B, T, ld, device="cuda", generator=g).bfloat16()
    w3 = torch.randn(3 * C, W, device="cuda", generator=g).bfloat16()
    dy3 = torch.randn(B, T, 3 * C, device="cuda", generator=g).bfloat16()
    dxp = torch.zeros_like(packed)
    xs, dxs = packed[..., :3 * C], dxp[..., :3 * C]
    rec("conv_bwd_trainer_3proj", graph_time_us(
        torch, lambda: ops.causal_conv_backward(xs, w3, None, dy3, None, dx_out=dxs)), 3 * B * T * 3 * C * 2)
    o = torch.randn(B, T, 3, 128, device="cuda", generator=g).bfloat16()
    gt = torch.randn(B, T, 3, 128, device="cuda", generator=g).bfloat16()
    nw = torch.ones(128, device="cuda")
    _, inv = ops.rmsnorm_gate_forward(o, gt, nw, 1e-5)
    rows = B * T * 3
    rec("norm_gate_fwd", graph_time_us(torch, lambda: ops.rmsnorm_gate_forward(o, gt, nw, 1e-5)),
        3 * o.numel() * 2 + rows * 4)
    rec("norm_gate_bwd", graph_time_us(torch, lambda: ops.rmsnorm_gate_backward(o, gt, nw, inv, dy.view_as(o), 1e-5)),
        5 * o.numel() * 2 + rows * 4)
    # decode (config 3): B64 H3 D128, f32 state updated in place
    Bd, H, D = 64, 3, 128
    q, k, raw = (torch.randn(Bd, 1, H, D, device="cuda", generator=g).bfloat16() for _ in range(3))
    v = torch.randn(Bd, 1, H, D, device="cuda", generator=g).bfloat16()
    bl = torch.randn(Bd, 1, H, device="cuda", generator=g).bfloat16()
    A_log = torch.zeros(H, device="cuda")
    dt = torch.zeros(H * D, device="cuda")
    state = torch.randn(Bd, H, D, D, device="cuda", generator=g) * 0.05
    us = graph_time_us(torch, lambda: ops.recurrent_decode(q, k, v, raw, bl, A_log, dt, state, True, -5.0,
                                                           D ** -0.5, out_state=state), n=256, reps=3)
    rec("decode_step", us, 2 * state.numel() * 4 + (4 * q.numel() + bl.numel()) * 2)
    out["decode_step"]["config"] = "config3: B64 H3 D128, one token per step, 256 steps in one graph, state in place"
    return out


def hbm_sweep(torch, batches=(2, 4, 8, 16, 32)):
    """Fraction of the HBM peak reached by conv, RMSNorm*gate and a plain copy of the same
    bytes as the batch grows (T = 4096, C = 384): separates launch / ramp cost from kernel
    efficiency.  One JSON line per batch."""
    from experiment_swa_kda_amd import ops

    g = torch.Generator(device="cuda").manual_seed(42)
    for B in batches:
        T, C, W = 4096, 384, 4
        x = torch.randn(B, T, C, device="cuda", generator=g).bfloat16()
        w = torch.randn(C, W, device="cuda", generator=g).bfloat16()
        dy = torch.randn(B, T, C, device="cuda", generator=g).bfloat16()
        o, gt = x.view(B, T, 3, 128), dy.view(B, T, 3, 128)
        nw = torch.ones(128, device="cuda")
        _, inv = ops.rmsnorm_gate_forward(o, gt, nw, 1e-5)
        c = torch.empty_like(x)
        n = x.numel() * 2
        cases = {
            "conv_fwd": (2 * n, lambda: ops.causal_conv_forward(x, w, None, False)),
            "conv_bwd": (3 * n, lambda: ops.causal_conv_backward(x, w, None, dy, None)),
            "norm_gate_fwd": (3 * n, lambda: ops.rmsnorm_gate_forward(o, gt, nw, 1e-5)),
            "norm_gate_bwd": (5 * n, lambda: ops.rmsnorm_gate_backward(o, gt, nw, inv, gt, 1e-5)),
            "copy": (2 * n, lambda: c.copy_(x)),
        }
        line = {"batch": B}
        for name, (nbytes, fn) in cases.items():
            line[name] = round(nbytes / (graph_time_us(torch, fn, n=20) * 1e-6) / 1e9 / PEAK_HBM_GBS, 3)
        print(json.dumps(line), flush=True)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sample_len):
    """The reference's eager f32 CPU path (restated in oracle/reference_path.py), fwd+bwd,
    on every host core: config 1 in full, and a config-2 sample of length ``sample_len``
    (B2 H3 D128) extrapolated linearly in T to 4096 (the loop is sequential in T)."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.reference_path import time_fwd_bwd

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    ms_c1 = time_fwd_bwd(1, 256, 2, 64, 64, repeats=5) * 1e3
    sec = time_fwd_bwd(2, sample_len, 3, 128, 128, repeats=3)
    ms_full = sec * 1e3 * (4096 / sample_len)
    flop = 384 * 3 * FWD_FLOP_PER_TILE
    return {"value": round(flop / (ms_full * 1e-3) / 1e12, 6), "unit": "TFLOP/s", "cores": cores,
            "kind": "port", "cpu_model": _cpu_model(), "ms_per_layer_fwd_bwd": round(ms_full, 1),
            "config1_ms_fwd_bwd": round(ms_c1, 2),
            "sample": f"eager f32 token loop + autograd on {cores} threads: config 1 (B1 T256 H2 D64) in full, "
                      f"median of 5; config 2 as B2 H3 D128 T={sample_len} fwd+bwd, median of 3, "
                      f"extrapolated linearly to T=4096 (value)"}


def pmc_workload(torch):
    """One launch of every kernel of the path at config 2/3 shapes, preceded by a copy of
    known size (64 MiB read + 64 MiB written) that calibrates FETCH_SIZE / WRITE_SIZE."""
    from experiment_swa_kda_amd import kda, ops

    src = torch.ones(32 * 1024 * 1024, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    t, do = make_inputs(torch, gate="precomputed")
    out, _ = kda(t["q"], t["k"], t["v"], t["g"], t["beta"], t["A_log"], t["dt_bias"], mode="project_chunk",
                 gate="precomputed", allow_fallback=False)
    out.backward(do)
    torch.cuda.synchronize()
    g = torch.Generator(device="cuda").manual_seed(1)
    x, dy, gt = (torch.randn(2, 4096, 384, device="cuda", generator=g).bfloat16() for _ in range(3))
    w = torch.randn(384, 4, device="cuda", generator=g).bfloat16()
    ops.causal_conv_forward(x, w, None, False)
    ops.causal_conv_backward(x, w, None, dy, None)
    o, gto, dyo = (t.view(2, 4096, 3, 128) for t in (x, gt, dy))
    _, inv = ops.rmsnorm_gate_forward(o, gto, torch.ones(128, device="cuda"), 1e-5)
    ops.rmsnorm_gate_backward(o, gto, torch.ones(128, device="cuda"), inv, dyo, 1e-5)
    q = torch.randn(64, 1, 3, 128, device="cuda", generator=g).bfloat16()
    st = torch.randn(64, 3, 128, 128, device="cuda", generator=g)
    ops.recurrent_decode(q, q, q, q, q[..., 0], torch.zeros(3, device="cuda"), torch.zeros(384, device="cuda"),
                         st, True, -5.0, 128 ** -0.5, out_state=st)
    torch.cuda.synchronize()
    print("pmc workload done", flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the KDA operator path is benchmarked on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    from experiment_swa_kda_amd import kda

    if args.pmc_workload:
        pmc_workload(torch)
        return
    if args.hbm_kernels:
        print(json.dumps(hbm_kernels(torch)), flush=True)
        return
    if args.train_only:
        print(json.dumps(train_throughput(torch, updates=3, warmup=1)), flush=True)
        return
    if args.mfma_probe:
        for shape in (0, 1):
            for per_cu in (4, 8):
                print(json.dumps(dict(mfma_probe(torch, shape, per_cu=per_cu),
                                      peak_published_tflops=PEAK_BF16_TFLOPS)), flush=True)
        return
    if args.hbm_sweep:
        hbm_sweep(torch)
        return
    B, T, H, K, V = 2, 4096, 3, 128, 128
    tiles = B * (T // 64) * H
    flop = 3 * tiles * FWD_FLOP_PER_TILE  # fwd + bwd (bwd := 2 x fwd)

    results = {}
    for gate in ("precomputed", "k3"):
        t, do = make_inputs(torch, gate=gate)

        def step():
            for x in t.values():
                x.grad = None
            out, _ = kda(t["q"], t["k"], t["v"], t["g"], t["beta"], t["A_log"], t["dt_bias"],
                         mode="project_chunk", gate=gate, allow_fallback=False)
            out.backward(do)

        def fwd():
            with torch.no_grad():
                kda(t["q"], t["k"], t["v"], t["g"], t["beta"], t["A_log"], t["dt_bias"],
                    mode="project_chunk", gate=gate, allow_fallback=False)

        torch.cuda.synchronize()
        ms_eager = time_steps(torch, step, args.steps, args.warmup)
        ms = time_graph_steps(torch, step, args.steps, args.warmup)
        ms_fwd = time_graph_steps(torch, fwd, args.steps, args.warmup)
        results[gate] = (ms, ms_fwd, t, do, ms_eager)

    ms, ms_fwd, t, do, ms_eager = results["precomputed"]
    kt = kernel_times(torch, t, do, "precomputed")
    traffic = load_traffic()
    dom = max(STEP_KERNELS, key=kt.get)  # the largest per-step kernel
    achieved = tiles * KERNEL_FLOP_PER_TILE[dom] / (kt[dom] * 1e-3) / 1e12
    busy = load_mfma_busy()
    # The chunk kernels are priced on the bf16 MFMA roofline: algorithmic FLOPs of the
    # kernel's products over its live time, against the published dense peak and against
    # the rate an MFMA-only probe sustains on this device.  The HBM side (copy-calibrated
    # FETCH + WRITE bytes of the committed --pmc summary over the live time) and the
    # MFMA-busy counter are reported beside it.
    peak_meas, peak_shapes = mfma_peak_measured(torch)
    hbm_frac = traffic[dom] / (kt[dom] * 1e-3) / 1e9 / PEAK_HBM_GBS if dom in traffic else None
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 5), "traffic": traffic.get(dom),
                "flop_per_launch": tiles * KERNEL_FLOP_PER_TILE[dom], "kernel_ms": round(kt[dom], 5),
                "peak_measured": round(peak_meas, 1),
                "peak_measured_by_shape": {"16x16x32": peak_shapes[0], "32x32x16": peak_shapes[1]},
                "frac_of_measured_peak": round(achieved / peak_meas, 5),
                "busy_frac": busy.get(dom),
                "measured_hbm_frac": None if hbm_frac is None else round(hbm_frac, 4),
                "compulsory_bytes": BWD_COMPULSORY_BYTES if dom == "bwd_fused" else None}
    if dom == "bwd_fused":
        roofline["launches"] = ("one kda_chunk_backward call: chunk_bwd_sched_kernel (clears the sync words "
                                "and writes the tile order) + chunk_bwd_fused_kernel (scan members, prep "
                                "workgroups and ticketed dense / decay tiles; kernel_ms, traffic and busy_frac "
                                "cover both launches)")
    line = {
        "metric": "KDA fwd+bwd TFLOP/s (B2 T4096 H3 D128 bf16)",
        "value": round(flop / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config2: single KDA layer fwd+bwd, precomputed gate g=-exp(A_log)softplus(.)",
                   "batch": B, "seq_len": T, "heads": H, "key_dim": K, "value_dim": V, "chunk": 64,
                   "parallelism": "single GPU"},
        "ms_per_step_eager": round(ms_eager, 4),
        "ms_fwd": round(ms_fwd, 4),
        "tflops_fwd": round(flop / 3 / (ms_fwd * 1e-3) / 1e12, 3),
        "tokens_per_s_fwd_bwd": round(B * T / (ms * 1e-3), 1),
        "k3_gate": {"ms_per_step": round(results["k3"][0], 4), "ms_fwd": round(results["k3"][1], 4),
                    "ms_per_step_eager": round(results["k3"][4], 4)},
        "kernel_ms": {n: round(v, 4) for n, v in kt.items()},
        "roofline": roofline,
        "mfma_busy_frac": busy or None,
        "hbm_traffic_bytes": traffic or None,
        "reference_gb10_ms_fwd_bwd": 3.916,
    }
    line["hbm_kernels"] = hbm_kernels(torch)
    if not args.no_train:
        line["train_6layer"] = train_throughput(torch)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_sample_len)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
