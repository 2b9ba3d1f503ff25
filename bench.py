#!/usr/bin/env python3
"""int4 dequant + GEMM benchmark on one MI355X.

Headline (``value``): packed-weight GB/s of the act-order decode sweep at
M=1 - one step = one GEMV over each of the (K, N) shapes (5120,5120),
(5120,17408), (17408,5120), (5120,1024), GPTQ v1, groupsize 32, act-order
g_idx, bf16 activations. Weight copies are rotated so every step streams
more distinct weight bytes than the 256 MB Infinity Cache holds.

``sub_results`` time the other workloads (decode M=8, M=16 gs32, M=4096 v2
DiT shapes, odd groupsize 26, RTN linear, RTN embedding, 64-expert MoE).
``roofline`` is the dominant kernel (the decode GEMV at K=5120, N=17408,
M=1) timed with HIP events on the launch stream; its ``traffic`` (HBM bytes
per launch) is read from ``profiles/gemv_stream_k5120_n17408_traffic.json``,
written from two rocprofv3 --pmc runs of this script (FETCH_SIZE, WRITE_SIZE)
scaled by the same counters on a plain copy of known size, which this script
also launches. ``cpu_baseline`` times the reference's two CPU paths in torch
on the host (oracle/cpu_paths.py: "packed" = dequantize per call + F.linear,
"eager" = F.linear on a weight dequantized once) for every workload; each
sub-result carries its CPU medians and the GPU speed-up over both paths.

    python bench.py [--steps K] [--warmup W] [--workloads all|decode,...]
"""
from __future__ import annotations

import argparse
import copy
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "onecompression-runtime_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "int4 GEMM TFLOP/s & weight GB/s at M=1/16/4096; % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
CALIB_COPY_BYTES = 512 << 20
DECODE_SHAPES = [(5120, 5120), (5120, 17408), (17408, 5120), (5120, 1024)]
DIT_SHAPES = [(3072, 3072), (3072, 12288), (12288, 3072)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gptq_bytes(K: int, N: int, gs: int = 32) -> int:
    """qweight + fp16 scales + qzeros of a GPTQ layer (0.578125 B/weight at gs 32)."""
    G = math.ceil(K / gs)
    return (math.ceil(K / 8) * N * 4) + G * N * 2 + G * (N // 8) * 4


def time_ms(launch, iters: int, warmup: int) -> float:
    """Average ms per call of ``launch(i)`` between two HIP events on the current stream."""
    import torch

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        launch(i)
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / iters


def graph_ms(calls, replays: int = 10) -> float:
    """Average ms per call of ``calls`` (zero-argument launches, e.g. one per
    weight copy) captured back to back into one HIP graph and replayed."""
    import torch

    for c in calls:  # eager once: workspaces reach their size before capture
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / (replays * len(calls))


def build_gptq(K, N, *, seed, dev, copies, **kw):
    """One module per weight copy (distinct device memory), same values."""
    import torch

    from onecomp_runtime import backend, synthetic

    layer = synthetic.gptq_layer(K, N, seed=seed, **kw)
    entry = dict(in_features=K, out_features=N, wbits=4, groupsize=layer.groupsize,
                 actorder=layer.g_idx is not None, checkpoint_format="gptq" if layer.v1 else "gptq_v2",
                 name="bench")
    st = dict(qweight=layer.qweight, scales=layer.scales, qzeros=layer.qzeros)
    if layer.g_idx is not None:
        st["g_idx"] = layer.g_idx
    mod, _ = backend.build_quant_layer(entry, st, "hip", torch.bfloat16, dev)
    mods = [mod] + [copy.deepcopy(mod) for _ in range(copies - 1)]
    return layer, mods


def decode_workload(dev, M, steps, warmup, layers_cache):
    """The act-order decode sweep at one M; returns (result dict, per-shape data)."""
    import torch

    from onecomp_runtime import synthetic

    per_copy = sum(gptq_bytes(K, N) for K, N in DECODE_SHAPES)
    copies = max(2, math.ceil(2 * MALL_BYTES / per_copy))
    if "decode" not in layers_cache:
        built = []
        for i, (K, N) in enumerate(DECODE_SHAPES):
            log(f"building decode layer K={K} N={N} x{copies}")
            built.append(build_gptq(K, N, seed=20270 + i, dev=dev, copies=copies, act_order=True))
        layers_cache["decode"] = built
    built = layers_cache["decode"]
    xs = [synthetic.activations(M, K, seed=20271 + M).to(dev) for K, _ in DECODE_SHAPES]

    def step(i):
        c = i % copies
        for (layer, mods), x in zip(built, xs):
            mods[c](x)

    with torch.no_grad():
        ms_eager = time_ms(step, steps, warmup)
        # The W warmup steps and the K timed steps each captured into one HIP
        # graph (4 kernel nodes per step, weight copies rotated), as a decode
        # loop runs them; the timed graph is replayed once between two events,
        # with device synchronizations on both sides.
        def capture(first, n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(first, first + n):
                    step(i)
            return g

        g_warm, g_timed = capture(0, max(warmup, 1)), capture(warmup, steps)
        g_warm.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        g_timed.replay()
        end.record()
        end.synchronize()
        ms = start.elapsed_time(end) / steps
        del g_warm, g_timed
    wbytes = sum(gptq_bytes(K, N) for K, N in DECODE_SHAPES)
    flops = sum(2 * M * K * N for K, N in DECODE_SHAPES)
    res = {
        "ms_per_step": ms,
        "weight_GBps": wbytes / (ms * 1e-3) / 1e9,
        "TFLOPs": flops / (ms * 1e-3) / 1e12,
        "hbm_frac": wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "ms_per_step_eager": ms_eager,
        "weight_GBps_eager": wbytes / (ms_eager * 1e-3) / 1e9,
        "rotation_bytes": per_copy * copies,
    }
    return res, built, xs, copies


def dominant_kernel(dev, built, xs, copies, iters):
    """Decode GEMV at K=5120, N=17408, M=1, timed alone (events over the region)."""
    import torch

    idx = DECODE_SHAPES.index((5120, 17408))
    _, mods = built[idx]
    x = xs[idx]
    reps = 4
    with torch.no_grad():
        # one graph = reps x copies back-to-back launches of this kernel alone
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                for c in range(copies):
                    mods[c](x)
        ms = time_ms(lambda i: g.replay(), max(5, iters // (reps * copies)), 3) / (reps * copies)
    K, N = DECODE_SHAPES[idx]
    M = x.shape[0]
    # packed weights + kinv (uint16) + activations + output
    algo = gptq_bytes(K, N) + K * 2 + M * K * 2 + M * N * 2
    achieved = algo / (ms * 1e-3) / 1e9
    # Calibration for the --pmc runs: one plain device copy of known size.
    src = torch.empty(CALIB_COPY_BYTES, dtype=torch.uint8, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    traffic = None
    tfile = ROOT / "profiles" / "gemv_stream_k5120_n17408_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "gemv_stream_kernel<bf16,f16,MR=1,act-order scatter,2 units in flight>",
            "shape": f"M={M} K={K} N={N}",
            "launch_us": round(ms * 1e3, 3), "algorithmic_bytes_per_launch": algo,
            "calibration_copy_bytes": CALIB_COPY_BYTES}


def dense_library_us(dev, M, K, N, copies=2):
    """Context only: the same-shape GEMM on already dequantized bf16 weights as
    the vendor library (hipBLASLt, via F.linear) runs it, weight copies
    rotated like the packed layer's, graph replays."""
    import torch

    x = torch.randn(M, K, dtype=torch.bfloat16, device=dev)
    ws = [torch.randn(N, K, dtype=torch.bfloat16, device=dev) for _ in range(copies)]
    with torch.no_grad():
        ms = graph_ms([lambda w=w: torch.nn.functional.linear(x, w) for w in ws])
    del x, ws
    return ms * 1e3


def gptq_m16_workload(dev, steps, warmup):
    import torch

    from onecomp_runtime import synthetic

    K = N = 4096
    copies = math.ceil(2 * MALL_BYTES / gptq_bytes(K, N))
    log(f"building gptq_gs32 layer x{copies}")
    _, mods = build_gptq(K, N, seed=20260, dev=dev, copies=copies)
    x = synthetic.activations(16, K, seed=20261).to(dev)
    with torch.no_grad():  # (the graph pass calls every copy once first)
        ms = graph_ms([lambda m=m: m(x) for m in mods])
        ms_eager = time_ms(lambda i: mods[i % copies](x), steps * 4, warmup)
    gbps = gptq_bytes(K, N) / (ms * 1e-3) / 1e9
    dense_copies = math.ceil(2 * MALL_BYTES / (K * N * 2))
    return {"M": 16, "K": K, "N": N, "us": ms * 1e3, "weight_GBps": gbps, "hbm_frac": gbps / HBM_PEAK_GBS,
            "TFLOPs": 2 * 16 * K * N / (ms * 1e-3) / 1e12, "us_eager": ms_eager * 1e3,
            "dense_bf16_library_us": dense_library_us(dev, 16, K, N, dense_copies)}


def dit_workload(dev, steps, warmup):
    import torch

    from onecomp_runtime import synthetic

    out = {}
    tot_flops = tot_ms = 0.0
    for i, (K, N) in enumerate(DIT_SHAPES):
        log(f"building dit layer K={K} N={N}")
        _, mods = build_gptq(K, N, seed=20280 + i, dev=dev, copies=1, v1=False)
        x = synthetic.activations(4096, K, seed=20281, outliers=True).to(dev)
        with torch.no_grad():
            ms = graph_ms([lambda: mods[0](x)] * 4, replays=max(3, steps // 4))
            # Context only: a dense bf16 GEMM of the same shape on an already
            # dequantized weight, as the vendor library (hipBLASLt) runs it.
            wd = torch.randn(N, K, dtype=torch.bfloat16, device=dev)
            ms_ref = time_ms(lambda j: torch.nn.functional.linear(x, wd), steps, warmup)
        flops = 2 * 4096 * K * N
        tf = flops / (ms * 1e-3) / 1e12
        out[f"K{K}_N{N}"] = {"us": ms * 1e3, "TFLOPs": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS,
                             "dense_bf16_library_TFLOPs": flops / (ms_ref * 1e-3) / 1e12}
        tot_flops += flops
        tot_ms += ms
        del mods, x, wd
    tf = tot_flops / (tot_ms * 1e-3) / 1e12
    out["aggregate"] = {"TFLOPs": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS}
    return out


def padded_workload(dev, steps, warmup):
    import torch

    from onecomp_runtime import synthetic

    K, N, M = 1040, 3072, 256
    copies = math.ceil(2 * MALL_BYTES / gptq_bytes(1056, N))
    _, mods = build_gptq(K, N, seed=20290, dev=dev, copies=copies, groupsize=26, pad_rows_to=1056)
    x = synthetic.activations(M, K, seed=20291).to(dev)
    with torch.no_grad():  # (the graph pass calls every copy once first)
        ms = graph_ms([lambda m=m: m(x) for m in mods])
        ms_eager = time_ms(lambda i: mods[i % copies](x), steps * 4, warmup)
    tf = 2 * M * K * N / (ms * 1e-3) / 1e12
    wb = 1056 // 8 * N * 4 + 40 * N * 2 + 40 * N // 8 * 4
    return {"us": ms * 1e3, "TFLOPs": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS,
            "GBps": (wb + M * K * 2 + M * N * 2) / (ms * 1e-3) / 1e9, "us_eager": ms_eager * 1e3,
            "dense_bf16_library_us": dense_library_us(dev, M, K, N)}


def rtn_workload(dev, steps, warmup):
    import torch

    from onecomp_runtime import PackedEmbedding, PackedRTNLinear, synthetic

    res = {}
    M, K, N = 512, 1024, 2048
    layer = synthetic.rtn_layer(N, K, seed=20300)
    mod = PackedRTNLinear(K, N, layer.qweight_u8.to(dev), layer.scales.to(dev), layer.zeros.to(dev))
    x = synthetic.activations(M, K, seed=20301).to(dev)
    with torch.no_grad():
        ms_eager = time_ms(lambda i: mod(x), steps * 4, warmup)
        ms = graph_ms([lambda: mod(x)] * 8)
    tf = 2 * M * K * N / (ms * 1e-3) / 1e12
    res["rtn_linear_m512"] = {"us": ms * 1e3, "TFLOPs": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS,
                              "us_eager": ms_eager * 1e3, "dense_bf16_library_us": dense_library_us(dev, M, K, N)}
    V, D, T = 32768, 1024, 4096
    for G in (1, 32):
        emb_layer = synthetic.rtn_layer(V, D, seed=20310, groups=G)
        # Table copies covering twice the Infinity Cache, each with its own
        # token ids: every call gathers rows the caches have not seen lately.
        table_bytes = V * (D // 2 + 4 * G)
        copies = max(2, -(-2 * MALL_BYTES // table_bytes))
        embs = [PackedEmbedding(V, D, emb_layer.qweight_u8.to(dev), emb_layer.scales.to(dev),
                                emb_layer.zeros.to(dev)) for _ in range(copies)]
        idss = [torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(20311 + i)).to(dev)
                for i in range(copies)]
        with torch.no_grad():  # (the graph pass calls every copy once first)
            ms = graph_ms([lambda i=i: embs[i](idss[i]) for i in range(copies)])
            ms_eager = time_ms(lambda i: embs[i % copies](idss[i % copies]), steps * 4, warmup)
        nbytes = T * (D // 2 + 4 * G) + T * 8 + T * D * 2
        res[f"rtn_embedding_G{G}"] = {"us": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9,
                                      "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                      "us_eager": ms_eager * 1e3, "table_copies": copies}
        del embs, idss
    return res


def moe_workload(dev, steps, warmup):
    import torch

    from onecomp_runtime import kernels, synthetic

    E, K, N, T, topk = 64, 4096, 2048, 512, 8
    log("building 64 experts")
    experts = synthetic.moe_experts(E, K, N, seed=20330, keep_codes=False)
    copies = 2
    w = [kernels.prepare_experts(experts.qweight.to(dev), experts.scales.to(dev), experts.qzeros.to(dev))
         for _ in range(copies)]
    x = synthetic.activations(T, K, seed=20331).to(dev)
    ids = synthetic.router_topk(T, E, topk, seed=20332).to(dev)

    def step(i):
        off, pairs = kernels.moe_route(ids, E)
        kernels.int4_moe_gemm(x, topk, w[i % copies], off, pairs)

    with torch.no_grad():
        ms_eager = time_ms(step, steps, warmup)
        ms = graph_ms([lambda c=c: step(c) for c in range(copies)] * 2)
    wbytes = E * gptq_bytes(K, N)
    flops = 2 * T * topk * K * N
    return {"us": ms * 1e3, "weight_GBps": wbytes / (ms * 1e-3) / 1e9,
            "hbm_frac": wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "TFLOPs": flops / (ms * 1e-3) / 1e12,
            "us_eager": ms_eager * 1e3}


PCIE_H2D_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction


def next_rows_workload(dev, steps, warmup):
    """The rows after the hot path, measured the same way: GPTQ groupsize 128
    in 4 and 8 bits (Qwen-style K=N=5120) at M=1 and 16; DSV4 int4 / int2
    gs128 K=7168 N=2048 at M=1, device-resident and as host-resident routed
    experts (pinned copies per call); packed Conv1d / ConvTranspose1d."""
    import torch

    from onecomp_runtime import PackedGPTQLinear, synthetic
    from onecomp_runtime.layers import (Dsv4PackedLinear, PackedInt4Conv1d, PackedInt4ConvTranspose1d,
                                        run_routed_experts)

    res = {}
    K = N = 5120
    for wbits in (4, 8):
        if wbits == 4:
            nbytes = gptq_bytes(K, N, gs=128)
            copies = math.ceil(2 * MALL_BYTES / nbytes)
            _, mods = build_gptq(K, N, seed=20480, dev=dev, copies=copies, groupsize=128)
        else:
            G = K // 128
            nbytes = K * N + G * N * 2 + G * (N // 4) * 4
            copies = math.ceil(2 * MALL_BYTES / nbytes)
            l8 = synthetic.gptq8_layer(K, N, seed=20481, groupsize=128)
            mods = [PackedGPTQLinear(K, N, l8.qweight.to(dev), l8.scales.to(dev), l8.qzeros.to(dev), groupsize=128,
                                     wbits=8) for _ in range(copies)]
        for M in (1, 16):
            x = synthetic.activations(M, K, seed=20482 + M).to(dev)
            with torch.no_grad():  # (the graph pass calls every copy once first)
                ms = graph_ms([lambda m=m: m(x) for m in mods])
                ms_eager = time_ms(lambda i: mods[i % copies](x), steps * 2, warmup)
            gbps = nbytes / (ms * 1e-3) / 1e9
            res[f"gptq{wbits}_gs128_k5120_m{M}"] = {"us": ms * 1e3, "weight_GBps": gbps,
                                                     "hbm_frac": gbps / HBM_PEAK_GBS, "us_eager": ms_eager * 1e3}
        del mods
        torch.cuda.empty_cache()
    K, N = 7168, 2048
    for wbits in (4, 2):
        pk = synthetic.dsv4_layer(N, K, wbits=wbits, seed=20490 + wbits)
        nbytes = N * K * wbits // 8 + 2 * (K // 128) * N * 2
        copies = math.ceil(2 * MALL_BYTES / nbytes)
        mods = [Dsv4PackedLinear(pk, buffer_device=dev) for _ in range(copies)]
        x = synthetic.activations(1, K, seed=20492).to(dev)
        with torch.no_grad():
            ms = graph_ms([lambda m=m: m(x) for m in mods])
        gbps = nbytes / (ms * 1e-3) / 1e9
        res[f"dsv4_int{wbits}_k7168_n2048_m1"] = {"us": ms * 1e3, "weight_GBps": gbps, "hbm_frac": gbps / HBM_PEAK_GBS}
        del mods
    # Host-resident int2 experts, 4 tokens x top-8 of 32: each call copies
    # every routed expert (more than the stager's slots) and runs its GEMV.
    E, T, topk = 32, 4, 8
    packs = [synthetic.dsv4_layer(N, K, wbits=2, seed=20500 + e) for e in range(E)]
    experts = [Dsv4PackedLinear(p, buffer_device="cpu") for p in packs]
    ebytes = N * K // 4 + 2 * (K // 128) * N * 2
    x = synthetic.activations(T, K, seed=20540).to(dev)
    idss = [synthetic.router_topk(T, E, topk, seed=20541 + i).to(dev) for i in range(max(4, steps // 4))]
    used = [len(set(ids.flatten().tolist())) for ids in idss]
    with torch.no_grad():
        ms = time_ms(lambda i: run_routed_experts(experts, x, idss[i % len(idss)]), len(idss), 2)
    h2d = sum(used) / len(used) * ebytes
    res["dsv4_int2_host_experts_t4_top8"] = {"ms": ms, "experts_per_call": sum(used) / len(used),
                                             "h2d_GBps": h2d / (ms * 1e-3) / 1e9,
                                             "pcie_frac": h2d / (ms * 1e-3) / 1e9 / PCIE_H2D_PEAK_GBS}
    del experts, packs
    # Packed convolutions (one batch, bf16).
    cases = [("conv1d_512_512_k7_L8192", PackedInt4Conv1d, 512, 512, 7, dict(padding=3), 8192),
             ("convT_1024_512_k16_s8_L1024", PackedInt4ConvTranspose1d, 1024, 512, 16, dict(stride=8), 1024)]
    for name, cls, cin, cout, k, kw, L in cases:
        rows, cols = (cout, cin * k) if cls is PackedInt4Conv1d else (cin, cout * k)
        rl = synthetic.rtn_layer(rows, cols, seed=20550, groups=cols // 32)
        mod = cls(cin, cout, k, qweight=rl.qweight_u8, scales=rl.scales, zeros=rl.zeros, cols=cols,
                  pad_mode="none", **kw).to(dev)
        x = synthetic.activations(cin, L, seed=20551).reshape(1, cin, L).to(dev)
        with torch.no_grad():
            y = mod(x)
            ms = graph_ms([lambda: mod(x)] * 4)
            # The reference's forward on this GPU (layers/packed_conv.py:196-222): the weight dequantized on
            # every call, then the library convolution; and the library convolution alone on a bf16 weight.
            wd = mod._materialize(torch.bfloat16)
            if cls is PackedInt4Conv1d:
                conv = lambda w: torch.nn.functional.conv1d(x, w, None, 1, kw["padding"])
            else:
                conv = lambda w: torch.nn.functional.conv_transpose1d(x, w, None, kw["stride"])
            ref_ms = time_ms(lambda i: conv(mod._materialize(torch.bfloat16)), 20, 3)
            lib_ms = time_ms(lambda i: conv(wd), 20, 3)
            del wd
        flops = 2 * cin * cout * k * (y.shape[-1] if cls is PackedInt4Conv1d else L)
        res[name] = {"us": ms * 1e3, "TFLOPs": flops / (ms * 1e-3) / 1e12,
                     "mfma_frac": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                     "reference_path_us": ref_ms * 1e3, "bf16_library_conv_us": lib_ms * 1e3}
    return res


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(max_s_per_case: float = 4.0):
    """The reference's CPU paths in torch on the host (oracle/cpu_paths.py):
    "packed" dequantizes the weight on every call then F.linear
    (packed_gptq_linear.py:66-74, packed_linear.py:53-56); "eager" runs F.linear
    on a weight dequantized once (backend.py:246-264). Same seeded inputs as the
    GPU workloads; torch.set_num_threads(<CPUs this process may run on>); the
    median of 5 timed calls after 2 warmups per case. The DiT and MoE cases run
    on a stated sample (fewer rows / experts) and report rates per byte / flop."""
    import numpy as np
    import torch

    from onecomp_runtime import synthetic
    from oracle import cpu_paths as C

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    bf = torch.bfloat16

    def median_s(fn, n=5, warm=2):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def gptq(K, N, seed, **kw):
        lay = synthetic.gptq_layer(K, N, seed=seed, **kw)
        g = lay.g_idx if lay.g_idx is not None else torch.arange(K) // lay.groupsize
        return C.PackedGPTQ(lay.qweight, lay.scales, lay.qzeros, g, K, N, bf, lay.v1)

    def both(make_calls, nbytes=None, flops=None, sample=None):
        """make_calls() -> (packed step, eager step); rates from the medians."""
        packed, eager = make_calls()
        out = {}
        with torch.no_grad():
            for name, fn in (("packed", packed), ("eager", eager)):
                t = median_s(fn)
                r = {"ms": round(t * 1e3, 3)}
                if nbytes:
                    r["weight_GBps"] = round(nbytes / t / 1e9, 4)
                if flops:
                    r["TFLOPs"] = round(flops / t / 1e12, 5)
                out[name] = r
        if sample:
            out["sample"] = sample
        return out

    res = {}
    for M in (1, 8):
        log(f"cpu: decode sweep M={M}")
        mods = [gptq(K, N, seed=20270 + i, act_order=True) for i, (K, N) in enumerate(DECODE_SHAPES)]
        eag = [m.eager() for m in mods]
        xs = [synthetic.activations(M, K, seed=20271 + M) for K, _ in DECODE_SHAPES]
        wb = sum(gptq_bytes(K, N) for K, N in DECODE_SHAPES)
        fl = sum(2 * M * K * N for K, N in DECODE_SHAPES)
        res[f"decode_actorder_m{M}"] = both(
            lambda: (lambda: [m(x) for m, x in zip(mods, xs)], lambda: [e(x) for e, x in zip(eag, xs)]),
            wb, fl, "one step = the 4 shapes")
        del mods, eag
    log("cpu: gs32 M=16")
    m = gptq(4096, 4096, seed=20260)
    x = synthetic.activations(16, 4096, seed=20261)
    e = m.eager()
    res["gptq_gs32_m16"] = both(lambda: (lambda: m(x), lambda: e(x)), gptq_bytes(4096, 4096), 2 * 16 * 4096 * 4096)
    log("cpu: DiT (row sample)")
    dit = {}
    rows = 512
    for i, (K, N) in enumerate(DIT_SHAPES):
        m = gptq(K, N, seed=20280 + i, v1=False)
        x = synthetic.activations(4096, K, seed=20281, outliers=True)[:rows]
        e = m.eager()
        dit[f"K{K}_N{N}"] = both(lambda: (lambda: m(x), lambda: e(x)), None, 2 * rows * K * N,
                                 f"{rows} of the 4096 rows")
    res["dit_large_m_m4096"] = dit
    log("cpu: padded gs26")
    lay = synthetic.gptq_layer(1040, 3072, seed=20290, groupsize=26, pad_rows_to=1056)
    m = C.PackedGPTQ(lay.qweight, lay.scales, lay.qzeros, torch.arange(1040) // 26, 1040, 3072, bf, True)
    x = synthetic.activations(256, 1040, seed=20291)
    e = m.eager()
    res["padded_gs26_m256"] = both(lambda: (lambda: m(x), lambda: e(x)), None, 2 * 256 * 1040 * 3072)
    log("cpu: RTN linear / embedding")
    rl = synthetic.rtn_layer(2048, 1024, seed=20300)
    m = C.PackedRTN(rl.qweight_u8, rl.scales, rl.zeros, 1024, bf)
    x = synthetic.activations(512, 1024, seed=20301)
    e = m.eager()
    res["rtn_linear_m512"] = both(lambda: (lambda: m(x), lambda: e(x)), None, 2 * 512 * 1024 * 2048)
    V, D, T = 32768, 1024, 4096
    for G in (1, 32):
        el = synthetic.rtn_layer(V, D, seed=20310, groups=G)
        ids = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(20311))
        table = C.rtn_dequant(el.qweight_u8, el.scales, el.zeros, D, el.scales.dtype)
        nbytes = T * (D // 2 + 4 * G) + T * 8 + T * D * 2
        res[f"rtn_embedding_G{G}"] = both(
            lambda: (lambda: C.embedding(ids, el.qweight_u8, el.scales, el.zeros, D), lambda: table[ids]),
            nbytes, None, "eager = rows of a table dequantized once")
        del el, table
    log("cpu: MoE (expert sample)")
    E, K, N, T, topk, sampled = 64, 4096, 2048, 512, 8, 8
    ids = synthetic.router_topk(T, E, topk, seed=20332)
    x = synthetic.activations(T, K, seed=20331)
    flat = ids.reshape(-1)
    experts = [C.PackedGPTQ(*(lambda l: (l.qweight, l.scales, l.qzeros, torch.arange(K) // 32))(
        synthetic.gptq_layer(K, N, seed=20330 + 1000 * e)), K, N, bf, True) for e in range(sampled)]
    eag = [p.eager() for p in experts]
    pairs = [torch.nonzero(flat == e).flatten() for e in range(sampled)]

    def moe(mods):
        return [mods[e](x[pairs[e] // topk]) for e in range(sampled)]

    res["moe_64x_top8"] = both(lambda: (lambda: moe(experts), lambda: moe(eag)), sampled * gptq_bytes(K, N),
                               2 * sum(len(p) for p in pairs) * K * N,
                               f"experts 0..{sampled - 1} of 64 with their routed rows")
    head = res["decode_actorder_m1"]
    return {
        "value": head["packed"]["weight_GBps"], "unit": "GB/s", "cores": threads, "kind": "port",
        "path": "packed", "eager_value": head["eager"]["weight_GBps"],
        "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
        "sample": "M=1 act-order decode sweep (4 shapes, packed weights per step); torch CPU, per call "
                  "dequant + F.linear (packed); median of 5 after 2 warmups",
        "per_config": res,
    }


def attach_cpu_ratios(sub: dict, head: dict, cpu: dict) -> None:
    """Beside each GPU result: the CPU medians and GPU speed-up over each path."""
    per = cpu["per_config"]

    def put(dst: dict, src: dict, gpu_ms: float) -> None:
        dst["cpu"] = src
        for path in ("packed", "eager"):
            dst[f"speedup_vs_cpu_{path}"] = round(src[path]["ms"] / gpu_ms, 1)

    head["cpu"] = per["decode_actorder_m1"]
    for path in ("packed", "eager"):
        head[f"speedup_vs_cpu_{path}"] = round(per["decode_actorder_m1"][path]["ms"] / head["ms_per_step"], 1)
    if "decode_actorder_m8" in sub:
        put(sub["decode_actorder_m8"], per["decode_actorder_m8"], sub["decode_actorder_m8"]["ms_per_step"])
    for key in ("gptq_gs32_m16", "padded_gs26_m256", "rtn_linear_m512", "rtn_embedding_G1", "rtn_embedding_G32"):
        if key in sub:
            put(sub[key], per[key], sub[key]["us"] / 1e3)
    if "dit_large_m_m4096" in sub:
        for shape, r in per["dit_large_m_m4096"].items():
            g = sub["dit_large_m_m4096"][shape]
            g["cpu"] = r
            for path in ("packed", "eager"):
                g[f"speedup_vs_cpu_{path}"] = round(g["TFLOPs"] / r[path]["TFLOPs"], 1)
    if "moe_64x_top8" in sub:
        g = sub["moe_64x_top8"]
        g["cpu"] = per["moe_64x_top8"]
        for path in ("packed", "eager"):
            g[f"speedup_vs_cpu_{path}"] = round(g["weight_GBps"] / per["moe_64x_top8"][path]["weight_GBps"], 1)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workloads", default="all",
                    help="comma list of: m16,dit,padded,rtn,moe,next (the headline always runs)")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this package runs the workload on one GPU", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = ({"m16", "dit", "padded", "rtn", "moe", "next"} if args.workloads == "all"
          else set(args.workloads.split(",")))
    if "none" in wl:
        wl = set()

    cache: dict = {}
    log("decode sweep M=1 (headline)")
    head, built, xs, copies = decode_workload(dev, 1, args.steps, args.warmup, cache)
    log(f"headline {head['weight_GBps']:.1f} GB/s, {head['ms_per_step']*1e3:.1f} us/step")
    roof = dominant_kernel(dev, built, xs, copies, max(100, args.steps * 4))
    log(f"dominant kernel {roof['achieved']} GB/s ({roof['launch_us']} us/launch)")
    sub = {}
    m8, _, _, _ = decode_workload(dev, 8, args.steps, args.warmup, cache)
    sub["decode_actorder_m8"] = m8
    per_shape = {}
    for (K, N), (layer, mods), x in zip(DECODE_SHAPES, built, xs):
        with torch.no_grad():
            ms = graph_ms([lambda m=m: m(x) for m in mods] * 2)
            ms_eager = time_ms(lambda i: mods[i % copies](x), args.steps * 2, args.warmup)
        per_shape[f"K{K}_N{N}"] = {"us": ms * 1e3, "weight_GBps": gptq_bytes(K, N) / (ms * 1e-3) / 1e9,
                                   "us_eager": ms_eager * 1e3}
    sub["decode_actorder_m1_per_shape"] = per_shape
    del built, xs, cache
    torch.cuda.empty_cache()
    if "m16" in wl:
        log("gptq_gs32 M=16")
        sub["gptq_gs32_m16"] = gptq_m16_workload(dev, args.steps, args.warmup)
    if "dit" in wl:
        log("dit M=4096")
        sub["dit_large_m_m4096"] = dit_workload(dev, max(5, args.steps // 5), 3)
    if "padded" in wl:
        log("padded gs26")
        sub["padded_gs26_m256"] = padded_workload(dev, args.steps, args.warmup)
    if "rtn" in wl:
        log("rtn linear / embedding")
        sub.update(rtn_workload(dev, args.steps, args.warmup))
    if "moe" in wl:
        log("moe")
        sub["moe_64x_top8"] = moe_workload(dev, max(5, args.steps // 2), 3)
    if "next" in wl:
        log("gs128 4/8-bit, DSV4, conv")
        sub.update(next_rows_workload(dev, args.steps, args.warmup))
    torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (torch CPU packed / eager paths)")
        t0 = time.perf_counter()
        cpu = cpu_baseline()
        log(f"cpu baseline done in {time.perf_counter() - t0:.0f} s")
        attach_cpu_ratios(sub, head, cpu)

    def rnd(o):
        if isinstance(o, float):
            return round(o, 4)
        if isinstance(o, dict):
            return {k: rnd(v) for k, v in o.items()}
        return o

    line = {
        "metric": METRIC,
        "value": round(head["weight_GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode_actorder_m1", "M": 1, "shapes_KN": DECODE_SHAPES, "groupsize": 32,
                   "act_order": True, "format": "gptq (v1 zeros)", "activations": "bf16",
                   "weight_rotation_bytes": head["rotation_bytes"],
                   "value_bytes": "packed qweight+scales+qzeros per step",
                   "launch": "the K timed steps captured into one HIP graph (4 kernel nodes per step, "
                             "weight copies rotated) and replayed once; eager python launches reported "
                             "as ms_per_step_eager",
                   "ms_per_step_eager": round(head["ms_per_step_eager"], 5),
                   "weight_GBps_eager": round(head["weight_GBps_eager"], 2)},
        "roofline": roof,
        "cpu_baseline": cpu and {k: v for k, v in cpu.items() if k != "per_config"},
        "hbm_frac_step": round(head["hbm_frac"], 4),
        "headline_vs_cpu": head.get("cpu") and {k: head[k] for k in ("cpu", "speedup_vs_cpu_packed",
                                                                     "speedup_vs_cpu_eager")},
        "sub_results": rnd(sub),
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
