#!/usr/bin/env python3
"""Benchmark of the fused dequant-matmul path on one MI355X.

Default workload (one "step" = one decoded token): the Qwen3-4B-shaped q4_0 decode linear
stack, batch 1, 36 layers x {q 2560->4096, k/v 2560->1024, o 4096->2560, gate/up 2560->9728,
down 9728->2560}, fp16 activations, seeded synthetic weights (fp16 scales |N(0, 0.01)|,
uniform nibbles). Per layer four launches: q|k|v fused (one shared x), o, gate|up fused, down;
the whole token is captured once as a HIP graph and replayed.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config stack|gemv1|...]

Prints one JSON line. ``value`` = aggregate algorithmic GB/s per token (weights + activations
read and written once per token) with all inputs resident in HBM.
``roofline`` = the dominant kernel (the q4_0 GEMV family) measured live with HIP events on
the launch stream; ``cpu_baseline`` = the numpy oracle path (f32 decode + BLAS matvec) timed
on a bounded sample of the same workload on this host.
"""

import argparse
import json
import os
import sys
import time

# roofline constants (MI355X datasheet, dense) live in roofline.json beside this file
with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "roofline.json")) as _f:
    ROOFLINE = json.load(_f)
HBM_PEAK_GBS = float(ROOFLINE["hbm_GBps"])
METRIC = "dequant-GEMV GB/s (% HBM peak) + prefill/MoE GEMM TFLOP/s (% MFMA peak)"

QWEN3_4B = dict(hidden=2560, q=4096, kv=1024, inter=9728, layers=36)
STACK_TRAFFIC_PER_LAUNCH = 14402381  # measured HBM bytes per decode-stack launch (see run_stack)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="stack",
                    choices=["stack", "stack_chain", "gemv1", "kquant", "producers", "router", "exl3", "prefill",
                             "prefill_i8", "moe", "copy"])
    ap.add_argument("--wtype", type=int, default=12, choices=[12, 13, 14, 22],
                    help="GGML type id for --config kquant (12 Q4_K, 13 Q5_K, 14 Q6_K, 22 IQ2_S)")
    ap.add_argument("--tokens", type=int, default=16, help="tokens for --config moe / router")
    ap.add_argument("--batch", type=int, default=1, help="batch for --config exl3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


def q4_0_blocks_gpu(torch, gen, N, K, dev):
    """Seeded packed q4_0 rows generated on the device: uint8 [N * K/32 * 18]."""
    nb = N * (K // 32)
    blk = torch.empty((nb, 18), dtype=torch.uint8, device=dev)
    d = (torch.randn(nb, generator=gen, device=dev) * 0.01).abs().to(torch.float16)
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:] = torch.randint(0, 256, (nb, 16), generator=gen, device=dev, dtype=torch.uint8)
    return blk.view(-1)


def kquant_blocks_gpu(torch, gen, ty, N, K, dev):
    """Seeded packed Q4_K / Q5_K / Q6_K rows on the device: uniform random bytes, the fp16
    scale fields = |N(0, 1e-4)|."""
    sbytes = {12: 144, 13: 176, 14: 210, 22: 82}[ty]
    nb = N * (K // 256)
    blk = torch.randint(0, 256, (nb, sbytes), generator=gen, device=dev, dtype=torch.uint8)
    for off in {12: (0, 2), 13: (0, 2), 14: (208,), 22: (0,)}[ty]:
        d = (torch.randn(nb, generator=gen, device=dev) * 1e-4).abs().to(torch.float16)
        blk[:, off:off + 2] = d.view(torch.uint8).view(nb, 2)
    return blk.view(-1)


def build_stack(torch, dev, seed):
    c = QWEN3_4B
    H, Q, KV, I = c["hidden"], c["q"], c["kv"], c["inter"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers = []
    for _ in range(c["layers"]):
        layers.append(dict(
            q=q4_0_blocks_gpu(torch, gen, Q, H, dev), k=q4_0_blocks_gpu(torch, gen, KV, H, dev),
            v=q4_0_blocks_gpu(torch, gen, KV, H, dev), o=q4_0_blocks_gpu(torch, gen, H, Q, dev),
            gate=q4_0_blocks_gpu(torch, gen, I, H, dev), up=q4_0_blocks_gpu(torch, gen, I, H, dev),
            down=q4_0_blocks_gpu(torch, gen, H, I, dev)))
    f16 = torch.float16
    acts = dict(
        x_attn=torch.randn(H, generator=gen, device=dev).to(f16),
        x_o=torch.randn(Q, generator=gen, device=dev).to(f16),
        x_mlp=torch.randn(H, generator=gen, device=dev).to(f16),
        x_down=torch.randn(I, generator=gen, device=dev).to(f16),
        yq=torch.empty(Q, dtype=f16, device=dev), yk=torch.empty(KV, dtype=f16, device=dev),
        yv=torch.empty(KV, dtype=f16, device=dev), yo=torch.empty(H, dtype=f16, device=dev),
        yg=torch.empty(I, dtype=f16, device=dev), yu=torch.empty(I, dtype=f16, device=dev),
        yd=torch.empty(H, dtype=f16, device=dev))
    return layers, acts


def stack_bytes():
    c = QWEN3_4B
    H, Q, KV, I = c["hidden"], c["q"], c["kv"], c["inter"]
    shapes = [(Q, H), (KV, H), (KV, H), (H, Q), (I, H), (I, H), (H, I)]
    w = sum(n * k // 32 * 18 for n, k in shapes)
    act = sum(2 * k + 2 * n for n, k in shapes)
    flops = sum(2 * n * k for n, k in shapes)
    return shapes, (w + act) * c["layers"], flops * c["layers"], w


def stack_launches(ops, layers, a):
    """The launches of one token, in order, as closures (for graph capture and timing)."""
    H, Q, KV, I = QWEN3_4B["hidden"], QWEN3_4B["q"], QWEN3_4B["kv"], QWEN3_4B["inter"]
    out = []
    for L in layers:
        out.append(lambda L=L: ops.gemv_q4_0_seg3(a["x_attn"], H, [(L["q"], a["yq"], Q), (L["k"], a["yk"], KV),
                                                                    (L["v"], a["yv"], KV)]))
        out.append(lambda L=L: ops.gemv(ops.GGML_Q4_0, L["o"], a["x_o"], H, Q, out=a["yo"].view(1, H)))
        out.append(lambda L=L: ops.gemv_q4_0_seg3(a["x_mlp"], H, [(L["gate"], a["yg"], I), (L["up"], a["yu"], I)]))
        out.append(lambda L=L: ops.gemv(ops.GGML_Q4_0, L["down"], a["x_down"], H, I, out=a["yd"].view(1, H)))
    return out


def cpu_baseline_stack(target_s=10.0, target_all_s=6.0):
    """numpy oracle path on a bounded sample: q4_0 -> f32 decode, then BLAS matvec. The reported
    value is one thread; the same sample is also timed with BLAS on every host core."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    from oracle import formats
    from vybforge_amd import synth
    shapes, _, _, _ = stack_bytes()
    rng = np.random.default_rng(1)
    mats = [(synth.q4_0_weights(rng, n, k), n, k) for n, k in shapes]
    xs = {k: rng.standard_normal(k).astype(np.float16) for _, k in shapes}
    layer_bytes = sum(raw.size + 2 * k + 2 * n for raw, n, k in mats)

    def run(limit, seconds):
        done = 0
        t0 = time.perf_counter()
        with threadpool_limits(limits=limit):
            while True:
                for raw, n, k in mats:
                    w = formats.dequant_q4_0(raw).reshape(n, k)
                    y = w @ xs[k].astype(np.float32)
                    y.astype(np.float16)
                done += 1
                el = time.perf_counter() - t0
                if el >= seconds:
                    return done, el

    done, el = run(1, target_s)
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    done_all, el_all = run(ncpu, target_all_s)
    blas = ", ".join(f"{i.get('internal_api')} {i.get('version')}" for i in threadpool_info()
                     if i.get("user_api") == "blas") or "unknown"
    return dict(value=round(layer_bytes * done / el / 1e9, 3), unit="GB/s", cores=1, kind="port",
                sample=f"{done} layers of the 36-layer stack (7 GEMVs each, 56.8 MB packed), "
                       "numpy f32 decode + BLAS matvec, 1 thread",
                value_all_cores=round(layer_bytes * done_all / el_all / 1e9, 3), cores_all=ncpu,
                host=dict(cpu_count=os.cpu_count(), affinity=ncpu, blas=blas,
                          omp_num_threads=os.environ.get("OMP_NUM_THREADS")))


def stack_chain(ops, layers, a, dev):
    """The token as one persistent chain: 144 dependent stages, one launch."""
    H, Q, KV, I = QWEN3_4B["hidden"], QWEN3_4B["q"], QWEN3_4B["kv"], QWEN3_4B["inter"]
    stages = []
    for L in layers:
        stages.append(ops.pblock(a["x_attn"], H, [(L["q"], a["yq"], Q), (L["k"], a["yk"], KV), (L["v"], a["yv"], KV)]))
        stages.append(ops.pblock(a["x_o"], Q, [(L["o"], a["yo"], H)]))
        stages.append(ops.pblock(a["x_mlp"], H, [(L["gate"], a["yg"], I), (L["up"], a["yu"], I)]))
        stages.append(ops.pblock(a["x_down"], I, [(L["down"], a["yd"], H)]))
    return ops.GemvChain(ops.GGML_Q4_0, stages, dev)


def run_stack(args, torch, dev):
    from vybforge_amd import ops
    shapes, bytes_tok, flops_tok, wbytes_layer = stack_bytes()
    layers, acts = build_stack(torch, dev, args.seed)
    if args.config == "stack_chain":
        chain = stack_chain(ops, layers, acts, dev)
        launches = [chain]
        kernel = "k_gemv_chain<q4_0> (one persistent launch per token, 144 dependent stages)"
    else:
        launches = stack_launches(ops, layers, acts)
        kernel = "k_gemv_pair<q4_0> (all 144 launches per token)"
    torch.cuda.synchronize()

    # capture one token as a graph
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in launches:
            f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in launches:
            f()
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_ev = ev0.elapsed_time(ev1)
    ms_step = ms_ev / args.steps
    value = bytes_tok / (ms_step * 1e-3) / 1e9

    if args.config == "stack_chain":
        st = chain.status()
        if st != 0:
            raise RuntimeError(f"gemv chain reported status {st}")
    # dominant kernel, live: the token's launches back to back on one stream, event-timed
    # over many tokens; the per-launch average includes inter-launch gaps
    n_launch = len(launches)
    achieved = bytes_tok / n_launch / (ms_step * 1e-3 / n_launch) / 1e9
    # HBM bytes per launch from rocprofv3 FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00 (factors from a
    # plain 256 MiB copy), averaged over the four launches of a layer: profiles/q4_0_gemv_decode_stack.md
    traffic = STACK_TRAFFIC_PER_LAUNCH if args.config == "stack" else None
    roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic,
                    kernel=kernel,
                    avg_launch_us=round(ms_step * 1e3 / n_launch, 3),
                    bytes_per_launch=round(bytes_tok / n_launch))
    return dict(value=value, ms_step=ms_step, wall=wall, roofline=roofline, flops=flops_tok,
                workload="qwen3-4b q4_0 decode linear stack: 36 layers x 7 GEMVs, batch 1, fp16 act",
                bytes_per_step=bytes_tok, launches_per_step=n_launch)


def run_gemv1(args, torch, dev):
    """Config 1: q4_0 GEMV 9728x2560, fp32 x, fp32 y, rotating 24 weight copies (>300 MB)."""
    from vybforge_amd import ops
    N, K = 9728, 2560
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    copies = [q4_0_blocks_gpu(torch, gen, N, K, dev) for _ in range(24)]
    x = torch.randn(K, generator=gen, device=dev)
    y = torch.empty(1, N, device=dev)
    launch = [lambda W=W: ops.gemv(ops.GGML_Q4_0, W, x, N, K, out=y) for W in copies]
    for f in launch:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in launch:
            f()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = ev0.elapsed_time(ev1) / args.steps / len(launch)
    bytes_call = N * K // 32 * 18 + 4 * K + 4 * N
    value = bytes_call / (per * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(value, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(value / HBM_PEAK_GBS, 4), traffic=None, kernel="k_gemv_pair<q4_0,f32>",
                    avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call)
    return dict(value=value, ms_step=per * len(launch), wall=wall, roofline=roofline,
                flops=2 * N * K * len(launch), workload="q4_0 GEMV 9728x2560 fp32 x (24 rotated copies)",
                bytes_per_step=bytes_call * len(launch), launches_per_step=len(launch))


def run_kquant(args, torch, dev):
    """K-quant GEMV at the Qwen3-4B MLP shape 9728x2560 (fp16 x, f32 y), 24 rotated weight copies
    (> the 256 MB MALL), one GEMV per copy in one graph."""
    from vybforge_amd import ops
    N, K, ty = 9728, 2560, args.wtype
    name = {12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 22: "IQ2_S"}[ty]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    copies = [kquant_blocks_gpu(torch, gen, ty, N, K, dev) for _ in range(24)]
    x = torch.randn(K, generator=gen, device=dev).to(torch.float16)
    y = torch.empty(1, N, device=dev)
    ms, wall = timed_graph(torch, [lambda W=W: ops.gemv(ty, W, x, N, K, out=y) for W in copies], args.steps,
                           args.warmup)
    per = ms / len(copies)
    bytes_call = ops.row_bytes(ty, K) * N + 2 * K + 4 * N
    value = bytes_call / (per * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(value, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(value / HBM_PEAK_GBS, 4), traffic=None, kernel=f"k_gemv_pair<{name}>",
                    avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call)
    return dict(value=value, ms_step=ms, wall=wall, roofline=roofline, flops=2 * N * K * len(copies),
                workload=f"{name} GEMV 9728x2560 fp16 x (24 rotated copies)",
                bytes_per_step=bytes_call * len(copies), launches_per_step=len(copies))


def run_producers(args, torch, dev):
    """Producer-side q8 at the 27B decode shapes: RMSNorm of one float64 row of 5120 (float32 copy
    + q8 copy) and SwiGLU of 17408 float64 pairs (float32 h + q8 copy), 16 of each per graph."""
    from vybforge_amd import ops
    N, F = 5120, 17408
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    xs = [torch.randn(1, N, generator=gen, device=dev, dtype=torch.float64) for _ in range(16)]
    w = torch.rand(N, generator=gen, device=dev, dtype=torch.float64) + 0.5
    gs = [torch.randn(F, generator=gen, device=dev, dtype=torch.float64) for _ in range(16)]
    u = torch.randn(F, generator=gen, device=dev, dtype=torch.float64)
    launches = [lambda x=x: ops.rmsnorm_q8(x, w, 1e-6, f32_copy=True) for x in xs]
    launches += [lambda g=g: ops.swiglu_q8(g, u) for g in gs]
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    rms_bytes = 8 * N * 2 + 4 * N + N + 4 * (N // 32)
    swi_bytes = 8 * F * 2 + 4 * F + F + 4 * (F // 32)
    per = ms / len(launches)
    value = (rms_bytes + swi_bytes) * 16 / (ms * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(value, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(value / HBM_PEAK_GBS, 4), traffic=None, kernel="k_rms_q8 + k_swiglu_q8",
                    avg_launch_us=round(per * 1e3, 3), bytes_per_launch=(rms_bytes + swi_bytes) // 2)
    return dict(value=value, ms_step=ms, wall=wall, roofline=roofline, flops=0,
                workload="RMSNorm+q8 (1x5120 f64) and SwiGLU+q8 (17408 f64), 16 each per step",
                bytes_per_step=(rms_bytes + swi_bytes) * 16, launches_per_step=len(launches))


def run_router(args, torch, dev):
    """GLM-5 router logits: T tokens of 6144 (bf16) against the 256 x 6144 bf16 gate weight,
    float64 accumulation and output, 8 rotated weight copies per graph."""
    from vybforge_amd import ops
    T, E, H = args.tokens, 256, 6144
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ws = [(torch.randn(E, H, generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(8)]
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    ms, wall = timed_graph(torch, [lambda w=w: ops.router_logits(x, w) for w in ws], args.steps, args.warmup)
    per = ms / len(ws)
    nbytes = E * H * 2 + T * H * 2 + T * E * 8
    value = nbytes / (per * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(value, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(value / HBM_PEAK_GBS, 4), traffic=None, kernel="k_router_logits<bf16, bf16>",
                    avg_launch_us=round(per * 1e3, 3), bytes_per_launch=nbytes)
    return dict(value=value, ms_step=ms, wall=wall, roofline=roofline, flops=2 * T * E * H * len(ws),
                workload=f"GLM-5 router logits T={T}: 256 x 6144 bf16 gate, float64 accumulation",
                bytes_per_step=nbytes * len(ws), launches_per_step=len(ws))


def timed_graph(torch, launches, steps, warmup):
    """Capture the launches as one graph; return (ms per replay, wall seconds)."""
    for f in launches:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in launches:
            f()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps, time.perf_counter() - t0


def run_exl3(args, torch, dev):
    """Config 4: EXL3 4-bpw GEMM K=5120 x N=17408, batch 1 or 16, 8 rotated trellis copies."""
    from vybforge_amd import ops
    K, N, B = 5120, 17408, args.batch
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ncopy = 8
    lins = []
    for _ in range(ncopy):
        t = torch.randint(0, 65536, (K // 16, N // 16, 64), generator=gen, device=dev, dtype=torch.int32).to(torch.uint16)
        suh = ((torch.randn(K, generator=gen, device=dev) * 0.01).abs() * (torch.randint(0, 2, (K,), generator=gen, device=dev) * 2 - 1)).to(torch.float16)
        svh = ((torch.randn(N, generator=gen, device=dev) * 0.01).abs() * (torch.randint(0, 2, (N,), generator=gen, device=dev) * 2 - 1)).to(torch.float16)
        lins.append(ops.Exl3Linear(t, suh, svh, K, N))
    x = torch.randn(B, K, generator=gen, device=dev).to(torch.float16)
    y = torch.empty(B, N, device=dev)
    launches = [lambda L=L: L(x, out=y) for L in lins]
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    per = ms / ncopy
    bytes_call = K * N // 2 + 2 * K + 2 * N + B * (2 * K + 4 * N)
    value = bytes_call / (per * 1e-3) / 1e9
    flops = 2 * K * N * B
    roofline = dict(bound="hbm", achieved=round(value, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(value / HBM_PEAK_GBS, 4), traffic=None,
                    kernel=("k_exl3_gemm, one launch with the x and output rotations" if B <= 2 else
                            "k_exl3_xprep + k_exl3_gemm + k_exl3_out") + " (VALU-bound trellis decode)",
                    avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call)
    return dict(value=value, ms_step=ms, wall=wall, roofline=roofline, flops=flops * ncopy,
                workload=f"EXL3 4-bpw mcg GEMM K=5120 N=17408 batch {B} (8 rotated trellis copies)",
                bytes_per_step=bytes_call * ncopy, launches_per_step=ncopy)


MFMA_BF16_PEAK_TFLOPS = float(ROOFLINE["mfma_dense_TFLOPs"]["bf16"])


def q8_0_blocks_gpu(torch, gen, N, K, dev):
    """Seeded packed Q8_0 rows on the device: fp16 d = |N(0, 0.01)|, int8 uniform in [-127, 127]."""
    nb = N * (K // 32)
    blk = torch.empty((nb, 34), dtype=torch.uint8, device=dev)
    d = (torch.randn(nb, generator=gen, device=dev) * 0.01).abs().to(torch.float16)
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:] = torch.randint(-127, 128, (nb, 32), generator=gen, device=dev, dtype=torch.int8).view(torch.uint8)
    return blk.view(-1)


def run_prefill(args, torch, dev):
    """Config 3: Q8_0 prefill GEMMs M=512 (up K=5120 -> N=17408, down K=17408 -> N=5120), bf16 X,
    f32 Y, 3 rotated weight copies of each (>500 MB, past the 256 MB MALL)."""
    from vybforge_amd import ops
    M = 512
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    shapes = [(17408, 5120), (5120, 17408)]
    ncopy = 3
    ws = ops.GemmWorkspace([(M, N, K) for N, K in shapes], dev, ops.GGML_Q8_0)
    launches, flops, nbytes = [], 0, 0
    for N, K in shapes:
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(M, N, device=dev)
        for _ in range(ncopy):
            W = q8_0_blocks_gpu(torch, gen, N, K, dev)
            launches.append(lambda W=W, x=x, y=y, N=N, K=K: ops.gemm(ops.GGML_Q8_0, W, x, N, K, out=y, workspace=ws))
            flops += 2 * M * N * K
            nbytes += N * K // 32 * 34 + 2 * M * K + 4 * M * N
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    per = ms / len(launches)
    roofline = dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), traffic=None,
                    kernel="k_mmq<Q8_0,bf16> (fp16 MFMA 16x16x32, weights dequantized into operand registers)", avg_launch_us=round(per * 1e3, 3),
                    flops_per_launch=flops // len(launches))
    return dict(value=tflops, unit="TFLOP/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload="Q8_0 prefill GEMMs M=512: 5120->17408 and 17408->5120 (bf16 X, f32 Y)",
                bytes_per_step=nbytes, launches_per_step=len(launches))


MFMA_I8_PEAK_TOPS = float(ROOFLINE["mfma_dense_TFLOPs"]["int8_TOPs"])


def run_prefill_i8(args, torch, dev):
    """Config 3, int8 path: the same two Q8_0 GEMMs with the activations quantized per 32-value
    block (xq8) on the device and int8 MFMA; the quantizer runs inside the timed step."""
    from vybforge_amd import ops
    M = 512
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    shapes = [(17408, 5120), (5120, 17408)]
    ncopy = 3
    ws = ops.GemmWorkspace([(M, N, K) for N, K in shapes], dev, int8=True)
    launches, flops, nbytes = [], 0, 0
    for N, K in shapes:
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        q = (torch.empty(M, K, dtype=torch.int8, device=dev), torch.empty(M, K // 32, device=dev))
        y = torch.empty(M, N, device=dev)
        for _ in range(ncopy):
            W = q8_0_blocks_gpu(torch, gen, N, K, dev)

            def f(W=W, x=x, q=q, y=y, N=N, K=K):
                ops.quant_q8_act(x, out=q)
                ops.gemm_q8_0_i8(W, q[0], q[1], N, K, out=y, workspace=ws)
            launches.append(f)
            flops += 2 * M * N * K
            nbytes += N * K // 32 * 34 + 2 * M * K + 4 * M * N
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    tops = flops / (ms * 1e-3) / 1e12
    per = ms / len(launches)
    roofline = dict(bound="mfma", achieved=round(tops, 2), peak=MFMA_I8_PEAK_TOPS, unit="TOP/s",
                    frac=round(tops / MFMA_I8_PEAK_TOPS, 4), traffic=None,
                    kernel="xq8 + k_mmq_i8 (int8 MFMA 16x16x32 per block, float32 block scaling; VALU-bound)",
                    avg_launch_us=round(per * 1e3, 3), flops_per_launch=flops // len(launches),
                    frac_of_bf16_peak=round(tops / MFMA_BF16_PEAK_TFLOPS, 4))
    return dict(value=tops, unit="TOP/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload="Q8_0 prefill GEMMs M=512 int8 path: xq8(X bf16) then int8 MFMA, 5120->17408 and 17408->5120",
                bytes_per_step=nbytes, launches_per_step=len(launches))


def run_moe(args, torch, dev):
    """Config 5: GLM-5-style MoE layer, H=6144, 256 routed + 1 shared expert, top-8, I=2048,
    q4_0 expert tensors (5.46 GB), T tokens bf16, router logits N(0,1)."""
    from vybforge_amd import ops
    H, I, E, k, T = 6144, 2048, 256, 8, args.tokens
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    wg = q4_0_blocks_gpu(torch, gen, E * I, H, dev)
    wu = q4_0_blocks_gpu(torch, gen, E * I, H, dev)
    wd = q4_0_blocks_gpu(torch, gen, E * H, I, dev)
    sh = (q4_0_blocks_gpu(torch, gen, I, H, dev), q4_0_blocks_gpu(torch, gen, I, H, dev),
          q4_0_blocks_gpu(torch, gen, H, I, dev))
    layer = ops.MoeLayer(ops.GGML_Q4_0, wg, wu, wd, H, I, E, k, shared=sh)
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=gen, device=dev)
    out = torch.empty(T, H, device=dev)
    _, idx, _ = layer(x, logits, out=out, routing=True)
    distinct = int(torch.unique(idx).numel())
    ms, wall = timed_graph(torch, [lambda: layer(x, logits, out=out)], args.steps, args.warmup)
    per_expert = 3 * I * H // 32 * 18
    nbytes = (distinct + 1) * per_expert + T * H * 2 + T * E * 4 + T * H * 4
    flops = T * (k + 1) * 3 * 2 * I * H
    gbs = nbytes / (ms * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(gbs / HBM_PEAK_GBS, 4), traffic=None,
                    kernel=f"MoE layer: route, bucket, {'k_moe_gemv' if T <= 64 else 'k_moe_mm'} gate|up+SwiGLU "
                           "and down over the routed and shared experts, combine",
                    avg_launch_us=round(ms * 1e3, 3), bytes_per_launch=nbytes)
    return dict(value=gbs, ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload=f"GLM-5-style MoE layer T={T}: H=6144, 256+1 experts, top-8, I=2048, q4_0 "
                         f"({distinct} distinct routed experts hit)",
                bytes_per_step=nbytes, launches_per_step=1)


def run_copy(args, torch, dev):
    """Calibration leg for the HBM traffic counters: a plain device copy of known size, 256 MiB
    read + 256 MiB written per step. rocprofv3 FETCH_SIZE / WRITE_SIZE of this run, divided by
    those sizes, give the factors that turn the counters of the other configs into bytes."""
    n = 64 * 1024 * 1024
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    nbytes = 2 * n * 4
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    roofline = dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(gbs / HBM_PEAK_GBS, 4), traffic=None, kernel="torch device copy (calibration)")
    return dict(value=gbs, ms_step=ms_step, wall=wall, roofline=roofline, flops=0,
                workload="device copy 256 MiB -> 256 MiB (counter calibration)", bytes_per_step=nbytes,
                launches_per_step=1)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the fused dequant-matmul path runs on a single GPU "
              "(each GPU would hold a row / expert shard); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        sys.exit("no GPU visible")
    dev = torch.device("cuda:0")
    if args.config == "gemv1":
        r = run_gemv1(args, torch, dev)
    elif args.config == "kquant":
        r = run_kquant(args, torch, dev)
    elif args.config == "producers":
        r = run_producers(args, torch, dev)
    elif args.config == "router":
        r = run_router(args, torch, dev)
    elif args.config == "exl3":
        r = run_exl3(args, torch, dev)
    elif args.config == "prefill":
        r = run_prefill(args, torch, dev)
    elif args.config == "prefill_i8":
        r = run_prefill_i8(args, torch, dev)
    elif args.config == "moe":
        r = run_moe(args, torch, dev)
    elif args.config == "copy":
        r = run_copy(args, torch, dev)
    else:
        r = run_stack(args, torch, dev)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_stack() if args.config in ("stack", "stack_chain") else None
    line = dict(
        metric=METRIC, value=round(r["value"], 2), unit=r.get("unit", "GB/s"), n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=round(r["ms_step"], 4), higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype="f16",
        data="synthetic (seeded q4_0 weights generated on the device, fp16 activations N(0,1))",
        config=dict(workload=r["workload"], bytes_per_step=r["bytes_per_step"],
                    launches_per_step=r["launches_per_step"],
                    hbm_frac=round(r["bytes_per_step"] / (r["ms_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    tflops=round(r["flops"] / (r["ms_step"] * 1e-3) / 1e12, 3)),
        roofline=r["roofline"], cpu_baseline=cpu)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
