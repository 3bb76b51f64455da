#!/usr/bin/env python3
"""Benchmark of the fused dequant-matmul path on one MI355X.

Headline (one "step" = one decoded token): the Qwen3-4B-shaped q4_0 decode linear stack, batch 1,
36 layers x {q 2560->4096, k/v 2560->1024, o 4096->2560, gate/up 2560->9728, down 9728->2560},
fp16 activations, seeded synthetic weights (fp16 scales |N(0, 0.01)|, uniform nibbles). Per layer
four launches (q|k|v fused on one shared x, o, gate|up fused, down), captured once as a HIP graph
and replayed.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|stack|gemv1|...]

The default (``--config all``) prints ONE JSON line: the headline stack figures plus a ``configs``
record per workload of the metric (q4_0 GEMV 9728x2560, Q8_0 prefill GEMM M=512 on both paths,
EXL3 K=5120 N=17408 at batch 1 and 16, the GLM-5 MoE layer at T=1/16/256), each timed with HIP
events on its launch stream and each output checked against the numpy oracle after its timed
region (a mismatch exits non-zero). ``--config X`` runs one workload alone (for profiling).
Inputs are resident in HBM before timing; every workload whose weights fit the 256 MB MALL is
rotated over enough distinct copies to exceed it.
"""

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
# roofline constants (MI355X datasheet, dense) live in roofline.json beside this file
with open(os.path.join(HERE, "roofline.json")) as _f:
    ROOFLINE = json.load(_f)
HBM_PEAK_GBS = float(ROOFLINE["hbm_GBps"])
MFMA_BF16_PEAK_TFLOPS = float(ROOFLINE["mfma_dense_TFLOPs"]["bf16"])
MFMA_I8_PEAK_TOPS = float(ROOFLINE["mfma_dense_TFLOPs"]["int8_TOPs"])
METRIC = "dequant-GEMV GB/s (% HBM peak) + prefill/MoE GEMM TFLOP/s (% MFMA peak)"
GATE = 2e-3  # max|y - ref| / max|ref| against the float64 oracle (native/glm53/verify_layer0.py:134-139)

QWEN3_4B = dict(hidden=2560, q=4096, kv=1024, inter=9728, layers=36)
# HBM bytes per decode-stack launch from rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a plain
# copy's counters), averaged over the four launches of a layer: measured by the profile below,
# not by this run
STACK_TRAFFIC = dict(bytes_per_launch=14413517, source="profiles/q4_0_gemv_decode_stack.md (rocprofv3 --pmc)")

CONFIGS = ["stack", "stack_chain", "gemv1", "kquant", "xq8", "producers", "router", "exl3", "prefill", "prefill_i8",
           "prefill_kq", "moe", "moe_exl3", "pblock", "copy"]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="all", choices=["all"] + CONFIGS)
    ap.add_argument("--wtype", type=int, default=12, choices=[12, 13, 14, 22],
                    help="GGML type id for --config kquant / prefill_kq (12 Q4_K, 13 Q5_K, 14 Q6_K, 22 IQ2_S)")
    ap.add_argument("--tokens", type=int, default=16, help="tokens for --config moe / router")
    ap.add_argument("--batch", type=int, default=1, help="batch for --config exl3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle checks after timing")
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


class CheckFailed(RuntimeError):
    pass


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---- timing ---------------------------------------------------------------------------------

def timed_graph(torch, launches, steps, warmup):
    """Capture the launches as one graph on a side stream; replay warmup + steps times on that
    stream; return (ms per replay from HIP events recorded on the replay stream, wall seconds)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in launches:  # eager warm-up on the capture stream (first-use set-up stays out of the graph)
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in launches:
            f()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(s)
        for _ in range(steps):
            g.replay()
        ev1.record(s)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall


def hbm_roofline(gbs, kernel, basis, traffic=None, **extra):
    r = dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4),
             traffic=traffic, kernel=kernel, basis=basis)
    r.update(extra)
    return r


# ---- oracle checks (outside the timed regions) ------------------------------------------------

def rel_gate(y, ref, dtype_bits=None):
    """max|y - ref| / max|ref|; for 16-bit outputs half an output ulp of ref is forgiven first."""
    import numpy as np
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(y - ref)
    if dtype_bits is not None:
        half = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - dtype_bits - 1)
        d = np.maximum(d - half, 0)
    return float(d.max() / max(float(np.abs(ref).max()), 1e-300))


def expect(name, rel, tol=GATE):
    if not rel < tol:
        raise CheckFailed(f"{name}: rel {rel:.3e} >= {tol:.1e}")
    return float(f"{rel:.3e}")


# ---- synthetic inputs -----------------------------------------------------------------------

def kquant_blocks_gpu(torch, gen, ty, N, K, dev):
    """Seeded packed Q4_K / Q5_K / Q6_K / IQ2_S rows on the device: uniform random bytes, the fp16
    scale fields = |N(0, 1e-4)|."""
    sbytes = {12: 144, 13: 176, 14: 210, 22: 82}[ty]
    nb = N * (K // 256)
    blk = torch.randint(0, 256, (nb, sbytes), generator=gen, device=dev, dtype=torch.uint8)
    for off in {12: (0, 2), 13: (0, 2), 14: (208,), 22: (0,)}[ty]:
        d = (torch.randn(nb, generator=gen, device=dev) * 1e-4).abs().to(torch.float16)
        blk[:, off:off + 2] = d.view(torch.uint8).view(nb, 2)
    return blk.view(-1)


# ---- headline: the decode stack ---------------------------------------------------------------

def build_stack(torch, dev, seed):
    from vybforge_amd import synth
    c = QWEN3_4B
    H, Q, KV, I = c["hidden"], c["q"], c["kv"], c["inter"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q4 = lambda n, k: synth.q4_0_weights_torch(gen, n, k, dev)
    layers = [dict(q=q4(Q, H), k=q4(KV, H), v=q4(KV, H), o=q4(H, Q), gate=q4(I, H), up=q4(I, H), down=q4(H, I))
              for _ in range(c["layers"])]
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


def check_stack(torch, layers, a):
    """The outputs of the last replay are the last layer's: each of its 7 GEMVs against float64."""
    from oracle import matmul
    H, Q, KV, I = QWEN3_4B["hidden"], QWEN3_4B["q"], QWEN3_4B["kv"], QWEN3_4B["inter"]
    L = layers[-1]
    worst = 0.0
    for w, x, y, n, k in [("q", "x_attn", "yq", Q, H), ("k", "x_attn", "yk", KV, H), ("v", "x_attn", "yv", KV, H),
                          ("o", "x_o", "yo", H, Q), ("gate", "x_mlp", "yg", I, H), ("up", "x_mlp", "yu", I, H),
                          ("down", "x_down", "yd", H, I)]:
        ref = matmul.gemv_q4_0_f64(L[w].cpu().numpy(), a[x].float().cpu().numpy(), n, k)[0]
        worst = max(worst, expect(f"stack {w}", rel_gate(a[y].float().cpu().numpy(), ref, 10)))
    return dict(ok=True, rel=worst, what="last layer, all 7 GEMVs (fp16 out), float64 oracle")


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
    ms_step, wall = timed_graph(torch, launches, args.steps, args.warmup)
    value = bytes_tok / (ms_step * 1e-3) / 1e9
    if args.config == "stack_chain":
        st = chain.status()
        if st != 0:
            raise RuntimeError(f"gemv chain reported status {st}")
    n_launch = len(launches)
    per_launch_us = ms_step * 1e3 / n_launch
    achieved = bytes_tok / n_launch / (per_launch_us * 1e-6) / 1e9
    # the graph of launches (not the persistent chain) is what the profile's counters measured
    traffic = STACK_TRAFFIC["bytes_per_launch"] if args.config in ("stack", "all") else None
    roofline = hbm_roofline(achieved, kernel,
                            basis="algorithmic bytes per launch / (HIP-event time of the timed replays / launches); "
                                  "the per-launch time includes the gap between dependent launches",
                            traffic=traffic, traffic_source=STACK_TRAFFIC["source"] if traffic else None,
                            avg_launch_us=round(per_launch_us, 3), bytes_per_launch=round(bytes_tok / n_launch))
    check = None if args.no_check else check_stack(torch, layers, acts)
    return dict(value=value, ms_step=ms_step, wall=wall, roofline=roofline, flops=flops_tok,
                workload="qwen3-4b q4_0 decode linear stack: 36 layers x 7 GEMVs, batch 1, fp16 act",
                bytes_per_step=bytes_tok, launches_per_step=n_launch, check=check)


# ---- CPU baselines: the repo's numpy path (oracle decode + BLAS) on the host's cores ----------------

CPU_RUNS = 5  # timed runs per leg after one warm-up; the median is reported


def _cpu_share():
    """Host threads for the all-cores leg: the affinity mask, capped at the 16-thread share of one
    GPU on a shared host."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(n, 16))


def _cpu_leg(fn, threads):
    """Median wall time of CPU_RUNS calls of fn(threads) after one warm-up; BLAS limited to 1 thread
    per caller thread (the all-cores legs split the work over `threads` host threads themselves)."""
    import statistics
    from threadpoolctl import threadpool_limits
    with threadpool_limits(limits=1):
        fn(threads)
        ts = []
        for _ in range(CPU_RUNS):
            t0 = time.perf_counter()
            fn(threads)
            ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _split(n, parts):
    step = (n + parts - 1) // parts
    return [(a, min(a + step, n)) for a in range(0, n, step)]


def _par(fn, ranges, threads):
    """fn over row ranges on `threads` host threads (numpy releases the GIL in its vector loops)."""
    import concurrent.futures as cf
    if threads == 1:
        return [fn(r) for r in ranges]
    with cf.ThreadPoolExecutor(threads) as ex:
        return list(ex.map(fn, ranges))


def _q4_gemv_rows(raw, N, K, x):
    """The float32 numpy path of one q4_0 GEMV, as a function of a row range."""
    from oracle import formats
    rb = K // 32 * 18
    rows = raw.reshape(N, rb)

    def part(r):
        w = formats.dequant_q4_0(rows[r[0]:r[1]].reshape(-1)).reshape(r[1] - r[0], K)
        return w @ x
    return part


def cpu_baselines():
    """Each configuration's workload (or a bounded sample of it) through this repo's numpy path: the
    oracle's vectorised decode to float32, then numpy matmul (BLAS), 1 thread and the host's thread
    share; the median of CPU_RUNS runs each. Returns {config: record}, records in the units of the GPU
    figures with the same algorithmic bytes / flops."""
    import numpy as np
    from threadpoolctl import threadpool_info
    from oracle import exl3, formats, kquants, matmul, moe
    from vybforge_amd import synth
    ncpu = _cpu_share()
    rng = np.random.default_rng(1)
    out = {}

    def record(value_fn, unit, sample, run, gate=None):
        t1 = _cpu_leg(run, 1)
        tn = _cpu_leg(run, ncpu)
        rec = dict(value=round(value_fn(t1), 4), unit=unit, cores=1, kind="port", sample=sample,
                   median_of=CPU_RUNS, value_all_cores=round(value_fn(tn), 4), cores_all=ncpu)
        if gate is not None:
            tg = _cpu_leg(gate, 1)
            rec["value_fp64_gate"] = round(value_fn(tg), 4)
        return rec

    # the decode stack: one layer's 7 GEMVs (fp16 activations computed in float32)
    shapes, _, _, _ = stack_bytes()
    mats = [(synth.q4_0_weights(rng, n, k), n, k) for n, k in shapes]
    xs = {k: rng.standard_normal(k).astype(np.float16).astype(np.float32) for _, k in shapes}
    layer_bytes = sum(raw.size + 2 * k + 2 * n for raw, n, k in mats)
    parts = [(_q4_gemv_rows(raw, n, k, xs[k]), n) for raw, n, k in mats]

    def stack_run(threads):
        for f, n in parts:
            np.concatenate(_par(f, _split(n, threads), threads))

    def stack_gate(_):
        for raw, n, k in mats:
            matmul.gemv_q4_0_f64(raw, xs[k], n, k)
    out["stack"] = record(lambda t: layer_bytes / t / 1e9, "GB/s",
                          "one layer of the 36-layer q4_0 stack (7 GEMVs, 56.8 MB packed) per run",
                          stack_run, stack_gate)

    # config 1: q4_0 GEMV 9728 x 2560, f32 x
    N, K = 9728, 2560
    raw1 = synth.q4_0_weights(rng, N, K)
    x1 = rng.standard_normal(K).astype(np.float32)
    f1 = _q4_gemv_rows(raw1, N, K, x1)
    b1 = raw1.size + 4 * K + 4 * N
    out["cfg1_q4_0_gemv_9728x2560"] = record(
        lambda t: b1 / t / 1e9, "GB/s", "the whole GEMV per run",
        lambda th: np.concatenate(_par(f1, _split(N, th), th)),
        lambda _: matmul.gemv_q4_0_f64(raw1, x1, N, K))

    # config 3: Q8_0 prefill M = 512, both projections on a 512-column slice of the output
    M, cols = 512, 512
    pre = []
    for N, K in PREFILL_SHAPES:
        raw = synth.q8_0_weights(rng, cols, K)
        pre.append((raw, K, rng.standard_normal((M, K)).astype(np.float32)))
    pflops = sum(2 * M * cols * K for _, K, _ in pre)

    def prefill_run(threads):
        for raw, K, x in pre:
            rows = raw.reshape(cols, K // 32 * 34)
            ws = _par(lambda r: formats.dequant_q8_0(rows[r[0]:r[1]].reshape(-1)).reshape(r[1] - r[0], K),
                      _split(cols, threads), threads)
            w = np.concatenate(ws)
            _par(lambda r: x[r[0]:r[1]] @ w.T, _split(M, threads), threads)
    out["cfg3_q8_0_prefill_m512"] = record(
        lambda t: pflops / t / 1e12, "TFLOP/s",
        "M=512, 5120->17408 and 17408->5120 on 512 output columns each (1.93 GFLOP per run)", prefill_run,
        lambda _: [matmul.gemm_rows_f64(x, matmul.q8_0_matrix(raw, cols, K)) for raw, K, x in pre])

    # config 4: EXL3 K=5120, batch 1 and 16, on a 1024-column slice (the oracle's float64 dequant)
    K, ncol = 5120, 1024
    t4, suh, svh = synth.exl3_tensors(rng, K, ncol)
    for B in (1, 16):
        x4 = rng.standard_normal((B, K)).astype(np.float32)
        b4 = t4.size * 2 + 2 * K + 2 * ncol + B * (2 * K + 4 * ncol)

        def exl3_run(threads, x4=x4):
            w = np.concatenate(_par(lambda r: exl3.dequant_exl3_f64(t4[:, r[0] // 16:r[1] // 16], suh,
                                                                     svh[r[0]:r[1]]).astype(np.float32),
                                    [(128 * a, 128 * b) for a, b in _split(ncol // 128, threads)], threads), axis=1)
            return x4 @ w
        out[f"cfg4_exl3_b{B}"] = record(lambda t: b4 / t / 1e9, "GB/s",
                                        f"K=5120 x 1024 columns of the 17408, batch {B}", exl3_run)

    # config 5: GLM-5 MoE, one routed expert's FFN (3 q4_0 matrices 6144 x 2048) on 2 tokens per run
    H, I = MOE["H"], MOE["I"]
    ex = [synth.q4_0_weights(rng, I, H), synth.q4_0_weights(rng, I, H), synth.q4_0_weights(rng, H, I)]
    x5 = rng.standard_normal((2, H)).astype(np.float32)
    b5 = sum(a.size for a in ex) + 2 * 2 * H + 4 * 2 * H

    def moe_run(threads):
        dq = lambda raw, n, k: np.concatenate(_par(
            lambda r: formats.dequant_q4_0(raw.reshape(n, k // 32 * 18)[r[0]:r[1]].reshape(-1)).reshape(r[1] - r[0], k),
            _split(n, threads), threads))
        wg, wu, wd = dq(ex[0], I, H), dq(ex[1], I, H), dq(ex[2], H, I)
        return moe.swiglu(x5 @ wg.T, x5 @ wu.T) @ wd.T
    out["cfg5_moe"] = record(lambda t: b5 / t / 1e9, "GB/s",
                             "one routed expert's FFN (21.2 MB of q4_0) on 2 tokens per run", moe_run)

    # GLM-5.3 MoE with EXL3 experts: one routed expert's FFN (EXL3 gate / up 4096 -> 2048, down
    # 2048 -> 4096, the oracle's float64 dequant) on 2 tokens per run
    Hx, Ix = MOE53["H"], MOE53["I"]
    mats = [synth.exl3_tensors(rng, Hx, Ix), synth.exl3_tensors(rng, Hx, Ix), synth.exl3_tensors(rng, Ix, Hx)]
    x6 = rng.standard_normal((2, Hx)).astype(np.float32)
    b6 = sum(t.size * 2 + s1.size * 2 + s2.size * 2 for t, s1, s2 in mats) + 2 * 2 * Hx + 4 * 2 * Hx

    def exl3_moe_run(threads):
        def dq(t, su, sv):
            n = sv.size
            return np.concatenate(_par(lambda r: exl3.dequant_exl3_f64(t[:, r[0] // 16:r[1] // 16], su,
                                                                         sv[r[0]:r[1]]).astype(np.float32),
                                       [(128 * a, 128 * b) for a, b in _split(n // 128, threads)], threads), axis=1)
        wg, wu, wd = (dq(*m) for m in mats)
        return moe.swiglu(x6 @ wg, x6 @ wu) @ wd
    out["glm53_moe_exl3"] = record(lambda t: b6 / t / 1e9, "GB/s",
                                   "one routed EXL3 expert's FFN (12.6 MB of trellis) on 2 tokens per run",
                                   exl3_moe_run)

    blas = ", ".join(f"{i.get('internal_api')} {i.get('version')}" for i in threadpool_info()
                     if i.get("user_api") == "blas") or "unknown"
    host = dict(cpu_count=os.cpu_count(), affinity=len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity")
                else None, threads_all_cores=ncpu, blas=blas, omp_num_threads=os.environ.get("OMP_NUM_THREADS"))
    for r in out.values():
        r["host"] = host
    return out


# ---- config 1: one q4_0 GEMV ----------------------------------------------------------------

def run_gemv1(args, torch, dev):
    """q4_0 GEMV 9728x2560, fp32 x, fp32 y, rotating 24 weight copies (336 MB > the MALL)."""
    from oracle import matmul
    from vybforge_amd import ops, synth
    N, K = 9728, 2560
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 1)
    copies = [synth.q4_0_weights_torch(gen, N, K, dev) for _ in range(24)]
    x = torch.randn(K, generator=gen, device=dev)
    y = torch.empty(1, N, device=dev)
    ms, wall = timed_graph(torch, [lambda W=W: ops.gemv(ops.GGML_Q4_0, W, x, N, K, out=y) for W in copies],
                           args.steps, args.warmup)
    per = ms / len(copies)
    bytes_call = N * K // 32 * 18 + 4 * K + 4 * N
    value = bytes_call / (per * 1e-3) / 1e9
    check = None
    if not args.no_check:
        ref = matmul.gemv_q4_0_f64(copies[-1].cpu().numpy(), x.cpu().numpy(), N, K)
        check = dict(ok=True, rel=expect("gemv1", rel_gate(y.cpu().numpy(), ref)), what="last copy, all 9728 rows")
    return dict(value=value, unit="GB/s", ms_step=ms, wall=wall, flops=2 * N * K * len(copies),
                roofline=hbm_roofline(value, "k_gemv_pair<q4_0, f32 x>", "bytes per GEMV / (event time / 24 launches)",
                                      avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call),
                workload="q4_0 GEMV 9728x2560 fp32 x -> fp32 y (24 rotated weight copies)",
                bytes_per_step=bytes_call * len(copies), launches_per_step=len(copies), check=check)


def run_kquant(args, torch, dev):
    """K-quant GEMV at the Qwen3-4B MLP shape 9728x2560 (fp16 x, f32 y), 24 rotated weight copies."""
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
    return dict(value=value, ms_step=ms, wall=wall, flops=2 * N * K * len(copies),
                roofline=hbm_roofline(value, f"k_gemv_pair<{name}>", "bytes per GEMV / (event time / 24 launches)",
                                      avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call),
                workload=f"{name} GEMV 9728x2560 fp16 x (24 rotated copies)",
                bytes_per_step=bytes_call * len(copies), launches_per_step=len(copies))


def run_xq8(args, torch, dev):
    """Decode GEMV on an xq8 activation row (int8 + f32 scale per 32) at 9728x2560, 24 rotated weight
    copies; --wtype 12 / 13 / 22. The last output is checked against the float64 gate of x'."""
    from vybforge_amd import ops
    N, K, ty = 9728, 2560, args.wtype
    if ty not in ops.XQ8_TYPES:
        raise SystemExit("--config xq8 takes --wtype 12, 13 or 22")
    name = {12: "Q4_K", 13: "Q5_K", 22: "IQ2_S"}[ty]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    copies = [kquant_blocks_gpu(torch, gen, ty, N, K, dev) for _ in range(24)]
    xq, xd = ops.quant_q8_act(torch.randn(K, generator=gen, device=dev))
    xq, xd = xq.reshape(K), xd.reshape(K // 32)
    y = torch.empty(N, device=dev)
    ms, wall = timed_graph(torch, [lambda W=W: ops.gemv_xq8(ty, W, xq, xd, N, K, out=y) for W in copies], args.steps,
                           args.warmup)
    per = ms / len(copies)
    bytes_call = ops.row_bytes(ty, K) * N + K + K // 8 + 4 * N
    value = bytes_call / (per * 1e-3) / 1e9
    check = None
    if not args.no_check:
        from oracle import matmul
        ref = matmul.gemv_xq8_f64(ty, copies[-1].cpu().numpy(), xq.cpu().numpy(), xd.cpu().numpy(), N, K)
        check = dict(ok=True, rel=expect(f"xq8 {name}", rel_gate(y.cpu().numpy(), ref), 1e-5),
                     what="last copy, all rows, float64 gate of the xq8-dequantized x")
    return dict(value=value, ms_step=ms, wall=wall, flops=2 * N * K * len(copies),
                roofline=hbm_roofline(value, f"k_gemv_xq8<{name}>", "bytes per GEMV / (event time / 24 launches)",
                                      avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call),
                workload=f"{name} GEMV 9728x2560 on xq8 x (24 rotated copies)",
                bytes_per_step=bytes_call * len(copies), launches_per_step=len(copies), check=check)


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
    return dict(value=value, ms_step=ms, wall=wall, flops=0,
                roofline=hbm_roofline(value, "k_rms_q8 + k_swiglu_q8", "bytes / event time",
                                      avg_launch_us=round(per * 1e3, 3)),
                workload="RMSNorm+q8 (1x5120 f64) and SwiGLU+q8 (17408 f64), 16 each per step",
                bytes_per_step=(rms_bytes + swi_bytes) * 16, launches_per_step=len(launches))


def run_router(args, torch, dev):
    """GLM-5 router logits: T tokens of 6144 (bf16) against the 256 x 6144 bf16 gate weight,
    float64 accumulation and output, 96 rotated weight copies per graph (302 MB > the MALL)."""
    from vybforge_amd import ops
    T, E, H = args.tokens, 256, 6144
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ws = [(torch.randn(E, H, generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(96)]
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    y = torch.empty(T, E, dtype=torch.float64, device=dev)

    def launch(w):
        from vybforge_amd._lib import call
        call("vybdq_router_logits", x.data_ptr(), ops.BF16, w.data_ptr(), ops.BF16, y.data_ptr(), ops.F64, T, E, H,
             torch.cuda.current_stream().cuda_stream)
    ms, wall = timed_graph(torch, [lambda w=w: launch(w) for w in ws], args.steps, args.warmup)
    per = ms / len(ws)
    nbytes = E * H * 2 + T * H * 2 + T * E * 8
    value = nbytes / (per * 1e-3) / 1e9
    return dict(value=value, ms_step=ms, wall=wall, flops=2 * T * E * H * len(ws),
                roofline=hbm_roofline(value, "k_router_logits<bf16, bf16>", "bytes per call / (event time / 96)",
                                      avg_launch_us=round(per * 1e3, 3), bytes_per_launch=nbytes),
                workload=f"GLM-5 router logits T={T}: 256 x 6144 bf16 gate, float64 accumulation (96 rotated copies)",
                bytes_per_step=nbytes * len(ws), launches_per_step=len(ws))


# ---- config 4: EXL3 ---------------------------------------------------------------------------

def run_exl3(args, torch, dev, batch=None):
    """EXL3 4-bpw GEMM K=5120 x N=17408, 8 rotated trellis copies (357 MB > the MALL)."""
    import numpy as np
    from oracle import exl3
    from vybforge_amd import ops
    K, N = 5120, 17408
    B = batch or args.batch
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 4)
    ncopy = 8
    lins = []
    for _ in range(ncopy):
        t = torch.randint(0, 65536, (K // 16, N // 16, 64), generator=gen, device=dev, dtype=torch.int32).to(torch.uint16)
        sgn = lambda n: torch.randint(0, 2, (n,), generator=gen, device=dev) * 2 - 1
        suh = ((torch.randn(K, generator=gen, device=dev) * 0.01).abs() * sgn(K)).to(torch.float16)
        svh = ((torch.randn(N, generator=gen, device=dev) * 0.01).abs() * sgn(N)).to(torch.float16)
        lins.append(ops.Exl3Linear(t, suh, svh, K, N))
    x = torch.randn(B, K, generator=gen, device=dev).to(torch.float16)
    y = torch.empty(B, N, device=dev)
    ms, wall = timed_graph(torch, [lambda L=L: L(x, out=y) for L in lins], args.steps, args.warmup)
    per = ms / ncopy
    bytes_call = K * N // 2 + 2 * K + 2 * N + B * (2 * K + 4 * N)
    value = bytes_call / (per * 1e-3) / 1e9
    check = None
    if not args.no_check:
        L = lins[-1]
        t_last = L.t.view(torch.int16).cpu().numpy().view(np.uint16)
        w = exl3.dequant_exl3_f64(t_last[:, -64:], L.suh.cpu().numpy(), L.svh.cpu().numpy()[-1024:])
        ref = x.to(torch.float64).cpu().numpy() @ w
        check = dict(ok=True, rel=expect(f"exl3 b{B}", rel_gate(y[:, -1024:].cpu().numpy(), ref)),
                     what="last copy, last 1024 columns, float64 oracle")
    kernel = ("k_exl3_gemm, one launch with the x and output rotations" if B <= 2 else
              "k_exl3_xprep + k_exl3_gemm (matrix-core products) + k_exl3_out")
    return dict(value=value, unit="GB/s", ms_step=ms, wall=wall, flops=2 * K * N * B * ncopy,
                roofline=hbm_roofline(value, kernel, "bytes per call / (event time / 8 calls)",
                                      avg_launch_us=round(per * 1e3, 3), bytes_per_launch=bytes_call),
                workload=f"EXL3 4-bpw mcg GEMM K=5120 N=17408 batch {B} fp16 x (8 rotated trellis copies)",
                bytes_per_step=bytes_call * ncopy, launches_per_step=ncopy, check=check)


# ---- config 3: Q8_0 prefill ---------------------------------------------------------------------

PREFILL_SHAPES = [(17408, 5120), (5120, 17408)]  # (N, K): up, down


def _prefill_check(args, name, W, y, N, K, xref, ty=8):
    """The first 256 output columns of a prefill GEMM against the float64 oracle (GGUF type ty)."""
    from oracle import iquants, kquants, matmul
    from vybforge_amd import ops
    if args.no_check:
        return None
    cols = 256
    rb = ops.row_bytes(ty, K)
    raw = W[:cols * rb].cpu().numpy()
    if ty == ops.GGML_Q8_0:
        wrows = matmul.q8_0_matrix(raw, cols, K)
    elif ty == ops.GGML_IQ2_S:
        wrows = iquants.dequant_iq2_s(raw).reshape(cols, K)
    else:
        wrows = kquants.DEQUANT[ty](raw).reshape(cols, K)
    ref = matmul.gemm_rows_f64(xref, wrows)
    return expect(f"{name} N={N} K={K}", rel_gate(y[:, :cols].cpu().numpy(), ref))


def run_prefill(args, torch, dev):
    """Q8_0 prefill GEMMs M=512 (up K=5120 -> N=17408, down K=17408 -> N=5120), bf16 X, f32 Y, 3 rotated
    weight copies of each (568 MB > the MALL)."""
    from vybforge_amd import ops, synth
    M = 512
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 3)
    ncopy = 3
    ws = ops.GemmWorkspace([(M, N, K) for N, K in PREFILL_SHAPES], dev, ops.GGML_Q8_0)
    launches, flops, nbytes, last = [], 0, 0, []
    for N, K in PREFILL_SHAPES:
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(M, N, device=dev)
        for _ in range(ncopy):
            W = synth.q8_0_weights_torch(gen, N, K, dev)
            launches.append(lambda W=W, x=x, y=y, N=N, K=K: ops.gemm(ops.GGML_Q8_0, W, x, N, K, out=y, workspace=ws))
            flops += 2 * M * N * K
            nbytes += N * K // 32 * 34 + 2 * M * K + 4 * M * N
        last.append((W, x, y, N, K))
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    per = ms / len(launches)
    check = None
    if not args.no_check:
        rels = [_prefill_check(args, "prefill", W, y, N, K, x.to(torch.float64).cpu().numpy()) for W, x, y, N, K in last]
        check = dict(ok=True, rel=max(rels), what="last copy of each shape, 512 rows x first 256 columns, float64 oracle")
    roofline = dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), traffic=None,
                    kernel="k_mmq<Q8_0, fp16 X, 8 waves> (bf16 X converted once per GEMM; fp16 MFMA 16x16x32, "
                           "weights dequantized into operand registers)",
                    basis="flops per step / event time", avg_launch_us=round(per * 1e3, 3),
                    flops_per_launch=flops // len(launches))
    return dict(value=tflops, unit="TFLOP/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload="Q8_0 prefill GEMMs M=512: 5120->17408 and 17408->5120 (bf16 X, f32 Y)",
                bytes_per_step=nbytes, launches_per_step=len(launches), check=check)


def run_prefill_kq(args, torch, dev):
    """The prefill GEMM shapes (M=512: 5120->17408 and 17408->5120, bf16 X, f32 Y) on the super-block
    types (--wtype 12 Q4_K, 13 Q5_K, 14 Q6_K, 22 IQ2_S), 3 rotated weight copies of each."""
    from vybforge_amd import ops
    M, ty = 512, args.wtype
    name = {12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 22: "IQ2_S"}[ty]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 6)
    launches, flops, nbytes, last = [], 0, 0, []
    # every type uses the workspace: bf16 X converted once; Q4_K / Q5_K then run the register-operand
    # body, Q6_K / IQ2_S the 128-row tiles (with the K split's partials)
    ws = ops.GemmWorkspace([(M, N, K) for N, K in PREFILL_SHAPES], dev, ty)
    wsa = ws if ws.nbytes else None
    for N, K in PREFILL_SHAPES:
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(M, N, device=dev)
        for _ in range(3):
            W = kquant_blocks_gpu(torch, gen, ty, N, K, dev)
            launches.append(lambda W=W, x=x, y=y, N=N, K=K: ops.gemm(ty, W, x, N, K, out=y, workspace=wsa))
            flops += 2 * M * N * K
            nbytes += ops.row_bytes(ty, K) * N + 2 * M * K + 4 * M * N
        last.append((W, x, y, N, K))
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    check = None
    if not args.no_check:
        rels = [_prefill_check(args, f"prefill_kq {name}", W, y, N, K, x.to(torch.float64).cpu().numpy(), ty)
                for W, x, y, N, K in last]
        check = dict(ok=True, rel=max(rels), what="last copy of each shape, 512 rows x first 256 columns, float64 oracle")
    roofline = dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                    frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), traffic=None,
                    kernel=(f"k_mmq<{name}, fp16 X, 8 waves> (bf16 X converted once per GEMM; weights dequantized "
                            "into operand registers, super-block heads staged in LDS)" if ty in (12, 13) else
                            f"k_kq_mm<{name}> (bf16 X converted once per GEMM; 128-row tiles, runs decoded "
                            "to fp16 in LDS, fp16 MFMA 16x16x32, K split reduced in the workspace)"),
                    basis="flops per step / event time", avg_launch_us=round(ms * 1e3 / len(launches), 3))
    return dict(value=tflops, unit="TFLOP/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload=f"{name} prefill GEMMs M=512: 5120->17408 and 17408->5120 (bf16 X, f32 Y)",
                bytes_per_step=nbytes, launches_per_step=len(launches), check=check)


def run_prefill_i8(args, torch, dev):
    """The same two Q8_0 GEMMs with the activations quantized per 32-value block (xq8) on the device
    and int8 MFMA; the quantizer runs inside the timed step."""
    from oracle import formats
    from vybforge_amd import ops, synth
    M = 512
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 3)
    ncopy = 3
    ws = ops.GemmWorkspace([(M, N, K) for N, K in PREFILL_SHAPES], dev, int8=True)
    launches, flops, nbytes, last = [], 0, 0, []
    for N, K in PREFILL_SHAPES:
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        q = (torch.empty(M, K, dtype=torch.int8, device=dev), torch.empty(M, K // 32, device=dev))
        y = torch.empty(M, N, device=dev)
        for _ in range(ncopy):
            W = synth.q8_0_weights_torch(gen, N, K, dev)

            def f(W=W, x=x, q=q, y=y, N=N, K=K):
                ops.quant_q8_act(x, out=q)
                ops.gemm_q8_0_i8(W, q[0], q[1], N, K, out=y, workspace=ws)
            launches.append(f)
            flops += 2 * M * N * K
            nbytes += N * K // 32 * 34 + 2 * M * K + 4 * M * N
        last.append((W, q, y, N, K))
    ms, wall = timed_graph(torch, launches, args.steps, args.warmup)
    tops = flops / (ms * 1e-3) / 1e12
    per = ms / len(launches)
    check = None
    if not args.no_check:
        rels = [_prefill_check(args, "prefill_i8", W, y, N, K,
                               formats.dequant_q8_act(q[0].cpu().numpy(), q[1].cpu().numpy()).astype("float64"))
                for W, q, y, N, K in last]
        check = dict(ok=True, rel=max(rels), what="last copy of each shape, 512 rows x first 256 columns, float64 "
                                                  "oracle of the xq8-dequantized X")
    roofline = dict(bound="mfma", achieved=round(tops, 2), peak=MFMA_I8_PEAK_TOPS, unit="TOP/s",
                    frac=round(tops / MFMA_I8_PEAK_TOPS, 4), traffic=None,
                    kernel="xq8 + k_mmq_i8 (int8 MFMA 16x16x32 per block, float32 block scaling)",
                    basis="ops per step / event time (the xq8 launches included)", avg_launch_us=round(per * 1e3, 3),
                    flops_per_launch=flops // len(launches), frac_of_bf16_peak=round(tops / MFMA_BF16_PEAK_TFLOPS, 4))
    return dict(value=tops, unit="TOP/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                workload="Q8_0 prefill GEMMs M=512 int8 path: xq8(X bf16) then int8 MFMA, 5120->17408 and 17408->5120",
                bytes_per_step=nbytes, launches_per_step=len(launches), check=check)


# ---- config 5: GLM-5 MoE layer --------------------------------------------------------------------

MOE = dict(H=6144, I=2048, E=256, k=8)


def build_moe(torch, dev, seed):
    from vybforge_amd import ops, synth
    H, I, E, k = MOE["H"], MOE["I"], MOE["E"], MOE["k"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q4 = lambda n, kk: synth.q4_0_weights_torch(gen, n, kk, dev)
    layer = ops.MoeLayer(ops.GGML_Q4_0, q4(E * I, H), q4(E * I, H), q4(E * H, I), H, I, E, k,
                         shared=(q4(I, H), q4(I, H), q4(H, I)))
    return layer, gen


def check_moe(torch, layer, x, logits, out, idx, w, ntok=2):
    """Routing of every token against the oracle router (identical sets, |dw| < 1e-4,
    native/glm53/verify_moe_vyb.py:54-59); ntok tokens' outputs on 256 columns of H against the
    float64 oracle (gate/up of each hit expert and the slice's down rows decoded on the host)."""
    import numpy as np
    from oracle import matmul, moe
    H, I, k = MOE["H"], MOE["I"], MOE["k"]
    rbh, rbi = H // 32 * 18, I // 32 * 18
    T = x.shape[0]
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    ridx, rw = moe.route_logits(logits.to(torch.float64).cpu().numpy(), k)
    for t in range(T):
        a, b = dict(zip(idx[t].tolist(), w[t].tolist())), dict(zip(ridx[t].tolist(), rw[t].tolist()))
        if set(a) != set(b) or max(abs(a[e] - b[e]) for e in a) >= 1e-4:
            raise CheckFailed(f"moe T={T}: routing of token {t} differs from the oracle")
    c0 = (T * 997) % (H - 256) // 64 * 64
    cols = slice(c0, c0 + 256)
    x64 = x.to(torch.float64).cpu().numpy()
    toks = sorted({0, T - 1})[:ntok]

    def ffn(e, xt):
        if e < 0:
            gb, ub, db = layer.shared
        else:
            gb = layer.w[0][e * I * rbh:(e + 1) * I * rbh]
            ub = layer.w[1][e * I * rbh:(e + 1) * I * rbh]
            db = layer.w[2][e * H * rbi:(e + 1) * H * rbi]
        g = matmul.q4_0_matrix(gb.cpu().numpy(), I, H)
        u = matmul.q4_0_matrix(ub.cpu().numpy(), I, H)
        d = matmul.q4_0_matrix(db[c0 * rbi:(c0 + 256) * rbi].cpu().numpy(), 256, I)
        return moe.ffn_rows(xt, g, u, d)[0]
    ref = np.zeros((len(toks), 256))
    for r, t in enumerate(toks):
        xt = x64[t:t + 1]
        ref[r] = sum(rw[t, s] * ffn(int(ridx[t, s]), xt) for s in range(k)) + ffn(-1, xt)
    return expect(f"moe T={T}", rel_gate(out.cpu().numpy()[toks][:, cols], ref))


def run_moe(args, torch, dev, tokens=None, built=None):
    """GLM-5-style MoE layer, H=6144, 256 routed + 1 shared expert, top-8, I=2048, q4_0 expert tensors
    (5.46 GB), T tokens bf16, router logits N(0,1). T <= 16: the step is R layer calls on R distinct
    (x, logits) pairs, each call with its own shared expert (as each layer of a model has), so the
    experts hit per step exceed the 256 MB MALL."""
    from vybforge_amd import ops, synth
    H, E, k = MOE["H"], MOE["E"], MOE["k"]
    I = MOE["I"]
    T = tokens or args.tokens
    base, gen = built or build_moe(torch, dev, args.seed + 5)
    R = 8 if T == 1 else (2 if T <= 16 else 1)
    q4 = lambda n, kk: synth.q4_0_weights_torch(gen, n, kk, dev)
    layers = [base] + [ops.MoeLayer(ops.GGML_Q4_0, *base.w, H, I, E, k, shared=(q4(I, H), q4(I, H), q4(H, I)))
                       for _ in range(R - 1)]
    xs = [torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16) for _ in range(R)]
    lgs = [torch.randn(T, E, generator=gen, device=dev) for _ in range(R)]
    outs = [torch.empty(T, H, device=dev) for _ in range(R)]
    routed = [layers[r](xs[r], lgs[r], routing=True) for r in range(R)]
    distinct = [int(torch.unique(rt[1]).numel()) for rt in routed]
    union = int(torch.unique(torch.cat([rt[1].reshape(-1) for rt in routed])).numel())
    ms, wall = timed_graph(torch, [lambda r=r: layers[r](xs[r], lgs[r], out=outs[r]) for r in range(R)], args.steps,
                           args.warmup)
    per_expert = 3 * I * H // 32 * 18
    nbytes = sum((d + 1) * per_expert + T * H * 2 + T * E * 4 + T * H * 4 for d in distinct)
    flops = R * T * (k + 1) * 3 * 2 * I * H
    gbs = nbytes / (ms * 1e-3) / 1e9
    check = None
    if not args.no_check:
        rels = []
        for r in sorted({0, R - 1}):
            if not torch.equal(outs[r], routed[r][0]):
                raise CheckFailed(f"moe T={T}: graph replay output differs from the eager call")
            rels.append(check_moe(torch, layers[r], xs[r], lgs[r], outs[r], routed[r][1], routed[r][2]))
        check = dict(ok=True, rel=max(rels), what="routing of every token; 2 tokens x 256 columns vs float64 oracle; "
                                                  "graph replay == eager")
    # q4_0 experts: the grouped GEMV at one token, the LDS-staged grouped MFMA GEMM above
    path = "k_moe_gemv" if T <= 1 else "k_moe_mm_lds"
    roofline = hbm_roofline(gbs, f"MoE layer: route+bucket, {path} gate|up+SwiGLU and down, combine",
                            "algorithmic bytes (hit experts + shared + activations) / event time",
                            avg_layer_us=round(ms * 1e3 / R, 3), bytes_per_layer=nbytes // R)
    return dict(value=gbs, unit="GB/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                tflops=round(flops / (ms * 1e-3) / 1e12, 3),
                workload=f"GLM-5-style MoE layer T={T}: H=6144, 256+1 experts, top-8, I=2048, q4_0; {R} layer "
                         f"call(s) per step on distinct inputs, each with its own shared expert "
                         f"({sum(distinct) / R:.1f} routed experts hit per call, {union} distinct per step)",
                bytes_per_step=nbytes, launches_per_step=R, check=check)


# ---- the reference's GLM-5.3 MoE layer: EXL3 routed experts + bf16 shared expert ----------------

MOE53 = dict(H=4096, I=2048, E=288, k=8)


def build_moe_exl3(torch, dev, seed, n_shared=1):
    """288 EXL3 4-bpw experts (distinct seeded trellis, suh/svh = +-|N(0, 0.12)|, so that the expert
    matrices have entries of about N(0, 0.02) like a real checkpoint's; 3.6 GB) and n_shared bf16 shared
    experts (N(0, 0.02)), e_score_correction_bias N(0, 0.05); layer j uses shared expert j."""
    from vybforge_amd import ops
    H, I, E, k = MOE53["H"], MOE53["I"], MOE53["E"], MOE53["k"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    sgn = lambda n: torch.randint(0, 2, (n,), generator=gen, device=dev) * 2 - 1
    sc = lambda n: ((torch.randn(n, generator=gen, device=dev) * 0.12).abs() * sgn(n)).to(torch.float16)
    experts = []
    for _ in range(E):
        ts = []
        for K, N in ((H, I), (H, I), (I, H)):
            t = torch.randint(0, 65536, (K // 16, N // 16, 64), generator=gen, device=dev,
                              dtype=torch.int32).to(torch.uint16).view(torch.int16)
            ts += [t, sc(K), sc(N)]
        experts.append(ts)
    bf = lambda n, kk: (torch.randn(n, kk, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    bias = torch.randn(E, generator=gen, device=dev) * 0.05
    layers = [ops.MoeExl3Layer(experts, H, I, topk=k, shared=(bf(I, H), bf(I, H), bf(H, I)), bias=bias)
              for _ in range(n_shared)]
    return layers, gen


def check_moe_exl3(torch, layer, x, logits, out, idx, w):
    """Routing of every token against the oracle router (bias included; identical ids, |dw| < 1e-4);
    the last token's output on 256 columns of H against float64 (each hit expert decoded on the host,
    its products in the FWHT form x W = svh * fwht(fwht(x * suh) What))."""
    import numpy as np
    from oracle import exl3, moe
    H, k = MOE53["H"], MOE53["k"]
    T = x.shape[0]
    bias = layer.bias.cpu().numpy()
    ridx, rw = moe.route_logits(logits.to(torch.float64).cpu().numpy(), k, bias)
    if not np.array_equal(idx.cpu().numpy(), ridx) or np.abs(w.cpu().numpy() - rw).max() >= 1e-4:
        raise CheckFailed(f"moe_exl3 T={T}: routing differs from the oracle")
    c0 = (T * 997) % (H - 256) // 128 * 128
    t = T - 1
    xt = x[t:t + 1].to(torch.float64).cpu().numpy()
    h = lambda a: a.cpu().numpy().astype(np.float64)
    tr = lambda a: a.view(torch.int16).cpu().numpy().view(np.uint16)
    apply = lambda v, what, suh, svh: exl3.fwht128_rows(exl3.fwht128_rows(v * suh) @ what) * svh
    sg, su, sd = (a.to(torch.float64).cpu().numpy() for a in layer.shared)
    sh_ref = moe.ffn_rows(xt, sg, su, sd[c0:c0 + 256])[0]
    ref = np.zeros(256)
    for s in range(k):
        e = layer.experts[int(ridx[t, s])]
        g = apply(xt, exl3.decode_rotated(tr(e[0])).astype(np.float64), h(e[1]), h(e[2]))
        u = apply(xt, exl3.decode_rotated(tr(e[3])).astype(np.float64), h(e[4]), h(e[5]))
        # the down projection's 256 columns: two 128-column Hadamard blocks
        nb = slice(c0 // 16, (c0 + 256) // 16)
        wd = exl3.decode_rotated(tr(e[6])[:, nb]).astype(np.float64)
        ref += rw[t, s] * apply(moe.swiglu(g, u), wd, h(e[7]), h(e[8])[c0:c0 + 256])[0]
    got = out.cpu().numpy()[t:t + 1, c0:c0 + 256]
    # the whole output, and the routed experts' part alone (the shared expert cannot mask it)
    return max(expect(f"moe_exl3 T={T}", rel_gate(got, (sh_ref + ref)[None])),
               expect(f"moe_exl3 T={T} routed part", rel_gate(got - sh_ref[None], ref[None])))


def run_moe_exl3(args, torch, dev, tokens=None, built=None):
    """The reference's GLM-5.3 MoE layer (native/glm53/glm_engine.vyb:2728-2990) in one call: H=4096,
    288 EXL3 4-bpw routed experts + 1 bf16 shared expert, top-8 with the selection bias, I=2048, T tokens
    bf16. T <= 16: R layer calls per step on distinct inputs, each with its own shared expert."""
    H, I, E, k = MOE53["H"], MOE53["I"], MOE53["E"], MOE53["k"]
    T = tokens or args.tokens
    R = 8 if T == 1 else (2 if T <= 16 else 1)
    layers, gen = built or build_moe_exl3(torch, dev, args.seed + 9, n_shared=R)
    xs = [torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16) for _ in range(R)]
    lgs = [torch.randn(T, E, generator=gen, device=dev) for _ in range(R)]
    outs = [torch.empty(T, H, device=dev) for _ in range(R)]
    routed = [layers[r](xs[r], lgs[r], routing=True) for r in range(R)]
    distinct = [int(torch.unique(rt[1]).numel()) for rt in routed]
    ms, wall = timed_graph(torch, [lambda r=r: layers[r](xs[r], lgs[r], out=outs[r]) for r in range(R)], args.steps,
                           args.warmup)
    per_expert = 3 * H * I // 2 + 3 * 2 * (H + I)   # trellis (4 bits per weight) + suh / svh
    shared = 3 * H * I * 2
    nbytes = sum(d * per_expert + shared + T * H * 2 + T * E * 4 + T * H * 4 for d in distinct)
    flops = R * T * (k + 1) * 3 * 2 * I * H
    gbs = nbytes / (ms * 1e-3) / 1e9
    check = None
    if not args.no_check:
        r = R - 1
        if not torch.equal(outs[r], routed[r][0]):
            raise CheckFailed(f"moe_exl3 T={T}: graph replay output differs from the eager call")
        rel = check_moe_exl3(torch, layers[r], xs[r], lgs[r], outs[r], routed[r][1], routed[r][2])
        check = dict(ok=True, rel=rel, what="routing of every token; the last token x 256 columns vs float64 "
                                            "oracle; graph replay == eager")
    gemm = "k_mx_gemm<1>" if T == 1 else ("k_mx_gemm<2>" if T * k <= 2 * min(E, T * k) else "k_mx_gemm<16>")
    roofline = hbm_roofline(gbs, f"EXL3 MoE layer: route+bucket, x rotation, {gemm} gate|up and down (trellis "
                                 "decoded in registers), SwiGLU between rotations, bf16 shared expert, combine",
                            "algorithmic bytes (hit experts' trellis + scales, shared expert, activations) / "
                            "event time", avg_layer_us=round(ms * 1e3 / R, 3), bytes_per_layer=nbytes // R)
    return dict(value=gbs, unit="GB/s", ms_step=ms, wall=wall, roofline=roofline, flops=flops,
                tflops=round(flops / (ms * 1e-3) / 1e12, 3),
                workload=f"GLM-5.3 MoE layer T={T}: H=4096, 288 EXL3 4-bpw experts + 1 bf16 shared expert, top-8 "
                         f"with selection bias, I=2048; {R} layer call(s) per step on distinct inputs, each with its "
                         f"own shared expert ({sum(distinct) / R:.1f} routed experts hit per call)",
                bytes_per_step=nbytes, launches_per_step=R, check=check)


def exl3_map_file():
    """The reference's map.bin body (256 x 16-byte slots: 4 u16 nibble indices, 4 u8 positions,
    u16 row, u16 col; native/exl3/gen_map_bin.py) followed by its u32 inverse, from the tile-slot
    composition table kept with the test fixtures."""
    import struct
    with open(os.path.join(HERE, "tests", "golden", "exl3_tile_slot_composition.json")) as f:
        slots = sorted(json.load(f)["slots"], key=lambda sl: (sl[0], sl[1]))
    body, inv = b"", [0] * 256
    for i, (r, c, comp) in enumerate(slots):
        body += struct.pack("<4H4BHH", *[m for m, _ in comp], *[p for _, p in comp], r, c)
        inv[r * 16 + c] = i
    return body + struct.pack("<256I", *inv)


def run_pblock(args, torch, dev):
    """vybdq_launch_pblock on the reference's parameter blocks beside the direct entry points, at the
    q4_0 GEMV 9728x2560 (f32 x, 24 rotated weight copies), the four launches of the Qwen3-4B decode
    stack (f32 x, rotated copies over 256 MB each) and the Q8_0 prefill GEMMs M=512 (f32 X,
    3 rotated copies of each shape, no workspace); then the MoE fixture block at S=16 and the fused
    EXL3 decode + column transform at 2048x4096, which have no direct counterpart."""
    import numpy as np
    from vybforge_amd import _lib, ops, synth
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 7)
    stream = lambda: torch.cuda.current_stream().cuda_stream
    out = {}
    N, K = 9728, 2560
    copies = [synth.q4_0_weights_torch(gen, N, K, dev) for _ in range(24)]
    x = torch.randn(K, generator=gen, device=dev)
    y = torch.empty(1, N, device=dev)
    pbs = []
    for W in copies:
        w = np.zeros(32, np.int64)
        w[0:7] = [W.data_ptr(), x.data_ptr(), y.data_ptr(), 1, N, K, 4]
        w[10], w[14] = 8, 8
        pbs.append(torch.from_numpy(w).to(dev))
    ms_d, _ = timed_graph(torch, [lambda W=W: ops.gemv(ops.GGML_Q4_0, W, x, N, K, out=y) for W in copies],
                          args.steps, args.warmup)
    ms_p, _ = timed_graph(torch, [lambda pb=pb: _lib.call("vybdq_launch_pblock", _lib.PB_GEMV + 2, pb.data_ptr(),
                                                             stream()) for pb in pbs], args.steps, args.warmup)
    b = N * K // 32 * 18 + 4 * K + 4 * N
    out["gemv_q4_0_9728x2560"] = dict(direct_us=round(ms_d * 1e3 / 24, 3), pblock_us=round(ms_p * 1e3 / 24, 3),
                                      direct_GBs=round(b / (ms_d / 24 * 1e-3) / 1e9, 1),
                                      pblock_GBs=round(b / (ms_p / 24 * 1e-3) / 1e9, 1))
    del copies, pbs
    # the four launches of the Qwen3-4B decode stack (q|k|v, o, gate|up, down), f32 x, rotated copies
    # of each (> 256 MB per shape)
    H, Q, KV, I = QWEN3_4B["hidden"], QWEN3_4B["q"], QWEN3_4B["kv"], QWEN3_4B["inter"]
    for name, Kk, Ns in (("qkv", H, (Q, KV, KV)), ("o", Q, (H,)), ("gate_up", H, (I, I)), ("down", I, (H,))):
        nb = sum(Ns) * Kk // 32 * 18
        nc = (300 << 20) // nb + 1
        xs = torch.randn(Kk, generator=gen, device=dev)
        ys = [torch.empty(n, device=dev) for n in Ns]
        sets = [[synth.q4_0_weights_torch(gen, n, Kk, dev) for n in Ns] for _ in range(nc)]
        blocks = []
        for Ws in sets:
            w = np.zeros(32, np.int64)
            w[1], w[3], w[5] = xs.data_ptr(), 1, Kk
            for i, (slot_w, slot_y, slot_n, slot_e) in enumerate(((0, 2, 4, 6), (7, 9, 8, 10), (11, 13, 12, 14))):
                if i < len(Ns):
                    w[slot_w], w[slot_y], w[slot_n], w[slot_e] = Ws[i].data_ptr(), ys[i].data_ptr(), Ns[i], 4
                else:
                    w[slot_e] = 8
            blocks.append(torch.from_numpy(w).to(dev))
        ms_d, _ = timed_graph(torch, [lambda Ws=Ws: ops.gemv_seg3(ops.GGML_Q4_0, xs, Kk, list(zip(Ws, ys, Ns)))
                                      for Ws in sets], args.steps, args.warmup)
        ms_p, _ = timed_graph(torch, [lambda pb=pb: _lib.call("vybdq_launch_pblock", _lib.PB_GEMV + 2, pb.data_ptr(),
                                                                 stream()) for pb in blocks], args.steps, args.warmup)
        out[f"gemv_stack_{name}"] = dict(direct_us=round(ms_d * 1e3 / nc, 3), pblock_us=round(ms_p * 1e3 / nc, 3),
                                         ratio=round(ms_p / ms_d, 3))
        del sets, blocks
    M = 512
    direct, pblk, flops = [], [], 0
    keep = []
    for Nn, Kk in PREFILL_SHAPES:
        X = torch.randn(M, Kk, generator=gen, device=dev)
        Y = torch.empty(M, Nn, device=dev)
        for _ in range(3):
            W = synth.q8_0_weights_torch(gen, Nn, Kk, dev)
            direct.append(lambda W=W, X=X, Y=Y, Nn=Nn, Kk=Kk: ops.gemm(ops.GGML_Q8_0, W, X, Nn, Kk, out=Y))
            w = np.zeros(32, np.int64)
            w[0:10] = [W.data_ptr(), X.data_ptr(), Y.data_ptr(), M, Nn, Kk, -Nn, 0, 0, (M + 63) // 64]
            pb = torch.from_numpy(w).to(dev)
            pblk.append(lambda pb=pb: _lib.call("vybdq_launch_pblock", _lib.PB_GEMM + 8, pb.data_ptr(), stream()))
            keep += [W, X, Y, pb]
            flops += 2 * M * Nn * Kk
    ms_d, _ = timed_graph(torch, direct, args.steps, args.warmup)
    ms_p, _ = timed_graph(torch, pblk, args.steps, args.warmup)
    out["gemm_q8_0_prefill_m512_f32x"] = dict(direct_tflops=round(flops / (ms_d * 1e-3) / 1e12, 1),
                                              pblock_tflops=round(flops / (ms_p * 1e-3) / 1e12, 1))
    n_gemm = len(pblk)
    del keep, direct, pblk
    # the MoE fixture block (dense f32 expert weights, H=4096, I=2048, 288 experts, top-8) at S=16
    S, H, I, E = 16, 4096, 2048, 288
    mw = [torch.randn(*sh, generator=gen, device=dev) * 0.02 for sh in [(H, I), (H, I), (I, H)] * 2]
    my = torch.randn(S, H, generator=gen, device=dev)
    mg = torch.randn(E, H, generator=gen, device=dev) * 0.03
    mb = torch.zeros(E, device=dev)
    mo = [torch.empty(n, device=dev) for n in (S * E, S * 8, S * 8, S * 9 * I, S * H)]
    words = np.array([my.data_ptr(), mg.data_ptr(), mb.data_ptr(), mo[0].data_ptr(), mo[1].data_ptr(),
                      mo[2].data_ptr(), mo[3].data_ptr(), *[w.data_ptr() for w in mw], mo[4].data_ptr(), S], np.int64)
    mpb = torch.from_numpy(words).to(dev)
    ms_m, _ = timed_graph(torch, [lambda: _lib.call("vybdq_launch_pblock", _lib.PB_MOE, mpb.data_ptr(), stream())],
                          args.steps, args.warmup)
    mbytes = sum(w.numel() * 4 for w in mw) + mg.numel() * 4
    out["moe_fixture_s16"] = dict(us=round(ms_m * 1e3, 2), weight_GBs=round(mbytes / (ms_m * 1e-3) / 1e9, 1))
    del mw, mo
    # the fused EXL3 decode + column transform (exl3dq1s) of the 2048 x 4096 down_proj the map is for
    rows, cw = 2048, 4096
    q = torch.randint(0, 256, ((rows // 16) * (cw // 16) * 128,), generator=gen, device=dev, dtype=torch.uint8)
    td = torch.from_numpy(np.frombuffer(np.array([cw, rows * cw // 256], "<i8").tobytes() + exl3_map_file(),
                                        np.uint8).copy()).to(dev)
    Hm = torch.tensor([[1.0 if bin(r & c).count("1") % 2 == 0 else -1.0 for c in range(128)] for r in range(128)],
                      device=dev) / 128 ** 0.5  # Sylvester Hadamard-128, orthonormal
    T = torch.empty(rows * cw, device=dev)
    xpb = torch.tensor([q.data_ptr(), td.data_ptr(), Hm.data_ptr(), T.data_ptr(), cw, td.data_ptr() + 16 + 4096],
                       dtype=torch.int64, device=dev)
    ms_x, _ = timed_graph(torch, [lambda: _lib.call("vybdq_launch_pblock_grid", _lib.PB_EXL3DQ, xpb.data_ptr(),
                                                    rows * cw // 256, 256, stream())], args.steps, args.warmup)
    out["exl3dq_2048x4096"] = dict(us=round(ms_x * 1e3, 2),
                                   tflops=round(2 * rows * cw * 128 / (ms_x * 1e-3) / 1e12, 1),
                                   out_GBs=round(rows * cw * 4 / (ms_x * 1e-3) / 1e9, 1))
    # the other stages of the reference's f32 reconstruction at the same shape: exl3deq32 (map
    # decode), exl3had132, exl3had232 (with suh / svh), exl3cvt32, and the exl3_deq32 chain
    # dq1s -> had232 -> cvt32 as one graph
    nbc, nblocks = cw // 128, rows // 128 * (cw // 128)
    su = torch.ones(rows, dtype=torch.float16, device=dev)
    sv = torch.ones(cw, dtype=torch.float16, device=dev)
    od = torch.empty(rows * cw, device=dev)
    fd = torch.empty(rows * cw, device=dev)
    f64 = torch.empty(rows * cw, dtype=torch.float64, device=dev)
    i64 = lambda ws: torch.tensor([int(w) for w in ws], dtype=torch.int64, device=dev)
    p1 = i64([od.data_ptr(), T.data_ptr(), Hm.data_ptr(), cw, nbc, nblocks])
    p2 = i64([T.data_ptr(), fd.data_ptr(), Hm.data_ptr(), su.data_ptr(), sv.data_ptr(), cw, nbc, nblocks])
    p3 = i64([fd.data_ptr(), f64.data_ptr(), rows * cw])
    deq = lambda: _lib.call("vybdq_exl3_deq_map", q.data_ptr(), td.data_ptr(), od.data_ptr(), _lib.F32, stream())
    had1 = lambda: _lib.call("vybdq_launch_pblock", _lib.PB_EXL3HAD132, p1.data_ptr(), stream())
    had2 = lambda: _lib.call("vybdq_launch_pblock", _lib.PB_EXL3HAD232, p2.data_ptr(), stream())
    cvt = lambda: _lib.call("vybdq_launch_pblock", _lib.PB_EXL3CVT32, p3.data_ptr(), stream())
    dq1s = lambda: _lib.call("vybdq_launch_pblock_grid", _lib.PB_EXL3DQ, xpb.data_ptr(), rows * cw // 256, 256, stream())
    stages = {}
    for name, fns in [("deq32", [deq]), ("had132", [had1]), ("had232", [had2]), ("cvt32", [cvt]),
                      ("chain_dq1s_had232_cvt32", [dq1s, had2, cvt])]:
        ms_s, _ = timed_graph(torch, fns, args.steps, args.warmup)
        stages[name + "_us"] = round(ms_s * 1e3, 2)
    out["exl3_stages_2048x4096"] = stages
    del od, fd, f64
    if _lib.lib.vybdq_pblock_status() != 0:
        raise CheckFailed("a p-block launch reported: " + _lib.last_error())
    ratio = out["gemv_q4_0_9728x2560"]["direct_us"] / out["gemv_q4_0_9728x2560"]["pblock_us"]
    return dict(value=ratio, unit="x", ms_step=ms_p, wall=0.0, flops=flops, roofline=out,
                workload="vybdq_launch_pblock vs the direct entry points (GEMV 9728x2560 q4_0, Q8_0 prefill M=512)",
                bytes_per_step=0, launches_per_step=n_gemm)


def run_copy(args, torch, dev):
    """Calibration leg for the HBM traffic counters: a plain device copy of known size, 256 MiB
    read + 256 MiB written per step. rocprofv3 FETCH_SIZE / WRITE_SIZE of this run, divided by
    those sizes, give the factors that turn the counters of the other configs into bytes."""
    n = 64 * 1024 * 1024
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)
    ms, wall = timed_graph(torch, [lambda: dst.copy_(src)], args.steps, args.warmup)
    nbytes = 2 * n * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(value=gbs, ms_step=ms, wall=wall, flops=0,
                roofline=hbm_roofline(gbs, "torch device copy (calibration)", "bytes / event time"),
                workload="device copy 256 MiB -> 256 MiB (counter calibration)", bytes_per_step=nbytes,
                launches_per_step=1)


# ---- driver ---------------------------------------------------------------------------------------

def sub_record(r):
    rec = dict(workload=r["workload"], value=round(r["value"], 2), unit=r.get("unit", "GB/s"),
               ms_per_step=round(r["ms_step"], 4), roofline=r["roofline"], check=r.get("check"))
    if "tflops" in r:
        rec["tflops"] = r["tflops"]
    return rec


def run_all(args, torch, dev):
    """Every workload of the metric, each as a sub-record (at most 100 timed replays after at most
    10 warm-up replays; each replay is 0.3-15 ms of GPU work)."""
    import copy
    sub = copy.copy(args)
    sub.steps, sub.warmup = max(5, min(args.steps, 100)), max(2, min(args.warmup, 10))
    recs = {}

    def leg(name, fn, *a, **kw):
        log(f"config {name} ...")
        t0 = time.perf_counter()
        r = fn(sub, torch, dev, *a, **kw)
        recs[name] = sub_record(r)
        recs[name].update(steps=sub.steps, warmup=sub.warmup)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        log(f"config {name}: {recs[name]['value']} {recs[name]['unit']} ({time.perf_counter() - t0:.1f} s)")

    leg("cfg1_q4_0_gemv_9728x2560", run_gemv1)
    leg("cfg3_q8_0_prefill_m512_fp16mfma", run_prefill)
    leg("cfg3_q8_0_prefill_m512_int8mfma", run_prefill_i8)
    leg("cfg4_exl3_b1", run_exl3, batch=1)
    leg("cfg4_exl3_b16", run_exl3, batch=16)
    built = build_moe(torch, dev, args.seed + 5)
    for T in (1, 16, 256):
        leg(f"cfg5_moe_T{T}", run_moe, tokens=T, built=built)
    del built
    torch.cuda.empty_cache()
    built = build_moe_exl3(torch, dev, args.seed + 9, n_shared=8)
    for T in (1, 16, 256):
        leg(f"glm53_moe_exl3_T{T}", run_moe_exl3, tokens=T, built=built)
    del built
    torch.cuda.empty_cache()
    return recs


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the fused dequant-matmul path runs on a single GPU "
              "(each GPU would hold a row / expert shard); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, HERE)
    import torch
    if not torch.cuda.is_available():
        sys.exit("no GPU visible")
    dev = torch.device("cuda:0")
    runners = dict(gemv1=run_gemv1, kquant=run_kquant, xq8=run_xq8, producers=run_producers, router=run_router, exl3=run_exl3,
                   prefill=run_prefill, prefill_i8=run_prefill_i8, prefill_kq=run_prefill_kq, moe=run_moe,
                   moe_exl3=run_moe_exl3,
                   pblock=run_pblock, copy=run_copy)
    configs = None
    try:
        if args.config in ("all", "stack", "stack_chain"):
            log("headline: decode stack ...")
            r = run_stack(args, torch, dev)
            torch.cuda.empty_cache()
            if args.config == "all":
                configs = run_all(args, torch, dev)
        else:
            r = runners[args.config](args, torch, dev)
    except CheckFailed as e:
        print(f"bench.py: output check failed: {e}", file=sys.stderr)
        sys.exit(3)
    cpu = None
    if not args.no_cpu and args.config in ("all", "stack", "stack_chain"):
        log("cpu baselines ...")
        t0 = time.perf_counter()
        cpus = cpu_baselines()
        log(f"cpu baselines: {time.perf_counter() - t0:.1f} s")
        cpu = cpus["stack"]
        for name, rec in (configs or {}).items():
            key = max((k for k in cpus if name == k or name.startswith(k + "_")), key=len, default=None)
            if key is not None:
                rec["cpu_baseline"] = cpus[key]
    line = dict(
        metric=METRIC, value=round(r["value"], 2), unit=r.get("unit", "GB/s"), n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=round(r["ms_step"], 4), higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype="f16",
        data="synthetic (seeded q4_0 / Q8_0 / EXL3 weights generated on the device, activations N(0,1))",
        config=dict(workload=r["workload"], bytes_per_step=r["bytes_per_step"],
                    launches_per_step=r["launches_per_step"],
                    hbm_frac=round(r["bytes_per_step"] / (r["ms_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    tflops=round(r["flops"] / (r["ms_step"] * 1e-3) / 1e12, 3)),
        roofline=r["roofline"], cpu_baseline=cpu, check=r.get("check"))
    if configs is not None:
        line["configs"] = configs
    print(json.dumps(line))


if __name__ == "__main__":
    main()
