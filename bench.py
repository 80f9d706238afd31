"""Benchmark: one GPT-OSS-120B-shaped pipeline stage's continuous-batch forward step on one MI355X.

Workload (default, c1): 9 decoder layers (sliding window 128 on even layers, full attention on odd),
64 query / 8 KV heads of dim 64 with learned sinks, 128-expert top-4 MXFP4 MoE (H = I = 2880); a
ragged batch of 32 sequences -- 24 single-token decode rows and 8 four-token spec-verify rows (56
tokens) -- with per-sequence KV length uniform in [512, 8192]; KV and activations bf16 N(0,1),
weights random-init (synthetic data, seed 0).

A step is one stage forward over that batch.  value = tokens / second over the timed steps, inputs
resident in HBM.  Beside it:
* roofline -- the dominant kernel (the MXFP4 gate_up expert GEMM), HIP events on the stream it runs
  on; its algorithmic bytes count every touched expert's codes, scales and bias once plus
  activations in and out;
* moe_layer_us -- one MoE block as a unit: route + top-k/permute, gate_up, down, combine (HIP
  events over 100 replays after 20 warmup calls, the reference's convention,
  research/v4_fp8_gemv_bench.py:11-17);
* hbm_read_ceiling -- what a kernel that only streams reads reaches on this GPU;
* cpu_baseline -- the CPU oracle on one sliding and one full layer of the same batch (warmup, then
  the median of 3), scaled to the 9-layer stage; for c2 and c4 on a stated subset of the rows (the
  chunk's last rows and decode rows), since one oracle layer of a whole prefill chunk takes minutes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

--workload c2: one 2048-token prefill chunk (prior KV 4096) + 48 decode rows on the same stage.
--workload c3: the DeepSeek-V3-shaped FP8 stage: 4 MoE layers (H 7168, 256 experts, top-8 grouped
  sigmoid routing with a Zipf-shaped selection bias, one shared expert, I 2048, e4m3 weights with
  128x128 E8M0 block scales), a ragged batch of 64 sequences of 1, 2 or 4 tokens.
--workload wire: activation frames over loopback TCP, HBM to HBM (decode rows h[8, 4, 2880] and a
  4096-token prefill chunk), through the pageable path and the pinned ring.
"""
import argparse
import json
import os
import socket
import statistics
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 5000.0}
READ_PROBE_WG_PER_CU = 8   # workgroups per CU of the read-streaming probe
# sizes of the read probe's shorter runs: about one projection weight, one down and one gate_up launch
READ_PROBE_SIZES_MIB = (30, 454, 903)


# ---- workloads -----------------------------------------------------------------------------------

def c1_batch(seed=0):
    """32 sequences: 24 single-token decode rows, 8 four-token verify rows; KV U[512, 8192]."""
    rng = np.random.default_rng(seed)
    q_lens = [1] * 24 + [4] * 8
    starts = [int(v) for v in rng.integers(512, 8192 + 1, size=32)]
    return q_lens, starts


def c2_batch(seed=0):
    """One 2048-token prefill chunk at prior KV 4096 plus 48 single-token decode rows."""
    rng = np.random.default_rng(seed)
    return [2048] + [1] * 48, [4096] + [int(v) for v in rng.integers(512, 8192 + 1, size=48)]


def c3_batch(seed=0):
    rng = np.random.default_rng(seed)
    return [int(v) for v in rng.choice([1, 2, 4], size=64)]


C4_MAXLEN = 32768


def c4_batch(seed=4, S=256):
    """256 sequences: Zipf(2.2) query lengths capped at 8 (mostly single-token decode, verify chunks up
    to 8), two of them 1024-token prefill chunks; KV lengths log-uniform in [128, 32768]."""
    rng = np.random.default_rng(seed)
    q = np.minimum(rng.zipf(2.2, size=S), 8)
    prefill = rng.choice(S, size=2, replace=False)
    q[prefill] = 1024
    kv = np.exp(rng.uniform(np.log(128), np.log(C4_MAXLEN), size=S)).astype(np.int64)
    starts = np.maximum(kv - q, 0)
    return [int(v) for v in q], [int(v) for v in starts], [int(v) for v in prefill]


def c4_skew_router(layer, E, seed=9, boost=1.2):
    """The stress routing: +boost on the router bias of 10% of the experts, which then take about half
    of the token-assignments."""
    import torch
    hot = torch.randperm(E, generator=torch.Generator().manual_seed(seed))[:E // 10]
    rb = layer.router_b.float()
    rb[hot.to(rb.device)] += boost
    layer.router_b = rb.to(torch.bfloat16)


def gate_up_algorithmic_bytes(shape, hist, T, k):
    """Touched experts' gate_up codes + scales + fp32 bias, once each, plus x in, h out, perm."""
    H, I = shape.hidden, shape.intermediate
    touched = int((hist > 0).sum())
    per_expert = (2 * I) * H // 2 + (2 * I) * H // 32 + 4 * (2 * I)
    return touched * per_expert + T * H * 2 + T * k * I * 2 + T * k * 4, touched


def down_algorithmic_bytes(shape, hist, T, k):
    H, I = shape.hidden, shape.intermediate
    touched = int((hist > 0).sum())
    per_expert = H * I // 2 + H * I // 32 + 4 * H
    return touched * per_expert + T * k * I * 2 + T * k * H * 4, touched


def moe_layer_algorithmic_bytes(shape, hist, T, k):
    """The MoE block's bytes (route + permute + experts + combine): every touched expert's weights,
    scales and biases once, x in (router and experts), y out, ids and weights."""
    H, I, E = shape.hidden, shape.intermediate, shape.n_experts
    touched = int((hist > 0).sum())
    per_expert = 2 * I * H // 2 + 2 * I * H // 32 + H * I // 2 + H * I // 32 + 4 * (2 * I + H)
    return touched * per_expert + E * H * 2 + T * H * 2 + T * H * 2 + T * k * 8


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=9)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--moe-reps", type=int, default=100)
    ap.add_argument("--read-probe-mib", type=int, default=2048,
                    help="buffer size of the HBM read-streaming ceiling (0: skip)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after timing, copy a buffer of this many MiB 3 times (a known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    ap.add_argument("--workload", choices=("c0", "c1", "c2", "c3", "c4", "wire"), default="c1")
    ap.add_argument("--frames", type=int, default=20, help="--workload wire: frames per path")
    ap.add_argument("--split-keys", type=int, default=1024,
                    help="keys per attention item of the GPT-OSS stages (a multiple of 64)")
    ap.add_argument("--dense", choices=("fp8", "bf16"), default="bf16",
                    help="--workload c2: dense expert groups on the scaled MFMA with two-term fp8 activations "
                         "(fp8) or on the bf16-activation tiled GEMM (bf16)")
    ap.add_argument("--graphs", action="store_true",
                    help="replay the stage step as a HIP graph (measured slower than direct launches "
                         "on this stack, so off by default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the stage is single-GPU by design: no collectives, no sharding)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "c0":
        run_c0(args)
    elif args.workload == "c3":
        run_c3(args)
    elif args.workload == "wire":
        run_wire(args)
    else:
        run_gptoss(args, args.workload)


# ---- measurement helpers ---------------------------------------------------------------------------

def copy_probe(mib, dev):
    import torch
    if mib > 0:
        src = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()


def hip_event_us(fn, reps, warmup=0):
    """Average microseconds of fn() over reps calls (HIP events on the current stream, which is the
    stream flyai_amd.ops passes to the library)."""
    import torch
    for _ in range(warmup):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def hbm_read_ceiling(mib, dev, reps=20, grid_per_cu=None):
    """GB/s of a read-only streaming kernel over `mib` MiB (normal and nontemporal loads)."""
    import ctypes as C
    import torch
    from flyai_amd._lib import check, lib
    if mib <= 0:
        return None
    buf = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    grid = cus * (grid_per_cu or READ_PROBE_WG_PER_CU)
    out = {"bytes": buf.numel(), "grid": grid}
    for name, nt in (("normal_GBps", 0), ("nontemporal_GBps", 1)):
        def run():
            check(lib().flyai_hbm_read_probe(C.c_void_p(buf.data_ptr()), buf.numel(), nt, grid,
                                             C.c_void_p(sink.data_ptr()),
                                             C.c_void_p(torch.cuda.current_stream().cuda_stream)))
        us = hip_event_us(run, reps, warmup=3)
        out[name] = round(buf.numel() / (us * 1e-6) / 1e9, 1)
    # smaller reads, each launch on the next slice of the buffer (a slice is not re-read before the
    # others, so its bytes are gone from the 256 MiB memory-side cache): the time a kernel that only
    # streams that many bytes takes, launch included -- the floor for a kernel of the same bytes
    by_size = {}
    for smib in READ_PROBE_SIZES_MIB:
        nslice = mib // smib
        if nslice < 2:
            continue
        nbytes = smib << 20
        turn = [0]

        def run_slice():
            off = (turn[0] % nslice) * nbytes
            turn[0] += 1
            check(lib().flyai_hbm_read_probe(C.c_void_p(buf.data_ptr() + off), nbytes, 1, grid,
                                             C.c_void_p(sink.data_ptr()),
                                             C.c_void_p(torch.cuda.current_stream().cuda_stream)))
        us = hip_event_us(run_slice, max(reps, 2 * nslice), warmup=3)
        by_size[f"{smib}MiB"] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    out["nontemporal_by_size"] = by_size
    del buf
    return out


def committed_traffic(profile, kernels):
    """HBM bytes of one launch of each named kernel (FETCH_SIZE + WRITE_SIZE per dispatch, calibrated
    against a plain copy: flyai_amd.profiling), summed, from a counters profile committed under
    profiles/; None when the profile or a kernel is missing.  A kernel name matches by prefix; of
    several launch shapes of it, the one with the most dispatches is taken."""
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        ents = json.load(f)
    total = 0
    for name in kernels:
        hits = [e for e in ents if e["kernel"].startswith(name) and "FETCH_SIZE_bytes" in e]
        if not hits:
            return None
        e = max(hits, key=lambda x: x.get("calls") or 0)
        total += e["FETCH_SIZE_bytes"] + e.get("WRITE_SIZE_bytes", 0.0)
    return int(round(total))


def cpu_threads():
    """Intra-op threads for the CPU oracle: every CPU this process may run on (its affinity mask,
    which is the host's CPU share), unless OMP_NUM_THREADS narrows it."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "").strip()
    return max(1, min(n, int(env))) if env.isdigit() else n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def timed_median(fn, runs=3, warmup=1):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


# ---- GPT-OSS stage (c1, c2) ------------------------------------------------------------------------

def run_gptoss(args, workload="c1"):
    import torch
    from flyai_amd import ops
    from flyai_amd.rope import YarnRotary
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    from flyai_amd.weights import GptOssShape, synthetic_layer

    dev = "cuda"
    torch.cuda.set_device(0)
    shape = GptOssShape()
    chunked_prefill = workload in ("c2", "c4")   # prefill-sized expert groups: the MFMA roofline
    caps = None
    prefill_seqs = []
    if workload == "c4":
        q_lens, starts, prefill_seqs = c4_batch()
        caps = [s_ + q_ for s_, q_ in zip(starts, q_lens)]   # a per-sequence workspace, sized to each context
        maxlen = C4_MAXLEN + 64
    else:
        q_lens, starts = c2_batch(0) if workload == "c2" else c1_batch(0)
        maxlen = 8192 + 64
    S, T = len(q_lens), sum(q_lens)
    E, k = shape.n_experts, shape.top_k
    with_cpu = not args.no_cpu
    print(f"[bench] building {args.layers}-layer stage ...", file=sys.stderr, flush=True)
    layers = [synthetic_layer(shape, 1000 + i, dev, sliding=(i % 2 == 0), keep_hf=(i < 2 and with_cpu))
              for i in range(args.layers)]
    if workload == "c4":
        for lw_ in layers:
            c4_skew_router(lw_, E)
    rot = YarnRotary(maxlen, device=dev)
    kv = KVWorkspace(args.layers, S, maxlen, shape.n_kv_heads, shape.head_dim, dev, caps=caps)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    for t in kv.k + kv.v:
        t.copy_(torch.randn(t.shape, device=dev, generator=g).to(torch.bfloat16))
    hidden0 = torch.randn(T, shape.hidden, device=dev, generator=g).to(torch.bfloat16)
    cpu_inputs = None
    cpu_rows = cpu_sub = None
    if with_cpu:   # the oracle's copies of layers 0-1 and their KV, taken before any step writes
        if chunked_prefill:   # a stated subset of the rows (the whole chunk takes minutes per layer)
            cpu_rows, cpu_sub = cpu_row_subset(workload, q_lens, starts, prefill_seqs)
            cpu_inputs = cpu_layer_inputs(layers[:2], kv, hidden0[torch.as_tensor(cpu_rows, device=dev)],
                                          cpu_sub["slots"])
        else:
            cpu_inputs = cpu_layer_inputs(layers[:2], kv, hidden0, list(range(S)))
    fp8 = chunked_prefill and args.dense == "fp8"
    stage = RaggedStage(shape, layers, rot, kv, max_tokens=max(64, T), max_seqs=S, use_graphs=args.graphs,
                        dense_fp8=fp8, split_keys=args.split_keys)
    slots = list(range(S))
    torch.cuda.synchronize()
    print("[bench] warmup", file=sys.stderr, flush=True)
    h = hidden0.clone()
    for _ in range(args.warmup):
        h.copy_(hidden0)
        stage.forward(h, q_lens, starts, slots)
    torch.cuda.synchronize()
    print("[bench] timed steps", file=sys.stderr, flush=True)
    hs = [hidden0.clone() for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        stage.forward(hs[i], q_lens, starts, slots)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = T * args.steps / elapsed

    # ---- kernels of one MoE block, layer 1's weights, the stage's own RMS-normed rows -------------
    lw = layers[1]
    xn = stage.debug_buffer(0, torch.bfloat16, (T, shape.hidden)).clone()
    resid = hidden0.clone()
    I, H = shape.intermediate, shape.hidden
    ids, wts, hist, off, perm, inv = ops.moe_route_permute(xn, lw.router_w, lw.router_b, k)
    hmoe = ops.moe_gate_up(xn, perm, off, k, lw.w13_packed, lw.b13, E, I)
    torch.cuda.synchronize()
    hist_np = hist.cpu().numpy()
    reps = args.kernel_reps
    if fp8:   # the dense groups' path in this stage: fp8 activation operands, scaled MFMA
        xq, xs = ops.mx_act_quant(xn)
        hq, hs = ops.mx_act_quant(hmoe)
        gate_up = lambda: ops.moe_gate_up_fp8act(xn, xq, xs, perm, off, k, lw.w13_packed, lw.b13, E, I)
        down = lambda: ops.moe_down_fp8act(hmoe, hq, hs, off, lw.w2_packed, lw.b2, E, H)
        quant_us = hip_event_us(lambda: ops.mx_act_quant(xn), reps, warmup=5) + \
            hip_event_us(lambda: ops.mx_act_quant(hmoe), reps, warmup=5)
    else:
        gate_up = lambda: ops.moe_gate_up(xn, perm, off, k, lw.w13_packed, lw.b13, E, I)
        down = lambda: ops.moe_down(hmoe, off, lw.w2_packed, lw.b2, E, H)
        quant_us = 0.0
    gu_us = hip_event_us(gate_up, reps, warmup=10)
    dn_us = hip_event_us(down, reps, warmup=10)

    def moe_block():
        i_, w_, _, o_, p_, v_ = ops.moe_route_permute(xn, lw.router_w, lw.router_b, k)
        if fp8:
            xq_, xs_ = ops.mx_act_quant(xn)
            h_ = ops.moe_gate_up_fp8act(xn, xq_, xs_, p_, o_, k, lw.w13_packed, lw.b13, E, I)
            hq_, hs_ = ops.mx_act_quant(h_)
            y_ = ops.moe_down_fp8act(h_, hq_, hs_, o_, lw.w2_packed, lw.b2, E, H)
        else:
            h_ = ops.moe_gate_up(xn, p_, o_, k, lw.w13_packed, lw.b13, E, I)
            y_ = ops.moe_down(h_, o_, lw.w2_packed, lw.b2, E, H)
        ops.moe_combine(y_, v_, w_, residual=resid, out=resid)

    moe_us = hip_event_us(moe_block, args.moe_reps, warmup=20)
    gu_bytes, touched = gate_up_algorithmic_bytes(shape, hist_np, T, k)
    dn_bytes, _ = down_algorithmic_bytes(shape, hist_np, T, k)
    moe_bytes = moe_layer_algorithmic_bytes(shape, hist_np, T, k)
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_gbs = dn_bytes / (dn_us * 1e-6) / 1e9
    if chunked_prefill:
        prof = f"stage_step_{workload}{'_fp8' if fp8 else ''}_counters.json"
        traffic = committed_traffic(prof, ("moe_mx_gemm_kernel<true>", "moe_mxfp4_kernel<true") if fp8 else
                                    ("moe_mxfp4_gemm_kernel<true>", "moe_mxfp4_kernel<true"))
    else:
        traffic = committed_traffic("stage_step_c1_counters.json", ("moe_mxfp4_kernel<true",))
    ceiling = hbm_read_ceiling(args.read_probe_mib, dev)
    copy_probe(args.copy_probe_mib, dev)
    step_launch = "hip graph replay" if args.graphs else "direct launches"
    moe = {"us": round(moe_us, 2),
           "ops": "route+top-k/permute, " + ("fp8 act quant x2, " if fp8 else "") + "gate_up, down, combine",
           "GB/s": round(moe_bytes / (moe_us * 1e-6) / 1e9, 1),
           "frac": round(moe_bytes / (moe_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_bytes": moe_bytes, "experts_us": round(gu_us + dn_us, 2)}
    if fp8:
        moe["act_quant_us"] = round(quant_us, 2)

    if chunked_prefill:
        # dense groups (the prefill chunk: ~65 rows per expert; the stress batch: its hot experts):
        # gate_up against the MFMA peak
        P = T * k
        flops = 2.0 * P * shape.hidden * 2 * shape.intermediate
        tflops = flops / (gu_us * 1e-6) / 1e12
        peak = MFMA_PEAK_TFLOPS["fp8" if fp8 else "bf16"]
        dtype = ("mxfp4-e2m1 weights x two-term fp8-e4m3 activations (high + low term, E8M0 per-32 scales, "
                 "scaled MFMA) in the dense expert groups, bf16 elsewhere; fp32 accumulate") if fp8 \
            else "mxfp4-e2m1/bf16 (fp32 accumulate)"
        kname = "moe_mx_gemm_kernel<gate_up> (scaled f8f6f4 MFMA)" if fp8 else "moe_mxfp4_gemm_kernel<gate_up>"
        line = {
            "metric": ("stage tokens/sec at a chunked-prefill mixed batch; MoE layer us; % MFMA roofline"
                       if workload == "c2" else
                       "stage tokens/sec at a 256-sequence stress batch; MoE layer us; % MFMA roofline"),
            "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (seeded random-init weights, N(0,1) KV and activations)",
            "config": {"workload": ("gpt-oss-120b-shaped 9-layer MXFP4 stage, one 2048-token prefill chunk "
                                    "(prior KV 4096) + 48 decode rows (KV 512-8192)") if workload == "c2" else
                                   ("gpt-oss-120b-shaped 9-layer MXFP4 stage, 256 sequences: Zipf query lengths "
                                    "(decode, verify up to 8, two 1024-token prefill chunks), KV log-uniform "
                                    "128-32768 in per-sequence slabs, 10% of experts take ~50% of assignments"),
                       "layers": args.layers, "tokens": T, "sequences": S, "experts": E,
                       "top_k": k, "hidden": shape.hidden, "parallelism": "single GPU", "step_launch": step_launch,
                       "dense_path": args.dense},
            "moe_layer_us": moe["us"], "moe_layer": moe,
            "roofline": {"bound": "mfma", "kernel": kname, "achieved": round(tflops, 1),
                         "peak": peak, "unit": "TFLOP/s", "frac": round(tflops / peak, 4), "traffic": traffic,
                         "algorithmic_flops": flops, "avg_us": round(gu_us, 2), "hbm_GB/s": round(gu_gbs, 1)},
            "kernels": {"moe_down": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                     "TFLOP/s": round(flops / 2 / (dn_us * 1e-6) / 1e12, 1)}},
            "hbm_read_ceiling": ceiling,
            "cpu_baseline": (cpu_baseline(cpu_inputs, cpu_sub["q_lens"], cpu_sub["starts"], maxlen, args.layers,
                                          subset=cpu_sub["what"]) if with_cpu else None),
        }
        print(json.dumps(line))
        return

    cpu = cpu_baseline(cpu_inputs, q_lens, starts, maxlen, args.layers) if with_cpu else None
    line = {
        "metric": "stage tokens/sec at ragged batch 32; MoE layer us; % HBM/MFMA roofline",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4-e2m1/bf16 (fp32 accumulate)",
        "data": "synthetic (seeded random-init weights, N(0,1) KV and activations)",
        "config": {"workload": "gpt-oss-120b-shaped 9-layer MXFP4 stage, ragged batch of 32 sequences "
                               "(24 decode + 8 four-token verify = 56 tokens), KV 512-8192",
                   "layers": args.layers, "tokens": T, "sequences": S, "experts": E,
                   "top_k": k, "hidden": shape.hidden, "parallelism": "single GPU", "step_launch": step_launch},
        "moe_layer_us": moe["us"], "moe_layer": moe,
        "roofline": {"bound": "hbm", "kernel": "moe_mxfp4_kernel<gate_up>", "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": gu_bytes, "avg_us": round(gu_us, 2),
                     "experts_touched": touched},
        "kernels": {"moe_down": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                 "frac": round(dn_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": dn_bytes}},
        "hbm_read_ceiling": ceiling,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_row_subset(workload, q_lens, starts, prefill_seqs):
    """The rows the CPU baseline runs for a chunked-prefill batch: the chunk's last 4 rows and every
    decode row (c2); the last 4 rows of both prefill chunks and the last row of 60 other sequences
    (c4).  Each picked run is a sub-sequence at its own positions, over its sequence's slab."""
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    if workload == "c2":
        picks = [(0, 4)] + [(b, 1) for b in range(1, len(q_lens))]
        what = "the 2048-token chunk's last 4 rows and the 48 decode rows"
    else:
        others = [b for b in range(len(q_lens)) if b not in set(prefill_seqs)]
        picks = [(b, 4) for b in prefill_seqs] + [(b, 1) for b in others[::4][:60]]
        what = "the last 4 rows of both 1024-token prefill chunks and the last row of 60 other sequences"
    rows, sub_q, sub_starts = [], [], []
    for b, n in picks:
        rows.extend(range(int(cu[b + 1]) - n, int(cu[b + 1])))
        sub_q.append(n)
        sub_starts.append(starts[b] + q_lens[b] - n)
    return rows, {"q_lens": sub_q, "starts": sub_starts, "slots": [b for b, _ in picks],
                  "what": f"{len(rows)} rows: {what}"}


def cpu_layer_inputs(layers, kv, hidden0, slots):
    """Host copies of the given layers (oracle parameters) and of their KV for the given slots."""
    import torch
    from oracle import experts as oexperts
    from oracle import layer as olayer
    f = lambda t: t.detach().float().cpu()
    out = []
    for i, lw in enumerate(layers):
        moe = oexperts.MxExpertWeights(lw.w13_blocks.cpu().numpy(), lw.w13_scales.cpu().numpy(),
                                       lw.b13.cpu().numpy(), lw.w2_blocks.cpu().numpy(),
                                       lw.w2_scales.cpu().numpy(), lw.b2.cpu().numpy())
        p = olayer.LayerParams(f(lw.ln1), f(lw.ln2), f(lw.wqkv), f(lw.bqkv), f(lw.wo), f(lw.bo), f(lw.sinks),
                               f(lw.router_w), f(lw.router_b), moe, lw.sliding)
        ks = [f(kv.k_dense(i, s)) for s in slots]
        vs = [f(kv.v_dense(i, s)) for s in slots]
        out.append((p, ks, vs))
    torch.cuda.synchronize()
    return {"layers": out, "h": f(hidden0)}


def cpu_baseline(inp, q_lens, starts, maxlen, n_layers, subset=None):
    """The CPU oracle on one sliding (layer 0) and one full-attention layer (layer 1) of the same
    batch, each a warmup then the median of 3 runs; the stage estimate is the 9-layer mix (5 sliding,
    4 full) of those medians.  subset: the rows are a stated subset of the batch (tokens/s is then the
    subset's rows over its stage time)."""
    import torch
    from oracle import layer as olayer
    threads = cpu_threads()
    torch.set_num_threads(threads)
    cos, sin = olayer.rope_table(maxlen)
    print(f"[bench] cpu oracle: one sliding + one full layer, {threads} threads", file=sys.stderr, flush=True)
    med = []
    for p, ks, vs in inp["layers"]:
        def run():   # the layer rewrites the same K/V values at the batch's positions on every run
            olayer.decoder_layer(inp["h"], p, (ks, vs), q_lens, starts, cos, sin)
        m, _ = timed_median(run)
        med.append(m)
    n_sliding = (n_layers + 1) // 2
    stage_s = n_sliding * med[0] + (n_layers - n_sliding) * med[1]
    T = sum(q_lens)
    return {"value": round(T / stage_s, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": f"CPU oracle (torch fp32 + numpy) on layer 0 (sliding, median {med[0]:.2f} s) and "
                      f"layer 1 (full attention, median {med[1]:.2f} s) of "
                      f"{'a subset of the batch, ' + subset if subset else f'the same {T}-token batch'}, warmup + "
                      f"median of 3 each; stage = {n_sliding} x sliding + {n_layers - n_sliding} x full = "
                      f"{stage_s:.2f} s"}


# ---- one GPT-OSS MoE block on the 12-token ragged batch (c0) ----------------------------------------

def run_c0(args):
    """The MoE block (RMSNorm'd input -> router top-4 -> permute -> gate_up -> down -> combine) on
    sequences of 1, 1, 3 and 7 tokens; a step is one block.  E2M1 codes uniform, E8M0 scale bytes
    119..123 (2^-8..2^-4), bf16 N(0,1) activations; the CPU oracle runs the same block."""
    import torch
    from flyai_amd import ops
    from flyai_amd.weights import GptOssShape, synthetic_moe
    dev = "cuda"
    torch.cuda.set_device(0)
    shape = GptOssShape()
    E, k, H, I = shape.n_experts, shape.top_k, shape.hidden, shape.intermediate
    q_lens = [1, 1, 3, 7]
    T = sum(q_lens)

    def gen(seed):
        g_ = torch.Generator(device=dev)
        g_.manual_seed(seed)
        return g_
    m = synthetic_moe(shape, gen(0), dev)
    w13 = ops.mxfp4_repack(m["w13_blocks"], m["w13_scales"])
    w2 = ops.mxfp4_repack(m["w2_blocks"], m["w2_scales"])
    x = torch.randn(T, H, device=dev, generator=gen(1)).to(torch.bfloat16)
    lnw = torch.ones(H, device=dev)
    rw = (torch.randn(E, H, device=dev, generator=gen(2)) * 0.02).to(torch.bfloat16)
    rb = (torch.randn(E, device=dev, generator=gen(3)) * 0.02).to(torch.bfloat16)
    xn = ops.rmsnorm(x, lnw)
    resid = x.clone()

    def block():
        ids, wts, _, off, perm, inv = ops.moe_route_permute(xn, rw, rb, k)
        h = ops.moe_gate_up(xn, perm, off, k, w13, m["b13"], E, I)
        y = ops.moe_down(h, off, w2, m["b2"], E, H)
        ops.moe_combine(y, inv, wts, residual=resid, out=resid)
    for _ in range(args.warmup + 20):
        block()
    torch.cuda.synchronize()
    us = hip_event_us(block, max(args.steps, 100))
    _, _, hist, _, _, _ = ops.moe_route_permute(xn, rw, rb, k)
    hist_np = hist.cpu().numpy()
    moe_bytes = moe_layer_algorithmic_bytes(shape, hist_np, T, k)
    gbs = moe_bytes / (us * 1e-6) / 1e9
    traffic = committed_traffic("moe_block_c0_counters.json", ("moe_mxfp4_kernel<true", "moe_mxfp4_kernel<false"))
    ceiling = hbm_read_ceiling(args.read_probe_mib, dev)
    copy_probe(args.copy_probe_mib, dev)
    cpu = None
    if not args.no_cpu:
        from oracle import experts as oexperts
        from oracle import routing as oroute
        threads = cpu_threads()
        torch.set_num_threads(threads)
        wo = oexperts.MxExpertWeights(*(m[n].cpu().numpy() for n in
                                        ("w13_blocks", "w13_scales", "b13", "w2_blocks", "w2_scales", "b2")))
        xc, rwc, rbc, xres = xn.float().cpu(), rw.float().cpu(), rb.float().cpu(), x.float().cpu()

        def cpu_block():
            rids, rwts, _ = oroute.gptoss_route(xc, rwc, rbc, k)
            _, roff, rperm, rinv = oroute.permute(rids, E)
            ry = oexperts.experts_mxfp4(xc, rperm, roff, k, wo)
            oroute.combine(ry, rinv, rwts, residual=xres)
        print(f"[bench] cpu oracle: the MoE block, {threads} threads", file=sys.stderr, flush=True)
        med, _ = timed_median(cpu_block)
        cpu = {"value": round(T / med, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
               "cpu": cpu_model(), "host_cpus": os.cpu_count(),
               "sample": f"CPU oracle (torch fp32 + numpy) on the whole block, warmup + median of 3: {med:.2f} s"}
    line = {
        "metric": "MoE layer us (one GPT-OSS MoE block, ragged batch of 4 sequences); % HBM roofline",
        "value": round(T / (us * 1e-6), 2), "unit": "tokens/s", "n_gpus": 1, "steps": max(args.steps, 100),
        "warmup": args.warmup + 20, "ms_per_step": round(us / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4-e2m1/bf16 (fp32 accumulate)",
        "data": "synthetic (E2M1 codes uniform, E8M0 scale bytes 119..123, N(0,1) activations RMS-normed)",
        "config": {"workload": "one gpt-oss-120b-shaped MXFP4 MoE block (128 experts, top-4, H = I = 2880), "
                               "sequences of 1, 1, 3 and 7 tokens", "tokens": T, "sequences": len(q_lens),
                   "experts": E, "top_k": k, "hidden": H, "parallelism": "single GPU"},
        "moe_layer_us": round(us, 2),
        "roofline": {"bound": "hbm", "kernel": "MoE block (route + permute + gate_up + down + combine)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes": moe_bytes,
                     "avg_us": round(us, 2), "experts_touched": int((hist_np > 0).sum())},
        "hbm_read_ceiling": ceiling,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


# ---- DeepSeek-V3-shaped FP8 stage (c3) ------------------------------------------------------------

def run_c3(args):
    import torch
    from flyai_amd import ops
    from flyai_amd.runtime import Fp8MoeStage
    from flyai_amd.weights import DsV3Shape, synthetic_fp8_moe_layer

    dev = "cuda"
    torch.cuda.set_device(0)
    sh = DsV3Shape()
    n_layers = 4
    q_lens = c3_batch(0)
    T = sum(q_lens)
    E, k, H, I = sh.n_experts, sh.top_k, sh.hidden, sh.intermediate
    print(f"[bench] building {n_layers}-layer FP8 stage (T={T}) ...", file=sys.stderr, flush=True)
    layers = [synthetic_fp8_moe_layer(sh, 2000 + i, dev, keep_raw=(i == 0 and not args.no_cpu))
              for i in range(n_layers)]
    stage = Fp8MoeStage(sh, layers)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    hidden0 = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    torch.cuda.synchronize()
    print("[bench] warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        stage.forward(hidden0.clone())
    torch.cuda.synchronize()
    print("[bench] timed steps", file=sys.stderr, flush=True)
    hs = [hidden0.clone() for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        stage.forward(hs[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = T * args.steps / elapsed

    # dominant op: the FP8 gate_up of layer 0 (routed + shared groups; tail and dense launches)
    lw = layers[0]
    xn = ops.rmsnorm(hidden0, lw.ln, sh.rms_eps)
    ids, wts, _ = ops.router_grouped_sigmoid(xn, lw.router_w, lw.e_bias, sh.n_group, sh.topk_group, k,
                                             sh.route_scale)
    hist, off, perm, inv = ops.moe_permute(ids, E)
    xq, xs = ops.fp8_act_quant(xn)
    h = ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, lw.w13_packed, E, I, n_shared=T)
    hq, hsc = ops.fp8_act_quant(h)
    torch.cuda.synchronize()
    hist_np = hist.cpu().numpy()
    groups = int((hist_np > 0).sum()) + 1
    reps = args.kernel_reps
    gu_us = hip_event_us(lambda: ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, lw.w13_packed, E, I, n_shared=T),
                         reps, warmup=10)
    dn_us = hip_event_us(lambda: ops.moe_down_fp8(hq, hsc, off, lw.w2_packed, E, H, n_shared=T), reps, warmup=10)
    resid = hidden0.clone()
    moe_us = hip_event_us(lambda: stage.moe(lw, hidden0, resid), args.moe_reps, warmup=20)
    P = T * k + T
    gu_bytes = groups * (2 * I * H + 2 * (I // 128) * (H // 128)) + T * H + T * (H // 128) + P * I * 2
    dn_bytes = groups * (H * I + (H // 128) * (I // 128)) + P * I + P * (I // 128) + P * H * 2
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_gbs = dn_bytes / (dn_us * 1e-6) / 1e9
    ceiling = hbm_read_ceiling(args.read_probe_mib, dev)
    copy_probe(args.copy_probe_mib, dev)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_c3(sh, lw, hidden0, n_layers, n_tokens=16)

    line = {
        "metric": "stage tokens/sec at ragged batch 64 (FP8 MoE stage); MoE layer us; % HBM roofline",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 (E8M0 128x128 block scales), fp32 accumulate",
        "data": "synthetic (seeded random-init weights quantised per 128x128 block, N(0,1) activations)",
        "config": {"workload": "DeepSeek-V3-shaped 4-layer FP8 MoE stage, ragged batch of 64 sequences of "
                               "1/2/4 tokens, 256 experts top-8 grouped sigmoid (Zipf-shaped bias) + 1 shared",
                   "layers": n_layers, "tokens": T, "sequences": len(q_lens), "experts": E, "top_k": k,
                   "hidden": H, "intermediate": I, "parallelism": "single GPU"},
        "moe_layer_us": round(moe_us, 2),
        "moe_layer": {"us": round(moe_us, 2), "ops": "rmsnorm, grouped router, permute, act quant, gate_up, "
                                                      "act quant, down, combine (+ shared expert, residual)",
                      "experts_us": round(gu_us + dn_us, 2)},
        "roofline": {"bound": "hbm", "kernel": "moe_fp8_kernel<gate_up> (tail + dense launches)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": committed_traffic("stage_step_c3_counters.json",
                                                  ("moe_fp8_kernel<true, 1", "moe_fp8_kernel<true, 8")),
                     "algorithmic_bytes": gu_bytes, "avg_us": round(gu_us, 2), "groups_touched": groups},
        "kernels": {"moe_down_fp8": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                     "frac": round(dn_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": dn_bytes}},
        "hbm_read_ceiling": ceiling,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_baseline_c3(sh, lw, hidden0, n_layers, n_tokens):
    """The CPU oracle's FP8 MoE layer on the first n_tokens tokens of the batch (every expert those
    tokens route to, plus the shared expert), warmup + median of 3; stage tokens/s =
    n_tokens / (n_layers * t)."""
    import torch
    from oracle import experts as oexperts
    from oracle import layer as olayer
    threads = cpu_threads()
    torch.set_num_threads(threads)

    class Experts:
        def __init__(self, raw):
            self.raw = {n: t.cpu() for n, t in raw.items()}

        def expert(self, e, x, weight=None):
            r = self.raw
            f8 = lambda t: t[e].view(torch.float8_e4m3fn).float().numpy()
            e8 = lambda t: np.ldexp(np.float32(1.0), t[e].numpy().astype(np.int32) - 127).astype(np.float32)
            return oexperts.deepseek_expert(x, f8(r["w1"]), e8(r["s1"]), f8(r["w3"]), e8(r["s3"]),
                                            f8(r["w2"]), e8(r["s2"]), weight)

    h = hidden0[:n_tokens].float().cpu()
    ln, rw, eb = lw.ln.cpu(), lw.router_w.float().cpu().numpy(), lw.e_bias.cpu().numpy()
    routed, shared = Experts(lw.raw), Experts(lw.shared_raw)
    print("[bench] cpu oracle: one FP8 MoE layer", file=sys.stderr, flush=True)
    m, _ = timed_median(lambda: olayer.deepseek_moe_layer(h, ln, sh.rms_eps, rw, eb, sh.n_group, sh.topk_group,
                                                          sh.top_k, sh.route_scale, routed, shared))
    return {"value": round(n_tokens / (m * n_layers), 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": f"CPU oracle (numpy fp64 block GEMMs + torch) on 1 of {n_layers} layers for the first "
                      f"{n_tokens} tokens of the batch, warmup + median of 3: {m:.2f} s; stage rate = "
                      f"{n_tokens} / ({n_layers} x layer time)"}


# ---- activation frames over loopback TCP (wire) ---------------------------------------------------

WIRE_GEOMETRIES = {"decode_8x4": (8, 4, 2880), "prefill_1x4096": (1, 4096, 2880)}


def _loopback_pair(W):
    lst = socket.socket()
    lst.bind(("127.0.0.1", 0))
    lst.listen(1)
    a = socket.create_connection(lst.getsockname(), timeout=60)
    b, _ = lst.accept()
    lst.close()
    for s in (a, b):
        W.tune_socket(s)
        s.settimeout(60)
    return a, b


def _wire_path(W, path, h, frames, warmup):
    """Frames of {"op": "verify", "h": h} sent by a thread and landed by the receiver: `socket_only`
    (CPU to CPU, the socket's own rate), `pageable` (h.cpu(), recv_msg, .to(device): the reference's
    call pattern) or `pinned_ring` (send_msg of the device tensor, recv_activation).  Time runs from
    the first timed frame to the last one ready on the receiver's stream."""
    import torch
    a, b = _loopback_pair(W)
    dev = h.device
    h_host = h.cpu()
    total = frames + warmup

    def sender():
        for _ in range(total):
            W.send_msg(a, {"op": "verify", "h": h.cpu() if path == "pageable" else h if path == "pinned_ring"
                           else h_host})

    t = threading.Thread(target=sender, daemon=True)
    torch.cuda.synchronize()
    t.start()
    last = None
    for i in range(total):
        if i == warmup:
            start = time.perf_counter()
        if path == "pageable":
            last = W.recv_msg(b)["h"].to(dev)
        elif path == "pinned_ring":
            last = W.recv_activation(b, dev)["h"]
        else:
            last = W.recv_msg(b)["h"]
        if path != "socket_only":
            torch.cuda.current_stream(dev).synchronize()
    elapsed = time.perf_counter() - start
    t.join(60)
    a.close(), b.close()
    nbytes = W.frame_length({"op": "verify", "h": h})
    return {"ms_per_frame": round(elapsed / frames * 1e3, 4), "GBps": round(nbytes * frames / elapsed / 1e9, 3),
            "frame_bytes": nbytes, "bytes_equal": bool(torch.equal(last.cpu(), h_host))}


def run_wire(args):
    import torch
    from flyai_amd import transport as W
    dev = "cuda"
    torch.cuda.set_device(0)
    results = {}
    for name, shp in WIRE_GEOMETRIES.items():
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        h = torch.randn(shp, device=dev, generator=g).to(torch.bfloat16)
        results[name] = {p: _wire_path(W, p, h, args.frames, 3) for p in ("socket_only", "pageable", "pinned_ring")}
        print(f"[bench] wire {name}: {json.dumps(results[name])}", file=sys.stderr, flush=True)
    pre = results["prefill_1x4096"]
    line = {"metric": "activation frame HBM-to-HBM over loopback TCP (prefill chunk)",
            "value": pre["pinned_ring"]["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.frames, "warmup": 3,
            "ms_per_step": pre["pinned_ring"]["ms_per_frame"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations)",
            "config": {"workload": "activation frames h[1, 4096, 2880] and h[8, 4, 2880] bf16, loopback TCP, "
                                   "32 MiB socket buffers", "chunk_bytes": W.CHUNK_BYTES, "ring_slots": W.RING_SLOTS,
                       "parallelism": "single GPU"},
            "results": results, "roofline": None, "cpu_baseline": None}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
