"""Benchmark: one GPT-OSS-120B-shaped pipeline stage's continuous-batch forward step on one MI355X.

Workload (default): 9 decoder layers (sliding window 128 on even layers, full attention on odd),
64 query / 8 KV heads of dim 64 with learned sinks, 128-expert top-4 MXFP4 MoE (H = I = 2880);
a ragged batch of 32 sequences -- 24 single-token decode rows and 8 four-token spec-verify rows
(56 tokens) -- with per-sequence KV length uniform in [512, 8192]; KV and activations bf16
N(0,1), weights random-init (synthetic data, seed 0).

A step is one stage forward over that batch.  value = tokens / second over the timed steps.
The roofline object covers the dominant kernel (the MXFP4 gate_up expert GEMM), timed with HIP
events on the stream it runs on; its algorithmic bytes count every touched expert's weights and
scales once plus activations in and out.  cpu_baseline runs the CPU oracle on one of the nine
layers (same inputs) and scales to the stage.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

--workload c3 measures the DeepSeek-V3-shaped FP8 stage instead: 4 MoE layers (H 7168, 256 experts,
top-8 grouped sigmoid routing with a Zipf-shaped selection bias, one shared expert, I 2048, e4m3
weights with 128x128 E8M0 block scales), a ragged batch of 64 sequences of 1, 2 or 4 tokens.
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


def c1_batch(seed=0):
    rng = np.random.default_rng(seed)
    q_lens = [1] * 24 + [4] * 8
    starts = [int(v) for v in rng.integers(512, 8192 + 1, size=32)]
    return q_lens, starts


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=9)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after timing, copy a buffer of this many MiB 3 times (a known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    ap.add_argument("--workload", choices=("c1", "c2", "c3"), default="c1")
    ap.add_argument("--graphs", action="store_true",
                    help="replay the stage step as a HIP graph (measured slower than direct launches "
                         "on this stack, so off by default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the stage is single-GPU by design: no collectives, no sharding)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "c3":
        run_c3(args)
    else:
        run_gptoss(args, chunked_prefill=args.workload == "c2")


def copy_probe(mib, dev):
    import torch
    if mib > 0:
        src = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()


def c2_batch(seed=0):
    """One 2048-token prefill chunk at prior KV 4096 plus 48 single-token decode rows."""
    rng = np.random.default_rng(seed)
    return [2048] + [1] * 48, [4096] + [int(v) for v in rng.integers(512, 8192 + 1, size=48)]


def run_gptoss(args, chunked_prefill=False):
    import torch
    from flyai_amd import ops
    from flyai_amd.rope import YarnRotary
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    from flyai_amd.weights import GptOssShape, synthetic_layer

    dev = "cuda"
    torch.cuda.set_device(0)
    shape = GptOssShape()
    q_lens, starts = c2_batch(0) if chunked_prefill else c1_batch(0)
    S, T = len(q_lens), sum(q_lens)
    maxlen = 8192 + 64
    with_cpu = not args.no_cpu and not chunked_prefill
    print(f"[bench] building {args.layers}-layer stage ...", file=sys.stderr, flush=True)
    layers = [synthetic_layer(shape, 1000 + i, dev, sliding=(i % 2 == 0), keep_hf=(i == 1 and with_cpu))
              for i in range(args.layers)]
    rot = YarnRotary(maxlen, device=dev)
    kv = KVWorkspace(args.layers, S, maxlen, shape.n_kv_heads, shape.head_dim, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    for t in kv.k + kv.v:
        t.copy_(torch.randn(t.shape, device=dev, generator=g).to(torch.bfloat16))
    hidden0 = torch.randn(T, shape.hidden, device=dev, generator=g).to(torch.bfloat16)
    stage = RaggedStage(shape, layers, rot, kv, max_tokens=max(64, T), max_seqs=S, use_graphs=args.graphs)
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

    # ---- dominant kernel: MXFP4 gate_up of layer 1 (full-attention layer), HIP events ----------
    lw = layers[1]
    xn = stage.debug_buffer(0, torch.bfloat16, (T, shape.hidden)).clone()
    ids, wts = ops.router_topk_softmax(xn, lw.router_w, lw.router_b, shape.top_k)
    hist, off, perm, inv = ops.moe_permute(ids, shape.n_experts)
    hmoe = ops.moe_gate_up(xn, perm, off, shape.top_k, lw.w13_packed, lw.b13, shape.n_experts, shape.intermediate)
    torch.cuda.synchronize()
    hist_np = hist.cpu().numpy()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    reps = args.kernel_reps
    ev[0].record()
    for _ in range(reps):
        ops.moe_gate_up(xn, perm, off, shape.top_k, lw.w13_packed, lw.b13, shape.n_experts, shape.intermediate)
    ev[1].record()
    for _ in range(reps):
        ops.moe_down(hmoe, off, lw.w2_packed, lw.b2, shape.n_experts, shape.hidden)
    ev[2].record()
    torch.cuda.synchronize()
    gu_us = ev[0].elapsed_time(ev[1]) * 1e3 / reps
    dn_us = ev[1].elapsed_time(ev[2]) * 1e3 / reps
    gu_bytes, touched = gate_up_algorithmic_bytes(shape, hist_np, T, shape.top_k)
    dn_bytes, _ = down_algorithmic_bytes(shape, hist_np, T, shape.top_k)
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_gbs = dn_bytes / (dn_us * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "moe_gate_up_c1_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    copy_probe(args.copy_probe_mib, dev)

    cpu = None
    if with_cpu:
        cpu = cpu_baseline(layers[1], kv, 1, hidden0, q_lens, starts, slots, shape, maxlen, args.layers)

    if chunked_prefill:
        # dense groups (~65 rows per expert): the gate_up GEMM against the bf16 MFMA peak
        P = T * shape.top_k
        flops = 2.0 * P * shape.hidden * 2 * shape.intermediate
        tflops = flops / (gu_us * 1e-6) / 1e12
        line = {
            "metric": "stage tokens/sec at a chunked-prefill mixed batch; MoE layer us; % MFMA roofline",
            "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4-e2m1/bf16 (fp32 accumulate)",
            "data": "synthetic (seeded random-init weights, N(0,1) KV and activations)",
            "config": {"workload": "gpt-oss-120b-shaped 9-layer MXFP4 stage, one 2048-token prefill chunk "
                                   "(prior KV 4096) + 48 decode rows (KV 512-8192)",
                       "layers": args.layers, "tokens": T, "sequences": S, "experts": shape.n_experts,
                       "top_k": shape.top_k, "hidden": shape.hidden, "parallelism": "single GPU",
                       "step_launch": "hip graph replay" if args.graphs else "direct launches"},
            "moe_layer_us": round(gu_us + dn_us, 2),
            "roofline": {"bound": "mfma", "kernel": "moe_mxfp4_gemm_kernel<gate_up>", "achieved": round(tflops, 1),
                         "peak": 2500.0, "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4), "traffic": None,
                         "algorithmic_flops": flops, "avg_us": round(gu_us, 2), "hbm_GB/s": round(gu_gbs, 1)},
            "kernels": {"moe_down": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                     "TFLOP/s": round(flops / 2 / (dn_us * 1e-6) / 1e12, 1)}},
            "cpu_baseline": None,
        }
        print(json.dumps(line))
        return

    line = {
        "metric": "stage tokens/sec at ragged batch 32; MoE layer us; % HBM/MFMA roofline",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4-e2m1/bf16 (fp32 accumulate)",
        "data": "synthetic (seeded random-init weights, N(0,1) KV and activations)",
        "config": {"workload": "gpt-oss-120b-shaped 9-layer MXFP4 stage, ragged batch of 32 sequences "
                               "(24 decode + 8 four-token verify = 56 tokens), KV 512-8192",
                   "layers": args.layers, "tokens": T, "sequences": S, "experts": shape.n_experts,
                   "top_k": shape.top_k, "hidden": shape.hidden, "parallelism": "single GPU",
                   "step_launch": "hip graph replay" if args.graphs else "direct launches"},
        "moe_layer_us": round(gu_us + dn_us, 2),
        "roofline": {"bound": "hbm", "kernel": "moe_mxfp4_kernel<gate_up>", "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": gu_bytes, "avg_us": round(gu_us, 2),
                     "experts_touched": touched},
        "kernels": {"moe_down": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                 "frac": round(dn_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": dn_bytes}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def c3_batch(seed=0):
    rng = np.random.default_rng(seed)
    return [int(v) for v in rng.choice([1, 2, 4], size=64)]


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
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record()
    for _ in range(reps):
        ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, lw.w13_packed, E, I, n_shared=T)
    ev[1].record()
    for _ in range(reps):
        ops.moe_down_fp8(hq, hsc, off, lw.w2_packed, E, H, n_shared=T)
    ev[2].record()
    torch.cuda.synchronize()
    gu_us = ev[0].elapsed_time(ev[1]) * 1e3 / reps
    dn_us = ev[1].elapsed_time(ev[2]) * 1e3 / reps
    P = T * k + T
    gu_bytes = groups * (2 * I * H + 2 * (I // 128) * (H // 128)) + T * H + T * (H // 128) + P * I * 2
    dn_bytes = groups * (H * I + (H // 128) * (I // 128)) + P * I + P * (I // 128) + P * H * 2
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_gbs = dn_bytes / (dn_us * 1e-6) / 1e9
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
        "moe_layer_us": round(gu_us + dn_us, 2),
        "roofline": {"bound": "hbm", "kernel": "moe_fp8_kernel<gate_up> (tail + dense launches)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": gu_bytes,
                     "avg_us": round(gu_us, 2), "groups_touched": groups},
        "kernels": {"moe_down_fp8": {"avg_us": round(dn_us, 2), "GB/s": round(dn_gbs, 1),
                                     "frac": round(dn_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": dn_bytes}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_baseline_c3(sh, lw, hidden0, n_layers, n_tokens):
    """The CPU oracle's FP8 MoE layer on the first n_tokens tokens of the batch (every expert those
    tokens route to, plus the shared expert); stage tokens/s = n_tokens / (n_layers * t)."""
    import torch
    from oracle import experts as oexperts
    from oracle import layer as olayer
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)

    class Experts:
        def __init__(self, raw):
            self.raw = raw

        def expert(self, e, x, weight=None):
            r = self.raw
            f8 = lambda t: t[e].cpu().view(torch.float8_e4m3fn).float().numpy()
            e8 = lambda t: np.ldexp(np.float32(1.0), t[e].cpu().numpy().astype(np.int32) - 127).astype(np.float32)
            return oexperts.deepseek_expert(x, f8(r["w1"]), e8(r["s1"]), f8(r["w3"]), e8(r["s3"]),
                                            f8(r["w2"]), e8(r["s2"]), weight)

    h = hidden0[:n_tokens].float().cpu()
    print("[bench] cpu oracle: one FP8 MoE layer", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    olayer.deepseek_moe_layer(h, lw.ln.cpu(), sh.rms_eps, lw.router_w.float().cpu().numpy(), lw.e_bias.cpu().numpy(),
                              sh.n_group, sh.topk_group, sh.top_k, sh.route_scale, Experts(lw.raw),
                              Experts(lw.shared_raw))
    dt = time.perf_counter() - t0
    return {"value": round(n_tokens / (dt * n_layers), 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle (numpy fp64 block GEMMs + torch) on 1 of {n_layers} layers for the first "
                      f"{n_tokens} tokens of the batch: {dt:.2f} s; stage rate = {n_tokens} / ({n_layers} x layer time)"}


def cpu_baseline(lw, kv, layer_idx, hidden0, q_lens, starts, slots, shape, maxlen, n_layers):
    """The CPU oracle on one decoder layer of the same batch; stage tokens/s = T / (n_layers * t)."""
    import torch
    from oracle import experts as oexperts
    from oracle import layer as olayer
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    f = lambda t: t.detach().float().cpu()
    moe = oexperts.MxExpertWeights(lw.w13_blocks.cpu().numpy(), lw.w13_scales.cpu().numpy(),
                                   lw.b13.cpu().numpy(), lw.w2_blocks.cpu().numpy(),
                                   lw.w2_scales.cpu().numpy(), lw.b2.cpu().numpy())
    p = olayer.LayerParams(f(lw.ln1), f(lw.ln2), f(lw.wqkv), f(lw.bqkv), f(lw.wo), f(lw.bo), f(lw.sinks),
                           f(lw.router_w), f(lw.router_b), moe, lw.sliding)
    ks = [f(kv.k_dense(layer_idx, s)) for s in slots]
    vs = [f(kv.v_dense(layer_idx, s)) for s in slots]
    cos, sin = olayer.rope_table(maxlen)
    h = f(hidden0)
    print("[bench] cpu oracle: one layer", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    olayer.decoder_layer(h, p, (ks, vs), q_lens, starts, cos, sin)
    dt = time.perf_counter() - t0
    T = sum(q_lens)
    return {"value": round(T / (dt * n_layers), 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle (torch fp32 + numpy) on 1 of {n_layers} layers (a full-attention layer) "
                      f"of the same 56-token batch: {dt:.2f} s; stage rate = 56 / ({n_layers} x layer time)"}


if __name__ == "__main__":
    main()
