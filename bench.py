#!/usr/bin/env python
"""Benchmark of the pi0.5 M1 denoise path on one MI355X.

Headline: ``denoise_step_kv`` microseconds per step at the full pi0.5 shape
(18 action-expert layers of width 1024 / MLP 4096, 8 query heads / 1 KV head /
head_dim 256, frozen prefix K/V of 968 tokens, horizon 50, action_dim 32, fp16
weights and activations, fp32 logits / statistics), plus the 10-step action chunk
(prefill of the 18-layer Gemma-2B-shaped prefix expert over 968 tokens with 800
valid, then the in-graph Euler loop, one hipGraph) in milliseconds, each as a
fraction of the 8 TB/s HBM roofline.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Prints one JSON line.  Weights are random N(0, 0.02) (no checkpoint), inputs
synthetic and resident in HBM before the timed region.  The CPU baseline is the
numpy float32 oracle of the same step on the host cores (not the reference's TVM
build, which is not installable here).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mlc-vla_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "denoise_step_kv µs/step + 10-step chunk ms @prefix 968; % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed denoise_step_kv calls")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--chunk-iters", type=int, default=20)
    ap.add_argument("--op-iters", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-q4", action="store_true")
    ap.add_argument("--no-embed", action="store_true", help="skip the embed_image timing")
    ap.add_argument("--summarize", metavar="KERNEL_TRACE_CSV",
                    help="print a per-kernel, per-launch-shape table of a rocprofv3 --kernel-trace CSV and exit")
    ap.add_argument("--summarize-pmc", metavar="COUNTER_CSV",
                    help="print the mean of each counter per dispatch of a rocprofv3 --pmc CSV, by kernel and "
                         "launch shape, and exit")
    ap.add_argument("--only-op", choices=sorted(set(OPS_PER_STEP) | set(OPS_PER_STEP_CHAIN) | {"attention_only", "prefill"}),
                    default=None,
                    help="after set-up, run --op-iters launches of one op of the step and exit (for --pmc runs)")
    ap.add_argument("--xt-timeline", nargs="?", const="fp16", choices=["fp16", "q4"], default=None,
                    help="with MLCV_LIB naming the phase-stamp build (mlc-vla_amd/build.py --trace): run the "
                         "fp16 (default) or q4f16_1 step and print the XCD step's per-phase timeline as "
                         "markdown, then exit")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="run --op-iters device copies of this many MiB and exit (counter calibration)")
    return ap.parse_args()


def kernel_name(raw):
    """Short kernel name: drop 'void ', the anonymous namespace and the parameter list."""
    n = raw[5:] if raw.startswith("void ") else raw
    n = n.replace("mlcv::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    if n.endswith(")"):
        depth = 0
        for i in range(len(n) - 1, -1, -1):
            depth += n[i] == ")"
            depth -= n[i] == "("
            if depth == 0:
                n = n[:i]
                break
    return n


def summarize_pmc(path):
    """Markdown table of a rocprofv3 --pmc counter CSV: mean per dispatch by (kernel, grid, workgroup)."""
    import csv

    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            key = (kernel_name(r["Kernel_Name"]), r["Grid_Size"], r["Workgroup_Size"])
            d = per.setdefault(key, {}).setdefault(r["Counter_Name"], {})
            d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    counters = sorted({c for v in per.values() for c in v})
    print("| kernel | grid (threads) | workgroup | dispatches | " + " | ".join(f"{c} (mean)" for c in counters) + " |")
    print("|---|---|---|---|" + "---|" * len(counters))
    for key, cs in sorted(per.items(), key=lambda kv: -max(len(v) for v in kv[1].values())):
        n = max(len(v) for v in cs.values())
        vals = [f"{sum(cs[c].values()) / len(cs[c]):.1f}" if c in cs else "" for c in counters]
        print(f"| {key[0][:48]} | {key[1]} | {key[2]} | {n} | " + " | ".join(vals) + " |")


XT_PHASES_A = [(0, "start"), (1, "reduce stored (waves 0-3)"), (11, "q/k/v weights in LDS (waves 4-5)"),
               (2, "barrier 1"), (3, "q/k/v MMA"), (4, "q/k/v epilogue stored"), (5, "barrier 2"),
               (14, "suffix keys: load start (waves 4-7)"), (15, "suffix keys in LDS"), (13, "attention start"),
               (6, "attention partials stored"), (7, "barrier 3"), (8, "combine stored"),
               (12, "o_proj weights in LDS (waves 4-7)"), (9, "barrier 4"), (10, "o_proj partials stored")]
XT_PHASES_B = [(0, "start"), (1, "reduce stored (waves 0-3)"), (11, "gate_up weights in LDS (waves 4-7)"),
               (2, "barrier 1"), (3, "gate_up MMA"), (4, "GeGLU stored"), (12, "down weights in LDS (waves 4-7)"),
               (5, "barrier 2"), (6, "down partials stored")]


def xt_timeline_report(tr, depth):
    """Markdown of the XCD step's phase stamps: tr[2 L + (MLP launch)][workgroup][stamp] in
    s_memrealtime ticks (100 MHz).  Per phase: min / median / max over the 256 workgroups of the
    time since the launch's first workgroup started, averaged over layers 1 .. depth - 1."""
    import numpy as np

    us = lambda t: t / 100.0  # noqa: E731
    lines = []
    ends = {0: 10, 1: 6}
    for half, (name, phases) in enumerate((("attention launch (A)", XT_PHASES_A), ("MLP launch (B)", XT_PHASES_B))):
        lines.append(f"\n{name}, layers 1-{depth - 1}: microseconds since the launch's first workgroup started\n")
        lines.append("| stamp | phase | min | median | max |")
        lines.append("|---|---|---|---|---|")
        for k, label in phases:
            mins, meds, maxs = [], [], []
            for L in range(1, depth):
                t = tr[2 * L + half]
                v = us(t[:, k] - t[:, 0].min())
                mins.append(v.min())
                meds.append(np.median(v))
                maxs.append(v.max())
            lines.append(f"| {k} | {label} | {np.mean(mins):.2f} | {np.mean(meds):.2f} | {np.mean(maxs):.2f} |")
    spans = {h: [us(tr[2 * L + h][:, ends[h]].max() - tr[2 * L + h][:, 0].min()) for L in range(depth)] for h in (0, 1)}
    gaps = [us(tr[i + 1][:, 0].min() - tr[i][:, ends[i % 2]].max()) for i in range(2 * depth - 1)]
    total = us(tr[2 * depth - 1][:, 6].max() - tr[0][:, 0].min())
    lines.append("")
    lines.append(f"- attention launch span (first workgroup start to last workgroup end): mean {np.mean(spans[0][1:]):.2f} us "
                 f"(layer 0, with action_in: {spans[0][0]:.2f} us)")
    lines.append(f"- MLP launch span: mean {np.mean(spans[1]):.2f} us")
    lines.append(f"- between launches (last end to next first start): mean {np.mean(gaps):.2f} us, "
                 f"A to B {np.mean(gaps[0::2]):.2f}, B to A {np.mean(gaps[1::2]):.2f}")
    lines.append(f"- the {2 * depth} layer launches, first start to last end: {total:.1f} us")
    return "\n".join(lines)


def f32_chunk_timing(dev):
    """The float32 model (Pi0Config(dtype="float32")) of the 2-layer configuration: one chunk
    (prefill + the 10-step loop through PiZeroRunner.sample_graph), weights 0.02 N(0,1)."""
    import numpy as np
    import torch

    from mlc_vla import runtime
    from mlc_vla.model.pi0 import Pi0Config
    from mlc_vla.sample import PiZeroRunner

    cfg = Pi0Config(paligemma_variant="tiny_vlm", action_expert_variant="tiny_action", image_keys=(),
                    max_token_len=32, action_horizon=8, action_dim=32, num_denoise_steps=10, dtype="float32")
    runner = PiZeroRunner(cfg, "rocm")
    g = torch.Generator(device="cuda").manual_seed(5)
    params = [runtime.Tensor(torch.randn(sp.shape, generator=g, device="cuda").mul_(0.02), "float32")
              for _, sp in runner.named_params]
    rng = np.random.default_rng(6)
    prefix = rng.standard_normal((1, cfg.prefix_len, cfg.vlm.width)).astype(np.float32)
    noise = rng.standard_normal((1, 8, 32)).astype(np.float32)
    for _ in range(3):
        runner.sample_graph(params, prefix, noise=noise)
    torch.cuda.synchronize()
    ts = []
    for _ in range(20):
        t0 = time.perf_counter()
        runner.sample_graph(params, prefix, noise=noise)
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    return {"ms_p50": round(sorted(ts)[len(ts) // 2], 3), "iters": len(ts),
            "workload": "2-layer model, fp32 (prefix 32, horizon 8, action 32): prefill + 10 Euler steps "
                        "through PiZeroRunner.sample_graph, host time per chunk incl. transfers"}


def q4_model(cfg, dev, npar, params):
    """The q4f16_1 model of `cfg` (compile_quant.py:71-103) on the fp16 parameters quantized on
    the GPU: (its VM, its parameter list)."""
    from mlc_vla import runtime
    from mlc_vla.compile_quant import compile_model_quant

    exq, qnp, qmap, quant = compile_model_quant(cfg, "rocm", None, "q4f16_1", cuda_graph=True)
    vmq = runtime.VirtualMachine(exq, dev)
    by_name = {n: t for (n, _), t in zip(npar, params)}
    qparams, cache = [], {}
    for n, _ in qnp:
        if n.endswith(".q_weight") or n.endswith(".q_scale"):
            base = n.rsplit(".", 1)[0]
            if base not in cache:
                cache[base] = quant.quantize_weight(by_name[base + ".weight"])
            qparams.append(cache[base][0 if n.endswith(".q_weight") else 1])
        else:
            qparams.append(by_name[n])
    return vmq, qparams


def summarize_trace(path):
    """Markdown table of a rocprofv3 kernel trace grouped by (kernel, grid, workgroup)."""
    import csv

    groups = {}
    total = 0
    with open(path) as f:
        for r in csv.DictReader(f):
            name = kernel_name(r["Kernel_Name"])
            grid = "x".join(r[f"Grid_Size_{a}"] for a in "XYZ")
            key = (name, grid, int(r["Workgroup_Size_X"]), int(r["LDS_Block_Size"]),
                   int(r["VGPR_Count"]) + int(r["Accum_VGPR_Count"]))
            dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            g = groups.setdefault(key, [])
            g.append(dur)
            total += dur
    print("| kernel | grid (threads) | workgroup | LDS B | VGPR+AGPR | calls | avg us | median us | min us | "
          "max us | share |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for key, d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        d.sort()
        print(f"| {key[0][:48]} | {key[1]} | {key[2]} | {key[3]} | {key[4]} | {len(d)} | {sum(d) / len(d) / 1e3:.2f} | "
              f"{d[len(d) // 2] / 1e3:.2f} | {d[0] / 1e3:.2f} | {d[-1] / 1e3:.2f} | {sum(d) / total:.1%} |")


def step_bytes(cfg, weight_bytes_per_param=2.0, q4=False):
    """Algorithmic HBM bytes of one denoise_step_kv: every weight it reads once, the prefix
    K (fp32) and V (fp16) cache once, and the step's inputs / output."""
    from mlc_vla.model.pi0.pi0_model import KV_FUNCS, named_params

    nbytes = 0.0
    for name, prm in named_params(cfg, KV_FUNCS):
        shape = prm.shape
        if ".experts.0." in name or ".mlp.0." in name or name.endswith("layernorm.0.weight") or \
                name == "backbone.final_norm.0.weight":
            continue  # expert-0 weights are not read by the suffix step
        n = 1
        for s in shape:
            n *= s
        if q4 and name.endswith(".weight") and len(shape) == 2:
            nbytes += n * 0.5 + (n / 32) * 2  # packed nibbles + fp16 group scales
        else:
            nbytes += n * weight_bytes_per_param
    v = cfg.vlm
    kv = v.depth * v.num_kv_heads * cfg.prefix_len * v.head_dim
    nbytes += kv * (4 + 2)
    T, A, hd = cfg.suffix_len, cfg.action_dim, v.head_dim
    nbytes += T * A * 2 + cfg.action_expert.width * 2 + 2 * T * hd // 2 * 4 + cfg.prefix_len * 4 + T * A * 4
    return nbytes


def step_flops(cfg):
    v, a = cfg.vlm, cfg.action_expert
    T, W, F, H, hd, KV = cfg.suffix_len, a.width, a.mlp_dim, v.num_heads, v.head_dim, v.num_kv_heads
    per_layer = 2 * T * W * (H * hd + 2 * KV * hd) + 2 * T * H * hd * W + 2 * T * W * 2 * F + 2 * T * F * W
    keys = cfg.prefix_len + T
    per_layer += 2 * 2 * H * T * keys * hd
    mod = 2 * (2 * v.depth + 1) * 3 * W * W + 2 * 2 * W * W
    return v.depth * per_layer + mod + 2 * T * cfg.action_dim * W * 2


def op_bytes_flops(cfg, op):
    """Algorithmic bytes / flops of one launch of an op of the step (layer 0)."""
    v, a = cfg.vlm, cfg.action_expert
    T, W, F, H, hd, KV, P = cfg.suffix_len, a.width, a.mlp_dim, v.num_heads, v.head_dim, v.num_kv_heads, cfg.prefix_len
    nq, nkv = H * hd, KV * hd
    if op == "modulation":
        nm = 2 * v.depth + 1
        return nm * (3 * W * W + 3 * W) * 2 + W * 2 + nm * 3 * W * 2, 2 * nm * 3 * W * W
    if op == "qkv":
        return (nq + 2 * nkv) * W * 2 + T * W * 2 + 2 * W * 2 + T * (nq + 2 * nkv) * 2, 2 * T * W * (nq + 2 * nkv)
    if op in ("attention", "attention_only"):
        return (KV * P * hd * 6 + T * nq * 2 + 2 * T * nkv * 2 + T * nq * 2 + P * 4 + T * hd * 4,
                4 * H * T * (P + T) * hd)
    if op == "o_proj":
        return W * nq * 2 + T * nq * 2 + 2 * T * W * 2 + W * 2, 2 * T * nq * W
    if op == "gate_up":
        return 2 * F * W * 2 + T * W * 2 + 2 * W * 2 + T * F * 2, 2 * T * W * 2 * F
    if op == "down":
        return W * F * 2 + T * F * 2 + 2 * T * W * 2 + W * 2, 2 * T * F * W
    if op == "head":
        return cfg.action_dim * W * 2 + T * W * 2 + T * cfg.action_dim * 4, 2 * T * W * cfg.action_dim
    if op == "xt_attn":  # the XCD step's attention launch: q/k/v + attention + o_proj of one layer
        b = (nq + 2 * nkv) * W * 2 + W * nq * 2  # q/k/v and o_proj weights
        b += KV * P * hd * 6 + P * 4 + T * hd * 4  # prefix K (f32) / V (f16), mask, RoPE tables
        b += 2 * T * W * 2 + 2 * 3 * W * 2  # residual stream in / out, two modulation rows
        return b, 2 * T * W * (nq + 2 * nkv) + 4 * H * T * (P + T) * hd + 2 * T * nq * W
    if op == "xt_mlp":  # the XCD step's MLP launch: gate_up + GeGLU + down of one layer
        return 2 * F * W * 2 + W * F * 2 + 2 * T * W * 2 + 2 * 3 * W * 2, 2 * T * W * 2 * F + 2 * T * F * W
    raise KeyError(op)


# the default step (the XCD tensor-parallel form) and the launch chain (one launch per operation:
# the form of the q4f16_1 step and of shapes the XCD step does not take)
OPS_PER_STEP = {"modulation": 1, "xt_attn": 18, "xt_mlp": 18, "head": 1}
OPS_PER_STEP_CHAIN = {"modulation": 1, "qkv": 18, "attention": 18, "o_proj": 18, "gate_up": 18, "down": 18, "head": 1}
OP_LAYER = {"xt_attn": 1}  # layer 0's attention launch also computes action_in
KERNEL_SYMBOLS = {"xt_attn": "xt_attn_kernel<false, false>", "xt_mlp": "xt_mlp_kernel<false>",
                  "attention": "attn_kernel<256, true, false, false, true, 8> + attn_combine_kernel<24>"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _pct(ts, q):
    ts = sorted(ts)
    return ts[min(len(ts) - 1, int(q * len(ts)))]


def cpu_baseline(cfg, seconds):
    """CPU restatement baseline (the numpy float32 oracle on the host cores; the reference's
    TVM llvm/c build is not available): 3 warm-ups, then at least 10 timed denoise_step_kv
    at the full shape within a bounded sample, and the config-1 run (the 2-layer model,
    prefill + 10 Euler steps) the same way."""
    import numpy as np

    from mlc_vla.model.pi0 import Pi0Config
    from oracle import pi0_oracle as O

    threads = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_info

        blas = [t for t in threadpool_info() if t.get("user_api") == "blas"]
        if blas:
            threads = max(t["num_threads"] for t in blas)
    except Exception:  # noqa: BLE001
        pass

    def timed_cpu(fn, budget, min_iters=10, warm=3):
        for _ in range(warm):
            fn()
        ts, t0 = [], time.perf_counter()
        while len(ts) < min_iters or (time.perf_counter() - t0 < budget and len(ts) < 5000):
            t1 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t1) * 1e6)
        return ts, time.perf_counter() - t0

    P = O.Prec("f32")
    d = O.dims_from_config(cfg)
    keep = lambda n: not (".experts.0." in n or ".mlp.0." in n)  # noqa: E731
    params = O.make_params([(n, s) for n, s in O.param_specs(d) if keep(n)], 0, "float32")
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((d.depth, 1, d.num_kv_heads, d.prefix_len, d.head_dim)).astype(np.float32)
    values = rng.standard_normal(keys.shape).astype(np.float32)
    x_t = rng.standard_normal((1, d.suffix_len, d.action_dim)).astype(np.float32)
    te = O.sinusoidal_time_emb(1.0, d.ae_width)
    cos, sin = O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    pm = O.make_prefix_mask_np(d.prefix_len)
    ts, el = timed_cpu(lambda: O.denoise_step_kv(params, d, keys, values, x_t, te, cos, sin, pm, P), seconds)

    # config 1: the 2-layer model (prefix 32, horizon 8, fp32), prefill + 10 host Euler steps
    c1 = Pi0Config(paligemma_variant="tiny_vlm", action_expert_variant="tiny_action", image_keys=(), max_token_len=32,
                   action_horizon=8, action_dim=32, num_denoise_steps=10, dtype="float32")
    d1 = O.dims_from_config(c1)
    p1 = O.make_params(O.param_specs(d1), 0, "float32")
    prefix = np.random.default_rng(1).standard_normal((1, d1.prefix_len, d1.vlm_width)).astype(np.float32)
    noise = np.random.default_rng(0).standard_normal((1, d1.suffix_len, d1.action_dim)).astype(np.float32)
    ts1, el1 = timed_cpu(lambda: O.sample(p1, d1, prefix, noise, P, num_steps=10), min(5.0, seconds / 4))
    return {"value": round(sum(ts) / len(ts), 1), "unit": "us/step", "cores": threads, "kind": "port",
            "p50_us": round(_pct(ts, 0.5), 1), "p90_us": round(_pct(ts, 0.9), 1), "cpu_model": _cpu_model(),
            "label": "CPU restatement baseline (numpy float32 oracle), not the reference TVM build",
            "sample": f"{len(ts)} float32 denoise_step_kv at the full pi0.5 shape (18 layers, P=968, T=50) "
                      f"with the numpy oracle after 3 warm-ups ({el:.1f} s)",
            "config1_chunk": {"p50_us": round(_pct(ts1, 0.5), 1), "p90_us": round(_pct(ts1, 0.9), 1),
                              "iters": len(ts1), "unit": "us/chunk",
                              "sample": "2-layer model (prefix 32, horizon 8, fp32): prefill + 10 Euler steps"}}


def main():
    args = parse()
    if args.summarize:
        summarize_trace(args.summarize)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the M1 denoise path is a single-request, single-device path and "
              f"this build has no multi-GPU mode (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from mlc_vla import _native as N
    from mlc_vla import runtime
    from mlc_vla.compile import compile_model
    from mlc_vla.compile_quant import compile_model_quant
    from mlc_vla.model.pi0 import Pi0Config
    from mlc_vla.sample import make_prefix_mask_np, make_rope_np, make_time_embs

    torch.cuda.set_device(0)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(max(1, args.op_iters)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_mib": args.copy_mib, "iters": args.op_iters,
                          "bytes_read_per_copy": src.numel() * 4, "bytes_written_per_copy": dst.numel() * 4}))
        return
    dev = runtime.device()
    cfg = Pi0Config(dtype="float16", action_horizon=50)  # prefix_len 968, 18 layers
    ex, npar = compile_model(cfg, "rocm", cuda_graph=True)
    vm = runtime.VirtualMachine(ex, dev)

    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    params = []
    for _, p in npar:
        t = torch.randn(p.shape, generator=gen, device="cuda", dtype=torch.float32).mul_(0.02).to(torch.float16)
        params.append(runtime.Tensor(t, "float16"))
    gen.manual_seed(3)
    prefix = runtime.Tensor(torch.randn((1, 968, 2048), generator=gen, device="cuda").to(torch.float16), "float16")
    rng = np.random.default_rng(0)
    noise = rng.standard_normal((1, 50, 32)).astype(np.float32)
    tes = make_time_embs(10, 1024)
    d = lambda a: runtime.tensor(a, dev)  # noqa: E731
    # config 3: all-valid prefix, suffix rope offset 968; config 5: 800 valid tokens
    pm_all, pm_800 = d(make_prefix_mask_np(968)), d(make_prefix_mask_np(968, num_valid=800))
    c968, s968 = (d(a) for a in make_rope_np(50, 256, 10_000.0, offset=968))
    c800, s800 = (d(a) for a in make_rope_np(50, 256, 10_000.0, offset=800))
    x_t = d(noise.astype(np.float16))
    te = d(tes[0].astype(np.float16))
    te_all = d(np.concatenate(tes, 0).astype(np.float16))
    x0 = d(noise)
    keys, values = vm["prefill"](prefix, pm_all, params)
    torch.cuda.synchronize()
    if args.xt_timeline:
        lib = N.load()
        if not hasattr(lib, "mlcv_xt_trace_ptr"):
            sys.exit("--xt-timeline needs MLCV_LIB naming the phase-stamp build (mlc-vla_amd/build.py --trace)")
        if args.xt_timeline == "q4":
            vmt, tparams = q4_model(cfg, dev, npar, params)
        else:
            vmt, tparams = vm, params
        for _ in range(10):
            vmt["denoise_step_kv"](keys, values, x_t, te, c968, s968, pm_all, tparams)
        torch.cuda.synchronize()
        lib.mlcv_xt_trace_ptr.restype = ctypes.c_void_p
        buf = np.zeros(64 * 256 * 16, np.uint64)
        hip = ctypes.CDLL("libamdhip64.so")
        if hip.hipMemcpy(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(lib.mlcv_xt_trace_ptr()),
                         ctypes.c_size_t(buf.nbytes), 2) != 0:
            sys.exit("hipMemcpy of the phase stamps failed")
        print(xt_timeline_report(buf.reshape(64, 256, 16).astype(np.int64), cfg.vlm.depth))
        return

    def timed(fn, iters, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters, (time.perf_counter() - w0) * 1e3 / iters

    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    scratch = torch.empty(512 << 18, device="cuda", dtype=torch.float32)  # 512 MiB for the cold protocol

    def per_step(fn, iters):
        """GPU time of each of `iters` back-to-back calls (events between them: the host stays ahead)."""
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
        fn()
        ev[0].record()
        for i in range(iters):
            fn()
            ev[i + 1].record()
        torch.cuda.synchronize()
        return [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(iters)]

    def per_cold(fn, iters):
        """Cold protocol: 512 MiB written between calls (outside the timed region), then a spin
        on the GPU so that the host has queued the call before its start event runs."""
        ts = []
        for i in range(iters):
            scratch.fill_(float(i))
            if hasattr(torch.cuda, "_sleep"):
                torch.cuda._sleep(1_000_000)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return ts

    def stage_step_inputs():
        """The op hooks read the context's staged copies of a step's inputs; a directly launched
        step reads the caller's tensors in place, so one step runs as a graph replay (staged)."""
        vm.set_step_graph(True)
        vm["denoise_step_kv"](keys, values, x_t, te, c968, s968, pm_all, params)
        vm.set_step_graph(False)
        torch.cuda.synchronize()

    if args.only_op == "prefill":  # the prefill graph alone (MFMA counters of the prefill GEMMs)
        for _ in range(args.op_iters):
            vm["prefill"](prefix, pm_800, params)
        torch.cuda.synchronize()
        print(json.dumps({"only_op": "prefill", "launches": args.op_iters}))
        return
    if args.only_op:
        op = N.OPS[args.only_op]
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        if args.only_op.startswith("xt_") or args.only_op == "head":
            stage_step_inputs()
        N.call("mlcv_bench_op", vm._ctx, op, OP_LAYER.get(args.only_op, 0), args.op_iters, runtime._ptr(keys),
               runtime._ptr(values), st)
        torch.cuda.synchronize()
        b, f = op_bytes_flops(cfg, args.only_op)
        print(json.dumps({"only_op": args.only_op, "launches": args.op_iters, "bytes_per_launch": int(b)}))
        return

    # ---- headline: denoise_step_kv ---------------------------------------------
    step = lambda: vm["denoise_step_kv"](keys, values, x_t, te, c968, s968, pm_all, params)  # noqa: E731
    step_ms, step_wall_ms = timed(step, args.steps, args.warmup)
    # ---- chunk: prefill + 10-step loop as one graph -----------------------------
    chunk = lambda: vm["chunk"](prefix, pm_800, x0, te_all, c800, s800, params)  # noqa: E731
    chunk_ms, _ = timed(chunk, args.chunk_iters, 3)
    prefill_ms, _ = timed(lambda: vm["prefill"](prefix, pm_800, params), args.chunk_iters, 3)
    loop_ms, _ = timed(lambda: vm["denoise_loop_kv"](keys, values, x0, te_all, c800, s800, pm_800, params),
                       args.chunk_iters, 3)
    vm.set_hoist(False)
    chunk_nh_ms, _ = timed(chunk, args.chunk_iters, 3)
    vm.set_hoist(True)

    # ---- single steps: percentiles warm, and the cold-cache protocol -----------
    warm_ts = per_step(step, max(20, min(args.steps, 200)))
    cold_ts = per_cold(step, 30)

    # ---- isolated attention (one layer; 18 layers back to back), cold -----------
    a_op = N.OPS["attention_only"]
    attn_one = lambda L: N.call("mlcv_bench_op", vm._ctx, a_op, L, 1, runtime._ptr(keys),  # noqa: E731
                                runtime._ptr(values), stream())
    a_single = per_cold(lambda: attn_one(0), 30)
    a_stack = per_cold(lambda: [attn_one(L) for L in range(18)], 10)
    a_bytes, _ = op_bytes_flops(cfg, "attention")

    # ---- measured HBM copy bandwidth (1 GiB device-to-device copies) -------------
    csrc = torch.ones(1 << 28, device="cuda", dtype=torch.float32)
    cdst = torch.empty_like(csrc)
    copy_ms, _ = timed(lambda: cdst.copy_(csrc), 20, 3)
    copy_gbs = 2 * csrc.numel() * 4 / (copy_ms * 1e-3) / 1e9
    del csrc, cdst

    # ---- per-op launch times (the step's kernels one op at a time, back to back) ---
    def op_table(ops):
        tab = {}
        for name, cnt in ops.items():
            op, layer = N.OPS[name], OP_LAYER.get(name, 0)
            run = lambda: N.call("mlcv_bench_op", vm._ctx, op, layer, args.op_iters,  # noqa: E731
                                 runtime._ptr(keys), runtime._ptr(values), stream())
            ms, _ = timed(run, 1, 1)
            us = ms * 1e3 / args.op_iters
            b, f = op_bytes_flops(cfg, name)
            tab[name] = {"us": round(us, 2), "per_step": cnt, "us_per_step": round(us * cnt, 1),
                         "GBps": round(b / (us * 1e-6) / 1e9, 1), "bytes": int(b), "flops": int(f)}
        return tab

    stage_step_inputs()
    per_op = op_table(OPS_PER_STEP)
    per_op_chain = op_table(OPS_PER_STEP_CHAIN)
    dom = max(per_op, key=lambda k: per_op[k]["us_per_step"])

    # ---- the isolated attention of the fp16-cache configuration (prefix K/V fp16, 900 of 968
    # prefix keys valid, 50 suffix keys, 8 heads, hd 256): mlcv_joint_attention, cold ---------
    g1 = torch.Generator(device="cuda").manual_seed(11)
    sc = 1.0 / 16.0  # N(0, 1) / sqrt(256)
    a1 = {n: (torch.randn(shp, generator=g1, device="cuda") * sc).half() for n, shp in
          (("q", (50, 8 * 256)), ("k", (1, 968, 256)), ("v", (1, 968, 256)), ("ks", (50, 256)), ("vs", (50, 256)))}
    m1 = torch.where(torch.arange(968, device="cuda") < 900, 0.0, -1e9).float()
    o1 = torch.empty((50, 8 * 256), dtype=torch.float16, device="cuda")
    tp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    attn1 = lambda: N.call("mlcv_joint_attention", tp(a1["q"]), 50, 8, 1, 256, tp(a1["k"]), 0,  # noqa: E731
                           tp(a1["v"]), 968, tp(m1), tp(a1["ks"]), tp(a1["vs"]), 50, tp(o1), stream())
    c1_single = per_cold(attn1, 30)
    c1_stack = per_cold(lambda: [attn1() for _ in range(18)], 10)
    c1_bytes = 968 * 256 * 2 * 2 + 50 * 8 * 256 * 2 * 2 + 50 * 256 * 2 * 2  # K, V, q, out, suffix k / v
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):  # calibrated PMC bytes per launch (see profiles/traffic_per_op_pmc.md)
        with open(tpath) as f:
            rec = json.load(f).get(dom)
        traffic = rec.get("traffic") if isinstance(rec, dict) else rec

    sbytes = step_bytes(cfg)
    step_us = step_ms * 1e3
    out = {
        "metric": METRIC,
        "value": round(step_us, 1),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "pi05_denoise_step_kv_fp16_P968_T50", "layers": 18, "ae_width": 1024,
                   "ae_mlp": 4096, "heads": 8, "kv_heads": 1, "head_dim": 256, "prefix_len": 968,
                   "horizon": 50, "action_dim": 32, "chunk_steps": 10, "chunk_valid_prefix": 800},
        "step_wall_us": round(step_wall_ms * 1e3, 1),
        "chunk_ms": round(chunk_ms, 3),
        "chunk_ms_per_step_modulation": round(chunk_nh_ms, 3),
        "step_percentiles": {"p50_us": round(_pct(warm_ts, 0.5), 1), "p90_us": round(_pct(warm_ts, 0.9), 1),
                             "iters": len(warm_ts)},
        "step_cold": {"p50_us": round(_pct(cold_ts, 0.5), 1), "p90_us": round(_pct(cold_ts, 0.9), 1),
                      "iters": len(cold_ts), "protocol": "512 MiB scratch written between steps, outside the timed region"},
        "attention_isolated": {
            "workload": "joint attention of one layer, P=968 prefix keys (fp32) + 50 suffix keys, 8 q heads, hd 256",
            "instance": "the step's own attention (q as hi/lo fragments from the q/k/v epilogue, roped fp32 suffix "
                        "keys, fp32 prefix K cache) + split combine, without prefetch workgroups (the launch chain's "
                        "attention; the XCD step runs its attention inside its attention launch); the prefix K is "
                        "fp32 because prefill writes the roped cache in fp32; its oracle check is the attention "
                        "gate of tests/test_gpu_chain_ops.py at this shape",
            "single_cold_p50_us": round(_pct(a_single, 0.5), 2),
            "stacked18_cold_us_per_layer": round(_pct(a_stack, 0.5) / 18, 2),
            "bytes_per_launch": int(a_bytes),
            "single_GBps": round(a_bytes / (_pct(a_single, 0.5) * 1e-6) / 1e9, 1),
            "stacked18_GBps": round(a_bytes * 18 / (_pct(a_stack, 0.5) * 1e-6) / 1e9, 1)},
        "attention_fp16_cache": {
            "workload": "joint attention, q [50, 8 x 256] f16, prefix K/V [968, 256] f16 with 900 valid, "
                        "suffix k/v [50, 256] f16, all N(0,1)/16 (mlcv_joint_attention; its oracle check is "
                        "tests/test_gpu_kernels.py::test_joint_attention_vs_oracle at this shape)",
            "single_cold_p50_us": round(_pct(c1_single, 0.5), 2),
            "stacked18_cold_us_per_layer": round(_pct(c1_stack, 0.5) / 18, 2),
            "bytes_per_launch": int(c1_bytes),
            "single_GBps": round(c1_bytes / (_pct(c1_single, 0.5) * 1e-6) / 1e9, 1),
            "stacked18_GBps": round(c1_bytes * 18 / (_pct(c1_stack, 0.5) * 1e-6) / 1e9, 1)},
        "prefill_ms": round(prefill_ms, 3),
        "loop_ms": round(loop_ms, 3),
        "step_roofline": {"bound": "hbm", "achieved": round(sbytes / (step_us * 1e-6) / 1e9, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(sbytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "bytes_per_step": int(sbytes), "flops_per_step": int(step_flops(cfg))},
        "roofline": {"kernel": dom, "symbol": KERNEL_SYMBOLS.get(dom, dom), "bound": "hbm",
                     "achieved": per_op[dom]["GBps"], "peak": HBM_PEAK_GBS,
                     "timing": "HIP events around --op-iters back-to-back launches on the step's stream (each "
                               "interval also holds the launch gap between dependent kernels)",
                     "unit": "GB/s", "frac": round(per_op[dom]["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": per_op[dom]["bytes"], "avg_launch_us": per_op[dom]["us"],
                     "measured_copy_GBps": round(copy_gbs, 1),
                     "frac_of_measured_copy": round(per_op[dom]["GBps"] / copy_gbs, 4)},
        "hbm_measured": {"copy_GBps": round(copy_gbs, 1), "spec_GBps": HBM_PEAK_GBS,
                         "protocol": "torch copy_ of 1 GiB fp32 device to device, 20 timed after 3 warm-ups; "
                                     "GB/s counts bytes read + written"},
        "per_op": per_op,
        "per_op_chain": per_op_chain,
    }
    # executed prefill flops: q/k/v of all 18 layers (their K/V are the output); attention,
    # o_proj, gate_up and down of the first 17 (the last layer's feed nothing)
    P0, W0, F0, NQ = 968, 2048, 16384, 2048
    pf_flops = 2 * P0 * W0 * 2560 * 18 + (2 * P0 * NQ * W0 + 2 * P0 * W0 * 2 * F0 + 2 * P0 * F0 * W0 +
                                          4 * 8 * P0 * P0 * 256) * 17
    out["prefill_mfma"] = {"tflops": round(pf_flops / (prefill_ms * 1e-3) / 1e12, 1),
                           "frac": round(pf_flops / (prefill_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                           "flops": int(pf_flops), "counted": "executed: q/k/v x 18 layers, the rest x 17"}

    if not args.no_q4:
        vmq, qparams = q4_model(cfg, dev, npar, params)
        vq = vmq["denoise_step_kv"](keys, values, x_t, te, c968, s968, pm_all, qparams)
        qstep = lambda: vmq["denoise_step_kv"](keys, values, x_t, te, c968, s968, pm_all, qparams)  # noqa: E731
        q_ms, _ = timed(qstep, args.steps, args.warmup)
        q_cold = per_cold(qstep, 30)
        qbytes = step_bytes(cfg, q4=True)
        v16 = step().numpy()
        cosq = float(np.dot(vq.numpy().ravel(), v16.ravel()) / (np.linalg.norm(vq.numpy()) * np.linalg.norm(v16)))
        out["q4f16_1_step"] = {"us": round(q_ms * 1e3, 1), "bytes_per_step": int(qbytes),
                               "frac": round(qbytes / (q_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                               "cos_vs_fp16": round(cosq, 5), "cold_p50_us": round(_pct(q_cold, 0.5), 1),
                               "cold_p90_us": round(_pct(q_cold, 0.9), 1)}
        del vmq, qparams

    # the float32 model at the 2-layer CPU-sized configuration (prefix expert 256 / 1024, action
    # expert 128 / 512, 2 heads of 64, prefix 32, horizon 8): prefill + 10 Euler steps
    out["f32_2layer_chunk"] = f32_chunk_timing(dev)

    if not args.no_embed:
        out["embed_image"] = embed_image_timing(cfg, dev)

    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def embed_image_timing(cfg, dev, iters: int = 10):
    """embed_image of one 224 x 224 image through the full SigLIP So400m/14 tower (27 layers)
    and the projector, random weights drawn on the GPU; HIP events around `iters` calls."""
    import torch

    from mlc_vla import runtime
    from mlc_vla.compile import compile_model

    ex, npar = compile_model(cfg, "rocm", functions=["embed_image"])
    vm = runtime.VirtualMachine(ex, dev)
    g = torch.Generator(device="cuda").manual_seed(0)
    params = []
    for name, p in npar:
        fan = p.shape[1] if len(p.shape) == 2 else 1
        t = torch.randn(p.shape, generator=g, device="cuda") / (fan ** 0.5 if len(p.shape) == 2 else 50.0)
        if "layer_norm" in name and name.endswith(".weight") or name.endswith("post_layernorm.weight"):
            t = t + 1.0
        params.append(runtime.as_tensor(t.half()))
    s = cfg.siglip
    img = runtime.as_tensor(torch.randn((1, s.image_size, s.image_size, s.num_channels), generator=g,
                                        device="cuda").half())
    for _ in range(2):
        vm["embed_image"](img, params)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        o = vm["embed_image"](img, params)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    flops = 2 * s.num_patches * (s.patch_size ** 2 * s.num_channels * s.hidden_size + s.num_hidden_layers * (
        4 * s.hidden_size ** 2 + 2 * s.hidden_size * s.intermediate_size + 2 * s.num_patches * s.hidden_size) +
        s.hidden_size * s.projection_dim)
    ok = bool(torch.isfinite(o.torch).all())
    del vm, params
    return {"workload": "SigLIP So400m/14 + projector, one 224x224 image (256 patches), fp16",
            "ms": round(ms, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 1), "finite": ok}


if __name__ == "__main__":
    main()
