#!/usr/bin/env python3
"""Benchmark: one AutonomousAICore TransformerLM training step on one MI355X.

Metric: train tokens/sec and % of bf16 MFMA peak for the 1B-class decoder
(16 layers, d 2048, 16 heads of 128, SwiGLU 5632, vocab 32000), B 4 x S 2048, bf16 AMP with
dynamic loss scaling, fp32 master weights and AdamW state, clip 1.0.  A step is forward +
backward + clip_grad_norm_ + AdamW on one synthetic batch (Zipf(1.1) ids) already resident
in HBM.  W warmup steps, then exactly K timed steps between device synchronisations.

Printed: one JSON line.  `roofline` describes the dominant kernel class (most GPU time in the
warm-up steps), timed with HIP events on the model's stream over the timed steps -- events on
that class only, since an event pair per launch adds queue time to every step;
`kernel_classes` gives every class from a second, fully event-timed run of the same steps.
`cpu_baseline` times the CPU oracle (restatement of the reference's AVX2 CPU step) on a
bounded sample on this host and extrapolates.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

CONFIGS = {
    "1b": dict(workload="1B-class decoder, bf16 AMP training step (BASELINE configs[2])", vocab=32000, d=2048, L=16,
               H=16, f=5632, B=4, S=2048, amp=True, resid_scale=False),
    "125m": dict(workload="125M-class decoder, bf16 AMP training step (BASELINE configs[1])", vocab=32000, d=768,
                 L=12, H=12, f=2048, B=8, S=1024, amp=True, resid_scale=True),
    "tiny": dict(workload="tiny decoder, fp32 training step, tied embeddings (BASELINE configs[0])", vocab=512,
                 d=128, L=2, H=4, f=352, B=8, S=64, amp=False, resid_scale=False, compute="float32", tied=True),
    "moe": dict(workload="sparse MoE decoder, 8 experts top-2, bf16 AMP training step (BASELINE configs[3])",
                vocab=32000, d=1024, L=12, H=16, f=2816, B=8, S=1024, amp=True, resid_scale=False, experts=8,
                top_k=2),
    "qlora": dict(workload="QLoRA step on the 1B shape: INT4 base (G 128, fp16 scales), rank-16 alpha-32 adapters "
                           "on 7 projections, bf16 AMP (BASELINE configs[4])", vocab=32000, d=2048, L=16, H=16,
                  f=5632, B=4, S=2048, amp=True, resid_scale=False, lora_rank=16, lora_alpha=32.0, group=128),
}


def matmul_params(c):
    """Matmul parameters a token passes through (the MoE router and its top_k experts only)."""
    d, f, V, L = c["d"], c["f"], c["vocab"], c["L"]
    if c.get("experts"):
        return L * (4 * d * d + c["experts"] * d + c["top_k"] * 3 * d * f) + V * d
    return L * (4 * d * d + 3 * d * f) + V * d  # lm_head; the embedding gather has no FLOPs


def total_params(c):
    d, f, V, L, E = c["d"], c["f"], c["vocab"], c["L"], c.get("experts", 0)
    per_layer = 4 * d * d + (E * d + E * 3 * d * f if E else 3 * d * f) + 2 * d
    return L * per_layer + d + V * d * (1 if c.get("tied") else 2)


def lora_params(c):
    d, f, r = c["d"], c["f"], c.get("lora_rank", 0)
    return c["L"] * (4 * 2 * r * d + 2 * (r * d + f * r) + r * f + d * r)


def step_flops(c):
    """Algorithmic FLOPs per step: 6 T P_mm + 6 L T S d (causal attention: forward Q K^T and
    P V at 2 S d per token per layer on the causal average, backward twice that).  QLoRA: the
    frozen base has no weight gradient, 4 T P_mm, plus 6 T P_lora for the adapters."""
    T = c["B"] * c["S"]
    attn = 6.0 * c["L"] * T * c["S"] * c["d"]
    if c.get("lora_rank"):
        return 4.0 * T * matmul_params(c) + 6.0 * T * lora_params(c) + attn
    return 6.0 * T * matmul_params(c) + attn


def profiled_traffic(kernel_class, config):
    """HBM bytes per launch of a kernel class in this workload, from its committed rocprofv3 PMC
    summary (lines `traffic <class> <bytes>` written by autonomousaicore_amd.rocprof_summary in
    profiles/lm_step_<config>_kernel_classes.txt), or None."""
    path = os.path.join(HERE, "profiles", f"lm_step_{config}_kernel_classes.txt")
    if not os.path.isfile(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel_class:
                return int(parts[2])
    return None


def host_cpu():
    """nproc (CPUs this process may run on), online CPUs, and the CPU model name (lscpu's)."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": nproc, "online_cpus": os.cpu_count(), "model": model}


def cpu_baseline(c, seed=1234):
    """Time the oracle on one layer at the config's widths, B=1 x S, and extrapolate to the
    full step (L layers, B sequences, all parameters in AdamW)."""
    from oracle import oracle as orc

    orc.build()
    host = host_cpu()
    # the reference's GEMM row split: min(hardware threads, 24) (src/ops/cpu_gemm.cpp:143-146);
    # hardware threads = the CPUs this process may run on
    threads = max(1, min(host["nproc"], 24))
    orc.set_threads(threads)
    S = c["S"]
    E = c.get("experts", 0)
    cfg = orc.make_config(c["vocab"], c["d"], 1, c["H"], c["f"], S, norm_eps=1e-6, n_experts=E,
                          top_k=c.get("top_k", 2), tied=c.get("tied", False))
    n = orc.num_params(cfg)
    import autonomousaicore_amd as aic
    params = aic.normal(5678, n, 0.0, 0.02)
    d = c["d"]
    # norms at 1: norm1/norm2 of the layer and the final norm (oracle order: embedding, q k v o,
    # FFN or router + experts, norm1, norm2, final norm, head)
    V, f = c["vocab"], c["f"]
    off = V * d + 4 * d * d + (E * d + E * 3 * d * f if E else 3 * d * f)
    params[off:off + 3 * d] = 1.0
    ids, tgt = aic.batch(seed, 1, S, c["vocab"], dist="zipf")
    r = c.get("lora_rank", 0)
    if r:
        nl = orc.qlora_num_params(cfg, r)
        lora = aic.normal(9012, nl, 0.0, 0.02)
        trainable = lora_params(c)

        def one_step():
            return orc.qlora_step(cfg, r, c["lora_alpha"], c["group"], params, lora.copy(), ids, tgt, 1, S)[0]
    else:
        trainable = total_params(c)

        def one_step():
            return orc.lm_step(cfg, params.copy(), ids, tgt, 1, S)[0]
    n_opt = nl if r else n
    full_params = trainable
    # one untimed warm-up, then the median of three sample steps (each from the same weights)
    one_step()
    t0 = time.perf_counter()
    est = []
    for _ in range(3):
        res = one_step()
        per_token = (res.t_embed + res.t_embed_bwd + res.t_head_fwd + res.t_loss + res.t_head_bwd)
        blocks = res.t_blocks_fwd + res.t_blocks_bwd
        est.append(c["B"] * (per_token + c["L"] * blocks) + res.t_optim * (full_params / n_opt))
    wall = time.perf_counter() - t0
    t_step = sorted(est)[1]
    tokens = c["B"] * S
    return {
        "value": round(tokens / t_step, 2),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "nproc": host["nproc"],
        "online_cpus": host["online_cpus"],
        "cpu_model": host["model"],
        "thread_rule": "min(nproc, 24) GEMM threads as src/ops/cpu_gemm.cpp:143-146; elementwise ops single-threaded",
        "sample": (f"oracle fp32 step (restatement of the reference AVX2 CPU path) on 1 layer at the "
                   f"config widths, B=1 x S={S}, median of 3 after 1 warm-up ({wall:.1f} s timed); extrapolated to {c['L']} layers, "
                   f"B={c['B']} and AdamW over {full_params / 1e6:.0f}M parameters: {t_step:.1f} s/step"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="1b", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="before the model, copy a buffer of this many MiB once (a known-size kernel that calibrates "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if args.warmup < 1 or args.steps < 1:
        ap.error("--warmup and --steps must be at least 1 (the last warm-up step names the dominant class)")

    import torch

    import autonomousaicore_amd as aic

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    c = CONFIGS[args.config]
    B, S = c["B"], c["S"]
    free0, total = torch.cuda.mem_get_info()
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    model = aic.TransformerLM(
        aic.TransformerLMConfig(vocab_size=c["vocab"], hidden_dim=c["d"], num_layers=c["L"], num_heads=c["H"],
                                intermediate_dim=c["f"], max_seq_len=S, rms_norm_eps=1e-6,
                                compute=c.get("compute", "bfloat16"), tie_word_embeddings=c.get("tied", False),
                                num_experts=c.get("experts", 0), top_k=c.get("top_k", 2), aux_loss_coef=0.01,
                                lora_rank=c.get("lora_rank", 0), lora_alpha=c.get("lora_alpha", 32.0),
                                quant_group=c.get("group", 128)),
        aic.TrainingConfig(adamw=aic.AdamWOptions(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1),
                           max_grad_norm=1.0, use_amp=c["amp"]))
    model.init_normal(5678, 0.02, residual_scaling=c["resid_scale"])
    ids, tgt = aic.batch(1234, B, S, c["vocab"], dist="zipf")
    ids_d = torch.from_numpy(ids).cuda()
    tgt_d = torch.from_numpy(tgt).cuda()
    torch.cuda.synchronize()

    def run(n):
        for _ in range(n):
            model.train_step(ids_d.data_ptr(), tgt_d.data_ptr(), B, S, sync=False)
        model.synchronize()
        torch.cuda.synchronize()

    def class_table(classes, steps):
        kc = {}
        for k in classes:
            avg_ms = k["total_ms"] / k["launches"]
            if k["mfma_bound"]:
                ach = k["flops"] / (k["total_ms"] * 1e-3) / 1e12
                kc[k["name"]] = dict(bound="mfma", launches=k["launches"], avg_ms=round(avg_ms, 4),
                                     ms_per_step=round(k["total_ms"] / steps, 3), achieved=round(ach, 1),
                                     unit="TFLOP/s", frac=round(ach / PEAK_BF16_TFLOPS, 4))
            else:
                ach = k["bytes"] / (k["total_ms"] * 1e-3) / 1e9
                kc[k["name"]] = dict(bound="hbm", launches=k["launches"], avg_ms=round(avg_ms, 4),
                                     ms_per_step=round(k["total_ms"] / steps, 3), achieved=round(ach, 1),
                                     unit="GB/s", frac=round(ach / PEAK_HBM_GBS, 4))
        return kc

    # warm-up; its last step has every class timed with HIP events and names the dominant class
    # (the most GPU time).  The first step also allocates the step's workspace, which would be
    # charged to whichever class's events bracket the allocation, so it is not the one timed.
    run(max(args.warmup - 1, 0))
    model.set_profiling(True)
    run(1)
    warm = model.profile_stats()
    model.set_profiling(False)
    dom_name = max(warm, key=lambda k: k["total_ms"])["name"]

    # timed region: only the dominant class carries events (an event pair adds a few microseconds
    # of queue time per launch, so timing every launch would lengthen the step being measured)
    model.set_profiling(True, classes=[dom_name])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps)
    elapsed = time.perf_counter() - t0
    stats = model.last_stats()
    timed = model.profile_stats()
    model.set_profiling(False)

    # the per-class table comes from a separate pass of the same steps with every class timed
    model.set_profiling(True)
    run(args.steps)
    kc = class_table(model.profile_stats(), args.steps)
    model.set_profiling(False)

    ms = 1000.0 * elapsed / args.steps
    tokens_per_s = B * S * args.steps / elapsed
    # device memory the model holds after the steps (parameters, optimiser state, the persistent
    # step workspace and the library's pool), from hipMemGetInfo around the whole run
    free1, _ = torch.cuda.mem_get_info()
    flops = step_flops(c)
    classes = timed
    d = class_table(classes, args.steps)[dom_name]
    roofline = {"kernel": dom_name, "bound": d["bound"], "achieved": d["achieved"],
                "peak": PEAK_BF16_TFLOPS if d["bound"] == "mfma" else PEAK_HBM_GBS, "unit": d["unit"],
                "frac": d["frac"], "avg_launch_ms": d["avg_ms"], "launches": d["launches"],
                "timed_in": "the timed steps (events on this class only)",
                "traffic": profiled_traffic(dom_name, args.config)}

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(c)
        except Exception as e:  # the GPU figure stands on its own; report why the baseline is missing
            cpu = {"value": None, "unit": "tokens/s", "cores": None, "kind": "port", "sample": f"failed: {e}"}

    out = {
        "metric": "train tokens/sec + % bf16 MFMA peak, 1B-class LM step on 1 MI355X",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if c.get("compute") == "float32" else "bf16",
        "data": "synthetic",
        "config": {"workload": c["workload"], "layers": c["L"], "d_model": c["d"], "heads": c["H"],
                   "d_ffn": c["f"], "vocab": c["vocab"], "global_batch": B, "seq_len": S,
                   "tokens_per_step": B * S, "parallelism": "none (1 GPU)",
                   **({"experts": c["experts"], "top_k": c["top_k"]} if c.get("experts") else {}),
                   **({"lora_rank": c["lora_rank"], "lora_alpha": c["lora_alpha"], "quant_group": c["group"],
                       "trainable_params": lora_params(c)} if c.get("lora_rank") else {})},
        "step_flops": flops,
        "mfma_peak_frac_step": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "loss": round(float(stats.loss), 5),
        "loss_scale": stats.loss_scale,
        "hbm_in_use_gib": round((free0 - free1) / 2**30, 2),
        "roofline": roofline,
        "kernel_classes": kc,
        "kernel_classes_pass": "a second run of the same steps after the timed region, every class timed",
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    model.close()


if __name__ == "__main__":
    main()
