"""Summarise rocprofv3 output of bench.py by kernel class.

    python -m autonomousaicore_amd.rocprof_summary --stats DIR/run_kernel_stats.csv \
        [--fetch DIR/run_counter_collection.csv --write DIR/run_counter_collection.csv \
         --copy-probe-mib 1024] [--steps N]
    python -m autonomousaicore_amd.rocprof_summary --pmc DIR1/run_counter_collection.csv \
        [DIR2/run_counter_collection.csv ...]
    python -m autonomousaicore_amd.rocprof_summary --bench BENCH_JSON_LINE_FILE

--bench prints the per-class roofline table of a bench.py JSON line (its `kernel_classes`:
event-timed launches, achieved TFLOP/s or GB/s against the MI355X peak, fraction).

Kernel symbols map to the same classes as the library's event profiler (the class a launch
is timed under inside TransformerLM::train_step), so the per-class average launch time here
can be compared with bench.py's `kernel_classes[...].avg_ms`.

Traffic: FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are summed per class and divided by the
class's dispatch count.  Each counter is scaled by expected/measured on the copy kernel that
`bench.py --copy-probe-mib M` runs before the model (a device-to-device copy of M MiB reads
and writes exactly M MiB).  The scaled per-launch byte counts are printed as
`traffic <class> <bytes>` lines, which bench.py reads back for its `roofline.traffic`.

Counters (--pmc, one or more counter-collection files from separate rocprofv3 --pmc passes):
per kernel symbol of the MFMA classes (GEMMs, attention), the per-dispatch average of every
counter collected, and from them, with cycles = GRBM_GUI_ACTIVE / XCDs (rocprofv3 sums the
counter over the 8 XCDs, each counting the same kernel cycles):
  mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (cycles * SIMDs)   (the matrix pipes' duty)
  lds_util  = SQ_LDS_IDX_ACTIVE / (cycles * CUs)
  lds_confl = SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT)
  l2_hit    = TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)
  mfma_flop = SQ_INSTS_VALU_MFMA_MOPS_BF16 * 512 (the bf16 MFMA work executed)
  clock     = cycles / the kernel's duration (with --stats of the same command)
with the MI355X's 256 CUs of 4 SIMDs in 8 XCDs (--cus, --xcds).  Passes are run one counter
set at a time (rocprofv3 collects what one pass can hold), each on the same bench.py command.
"""
from __future__ import annotations

import argparse
import csv
import re
from collections import defaultdict

# (regex on the demangled or mangled symbol, class); first match wins.
_RULES = [
    # gemm_bf16_dma_q4<BM, BN, BK, STAGES, transB, C>: the INT4-operand forward / input gradient
    (r"gemm_bf16_dma_q4(<(\d+, )+true|I(Li\d+E)+Lb1E)", "gemm_fwd"),
    (r"gemm_bf16_dma_q4(<(\d+, )+false|I(Li\d+E)+Lb0E)", "gemm_dgrad"),
    # gemm_bf16_dma[_grouped|_ragged|_pers]<BM, BN, BK, STAGES, transA, transB, C, ...>, demangled
    # or mangled
    (r"gemm_bf16_dma(_grouped|_ragged|_pers)?(<(\d+, )+false, true|I(Li\d+E)+Lb0ELb1E)", "gemm_fwd"),
    (r"gemm_bf16_dma(_grouped|_ragged|_pers)?(<(\d+, )+false, false|I(Li\d+E)+Lb0ELb0E)", "gemm_dgrad"),
    (r"gemm_bf16_dma(_grouped|_ragged|_pers)?(<(\d+, )+true, false|I(Li\d+E)+Lb1ELb0E)", "gemm_wgrad"),
    # the K-split last round of an expert-ragged product, gemm_bf16_dma_rag_tail<transB>
    (r"gemm_bf16_dma_rag_tail(<true>|ILb1E)", "gemm_fwd"),
    (r"gemm_bf16_dma_rag_tail(<false>|ILb0E)", "gemm_dgrad"),
    (r"attn_fwd", "attn_fwd"),
    (r"attn_bwd|attn_dot", "attn_bwd"),
    (r"rmsnorm_fwd", "rmsnorm_fwd"),
    (r"rmsnorm_bwd|reduce_parts", "rmsnorm_bwd"),
    (r"rope_k|rope_v", "rope"),
    (r"swiglu_fwd", "swiglu_fwd"),
    (r"swiglu_bwd", "swiglu_bwd"),
    # a training step's loss: count, fused forward+backward and the mean in one event scope
    (r"ce_fused|ce_count|ce_mean", "ce_fwd_bwd"),
    (r"ce_fwd", "ce_fwd"),
    (r"ce_bwd", "ce_bwd"),
    (r"embed_fwd", "embed_fwd"),
    (r"embed_chunk_sort|embed_merge_rank|embed_seg|embed_run|embed_zero_absent", "embed_bwd"),
    # the norm pass, or (fused) the slot clear, the embedding / norm-weight partials and the
    # two-level sum of every slot
    (r"sqnorm|sqsum|sqslot|finalize", "grad_norm"),
    (r"sq_matrix", "gemm_wgrad"),
    (r"adamw", "adamw"),
    (r"lora_skinny|lora_reduce|lora_xa", "lora"),
    # kernels outside bench.py's event classes (the MoE and QLoRA configurations)
    (r"moe_", "moe_routing"),
    (r"int4_quantize", "other"),  # the base's one-time quantization at set-up, like the weight init
    (r"int4_", "int4"),
    (r"splitk_reduce|rag_tail_reduce", "gemm_splitk_reduce"),
]


# Classes timed as one event scope around several kernels: the kernel launched once per
# scope, so per-launch figures here are per scope, as in bench.py.
_ANCHOR = {
    # an expert-ragged product's split last round runs in the same scope as its persistent launch
    "gemm_fwd": r"gemm_bf16_dma(?!_rag_tail)",
    "gemm_dgrad": r"gemm_bf16_dma(?!_rag_tail)",
    "attn_bwd": r"attn_bwd_dq",
    "rmsnorm_bwd": r"rmsnorm_bwd",
    "grad_norm": r"sqnorm_final",
    "ce_fwd_bwd": r"ce_fused",
    "embed_bwd": r"embed_chunk_sort",
}


def is_anchor(cls: str, name: str) -> bool:
    pat = _ANCHOR.get(cls)
    return pat is None or re.search(pat, name) is not None


def kernel_class(name: str) -> str:
    for pat, cls in _RULES:
        if re.search(pat, name):
            return cls
    return "other"


def read_stats(path):
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((r["Name"], int(r["Calls"]), float(r["TotalDurationNs"])))
    return rows


def read_counter(path, counter):
    """Per-dispatch values of one counter: list of (kernel name, KiB)."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                out.append((r["Kernel_Name"], float(r["Counter_Value"])))
    return out


def copy_factor(disp, mib):
    """expected / measured for the largest device copy in the run."""
    copies = [v for n, v in disp if "copyBuffer" in n]
    if not copies or mib <= 0:
        return None
    return (mib * 1024.0) / max(copies)


MFMA_CLASSES = ("gemm_fwd", "gemm_dgrad", "gemm_wgrad", "attn_fwd", "attn_bwd")


def pmc_summary(paths, cus, xcds):
    """Per-kernel per-dispatch counter averages over the MFMA classes, with derived ratios."""
    vals = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(lambda: defaultdict(set))
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                k, c = r["Kernel_Name"], r["Counter_Name"]
                vals[k][c] += float(r["Counter_Value"])
                disp[k][c].add(r.get("Dispatch_Id", len(disp[k][c])))
    rows = []
    for k, cs in vals.items():
        cls = kernel_class(k)
        if cls not in MFMA_CLASSES:
            continue
        avg = {c: v / max(len(disp[k][c]), 1) for c, v in cs.items()}
        n = max(len(d) for d in disp[k].values())
        rows.append((cls, -n, k, n, avg))
    rows.sort()
    simds = 4 * cus
    print("# MFMA-class kernels: per-dispatch counter averages (rocprofv3 --pmc passes)")
    print(f"{'class':<11} {'disp':>5} {'mfma_busy':>9} {'lds_util':>8} {'lds_confl':>9} {'l2_hit':>6} "
          f"{'mfma_TFLOP':>10}  kernel")
    for cls, _, k, n, a in rows:
        def ratio(num, den):
            return a[num] / a[den] if num in a and den in a and a[den] > 0 else float("nan")
        act = a.get("GRBM_GUI_ACTIVE", float("nan")) / xcds
        mb = a["SQ_VALU_MFMA_BUSY_CYCLES"] / (act * simds) if "SQ_VALU_MFMA_BUSY_CYCLES" in a else float("nan")
        lu = a["SQ_LDS_IDX_ACTIVE"] / (act * cus) if "SQ_LDS_IDX_ACTIVE" in a else float("nan")
        lc = (a["SQ_LDS_BANK_CONFLICT"] / (a["SQ_LDS_IDX_ACTIVE"] - a["SQ_LDS_BANK_CONFLICT"])
              if "SQ_LDS_BANK_CONFLICT" in a and "SQ_LDS_IDX_ACTIVE" in a else float("nan"))
        hit, miss = a.get("TCC_HIT_sum"), a.get("TCC_MISS_sum")
        l2 = hit / (hit + miss) if hit is not None and miss is not None and hit + miss > 0 else float("nan")
        fl = a.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", float("nan")) * 512 / 1e12
        short = k if len(k) <= 100 else k[:97] + "..."
        print(f"{cls:<11} {n:>5} {mb:>9.3f} {lu:>8.3f} {lc:>9.3f} {l2:>6.3f} {fl:>10.4f}  {short}")
    issue = [r for r in rows if "SQ_WAVE_CYCLES" in r[4] and "SQ_INSTS_MFMA" in r[4]]
    if issue:
        # where a wave's cycles go: issuing (SQ_ACTIVE_INST_ANY), waiting on a counter or barrier
        # (SQ_WAIT_ANY), waiting for an instruction to be issuable (SQ_WAIT_INST_ANY), as fractions
        # of SQ_WAVE_CYCLES; and the instructions the waves executed per MFMA
        print("\n# issue and waits per wave cycle; instructions per MFMA")
        print(f"{'class':<11} {'issue':>6} {'wait':>6} {'wait_inst':>9} {'valu/mfma':>9} {'trans/mfma':>10} "
              f"{'lds/mfma':>8}  kernel")
        for cls, _, k, n, a in issue:
            wc, mf = a["SQ_WAVE_CYCLES"], max(a["SQ_INSTS_MFMA"], 1.0)

            def frac(c):
                return a[c] / wc if c in a and wc > 0 else float("nan")

            def per(c):
                return a[c] / mf if c in a else float("nan")

            valu = (a["SQ_INSTS_VALU"] - a["SQ_INSTS_MFMA"]) / mf if "SQ_INSTS_VALU" in a else float("nan")
            short = k if len(k) <= 100 else k[:97] + "..."
            print(f"{cls:<11} {frac('SQ_ACTIVE_INST_ANY'):>6.3f} {frac('SQ_WAIT_ANY'):>6.3f} "
                  f"{frac('SQ_WAIT_INST_ANY'):>9.3f} {valu:>9.2f} {per('SQ_INSTS_VALU_TRANS_F32'):>10.2f} "
                  f"{per('SQ_INSTS_LDS'):>8.2f}  {short}")
    print("\n# raw per-dispatch averages")
    for cls, _, k, n, a in rows:
        short = k if len(k) <= 100 else k[:97] + "..."
        print(f"{cls} {short}")
        print("    " + ", ".join(f"{c}={v:.4g}" for c, v in sorted(a.items())))


def bench_summary(path):
    """The kernel_classes table of the last bench.py JSON line in a file."""
    import json

    line = None
    with open(path) as f:
        for ln in f:
            ln = ln.strip()
            if ln.startswith("{") and '"kernel_classes"' in ln:
                line = ln
    if line is None:
        raise SystemExit(f"{path}: no bench.py JSON line")
    b = json.loads(line)
    print(f"# bench.py: {b['value'] / 1e3:.1f} k tokens/s, {b['ms_per_step']:.2f} ms/step, "
          f"{100 * b['mfma_peak_frac_step']:.1f}% of the bf16 peak over the step ({b['steps']} timed steps)")
    print("# per-class roofline (bench.py kernel_classes: HIP events on every class; MFMA classes against "
          "2500 TFLOP/s, HBM classes against 8000 GB/s)")
    print(f"{'class':<13} {'bound':>5} {'launches':>8} {'avg_ms':>8} {'ms/step':>8} {'achieved':>13} {'frac':>6}")
    for name, k in sorted(b["kernel_classes"].items(), key=lambda kv: -kv[1]["ms_per_step"]):
        unit = "TFLOP/s" if k["unit"] == "TFLOP/s" else "GB/s"
        print(f"{name:<13} {k['bound']:>5} {k['launches']:>8} {k['avg_ms']:>8.4f} {k['ms_per_step']:>8.3f} "
              f"{k['achieved']:>7.1f} {unit:<5} {k['frac']:>6.3f}")


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--stats")
    ap.add_argument("--pmc", nargs="+", help="counter-collection CSVs of rocprofv3 --pmc passes")
    ap.add_argument("--cus", type=int, default=256, help="compute units (MI355X: 256, 4 SIMDs each)")
    ap.add_argument("--xcds", type=int, default=8, help="XCDs the GRBM counter is summed over (MI355X: 8)")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-probe-mib", type=int, default=0)
    ap.add_argument("--steps", type=int, default=0, help="train steps in the profiled run (for ms/step)")
    ap.add_argument("--bench", help="a file holding bench.py's JSON line")
    args = ap.parse_args(argv)
    if args.bench:
        bench_summary(args.bench)
        if not (args.stats or args.pmc):
            return
        print()
    if args.pmc:
        pmc_summary(args.pmc, args.cus, args.xcds)
        if not args.stats:
            return
    if not args.stats:
        ap.error("--stats or --pmc is required")

    per = defaultdict(lambda: [0, 0.0])
    kernels = []
    for name, calls, tot in read_stats(args.stats):
        cls = kernel_class(name)
        if is_anchor(cls, name):
            per[cls][0] += calls
        per[cls][1] += tot
        kernels.append((tot, calls, cls, name))
    grand = sum(v[1] for v in per.values())
    print("# kernel classes (rocprofv3 --kernel-trace --stats); launches = event scopes, avg = per scope")
    print(f"{'class':<13} {'launches':>8} {'total_ms':>10} {'avg_us':>9} {'share':>6}" +
          (f" {'ms/step':>8}" if args.steps else ""))
    for cls, (calls, tot) in sorted(per.items(), key=lambda kv: -kv[1][1]):
        line = f"{cls:<13} {calls:>8} {tot / 1e6:>10.3f} {tot / max(calls, 1) / 1e3:>9.1f} {100 * tot / grand:>5.1f}%"
        if args.steps:
            line += f" {tot / 1e6 / args.steps:>8.3f}"
        print(line)
    print("\n# kernels (top 20 by total time)")
    for tot, calls, cls, name in sorted(kernels, reverse=True)[:20]:
        short = name if len(name) <= 110 else name[:107] + "..."
        print(f"{cls:<13} {calls:>6} {tot / calls / 1e3:>9.1f} us  {short}")

    if args.fetch and args.write:
        fd = read_counter(args.fetch, "FETCH_SIZE")
        wd = read_counter(args.write, "WRITE_SIZE")
        ff = copy_factor(fd, args.copy_probe_mib)
        wf = copy_factor(wd, args.copy_probe_mib)
        print("\n# HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)")
        print(f"copy probe {args.copy_probe_mib} MiB: FETCH_SIZE scale {ff:.4f}, WRITE_SIZE scale {wf:.4f}")
        acc = defaultdict(lambda: [0, 0.0, 0, 0.0])
        for n, v in fd:
            c = kernel_class(n)
            a = acc[c]
            a[0] += is_anchor(c, n)
            a[1] += v
        for n, v in wd:
            c = kernel_class(n)
            a = acc[c]
            a[2] += is_anchor(c, n)
            a[3] += v
        print(f"{'class':<13} {'launches':>8} {'fetch_MB':>10} {'write_MB':>10}")
        for cls, (nf, sf, nw, sw) in sorted(acc.items()):
            if cls == "other" or nf == 0 or nw == 0:
                continue
            fb = sf * 1024.0 * ff / nf
            wb = sw * 1024.0 * wf / nw
            print(f"{cls:<13} {nf:>8} {fb / 1e6:>10.2f} {wb / 1e6:>10.2f}")
        print()
        for cls, (nf, sf, nw, sw) in sorted(acc.items()):
            if cls == "other" or nf == 0 or nw == 0:
                continue
            print(f"traffic {cls} {int(round(sf * 1024.0 * ff / nf + sw * 1024.0 * wf / nw))}")


if __name__ == "__main__":
    main()
