"""Per-shape GEMM timing against the vendor library, and the HBM streaming ceiling, on one GPU.

    python -m autonomousaicore_amd.gemm_shapes [--config 1b] [--reps 10] [--rounds 3]

For every product of the configuration's training step (forward x W^T, input gradient dy W and
weight gradient dy^T x of the q/k/v, output, gate/up and down projections and the head), the
library's plain GEMM entry (aic_hip_gemm: no fused epilogue) and torch.matmul on the same
operands (hipBLASLt on ROCm for bf16) are timed with HIP events on one stream: `reps` launches
per timing, `rounds` alternating timings of each, the best round kept.  Weight gradients are
fp32 outputs in the library (the step's master gradients); torch is given out_dtype=float32
where its mm accepts it, else it writes bf16 (stated per row).

The streaming ceiling: torch's own device kernels over 2 GiB buffers -- copy (read + write),
sum (read), fill (write) and add_ (2 reads + 1 write) -- timed the same way, in GB/s of
algorithmic bytes.  It is what a plain streaming kernel reaches on this GPU, the practical
ceiling for the HBM-bound classes (the MI355X's published 8 TB/s is the roofline peak).
Beside it, the library's own streaming probe (aic_hip_stream_probe: one pass in the AdamW
kernel's form, plain and non-temporal accesses) over the same buffers for the read, write,
copy, add and AdamW byte mixes (4 fp32 reads, 3 fp32 writes and a bf16 copy per element), and
the AdamW kernel itself (aic_hip_adamw_multi with the bf16 copy) over that many elements.
"""
from __future__ import annotations

import argparse
import json

import torch

from . import _lib

CONFIGS = {
    "1b": dict(T=8192, d=2048, f=5632, V=32000),
    "125m": dict(T=8192, d=768, f=2048, V=32000),
}


def shapes(c):
    """(name, kind, M, N, K) of the step's products: fwd C = x W^T, dgrad C = dy W, wgrad C = dy^T x."""
    T, d, f, V = c["T"], c["d"], c["f"], c["V"]
    proj = [("qkv", 3 * d, d), ("o", d, d), ("gate_up", 2 * f, d), ("down", d, f), ("head", V, d)]
    out = []
    for name, n_out, n_in in proj:
        out.append((name, "fwd", T, n_out, n_in))
        out.append((name, "dgrad", T, n_in, n_out))
        out.append((name, "wgrad", n_out, n_in, T))
    return out


def _time(fn, reps, stream):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def gemm_table(c, reps, rounds):
    lib = _lib.load()
    BF16, F32 = _lib.AIC_BF16, _lib.AIC_F32
    s = torch.cuda.current_stream()
    rows = []
    for name, kind, M, N, K in shapes(c):
        g = torch.Generator(device="cuda").manual_seed(M + N + K)
        if kind == "fwd":
            a = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)   # x [T, in]
            b = torch.randn((N, K), device="cuda", generator=g).to(torch.bfloat16)   # W [out, in]
            ta, tb, lda, ldb, ct = 0, 1, K, K, torch.bfloat16

            def ref():
                return torch.nn.functional.linear(a, b)
        elif kind == "dgrad":
            a = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)   # dy [T, out]
            b = torch.randn((K, N), device="cuda", generator=g).to(torch.bfloat16)   # W [out, in]
            ta, tb, lda, ldb, ct = 0, 0, K, N, torch.bfloat16

            def ref():
                return torch.mm(a, b)
        else:
            a = torch.randn((K, M), device="cuda", generator=g).to(torch.bfloat16)   # dy [T, out]
            b = torch.randn((K, N), device="cuda", generator=g).to(torch.bfloat16)   # x [T, in]
            ta, tb, lda, ldb, ct = 1, 0, M, N, torch.float32
            at = a.t()

            def ref():
                return torch.mm(at, b, out_dtype=torch.float32)
        out = torch.empty((M, N), dtype=ct, device="cuda")
        cdt = F32 if ct == torch.float32 else BF16
        ref_note = "bf16 out"
        if kind == "wgrad":
            try:
                ref()
                ref_note = "fp32 out"
            except (TypeError, RuntimeError):
                def ref():
                    return torch.mm(at, b)

        def ours():
            _lib.check(lib.aic_hip_gemm(ta, tb, M, N, K, 1.0, a.data_ptr(), lda, b.data_ptr(), ldb, 0.0,
                                        out.data_ptr(), N, None, 0, BF16, cdt, s.cuda_stream))
        for fn in (ours, ref, ours, ref):  # warm-up (and the libraries' first-call set-up)
            fn()
        torch.cuda.synchronize()
        t_ours, t_ref = [], []
        for _ in range(rounds):
            t_ours.append(_time(ours, reps, s))
            t_ref.append(_time(ref, reps, s))
        flops = 2.0 * M * N * K
        to, tr = min(t_ours), min(t_ref)
        rows.append(dict(product=name, kind=kind, M=M, N=N, K=K, ours_us=round(1e3 * to, 1),
                         ours_tflops=round(flops / (to * 1e-3) / 1e12, 1), ours_frac=round(flops / (to * 1e-3) / 2.5e15, 3),
                         lib_us=round(1e3 * tr, 1), lib_tflops=round(flops / (tr * 1e-3) / 1e12, 1),
                         lib_frac=round(flops / (tr * 1e-3) / 2.5e15, 3), lib_out=ref_note if kind == "wgrad" else "bf16 out"))
        del a, b, out
        torch.cuda.empty_cache()
    return rows


def stream_ceiling(reps, rounds, gib=2):
    n = gib * (1 << 30) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.ones(n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    nb = 4.0 * n
    tests = [("copy (read + write)", lambda: y.copy_(x), 2 * nb), ("sum (read)", lambda: x.sum(), nb),
             ("fill (write)", lambda: y.fill_(1.0), nb), ("add_ (2 reads + 1 write)", lambda: y.add_(x), 3 * nb)]
    out = []
    for name, fn, bytes_ in tests:
        fn()
        torch.cuda.synchronize()
        t = min(_time(fn, reps, s) for _ in range(rounds))
        out.append(dict(kernel=name, bytes=int(bytes_), ms=round(t, 4), gbs=round(bytes_ / (t * 1e-3) / 1e9, 1)))
    return out


def probe_ceiling(reps, rounds, gib=2):
    import ctypes as C

    lib = _lib.load()
    n = gib * (1 << 30) // 4
    ins = [torch.full((n,), 1.0 + k, dtype=torch.float32, device="cuda") for k in range(4)]
    outs = [torch.empty(n, dtype=torch.float32, device="cuda") for _ in range(3)]
    ob = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    sink = torch.empty(1, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    vp = C.c_void_p
    mixes = [("read", 1, 0, False), ("write", 0, 1, False), ("copy (read + write)", 1, 1, False),
             ("add (2 reads + 1 write)", 2, 1, False), ("AdamW mix (4r + 3w + bf16)", 4, 3, True)]
    out = []
    for name, ni, no, b16 in mixes:
        for nt in (0, 1):
            pin = (vp * 4)(*[t.data_ptr() for t in ins])
            pout = (vp * 3)(*[t.data_ptr() for t in outs])

            def fn(ni=ni, no=no, b16=b16, nt=nt, pin=pin, pout=pout):
                _lib.check(lib.aic_hip_stream_probe(pin, ni, pout, no, ob.data_ptr() if b16 else None,
                                                    sink.data_ptr(), n, nt, s.cuda_stream))

            fn()
            torch.cuda.synchronize()
            if no:  # the probe's result on a prefix: out_j = sum of the inputs + j
                want = sum(float(1 + k) for k in range(ni)) + (no - 1)
                assert bool((outs[no - 1][:1 << 20] == want).all()), name
            t = min(_time(fn, reps, s) for _ in range(rounds))
            bytes_ = n * (4 * ni + 4 * no + (2 if b16 else 0))
            out.append(dict(kernel=f"{name}, {'non-temporal' if nt else 'plain'}", bytes=int(bytes_), ms=round(t, 4),
                            gbs=round(bytes_ / (t * 1e-3) / 1e9, 1)))
    # the AdamW kernel itself over the same element count (4 reads, 3 writes, bf16 copy)
    p, g, m, v = (t.clone() for t in ins)
    arr = lambda t: (vp * 1)(t.data_ptr())
    sizes = (C.c_int64 * 1)(n)
    ap, ag, am, av, ab = arr(p), arr(g), arr(m), arr(v), (vp * 1)(ob.data_ptr())

    def adam():
        _lib.check(lib.aic_hip_adamw_multi(ap, ag, am, av, ab, sizes, 1, 1e-4, 0.9, 0.95, 1e-8, 0.1, 1, None,
                                           s.cuda_stream))

    adam()
    torch.cuda.synchronize()
    t = min(_time(adam, reps, s) for _ in range(rounds))
    bytes_ = n * 30
    out.append(dict(kernel="AdamW kernel (adamw_k)", bytes=int(bytes_), ms=round(t, 4),
                    gbs=round(bytes_ / (t * 1e-3) / 1e9, 1)))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="1b", choices=sorted(CONFIGS))
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--json", help="also write the rows to this file")
    ap.add_argument("--stream-only", action="store_true", help="only the streaming ceilings (no GEMM table)")
    args = ap.parse_args(argv)
    torch.cuda.set_device(0)
    blas = getattr(torch.backends.cuda, "preferred_blas_library", lambda: "unknown")()
    print(f"# {torch.cuda.get_device_name(0)}, torch {torch.__version__}, preferred BLAS {blas}; "
          f"config {args.config} {CONFIGS[args.config]}; best of {args.rounds} rounds of {args.reps} launches")
    rows = [] if args.stream_only else gemm_table(CONFIGS[args.config], args.reps, args.rounds)
    if rows:
        print_gemm(rows)
    st = stream_ceiling(args.reps, args.rounds)
    print("\n# HBM streaming ceiling (torch device kernels over 2 GiB fp32 buffers; algorithmic bytes)")
    for r in st:
        print(f"{r['kernel']:<26} {r['ms']:>8.3f} ms {r['gbs']:>8.1f} GB/s  ({r['gbs'] / 8000:.3f} of 8 TB/s)")
    pr = probe_ceiling(args.reps, args.rounds)
    print("\n# the library's streaming probe (aic_hip_stream_probe, 2 GiB per fp32 buffer; algorithmic bytes)")
    for r in pr:
        print(f"{r['kernel']:<42} {r['ms']:>8.3f} ms {r['gbs']:>8.1f} GB/s  ({r['gbs'] / 8000:.3f} of 8 TB/s)")
    if args.json:
        with open(args.json, "w") as fh:
            json.dump({"gemm": rows, "stream": st, "probe": pr}, fh)


def print_gemm(rows):
    print(f"{'product':<8} {'kind':<6} {'M':>6} {'N':>6} {'K':>6} {'ours_us':>8} {'TFLOP/s':>8} {'frac':>6} "
          f"{'lib_us':>8} {'TFLOP/s':>8} {'frac':>6} {'ours/lib':>8}")
    for r in rows:
        print(f"{r['product']:<8} {r['kind']:<6} {r['M']:>6} {r['N']:>6} {r['K']:>6} {r['ours_us']:>8.1f} "
              f"{r['ours_tflops']:>8.1f} {r['ours_frac']:>6.3f} {r['lib_us']:>8.1f} {r['lib_tflops']:>8.1f} "
              f"{r['lib_frac']:>6.3f} {r['lib_us'] / r['ours_us']:>8.3f}" + ("  (lib " + r["lib_out"] + ")"
                                                                         if r["kind"] == "wgrad" else ""))
    tot_o = sum(r["ours_us"] for r in rows)
    tot_l = sum(r["lib_us"] for r in rows)
    print(f"sum over the table: ours {tot_o / 1e3:.3f} ms, library {tot_l / 1e3:.3f} ms")


if __name__ == "__main__":
    main()
