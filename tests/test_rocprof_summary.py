"""The rocprofv3 summariser that bench.py's roofline traffic is read from: kernel symbols map to
the library's event classes (plain and grouped GEMM launches alike), scopes that span several
kernels count once, and FETCH_SIZE / WRITE_SIZE are scaled by the copy probe."""
import csv

from autonomousaicore_amd import rocprof_summary as rs

SYMS = {
    "_ZN3aic3hip12_GLOBAL__N_113gemm_bf16_dmaILi256ELi256ELi64ELi2ELb0ELb1EDF16bEEvNS1_10MfmaParamsE": "gemm_fwd",
    "_ZN3aic3hip12_GLOBAL__N_113gemm_bf16_dmaILi256ELi256ELi64ELi2ELb0ELb0EDF16bEEvNS1_10MfmaParamsE": "gemm_dgrad",
    "void aic::hip::(anonymous namespace)::gemm_bf16_dma<128, 128, 64, 4, true, false, float>(x)": "gemm_wgrad",
    "void aic::hip::(anonymous namespace)::gemm_bf16_dma_grouped<256, 256, 64, 2, true, false, float>(x)": "gemm_wgrad",
    "void aic::hip::(anonymous namespace)::gemm_bf16_dma_grouped<256, 256, 64, 2, false, true, float>(x)": "gemm_fwd",
    "_ZN3aic3hip12_GLOBAL__N_121gemm_bf16_dma_groupedILi256ELi256ELi64ELi2ELb0ELb0EDF16bEEvNS1_9DmaParamsE": "gemm_dgrad",
    "void aic::hip::(anonymous namespace)::gemm_bf16_dma_ragged<256, 256, 64, 2, true, false, float>(x)": "gemm_wgrad",
    "_ZN3aic3hip12_GLOBAL__N_120gemm_bf16_dma_raggedILi256ELi256ELi64ELi2ELb0ELb1EDF16bEEvNS1_12RaggedParamsE": "gemm_fwd",
    "void aic::hip::(anonymous namespace)::attn_bwd_dkdv_mfma<128>(x)": "attn_bwd",
    "_ZN3aic3hip12_GLOBAL__N_110attn_dot_kIDF16bEEvPKT_S5_lPfliii": "attn_bwd",
    "aic::hip::(anonymous namespace)::sqnorm_k(float const*, long, double*, int*)": "grad_norm",
    "void aic::hip::(anonymous namespace)::adamw_k<true>(float*)": "adamw",
    "aic::hip::(anonymous namespace)::splitk_reduce_k(x)": "gemm_splitk_reduce",
    "void aic::hip::(anonymous namespace)::gemm_bf16_dma_rag_tail<true>(x)": "gemm_fwd",
    "_ZN3aic3hip12_GLOBAL__N_122gemm_bf16_dma_rag_tailILb0EEEvNS1_12RaggedParamsEPfi": "gemm_dgrad",
    "_ZN3aic3hip12_GLOBAL__N_117rag_tail_reduce_kENS1_12RaggedParamsEPKfii": "gemm_splitk_reduce",
    "__amd_rocclr_copyBuffer": "other",
}


def test_kernel_classes():
    for name, cls in SYMS.items():
        assert rs.kernel_class(name) == cls, name


def test_scopes_and_traffic(tmp_path, capsys):
    stats = tmp_path / "stats.csv"
    with open(stats, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs"])
        w.writerow(["attn_bwd_dq_mfma<128>", 4, 4000.0])
        w.writerow(["attn_bwd_dkdv_mfma<128>", 4, 8000.0])
        w.writerow(["attn_dot_k<bf16>", 4, 1000.0])
    ctr = tmp_path / "fetch.csv"
    with open(ctr, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writerow(["__amd_rocclr_copyBuffer", "FETCH_SIZE", 2048.0])   # 1 MiB probe read twice over
        w.writerow(["attn_bwd_dq_mfma<128>", "FETCH_SIZE", 100.0])
        w.writerow(["attn_bwd_dkdv_mfma<128>", "FETCH_SIZE", 300.0])
        w.writerow(["attn_dot_k<bf16>", "FETCH_SIZE", 20.0])
    wr = tmp_path / "write.csv"
    with open(wr, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writerow(["__amd_rocclr_copyBuffer", "WRITE_SIZE", 1024.0])   # written once
        w.writerow(["attn_bwd_dq_mfma<128>", "WRITE_SIZE", 50.0])
        w.writerow(["attn_bwd_dkdv_mfma<128>", "WRITE_SIZE", 150.0])
        w.writerow(["attn_dot_k<bf16>", "WRITE_SIZE", 10.0])
    rs.main(["--stats", str(stats), "--fetch", str(ctr), "--write", str(wr), "--copy-probe-mib", "1", "--steps", "4"])
    out = capsys.readouterr().out
    row = [ln.split() for ln in out.splitlines() if ln.startswith("attn_bwd ")][0]
    assert row[1] == "4" and abs(float(row[3]) - 3.25) <= 0.051   # 13 us over 4 scopes
    # per scope: (100 + 300 + 20) KiB of fetches scaled by 1024 / 2048, and 210 KiB written
    tr = [ln.split() for ln in out.splitlines() if ln.startswith("traffic attn_bwd")][0]
    assert int(tr[2]) == 2 * 210 * 1024
