"""GPU parity of each HIP kernel, called through the C-ABI, against the CPU oracle (fp32
kernels) or the oracle / float64 on bf16-rounded inputs (bf16 kernels).  Tolerances are
stated per test: fp32 paths at reference precision, bf16 paths at the bf16 rounding level."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import bf16_round, call, dev, host, ptr, rel, stream  # noqa: E402

F32, BF16 = _lib.AIC_F32, _lib.AIC_BF16


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _gemm(ta, tb, M, N, K, A, B, ab, ct, R=None, alpha=1.0, beta=0.0, C0=None):
    lda = A.shape[1]
    ldb = B.shape[1]
    Cout = C0.clone() if C0 is not None else torch.empty((M, N), dtype=ct, device="cuda")
    call("aic_hip_gemm", ta, tb, M, N, K, alpha, ptr(A), lda, ptr(B), ldb, beta, ptr(Cout), N, ptr(R),
         N if R is not None else 0, ab, F32 if ct == torch.float32 else BF16, stream())
    return Cout


def _ref_gemm(ta, tb, A, B):
    a = A.astype(np.float64)
    b = B.astype(np.float64)
    return (a.T if ta else a) @ (b.T if tb else b)


# ----------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (512, 384, 320), (136, 200, 72), (4096, 4096, 128)])
def test_gemm_bf16_mfma(ta, tb, M, N, K):
    rng = np.random.default_rng(M + 7 * N + 13 * K + 2 * ta + tb)
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    ref = _ref_gemm(ta, tb, A, B)
    Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
    c32 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32)
    assert rel(host(c32), ref) < 1e-5  # fp32 accumulation of exact bf16 products
    c16 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.bfloat16)
    assert rel(host(c16), ref) < 4e-3  # one bf16 rounding of the result


def test_gemm_epilogue_residual_alpha_beta():
    rng = np.random.default_rng(3)
    M, N, K = 384, 256, 128
    A = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    R = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    ref = 0.5 * _ref_gemm(0, 1, A, B) + 2.0 * C0 + R
    out = _gemm(0, 1, M, N, K, dev(A, torch.bfloat16), dev(B, torch.bfloat16), BF16, torch.float32,
                R=dev(R), alpha=0.5, beta=2.0, C0=dev(C0))
    assert rel(host(out), ref) < 1e-5


# Weight-gradient shapes of the 1B step (o_proj, gate/up) over the full K = 8192, partial
# tiles with long K, each with residual / alpha / beta epilogues; runs must be bit-identical.
# Few-tile shapes (the LoRA adapter products: dB, dA, x A^T, dy B; 32-127 tiles of 256x256 over a
# long K) take the split-K paths; 136 tiles of 256x256 take the big-tile path.
LONG_K_CASES = [(1, 0, 2048, 2048, 8192), (1, 0, 11264, 2048, 8192), (0, 1, 600, 520, 8192),
                (0, 0, 1000, 1000, 4096), (1, 1, 264, 1032, 8192), (1, 0, 2048, 16, 8192), (1, 0, 48, 2048, 8192),
                (0, 1, 8192, 48, 2048), (0, 0, 4096, 16, 5632), (0, 1, 2048, 4352, 512), (1, 0, 1024, 2048, 4096)]


@pytest.mark.parametrize("ta,tb,M,N,K", LONG_K_CASES)
def test_gemm_long_k_and_epilogues(ta, tb, M, N, K):
    rng = np.random.default_rng(M + N + K + ta)
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    R = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    ref = _ref_gemm(ta, tb, A, B)
    Ad, Bd, Rd = dev(A, torch.bfloat16), dev(B, torch.bfloat16), dev(R)
    c1 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32)
    c2 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32)
    assert rel(host(c1), ref) < 1e-5
    np.testing.assert_array_equal(host(c1), host(c2))   # deterministic
    c16 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.bfloat16, R=dev(R, torch.bfloat16), alpha=0.5)
    assert rel(host(c16), 0.5 * ref + R) < 4e-3
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    cb = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32, R=Rd, alpha=0.25, beta=-1.5, C0=dev(C0))
    assert rel(host(cb), 0.25 * ref - 1.5 * C0 + R) < 1e-5


# Under one round of 256x256 tiles: one round of 128x256 tiles (the 125M / MoE 768- and 1024-wide
# products; partial tiles in both dimensions), and a long K split in two (128 tiles of 256x256,
# the 1024-wide head's input gradient).
WIDE_CASES = [(8192, 768, 768), (2048, 2048, 512), (3000, 1500, 192), (8192, 1024, 4096)]


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", WIDE_CASES)
def test_gemm_wide_tiles_and_split(ta, tb, M, N, K):
    """fp32 output against float64; bf16 output equal to the fp32 output rounded once (the same
    MFMA sequence per element); residual / alpha / beta epilogue; run-to-run bit-identical."""
    rng = np.random.default_rng(5 * M + N + K + 2 * ta + tb)
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    ref = _ref_gemm(ta, tb, A, B)
    Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
    c32 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32)
    assert rel(host(c32), ref) < 1e-5
    c16 = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.bfloat16)
    if K < 4096:  # no K split: one rounding of the same fp32 sum
        np.testing.assert_array_equal(host(c16), bf16_round(host(c32)))
    else:
        assert rel(host(c16), ref) < 4e-3
    R = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    cb = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32, R=dev(R), alpha=0.25, beta=-1.5, C0=dev(C0))
    assert rel(host(cb), 0.25 * ref - 1.5 * C0 + R) < 1e-5
    c16r = _gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.bfloat16, R=dev(R, torch.bfloat16), alpha=0.5)
    assert rel(host(c16r), 0.5 * ref + R) < 4e-3
    np.testing.assert_array_equal(host(_gemm(ta, tb, M, N, K, Ad, Bd, BF16, torch.float32)), host(c32))


def _gemm_lowrank(ta, tb, M, N, K, A, B, X2, Y2, r2, seg_n, y2k, ab, ct, R=None, alpha=1.0, beta=0.0, C0=None):
    Cout = C0.clone() if C0 is not None else torch.empty((M, N), dtype=ct, device="cuda")
    call("aic_hip_gemm_lowrank", ta, tb, M, N, K, alpha, ptr(A), A.shape[1], ptr(B), B.shape[1], ptr(X2),
         X2.shape[1], ptr(Y2), Y2.shape[1], r2, seg_n, y2k, beta, ptr(Cout), N, ptr(R), N if R is not None else 0,
         ab, F32 if ct == torch.float32 else BF16, stream())
    return Cout


# (ta, tb, M, N, K, r2, seg_n, y2_kmajor): LoRA forward (q/k/v or gate/up segments, single
# projections), LoRA input gradients (k-major A), a 256x256-tile launch, and shapes the kernel
# tail cannot take (segments not a multiple of the tile, rank not a multiple of 8)
LOWRANK_CASES = [(0, 1, 512, 768, 256, 16, 256, 0), (0, 1, 384, 256, 128, 16, 0, 0), (0, 0, 512, 256, 384, 48, 0, 1),
                 (0, 0, 300, 136, 192, 32, 0, 1), (0, 1, 4096, 6144, 256, 16, 2048, 0), (0, 1, 256, 384, 128, 16, 192, 0),
                 (0, 1, 256, 256, 128, 4, 0, 0), (0, 0, 256, 256, 128, 12, 0, 1)]


@pytest.mark.parametrize("ta,tb,M,N,K,r2,seg,y2k", LOWRANK_CASES)
def test_gemm_lowrank_term(ta, tb, M, N, K, r2, seg, y2k):
    rng = np.random.default_rng(M + N + K + r2 + seg)
    nseg = N // seg if seg else 1
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    X2 = bf16_round(rng.standard_normal((M, nseg * r2)).astype(np.float32))
    Y2 = bf16_round(rng.standard_normal((r2, N) if y2k else (N, r2)).astype(np.float32))
    R = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    ref = _ref_gemm(ta, tb, A, B)
    y = Y2.T.astype(np.float64) if y2k else Y2.astype(np.float64)  # [N, r2]
    nn = seg if seg else N
    for g in range(nseg):
        ref[:, g * nn:(g + 1) * nn] += X2[:, g * r2:(g + 1) * r2].astype(np.float64) @ y[g * nn:(g + 1) * nn].T
    Ad, Bd, X2d, Y2d = (dev(t, torch.bfloat16) for t in (A, B, X2, Y2))
    c32 = _gemm_lowrank(ta, tb, M, N, K, Ad, Bd, X2d, Y2d, r2, seg, y2k, BF16, torch.float32, R=dev(R), alpha=0.5)
    assert rel(host(c32), 0.5 * ref + R) < 1e-5
    c16 = _gemm_lowrank(ta, tb, M, N, K, Ad, Bd, X2d, Y2d, r2, seg, y2k, BF16, torch.bfloat16,
                        R=dev(R, torch.bfloat16))
    assert rel(host(c16), ref + R) < 4e-3
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    cb = _gemm_lowrank(ta, tb, M, N, K, Ad, Bd, X2d, Y2d, r2, seg, y2k, BF16, torch.float32, beta=-1.0, C0=dev(C0))
    assert rel(host(cb), ref - C0) < 1e-5
    # fp32 operands take the SIMT kernels for both terms
    f32 = _gemm_lowrank(ta, tb, M, N, K, dev(A), dev(B), dev(X2), dev(Y2), r2, seg, y2k, F32, torch.float32)
    assert rel(host(f32), ref) < 1e-5


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0)])
def test_gemm_fp32_matches_oracle(orc, ta, tb):
    rng = np.random.default_rng(10 + ta + 2 * tb)
    M, N, K = 96, 160, 136
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    ref = orc.gemm(np.ascontiguousarray(A.T) if ta else A, np.ascontiguousarray(B.T) if tb else B)
    out = _gemm(ta, tb, M, N, K, dev(A), dev(B), F32, torch.float32)
    assert rel(host(out), ref) < 1e-6


# ----------------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("rows,dim", [(64, 128), (257, 768), (33, 2048), (5, 100)])
def test_rmsnorm(orc, dt, rows, dim):
    rng = np.random.default_rng(rows * dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32) * 1.7
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    dy = rng.standard_normal((rows, dim)).astype(np.float32)
    dres = rng.standard_normal((rows, dim)).astype(np.float32)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    if dt == BF16:
        x, dy, dres = bf16_round(x), bf16_round(dy), bf16_round(dres)
    y_ref, rms_ref = orc.rmsnorm_fwd(x, w, 1e-6)
    dx_ref, dw_ref = orc.rmsnorm_bwd(dy, x, w, rms_ref)
    xd, wd = dev(x, tdt), dev(w)
    y = torch.empty_like(xd)
    rms = torch.empty(rows, dtype=torch.float32, device="cuda")
    call("aic_hip_rmsnorm_fwd", ptr(xd), dim, ptr(wd), ptr(y), dim, ptr(rms), rows, dim, 1e-6, dt, stream())
    tol = 1e-6 if dt == F32 else 4e-3
    assert rel(host(y), y_ref) < tol
    assert rel(host(rms), rms_ref) < 1e-6
    dyd, dresd = dev(dy, tdt), dev(dres, tdt)
    dx = torch.empty_like(xd)
    dw = torch.full((dim,), 7.0, dtype=torch.float32, device="cuda")
    call("aic_hip_rmsnorm_bwd", ptr(dyd), dim, ptr(xd), dim, ptr(wd), ptr(rms), ptr(dresd), dim, ptr(dx), dim,
         ptr(dw), 0, rows, dim, dt, stream())
    assert rel(host(dx), dx_ref + dres) < (1e-5 if dt == F32 else 4e-3)
    assert rel(host(dw), dw_ref) < 1e-5
    # accumulate = 1 adds to the existing weight gradient
    call("aic_hip_rmsnorm_bwd", ptr(dyd), dim, ptr(xd), dim, ptr(wd), ptr(rms), None, 0, ptr(dx), dim, ptr(dw), 1,
         rows, dim, dt, stream())
    assert rel(host(dw), 2 * dw_ref) < 1e-5
    assert rel(host(dx), dx_ref) < (1e-5 if dt == F32 else 4e-3)


# ----------------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("B,S,H,hd", [(2, 64, 4, 32), (1, 300, 3, 64), (2, 128, 2, 128)])
def test_rope_on_fused_qkv(orc, dt, B, S, H, hd):
    rng = np.random.default_rng(S + hd)
    d = H * hd
    qkv = rng.standard_normal((B * S, 3 * d)).astype(np.float32)
    if dt == BF16:
        qkv = bf16_round(qkv)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    cos, sin = orc.rope_tables(S + 5, hd)
    cosd, sind = dev(cos), dev(sin)  # keep both alive: a freed temporary's block is reused
    x = dev(qkv, tdt)
    call("aic_hip_rope", ptr(x), 3 * d, B, S, 2 * H, hd, 0, ptr(cosd), ptr(sind), 0, dt, stream())
    got = host(x)
    q_ref = orc.rope_fwd(qkv[:, :d], B, S, H, hd)
    k_ref = orc.rope_fwd(qkv[:, d:2 * d], B, S, H, hd)
    tol = 1e-6 if dt == F32 else 4e-3
    assert rel(got[:, :d], q_ref) < tol and rel(got[:, d:2 * d], k_ref) < tol
    np.testing.assert_array_equal(got[:, 2 * d:], qkv[:, 2 * d:])  # v untouched
    # inverse rotation restores the input
    call("aic_hip_rope", ptr(x), 3 * d, B, S, 2 * H, hd, 0, ptr(cosd), ptr(sind), 1, dt, stream())
    assert rel(host(x), qkv) < (1e-6 if dt == F32 else 8e-3)


# ----------------------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("dt", [F32, BF16])
def test_swiglu(orc, dt):
    rng = np.random.default_rng(21)
    T, f = 96, 352
    gu = (3 * rng.standard_normal((T, 2 * f))).astype(np.float32)
    dh = rng.standard_normal((T, f)).astype(np.float32)
    if dt == BF16:
        gu, dh = bf16_round(gu), bf16_round(dh)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    g, u = np.ascontiguousarray(gu[:, :f]), np.ascontiguousarray(gu[:, f:])
    gud, dhd = dev(gu, tdt), dev(dh, tdt)
    h = torch.empty((T, f), dtype=tdt, device="cuda")
    es = gud.element_size()
    call("aic_hip_swiglu_fwd", ptr(gud), ptr(gud) + es * f, 2 * f, ptr(h), f, T, f, dt, stream())
    tol = 1e-6 if dt == F32 else 4e-3
    assert rel(host(h), orc.swiglu_fwd(g, u)) < tol
    dgu = torch.empty_like(gud)
    call("aic_hip_swiglu_bwd", ptr(gud), ptr(gud) + es * f, 2 * f, ptr(dhd), f, ptr(dgu), ptr(dgu) + es * f, 2 * f,
         T, f, dt, stream())
    dg_ref, du_ref = orc.swiglu_bwd(g, u, dh)
    out = host(dgu)
    assert rel(out[:, :f], dg_ref) < tol * 2 and rel(out[:, f:], du_ref) < tol * 2


# ----------------------------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("N,Cn", [(64, 512), (37, 32000), (8, 77)])
def test_cross_entropy(orc, dt, N, Cn):
    rng = np.random.default_rng(N + Cn)
    z = (2 * rng.standard_normal((N, Cn))).astype(np.float32)
    t = rng.integers(0, Cn, N).astype(np.int64)
    t[::7] = -100
    if dt == BF16:
        z = bf16_round(z)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    loss_ref, losses_ref, lse_ref, valid_ref = orc.ce_fwd(z, t)
    zd, td = dev(z, tdt), dev(t)
    lse = torch.empty(N, dtype=torch.float32, device="cuda")
    losses = torch.empty(N, dtype=torch.float32, device="cuda")
    mean = torch.empty(1, dtype=torch.float32, device="cuda")
    valid = torch.empty(1, dtype=torch.int64, device="cuda")
    call("aic_hip_ce_fwd", ptr(zd), Cn, ptr(td), N, Cn, -100, ptr(losses), ptr(lse), ptr(mean), ptr(valid), dt,
         stream())
    assert int(host(valid)[0]) == valid_ref
    assert abs(float(host(mean)[0]) - loss_ref) < 1e-5 * abs(loss_ref)
    assert rel(host(lse), lse_ref) < 1e-6
    g = torch.tensor([3.0], dtype=torch.float32, device="cuda")
    d = torch.empty_like(zd)
    call("aic_hip_ce_bwd", ptr(zd), Cn, ptr(td), ptr(lse), N, Cn, -100, ptr(g), ptr(valid), ptr(d), Cn, dt, stream())
    d_ref = orc.ce_bwd(z, t, lse_ref, valid_ref, g=3.0)
    assert rel(host(d), d_ref) < (1e-5 if dt == F32 else 4e-3)
    assert np.all(host(d)[t == -100] == 0)
    # in place (dlogits aliases logits)
    call("aic_hip_ce_bwd", ptr(zd), Cn, ptr(td), ptr(lse), N, Cn, -100, ptr(g), ptr(valid), ptr(zd), Cn, dt,
         stream())
    assert rel(host(zd), d_ref) < (1e-5 if dt == F32 else 4e-3)


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("N,Cn", [(64, 512), (37, 32000), (8, 77), (5, 2056), (3, 65536), (2, 70000), (0, 64)])
def test_cross_entropy_fused(orc, dt, N, Cn):
    """aic_hip_ce_fwd_bwd: equal bit for bit to aic_hip_ce_fwd then aic_hip_ce_bwd in place (row
    widths that take each register-resident variant, one past their limit, odd widths and f32
    that run the two passes), and to the oracle within the bf16 bound; out-of-range targets are
    valid rows of loss lse - 0."""
    rng = np.random.default_rng(N * 7 + Cn)
    z = (3 * rng.standard_normal((N, Cn))).astype(np.float32)
    t = rng.integers(0, Cn, N).astype(np.int64)
    t[::5] = -100
    if N > 4:
        t[1] = Cn - 1  # the last column of the row
        t[2] = 0
    if dt == BF16:
        z = bf16_round(z)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    g = torch.tensor([2.5], dtype=torch.float32, device="cuda")

    def outs():
        return (torch.empty(max(N, 1), dtype=torch.float32, device="cuda"),
                torch.empty(max(N, 1), dtype=torch.float32, device="cuda"),
                torch.empty(1, dtype=torch.float32, device="cuda"), torch.empty(1, dtype=torch.int64, device="cuda"))

    zf, td = dev(z, tdt), dev(t)
    lf, sf, mf, vf = outs()
    call("aic_hip_ce_fwd_bwd", ptr(zf), Cn, ptr(td), N, Cn, -100, ptr(lf), ptr(sf), ptr(mf), ptr(vf), ptr(g), dt,
         stream())
    z2 = dev(z, tdt)
    l2, s2, m2, v2 = outs()
    call("aic_hip_ce_fwd", ptr(z2), Cn, ptr(td), N, Cn, -100, ptr(l2), ptr(s2), ptr(m2), ptr(v2), dt, stream())
    if N:
        call("aic_hip_ce_bwd", ptr(z2), Cn, ptr(td), ptr(s2), N, Cn, -100, ptr(g), ptr(v2), ptr(z2), Cn, dt,
             stream())
    assert int(host(vf)[0]) == int(host(v2)[0])
    np.testing.assert_array_equal(host(mf), host(m2))
    if N:
        np.testing.assert_array_equal(host(lf)[:N], host(l2)[:N])
        np.testing.assert_array_equal(host(sf)[:N], host(s2)[:N])
        np.testing.assert_array_equal(host(zf), host(z2))
        loss_ref, _, lse_ref, valid_ref = orc.ce_fwd(z, t)
        assert int(host(vf)[0]) == valid_ref
        assert abs(float(host(mf)[0]) - loss_ref) < 1e-5 * abs(loss_ref)
        assert rel(host(sf)[:N], lse_ref) < 1e-6
        assert rel(host(zf), orc.ce_bwd(z, t, lse_ref, valid_ref, g=2.5)) < (1e-5 if dt == F32 else 4e-3)
        assert np.all(host(zf)[t == -100] == 0)
    else:
        assert int(host(vf)[0]) == 0 and float(host(mf)[0]) == 0.0
    # without losses / lse outputs and without grad (a unit gradient)
    if N:
        z3 = dev(z, tdt)
        call("aic_hip_ce_fwd_bwd", ptr(z3), Cn, ptr(td), N, Cn, -100, None, None, ptr(mf), ptr(vf), None, dt,
             stream())
        assert rel(host(z3), orc.ce_bwd(z, t, lse_ref, valid_ref, g=1.0)) < (1e-5 if dt == F32 else 4e-3)
    # a target outside [0, C) is a valid row of loss lse - 0 whose gradient is the softmax (no -1
    # term), as the reference's CUDA launcher computes it (cuda_loss.cu:114-121, 170-176)
    if N > 4:
        tb = t.copy()
        tb[3], tb[4] = Cn + 5, -3
        z4 = dev(z, tdt)
        s4 = torch.empty(N, dtype=torch.float32, device="cuda")
        call("aic_hip_ce_fwd_bwd", ptr(z4), Cn, ptr(dev(tb)), N, Cn, -100, ptr(lf), ptr(s4), ptr(mf), ptr(vf), ptr(g),
             dt, stream())
        lo, s4h = host(lf)[:N], host(s4)
        np.testing.assert_array_equal(lo[[3, 4]], s4h[[3, 4]])
        assert int(host(vf)[0]) == valid_ref + (t[3] == -100) + (t[4] == -100)
        inr = np.where((tb >= 0) & (tb < Cn), tb, 0)
        losses_ref = orc.ce_fwd(z, inr)[1]
        keep = (tb != -100) & (tb >= 0) & (tb < Cn)
        assert rel(lo[keep], losses_ref[keep]) < 1e-6
        valid4 = int(host(vf)[0])
        soft = np.exp(z[[3, 4]].astype(np.float64) - lse_ref[[3, 4], None]) * 2.5 / valid4
        assert rel(host(z4)[[3, 4]], soft) < (1e-5 if dt == F32 else 4e-3)


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_cross_entropy_reductions(orc, dt, reduction):
    """aic_hip_ce_bwd_rows: the launcher-level backward with the reference's reduction string and
    host valid_count (cuda_loss.cuh:35-52), against orc_ce_bwd_reduction; with and without an
    incoming gradient; an all-ignored batch ("mean" with valid_count 0) gives zeros."""
    N, Cn = 300, 1000
    rng = np.random.default_rng(N + Cn + len(reduction))
    z = (2 * rng.standard_normal((N, Cn))).astype(np.float32)
    t = rng.integers(0, Cn, N).astype(np.int64)
    t[::5] = -100
    if dt == BF16:
        z = bf16_round(z)
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    _, _, lse_ref, valid_ref = orc.ce_fwd(z, t)
    zd, td, lsed = dev(z, tdt), dev(t), dev(lse_ref)
    g = rng.standard_normal(N).astype(np.float32) if reduction == "none" else np.float32([0.75])
    tol = 1e-5 if dt == F32 else 4e-3
    per_row = 1 if reduction == "none" else 0
    divisor = float(valid_ref) if reduction == "mean" else 1.0
    for gg in (g, None):
        d = torch.empty_like(zd)
        gd = dev(gg) if gg is not None else None
        call("aic_hip_ce_bwd_rows", ptr(zd), Cn, ptr(td), ptr(lsed), N, Cn, -100, ptr(gd), per_row, divisor, ptr(d),
             Cn, dt, stream())
        ref = orc.ce_bwd_reduction(z, t, lse_ref, valid_ref, reduction, gg)
        assert rel(host(d), ref) < tol
        assert np.all(host(d)[t == -100] == 0)
    if reduction == "mean":
        ti = np.full(N, -100, np.int64)
        d = torch.full_like(zd, 7.0)
        call("aic_hip_ce_bwd_rows", ptr(zd), Cn, ptr(dev(ti)), ptr(lsed), N, Cn, -100, None, 0, 0.0, ptr(d), Cn, dt,
             stream())
        assert not host(d).any()


# ----------------------------------------------------------------------------- embedding
@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("V,D,N", [(1000, 136, 4096), (1500, 1024, 8192), (32000, 2048, 2048), (32000, 1024, 40000),
                                   (32000, 768, 8192), (1000, 320, 4096)])
def test_embedding_gather_bit_exact_and_scatter(orc, dt, V, D, N):
    # D = 136: the per-column path; D * element size a multiple of 256 bytes: the run-list path
    # with 16-, 8- or 4-byte loads per lane (the 1B and 125M shapes among them), Zipf ids so one
    # id repeats hundreds of times; 40000 tokens: twenty sorted chunks of 2048 merged, the last
    # one partial
    rng = np.random.default_rng(31 + D)
    W = rng.standard_normal((V, D)).astype(np.float32)
    if dt == BF16:
        W = bf16_round(W)
    ids = np.minimum(rng.zipf(1.1, N) - 1, V - 1).astype(np.int64)
    ids[5] = -1
    ids[9] = V  # out of range: zero row, no gradient
    tdt = torch.float32 if dt == F32 else torch.bfloat16
    Wd, idd = dev(W, tdt), dev(ids)
    out = torch.empty((N, D), dtype=tdt, device="cuda")
    call("aic_hip_embed_fwd", ptr(idd), N, ptr(Wd), V, D, ptr(out), dt, stream())
    np.testing.assert_array_equal(host(out), orc.embedding_fwd(ids, W))  # bit-exact gather
    dout = rng.standard_normal((N, D)).astype(np.float32)
    if dt == BF16:
        dout = bf16_round(dout)
    dd = dev(dout, tdt)
    dW = torch.full((V, D), 5.0, dtype=torch.float32, device="cuda")
    call("aic_hip_embed_bwd", ptr(idd), N, ptr(dd), V, D, ptr(dW), 0, dt, stream())
    ref = orc.embedding_bwd(ids, dout, V)
    got = host(dW)
    # The kernels add a run of n equal ids as P interleaved float32 chains (P = 16 waves on the
    # run-list path, 4 on the per-column path) combined in order, or, on the run-list path for
    # n <= 16, as one chain in token order: a float32 sum of depth at most ceil(n / P) + P, so
    # |got - exact| <= depth * 2^-24 * sum |dout| per element, where a dropped or doubled row of
    # N(0, 1) gradients would exceed it.
    ok = (ids >= 0) & (ids < V)
    exact = np.zeros((V, D))
    np.add.at(exact, ids[ok], dout[ok].astype(np.float64))
    mag = np.zeros((V, D))
    np.add.at(mag, ids[ok], np.abs(dout[ok].astype(np.float64)))
    run_list = (D * (4 if dt == F32 else 2)) % 256 == 0
    P = 16 if run_list else 4
    n = np.bincount(ids[ok], minlength=V)[:, None]
    bound = (np.ceil(n / P) + P) * 2.0 ** -24 * mag
    assert np.all(np.abs(got - exact) <= bound)
    if run_list:  # a short run is the reference's own token-order float32 sum, bit for bit
        short = (n[:, 0] > 0) & (n[:, 0] <= 16)
        assert short.any()
        np.testing.assert_array_equal(got[short], ref[short])
    # and the oracle (the reference's token-order float32 sum, depth n) within its own bound
    assert np.all(np.abs(ref - exact) <= n * 2.0 ** -24 * mag)
    assert np.all(got[np.setdiff1d(np.arange(V), ids)] == 0)
    # deterministic: a second run is bit-identical
    dW2 = torch.zeros_like(dW)
    call("aic_hip_embed_bwd", ptr(idd), N, ptr(dd), V, D, ptr(dW2), 0, dt, stream())
    np.testing.assert_array_equal(host(dW2), got)
    # accumulate adds to what is there
    call("aic_hip_embed_bwd", ptr(idd), N, ptr(dd), V, D, ptr(dW2), 1, dt, stream())
    acc = host(dW2)
    assert np.all(np.abs(acc - 2 * exact) <= 2 * bound + 2.0 ** -24 * np.abs(acc))


@pytest.mark.parametrize("dt", [F32, BF16])
def test_embedding_bwd_no_tokens(dt):
    """N = 0: overwrite leaves every row zero (all ids absent), accumulate leaves dW as it was."""
    V, D = 1000, 136
    dW = torch.full((V, D), 5.0, dtype=torch.float32, device="cuda")
    call("aic_hip_embed_bwd", None, 0, None, V, D, ptr(dW), 1, dt, stream())
    assert np.all(host(dW) == 5.0)
    call("aic_hip_embed_bwd", None, 0, None, V, D, ptr(dW), 0, dt, stream())
    assert not host(dW).any()


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("B,S,H,hd,causal", [(2, 64, 4, 32, 1), (1, 100, 2, 64, 1), (1, 128, 2, 16, 1),
                                               (1, 96, 2, 128, 1), (2, 100, 2, 64, 0), (1, 77, 3, 128, 0)])
def test_attention_fp32_matches_oracle(orc, B, S, H, hd, causal):
    """causal = 0 is the reference launcher's is_causal = false (cuda_flash_attention.cuh:12-46)."""
    rng = np.random.default_rng(S * hd)
    d = H * hd
    qkv = rng.standard_normal((B * S, 3 * d)).astype(np.float32)
    q, k, v = (np.ascontiguousarray(qkv[:, i * d:(i + 1) * d]) for i in range(3))
    do = rng.standard_normal((B * S, d)).astype(np.float32)
    o_ref, E, rs = orc.attention_fwd(q, k, v, B, S, H, hd, causal=bool(causal))
    dq_ref, dk_ref, dv_ref = orc.attention_bwd(q, k, v, E, rs, do, B, S, H, hd)
    x = dev(qkv)
    o = torch.empty((B * S, d), dtype=torch.float32, device="cuda")
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    sc = 1.0 / np.sqrt(hd)
    call("aic_hip_attn_fwd", ptr(x), ptr(x) + 4 * d, ptr(x) + 8 * d, 3 * d, ptr(o), d, ptr(lse), B, H, S, hd, causal,
         sc, F32, stream())
    assert rel(host(o), o_ref) < 1e-5
    dqkv = torch.empty_like(x)
    dod = dev(do)
    call("aic_hip_attn_bwd", ptr(x), ptr(x) + 4 * d, ptr(x) + 8 * d, 3 * d, ptr(o), ptr(dod), d, ptr(lse),
         ptr(dqkv), ptr(dqkv) + 4 * d, ptr(dqkv) + 8 * d, 3 * d, B, H, S, hd, causal, sc, F32, stream())
    g = host(dqkv)
    assert rel(g[:, :d], dq_ref) < 1e-4
    assert rel(g[:, d:2 * d], dk_ref) < 1e-4
    assert rel(g[:, 2 * d:], dv_ref) < 1e-4


# (1, 2048, 2, 128): the 1B configuration's sequence and head width; causal = 0 with S not a
# multiple of the 128-row tiles
@pytest.mark.parametrize("B,S,H,hd,causal", [(1, 256, 2, 128, 1), (2, 192, 3, 64, 1), (1, 1024, 2, 128, 1),
                                               (1, 72, 1, 64, 1), (1, 2048, 2, 128, 1), (2, 200, 2, 128, 0),
                                               (1, 333, 2, 64, 0)])
def test_attention_bf16_mfma(orc, B, S, H, hd, causal):
    rng = np.random.default_rng(S + hd + H)
    d = H * hd
    qkv = bf16_round(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
    do = bf16_round(rng.standard_normal((B * S, d)).astype(np.float32))
    q, k, v = (np.ascontiguousarray(qkv[:, i * d:(i + 1) * d]) for i in range(3))
    o_ref, E, rs = orc.attention_fwd(q, k, v, B, S, H, hd, causal=bool(causal))
    dq_ref, dk_ref, dv_ref = orc.attention_bwd(q, k, v, E, rs, do, B, S, H, hd)
    x = dev(qkv, torch.bfloat16)
    o = torch.empty((B * S, d), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    sc = 1.0 / np.sqrt(hd)
    call("aic_hip_attn_fwd", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), d, ptr(lse), B, H, S, hd, causal,
         sc, BF16, stream())
    # bf16 P and a bf16 output: errors at the bf16 rounding level
    assert rel(host(o), o_ref) < 1e-2
    dqkv = torch.empty_like(x)
    dod = dev(do, torch.bfloat16)
    call("aic_hip_attn_bwd", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), ptr(dod), d,
         ptr(lse), ptr(dqkv), ptr(dqkv) + 2 * d, ptr(dqkv) + 4 * d, 3 * d, B, H, S, hd, causal, sc, BF16, stream())
    g = host(dqkv)
    assert rel(g[:, :d], dq_ref) < 2e-2
    assert rel(g[:, d:2 * d], dk_ref) < 2e-2
    assert rel(g[:, 2 * d:], dv_ref) < 2e-2
    # deterministic backward
    dqkv2 = torch.empty_like(x)
    call("aic_hip_attn_bwd", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), ptr(dod), d,
         ptr(lse), ptr(dqkv2), ptr(dqkv2) + 2 * d, ptr(dqkv2) + 4 * d, 3 * d, B, H, S, hd, causal, sc, BF16, stream())
    np.testing.assert_array_equal(host(dqkv2), g)


# (M, f, K): 32 x 22 = 704 paired tiles (the 1B shape's f over fewer rows) and 256 take the GEMM's
# SwiGLU epilogue; fewer tiles or f not a multiple of 128 run the product and then swiglu_fwd
@pytest.mark.parametrize("M,f,K", [(8192, 5632, 128), (4096, 2048, 256), (1024, 1024, 128), (4096, 1088, 128),
                                   (300, 512, 64)])
def test_gemm_swiglu_epilogue(orc, M, f, K):
    """aic_hip_gemm_swiglu = aic_hip_gemm (x W^T over the gate and up rows) then
    aic_hip_swiglu_fwd: both outputs bit-identical (the same bf16 product, the same activation
    arithmetic), and against the oracle's SwiGLU of the float64 product within the bf16 bound."""
    rng = np.random.default_rng(M + f + K)
    A = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    W = bf16_round((rng.standard_normal((2 * f, K)) / np.sqrt(K)).astype(np.float32))
    Ad, Wd = dev(A, torch.bfloat16), dev(W, torch.bfloat16)
    gu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((M, f), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_swiglu", M, f, K, ptr(Ad), K, ptr(Wd), K, ptr(gu), 2 * f, ptr(h), f, stream())
    gu2 = _gemm(0, 1, M, 2 * f, K, Ad, Wd, BF16, torch.bfloat16)
    h2 = torch.empty_like(h)
    call("aic_hip_swiglu_fwd", ptr(gu2), ptr(gu2) + 2 * f, 2 * f, ptr(h2), f, M, f, BF16, stream())
    np.testing.assert_array_equal(host(gu), host(gu2))
    np.testing.assert_array_equal(host(h), host(h2))
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    assert rel(host(h), orc.swiglu_fwd(ref[:, :f], ref[:, f:])) < 1e-2


# (M, f, K): 32 x 22 = 704 tiles (the 1B down projection's input gradient) and 256 take the GEMM's
# SwiGLU-backward epilogue; fewer tiles or f not a multiple of 256 go through dh and swiglu_bwd
@pytest.mark.parametrize("M,f,K", [(8192, 5632, 256), (4096, 2048, 128), (1024, 1024, 128), (4096, 1152, 128),
                                   (300, 512, 64)])
def test_gemm_swiglu_bwd_epilogue(orc, M, f, K):
    """aic_hip_gemm_swiglu_bwd = aic_hip_gemm (dh = dy W) then aic_hip_swiglu_bwd: the gate/up
    gradients bit-identical, and against the oracle's SwiGLU backward of the float64 product
    within the bf16 bound."""
    rng = np.random.default_rng(M + f + K + 1)
    A = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    Bm = bf16_round((rng.standard_normal((K, f)) / np.sqrt(K)).astype(np.float32))
    GU = bf16_round(rng.standard_normal((M, 2 * f)).astype(np.float32))
    Ad, Bd, GUd = dev(A, torch.bfloat16), dev(Bm, torch.bfloat16), dev(GU, torch.bfloat16)
    dh = torch.empty((M, f), dtype=torch.bfloat16, device="cuda")
    dgu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_swiglu_bwd", M, f, K, ptr(Ad), K, ptr(Bd), f, ptr(GUd), 2 * f, ptr(dh), f, ptr(dgu), stream())
    dh2 = _gemm(0, 0, M, f, K, Ad, Bd, BF16, torch.bfloat16)
    dgu2 = torch.empty_like(dgu)
    call("aic_hip_swiglu_bwd", ptr(GUd), ptr(GUd) + 2 * f, 2 * f, ptr(dh2), f, ptr(dgu2), ptr(dgu2) + 2 * f, 2 * f,
         M, f, BF16, stream())
    np.testing.assert_array_equal(host(dgu), host(dgu2))
    ref = A.astype(np.float64) @ Bm.astype(np.float64)
    dg_ref, du_ref = orc.swiglu_bwd(GU[:, :f], GU[:, f:], ref)
    got = host(dgu)
    assert rel(got[:, :f], dg_ref) < 1e-2 and rel(got[:, f:], du_ref) < 1e-2


# (T, d, K, hd, seq, start): 192 tiles of 256x256 with heads of 128 or 64 take the GEMM's rotary
# epilogue, also at a start position past 0 (tables of start + seq rows); fewer tiles or a ragged
# M run the product and then the rope pass
@pytest.mark.parametrize("T,d,K,hd,seq,start", [(4096, 1024, 256, 128, 2048, 0), (4096, 1024, 256, 128, 1024, 0),
                                                 (1024, 512, 128, 128, 512, 0), (4096, 1024, 256, 64, 2048, 0),
                                                 (4096, 1024, 256, 128, 2048, 5), (300, 512, 128, 128, 100, 7)])
def test_gemm_rope_epilogue(orc, T, d, K, hd, seq, start):
    """aic_hip_gemm_rope = aic_hip_gemm (x W^T over the q, k, v columns) then aic_hip_rope on the
    q and k columns: v columns bit-identical, q / k within one bf16 rounding of the rotation of
    the same bf16 product (the same arithmetic; operation fusing may differ in the last bit), and
    the oracle's RoPE of the float64 product within the bf16 bound."""
    rng = np.random.default_rng(T + d + hd + start)
    N = 3 * d
    A = bf16_round(rng.standard_normal((T, K)).astype(np.float32))
    W = bf16_round((rng.standard_normal((N, K)) / 8).astype(np.float32))
    cos_t = np.empty((start + seq, hd // 2), np.float32)
    sin_t = np.empty_like(cos_t)
    _lib.check(_lib.load().aic_hip_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, start + seq, hd, 10000.0))
    Ad, Wd, cd, sd = dev(A, torch.bfloat16), dev(W, torch.bfloat16), dev(cos_t), dev(sin_t)
    fused = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_rope", T, N, K, ptr(Ad), K, ptr(Wd), K, ptr(fused), N, 2 * d, hd, seq, start, ptr(cd), ptr(sd),
         stream())
    sep = _gemm(0, 1, T, N, K, Ad, Wd, BF16, torch.bfloat16)
    call("aic_hip_rope", ptr(sep), N, T // seq, seq, 2 * d // hd, hd, start, ptr(cd), ptr(sd), 0, BF16, stream())
    f, g = host(fused), host(sep)
    np.testing.assert_array_equal(f[:, 2 * d:], g[:, 2 * d:])
    assert np.max(np.abs(f[:, :2 * d] - g[:, :2 * d]) / (np.abs(g[:, :2 * d]) + 1e-3)) < 1e-2
    assert rel(f[:, :2 * d], g[:, :2 * d]) < 2e-3
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    qk = orc.rope_fwd(ref[:, :2 * d], T // seq, seq, 2 * d // hd, hd, start_pos=start)
    assert rel(f[:, :2 * d], qk) < 8e-3
    # deterministic
    again = torch.empty_like(fused)
    call("aic_hip_gemm_rope", T, N, K, ptr(Ad), K, ptr(Wd), K, ptr(again), N, 2 * d, hd, seq, start, ptr(cd), ptr(sd),
         stream())
    np.testing.assert_array_equal(host(again), f)


@pytest.mark.parametrize("B,S,H,hd,causal", [(2, 256, 2, 128, 1), (1, 200, 3, 64, 1), (2, 130, 2, 128, 0),
                                               (1, 72, 1, 64, 0)])
def test_attention_bwd_with_rope(orc, B, S, H, hd, causal):
    """aic_hip_attn_bwd_rope = aic_hip_attn_bwd then the rotary embedding's inverse (RoPEBackward)
    on dq and dk: dv bit-identical, dq / dk within one bf16 rounding (the fused form rotates the
    fp32 accumulator instead of its bf16 copy), and both against the oracle's attention backward
    followed by its RoPE backward."""
    rng = np.random.default_rng(S + 3 * hd + H + causal)
    d = H * hd
    qkv = bf16_round(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
    do = bf16_round(rng.standard_normal((B * S, d)).astype(np.float32))
    cos_t = np.empty((S, hd // 2), np.float32)
    sin_t = np.empty_like(cos_t)
    _lib.check(_lib.load().aic_hip_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, S, hd, 10000.0))
    cd, sd = dev(cos_t), dev(sin_t)
    x = dev(qkv, torch.bfloat16)
    o = torch.empty((B * S, d), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    sc = 1.0 / np.sqrt(hd)
    call("aic_hip_attn_fwd", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), d, ptr(lse), B, H, S, hd, causal,
         sc, BF16, stream())
    dod = dev(do, torch.bfloat16)
    sep = torch.empty_like(x)
    call("aic_hip_attn_bwd", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), ptr(dod), d,
         ptr(lse), ptr(sep), ptr(sep) + 2 * d, ptr(sep) + 4 * d, 3 * d, B, H, S, hd, causal, sc, BF16, stream())
    call("aic_hip_rope", ptr(sep), 3 * d, B, S, 2 * H, hd, 0, ptr(cd), ptr(sd), 1, BF16, stream())
    fused = torch.empty_like(x)
    call("aic_hip_attn_bwd_rope", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), ptr(dod), d,
         ptr(lse), ptr(fused), ptr(fused) + 2 * d, ptr(fused) + 4 * d, 3 * d, B, H, S, hd, causal, sc,
         ptr(cd), ptr(sd), BF16, stream())
    f, g = host(fused), host(sep)
    np.testing.assert_array_equal(f[:, 2 * d:], g[:, 2 * d:])
    assert rel(f[:, :2 * d], g[:, :2 * d]) < 4e-3
    q, k, v = (np.ascontiguousarray(qkv[:, i * d:(i + 1) * d]) for i in range(3))
    _, E, rs = orc.attention_fwd(q, k, v, B, S, H, hd, causal=bool(causal))
    dq_ref, dk_ref, _ = orc.attention_bwd(q, k, v, E, rs, do, B, S, H, hd)
    # the oracle's RoPE backward of the oracle's attention gradients
    assert rel(f[:, :d], orc.rope_bwd(dq_ref, B, S, H, hd)) < 2e-2
    assert rel(f[:, d:2 * d], orc.rope_bwd(dk_ref, B, S, H, hd)) < 2e-2
    # deterministic
    again = torch.empty_like(x)
    call("aic_hip_attn_bwd_rope", ptr(x), ptr(x) + 2 * d, ptr(x) + 4 * d, 3 * d, ptr(o), ptr(dod), d,
         ptr(lse), ptr(again), ptr(again) + 2 * d, ptr(again) + 4 * d, 3 * d, B, H, S, hd, causal, sc,
         ptr(cd), ptr(sd), BF16, stream())
    np.testing.assert_array_equal(host(again), f)


# ----------------------------------------------------------------------------- optimizer tail
def test_grad_sqnorm_and_nonfinite():
    rng = np.random.default_rng(41)
    a = rng.standard_normal(1_000_003).astype(np.float32)
    b = rng.standard_normal(77).astype(np.float32)
    ad, bd = dev(a), dev(b)
    sq = torch.empty(1, dtype=torch.float64, device="cuda")
    nf = torch.empty(1, dtype=torch.int32, device="cuda")
    import ctypes as C
    ptrs = (C.c_void_p * 2)(ptr(ad), ptr(bd))
    sizes = (C.c_int64 * 2)(a.size, b.size)
    call("aic_hip_grad_sqnorm_multi", ptrs, sizes, 2, ptr(sq), ptr(nf), stream())
    ref = float((a.astype(np.float64) ** 2).sum() + (b.astype(np.float64) ** 2).sum())
    assert abs(float(host(sq)[0]) - ref) < 1e-9 * ref and int(host(nf)[0]) == 0
    bd[13] = float("inf")
    call("aic_hip_grad_sqnorm_multi", ptrs, sizes, 2, ptr(sq), ptr(nf), stream())
    assert int(host(nf)[0]) == 1


def test_adamw_matches_oracle(orc):
    import ctypes as C
    rng = np.random.default_rng(42)
    n = 100_001
    p = rng.standard_normal(n).astype(np.float32)
    pm, m, v = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    pd, md, vd = dev(p), dev(np.zeros(n, np.float32)), dev(np.zeros(n, np.float32))
    low = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    for step in (1, 2, 3):
        g = rng.standard_normal(n).astype(np.float32)
        orc.adamw(pm, g, m, v, 3e-4, 0.9, 0.95, 1e-8, 0.1, step)
        gd = dev(g)
        args = [(C.c_void_p * 1)(ptr(t)) for t in (pd, gd, md, vd, low)]
        call("aic_hip_adamw_multi", *args, (C.c_int64 * 1)(n), 1, 3e-4, 0.9, 0.95, 1e-8, 0.1, step, None, stream())
    assert np.max(np.abs(host(pd) - pm)) < 1e-6
    assert rel(host(md), m) < 1e-6 and rel(host(vd), v) < 1e-6
    np.testing.assert_array_equal(host(low), bf16_round(host(pd)))


def test_adamw_step_with_caller_bias_corrections(orc):
    # the reference's cuda_adamw_step contract: bias corrections computed by the caller
    rng = np.random.default_rng(43)
    n = 50_003
    p = rng.standard_normal(n).astype(np.float32)
    pm, m, v = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    pd, md, vd = dev(p), dev(np.zeros(n, np.float32)), dev(np.zeros(n, np.float32))
    for step in (1, 2, 3, 10):
        g = rng.standard_normal(n).astype(np.float32)
        orc.adamw(pm, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, step)
        gd = dev(g)
        bc1 = float(np.float32(1) - np.float32(0.9) ** np.float32(step))
        bc2 = float(np.float32(1) - np.float32(0.999) ** np.float32(step))
        call("aic_hip_adamw_step", ptr(pd), ptr(gd), ptr(md), ptr(vd), n, 1e-3, 0.9, 0.999, 1e-8, 0.01, bc1, bc2,
             stream())
    assert np.max(np.abs(host(pd) - pm)) < 1e-6
    assert rel(host(md), m) < 1e-6 and rel(host(vd), v) < 1e-5
    # a zero bias correction is an argument error, not a division by zero
    assert _lib.load().aic_hip_adamw_step(ptr(pd), ptr(gd), ptr(md), ptr(vd), n, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.0,
                                          bc2, stream()) != 0


def _ctl(**kw):
    c = _lib.OptimCtl()
    c.scale, c.use_scaler, c.growth_factor, c.backoff_factor = 1024.0, 1, 2.0, 0.5
    c.growth_interval, c.min_scale, c.max_scale, c.max_grad_norm = 1000, 1.0, 16777216.0, 0.0
    for k, val in kw.items():
        setattr(c, k, val)
    return c


def _finalize(c, sq, nf):
    import ctypes as C
    buf = torch.tensor(np.frombuffer(bytes(c), np.uint8).copy(), device="cuda")
    sqd = torch.tensor([sq], dtype=torch.float64, device="cuda")
    nfd = torch.tensor([nf], dtype=torch.int32, device="cuda")
    call("aic_hip_optim_finalize", ptr(sqd), ptr(nfd), ptr(buf), stream())
    out = _lib.OptimCtl()
    C.memmove(C.addressof(out), host(buf).astype(np.uint8).tobytes(), C.sizeof(out))
    return out


def test_optim_finalize_scaler_and_clip_semantics(orc):
    # backoff on non-finite (tests/unit/test_amp.cpp:86-116)
    c = _finalize(_ctl(), 1.0, 1)
    assert c.skip == 1 and c.scale == 512.0 and c.skipped_steps == 1 and c.step == 0
    # growth after growth_interval good steps (tests/unit/test_amp.cpp:118-142)
    c = _ctl(scale=128.0, growth_interval=3, max_scale=1024.0)
    seen = []
    for _ in range(6):
        c = _finalize(c, 4.0, 0)
        seen.append(c.scale)
    assert seen == [128, 128, 256, 256, 256, 512] and c.step == 6
    # clip: unscaled norm sqrt(91) -> coefficient 5/sqrt(91) (tests/unit/test_optim.cpp:191-207)
    scale = 4.0
    c = _finalize(_ctl(scale=scale, max_grad_norm=5.0), 91.0 * scale * scale, 0)
    assert abs(c.grad_norm - np.sqrt(91)) < 1e-4
    assert abs(c.grad_mult - (5.0 / (np.sqrt(91) + 1e-6)) / scale) < 1e-7
    # below the threshold only the unscale remains
    c = _finalize(_ctl(scale=scale, max_grad_norm=100.0), 91.0 * scale * scale, 0)
    assert c.grad_mult == 1.0 / scale


# (ta, tb, [(M, N, K), ...]): MoE experts of different row counts, the q/k/v + out_proj weight
# gradients together, a 128x128-tile group, and a mixed set that falls back to single launches
GROUPED_CASES = [(0, 1, [(192, 704, 256), (64, 704, 256), (448, 704, 256), (128, 704, 256)]),
                 (1, 0, [(768, 256, 1024), (256, 256, 1024)]),
                 (0, 0, [(64, 256, 128), (128, 128, 256), (256, 192, 64)]),
                 (1, 0, [(1536, 512, 2048), (512, 512, 2048)]),
                 (1, 0, [(4096, 2048, 512), (2048, 2048, 512)]),
                 # 272 and 264 tiles of 256x256: the tiles past one round leave the launch as their
                 # own GEMM (two tile-columns of the third product, one of them partial; the last
                 # tile-row of the third product with A row-major)
                 (1, 0, [(2048, 2048, 512), (4096, 2048, 512), (2048, 1800, 512), (2048, 512, 512)]),
                 (0, 0, [(4096, 2048, 256), (2048, 2048, 256), (2304, 2048, 256)]),
                 # the 125M layer's four weight gradients (K shortened): 108 tiles of 256x256, 432 of
                 # 128x128, one round of 216 tiles of 128x256
                 (1, 0, [(2304, 768, 2048), (768, 768, 2048), (4096, 768, 2048), (768, 2048, 2048)])]


@pytest.mark.parametrize("ta,tb,shapes", GROUPED_CASES)
def test_gemm_grouped(ta, tb, shapes):
    rng = np.random.default_rng(len(shapes) + ta)
    descs, refs, outs, keep = [], [], [], []
    for M, N, K in shapes:
        A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
        B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
        Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
        Cd = torch.zeros((M, N), dtype=torch.float32, device="cuda")
        keep += [Ad, Bd]
        outs.append(Cd)
        refs.append(_ref_gemm(ta, tb, A, B))
        descs.append(_lib.GemmDesc(ta, tb, M, N, K, ptr(Ad), A.shape[1], ptr(Bd), B.shape[1], ptr(Cd), N))
    arr = (_lib.GemmDesc * len(descs))(*descs)
    call("aic_hip_gemm_grouped", len(descs), arr, 0.5, 0.0, BF16, F32, stream())
    first = [host(c).copy() for c in outs]
    for c, r in zip(first, refs):
        assert rel(c, 0.5 * r) < 1e-5
    call("aic_hip_gemm_grouped", len(descs), arr, 0.5, 0.0, BF16, F32, stream())
    for c, f in zip(outs, first):
        np.testing.assert_array_equal(host(c), f)


# ----------------------------------------------------------------------------- streaming probe
@pytest.mark.parametrize("ni,no,b16", [(1, 0, False), (0, 1, False), (1, 1, False), (2, 1, False), (4, 3, True)])
@pytest.mark.parametrize("nt", [0, 1])
def test_stream_probe(ni, no, b16, nt):
    """The probe computes what it states (out_j = sum of inputs + j, bf16 copy of the sum) over
    a length that leaves a partial last iteration, so its rates are those of real work."""
    import ctypes as C

    n = 3 * 256 * 8 + 4 * 37
    rng = np.random.default_rng(ni * 10 + no + nt)
    xs = [rng.standard_normal(n).astype(np.float32) for _ in range(ni)]
    ins = [dev(x, torch.float32) for x in xs]
    outs = [torch.full((n,), 7.0, device="cuda") for _ in range(3)]
    ob = torch.zeros(n, dtype=torch.bfloat16, device="cuda") if b16 else None
    sink = torch.full((1,), 5.0, device="cuda")
    vp = C.c_void_p
    pin = (vp * 4)(*([ptr(t) for t in ins] + [None] * (4 - ni)))
    pout = (vp * 3)(*[ptr(t) for t in outs])
    call("aic_hip_stream_probe", pin, ni, pout, no, ptr(ob), ptr(sink), n, nt, stream())
    torch.cuda.synchronize()
    s = np.zeros(n, np.float32)
    for x in xs:
        s = s + x  # the kernel's order: ((x0 + x1) + x2) + x3 in fp32
    for j in range(3):
        if j < no:
            np.testing.assert_array_equal(host(outs[j]), s + np.float32(j))
        else:
            assert bool((outs[j] == 7.0).all())
    if b16:
        np.testing.assert_array_equal(host(ob.float()), bf16_round(s))
    if no == 0 and not b16:
        assert float(sink[0]) == 5.0  # random inputs: no zero sums, so the sink is untouched
    with pytest.raises(_lib.AicError):  # a length that is not a multiple of 4
        call("aic_hip_stream_probe", pin, ni, pout, no, ptr(ob), ptr(sink), n - 2, nt, stream())
    with pytest.raises(_lib.AicError):  # a mix the probe does not provide
        call("aic_hip_stream_probe", pin, 3, pout, 1, None, ptr(sink), n, nt, stream())
