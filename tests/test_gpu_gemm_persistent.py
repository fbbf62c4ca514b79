"""GPU parity of the persistent 256x256 bf16 GEMM (gemm_bf16_dma_pers): products with more
output tiles than CUs, so that each block runs several tiles and the copies and epilogue
stores of one tile overlap the next.  Every output element keeps the MFMA sequence and k order
of the plain tile kernel, so a bf16 output equals the fp32-output product (the non-persistent
kernel, same tiles) rounded to bf16 once, bit for bit; the fused epilogues are checked against
the product followed by the standalone pass."""
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


def _gemm(ta, tb, M, N, K, A, B, ct, R=None, alpha=1.0, beta=0.0, C0=None):
    Cout = C0.clone() if C0 is not None else torch.empty((M, N), dtype=ct, device="cuda")
    call("aic_hip_gemm", ta, tb, M, N, K, alpha, ptr(A), A.shape[1], ptr(B), B.shape[1], beta, ptr(Cout), N, ptr(R),
         N if R is not None else 0, BF16, F32 if ct == torch.float32 else BF16, stream())
    return Cout


def _bf16(x):
    """float32 -> bf16 values (round to nearest even), as float32."""
    return bf16_round(np.asarray(x, np.float32))


# (ta, tb, M, N, K): 1024 tiles (four per block on 256 CUs), 272 tiles (16 blocks run two, the
# rest one), the 1B step's q/k/v forward (768 tiles) and down-projection input gradient (704)
SHAPES = [(0, 1, 8192, 8192, 256), (0, 0, 8192, 8192, 256), (1, 0, 8192, 8192, 256), (1, 1, 8192, 8192, 256),
          (0, 1, 4096, 4352, 384), (1, 0, 4352, 4096, 384), (0, 1, 8192, 6144, 512), (0, 0, 8192, 5632, 512)]


@pytest.mark.parametrize("ta,tb,M,N,K", SHAPES)
def test_persistent_bf16_equals_rounded_fp32(ta, tb, M, N, K):
    rng = np.random.default_rng(M + N + K + 2 * ta + tb)
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
    c32 = host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.float32, alpha=0.75))
    c16 = host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.bfloat16, alpha=0.75))
    np.testing.assert_array_equal(c16, _bf16(c32))
    # and against float64 on a sample of rows (fp32 accumulation of exact bf16 products)
    rows = rng.choice(M, 64, replace=False)
    a = (A.T if ta else A)[rows].astype(np.float64)
    ref = 0.75 * (a @ (B.T if tb else B).astype(np.float64))
    assert rel(c32[rows], ref) < 1e-5
    # run to run
    np.testing.assert_array_equal(host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.bfloat16, alpha=0.75)), c16)


@pytest.mark.parametrize("ta,tb,M,N,K", [(0, 1, 8192, 4096, 512), (0, 0, 8192, 2304, 768)])
def test_persistent_residual_and_beta(ta, tb, M, N, K):
    """C = bf16(bf16(alpha AB) + beta C0 + R): the residual epilogue of the output and down
    projections, as the plain kernel stages it (one bf16 rounding of the product, the additions
    in fp32, one rounding of the sum)."""
    rng = np.random.default_rng(M + N + K + 5)
    A = bf16_round(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = bf16_round(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    R = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    C0 = bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
    c32 = host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.float32, alpha=0.5))
    out = host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.bfloat16, R=dev(R, torch.bfloat16), alpha=0.5))
    np.testing.assert_array_equal(out, _bf16(_bf16(c32) + R))
    outb = host(_gemm(ta, tb, M, N, K, Ad, Bd, torch.bfloat16, R=dev(R, torch.bfloat16), alpha=0.5, beta=-1.25,
                      C0=dev(C0, torch.bfloat16)))
    np.testing.assert_array_equal(outb, _bf16((_bf16(c32) + np.float32(-1.25) * C0) + R))


@pytest.mark.parametrize("T,d,K,hd,start", [(8192, 2048, 256, 128, 0), (8192, 2048, 256, 128, 5),
                                             (8192, 1024, 256, 64, 3)])
def test_persistent_rope_epilogue(orc, T, d, K, hd, start):
    """q/k/v product with more tiles than CUs: the rotary epilogue (heads of 128 exchanged
    between waves, heads of 64 within one) equals the bf16 product followed by aic_hip_rope
    within one bf16 rounding, v bit for bit; a nonzero start position offsets the table rows."""
    rng = np.random.default_rng(T + d + hd + start)
    N, seq = 3 * d, 2048
    A = bf16_round(rng.standard_normal((T, K)).astype(np.float32))
    W = bf16_round((rng.standard_normal((N, K)) / 8).astype(np.float32))
    cos_t = np.empty((start + seq, hd // 2), np.float32)
    sin_t = np.empty_like(cos_t)
    _lib.check(_lib.load().aic_hip_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, start + seq, hd, 10000.0))
    Ad, Wd, cd, sd = dev(A, torch.bfloat16), dev(W, torch.bfloat16), dev(cos_t), dev(sin_t)
    fused = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_rope", T, N, K, ptr(Ad), K, ptr(Wd), K, ptr(fused), N, 2 * d, hd, seq, start, ptr(cd), ptr(sd),
         stream())
    sep = _gemm(0, 1, T, N, K, Ad, Wd, torch.bfloat16)
    call("aic_hip_rope", ptr(sep), N, T // seq, seq, 2 * d // hd, hd, start, ptr(cd), ptr(sd), 0, BF16, stream())
    f, g = host(fused), host(sep)
    np.testing.assert_array_equal(f[:, 2 * d:], g[:, 2 * d:])
    assert np.max(np.abs(f[:, :2 * d] - g[:, :2 * d]) / (np.abs(g[:, :2 * d]) + 1e-3)) < 1e-2
    assert rel(f[:, :2 * d], g[:, :2 * d]) < 2e-3
    rows = np.arange(0, T, 61)
    ref = A[rows].astype(np.float64) @ W.astype(np.float64).T
    pos = rows % seq
    qk = np.stack([orc.rope_fwd(ref[i:i + 1, :2 * d], 1, 1, 2 * d // hd, hd, start_pos=start + int(pos[i]))[0]
                   for i in range(len(rows))])
    assert rel(f[rows, :2 * d], qk) < 8e-3


def test_persistent_swiglu_epilogues(orc):
    """gate/up product (704 paired tiles, K 256) with silu(g) u in the epilogue, and the down
    projection's input gradient with SwiGLU's backward in the epilogue: bit-identical to the
    product followed by the standalone passes."""
    rng = np.random.default_rng(11)
    M, f, K = 8192, 5632, 256
    A = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    W = bf16_round((rng.standard_normal((2 * f, K)) / np.sqrt(K)).astype(np.float32))
    Ad, Wd = dev(A, torch.bfloat16), dev(W, torch.bfloat16)
    gu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((M, f), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_swiglu", M, f, K, ptr(Ad), K, ptr(Wd), K, ptr(gu), 2 * f, ptr(h), f, stream())
    gu2 = _gemm(0, 1, M, 2 * f, K, Ad, Wd, torch.bfloat16)
    h2 = torch.empty_like(h)
    call("aic_hip_swiglu_fwd", ptr(gu2), ptr(gu2) + 2 * f, 2 * f, ptr(h2), f, M, f, BF16, stream())
    np.testing.assert_array_equal(host(gu), host(gu2))
    np.testing.assert_array_equal(host(h), host(h2))
    # backward: dh = dy W_down (K = 512 rows of W_down here), then SwiGLU's backward with gu
    Kd = 512
    dy = bf16_round(rng.standard_normal((M, Kd)).astype(np.float32))
    Wdn = bf16_round((rng.standard_normal((Kd, f)) / np.sqrt(Kd)).astype(np.float32))
    dyd, Wdnd = dev(dy, torch.bfloat16), dev(Wdn, torch.bfloat16)
    dh = torch.empty((M, f), dtype=torch.bfloat16, device="cuda")
    dgu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_gemm_swiglu_bwd", M, f, Kd, ptr(dyd), Kd, ptr(Wdnd), f, ptr(gu), 2 * f, ptr(dh), f, ptr(dgu), stream())
    dh2 = _gemm(0, 0, M, f, Kd, dyd, Wdnd, torch.bfloat16)
    dgu2 = torch.empty_like(dgu)
    call("aic_hip_swiglu_bwd", ptr(gu), ptr(gu) + 2 * f, 2 * f, ptr(dh2), f, ptr(dgu2), ptr(dgu2) + 2 * f, 2 * f,
         M, f, BF16, stream())
    np.testing.assert_array_equal(host(dgu), host(dgu2))
    ref = dy[:64].astype(np.float64) @ Wdn.astype(np.float64)
    g = host(gu)[:64]
    dg_ref, du_ref = orc.swiglu_bwd(g[:, :f], g[:, f:], ref)
    got = host(dgu)[:64]
    assert rel(got[:, :f], dg_ref) < 1e-2 and rel(got[:, f:], du_ref) < 1e-2
