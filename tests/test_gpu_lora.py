"""GPU parity of the one-pass LoRA adapter products (aic_hip_lora_skinny) against float64 products
of the same bf16 inputs: the forward x A^T, the backward pair dy^T xs / dy B over stacked
segments (q, k, v or gate, up) in one pass, and dxa^T x -- the rank-r matmuls of LoRALinear
(src/nn/lora.cpp:75-93) and their MatMulBackward gradients.  fp32 outputs are fp32 sums of exact
bf16 products (relative 1e-5 against float64); bf16 outputs are one rounding of such a sum.
Ragged token counts (not a multiple of 64), the row-block and column-group partial sums, the
accumulate flag, run-to-run equality and the shapes the kernel declines are covered."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import bf16_round, call, dev, host, ptr, rel, stream  # noqa: E402

NOT_IMPLEMENTED = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _r(rng, *shape, scale=1.0):
    return bf16_round((scale * rng.standard_normal(shape)).astype(np.float32))


def _skinny(Y, T, N, n_seg, r_seg, W=None, w_n=0, w_j=0, out1=None, ldo1=0, scale=1.0, Z=None, ldz=0, out2=None,
            o2n=0, o2j=0, accumulate=0):
    call("aic_hip_lora_skinny", ptr(Y), Y.shape[1], T, N, n_seg, r_seg, ptr(W), w_n, w_j, ptr(out1), ldo1, scale,
         ptr(Z), ldz, ptr(out2), o2n, o2j, accumulate, stream())


@pytest.mark.parametrize("T,N,R", [(8192, 2048, 48), (8192, 5632, 16), (1000, 2048, 32), (64, 768, 16),
                                   (4100, 256, 48)])
def test_forward_x_at(T, N, R):
    """xs = bf16(s x A^T): A [R, in] rows (w_n = 1), one segment."""
    rng = np.random.default_rng(T + N + R)
    x, A = _r(rng, T, N), _r(rng, R, N, scale=0.05)
    xd, Ad = dev(x, torch.bfloat16), dev(A, torch.bfloat16)
    xs = torch.full((T, R), 3.0, dtype=torch.bfloat16, device="cuda")
    _skinny(xd, T, N, N, R, W=Ad, w_n=1, w_j=N, out1=xs, ldo1=R, scale=2.0)
    ref = 2.0 * (x.astype(np.float64) @ A.astype(np.float64).T)
    got = host(xs)
    assert rel(got, ref) < 3e-3
    assert np.max(np.abs(got - ref)) <= 2 ** -7 * np.max(np.abs(ref)) + 1e-6
    # the same as the library GEMM of the step's earlier path, within one bf16 rounding
    g = torch.empty_like(xs)
    call("aic_hip_gemm", 0, 1, T, R, N, 2.0, ptr(xd), N, ptr(Ad), N, 0.0, ptr(g), R, None, 0, _lib.AIC_BF16,
         _lib.AIC_BF16, stream())
    assert np.max(np.abs(host(g) - got)) <= 2 ** -7 * np.max(np.abs(ref)) + 1e-6
    xs2 = torch.empty_like(xs)
    _skinny(xd, T, N, N, R, W=Ad, w_n=1, w_j=N, out1=xs2, ldo1=R, scale=2.0)
    np.testing.assert_array_equal(host(xs2), got)


@pytest.mark.parametrize("T,n_seg,S,r", [(8192, 2048, 3, 16), (8192, 5632, 2, 16), (1000, 512, 3, 16),
                                         (8192, 2048, 1, 16), (300, 768, 1, 32), (2048, 256, 2, 48)])
def test_backward_db_dxa_one_pass(T, n_seg, S, r):
    """dB = dy^T xs and dxa = s dy B per segment, from one pass over dy [T, S n_seg]; B stacked
    [S n_seg, r] (w_j = 1), xs / dxa [T, S r]."""
    rng = np.random.default_rng(T + n_seg + S + r)
    N = S * n_seg
    dy, xs, B = _r(rng, T, N), _r(rng, T, S * r), _r(rng, N, r, scale=0.05)
    dyd, xsd, Bd = dev(dy, torch.bfloat16), dev(xs, torch.bfloat16), dev(B, torch.bfloat16)
    dxa = torch.full((T, S * r), 5.0, dtype=torch.bfloat16, device="cuda")
    dB = torch.full((N, r), 7.0, dtype=torch.float32, device="cuda")
    _skinny(dyd, T, N, n_seg, r, W=Bd, w_n=r, w_j=1, out1=dxa, ldo1=S * r, scale=0.5, Z=xsd, ldz=S * r, out2=dB,
            o2n=r, o2j=1)
    dy64, xs64, B64 = dy.astype(np.float64), xs.astype(np.float64), B.astype(np.float64)
    dB_ref = np.concatenate([dy64[:, g * n_seg:(g + 1) * n_seg].T @ xs64[:, g * r:(g + 1) * r] for g in range(S)])
    dxa_ref = np.concatenate([0.5 * dy64[:, g * n_seg:(g + 1) * n_seg] @ B64[g * n_seg:(g + 1) * n_seg]
                              for g in range(S)], axis=1)
    assert rel(host(dB), dB_ref) < 1e-5
    got = host(dxa)
    assert rel(got, dxa_ref) < 3e-3
    assert np.max(np.abs(got - dxa_ref)) <= 2 ** -7 * np.max(np.abs(dxa_ref)) + 1e-6
    # accumulate adds to dB; dxa is rewritten identically (run to run)
    dxa2 = torch.empty_like(dxa)
    dB_before = host(dB).copy()
    _skinny(dyd, T, N, n_seg, r, W=Bd, w_n=r, w_j=1, out1=dxa2, ldo1=S * r, scale=0.5, Z=xsd, ldz=S * r, out2=dB,
            o2n=r, o2j=1, accumulate=1)
    np.testing.assert_array_equal(host(dxa2), got)
    np.testing.assert_array_equal(host(dB), dB_before + dB_before)


@pytest.mark.parametrize("T,n_seg,S", [(8192, 2048, 3), (500, 768, 2)])
def test_dxa_alone_over_segments(T, n_seg, S):
    """The out1 product by itself on B-stacked segments (w_j = 1): dxa = s dy B per segment, the
    general kernel's column-group partial sums."""
    rng = np.random.default_rng(T + n_seg)
    N, r = S * n_seg, 16
    dy, B = _r(rng, T, N), _r(rng, N, r, scale=0.05)
    dyd, Bd = dev(dy, torch.bfloat16), dev(B, torch.bfloat16)
    dxa = torch.empty((T, S * r), dtype=torch.bfloat16, device="cuda")
    _skinny(dyd, T, N, n_seg, r, W=Bd, w_n=r, w_j=1, out1=dxa, ldo1=S * r, scale=0.25)
    ref = np.concatenate([0.25 * dy[:, g * n_seg:(g + 1) * n_seg].astype(np.float64) @
                          B[g * n_seg:(g + 1) * n_seg].astype(np.float64) for g in range(S)], axis=1)
    got = host(dxa)
    assert rel(got, ref) < 3e-3
    assert np.max(np.abs(got - ref)) <= 2 ** -7 * np.max(np.abs(ref)) + 1e-6


@pytest.mark.parametrize("T,N,R", [(8192, 2048, 48), (8192, 5632, 16), (777, 2048, 32), (64, 256, 16)])
def test_backward_da(T, N, R):
    """dA = dxa^T x, written transposed into A's [R, in] layout (o2n = 1, o2j = in)."""
    rng = np.random.default_rng(3 * T + N + R)
    x, dxa = _r(rng, T, N), _r(rng, T, R)
    xd, dxad = dev(x, torch.bfloat16), dev(dxa, torch.bfloat16)
    dA = torch.full((R, N), 9.0, dtype=torch.float32, device="cuda")
    _skinny(xd, T, N, N, R, Z=dxad, ldz=R, out2=dA, o2n=1, o2j=N)
    ref = dxa.astype(np.float64).T @ x.astype(np.float64)
    assert rel(host(dA), ref) < 1e-5
    dA2 = torch.empty_like(dA)
    _skinny(xd, T, N, N, R, Z=dxad, ldz=R, out2=dA2, o2n=1, o2j=N)
    np.testing.assert_array_equal(host(dA2), host(dA))


def test_declined_shapes():
    """r_seg outside {16, 32, 48}, segments not a multiple of 256 columns, misaligned leading
    dimensions: NotImplemented, and nothing is written."""
    x = torch.zeros((128, 512), dtype=torch.bfloat16, device="cuda")
    A = torch.zeros((8, 512), dtype=torch.bfloat16, device="cuda")
    out = torch.full((128, 8), 1.0, dtype=torch.bfloat16, device="cuda")
    for args in [(x, 128, 512, 512, 8), (x, 128, 512, 128, 16), (x, 128, 500, 500, 16)]:
        with pytest.raises(_lib.AicError) as e:
            _skinny(*args, W=A, w_n=1, w_j=512, out1=out, ldo1=8)
        assert e.value.code == NOT_IMPLEMENTED
    assert np.all(host(out) == 1.0)
