"""GPU parity of the expert-ragged GEMM (aic_hip_gemm_ragged: the experts' products of a MoE
layer, rows per expert read from device offsets) on shapes where its bf16 launch runs the
persistent kernel over the experts' 256x256 tiles -- several tiles per block, so a block's copies
of its next tile cross from one expert to the next, into and out of partial row tiles, past an
empty expert and a one-row one.  Each output element keeps the MFMA sequence and k order of the
fp32-output launch, so the bf16 output equals that product rounded once to bf16, bit for bit; the
SwiGLU epilogues equal the product followed by the standalone passes; rows outside the experts are
not written."""
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


# rows per expert: an empty expert, a one-row one, partial and whole 256-row tiles; 16384 rows in
# all is ~550 tiles of a 2048-column product (two or three per block on 256 CUs)
COUNTS = {"many": [3000, 0, 1, 2047, 2560, 5000, 1776, 2000], "few": [300, 257, 0, 511, 64, 100, 0, 800]}


def _ragged(transB, M, N, K, A, B, b_stride, C, offs, E, ct, alpha=1.0, glu_f=0, glu_out=None, ld_glu=0,
            dglu_gu=None, dglu_out=None, dglu_ld=0):
    call("aic_hip_gemm_ragged", transB, M, N, K, alpha, ptr(A), A.shape[1], ptr(B), B.shape[-1], b_stride, ptr(C),
         C.shape[1], ptr(offs), E, glu_f, ptr(glu_out), ld_glu, ptr(dglu_gu), ptr(dglu_out), dglu_ld, ct, stream())


def _setup(key, K, N, transB, seed):
    counts = COUNTS[key]
    E = len(counts)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    M = int(offs[-1]) + 256  # buffer rows past the experts' rows
    rng = np.random.default_rng(seed)
    A = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    Bs = bf16_round((rng.standard_normal((E, N, K) if transB else (E, K, N)) / np.sqrt(K)).astype(np.float32))
    return counts, E, offs, M, A, Bs


def _expert_ref(A, Bs, offs, transB, rows):
    """float64 product of the sampled rows, each with its expert's B."""
    out = []
    for r in rows:
        e = int(np.searchsorted(offs, r, side="right") - 1)
        b = Bs[e].astype(np.float64)
        out.append(A[r].astype(np.float64) @ (b.T if transB else b))
    return np.stack(out)


@pytest.mark.parametrize("key,transB,N,K", [("many", 1, 2048, 1024), ("many", 0, 1024, 2048), ("few", 1, 768, 512)])
def test_ragged_bf16_equals_rounded_fp32(key, transB, N, K):
    counts, E, offs, M, A, Bs = _setup(key, K, N, transB, N + K + transB)
    Ad, Bd, od = dev(A, torch.bfloat16), dev(Bs, torch.bfloat16), dev(offs)
    bs = N * K
    c32 = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    _ragged(transB, M, N, K, Ad, Bd, bs, c32, od, E, F32, alpha=0.5)
    c16 = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    _ragged(transB, M, N, K, Ad, Bd, bs, c16, od, E, BF16, alpha=0.5)
    end = int(offs[-1])
    h16, h32 = host(c16), host(c32)
    np.testing.assert_array_equal(h16[:end], bf16_round(h32[:end]))
    assert np.all(h16[end:] == 3.0)  # rows past the experts' rows untouched
    rows = np.concatenate([offs[1:-1] - 1, offs[1:-1], np.arange(0, end, 97)])
    rows = np.unique(rows[(rows >= 0) & (rows < end)])
    assert rel(h32[rows], 0.5 * _expert_ref(A, Bs, offs, transB, rows)) < 1e-5
    c16b = torch.empty_like(c16)
    _ragged(transB, M, N, K, Ad, Bd, bs, c16b, od, E, BF16, alpha=0.5)
    np.testing.assert_array_equal(host(c16b)[:end], h16[:end])


@pytest.mark.parametrize("key", ["many", "few"])
def test_ragged_swiglu_epilogues(key):
    """gate/up (transB, N = 2 glu_f) with silu(g) u in the epilogue, then the down projection's
    input gradient (K = d, N = f) with SwiGLU's backward in the epilogue: equal to the products
    followed by aic_hip_swiglu_fwd / aic_hip_swiglu_bwd."""
    f, d = (1024, 1024) if key == "many" else (384, 512)
    counts, E, offs, M, A, Wgu = _setup(key, d, 2 * f, 1, 7 + f)
    end = int(offs[-1])
    Ad, Wd_, od = dev(A, torch.bfloat16), dev(Wgu, torch.bfloat16), dev(offs)
    gu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    h = torch.full((M, f), 5.0, dtype=torch.bfloat16, device="cuda")
    _ragged(1, M, 2 * f, d, Ad, Wd_, 2 * f * d, gu, od, E, BF16, glu_f=f, glu_out=h, ld_glu=f)
    gu2 = torch.empty_like(gu)
    _ragged(1, M, 2 * f, d, Ad, Wd_, 2 * f * d, gu2, od, E, BF16)
    np.testing.assert_array_equal(host(gu)[:end], host(gu2)[:end])
    h2 = torch.empty_like(h)
    call("aic_hip_swiglu_fwd", ptr(gu2), ptr(gu2) + 2 * f, 2 * f, ptr(h2), f, end, f, BF16, stream())
    np.testing.assert_array_equal(host(h)[:end], host(h2)[:end])
    assert np.all(host(h)[end:] == 5.0)
    # backward: dh = dy Wd_e (Wd_e [d, f] as B [K = d, N = f]) into SwiGLU's backward with gu
    rng = np.random.default_rng(11 + f)
    dy = bf16_round(rng.standard_normal((M, d)).astype(np.float32))
    Wdn = bf16_round((rng.standard_normal((E, d, f)) / np.sqrt(d)).astype(np.float32))
    dyd, Wdnd = dev(dy, torch.bfloat16), dev(Wdn, torch.bfloat16)
    dh = torch.empty((M, f), dtype=torch.bfloat16, device="cuda")
    dgu = torch.full((M, 2 * f), 7.0, dtype=torch.bfloat16, device="cuda")
    _ragged(0, M, f, d, dyd, Wdnd, d * f, dh, od, E, BF16, dglu_gu=gu, dglu_out=dgu, dglu_ld=2 * f)
    dh2 = torch.empty_like(dh)
    _ragged(0, M, f, d, dyd, Wdnd, d * f, dh2, od, E, BF16)
    dgu2 = torch.empty_like(dgu)
    call("aic_hip_swiglu_bwd", ptr(gu), ptr(gu) + 2 * f, 2 * f, ptr(dh2), f, ptr(dgu2), ptr(dgu2) + 2 * f, 2 * f,
         end, f, BF16, stream())
    np.testing.assert_array_equal(host(dgu)[:end], host(dgu2)[:end])
    if f % 256 == 0:  # in the epilogue; otherwise the standalone pass runs over all M rows
        assert np.all(host(dgu)[end:] == 7.0)
