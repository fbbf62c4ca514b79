"""GPU parity of the expert-ragged GEMM (aic_hip_gemm_ragged: the experts' products of a MoE
layer, rows per expert read from device offsets) on shapes where its bf16 launch runs the
persistent kernel over the experts' 256x256 tiles -- several tiles per block, so a block's copies
of its next tile cross from one expert to the next, into and out of partial row tiles, past an
empty expert and a one-row one.  Each output element keeps the MFMA sequence and k order of the
fp32-output launch, so the bf16 output equals that product rounded once to bf16, bit for bit --
except on the tiles of a short last round, which a second launch computes in K parts and adds in
part order (one bf16 rounding of a differently ordered fp32 sum: within one bf16 unit, and the
same from run to run); the SwiGLU epilogues equal the product followed by the standalone passes;
rows outside the experts are not written."""
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


def _bf16_unit(x):
    """The spacing of bf16 values at |x| (x nonzero)."""
    return np.exp2(np.floor(np.log2(np.abs(x))) - 7)


def _equal_or_split_tail(got, ref, max_tiles):
    """got equals ref bit for bit, except on at most max_tiles 256 x 256 tiles (a K-split last
    round), where each element is within one bf16 unit of ref plus 2^-14 of ref's RMS: the two fp32
    sums of the same products in different orders differ by a few fp32 units of the products'
    magnitudes, which a bf16 rounding turns into at most one unit -- or, where the sum cancels to
    a small value, into that small absolute difference."""
    diff = got != ref
    if not diff.any():
        return
    assert diff.sum() <= max_tiles * 256 * 256, f"{diff.sum()} elements differ"
    d = np.abs(got[diff].astype(np.float64) - ref[diff].astype(np.float64))
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    tol = _bf16_unit(np.where(ref[diff] != 0, ref[diff], got[diff])) + 2.0 ** -14 * rms
    assert np.all(d <= tol), f"max |diff| {d.max()} (rms {rms})"


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
    _equal_or_split_tail(h16[:end], bf16_round(h32[:end]), max_tiles=64)
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
    followed by aic_hip_swiglu_fwd / aic_hip_swiglu_bwd.  (The plain bf16 launches may split a
    short last round along K, so the unsplit products come from the epilogue's own C output and
    from the fp32 launch rounded to bf16.)"""
    f, d = (1024, 1024) if key == "many" else (384, 512)
    counts, E, offs, M, A, Wgu = _setup(key, d, 2 * f, 1, 7 + f)
    end = int(offs[-1])
    Ad, Wd_, od = dev(A, torch.bfloat16), dev(Wgu, torch.bfloat16), dev(offs)
    gu = torch.empty((M, 2 * f), dtype=torch.bfloat16, device="cuda")
    h = torch.full((M, f), 5.0, dtype=torch.bfloat16, device="cuda")
    _ragged(1, M, 2 * f, d, Ad, Wd_, 2 * f * d, gu, od, E, BF16, glu_f=f, glu_out=h, ld_glu=f)
    gu2 = torch.empty_like(gu)
    _ragged(1, M, 2 * f, d, Ad, Wd_, 2 * f * d, gu2, od, E, BF16)
    _equal_or_split_tail(host(gu)[:end], host(gu2)[:end], max_tiles=64)
    h2 = torch.empty_like(h)
    call("aic_hip_swiglu_fwd", ptr(gu), ptr(gu) + 2 * f, 2 * f, ptr(h2), f, end, f, BF16, stream())
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
    dh32 = torch.empty((M, f), dtype=torch.float32, device="cuda")
    _ragged(0, M, f, d, dyd, Wdnd, d * f, dh32, od, E, F32)
    dh2 = dev(bf16_round(host(dh32)), torch.bfloat16)
    dgu2 = torch.empty_like(dgu)
    call("aic_hip_swiglu_bwd", ptr(gu), ptr(gu) + 2 * f, 2 * f, ptr(dh2), f, ptr(dgu2), ptr(dgu2) + 2 * f, 2 * f,
         end, f, BF16, stream())
    np.testing.assert_array_equal(host(dgu)[:end], host(dgu2)[:end])
    if f % 256 == 0:  # in the epilogue; otherwise the standalone pass runs over all M rows
        assert np.all(host(dgu)[end:] == 7.0)


@pytest.mark.parametrize("transB,N,K", [(1, 1024, 2816), (0, 1024, 5632)])
def test_ragged_split_tail(transB, N, K):
    """The MoE step's 1024-wide expert products (down forward, gate/up input gradient): 16384
    routed rows over 8 experts are 264 tiles of 256x256, one round and 8 tiles, whose last round
    runs split along K into fp32 parts added in part order.  The bf16 output is within one bf16
    unit of the fp32 launch's product rounded once (bit-equal off the split tiles), the same from
    run to run, within bf16 rounding of the float64 product, and rows past the experts are not
    written."""
    counts = [2100, 1990, 2060, 2150, 2000, 2080, 1904, 2100]
    E = len(counts)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    end = int(offs[-1])
    M = end + 256
    tiles = sum((c + 255) // 256 for c in counts) * (N // 256)
    bound = ((M + 255) // 256 + E) * (N // 256)
    assert tiles % 256 and tiles // 256 == bound // 256  # a short last round within the split's bound
    print(f"ragged split tail: transB {transB} N {N} K {K} tiles {tiles}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(N + K + transB)
    Ad = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    shape = (E, N, K) if transB else (E, K, N)
    Bd = (torch.randn(shape, device="cuda", generator=g) / np.sqrt(K)).to(torch.bfloat16)
    od = dev(offs)
    c32 = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    _ragged(transB, M, N, K, Ad, Bd, N * K, c32, od, E, F32)
    c16 = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    _ragged(transB, M, N, K, Ad, Bd, N * K, c16, od, E, BF16)
    h16, h32 = host(c16), host(c32)
    _equal_or_split_tail(h16[:end], bf16_round(h32[:end]), max_tiles=tiles % 256)
    assert np.all(h16[end:] == 3.0)
    c16b = torch.empty_like(c16)
    _ragged(transB, M, N, K, Ad, Bd, N * K, c16b, od, E, BF16)
    np.testing.assert_array_equal(host(c16b)[:end], h16[:end])
    rows = np.unique(np.concatenate([offs[1:-1] - 1, offs[1:-1], np.arange(0, end, 211)]))
    A64 = host(Ad).astype(np.float64)
    Bs = host(Bd)
    ref = _expert_ref(A64, Bs, offs, transB, rows)
    assert rel(h16[rows], ref) < 4e-3
