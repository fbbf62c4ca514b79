"""GPU parity of the mixture-of-experts path (routing, dispatch, expert SwiGLUs, combine and
their backward) through the C-ABI, against the CPU oracle (orc_moe_*), which the CPU suite
pins against a brute-force top-k, the reference's routing invariants (tests/unit/test_moe.cpp)
and a float64 autograd restatement of src/nn/moe.cpp.  Routing indices and counts must be
bit-exact; fp32 values at the reference tolerances; bf16 at the bf16 rounding level."""
import ctypes as C

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


def _route(logits, k, coef):
    T, E = logits.shape
    ld = dev(logits)
    idx = torch.empty((T, k), dtype=torch.int64, device="cuda")
    gsel = torch.empty((T, k), dtype=torch.float32, device="cuda")
    probs = torch.empty((T, E), dtype=torch.float32, device="cuda")
    rw = torch.empty((T, k), dtype=torch.float32, device="cuda")
    counts = torch.empty(E, dtype=torch.int64, device="cuda")
    mp = torch.empty(E, dtype=torch.float32, device="cuda")
    aux = torch.empty(1, dtype=torch.float32, device="cuda")
    call("aic_hip_moe_route", ptr(ld), T, E, k, coef, ptr(idx), ptr(gsel), ptr(probs), ptr(rw), ptr(counts), ptr(mp),
         ptr(aux), stream())
    return [host(t) for t in (idx, gsel, probs, rw, counts, mp, aux)] + [idx, counts]


@pytest.mark.parametrize("T,E,k", [(1000, 8, 2), (333, 4, 1), (257, 16, 4), (64, 64, 8)])
def test_moe_route_bit_exact(orc, T, E, k):
    rng = np.random.default_rng(T + E + k)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[::7, 1] = logits[::7, 0]            # exact ties: the lower index must win
    logits[::11, :] = 0.25                     # whole rows tied
    idx, gsel, probs, rw, counts, mp, aux, *_ = _route(logits, k, 0.01)
    r_idx, r_rw, r_gates, r_probs, r_counts, r_mp, r_aux = orc.moe_route(logits, k, 0.01)
    np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(counts, r_counts)
    np.testing.assert_allclose(probs, r_probs, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gsel, np.take_along_axis(r_gates, r_idx, axis=1), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(rw, r_rw, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(mp, r_mp, rtol=1e-6)
    assert abs(aux[0] - r_aux) <= 1e-6 * abs(r_aux)


def test_moe_permute_is_a_stable_expert_sort(orc):
    rng = np.random.default_rng(5)
    T, E, k = 700, 8, 2
    logits = rng.standard_normal((T, E)).astype(np.float32)
    *_, idx_d, counts_d = _route(logits, k, 0.0)
    idx, counts = host(idx_d), host(counts_d)
    rows = _lib.load().aic_hip_moe_max_rows(T, E, k)
    offsets = torch.empty(E + 1, dtype=torch.int64, device="cuda")
    dst = torch.empty(T * k, dtype=torch.int32, device="cuda")
    src = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    call("aic_hip_moe_permute", ptr(idx_d), ptr(counts_d), T, k, E, ptr(offsets), ptr(dst), ptr(src), stream())
    off, dst, src = host(offsets), host(dst), host(src)
    assert off[0] == 0 and np.all(off % 64 == 0) and off[E] <= rows
    for e in range(E):
        ents = np.flatnonzero(idx.ravel() == e)            # entries t*k+j of expert e, token order
        block = src[off[e]:off[e + 1]]
        np.testing.assert_array_equal(block[:counts[e]], ents)
        assert np.all(block[counts[e]:] == -1) and off[e + 1] - off[e] == -(-counts[e] // 64) * 64
        np.testing.assert_array_equal(dst[ents], off[e] + np.arange(counts[e]))


def _experts_blob(wg, wu, wd):
    E = wg.shape[0]
    return np.concatenate([np.concatenate([wg[e].ravel(), wu[e].ravel(), wd[e].ravel()]) for e in range(E)])


def _split_experts(blob, E, f, d):
    b = blob.reshape(E, 3 * f * d)
    return (b[:, :f * d].reshape(E, f, d), b[:, f * d:2 * f * d].reshape(E, f, d), b[:, 2 * f * d:].reshape(E, d, f))


def _ffn_run(h, wr, wg, wu, wd, k, coef, dy, daux, dtype, residual=None):
    T, d = h.shape
    E, f, _ = wg.shape
    tdt = torch.float32 if dtype == F32 else torch.bfloat16
    m = C.c_void_p()
    call("aic_moe_ffn_create", d, f, E, k, coef, dtype, C.byref(m))
    try:
        hd, wrd = dev(h, tdt), dev(wr, tdt)
        exd = dev(_experts_blob(wg, wu, wd), tdt)
        R = dev(residual, tdt) if residual is not None else None
        y = torch.empty((T, d), dtype=tdt, device="cuda")
        aux = torch.empty(1, dtype=torch.float32, device="cuda")
        call("aic_moe_ffn_forward", m, ptr(hd), T, ptr(wrd), ptr(exd), ptr(R), ptr(y), ptr(aux), stream())
        idx = np.empty((T, k), np.int64)
        counts = np.empty(E, np.int64)
        call("aic_moe_ffn_routing", m, idx.ctypes.data, counts.ctypes.data, stream())
        dyd = dev(dy, tdt)
        dh = torch.empty((T, d), dtype=tdt, device="cuda")
        dwr = torch.full((E, d), 3.0, dtype=torch.float32, device="cuda")
        dex = torch.full((E * 3 * f * d,), 3.0, dtype=torch.float32, device="cuda")
        call("aic_moe_ffn_backward", m, ptr(dyd), daux, ptr(dh), ptr(dwr), ptr(dex), stream())
        return host(y), float(host(aux)[0]), idx, counts, host(dh), host(dwr), _split_experts(host(dex), E, f, d)
    finally:
        call("aic_moe_ffn_destroy", m)


def _weights(rng, T, d, f, E, scale=0.2):
    h = rng.standard_normal((T, d)).astype(np.float32)
    wr = (0.3 * rng.standard_normal((E, d))).astype(np.float32)
    wg = (scale * rng.standard_normal((E, f, d))).astype(np.float32)
    wu = (scale * rng.standard_normal((E, f, d))).astype(np.float32)
    wd = (scale * rng.standard_normal((E, d, f))).astype(np.float32)
    dy = rng.standard_normal((T, d)).astype(np.float32)
    return h, wr, wg, wu, wd, dy


@pytest.mark.parametrize("T,d,f,E,k", [(64, 32, 48, 4, 2), (200, 64, 96, 8, 2), (48, 32, 32, 4, 1)])
def test_moe_ffn_fp32_matches_oracle(orc, T, d, f, E, k):
    rng = np.random.default_rng(T * d + E)
    h, wr, wg, wu, wd, dy = _weights(rng, T, d, f, E)
    coef, daux = 0.02, 1.3
    y, aux, idx, counts, dh, dwr, (dwg, dwu, dwd) = _ffn_run(h, wr, wg, wu, wd, k, coef, dy, daux, F32)
    y_ref, aux_ref, idx_ref, _ = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, coef)
    np.testing.assert_array_equal(idx, idx_ref)
    np.testing.assert_array_equal(counts, np.bincount(idx_ref.ravel(), minlength=E))
    assert rel(y, y_ref) < 1e-5
    assert abs(aux - aux_ref) <= 1e-6 * abs(aux_ref)
    ref = orc.moe_ffn_bwd(h, wr, wg, wu, wd, k, coef, dy, daux)
    for name, got, r in zip(["dh", "dwr", "dwg", "dwu", "dwd"], [dh, dwr, dwg, dwu, dwd], ref):
        # top-1 gates are p / (p + 1e-9): their derivative cancels to ~1e-9 relative, below fp32
        # resolution, so the router gradient's gate part is rounding noise in any fp32 evaluation
        # of the reference graph (the oracle differs from float64 there by ~5e-3 too)
        tol = 1e-2 if (k == 1 and name == "dwr") else 1e-4
        assert rel(got, r) < tol, name


def test_moe_ffn_residual_idle_expert_and_determinism(orc):
    # expert 3 gets no token: its gradient is exactly zero; the residual is added; runs are bit-identical
    rng = np.random.default_rng(17)
    T, d, f, E, k = 96, 32, 64, 4, 2
    h, wr, wg, wu, wd, dy = _weights(rng, T, d, f, E)
    wr[3] = -50.0 * np.abs(wr[3]) - 5.0
    h = np.abs(h)
    res = rng.standard_normal((T, d)).astype(np.float32)
    out1 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, F32, residual=res)
    out2 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, F32, residual=res)
    assert out1[3][3] == 0
    assert np.all(out1[6][0][3] == 0) and np.all(out1[6][1][3] == 0) and np.all(out1[6][2][3] == 0)
    y_ref, *_ = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, 0.01)
    assert rel(out1[0], y_ref + res) < 1e-5
    for a, b in zip(out1[:6], out2[:6]):
        np.testing.assert_array_equal(a, b)


def test_moe_ffn_bf16_close_to_fp32_oracle(orc):
    # MoE config widths scaled down (d 1024 -> 256, f 2816 -> 704), 8 experts, top-2, bf16 compute
    rng = np.random.default_rng(23)
    T, d, f, E, k = 512, 256, 704, 8, 2
    h, wr, wg, wu, wd, dy = _weights(rng, T, d, f, E, scale=0.05)
    h, wr, wg, wu, wd, dy = (bf16_round(a) for a in (h, wr, wg, wu, wd, dy))
    y, aux, idx, counts, dh, dwr, (dwg, dwu, dwd) = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, BF16)
    y_ref, aux_ref, idx_ref, _ = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, 0.01)
    # bf16 router logits can reorder near-ties; almost every token keeps its experts
    same = np.all(np.sort(idx, 1) == np.sort(idx_ref, 1), axis=1)
    assert np.mean(same) > 0.97
    assert rel(y[same], y_ref[same]) < 3e-2
    assert abs(aux - aux_ref) < 3e-2 * abs(aux_ref)
    ref = orc.moe_ffn_bwd(h, wr, wg, wu, wd, k, 0.01, dy, 1.0)
    for name, got, r in zip(["dh", "dwr", "dwg", "dwu", "dwd"], [dh, dwr, dwg, dwu, dwd], ref):
        assert rel(got, r) < 6e-2, name


def test_moe_ffn_bf16_fused_swiglu_rows(orc):
    """bf16 at widths whose expert products take SwiGLU in their epilogues (2f and f whole
    256-column tiles, f % 128 == 0: the gate/up product writes silu(gate) * up, the down
    projection's input gradient feeds SwiGLU's backward), with ragged expert row counts, so experts
    end in partial row tiles: every token's output and input-gradient row against the fp32 oracle
    (per-row relative error, so one wrong row at an expert boundary cannot hide in a global norm),
    the weight gradients within the bf16 tolerance, and two runs bit-identical."""
    rng = np.random.default_rng(4242)
    T, d, f, E, k = 1000, 256, 768, 8, 2
    h, wr, wg, wu, wd, dy = _weights(rng, T, d, f, E, scale=0.05)
    h, wr, wg, wu, wd, dy = (bf16_round(a) for a in (h, wr, wg, wu, wd, dy))
    out1 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, BF16)
    out2 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, BF16)
    for a, b in zip(out1[:6], out2[:6]):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(out1[6], out2[6]):
        np.testing.assert_array_equal(a, b)
    y, aux, idx, counts, dh, dwr, (dwg, dwu, dwd) = out1
    assert np.any(counts % 256 != 0)
    y_ref, aux_ref, idx_ref, _ = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, 0.01)
    same = np.all(np.sort(idx, 1) == np.sort(idx_ref, 1), axis=1)
    assert np.mean(same) > 0.97

    def row_err(got, r):
        return np.linalg.norm(got - r, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-6)

    ey = row_err(y[same], y_ref[same])
    ref = orc.moe_ffn_bwd(h, wr, wg, wu, wd, k, 0.01, dy, 1.0)
    edh = row_err(dh[same], ref[0][same])
    print(f"  rows: y max {ey.max():.3g} mean {ey.mean():.3g}; dh max {edh.max():.3g} mean {edh.mean():.3g}")
    assert ey.max() < 6e-2 and ey.mean() < 2e-2
    assert edh.max() < 1e-1 and edh.mean() < 3e-2
    for name, got, r in zip(["dwr", "dwg", "dwu", "dwd"], [dwr, dwg, dwu, dwd], ref[1:]):
        assert rel(got, r) < 6e-2, name


@pytest.mark.parametrize("T", [384, 4096])
def test_moe_ffn_bf16_idle_expert_and_determinism(orc, T):
    """bf16: the expert products read the row offsets on the device (128- and 256-row tiles at
    these sizes); an expert with no rows gets exactly zero weight gradients, the rest follow the
    fp32 oracle, and two runs are bit-identical."""
    rng = np.random.default_rng(29 + T)
    d, f, E, k = 256, 704, 8, 2
    h, wr, wg, wu, wd, dy = _weights(rng, T, d, f, E, scale=0.05)
    wr[5] = -50.0 * np.abs(wr[5]) - 5.0
    h = np.abs(h)
    h, wr, wg, wu, wd, dy = (bf16_round(a) for a in (h, wr, wg, wu, wd, dy))
    out1 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, BF16)
    out2 = _ffn_run(h, wr, wg, wu, wd, k, 0.01, dy, 1.0, BF16)
    y, aux, idx, counts, dh, dwr, (dwg, dwu, dwd) = out1
    assert counts[5] == 0 and counts.sum() == T * k
    assert np.all(dwg[5] == 0) and np.all(dwu[5] == 0) and np.all(dwd[5] == 0)
    for a, b in zip(out1[:6], out2[:6]):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(out1[6], out2[6]):
        np.testing.assert_array_equal(a, b)
    y_ref, aux_ref, idx_ref, _ = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, 0.01)
    same = np.all(np.sort(idx, 1) == np.sort(idx_ref, 1), axis=1)
    assert np.mean(same) > 0.97
    assert rel(y[same], y_ref[same]) < 3e-2
    ref = orc.moe_ffn_bwd(h, wr, wg, wu, wd, k, 0.01, dy, 1.0)
    for name, got, r in zip(["dh", "dwr", "dwg", "dwu", "dwd"], [dh, dwr, dwg, dwu, dwd], ref):
        assert rel(got, r) < 6e-2, name
