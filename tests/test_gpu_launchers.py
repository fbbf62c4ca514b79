"""GPU parity of the launcher-level entries that the reference's CUDA launchers reach beyond the
training step: attention with queries and keys of different lengths (KV-cached decode,
launch_flash_attention_forward/backward_gpu with seq_len_q != seq_len_k) and cross-entropy with
soft (probability) targets (cuda_cross_entropy_forward/backward with is_index_target false).
Called through the C-ABI with the layout the reference-side shim passes ([B, H, S, D]
contiguous as B*H batches of one head), against the oracle's restatement of the CPU paths
(src/ops/flash_attention.cpp:32-260, src/loss/cross_entropy.cpp:240-248).  fp32 at reference
precision; bf16 on bf16-rounded inputs within the stated bound."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import bf16_round, call, dev, host, ptr, rel, stream  # noqa: E402

F32, BF16 = _lib.AIC_F32, _lib.AIC_BF16
INVALID_ARGUMENT, NOT_IMPLEMENTED = 1, 8  # the library's status codes (the reference's ErrorCode numbering)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _tdt(dt):
    return torch.float32 if dt == F32 else torch.bfloat16


# (B, H, Sq, Sk, D, causal): decode steps against a longer cache (Sq < Sk), more queries than
# keys (Sq > Sk, causal: queries past the last key see every key), equal lengths through the
# same entry, and non-causal cross attention; ragged lengths that are not tile multiples
CASES = [(2, 3, 5, 300, 64, True), (1, 2, 1, 129, 128, True), (2, 2, 150, 77, 64, True), (1, 4, 96, 96, 32, True),
         (2, 2, 70, 200, 16, False), (1, 1, 257, 65, 128, False)]


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("B,H,Sq,Sk,D,causal", CASES)
def test_attention_q_k_lengths(orc, dt, B, H, Sq, Sk, D, causal):
    rng = np.random.default_rng(B * 1000 + H * 100 + Sq + Sk + D + causal)
    BH = B * H
    q, do = (rng.standard_normal((BH, Sq, D)).astype(np.float32) for _ in range(2))
    k, v = (rng.standard_normal((BH, Sk, D)).astype(np.float32) for _ in range(2))
    if dt == BF16:
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    scale = 1.0 / np.sqrt(D)
    o_ref, lse_ref = orc.flash_fwd(q, k, v, causal, scale)
    t = _tdt(dt)
    qd, kd, vd, dod = dev(q, t), dev(k, t), dev(v, t), dev(do, t)
    od = torch.empty_like(qd)
    lse = torch.empty((BH, Sq), dtype=torch.float32, device="cuda")
    call("aic_hip_attn_fwd_qk", ptr(qd), D, ptr(kd), ptr(vd), D, ptr(od), D, ptr(lse), BH, 1, Sq, Sk, D, int(causal),
         scale, dt, stream())
    o = host(od)
    assert np.max(np.abs(host(lse) - lse_ref)) < (2e-5 if dt == F32 else 1e-3)
    assert rel(o, o_ref) < (2e-6 if dt == F32 else 4e-3)
    # backward from the device's own o and lse, as the reference's autograd node passes them
    o_used = o if dt == F32 else bf16_round(o)
    dq_ref, dk_ref, dv_ref = orc.flash_bwd(q, k, v, o_used, do, host(lse), causal, scale)
    dqd, dkd, dvd = (torch.full_like(x, 7.0) for x in (qd, kd, vd))  # every element must be written
    call("aic_hip_attn_bwd_qk", ptr(qd), D, ptr(kd), ptr(vd), D, ptr(od), ptr(dod), D, ptr(lse), ptr(dqd), D, ptr(dkd),
         ptr(dvd), D, BH, 1, Sq, Sk, D, int(causal), scale, dt, stream())
    tol = 2e-5 if dt == F32 else 8e-3
    assert rel(host(dqd), dq_ref) < tol
    assert rel(host(dkd), dk_ref) < tol
    assert rel(host(dvd), dv_ref) < tol
    if causal:
        np.testing.assert_array_equal(o[:, 0], v[:, 0])  # query 0 sees key 0 only (v is bf16-exact)
        if Sk > Sq:  # keys that no query sees get zero gradients
            assert np.all(host(dkd)[:, Sq:] == 0) and np.all(host(dvd)[:, Sq:] == 0)


def test_attention_q_k_token_major_heads(orc):
    """The same entries on the step's token-major layout ([tokens, H*D] rows, heads side by side,
    leading dimensions wider than H*D): each head equals the oracle on its own columns."""
    rng = np.random.default_rng(5)
    B, H, Sq, Sk, D = 2, 3, 33, 100, 64
    ldq, ldk = H * D + 64, H * D + 128
    q = rng.standard_normal((B * Sq, ldq)).astype(np.float32)
    k = rng.standard_normal((B * Sk, ldk)).astype(np.float32)
    v = rng.standard_normal((B * Sk, ldk)).astype(np.float32)
    qd, kd, vd = dev(q), dev(k), dev(v)
    od = torch.zeros((B * Sq, ldq), dtype=torch.float32, device="cuda")
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device="cuda")
    call("aic_hip_attn_fwd_qk", ptr(qd), ldq, ptr(kd), ptr(vd), ldk, ptr(od), ldq, ptr(lse), B, H, Sq, Sk, D, 1,
         1.0 / np.sqrt(D), F32, stream())
    o = host(od)

    def heads(x, S):
        return x[:, :H * D].reshape(B, S, H, D).transpose(0, 2, 1, 3).reshape(B * H, S, D)

    o_ref, lse_ref = orc.flash_fwd(heads(q, Sq), heads(k, Sk), heads(v, Sk), True)
    assert rel(heads(o, Sq), o_ref) < 2e-6
    assert np.max(np.abs(host(lse).reshape(B * H, Sq) - lse_ref)) < 2e-5
    assert np.all(o[:, H * D:] == 0)  # columns past the heads untouched


def test_attention_q_k_edges():
    """No queries: the backward writes zero key gradients; no keys: InvalidArgument; an
    unsupported head dimension: NotImplemented."""
    D, Sk = 32, 40
    k = torch.randn((Sk, D), device="cuda")
    dk, dv = torch.full_like(k, 3.0), torch.full_like(k, 3.0)
    empty = torch.empty((1, D), device="cuda")
    call("aic_hip_attn_bwd_qk", ptr(empty), D, ptr(k), ptr(k), D, ptr(empty), ptr(empty), D, ptr(empty), ptr(empty),
         D, ptr(dk), ptr(dv), D, 1, 1, 0, Sk, D, 1, 0.2, F32, stream())
    assert np.all(host(dk) == 0) and np.all(host(dv) == 0)
    lse = torch.empty(4, device="cuda")
    q = torch.randn((4, D), device="cuda")
    with pytest.raises(_lib.AicError) as e:
        call("aic_hip_attn_fwd_qk", ptr(q), D, ptr(k), ptr(k), D, ptr(q), D, ptr(lse), 1, 1, 4, 0, D, 1, 0.2, F32,
             stream())
    assert e.value.code == INVALID_ARGUMENT
    q48 = torch.randn((4, 48), device="cuda")
    with pytest.raises(_lib.AicError) as e:
        call("aic_hip_attn_fwd_qk", ptr(q48), 48, ptr(q48), ptr(q48), 48, ptr(q48), 48, ptr(lse), 1, 1, 4, 4, 48, 1,
             0.2, F32, stream())
    assert e.value.code == NOT_IMPLEMENTED


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("N,Cn", [(64, 512), (37, 32000), (9, 77)])
def test_cross_entropy_soft_targets(orc, dt, N, Cn):
    rng = np.random.default_rng(N + Cn + dt)
    z = (2 * rng.standard_normal((N, Cn))).astype(np.float32)
    y = rng.random((N, Cn)).astype(np.float32) ** 4
    y /= y.sum(1, keepdims=True)
    y[0] = 0.0
    y[0, Cn - 1] = 1.0  # a one-hot row
    if dt == BF16:
        z = bf16_round(z)
    mean_ref, losses_ref, lse_ref = orc.ce_fwd_soft(z, y)
    zd, yd = dev(z, _tdt(dt)), dev(y)
    losses = torch.empty(N, dtype=torch.float32, device="cuda")
    lse = torch.empty(N, dtype=torch.float32, device="cuda")
    mean = torch.empty(1, dtype=torch.float32, device="cuda")
    call("aic_hip_ce_fwd_soft", ptr(zd), Cn, ptr(yd), Cn, N, Cn, ptr(losses), ptr(lse), ptr(mean), dt, stream())
    assert np.max(np.abs(host(lse) - lse_ref)) < 2e-5 * max(1.0, np.abs(lse_ref).max())
    assert np.max(np.abs(host(losses) - losses_ref)) < 5e-5 * max(1.0, np.abs(losses_ref).max())
    assert abs(float(host(mean)[0]) - mean_ref) < 2e-5 * max(1.0, abs(mean_ref))
    # reductions of the backward: mean (divisor N), sum, none (per-row incoming gradient)
    for per_row, divisor, g in [(0, float(N), np.float32([1.5])), (0, 1.0, np.float32([-0.5])),
                                (1, 1.0, rng.standard_normal(N).astype(np.float32))]:
        d = torch.empty_like(zd)
        call("aic_hip_ce_bwd_soft", ptr(zd), Cn, ptr(yd), Cn, ptr(lse), N, Cn, ptr(dev(g)), per_row, divisor, ptr(d),
             Cn, dt, stream())
        d_ref = orc.ce_bwd_soft(z, y, host(lse), g if per_row else g[0], per_row=bool(per_row), divisor=divisor)
        assert rel(host(d), d_ref) < (1e-5 if dt == F32 else 4e-3)
    # in place, no incoming gradient (unit), and the one-hot row equals the index-target backward
    call("aic_hip_ce_bwd_soft", ptr(zd), Cn, ptr(yd), Cn, ptr(lse), N, Cn, None, 0, float(N), ptr(zd), Cn, dt,
         stream())
    d_ref = orc.ce_bwd_soft(z, y, host(lse), 1.0, divisor=float(N))
    assert rel(host(zd), d_ref) < (1e-5 if dt == F32 else 4e-3)
    t = np.full(N, -100, np.int64)
    t[0] = Cn - 1
    z1 = dev(z, _tdt(dt))
    d1 = torch.empty_like(z1)
    call("aic_hip_ce_bwd_rows", ptr(z1), Cn, ptr(dev(t)), ptr(lse), N, Cn, -100, None, 0, float(N), ptr(d1), Cn, dt,
         stream())
    np.testing.assert_array_equal(host(d1)[0], host(zd)[0])


def test_cross_entropy_soft_targets_strided_and_empty(orc):
    """Leading dimensions wider than C for the logits and the targets; N = 0 writes a zero mean."""
    rng = np.random.default_rng(3)
    N, Cn, ld, ldy = 17, 1000, 1024, 1008
    z = rng.standard_normal((N, ld)).astype(np.float32)
    y = rng.random((N, ldy)).astype(np.float32)
    y[:, :Cn] /= y[:, :Cn].sum(1, keepdims=True)
    zd, yd = dev(z), dev(y)
    losses = torch.empty(N, dtype=torch.float32, device="cuda")
    lse = torch.empty(N, dtype=torch.float32, device="cuda")
    call("aic_hip_ce_fwd_soft", ptr(zd), ld, ptr(yd), ldy, N, Cn, ptr(losses), ptr(lse), None, F32, stream())
    _, losses_ref, lse_ref = orc.ce_fwd_soft(z[:, :Cn], y[:, :Cn])
    assert rel(host(losses), losses_ref) < 1e-6 and rel(host(lse), lse_ref) < 1e-6
    d = torch.full((N, ld), 9.0, device="cuda")
    call("aic_hip_ce_bwd_soft", ptr(zd), ld, ptr(yd), ldy, ptr(lse), N, Cn, None, 0, 1.0, ptr(d), ld, F32, stream())
    dh = host(d)
    assert rel(dh[:, :Cn], orc.ce_bwd_soft(z[:, :Cn], y[:, :Cn], lse_ref, 1.0)) < 1e-5
    assert np.all(dh[:, Cn:] == 9.0)
    mean = torch.full((1,), 5.0, device="cuda")
    call("aic_hip_ce_fwd_soft", ptr(zd), ld, ptr(yd), ldy, 0, Cn, None, None, ptr(mean), F32, stream())
    assert float(host(mean)[0]) == 0.0
