"""Pins the CPU oracle (oracle/liboracle.so) before any GPU result is compared with it.

Each check compares the oracle with something other than itself: the reference's own
known-answer tests (cited file:line under /root/reference/AutonomousAICore), a closed
form or invariant, or an independent torch float64 implementation built from library
routines.  CPU only.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests import torch_ref


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


# --------------------------------------------------------------------------- GEMM
def test_gemm_known_answers(orc):
    # tests/unit/test_matmul.cpp:17-37
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.array([[7, 8], [9, 1], [2, 3]], np.float32)
    np.testing.assert_array_equal(orc.gemm(a, b), np.array([[31, 19], [85, 55]], np.float32))
    # tests/unit/test_matmul.cpp:39-53 (SIMD remainders)
    c = orc.gemm(np.ones((67, 79), np.float32), np.full((79, 83), 2.0, np.float32))
    assert np.all(c == 158.0)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 17, 3), (64, 128, 64), (130, 70, 200), (257, 33, 129)])
def test_gemm_vs_float64(orc, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    assert rel(orc.gemm(A, B), ref) < 1e-6


def test_gemm_threads_do_not_change_rows(orc):
    rng = np.random.default_rng(3)
    A = rng.standard_normal((256, 96)).astype(np.float32)
    B = rng.standard_normal((96, 80)).astype(np.float32)
    orc.set_threads(1)
    c1 = orc.gemm(A, B)
    orc.set_threads(8)
    c8 = orc.gemm(A, B)
    orc.set_threads(0)
    np.testing.assert_array_equal(c1, c8)


def test_linear_fwd_bwd_vs_torch(orc):
    rng = np.random.default_rng(7)
    B, S, i, o = 3, 20, 48, 36
    x = rng.standard_normal((B * S, i)).astype(np.float32)
    W = rng.standard_normal((o, i)).astype(np.float32)
    dy = rng.standard_normal((B * S, o)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    Wt = torch.tensor(W, dtype=torch.float64, requires_grad=True)
    y = F.linear(xt, Wt)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    assert rel(orc.linear_fwd(x, W, B, S), y.detach().numpy()) < 1e-6
    dx, dW = orc.linear_bwd(x, W, dy, B, S)
    assert rel(dx, xt.grad.numpy()) < 1e-6
    assert rel(dW, Wt.grad.numpy()) < 1e-6


# --------------------------------------------------------------------------- RMSNorm
def test_rmsnorm_unit_rms(orc):
    # tests/unit/test_nn.cpp:58-81
    rng = np.random.default_rng(0)
    x = (2.5 * rng.standard_normal((64, 64))).astype(np.float32)
    y, _ = orc.rmsnorm_fwd(x, np.ones(64, np.float32), 1e-6)
    assert np.allclose((y.astype(np.float64) ** 2).mean(-1), 1.0, atol=1e-3)


def test_rmsnorm_vs_torch(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((33, 96)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(96)).astype(np.float32)
    dy = rng.standard_normal((33, 96)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    yt = F.rms_norm(xt, (96,), wt, 1e-6)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    y, rms = orc.rmsnorm_fwd(x, w, 1e-6)
    assert rel(y, yt.detach().numpy()) < 1e-6
    dx, dw = orc.rmsnorm_bwd(dy, x, w, rms)
    assert rel(dx, xt.grad.numpy()) < 1e-5
    assert rel(dw, wt.grad.numpy()) < 1e-5


# --------------------------------------------------------------------------- RoPE
def test_rope_invariants(orc):
    # tests/unit/test_nn.cpp:83-112: norm preservation and start_pos offset
    rng = np.random.default_rng(2)
    B, S, H, hd = 1, 8, 1, 16
    x = rng.standard_normal((B * S, H * hd)).astype(np.float32)
    xr = orc.rope_fwd(x, B, S, H, hd)
    np.testing.assert_allclose((xr.astype(np.float64) ** 2).sum(-1), (x.astype(np.float64) ** 2).sum(-1), rtol=1e-5)
    one = orc.rope_fwd(x[3:4], 1, 1, 1, hd, start_pos=3)
    np.testing.assert_allclose(one[0], xr[3], atol=1e-6)
    # position 0 is the identity rotation
    np.testing.assert_array_equal(xr[0], x[0])
    # backward is the inverse rotation, and the adjoint: <R x, g> == <x, R^T g>
    np.testing.assert_allclose(orc.rope_bwd(xr, B, S, H, hd), x, atol=1e-5)
    g = rng.standard_normal(x.shape).astype(np.float32)
    lhs = float((xr.astype(np.float64) * g).sum())
    rhs = float((x.astype(np.float64) * orc.rope_bwd(g, B, S, H, hd)).sum())
    assert abs(lhs - rhs) < 1e-4 * (abs(lhs) + 1)


def test_rope_pairs_are_half_split(orc):
    # a vector with only element i set rotates into elements i and i + hd/2 only
    hd, S = 8, 5
    x = np.zeros((S, hd), np.float32)
    x[:, 1] = 1.0
    xr = orc.rope_fwd(x, 1, S, 1, hd)
    cos, sin = torch_ref.rope_tables_np(S, hd)
    np.testing.assert_allclose(xr[:, 1], cos[:, 1], atol=1e-7)
    np.testing.assert_allclose(xr[:, 1 + hd // 2], sin[:, 1], atol=1e-7)
    assert np.count_nonzero(np.delete(xr, [1, 1 + hd // 2], axis=1)) == 0


# --------------------------------------------------------------------------- attention
@pytest.mark.parametrize("B,S,H,hd", [(2, 16, 2, 8), (1, 64, 4, 32), (2, 33, 3, 16)])
def test_attention_vs_sdpa(orc, B, S, H, hd):
    rng = np.random.default_rng(B * 100 + S)
    q, k, v, do = (rng.standard_normal((B * S, H * hd)).astype(np.float32) for _ in range(4))

    def t(a):
        return torch.tensor(a.reshape(B, S, H, hd), dtype=torch.float64).transpose(1, 2).requires_grad_(True)

    qt, kt, vt = t(q), t(k), t(v)
    ot = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
    ot.backward(torch.tensor(do.reshape(B, S, H, hd), dtype=torch.float64).transpose(1, 2))
    o, E, rs = orc.attention_fwd(q, k, v, B, S, H, hd)

    def back(x):
        return x.detach().transpose(1, 2).reshape(B * S, H * hd).numpy()

    assert rel(o, back(ot)) < 1e-5
    dq, dk, dv = orc.attention_bwd(q, k, v, E, rs, do, B, S, H, hd)
    assert rel(dq, qt.grad.transpose(1, 2).reshape(B * S, H * hd).numpy()) < 1e-5
    assert rel(dk, kt.grad.transpose(1, 2).reshape(B * S, H * hd).numpy()) < 1e-5
    assert rel(dv, vt.grad.transpose(1, 2).reshape(B * S, H * hd).numpy()) < 1e-5


@pytest.mark.parametrize("BH,Sq,Sk,D,causal", [(3, 5, 70, 16, True), (2, 70, 33, 32, True), (2, 40, 40, 8, True),
                                                (3, 7, 45, 16, False), (1, 65, 9, 8, False)])
def test_flash_attention_vs_masked_sdpa(orc, BH, Sq, Sk, D, causal):
    """The flash-attention CPU path (src/ops/flash_attention.cpp:32-260) with queries and keys of
    different lengths against torch float64 SDPA + autograd under the mask of the reference's own
    test (tests/unit/test_flash_attention.cpp:37-60: key j hidden from query i when j > i)."""
    rng = np.random.default_rng(BH * 1000 + Sq * 10 + Sk)
    q, do = (rng.standard_normal((BH, Sq, D)).astype(np.float32) for _ in range(2))
    k, v = (rng.standard_normal((BH, Sk, D)).astype(np.float32) for _ in range(2))
    qt, kt, vt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    mask = torch.ones(Sq, Sk, dtype=torch.bool).tril() if causal else None
    ot = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    ot.backward(torch.tensor(do, dtype=torch.float64))
    o, lse = orc.flash_fwd(q, k, v, causal)
    assert rel(o, ot.detach().numpy()) < 1e-5
    s = torch.tensor(q, dtype=torch.float64) @ torch.tensor(k, dtype=torch.float64).transpose(1, 2) / np.sqrt(D)
    if causal:
        s = s.masked_fill(~mask, -np.inf)
    assert np.max(np.abs(lse - torch.logsumexp(s, -1).numpy())) < 1e-5
    dq, dk, dv = orc.flash_bwd(q, k, v, o, do, lse, causal)
    assert rel(dq, qt.grad.numpy()) < 1e-5
    assert rel(dk, kt.grad.numpy()) < 1e-5
    assert rel(dv, vt.grad.numpy()) < 1e-5
    if causal:
        np.testing.assert_array_equal(o[:, 0], v[:, 0])  # query 0 sees key 0 only
        if Sk > Sq:
            assert np.all(dk[:, Sq:] == 0) and np.all(dv[:, Sq:] == 0)  # keys no query sees


def test_attention_first_row_copies_v(orc):
    # causal: query 0 sees only key 0, so o[0] == v[0] exactly
    rng = np.random.default_rng(5)
    B, S, H, hd = 1, 12, 2, 8
    q, k, v = (rng.standard_normal((B * S, H * hd)).astype(np.float32) for _ in range(3))
    o, _, _ = orc.attention_fwd(q, k, v, B, S, H, hd)
    np.testing.assert_array_equal(o[0], v[0])


# --------------------------------------------------------------------------- SwiGLU
def test_swiglu_vs_torch(orc):
    rng = np.random.default_rng(9)
    g, u, dh = (rng.standard_normal(1000).astype(np.float32) * 3 for _ in range(3))
    gt = torch.tensor(g, dtype=torch.float64, requires_grad=True)
    ut = torch.tensor(u, dtype=torch.float64, requires_grad=True)
    ht = F.silu(gt) * ut
    ht.backward(torch.tensor(dh, dtype=torch.float64))
    assert rel(orc.swiglu_fwd(g, u), ht.detach().numpy()) < 1e-6
    dg, du = orc.swiglu_bwd(g, u, dh)
    assert rel(dg, gt.grad.numpy()) < 1e-6
    assert rel(du, ut.grad.numpy()) < 1e-6


# --------------------------------------------------------------------------- cross-entropy
def test_ce_known_answer(orc):
    # tests/unit/test_optim.cpp:16-36
    z = np.array([[1, 2, 3], [1, -1, 0]], np.float32)
    loss, losses, lse, valid = orc.ce_fwd(z, np.array([2, 0]))
    assert abs(loss - 0.407606) < 1e-4 and valid == 2
    assert abs(losses.sum() - 2 * 0.407606) < 1e-4


def test_ce_stability_and_ignore(orc):
    # tests/unit/test_optim.cpp:38-65 and :101-129
    z = np.array([[1000, 1001, 999, 998], [-1000, -999, -1001, -1002]], np.float32)
    loss, _, lse, valid = orc.ce_fwd(z, np.array([1, 1]))
    d = orc.ce_bwd(z, np.array([1, 1]), lse, valid)
    assert math.isfinite(loss) and loss > 0 and np.all(np.isfinite(d))
    rng = np.random.default_rng(4)
    z = rng.standard_normal((6, 5)).astype(np.float32)
    t = np.array([0, 2, -100, -100, 4, 1])
    loss, _, lse, valid = orc.ce_fwd(z, t)
    d = orc.ce_bwd(z, t, lse, valid)
    assert valid == 4
    assert np.all(d[2] == 0) and np.all(d[3] == 0) and np.any(np.abs(d[0]) > 1e-6)


def test_ce_vs_torch(orc):
    rng = np.random.default_rng(11)
    z = (3 * rng.standard_normal((40, 77))).astype(np.float32)
    t = rng.integers(0, 77, 40)
    t[[3, 17]] = -100
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    lt = F.cross_entropy(zt, torch.tensor(t), ignore_index=-100)
    lt.backward(torch.tensor(2.0, dtype=torch.float64))
    loss, _, lse, valid = orc.ce_fwd(z, t)
    assert abs(loss - float(lt)) < 1e-6 * abs(float(lt))
    assert rel(orc.ce_bwd(z, t, lse, valid, g=2.0), zt.grad.numpy()) < 1e-6


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_ce_reductions_vs_torch(orc, reduction):
    """The reductions of CrossEntropyBackward (src/loss/cross_entropy.cpp:86-105) against torch
    float64 autograd of F.cross_entropy with the same reduction and incoming gradient."""
    rng = np.random.default_rng(12)
    z = (2 * rng.standard_normal((33, 50))).astype(np.float32)
    t = rng.integers(0, 50, 33)
    t[[0, 9, 10]] = -100
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    lt = F.cross_entropy(zt, torch.tensor(t), ignore_index=-100, reduction=reduction)
    g = rng.standard_normal(33).astype(np.float32) if reduction == "none" else np.float32(-1.5)
    lt.backward(torch.tensor(g, dtype=torch.float64))
    _, _, lse, valid = orc.ce_fwd(z, t)
    d = orc.ce_bwd_reduction(z, t, lse, valid, reduction, g)
    assert rel(d, zt.grad.numpy()) < 1e-6
    assert np.all(d[[0, 9, 10]] == 0)
    # mean with g equals the existing mean backward; sum = mean * valid; no g means g = 1
    if reduction == "mean":
        np.testing.assert_array_equal(d, orc.ce_bwd(z, t, lse, valid, g=-1.5))
    if reduction == "sum":
        assert rel(d, orc.ce_bwd(z, t, lse, valid, g=-1.5) * valid) < 1e-6
    if reduction == "none":
        ones = orc.ce_bwd_reduction(z, t, lse, valid, "none")
        assert rel(ones, orc.ce_bwd(z, t, lse, valid, g=float(valid))) < 1e-6


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_ce_soft_targets_vs_torch(orc, reduction):
    """Distribution targets (src/loss/cross_entropy.cpp:240-248, 120-125) against torch float64
    autograd of F.cross_entropy with probability targets; one-hot distributions reduce to the
    index-target loss and gradient."""
    rng = np.random.default_rng(13)
    N, Cn = 29, 61
    z = (2 * rng.standard_normal((N, Cn))).astype(np.float32)
    y = rng.random((N, Cn)).astype(np.float32)
    y /= y.sum(1, keepdims=True)
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    lt = F.cross_entropy(zt, torch.tensor(y, dtype=torch.float64), reduction=reduction)
    g = rng.standard_normal(N).astype(np.float32) if reduction == "none" else np.float32(0.75)
    lt.backward(torch.tensor(g, dtype=torch.float64))
    mean, losses, lse = orc.ce_fwd_soft(z, y)
    assert rel(losses, F.cross_entropy(torch.tensor(z, dtype=torch.float64), torch.tensor(y, dtype=torch.float64),
                                       reduction="none").numpy()) < 1e-6
    assert abs(mean - losses.astype(np.float64).mean()) < 1e-6 * abs(mean)
    per_row = reduction == "none"
    d = orc.ce_bwd_soft(z, y, lse, g, per_row=per_row, divisor=float(N) if reduction == "mean" else 1.0)
    assert rel(d, zt.grad.numpy()) < 1e-6
    # one-hot rows: the same numbers as index targets
    t = rng.integers(0, Cn, N)
    oh = np.eye(Cn, dtype=np.float32)[t]
    m1, l1, s1 = orc.ce_fwd_soft(z, oh)
    m0, l0, s0, valid = orc.ce_fwd(z, t)
    np.testing.assert_array_equal(l1, l0)
    np.testing.assert_array_equal(s1, s0)
    np.testing.assert_array_equal(orc.ce_bwd_soft(z, oh, s1, 1.0, divisor=float(N)), orc.ce_bwd(z, t, s0, valid))


# --------------------------------------------------------------------------- embedding
def test_embedding_known_answer(orc):
    # tests/unit/test_model.cpp:15-48
    rng = np.random.default_rng(6)
    W = rng.standard_normal((16, 8)).astype(np.float32)
    ids = np.array([0, 5, 12, 3, 5, 1])
    out = orc.embedding_fwd(ids, W)
    np.testing.assert_array_equal(out, W[ids])
    dW = orc.embedding_bwd(ids, np.ones((6, 8), np.float32), 16)
    assert np.all(dW[5] == 2.0) and np.all(dW[0] == 1.0) and np.all(dW[7] == 0.0)
    # out-of-range ids give zero rows and no gradient
    out = orc.embedding_fwd(np.array([-1, 16, 2]), W)
    assert np.all(out[:2] == 0) and np.array_equal(out[2], W[2])


# --------------------------------------------------------------------------- optimizer tail
def test_adamw_known_answer(orc):
    # tests/unit/test_optim.cpp:209-237
    p = np.ones(2, np.float32)
    m = np.zeros(2, np.float32)
    v = np.zeros(2, np.float32)
    orc.adamw(p, np.full(2, 0.1, np.float32), m, v, 0.01, 0.9, 0.999, 1e-8, 0.1, 1)
    np.testing.assert_allclose(p, 0.989, atol=1e-4)


def test_adamw_vs_torch(orc):
    rng = np.random.default_rng(12)
    p0 = rng.standard_normal(500).astype(np.float32)
    p = p0.copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    pt = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([pt], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for step in range(1, 4):
        g = rng.standard_normal(500).astype(np.float32)
        orc.adamw(p, g, m, v, 3e-4, 0.9, 0.95, 1e-8, 0.1, step)
        pt.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
    assert np.max(np.abs(p - pt.detach().numpy())) < 1e-6


def test_clip_known_answer(orc):
    # tests/unit/test_optim.cpp:191-207
    g1 = np.full(3, 3.0, np.float32)
    g2 = np.full(4, 4.0, np.float32)
    n = orc.clip_grad_norm([g1, g2], 5.0)
    assert abs(n - math.sqrt(91)) < 1e-3
    assert abs(orc.clip_grad_norm([g1, g2], 100.0) - 5.0) < 1e-3


def test_scaler_sequences(orc):
    # tests/unit/test_amp.cpp:56-84
    s = orc.LossScaler(initial_scale=1024.0)
    g = np.array([1024, 2048, -512, 0], np.float32)
    assert s.unscale_and_update([g]) and s.good_steps == 1 and s.skipped_steps == 0
    np.testing.assert_allclose(g, [1, 2, -0.5, 0])
    # :86-116 backoff on NaN then Inf
    for bad, expect in ((np.nan, 512.0), (np.inf, 256.0)):
        g = np.array([1, bad, 2, 3], np.float32)
        assert not s.unscale_and_update([g])
        assert s.scale == expect and s.good_steps == 0
    assert s.skipped_steps == 2
    # :118-142 growth every 3 good steps, capped at max
    s = orc.LossScaler(initial_scale=128.0, growth_interval=3, max_scale=1024.0)
    seen = []
    for _ in range(6):
        assert s.unscale_and_update([np.array([1, 2], np.float32)])
        seen.append(s.scale)
    assert seen == [128, 128, 256, 256, 256, 512]


# --------------------------------------------------------------------------- whole step
def _tiny_case(seed=1234, tied=True, vocab=512, d=128, L=2, H=4, f=352, B=8, S=64):
    rng = np.random.default_rng(seed)
    lay = torch_ref.layout(vocab, d, L, f, tied)
    params = []
    for name, shape in lay:
        if name.endswith("norm1.weight") or name.endswith("norm2.weight") or name == "norm.weight":
            params.append(np.ones(shape, np.float32).reshape(-1))
        else:
            params.append((0.02 * rng.standard_normal(shape)).astype(np.float32).reshape(-1))
    params = np.concatenate(params)
    seq = rng.integers(0, vocab, (B, S + 1))
    return params, seq[:, :S].copy(), seq[:, 1:].copy()


@pytest.mark.parametrize("tied", [True, False])
def test_lm_step_vs_torch(orc, tied):
    vocab, d, L, H, f, B, S = 512, 128, 2, 4, 352, 8, 64
    params, ids, tgt = _tiny_case(tied=tied)
    cfg = orc.make_config(vocab, d, L, H, f, S, tied=tied)
    assert orc.num_params(cfg) == params.size
    loss_t, norm_t, grads_t, new_t = torch_ref.lm_step(vocab, d, L, H, f, tied, params, ids, tgt, B, S)
    p = params.copy()
    res, grads, m, v, step = orc.lm_step(cfg, p, ids, tgt, B, S)
    assert abs(res.loss - loss_t) / abs(loss_t) < 1e-5
    assert abs(res.grad_norm - norm_t) / norm_t < 1e-4
    off = 0
    for name, shape in torch_ref.layout(vocab, d, L, f, tied):
        n = int(np.prod(shape))
        assert rel(grads[off:off + n], grads_t[off:off + n]) < 1e-4, name
        assert rel(p[off:off + n], new_t[off:off + n]) < 1e-4, name
        off += n
    assert step == 1


def test_lm_loss_matches_step_and_fd(orc):
    """orc_lm_loss equals the step's loss; a finite difference along the analytic gradient
    direction matches the directional derivative."""
    vocab, d, L, H, f, B, S = 64, 32, 1, 2, 48, 2, 8
    params, ids, tgt = _tiny_case(seed=5, tied=False, vocab=vocab, d=d, L=L, H=H, f=f, B=B, S=S)
    cfg = orc.make_config(vocab, d, L, H, f, S, tied=False)
    l0 = orc.lm_loss(cfg, params, ids, tgt, B, S)
    res, grads, _, _, _ = orc.lm_step(cfg, params.copy(), ids, tgt, B, S, max_grad_norm=1e9, do_update=False)
    assert l0 == res.loss
    u = grads / np.linalg.norm(grads)
    h = 1e-2
    lp = orc.lm_loss(cfg, (params + h * u).astype(np.float32), ids, tgt, B, S)
    lm = orc.lm_loss(cfg, (params - h * u).astype(np.float32), ids, tgt, B, S)
    fd = (lp - lm) / (2 * h)
    assert abs(fd - float(np.linalg.norm(grads))) < 2e-2 * float(np.linalg.norm(grads))


def test_lm_step_scaler_is_exact_power_of_two(orc):
    """With loss scaling the optimizer sees the same gradients (scale is a power of two)."""
    vocab, d, L, H, f, B, S = 64, 32, 1, 2, 48, 2, 8
    params, ids, tgt = _tiny_case(seed=8, tied=False, vocab=vocab, d=d, L=L, H=H, f=f, B=B, S=S)
    cfg = orc.make_config(vocab, d, L, H, f, S, tied=False)
    r0, g0, _, _, _ = orc.lm_step(cfg, params.copy(), ids, tgt, B, S, do_update=False)
    sc = orc.LossScaler()
    r1, g1, _, _, _ = orc.lm_step(cfg, params.copy(), ids, tgt, B, S, do_update=False, scaler=sc)
    assert r1.loss_scale_used == 65536.0 and not r1.found_inf
    np.testing.assert_array_equal(g0, g1)


# ----------------------------------------------------------------------------- mixture of experts
def test_moe_route_topk_brute_force_and_invariants(orc):
    # invariants of tests/unit/test_moe.cpp:25-76 (RouterTopKMath) plus a brute-force top-k
    rng = np.random.default_rng(11)
    T, E, k = 200, 8, 2
    logits = rng.standard_normal((T, E)).astype(np.float32)
    idx, rw, gates, probs, counts, mp, aux = orc.moe_route(logits, k, 0.01)
    np.testing.assert_array_equal(idx, torch_ref.moe_topk(logits, k))
    assert counts.sum() == T * k
    np.testing.assert_array_equal(counts, np.bincount(idx.ravel(), minlength=E))
    assert np.all(idx[:, 0] != idx[:, 1])
    assert np.all(rw > 0) and np.all(rw <= 1) and np.allclose(rw.sum(1), 1.0, atol=1e-4)
    np.testing.assert_allclose(gates.sum(1), 1.0, atol=1e-5)
    assert np.all(gates[np.arange(T)[:, None], idx] > 0) and np.count_nonzero(gates) == T * k


def test_moe_route_tie_rule(orc):
    # equal logits go to the lower expert index
    logits = np.array([[1, 1, 1, 0], [0, 2, 2, 2], [3, 0, 3, 3], [0.5, 0.5, 0.5, 0.5]], np.float32)
    idx, *_ = orc.moe_route(logits, 2, 0.0)
    np.testing.assert_array_equal(idx, [[0, 1], [1, 2], [0, 2], [0, 1]])
    idx3, *_ = orc.moe_route(logits, 3, 0.0)
    np.testing.assert_array_equal(idx3, [[0, 1, 2], [1, 2, 3], [0, 2, 3], [0, 1, 2]])


def test_moe_route_values_vs_float64(orc):
    import torch
    rng = np.random.default_rng(12)
    T, E, k, coef = 64, 8, 2, 0.05
    logits = (2 * rng.standard_normal((T, E))).astype(np.float32)
    idx, rw, gates, probs, counts, mp, aux = orc.moe_route(logits, k, coef)
    L = torch.tensor(logits, dtype=torch.float64)
    p = torch.softmax(L, -1).numpy()
    np.testing.assert_allclose(probs, p, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(mp, p.mean(0), rtol=1e-6)
    mask = np.zeros((T, E))
    np.put_along_axis(mask, idx, 1.0, axis=1)
    g = p * mask / ((p * mask).sum(1, keepdims=True) + 1e-9)
    np.testing.assert_allclose(gates, g, rtol=1e-6, atol=1e-7)
    sel = np.take_along_axis(logits.astype(np.float64), idx, axis=1)
    w = np.exp(sel - sel[:, :1])
    np.testing.assert_allclose(rw, w / w.sum(1, keepdims=True), rtol=1e-6)
    # aux = alpha * E / (T k) * sum_e count_e * mean_probs_e  (moe.cpp:84-101)
    assert abs(aux - coef * E / (T * k) * (counts * p.mean(0)).sum()) < 1e-7
    assert aux > 0
    # aux_coef = 0 gives a zero loss (tests/unit/test_moe.cpp:104-108)
    assert orc.moe_route(logits, k, 0.0)[6] == 0.0


@pytest.mark.parametrize("T,d,f,E,k", [(24, 16, 32, 4, 2), (40, 32, 48, 8, 2), (16, 16, 24, 4, 1)])
def test_moe_ffn_fwd_bwd_vs_float64(orc, T, d, f, E, k):
    rng = np.random.default_rng(T + d + E)
    h = rng.standard_normal((T, d)).astype(np.float32)
    wr = (0.3 * rng.standard_normal((E, d))).astype(np.float32)
    wg = (0.2 * rng.standard_normal((E, f, d))).astype(np.float32)
    wu = (0.2 * rng.standard_normal((E, f, d))).astype(np.float32)
    wd = (0.2 * rng.standard_normal((E, d, f))).astype(np.float32)
    dy = rng.standard_normal((T, d)).astype(np.float32)
    coef, daux = 0.02, 1.7
    y, aux, idx, gates = orc.moe_ffn_fwd(h, wr, wg, wu, wd, k, coef)
    y_ref, aux_ref, grads = torch_ref.moe_ffn_torch(h, wr, wg, wu, wd, k, coef, dy=dy, daux=daux)
    assert np.linalg.norm(y - y_ref) / np.linalg.norm(y_ref) < 1e-5
    assert abs(aux - aux_ref) <= 1e-6 * abs(aux_ref)
    got = orc.moe_ffn_bwd(h, wr, wg, wu, wd, k, coef, dy, daux)
    for name, gv, rv in zip(["dh", "dwr", "dwg", "dwu", "dwd"], got, grads):
        rv = np.zeros_like(gv) if rv is None else rv
        # top-1: the gate p / (p + 1e-9) has a derivative ~1e-9 relative, below fp32 resolution,
        # so the router gradient's gate part is fp32 rounding noise (the aux part dominates)
        tol = 1e-2 if (k == 1 and name == "dwr") else 1e-4
        assert np.linalg.norm(gv - rv) / max(np.linalg.norm(rv), 1e-12) < tol, name


# --------------------------------------------------------------------------- INT4 quantization
_NIBBLE = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]   # two's complement of 4 bits


def test_int4_every_byte_decodes_to_its_two_nibbles(orc):
    # all 256 bytes, scale 1: element 2i is the low nibble, 2i+1 the high nibble
    # (include/nn/quantization.hpp:41-56), both signed
    packed = np.arange(256, dtype=np.uint8)
    out = orc.int4_dequantize(packed, np.ones(1, np.float32), 512, 512)
    np.testing.assert_array_equal(out[0::2], np.array([_NIBBLE[b & 15] for b in range(256)], np.float32))
    np.testing.assert_array_equal(out[1::2], np.array([_NIBBLE[b >> 4] for b in range(256)], np.float32))


def _int4_zp_numpy(packed, scales, zp, is_signed, n, G):
    """The launcher's formula written independently: nibbles by shifts, sign by the xor-8 trick
    ((u ^ 8) - 8), groups by integer division, fp32 arithmetic."""
    b = np.asarray(packed, np.uint8).astype(np.int32)
    u = np.empty(2 * b.size, np.int32)
    u[0::2], u[1::2] = b & 15, b >> 4
    u = u[:n]
    val = ((u ^ 8) - 8) if is_signed else u
    g = np.arange(n) // G if G > 0 else np.zeros(n, np.int64)
    z = np.zeros(n, np.float32) if zp is None else np.asarray(zp, np.float32)[g]
    return (val.astype(np.float32) - z) * np.asarray(scales, np.float32)[g]


@pytest.mark.parametrize("is_signed", [True, False])
@pytest.mark.parametrize("G,with_zp", [(3, True), (8, True), (0, True), (7, False), (600, True)])
def test_int4_dequantize_zp_matches_the_launcher_formula(orc, is_signed, G, with_zp):
    # every byte, an odd element count, odd and <= 0 group sizes (launch_dequantize_int4,
    # src/cuda/cuda_quantize.cu:54-94: each element finds its own group; G <= 0 is group 0)
    packed = np.tile(np.arange(256, dtype=np.uint8), 2)
    n = 2 * packed.size - 1
    ng = (n + G - 1) // G if G > 0 else 1
    rng = np.random.default_rng(G + 2 * is_signed)
    scales = rng.uniform(0.01, 2.0, ng).astype(np.float32)
    zp = rng.integers(0, 16, ng).astype(np.float32) if with_zp else None
    got = orc.int4_dequantize_zp(packed, scales, zp, is_signed, n, G)
    np.testing.assert_array_equal(got, _int4_zp_numpy(packed, scales, zp, is_signed, n, G))


def test_int4_dequantize_zp_signed_without_zero_points_is_the_symmetric_form(orc):
    # INT4_SYMMETRIC goes through the same launcher with zp = nullptr (quantization.cpp:374-376)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1000) * 0.1).astype(np.float32)
    packed, s = orc.int4_quantize(x, 64)
    np.testing.assert_array_equal(orc.int4_dequantize_zp(packed, s, None, True, 1000, 64),
                                  orc.int4_dequantize(packed, s, 1000, 64))


def test_int4_known_bytes_and_exact_grid(orc):
    # a group whose absmax is 3.5 has s = 0.5 exactly, so x = q*s round-trips for q = -7..7
    q = np.arange(-7, 8, dtype=np.float32)
    x = np.concatenate([q * 0.5, [0.0]]).astype(np.float32)
    packed, s = orc.int4_quantize(x, 16)
    assert s.tolist() == [0.5]
    # pairs (-7,-6) (-5,-4) (-3,-2) (-1,0) (1,2) (3,4) (5,6) (7,0)
    assert packed.tolist() == [0xA9, 0xCB, 0xED, 0x0F, 0x21, 0x43, 0x65, 0x07]
    np.testing.assert_array_equal(orc.int4_dequantize(packed, s, 16, 16), x)


def test_int4_rounds_halves_away_from_zero(orc):
    # std::round, not round-half-even: 2.5 -> 3, -2.5 -> -3, 0.5 -> 1, 3.5 -> 4
    x = np.array([7.0, 2.5, -2.5, 0.5, -0.5, 3.5, -3.5, 1.4999], np.float32)
    packed, s = orc.int4_quantize(x, 8)
    assert s.tolist() == [1.0]
    np.testing.assert_array_equal(orc.int4_dequantize(packed, s, 8, 8), [7, 3, -3, 1, -1, 4, -4, 1])


def test_int4_scale_floor_and_group_layout(orc):
    x = np.zeros(10, np.float32)
    x[4:8] = [1.0, -2.0, 0.5, 0.25]
    packed, s = orc.int4_quantize(x, 4)           # groups [0:4] [4:8] [8:10]; the last one partial
    assert s.dtype == np.float32 and s.size == 3 and packed.size == 5
    assert s[0] == np.float32(1e-8) and s[2] == np.float32(1e-8)
    assert s[1] == np.float32(2.0) / np.float32(7.0)
    assert packed[0] == 0 and packed[1] == 0 and packed[4] == 0
    # G <= 0 or G > n: one group over the whole tensor (quantization.cpp:202-205)
    for G in (0, -1, 99):
        p1, s1 = orc.int4_quantize(x, G)
        assert s1.size == 1 and s1[0] == np.float32(2.0) / np.float32(7.0)
    # an odd group size with more than one group would split a byte between two groups
    with pytest.raises(ValueError):
        orc.int4_quantize(x, 3)


def test_int4_reference_packing_compression_and_cosine(orc):
    # tests/unit/test_quantization.cpp:47-67: 64x128 uniform(-2.5, 2.5), G = 32
    rng = np.random.default_rng(47)
    x = rng.uniform(-2.5, 2.5, (64, 128)).astype(np.float32)
    packed, s = orc.int4_quantize(x, 32)
    assert packed.size == 4096 and s.size == 256
    assert x.size * 4 / (packed.nbytes + s.nbytes) > 3.5
    deq = orc.int4_dequantize(packed, s, x.size, 32).astype(np.float64)
    xd = x.ravel().astype(np.float64)
    assert deq @ xd / (np.linalg.norm(deq) * np.linalg.norm(xd)) > 0.99


@pytest.mark.parametrize("n,G", [(4096, 128), (1000, 32), (777, 64), (513, 512)])
def test_int4_error_bound_and_idempotence(orc, n, G):
    rng = np.random.default_rng(n + G)
    x = (rng.standard_normal(n) * rng.uniform(0.01, 3.0)).astype(np.float32)
    packed, s = orc.int4_quantize(x, G)
    deq = orc.int4_dequantize(packed, s, n, G)
    sg = np.repeat(s, G)[:n].astype(np.float64)
    assert np.all(np.abs(deq - x) <= 0.5 * sg * (1 + 1e-6))          # round to nearest level
    # every group's absmax lands on +-7
    amax = np.array([np.abs(deq[i:i + G]).max() for i in range(0, n, G)])
    np.testing.assert_allclose(amax, 7 * s, rtol=0)
    p2, s2 = orc.int4_quantize(deq, G)                                # re-quantizing is a fixed point
    np.testing.assert_array_equal(p2, packed)
    np.testing.assert_allclose(s2, s, rtol=2e-7)


def test_f16_conversion_matches_numpy(orc):
    rng = np.random.default_rng(3)
    special = np.array([0.0, -0.0, 1e-8, 5.96e-8, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -24 * 1.5,
                        2.0 ** -24 * 2.5, 6.1e-5, 2.0 ** -14, 65504.0, 65519.0, 65520.0, 1e6, np.inf, -np.inf,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -11 + 2.0 ** -23], np.float32)
    x = np.concatenate([special, -special, np.float32(2.0) ** rng.uniform(-30, 17, 4000).astype(np.float32),
                        rng.standard_normal(2000).astype(np.float32) * 1e-6]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(orc.f32_to_f16_bits(x), ref)


def test_int4_fp16_scales(orc):
    # fp16 scale storage (the QLoRA configuration): the bytes are those of the fp32-scale run, the
    # scales are the fp16 rounding of the fp32 ones, dequantization multiplies by the widened fp16
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(8192) * 0.02).astype(np.float32)
    x[128:256] *= 1e-6                                                # an fp16-subnormal scale
    p32, s32 = orc.int4_quantize(x, 128)
    p16, s16 = orc.int4_quantize(x, 128, scale_f16=True)
    np.testing.assert_array_equal(p16, p32)
    np.testing.assert_array_equal(s16, s32.astype(np.float16))
    deq = orc.int4_dequantize(p16, s16, x.size, 128)
    q = orc.int4_dequantize(p32, np.ones_like(s32), x.size, 128)
    np.testing.assert_array_equal(deq, q * np.repeat(s16.astype(np.float32), 128))


# --------------------------------------------------------------------------- LoRA
def _lora_inputs(rng, Bt, S, inn, out, r):
    x = rng.standard_normal((Bt * S, inn)).astype(np.float32)
    W = (rng.standard_normal((out, inn)) / math.sqrt(inn)).astype(np.float32)
    A = rng.uniform(-1 / math.sqrt(inn), 1 / math.sqrt(inn), (r, inn)).astype(np.float32)
    Bm = rng.uniform(-0.5, 0.5, (out, r)).astype(np.float32)
    return x, W, A, Bm


def test_lora_zero_b_is_the_base_linear(orc):
    # tests/unit/test_lora.cpp:58-73: B = 0 at initialisation, so the output equals the base
    rng = np.random.default_rng(1)
    x, W, A, _ = _lora_inputs(rng, 2, 16, 64, 128, 8)
    y, _ = orc.lora_fwd(x, W, A, np.zeros((128, 8), np.float32), 16.0 / 8, 2, 16)
    np.testing.assert_array_equal(y, orc.linear_fwd(x, W, 2, 16))


def test_lora_merge_matches_unmerged_forward(orc):
    # tests/unit/test_lora.cpp:107-143 at its tolerance (1e-4), and unmerge restores W
    rng = np.random.default_rng(2)
    x, W, A, Bm = _lora_inputs(rng, 2, 8, 32, 48, 4)
    y, _ = orc.lora_fwd(x, W, A, Bm, 8.0 / 4, 2, 8)
    Wm = orc.lora_merge(W, A, Bm, 8.0 / 4)
    assert np.max(np.abs(orc.linear_fwd(x, Wm, 2, 8) - y)) < 1e-4
    assert np.max(np.abs(orc.lora_merge(Wm, A, Bm, 8.0 / 4, sign=-1) - W)) < 1e-6


@pytest.mark.parametrize("Bt,S,inn,out,r", [(2, 16, 64, 48, 8), (1, 40, 96, 32, 16), (3, 5, 17, 23, 3)])
def test_lora_fwd_bwd_vs_float64(orc, Bt, S, inn, out, r):
    rng = np.random.default_rng(Bt * S + inn + r)
    x, W, A, Bm = _lora_inputs(rng, Bt, S, inn, out, r)
    dy = rng.standard_normal((Bt * S, out)).astype(np.float32)
    scaling = 32.0 / r
    y, xa = orc.lora_fwd(x, W, A, Bm, scaling, Bt, S)
    dx, dA, dB = orc.lora_bwd(x, W, A, Bm, scaling, dy, Bt, S)
    xt, At, Bt_ = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (x, A, Bm))
    Wt = torch.tensor(W, dtype=torch.float64)
    yt = F.linear(xt, Wt) + F.linear(F.linear(xt, At), Bt_) * scaling
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    assert rel(y, yt.detach().numpy()) < 1e-6
    assert rel(xa, F.linear(xt, At).detach().numpy()) < 1e-6
    assert rel(dx, xt.grad.numpy()) < 1e-5
    assert rel(dA, At.grad.numpy()) < 1e-5
    assert rel(dB, Bt_.grad.numpy()) < 1e-5


# --------------------------------------------------------------------------- tensor primitives
def test_ops_reference_known_answers(orc):
    # tests/unit/test_ops.cpp:12-131
    a, b = np.full((2, 3), 4.0, np.float32), np.full((2, 3), 2.0, np.float32)
    for op, v in (("add", 6), ("sub", 2), ("mul", 8), ("div", 2)):
        assert np.all(orc.binary(op, a, b) == v)
    np.testing.assert_array_equal(orc.binary("add", np.arange(6, dtype=np.float32).reshape(2, 3),
                                             np.full((1, 3), 10.0, np.float32)),
                                  np.arange(10, 16, dtype=np.float32).reshape(2, 3))
    a5 = np.full((2, 2), 5.0, np.float32)                           # scalar operands are [1] tensors
    for op, sc, v in (("add", 3, 8), ("sub", 2, 3), ("div", 2, 2.5)):
        assert np.all(orc.binary(op, a5, np.full((1,), sc, np.float32)) == v)
    assert np.all(orc.binary("mul", np.full((1,), 2.0, np.float32), a5) == 10)
    x = np.arange(-2, 3, dtype=np.float32)
    assert orc.unary("sigmoid", x)[2] == 0.5 and orc.unary("tanh", x)[2] == 0
    assert orc.unary("gelu", x)[2] == 0 and orc.unary("silu", x)[2] == 0 and orc.unary("exp", np.zeros(1, np.float32))[0] == 1
    r = np.arange(1, 6, dtype=np.float32)
    assert [orc.reduce_all(op, r) for op in ("sum", "mean", "max", "min")] == [15, 3, 5, 1]
    m = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    np.testing.assert_array_equal(orc.reduce_dim("sum", m, 0), [5, 7, 9])
    np.testing.assert_array_equal(orc.reduce_dim("sum", m, 1, keepdim=True), [[6], [15]])
    np.testing.assert_array_equal(orc.reduce_dim("max", m, 1), [3, 6])


def test_shape_and_view_known_answers(orc):
    # tests/unit/test_shape.cpp:49-72 and tests/unit/test_tensor.cpp:45-69, 88-98
    assert orc.broadcast_shape((2, 1, 4), (3, 4)) == (2, 3, 4)
    with pytest.raises(ValueError):
        orc.broadcast_shape((2, 3, 4), (5, 4))
    t = orc.strided_copy(np.arange(6, dtype=np.float32), 0, [3, 2], [1, 3])   # transpose(0, 1) of [2, 3]
    np.testing.assert_array_equal(t.ravel(), [0, 3, 1, 4, 2, 5])
    f16 = orc.cast(np.arange(4, dtype=np.float32), "f16")
    np.testing.assert_array_equal(orc.cast(f16.view(np.float16), "f32"), np.arange(4, dtype=np.float32))


def test_binary_broadcast_and_strided_views_vs_numpy(orc):
    rng = np.random.default_rng(1)
    for sa, sb in [((4, 1, 5), (3, 1)), ((2, 3, 4), (4,)), ((1,), (7, 6)), ((5, 1), (1, 6)), ((2, 3), (2, 3))]:
        a = rng.standard_normal(sa).astype(np.float32)
        b = (rng.standard_normal(sb) + 3).astype(np.float32)
        for op, f in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)):
            np.testing.assert_array_equal(orc.binary(op, a, b), f(a, b))
    # non-contiguous views: a transposed [3, 4] view of a [4, 3] base with an offset, and a slice
    base = rng.standard_normal(40).astype(np.float32)
    va = (2, [3, 4], [1, 3])
    ref_a = np.lib.stride_tricks.as_strided(base[2:], (3, 4), (4, 12))
    vb = (5, [4], [2])
    ref_b = base[5::2][:4]
    np.testing.assert_array_equal(orc.binary("mul", base, base, va, vb), ref_a * ref_b)
    np.testing.assert_array_equal(orc.strided_copy(base, 2, [3, 4], [1, 3]), ref_a)
    # a 4-D permute
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    p = x.transpose(2, 0, 3, 1)
    np.testing.assert_array_equal(orc.strided_copy(x.ravel(), 0, list(p.shape), [s // 4 for s in p.strides]), p)


def test_unary_vs_float64(orc):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(4000) * 3).astype(np.float32)
    xd = x.astype(np.float64)
    ref = {"neg": -xd, "abs": np.abs(xd), "exp": np.exp(xd), "tanh": np.tanh(xd), "sigmoid": 1 / (1 + np.exp(-xd)),
           "gelu": 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3))),
           "silu": xd / (1 + np.exp(-xd))}
    for op, r in ref.items():
        np.testing.assert_allclose(orc.unary(op, x), r, rtol=3e-6, atol=1e-6, err_msg=op)
    xp = np.abs(x) + 1e-3
    np.testing.assert_allclose(orc.unary("log", xp), np.log(xp.astype(np.float64)), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(orc.unary("sqrt", xp), np.sqrt(xp))   # correctly rounded


def test_reductions_vs_numpy(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 50, 7)).astype(np.float32)
    assert orc.reduce_all("sum", x) == np.float32(x.astype(np.float64).sum())
    assert orc.reduce_all("mean", x) == np.float32(np.float32(x.astype(np.float64).sum()) / np.float32(x.size))
    assert orc.reduce_all("max", x) == x.max() and orc.reduce_all("min", x) == x.min()
    for d in range(3):
        np.testing.assert_array_equal(orc.reduce_dim("sum", x, d), x.astype(np.float64).sum(d).astype(np.float32))
        np.testing.assert_array_equal(orc.reduce_dim("mean", x, d), x.astype(np.float64).mean(d).astype(np.float32))
        np.testing.assert_array_equal(orc.reduce_dim("max", x, d), x.max(d))
        np.testing.assert_array_equal(orc.reduce_dim("min", x, d), x.min(d))
    y = x.copy()
    y[0, 0, 0] = np.nan                                                  # NaN never wins a comparison
    assert orc.reduce_all("max", y) == np.nanmax(y)


def test_cat_and_sum_to_shape_vs_numpy(orc):
    rng = np.random.default_rng(4)
    parts = [rng.standard_normal((2, k, 3)).astype(np.float32) for k in (1, 4, 2)]
    for d in (0, 1, 2, -1):
        ps = parts if d in (1,) else [rng.standard_normal((2, 3, 3)).astype(np.float32) for _ in range(3)]
        np.testing.assert_array_equal(orc.cat(ps, d), np.concatenate(ps, d))
    ids = [np.arange(5, dtype=np.int64), np.arange(3, dtype=np.int64)]
    np.testing.assert_array_equal(orc.cat(ids, 0), np.concatenate(ids))
    g = rng.standard_normal((4, 2, 3, 5)).astype(np.float32)
    for target in [(3, 5), (1, 5), (3, 1), (2, 1, 5), (1, 1), ()]:
        tgt = target if target else ()
        ref = g.astype(np.float64)
        lead = g.ndim - len(tgt)
        ref = ref.sum(tuple(range(lead))) if lead else ref
        for i, t in enumerate(tgt):
            if t == 1 and ref.shape[i] > 1:
                ref = ref.sum(i, keepdims=True)
        np.testing.assert_allclose(orc.sum_to_shape(g, tgt), ref.astype(np.float32).reshape(tgt), rtol=1e-6, atol=1e-6)


def test_casts_vs_numpy_and_torch(orc):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 3000),
                        np.array([0.0, -0.0, 65504, 65519, 65520, 1e9, -1e9, 2.0 ** -25, 2.0 ** -24 * 1.5,
                                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(orc.cast(x, "f16"), x.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(orc.cast(x, "bf16"), torch.from_numpy(x).to(torch.bfloat16).view(torch.int16)
                                  .numpy().view(np.uint16))
    nan = np.array([np.nan, -np.nan], np.float32)
    assert orc.cast(nan, "bf16").tolist() == [0x7FC0, 0xFFC0]          # the reference's canonical NaN
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)            # every f16 bit pattern
    fin = np.isfinite(h.view(np.float16))
    np.testing.assert_array_equal(orc.cast(h, "f32")[fin], h.view(np.float16)[fin].astype(np.float32))
    hb = h[~fin].astype(np.uint32)                                      # inf / NaN keep their payload
    np.testing.assert_array_equal(orc.cast(h[~fin], "f32").view(np.uint32),
                                  ((hb & 0x8000) << 16) | 0x7F800000 | ((hb & 0x3FF) << 13))
    bb = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    np.testing.assert_array_equal(orc.cast(bb, "f32", bf16_from=True).view(np.uint32), bb.astype(np.uint32) << 16)
    xi = (rng.standard_normal(1000) * 1e4).astype(np.float32)
    np.testing.assert_array_equal(orc.cast(xi, "i64"), xi.astype(np.int64))    # truncation toward zero
    np.testing.assert_array_equal(orc.cast(xi, "i32"), xi.astype(np.int32))
    iv = rng.integers(-2 ** 40, 2 ** 40, 1000)
    np.testing.assert_array_equal(orc.cast(iv, "f32"), iv.astype(np.float32))
    np.testing.assert_array_equal(orc.cast(iv, "i32"), iv.astype(np.int32))
    np.testing.assert_array_equal(orc.cast(iv.astype(np.int32), "i64"), iv.astype(np.int32).astype(np.int64))
    with pytest.raises(NotImplementedError):
        orc.cast(h, "bf16")                                            # f16 -> bf16 is not in the table


@pytest.mark.parametrize("E,k", [(4, 2), (3, 1)])
def test_moe_lm_step_vs_torch(orc, E, k):
    # MoETransformerLM: cross_entropy + total_aux_loss, backward through routers and experts,
    # clip and AdamW, against a float64 torch model (tests/unit/test_moe.cpp:190-240 trains this)
    vocab, d, L, H, f, B, S, coef = 64, 32, 2, 2, 48, 2, 16, 0.05
    rng = np.random.default_rng(40 + E)
    lay = torch_ref.layout(vocab, d, L, f, False, E)
    params = np.concatenate([(np.ones(s) if len(s) == 1 else rng.standard_normal(s) * 0.2).ravel()
                             for _, s in lay]).astype(np.float32)
    ids = rng.integers(0, vocab, B * S).astype(np.int64)
    tgt = np.roll(ids, -1)
    cfg = orc.make_config(vocab, d, L, H, f, S, n_experts=E, top_k=k, aux_coef=coef)
    assert orc.num_params(cfg) == params.size
    loss_t, norm_t, grads_t, new_t = torch_ref.lm_step(vocab, d, L, H, f, False, params, ids, tgt, B, S,
                                                        n_experts=E, top_k=k, aux_coef=coef)
    p = params.copy()
    res, grads, m, v, step = orc.lm_step(cfg, p, ids, tgt, B, S)
    assert res.aux_loss > 0
    assert abs(res.loss - loss_t) / abs(loss_t) < 1e-5
    assert abs(res.grad_norm - norm_t) / norm_t < 1e-4
    off = 0
    for name, shape in lay:
        n = int(np.prod(shape))
        # top-1 router gradients are rounding noise in fp32 (p / (p + 1e-9) cancels)
        tol = 2e-2 if (k == 1 and "router" in name) else 1e-4
        assert rel(grads[off:off + n], grads_t[off:off + n]) < tol, name
        off += n
    assert rel(p, new_t) < 1e-4


def test_moe_lm_step_forced_routing(orc):
    """The oracle's forced-routing control (orc_moe_set_routing), used to compare the device's MoE
    step on the device's own top-k: forcing the routing the routers chose (as the forward records
    it) reproduces the step bit for bit; forcing another valid routing matches the float64 torch
    model run on that routing (loss 1e-5, gradients 1e-4) and moves the loss and the aux loss."""
    vocab, d, L, H, f, B, S, coef, E, k = 64, 32, 2, 2, 48, 2, 16, 0.05, 4, 2
    rng = np.random.default_rng(77)
    lay = torch_ref.layout(vocab, d, L, f, False, E)
    params = np.concatenate([(np.ones(s) if len(s) == 1 else rng.standard_normal(s) * 0.2).ravel()
                             for _, s in lay]).astype(np.float32)
    ids = rng.integers(0, vocab, B * S).astype(np.int64)
    tgt = np.roll(ids, -1)
    cfg = orc.make_config(vocab, d, L, H, f, S, n_experts=E, top_k=k, aux_coef=coef)
    own = np.empty((L, B * S, k), np.int64)
    p0 = params.copy()
    res0, g0, _, _, _ = orc.lm_step(cfg, p0, ids, tgt, B, S, moe_route_out=own)
    p1 = params.copy()
    res1, g1, _, _, _ = orc.lm_step(cfg, p1, ids, tgt, B, S, moe_forced=own)
    assert res1.loss == res0.loss and res1.aux_loss == res0.aux_loss
    np.testing.assert_array_equal(g1, g0)
    np.testing.assert_array_equal(p1, p0)
    # another valid routing: each token's k experts drawn at random, in random order
    alt = np.stack([np.stack([rng.permutation(E)[:k] for _ in range(B * S)]) for _ in range(L)]).astype(np.int64)
    assert (alt != own).any()
    loss_t, norm_t, grads_t, new_t = torch_ref.lm_step(vocab, d, L, H, f, False, params, ids, tgt, B, S,
                                                        n_experts=E, top_k=k, aux_coef=coef, moe_forced=alt)
    p2 = params.copy()
    res2, g2, _, _, _ = orc.lm_step(cfg, p2, ids, tgt, B, S, moe_forced=alt)
    assert abs(res2.loss - loss_t) / abs(loss_t) < 1e-5
    assert abs(res2.grad_norm - norm_t) / norm_t < 1e-4
    assert rel(g2, grads_t) < 1e-4 and rel(p2, new_t) < 1e-4
    assert abs(res2.loss - res0.loss) > 1e-4 and res2.aux_loss != res0.aux_loss


def _qlora_case(rng, vocab, d, L, f, r, b_std):
    lay = torch_ref.layout(vocab, d, L, f, False)
    base = np.concatenate([(np.ones(s) if len(s) == 1 else rng.standard_normal(s) * 0.2).ravel()
                           for _, s in lay]).astype(np.float32)
    lora = np.concatenate([(rng.standard_normal(s) * (b_std if "lora_B" in n else 0.2)).ravel()
                           for n, s in torch_ref.lora_layout(d, L, f, r)]).astype(np.float32)
    return lay, base, lora


def test_qlora_base_round_trip_matches_numpy(orc):
    # the seven projections of every layer become their INT4 round trip (fp16 scales); embeddings,
    # norms and the head stay as they are
    vocab, d, L, f, G = 64, 32, 2, 48, 16
    rng = np.random.default_rng(77)
    lay, base, _ = _qlora_case(rng, vocab, d, L, f, 4, 0.0)
    cfg = orc.make_config(vocab, d, L, 2, f, 16)
    out = orc.qlora_dequantize_base(cfg, G, base)
    off = 0
    for name, shape in lay:
        n = int(np.prod(shape))
        want = base[off:off + n]
        if any(p + ".weight" in name for p in torch_ref.PROJ):
            want = torch_ref.int4_round_trip(want, G)
            assert not np.array_equal(want, base[off:off + n])
        np.testing.assert_array_equal(out[off:off + n], want, err_msg=name)
        off += n


def test_qlora_zero_b_is_the_quantized_dense_model(orc):
    # LoRA B = 0 (the reference's initialisation, tests/unit/test_lora.cpp:58-73): the loss is the
    # dense model's on the dequantized base, bit for bit, and every lora_A gradient is zero
    vocab, d, L, H, f, B, S, r, G = 64, 32, 2, 2, 48, 2, 16, 4, 32
    rng = np.random.default_rng(78)
    lay, base, lora = _qlora_case(rng, vocab, d, L, f, r, 0.0)
    ids = rng.integers(0, vocab, B * S).astype(np.int64)
    tgt = np.roll(ids, -1)
    cfg = orc.make_config(vocab, d, L, H, f, S)
    dense = orc.qlora_dequantize_base(cfg, G, base)
    want = orc.lm_loss(cfg, dense, ids, tgt, B, S)
    res, grads, _, _, _ = orc.qlora_step(cfg, r, 8.0, G, base, lora.copy(), ids, tgt, B, S, do_update=False)
    assert res.loss == want
    off = 0
    for name, shape in torch_ref.lora_layout(d, L, f, r):
        n = int(np.prod(shape))
        if "lora_A" in name:
            assert not grads[off:off + n].any(), name
        else:
            assert np.abs(grads[off:off + n]).max() > 0, name
        off += n


@pytest.mark.parametrize("r,alpha,G", [(4, 8.0, 32), (8, 32.0, 16)])
def test_qlora_lm_step_vs_torch(orc, r, alpha, G):
    # frozen INT4 base + LoRA on all seven projections: loss, global norm, every adapter gradient
    # and the AdamW update against a float64 torch model with an independent INT4 round trip
    vocab, d, L, H, f, B, S = 64, 32, 2, 2, 48, 2, 16
    rng = np.random.default_rng(80 + r)
    lay, base, lora = _qlora_case(rng, vocab, d, L, f, r, 0.1)
    ids = rng.integers(0, vocab, B * S).astype(np.int64)
    tgt = np.roll(ids, -1)
    cfg = orc.make_config(vocab, d, L, H, f, S)
    assert orc.qlora_num_params(cfg, r) == lora.size
    loss_t, norm_t, grads_t, new_t = torch_ref.lm_step(vocab, d, L, H, f, False, base, ids, tgt, B, S,
                                                        lora=(lora, r, alpha, G))
    p = lora.copy()
    res, grads, m, v, step = orc.qlora_step(cfg, r, alpha, G, base, p, ids, tgt, B, S)
    assert step == 1
    assert abs(res.loss - loss_t) / abs(loss_t) < 1e-5
    assert abs(res.grad_norm - norm_t) / norm_t < 1e-4
    off = 0
    for name, shape in torch_ref.lora_layout(d, L, f, r):
        n = int(np.prod(shape))
        assert rel(grads[off:off + n], grads_t[off:off + n]) < 1e-4, name
        off += n
    assert rel(p, new_t) < 1e-4


def test_lm_logits_match_the_step_loss(orc):
    # the forward-only logits give the step's cross-entropy
    vocab, d, L, H, f, B, S = 64, 32, 2, 2, 48, 2, 16
    rng = np.random.default_rng(90)
    lay = torch_ref.layout(vocab, d, L, f, False)
    params = np.concatenate([(np.ones(s) if len(s) == 1 else rng.standard_normal(s) * 0.2).ravel()
                             for _, s in lay]).astype(np.float32)
    ids = rng.integers(0, vocab, B * S).astype(np.int64)
    tgt = np.roll(ids, -1)
    cfg = orc.make_config(vocab, d, L, H, f, S)
    lg = orc.lm_logits(cfg, params, ids, B, S).reshape(B * S, vocab).astype(np.float64)
    lse = np.log(np.exp(lg - lg.max(1, keepdims=True)).sum(1)) + lg.max(1)
    ce = float(np.mean(lse - lg[np.arange(B * S), tgt]))
    assert abs(ce - orc.lm_loss(cfg, params, ids, tgt, B, S)) < 1e-5 * ce
