"""Every BASELINE configuration at its real widths on the GPU (through the aic_lm_* C-ABI).

Two kinds of check per configuration:

* parity -- the configuration's true d / heads / FFN / vocab with 2 layers and one sequence
  (the 1B widths also at the timed B 4 x S 2048), one bf16 AMP step against the fp32 CPU oracle
  on identical weights and ids (the reference's "AMP" computes in fp32, so the bf16 step is
  judged against the fp32 step): loss within 1e-2 relative; the global
  gradient norm and every gradient tensor (per-tensor relative L2) within tolerances set per
  configuration near twice the errors the GPU shows (both sides are deterministic; bf16
  activations and operand rounding give worst tensors of 1.3e-2 - 1.6e-2); the MoE step is
  compared on the device's own top-k selection;
* full size -- the whole configuration (all layers, the configured batch and sequence) with
  its optimizer (AdamW lr 3e-4, betas 0.9/0.95, wd 0.1, clip 1.0, loss scale 2^16):
  the forward loss of one sequence at full depth against the oracle within 1e-2; the first
  update equal to the oracle's AdamW (src/optim/adamw.cpp:68-84) applied to the device's
  gradients with the device's unscale-and-clip multiplier (1e-6 per tensor); three steps
  with finite losses and the loss scale kept at 2^16 (no overflow); a second model from the
  same seed reproducing the first step bit for bit (loss, norm and every parameter); and
  the loss falling over three steps on one batch at lr 1e-5.  At lr 3e-4 the reference's
  own first step raises the loss at these widths (its fp32 CPU step at the 1B widths with
  2 layers and one sequence: 10.98 -> 12.37 -> 11.34; Adam's first update moves every
  weight by lr), so "the loss falls" is a property of a small step, not of this config.

The reference's whole-model test is tests/unit/test_model.cpp:95-128 over
src/models/transformer_lm.cpp:14-62 (dense), src/models/moe_transformer_lm.cpp:56-66 (MoE)
and src/nn/lora.cpp:116-175 with src/nn/quantization.cpp:669-679 (QLoRA)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

import autonomousaicore_amd as aic  # noqa: E402
from tests.gpu_util import rel  # noqa: E402

ADAMW = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)

# BASELINE.json configs[1..4]
C125M = dict(vocab=32000, d=768, L=12, H=12, f=2048, B=8, S=1024)
C1B = dict(vocab=32000, d=2048, L=16, H=16, f=5632, B=4, S=2048)
CMOE = dict(vocab=32000, d=1024, L=12, H=16, f=2816, B=8, S=1024, E=8, k=2, coef=0.01)
CQLORA = dict(C1B, r=16, alpha=32.0, G=128)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _train(lr):
    return aic.TrainingConfig(adamw=aic.AdamWOptions(**dict(ADAMW, lr=lr)), max_grad_norm=1.0, use_amp=True)


def build_dense(c, L=None, lr=3e-4):
    cfg = aic.TransformerLMConfig(vocab_size=c["vocab"], hidden_dim=c["d"], num_layers=L or c["L"], num_heads=c["H"],
                                  intermediate_dim=c["f"], max_seq_len=c["S"], rms_norm_eps=1e-6, compute="bfloat16")
    return aic.TransformerLM(cfg, _train(lr))


def build_moe(c, L=None, lr=3e-4):
    cfg = aic.MoETransformerLMConfig(vocab_size=c["vocab"], hidden_dim=c["d"], num_layers=L or c["L"],
                                     num_heads=c["H"], intermediate_dim=c["f"], max_seq_len=c["S"], rms_norm_eps=1e-6,
                                     compute="bfloat16", num_experts=c["E"], top_k=c["k"], aux_loss_coef=c["coef"])
    return aic.TransformerLM(cfg, _train(lr))


def build_qlora(c, L=None, lr=3e-4):
    cfg = aic.QLoRATransformerLMConfig(vocab_size=c["vocab"], hidden_dim=c["d"], num_layers=L or c["L"],
                                       num_heads=c["H"], intermediate_dim=c["f"], max_seq_len=c["S"],
                                       rms_norm_eps=1e-6, compute="bfloat16", lora_rank=c["r"],
                                       lora_alpha=c["alpha"], quant_group=c["G"])
    return aic.TransformerLM(cfg, _train(lr))


def oracle_cfg(orc, c, L=None, S=None, moe=False):
    kw = dict(n_experts=c["E"], top_k=c["k"], aux_coef=c["coef"]) if moe else {}
    return orc.make_config(c["vocab"], c["d"], L or c["L"], c["H"], c["f"], S or c["S"], norm_eps=1e-6, **kw)


def normal_params(layout, seed, std=0.02):
    """N(0, std) for matrices, ones for norms (BASELINE: weights N(0, 0.02), norms 1)."""
    out = []
    for i, (name, shape, off) in enumerate(layout):
        n = int(np.prod(shape))
        out.append(np.ones(n, np.float32) if len(shape) == 1 else aic.normal(seed + 7919 * i, n, 0.0, std))
    return np.concatenate(out)


def lora_params(layout, seed, b_std=0.02):
    out = []
    for i, (name, shape, off) in enumerate(layout):
        n = int(np.prod(shape))
        out.append(aic.normal(seed + 104729 * i, n, 0.0, b_std if "lora_B" in name else 0.02))
    return np.concatenate(out)


def check_grads(model, got, ref, tol, expert_tol=None):
    """Per-tensor relative L2 error below tol.  With expert_tol (MoE), each expert's tensors are
    held to expert_tol and each layer's experts taken together to tol: at a near-tie of two
    router logits the bf16 step can route a token to another expert than the fp32 oracle does,
    which moves that token's whole contribution from one expert's gradient to another's."""
    worst = ("", 0.0)
    layer_experts = {}
    for name, shape, off in model.layout:
        n = int(np.prod(shape))
        r = rel(got[off:off + n], ref[off:off + n])
        if r > worst[1]:
            worst = (name, r)
        if expert_tol is not None and ".moe.experts." in name:
            assert r < expert_tol, f"grad {name}: rel {r:.3g}"
            layer = name.split(".moe.")[0]
            layer_experts.setdefault(layer, []).append((off, n))
        else:
            assert r < tol, f"grad {name}: rel {r:.3g}"
    for layer, parts in layer_experts.items():
        g = np.concatenate([got[o:o + n] for o, n in parts])
        rf = np.concatenate([ref[o:o + n] for o, n in parts])
        r = rel(g, rf)
        print(f"  {layer} experts together: rel {r:.3g}")
        assert r < tol, f"grad {layer} experts: rel {r:.3g}"
    print(f"  worst gradient tensor {worst[0]}: rel {worst[1]:.3g}")
    return worst


def grad_multiplier(st):
    """The factor AdamW applies to the loss-scaled gradients: 1/scale, times the clip coefficient
    max_norm / (norm + 1e-6) when that is below 1 (float32, as the device computes it)."""
    inv = np.float32(1.0) / np.float32(st.loss_scale)
    coef = np.float32(1.0) / (np.float32(st.grad_norm) + np.float32(1e-6))
    return inv * coef if coef < 1 else inv


def check_step_vs_oracle(st, res, grads, g_ref, model, grad_tol, norm_tol, expert_tol=None, tag=""):
    """bf16 AMP step against the fp32 oracle step: loss within 1e-2, the
    gradient norm within norm_tol and every gradient tensor within grad_tol (per-tensor relative
    L2), both set per configuration near twice the errors observed on the GPU."""
    loss_rel = abs(st.loss - res.loss) / abs(res.loss)
    norm_rel = abs(st.grad_norm - res.grad_norm) / res.grad_norm
    print(f"  loss {st.loss:.6f} vs oracle {res.loss:.6f} (rel {loss_rel:.2e}); "
          f"grad norm {st.grad_norm:.5f} vs {res.grad_norm:.5f} (rel {norm_rel:.2e})")
    assert loss_rel < 1e-2
    assert st.loss_scale == 65536.0 and not st.found_inf
    # the device keeps the loss-scaled, unclipped gradients; the oracle returns them clipped
    worst = check_grads(model, grads * grad_multiplier(st), g_ref, grad_tol, expert_tol)
    print(f"PARITY {tag}: loss_rel {loss_rel:.3e} norm_rel {norm_rel:.3e} worst_grad {worst[0]} {worst[1]:.3e}")
    assert norm_rel < norm_tol


def check_first_update(orc, model, p0, g, p1, st, names):
    """p1 = AdamW step 1 (the reference's update order) from p0 with the device's gradients times
    the device's multiplier, on the named tensors (AdamW is elementwise)."""
    mult = grad_multiplier(st)
    names = {n for n, _, _ in model.layout} if names is None else set(names)
    assert names <= {n for n, _, _ in model.layout}, names
    for name, shape, off in model.layout:
        if name not in names:
            continue
        n = int(np.prod(shape))
        p = p0[off:off + n].copy()
        gm = (g[off:off + n] * mult).astype(np.float32)
        m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
        orc.adamw(p, gm, m, v, ADAMW["lr"], ADAMW["beta1"], ADAMW["beta2"], ADAMW["eps"], ADAMW["weight_decay"], 1)
        r = rel(p1[off:off + n], p)
        assert r < 1e-6, f"update of {name}: rel {r:.3g}"


def full_size_properties(orc, make, init, c, oracle_loss_of_first_sequence, update_names):
    """The full configuration: full-depth loss of one sequence against the oracle, the first
    update against the oracle's AdamW, three steps, a bit-identical rerun of the first step, and
    the loss falling over three steps at a small learning rate."""
    B, S = c["B"], c["S"]
    ids, tgt = aic.batch(1234, B, S, c["vocab"], dist="zipf")
    model = make(3e-4)
    init(model)
    loss0 = model.eval_loss(ids[:1], tgt[:1], 1, S)
    ref0 = oracle_loss_of_first_sequence(model, ids[:1], tgt[:1])
    print(f"  first sequence at full depth: loss {loss0:.6f} vs oracle {ref0:.6f}")
    assert abs(loss0 - ref0) / abs(ref0) < 1e-2
    p0 = model.get_params()
    stats = [model.train_step(ids, tgt, B, S)]
    g1, p1 = model.get_grads(), model.get_params()
    check_first_update(orc, model, p0, g1, p1, stats[0], update_names)
    del p0, g1
    stats += [model.train_step(ids, tgt, B, S) for _ in range(2)]
    model.close()
    print("  lr 3e-4: losses", [round(s.loss, 5) for s in stats], "norms", [round(s.grad_norm, 4) for s in stats])
    for s in stats:
        assert np.isfinite(s.loss) and np.isfinite(s.grad_norm)
        assert not s.found_inf and s.loss_scale == 65536.0
    assert [s.step for s in stats] == [1, 2, 3]

    again = make(3e-4)
    init(again)
    st = again.train_step(ids, tgt, B, S)
    assert st.loss == stats[0].loss and st.grad_norm == stats[0].grad_norm
    assert np.array_equal(again.get_params(), p1)
    again.close()
    del p1

    slow = make(1e-5)
    init(slow)
    losses = [slow.train_step(ids, tgt, B, S).loss for _ in range(3)]
    slow.close()
    print("  lr 1e-5: losses", [round(x, 5) for x in losses])
    assert losses[0] > losses[1] > losses[2]
    return stats


# ----------------------------------------------------------------------------- 125M
def test_125m_residual_scaling_init():
    """init_normal(residual_scaling=True): out_proj and down_proj ~ N(0, 0.02/sqrt(2L)), the other
    matrices N(0, 0.02) and unchanged by the flag, norms 1 (configs[1]'s initialisation)."""
    c = C125M
    m = build_dense(c)
    m.init_normal(5678, 0.02, residual_scaling=True)
    scaled = m.get_params()
    m.init_normal(5678, 0.02, residual_scaling=False)
    plain = m.get_params()
    layout = m.layout
    m.close()
    rs = 1.0 / np.sqrt(2.0 * c["L"])
    n_resid = 0
    for name, shape, off in layout:
        n = int(np.prod(shape))
        a, b = scaled[off:off + n], plain[off:off + n]
        if len(shape) == 1:
            assert (a == 1.0).all() and (b == 1.0).all(), name
        elif "out_proj" in name or "down_proj" in name:
            n_resid += 1
            np.testing.assert_allclose(a, b * rs, rtol=1e-6, atol=0, err_msg=name)
            assert abs(a.std() / (0.02 * rs) - 1.0) < 0.01, name
        else:
            np.testing.assert_array_equal(a, b, err_msg=name)
            assert abs(a.std() / 0.02 - 1.0) < 0.01, name
    assert n_resid == 2 * c["L"]


def test_125m_full_config(orc):
    """12 layers, d 768, 12 heads of 64, SwiGLU 2048, vocab 32000, B 8 x S 1024, bf16
    AMP, residual projections scaled by 1/sqrt(2*12)."""
    c = C125M

    def oracle_loss(model, ids, tgt):
        return orc.lm_loss(oracle_cfg(orc, c), model.get_params(), ids, tgt, 1, c["S"])

    full_size_properties(orc, lambda lr: build_dense(c, lr=lr),
                         lambda m: m.init_normal(5678, 0.02, residual_scaling=True), c, oracle_loss,
                         {"tok_embeddings.weight", "layers.5.attn.out_proj.weight", "norm.weight", "lm_head.weight"})


# ----------------------------------------------------------------------------- 1B
def test_1b_widths_step_matches_oracle(orc):
    """configs[2]'s widths (d 2048, 16 heads of 128, SwiGLU 5632, vocab 32000) with 2 layers and
    one sequence of 2048 tokens: one bf16 AMP step against the fp32 oracle step."""
    c = C1B
    S = c["S"]
    model = build_dense(c, L=2)
    params = normal_params(model.layout, 5678)
    model.set_params(params)
    ids, tgt = aic.batch(1234, 1, S, c["vocab"], dist="zipf")
    st = model.train_step(ids, tgt, 1, S)
    grads = model.get_grads()
    res, g_ref, _, _, _ = orc.lm_step(oracle_cfg(orc, c, L=2), params.copy(), ids, tgt, 1, S)
    check_step_vs_oracle(st, res, grads, g_ref, model, grad_tol=3.5e-2, norm_tol=4e-4, tag="1b-widths B1xS2048")
    model.close()


def test_1b_widths_timed_shape_matches_oracle(orc):
    """configs[2]'s widths with 2 layers at the timed shape, B 4 x S 2048 (T 8192): the products run
    the dispatch of the measured step (the 256x256 persistent kernels with the residual, RoPE and
    SwiGLU epilogues, the grouped weight gradients over K 8192, the lm_head over 4000 tiles), one
    bf16 AMP step against the fp32 oracle step on identical weights and ids
    (tests/unit/test_model.cpp:95-128 is the reference's whole-model test)."""
    c = C1B
    B, S = c["B"], c["S"]
    model = build_dense(c, L=2)
    params = normal_params(model.layout, 4242)
    model.set_params(params)
    ids, tgt = aic.batch(777, B, S, c["vocab"], dist="zipf")
    st = model.train_step(ids, tgt, B, S)
    grads = model.get_grads()
    model.close()
    res, g_ref, _, _, _ = orc.lm_step(oracle_cfg(orc, c, L=2), params.copy(), ids, tgt, B, S)
    check_step_vs_oracle(st, res, grads, g_ref, model, grad_tol=3e-2, norm_tol=5e-5, tag="1b-widths B4xS2048")


def test_1b_widths_fused_grad_norm_equals_pass():
    """The step's gradient norm formed from the producers' partial sums (the weight-gradient
    GEMMs' epilogues, the split-K reduction of the grouped launch's carved tiles, then the
    embedding and norm weights) against the pass over every gradient, at configs[2]'s widths with
    2 layers: the same loss and gradients bit for bit, the norm within 1e-6 (the same fp64 sum of
    fp32 squares in another order), the same update within 1e-6 -- then a second step of 1000
    tokens, where the weight gradients leave the tile kernels (K not a multiple of 64) and other
    slots are written; a NaN in one weight is flagged by both forms and the step skipped with
    the parameters unchanged."""
    c = C1B
    S = c["S"]
    ids, tgt = aic.batch(1234, 1, S, c["vocab"], dist="zipf")
    ids2, tgt2 = aic.batch(4321, 1, 1000, c["vocab"], dist="zipf")
    out = {}
    for fused in (True, False):
        model = build_dense(c, L=2)
        assert model.fused_grad_norm(fused) == fused
        params = normal_params(model.layout, 5678)
        model.set_params(params)
        st = model.train_step(ids, tgt, 1, S)
        first = (st, model.get_grads(), model.get_params())
        st2 = model.train_step(ids2, tgt2, 1, 1000)
        out[fused] = (first, (st2, model.get_grads(), model.get_params()))
        model.close()
    for k in range(2):
        (sf, gf, pf), (sp, gp, pp) = out[True][k], out[False][k]
        print(f"  step {k + 1}: grad norm fused {sf.grad_norm!r} pass {sp.grad_norm!r}")
        assert not sf.found_inf and not sp.found_inf
        if k == 0:
            assert sf.loss == sp.loss
            np.testing.assert_array_equal(gf, gp)
        else:  # the weights differ by the first update's rounding
            assert abs(sf.loss - sp.loss) <= 1e-5 * abs(sp.loss) and rel(gf, gp) < 1e-4
        assert abs(sf.grad_norm - sp.grad_norm) <= (1e-6 if k == 0 else 1e-4) * sp.grad_norm
        assert rel(pf, pp) < 1e-6

    bad = params.copy()
    off = [e for e in model.layout if e[0] == "layers.1.norm2.weight"][0][2]
    bad[off + 5] = np.nan
    for fused in (True, False):
        model = build_dense(c, L=2)
        model.fused_grad_norm(fused)
        model.set_params(bad)
        st = model.train_step(ids, tgt, 1, S)
        assert st.found_inf and st.step == 0 and st.loss_scale == 65536.0
        np.testing.assert_array_equal(model.get_params(), bad)
        model.close()


def test_large_vocab_head_fused_grad_norm():
    """A 128k-vocabulary untied head at d_model 3072: its weight-gradient launch has 501 x 12 =
    6012 blocks of 256x256, each writing one partial-sum slot, more than a fixed 4096-slot region
    held.  The slot regions are sized from the producers' bounds at construction, so the fused
    gradient norm runs and equals the pass over every gradient (gradients bit for bit, the norm
    within 1e-6)."""
    c = dict(vocab=128256, d=3072, L=1, H=24, f=1024, S=256)
    ids, tgt = aic.batch(99, 1, c["S"], c["vocab"], dist="zipf")
    out = {}
    for fused in (True, False):
        model = build_dense(c)
        assert model.fused_grad_norm(fused) == fused
        model.init_normal(5678, 0.02)
        st = model.train_step(ids, tgt, 1, c["S"])
        out[fused] = (st, model.get_grads())
        model.close()
    (sf, gf), (sp, gp) = out[True], out[False]
    print(f"  grad norm fused {sf.grad_norm!r} pass {sp.grad_norm!r}")
    assert not sf.found_inf and not sp.found_inf and sf.loss == sp.loss
    np.testing.assert_array_equal(gf, gp)
    assert abs(sf.grad_norm - sp.grad_norm) <= 1e-6 * sp.grad_norm


def test_1b_full_config(orc):
    """configs[2] at full size: 16 layers, B 4 x S 2048, N(0, 0.02) weights, bf16 AMP, clip 1.0."""
    c = C1B

    def oracle_loss(model, ids, tgt):
        return orc.lm_loss(oracle_cfg(orc, c), model.get_params(), ids, tgt, 1, c["S"])

    full_size_properties(orc, lambda lr: build_dense(c, lr=lr), lambda m: m.init_normal(5678, 0.02), c, oracle_loss,
                         {"tok_embeddings.weight", "layers.7.attn.q_proj.weight", "layers.15.ffn.down_proj.weight",
                          "norm.weight", "lm_head.weight"})


# ----------------------------------------------------------------------------- MoE
def test_moe_widths_step_matches_oracle(orc):
    """configs[3]'s widths (d 1024, 16 heads of 64, 8 SwiGLU experts of 2816, top-2, aux 0.01,
    vocab 32000) with 2 layers and one sequence of 1024 tokens, against the fp32 oracle."""
    c = CMOE
    S = c["S"]
    model = build_moe(c, L=2)
    params = normal_params(model.layout, 2024)
    model.set_params(params)
    ids, tgt = aic.batch(99, 1, S, c["vocab"], dist="zipf")
    st = model.train_step(ids, tgt, 1, S)
    grads = model.get_grads()
    # The oracle runs on the device's top-k selection (orc_moe_set_routing): with bf16 router logits
    # a near-tie can send a token to another expert than the fp32 router would (for this seed about
    # 30 of the 1024 Zipf tokens sit at a bf16-resolved tie between experts 0 and 2 in layer 0),
    # which moves its whole contribution between experts' gradients; on the same routing every
    # expert tensor is held to the dense tolerance.
    routing = np.stack([model.moe_routing(l) for l in range(2)])
    model.close()
    own = np.empty_like(routing)
    orc.lm_step(oracle_cfg(orc, c, L=2, moe=True), params.copy(), ids, tgt, 1, S, moe_route_out=own)
    print(f"  tokens routed differently from the fp32 router: {int((np.sort(own, -1) != np.sort(routing, -1)).any(-1).sum())}"
          f" of {routing.shape[0] * routing.shape[1]}")
    res, g_ref, _, _, _ = orc.lm_step(oracle_cfg(orc, c, L=2, moe=True), params.copy(), ids, tgt, 1, S,
                                      moe_forced=routing)
    print(f"  aux {st.aux_loss:.6f} vs oracle {res.aux_loss:.6f}")
    assert abs(st.aux_loss - res.aux_loss) < 3e-2 * abs(res.aux_loss)
    check_step_vs_oracle(st, res, grads, g_ref, model, grad_tol=3e-2, norm_tol=1e-3, tag="moe-widths B1xS1024")


def test_moe_widths_fused_grad_norm_equals_pass():
    """The fused gradient norm with MoE FFNs (the experts' down and gate/up weight gradients from
    expert-ragged GEMMs, the router's from a split-K GEMM, each writing its partial sums) against
    the pass over every gradient, at configs[3]'s widths with 2 layers: the same loss and
    gradients bit for bit, the norm within 1e-6."""
    c = CMOE
    S = c["S"]
    ids, tgt = aic.batch(99, 1, S, c["vocab"], dist="zipf")
    out = {}
    for fused in (True, False):
        model = build_moe(c, L=2)
        assert model.fused_grad_norm(fused) == fused
        model.set_params(normal_params(model.layout, 2024))
        st = model.train_step(ids, tgt, 1, S)
        out[fused] = (st, model.get_grads())
        model.close()
    (sf, gf), (sp, gp) = out[True], out[False]
    print(f"  grad norm fused {sf.grad_norm!r} pass {sp.grad_norm!r}")
    assert sf.loss == sp.loss and not sf.found_inf and not sp.found_inf
    np.testing.assert_array_equal(gf, gp)
    assert abs(sf.grad_norm - sp.grad_norm) <= 1e-6 * sp.grad_norm


def test_moe_full_config(orc):
    """configs[3] at full size: 12 layers, B 8 x S 1024, every FFN 8 experts top-2."""
    c = CMOE

    def oracle_loss(model, ids, tgt):
        return orc.lm_loss(oracle_cfg(orc, c, moe=True), model.get_params(), ids, tgt, 1, c["S"])

    stats = full_size_properties(orc, lambda lr: build_moe(c, lr=lr), lambda m: m.init_normal(5678, 0.02), c,
                                 oracle_loss, {"tok_embeddings.weight", "layers.3.moe.router.gate.weight",
                                               "layers.5.moe.experts.6.up_proj.weight",
                                               "layers.11.attn.v_proj.weight", "lm_head.weight"})
    # per layer aux = coef * E * sum_e f_e P_e with sum f = sum P = 1, so 0 < aux <= coef * E
    assert all(0.0 < s.aux_loss <= c["coef"] * c["E"] * c["L"] for s in stats)


# ----------------------------------------------------------------------------- QLoRA
def test_qlora_1b_widths_step_matches_oracle(orc):
    """configs[4]'s widths (the 1B shape, INT4 base with groups of 128 and fp16 scales, rank 16,
    alpha 32 on all seven projections) with 2 layers and one sequence of 2048 tokens."""
    c = CQLORA
    S = c["S"]
    model = build_qlora(c, L=2)
    base = normal_params(model.base_layout, 61)
    lora = lora_params(model.layout, 67)
    model.set_base_params(base)
    model.set_params(lora)
    ids, tgt = aic.batch(71, 1, S, c["vocab"], dist="zipf")
    st = model.train_step(ids, tgt, 1, S)
    grads = model.get_grads()
    res, g_ref, _, _, _ = orc.qlora_step(oracle_cfg(orc, c, L=2), c["r"], c["alpha"], c["G"], base, lora.copy(),
                                         ids, tgt, 1, S)
    # the norm's relative error is second order in the per-element bf16 noise (about half the
    # squared relative error of the dominant gradient tensors, 1.5e-2 here, so up to ~1.2e-4);
    # observed 1.8e-5 with GEMM adapter products and 5.2e-5 with the one-pass ones (another,
    # equally exact summation order)
    check_step_vs_oracle(st, res, grads, g_ref, model, grad_tol=3.5e-2, norm_tol=1.2e-4, tag="qlora-widths B1xS2048")
    model.close()


def test_qlora_full_config(orc):
    """configs[4] at full size: 16 layers, B 4 x S 2048; base N(0, 0.02) quantized to INT4, adapters
    A ~ N(0, 0.02) and B = 0, so the first step moves only B and the loss starts at the base's."""
    c = CQLORA

    def oracle_loss(model, ids, tgt):
        # with B = 0 the adapted model is the dense model on the INT4 round trip of the base
        ocfg = oracle_cfg(orc, c)
        base = model.get_base_params()
        return orc.lm_loss(ocfg, orc.qlora_dequantize_base(ocfg, c["G"], base), ids, tgt, 1, c["S"])

    full_size_properties(orc, lambda lr: build_qlora(c, lr=lr), lambda m: m.init_normal(5678, 0.02), c, oracle_loss,
                         None)
