"""KV-cached inference on the GPU (aic_lm_forward_step / aic_lm_generate): prefill logits
against the oracle's forward, the reference's KVCacheAutoregressiveParity
(tests/unit/test_model.cpp:130-167: token-by-token cached logits equal the parallel forward at
1e-4), chunked continuation, batches, the MoE and QLoRA models, and generate's greedy path
against argmax chains of the oracle."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

import autonomousaicore_amd as aic  # noqa: E402
from tests.gpu_util import rel  # noqa: E402
from tests.test_gpu_step import TINY, build, build_moe, build_qlora, make_base, make_lora, make_params, oracle_cfg  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def test_prefill_matches_oracle_forward(orc):
    B, S = 2, 40
    m = build(TINY, max_seq=64)
    params = make_params(m, 31, std=0.05)
    m.set_params(params)
    ids, _ = aic.batch(5, B, S, TINY["vocab"])
    got = m.forward_step(ids, 0)
    ref = orc.lm_logits(oracle_cfg(orc, TINY, 64), params, ids, B, S)
    assert rel(got, ref) < 1e-5
    m.close()


@pytest.mark.parametrize("compute,tol", [("float32", 1e-4), ("bfloat16", 3e-2)])
def test_cached_steps_equal_the_parallel_forward(compute, tol):
    cfg = dict(vocab=512, d=128, L=2, H=2, f=256, tied=False)  # head_dim 64
    m = build(cfg, compute=compute, max_seq=64)
    m.set_params(make_params(m, 41, std=0.05))
    ids, _ = aic.batch(9, 3, 24, cfg["vocab"])
    full = m.forward_step(ids, 0)
    # token by token (the reference's prefill of generate), then chunks of 5 and 3 at offsets
    steps = np.concatenate([m.forward_step(ids[:, p:p + 1], p) for p in range(ids.shape[1])], axis=1)
    assert rel(steps, full) < tol
    assert np.abs(steps[:, -1] - full[:, -1]).max() < (1e-4 if compute == "float32" else 0.1)
    first = m.forward_step(ids[:, :16], 0)
    rest = np.concatenate([m.forward_step(ids[:, 16:21], 16), m.forward_step(ids[:, 21:], 21)], axis=1)
    assert rel(first, full[:, :16]) < tol and rel(rest, full[:, 16:]) < tol
    with pytest.raises(aic.AicError):
        m.forward_step(ids[:1, :1], 24)                 # a continuation must keep its batch size
    with pytest.raises(aic.AicError):
        m.forward_step(ids[:, :1], 64)                  # past max_seq_len
    m.close()


def test_moe_and_qlora_decode():
    cfg = dict(TINY, tied=False)
    ids, _ = aic.batch(3, 1, 20, cfg["vocab"])
    moe = build_moe(cfg, 4, 2, 0.01)
    moe.set_params(make_params(moe, 7, std=0.05))
    full = moe.forward_step(ids, 0)
    steps = np.concatenate([moe.forward_step(ids[:, p:p + 1], p) for p in range(20)], axis=1)
    assert rel(steps, full) < 1e-4
    moe.close()
    q = build_qlora(cfg, 16, 32.0, 128)
    q.set_base_params(make_base(q, 8))
    q.set_params(make_lora(q, 9, 0.02))
    full = q.forward_step(ids, 0)
    steps = np.concatenate([q.forward_step(ids[:, p:p + 1], p) for p in range(20)], axis=1)
    assert rel(steps, full) < 1e-4
    q.close()


def test_generate_greedy_follows_the_oracle_argmax(orc):
    m = build(TINY, max_seq=64)
    params = make_params(m, 53, std=0.08)
    m.set_params(params)
    prompt = [3, 7, 15]
    out = m.generate(prompt, 12, temperature=0.0)
    assert out[:3] == prompt and len(out) == 15
    seq = list(prompt)
    ocfg = oracle_cfg(orc, TINY, 64)
    for _ in range(12):
        lg = orc.lm_logits(ocfg, params, np.array(seq), 1, len(seq))[0, -1]
        seq.append(int(np.argmax(lg)))
    assert out == seq
    # top_k == 1 is greedy; a tiny top_p keeps only the most likely token; seeds reproduce
    assert m.generate(prompt, 12, temperature=0.8, top_k=1) == seq
    assert m.generate(prompt, 12, temperature=0.8, top_p=1e-6) == seq
    a = m.generate(prompt, 12, temperature=1.0, top_k=50, top_p=0.9, seed=5)
    assert a == m.generate(prompt, 12, temperature=1.0, top_k=50, top_p=0.9, seed=5)
    assert all(0 <= t < TINY["vocab"] for t in a)
    # eos stops the loop right after the token; an empty prompt starts from token 0
    stop = seq[5]
    e = m.generate(prompt, 12, temperature=0.0, eos_token_id=stop)
    assert e == seq[:6]
    assert m.generate([], 3, temperature=0.0)[0] == 0
    m.close()
