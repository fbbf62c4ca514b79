"""Checkpoints of a device-resident model (aic_lm_save_checkpoint / aic_lm_load_checkpoint):
the reference's SaveLoadVerification and Adler32CorruptionDetection
(tests/unit/test_train.cpp:47-122), the file byte-identical to the format written from
the host copy of the weights in named_parameters() order, and an exact resume with the
optimizer-state extension, for the dense, MoE and QLoRA models."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

import autonomousaicore_amd as aic  # noqa: E402
from tests.test_checkpoint import py_read, py_write, tree_order  # noqa: E402
from tests.test_gpu_step import TINY, build, build_moe, build_qlora, make_base, make_lora, make_params  # noqa: E402

SHAPE_MISMATCH, FORMAT_ERROR = 3, 11


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def test_save_load_bitwise_and_metadata(tmp_path):
    p = str(tmp_path / "m.aic")
    a = build(TINY)
    params = make_params(a, 11)
    a.set_params(params)
    a.save_checkpoint(p, aic.CheckpointMetadata(42, 2, 1.234, "unit_test_checkpoint"))
    b = build(TINY)
    b.set_params(make_params(b, 12))
    meta = b.load_checkpoint(p)
    assert (meta.step, meta.epoch, meta.description, meta.has_optimizer) == (42, 2, "unit_test_checkpoint", False)
    assert abs(meta.best_val_loss - 1.234) < 1e-6
    np.testing.assert_array_equal(b.get_params(), params)
    # the file is the format written from the host weights in named_parameters() order
    head, ts = py_read(p)
    names = [n for n, _, _ in a.layout]
    order = tree_order(names)
    assert [t[0] for t in ts] == order
    q = str(tmp_path / "ref.aic")
    by_name = {n: (s, o) for n, s, o in a.layout}
    py_write(q, 42, 2, 1.234, "unit_test_checkpoint",
             [(n, list(by_name[n][0]), 0, params[by_name[n][1]:by_name[n][1] + int(np.prod(by_name[n][0]))].tobytes())
              for n in order])
    assert open(p, "rb").read() == open(q, "rb").read()
    a.close()
    b.close()


def test_corruption_and_mismatch_are_errors(tmp_path):
    p = str(tmp_path / "c.aic")
    m = build(TINY)
    m.init_normal(3)
    m.save_checkpoint(p)
    raw = bytearray(open(p, "rb").read())
    raw[-20] ^= 0xFF
    open(p, "wb").write(bytes(raw))
    with pytest.raises(aic.AicError) as e:
        m.load_checkpoint(p)
    assert e.value.code == FORMAT_ERROR
    other = build(dict(TINY, f=384))                        # a different FFN width
    m.init_normal(3)
    m.save_checkpoint(p)
    with pytest.raises(aic.AicError) as e:
        other.load_checkpoint(p)
    assert e.value.code == SHAPE_MISMATCH
    m.close()
    other.close()


def test_resume_with_optimizer_state_is_exact(tmp_path):
    """Two steps, save with optimizer state, two more steps; a fresh model loaded from the file
    takes the same two steps bit for bit (loss, parameters, moments, step, loss scale)."""
    p = str(tmp_path / "r.aic")
    cfg = dict(vocab=1024, d=256, L=2, H=4, f=512, tied=False)
    B, S = 2, 128
    a = build(cfg, compute="bfloat16", amp=True)
    a.init_normal(21)
    batches = [aic.batch(100 + k, B, S, cfg["vocab"], dist="zipf") for k in range(4)]
    for ids, tgt in batches[:2]:
        a.train_step(ids, tgt, B, S)
    a.save_checkpoint(p, aic.CheckpointMetadata(step=2), with_optimizer=True)
    b = build(cfg, compute="bfloat16", amp=True)
    b.init_normal(99)
    meta = b.load_checkpoint(p)
    assert meta.has_optimizer and meta.step == 2
    for k, (ids, tgt) in enumerate(batches[2:]):
        sa = a.train_step(ids, tgt, B, S)
        sb = b.train_step(ids, tgt, B, S)
        assert sa.loss == sb.loss and sa.loss_scale == sb.loss_scale and sa.step == sb.step == 3 + k
    np.testing.assert_array_equal(a.get_params(), b.get_params())
    ma, va, ka = a.get_adam_state()
    mb, vb, kb = b.get_adam_state()
    np.testing.assert_array_equal(ma, mb)
    np.testing.assert_array_equal(va, vb)
    assert ka == kb == 4
    a.close()
    b.close()


def test_moe_and_qlora_round_trips(tmp_path):
    B, S = 2, 64
    ids, tgt = aic.batch(7, B, S, 512)
    p = str(tmp_path / "moe.aic")
    cfg = dict(TINY, tied=False)
    a = build_moe(cfg, 4, 2, 0.01)
    a.set_params(make_params(a, 5))
    a.save_checkpoint(p)
    names = [t[0] for t in py_read(p)[1]]
    assert any(".moe.experts.3.down_proj.weight" in n for n in names) and len(names) == len(a.layout)
    b = build_moe(cfg, 4, 2, 0.01)
    b.load_checkpoint(p)
    assert a.eval_loss(ids, tgt, B, S) == b.eval_loss(ids, tgt, B, S)
    a.close()
    b.close()
    # QLoRA: the frozen base (quantized again on load) and the adapters
    p = str(tmp_path / "q.aic")
    a = build_qlora(cfg, 16, 32.0, 128)
    a.set_base_params(make_base(a, 8))
    a.set_params(make_lora(a, 9, 0.02))
    a.save_checkpoint(p, with_optimizer=True)
    names = [t[0] for t in py_read(p)[1]]
    assert "layers.1.ffn.down_proj.lora_B" in names and "layers.1.ffn.down_proj.weight" in names
    assert names.index("layers.0.attn.k_proj.lora_A") < names.index("layers.0.attn.k_proj.weight")
    b = build_qlora(cfg, 16, 32.0, 128)
    meta = b.load_checkpoint(p)
    assert meta.has_optimizer
    assert a.eval_loss(ids, tgt, B, S) == b.eval_loss(ids, tgt, B, S)
    np.testing.assert_array_equal(a.get_params(), b.get_params())
    a.close()
    b.close()
