"""Telemetry hooks of the device-resident step: the step-history ring read after several
asynchronous steps equals the per-step statistics, a forced non-finite step shows up as
found_inf and feeds a NanOrInfGradient anomaly, and an HBM snapshot / restore rolls the model
back bit for bit (the rollback the reference's controller does through checkpoint files)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

import autonomousaicore_amd as aic  # noqa: E402
from autonomousaicore_amd.telemetry import TelemetryTracker  # noqa: E402
from tests.test_gpu_step import TINY, build, make_params  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def test_history_snapshot_and_rollback():
    B, S = 4, 64
    m = build(TINY, amp=False)
    params = make_params(m, 3)
    m.set_params(params)
    batches = [aic.batch(50 + k, B, S, TINY["vocab"]) for k in range(5)]
    synced = []
    for ids, tgt in batches[:3]:
        synced.append(m.train_step(ids, tgt, B, S))          # synchronising path, for reference
    hist, dropped = m.step_history()
    assert dropped == 0 and [h.step for h in hist] == [1, 2, 3]
    for h, st in zip(hist, synced):
        assert (h.loss, h.grad_norm, h.found_inf, h.loss_scale) == (st.loss, st.grad_norm, st.found_inf, st.loss_scale)
    m.snapshot()
    p3 = m.get_params()
    for ids, tgt in batches[3:]:
        m.train_step(ids, tgt, B, S, sync=False)             # no host synchronisation per step
    hist, _ = m.step_history()
    assert [h.step for h in hist] == [4, 5] and not any(h.found_inf for h in hist)
    tracker = TelemetryTracker(window_size=10)
    for h in hist:
        snap = tracker.record_step(h.step, h.loss, h.grad_norm, 3e-4, 0.0, 0.01, B * S, m.num_params, 0)
        assert snap["anomaly"] == "None" and snap["gpu_total_bytes"] > 0
    m.restore()
    np.testing.assert_array_equal(m.get_params(), p3)
    assert m.get_adam_state()[2] == 3
    ids, tgt = batches[3]
    again = m.train_step(ids, tgt, B, S)
    assert again.step == 4 and again.loss == hist[0].loss    # the same step 4 after the rollback
    m.close()


def test_non_finite_step_is_recorded_and_flagged():
    B, S = 2, 64
    m = build(TINY, amp=True)                                  # loss scaler on: the step is skipped
    params = make_params(m, 4)
    m.set_params(params)
    ids, tgt = aic.batch(8, B, S, TINY["vocab"])
    m.train_step(ids, tgt, B, S)
    bad = params.copy()
    bad[0] = np.inf
    m.set_params(bad)
    m.train_step(ids, tgt, B, S, sync=False)
    hist, _ = m.step_history()
    assert [h.found_inf for h in hist] == [False, True]
    tracker = TelemetryTracker()
    snaps = [tracker.record_step(h.step, h.loss, h.grad_norm if not h.found_inf else float("inf"), 3e-4, 0.0,
                                 0.01, B * S) for h in hist]
    assert snaps[-1]["anomaly"] in ("NanOrInfLoss", "NanOrInfGradient")
    m.close()
