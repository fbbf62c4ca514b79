"""TelemetryTracker on the CPU: the reference's tests (tests/unit/test_autonomous.cpp:19-111)
and closed forms of the EMAs and the windowed loss variance."""
import math

import numpy as np

from autonomousaicore_amd.telemetry import TelemetryTracker


def test_tracking_and_ema():
    t = TelemetryTracker(window_size=10, alpha_short=0.8, alpha_long=0.95)
    losses = [2.0 - s * 0.1 for s in range(1, 6)]
    for s, loss in enumerate(losses, 1):
        snap = t.record_step(s, loss, 1.0, 1e-3, 10000.0, 0.01, 100, 1000000)
        assert snap["step"] == s and snap["loss_ema_short"] > 0 and snap["loss_ema_long"] > 0
        assert snap["estimated_tflops"] == np.float32(6 * 1e6 * 1e4 / 1e12)
        assert snap["host_total_bytes"] > 0 and snap["host_free_bytes"] <= snap["host_total_bytes"]
    assert t.count() == 5
    assert not t.is_nan_or_inf() and not t.is_diverging() and not t.is_gradient_exploding()
    # closed forms: EMAs seeded with the first loss, population variance of the window
    es = el = np.float32(losses[0])
    for loss in losses[1:]:
        es = np.float32(0.8) * es + np.float32(0.2) * np.float32(loss)
        el = np.float32(0.95) * el + np.float32(1 - 0.95) * np.float32(loss)
    assert abs(snap["loss_ema_short"] - es) < 1e-6 and abs(snap["loss_ema_long"] - el) < 1e-6
    assert abs(snap["loss_variance"] - np.var(np.float32(losses).astype(np.float64))) < 1e-6
    j = t.latest_json()
    assert j["step"] == 5 and j["anomaly"] == "None"


def test_nan_and_inf_detection():
    t = TelemetryTracker()
    t.record_step(1, 1.5, 0.5, 1e-3, 5000.0, 0.01, 50)
    assert not t.is_nan_or_inf()
    snap = t.record_step(2, math.nan, 0.5, 1e-3, 5000.0, 0.01, 50)
    assert t.is_nan_or_inf() and snap["anomaly"] == "NanOrInfLoss"
    snap = t.record_step(3, 1.2, math.inf, 1e-3, 5000.0, 0.01, 50)
    assert t.is_nan_or_inf() and snap["anomaly"] == "NanOrInfGradient"


def test_divergence_and_spike_detection():
    t = TelemetryTracker(window_size=20, alpha_short=0.7, alpha_long=0.99)
    for i in range(1, 11):
        t.record_step(i, 1.0, 0.5, 1e-3, 5000.0, 0.01, 50)
    assert not t.is_diverging()
    t.record_step(11, 5.0, 0.5, 1e-3, 5000.0, 0.01, 50)
    t.record_step(12, 6.0, 0.5, 1e-3, 5000.0, 0.01, 50)
    snap = t.record_step(13, 7.0, 0.5, 1e-3, 5000.0, 0.01, 50)
    assert t.is_diverging() and snap["anomaly"] == "LossDivergence"
    g = TelemetryTracker(window_size=20)
    for i in range(1, 7):
        g.record_step(i, 1.0, 0.2, 1e-3, 5000.0, 0.01, 50)
    snap = g.record_step(7, 1.0, 5.0, 1e-3, 5000.0, 0.01, 50)
    assert g.is_gradient_exploding() and snap["anomaly"] == "GradientExplosion"
    v = TelemetryTracker()
    for i in range(1, 6):
        snap = v.record_step(i, 1.0, 1e-9, 1e-3, 5000.0, 0.01, 50)
    assert v.is_gradient_vanishing() and snap["anomaly"] == "GradientVanishing"
    v.reset()
    assert v.count() == 0
