"""Step telemetry (aic::autonomous::TelemetryTracker of the reference,
include/autonomous/telemetry.hpp), computed in libaic_hip.so."""
from __future__ import annotations

import ctypes as C
import json

from . import _lib

ANOMALIES = ["None", "NanOrInfLoss", "NanOrInfGradient", "LossDivergence", "GradientExplosion",
             "GradientVanishing", "MemoryCritical"]


class TelemetryTracker:
    def __init__(self, window_size: int = 50, alpha_short: float = 0.8, alpha_long: float = 0.98):
        h = C.c_void_p()
        _lib.call("aic_telemetry_create", window_size, alpha_short, alpha_long, C.byref(h))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.call("aic_telemetry_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def record_step(self, step, loss, grad_norm, lr, tokens_per_sec, step_duration_sec, total_tokens,
                    model_params=0, device_index=-1) -> dict:
        s = _lib.TelemetrySnapshot()
        _lib.call("aic_telemetry_record", self._h, step, loss, grad_norm, lr, tokens_per_sec, step_duration_sec,
                  total_tokens, model_params, device_index, C.byref(s))
        out = {k: getattr(s, k) for k, _ in s._fields_ if k != "pad"}
        out["anomaly"] = ANOMALIES[s.anomaly]
        return out

    def count(self) -> int:
        return int(_lib.load().aic_telemetry_count(self._h))

    def is_nan_or_inf(self) -> bool:
        return bool(_lib.load().aic_telemetry_is_nan_or_inf(self._h))

    def is_diverging(self, threshold_ratio: float = 1.4, min_consecutive: int = 3) -> bool:
        return bool(_lib.load().aic_telemetry_is_diverging(self._h, threshold_ratio, min_consecutive))

    def is_gradient_exploding(self, spike_factor: float = 4.0) -> bool:
        return bool(_lib.load().aic_telemetry_is_gradient_exploding(self._h, spike_factor))

    def is_gradient_vanishing(self, min_norm: float = 1e-7) -> bool:
        return bool(_lib.load().aic_telemetry_is_gradient_vanishing(self._h, min_norm))

    def reset(self) -> None:
        _lib.call("aic_telemetry_reset", self._h)

    def latest_json(self) -> dict:
        buf = C.create_string_buffer(2048)
        _lib.call("aic_telemetry_latest_json", self._h, buf, 2048)
        return json.loads(buf.value.decode())
