"""Python front end of the native TransformerLM training step.

Mirrors the reference's configuration structs and trainer entry points
(models::TransformerLMConfig, include/models/transformer_lm.hpp:19-29; optim::AdamWOptions,
include/optim/adamw.hpp:12-18; train::DynamicLossScalerOptions, include/train/amp.hpp:34-41;
Trainer::step, src/train/trainer.cpp:37-118).  All compute runs in libaic_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import AIC_BF16, AIC_F32


@dataclass
class TransformerLMConfig:
    vocab_size: int = 320
    hidden_dim: int = 128
    num_layers: int = 4
    num_heads: int = 4
    intermediate_dim: int = 384
    max_seq_len: int = 512
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = False
    compute: str = "float32"  # "float32" (reference precision) or "bfloat16" (AMP)
    num_experts: int = 0      # > 0: MoE FFNs (MoETransformerLMConfig)
    top_k: int = 2
    aux_loss_coef: float = 0.01
    lora_rank: int = 0        # > 0: QLoRA (frozen INT4 base, trained LoRA adapters)
    lora_alpha: float = 32.0
    quant_group: int = 128


@dataclass
class MoETransformerLMConfig(TransformerLMConfig):
    """models::MoETransformerLMConfig (include/models/moe_transformer_lm.hpp): the dense
    configuration plus the expert count, router top-k and aux-loss coefficient."""
    num_experts: int = 8


@dataclass
class QLoRATransformerLMConfig(TransformerLMConfig):
    """A TransformerLM fine-tuned the QLoRA way (LoRAAdapter::apply over
    QuantizedLinear::from_linear; src/nn/lora.cpp:116-175, src/nn/quantization.cpp:669-679):
    the base model frozen with its seven projections per layer quantized to INT4 (groups of
    quant_group, fp16 scales), and rank-lora_rank adapters with scaling lora_alpha / lora_rank
    on all seven projections as the only trained parameters."""
    lora_rank: int = 16


@dataclass
class AdamWOptions:
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01


@dataclass
class DynamicLossScalerOptions:
    initial_scale: float = 65536.0
    growth_factor: float = 2.0
    backoff_factor: float = 0.5
    growth_interval: int = 1000
    min_scale: float = 1.0
    max_scale: float = 16777216.0


@dataclass
class TrainingConfig:
    adamw: AdamWOptions = field(default_factory=AdamWOptions)
    max_grad_norm: float = 1.0
    use_amp: bool = False
    scaler: DynamicLossScalerOptions = field(default_factory=DynamicLossScalerOptions)


@dataclass
class CheckpointMetadata:
    """train::CheckpointMetadata (include/train/checkpoint.hpp:15-22)."""
    step: int = 0
    epoch: int = 0
    best_val_loss: float = 0.0
    description: str = ""
    has_optimizer: bool = False


@dataclass
class StepMetrics:
    loss: float
    grad_norm: float
    found_inf: bool
    loss_scale: float
    step: int
    aux_loss: float = 0.0


class TransformerLM:
    """One TransformerLM with its AdamW state on the current GPU."""

    def __init__(self, cfg: TransformerLMConfig, train: TrainingConfig | None = None):
        train = train or TrainingConfig()
        self.cfg = cfg
        self.train_cfg = train
        c = _lib.LMConfig(cfg.vocab_size, cfg.hidden_dim, cfg.num_layers, cfg.num_heads, cfg.intermediate_dim,
                          cfg.max_seq_len, cfg.rms_norm_eps, cfg.rope_theta, 1 if cfg.tie_word_embeddings else 0,
                          AIC_BF16 if cfg.compute == "bfloat16" else AIC_F32, cfg.num_experts, cfg.top_k,
                          cfg.aux_loss_coef, cfg.lora_rank, cfg.lora_alpha, cfg.quant_group)
        a, s = train.adamw, train.scaler
        t = _lib.TrainConfig(a.lr, a.beta1, a.beta2, a.eps, a.weight_decay, train.max_grad_norm,
                             1 if train.use_amp else 0, s.initial_scale, s.growth_factor, s.backoff_factor,
                             s.growth_interval, s.min_scale, s.max_scale)
        h = C.c_void_p()
        _lib.call("aic_lm_create", C.byref(c), C.byref(t), C.byref(h))
        self._h = h
        self.layout = self._layout("aic_lm_num_tensors", "aic_lm_tensor_info")
        self.base_layout = self._layout("aic_lm_num_base_tensors", "aic_lm_base_tensor_info")

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.call("aic_lm_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _layout(self, count: str, info: str):
        lib = _lib.load()
        n = getattr(lib, count)(self._h)
        out = []
        name = C.create_string_buffer(256)
        rank = C.c_int()
        dims = (C.c_int64 * 2)()
        off = C.c_int64()
        for i in range(n):
            _lib.check(getattr(lib, info)(self._h, i, name, 256, C.byref(rank), dims, C.byref(off)))
            out.append((name.value.decode(), tuple(dims[: rank.value]), int(off.value)))
        return out

    @property
    def num_params(self) -> int:
        return int(_lib.load().aic_lm_num_params(self._h))

    def named_parameters(self, flat: np.ndarray):
        """Views of a packed flat array as (name, array) pairs in arena order."""
        return [(n, flat[o:o + int(np.prod(s))].reshape(s)) for n, s, o in self.layout]

    @property
    def num_base_params(self) -> int:
        return int(_lib.load().aic_lm_num_base_params(self._h))

    def set_base_params(self, flat: np.ndarray) -> None:
        """QLoRA: the frozen base model (packed, in base_layout order); quantizes its projections."""
        flat = np.ascontiguousarray(flat, np.float32)
        assert flat.size == self.num_base_params
        _lib.call("aic_lm_set_base_params", self._h, flat.ctypes.data)

    def get_base_params(self) -> np.ndarray:
        """QLoRA: the frozen base model in base_layout order (fp32)."""
        out = np.empty(self.num_base_params, np.float32)
        _lib.call("aic_lm_get_base_params", self._h, out.ctypes.data)
        return out

    def set_params(self, flat: np.ndarray) -> None:
        flat = np.ascontiguousarray(flat, np.float32)
        assert flat.size == self.num_params
        _lib.call("aic_lm_set_params", self._h, flat.ctypes.data)

    def get_params(self) -> np.ndarray:
        out = np.empty(self.num_params, np.float32)
        _lib.call("aic_lm_get_params", self._h, out.ctypes.data)
        return out

    def get_grads(self) -> np.ndarray:
        out = np.empty(self.num_params, np.float32)
        _lib.call("aic_lm_get_grads", self._h, out.ctypes.data)
        return out

    def moe_routing(self, layer: int) -> np.ndarray:
        """MoE: the top-k selection [T, top_k] (int64) layer `layer` used in the last forward."""
        k = self.cfg.top_k
        cap = self.cfg.max_seq_len * 64 * k  # up to 64 sequences of the longest length
        out = np.empty(cap, np.int64)
        tokens = C.c_int64()
        _lib.call("aic_lm_moe_routing", self._h, layer, out.ctypes.data, cap, C.byref(tokens))
        return out[:tokens.value * k].reshape(tokens.value, k).copy()

    def get_adam_state(self):
        m = np.empty(self.num_params, np.float32)
        v = np.empty(self.num_params, np.float32)
        step = C.c_int64()
        _lib.call("aic_lm_get_adam_state", self._h, m.ctypes.data, v.ctypes.data, C.byref(step))
        return m, v, int(step.value)

    def init_normal(self, seed: int, std: float = 0.02, residual_scaling: bool = False) -> None:
        _lib.call("aic_lm_init_normal", self._h, C.c_uint64(seed), std, 1 if residual_scaling else 0)

    def train_step(self, ids, targets, B: int, S: int, sync: bool = True) -> StepMetrics | None:
        """ids/targets: numpy int64 [B, S] (host) or device pointers (int) of the same."""
        on_dev = isinstance(ids, int)
        if not on_dev:
            ids = np.ascontiguousarray(ids, np.int64)
            targets = np.ascontiguousarray(targets, np.int64)
            ip, tp = ids.ctypes.data, targets.ctypes.data
        else:
            ip, tp = ids, targets
        st = _lib.StepStats() if sync else None
        _lib.call("aic_lm_train_step", self._h, ip, tp, B, S, 1 if on_dev else 0,
                  C.byref(st) if st is not None else None)
        if st is None:
            return None
        return StepMetrics(st.loss, st.grad_norm, bool(st.found_inf), st.loss_scale, int(st.step), float(st.aux_loss))

    def eval_loss(self, ids, targets, B: int, S: int) -> float:
        on_dev = isinstance(ids, int)
        if not on_dev:
            ids = np.ascontiguousarray(ids, np.int64)
            targets = np.ascontiguousarray(targets, np.int64)
            ip, tp = ids.ctypes.data, targets.ctypes.data
        else:
            ip, tp = ids, targets
        loss = C.c_float()
        _lib.call("aic_lm_eval_loss", self._h, ip, tp, B, S, 1 if on_dev else 0, C.byref(loss))
        return float(loss.value)

    def step_history(self, cap: int = 1024):
        """Records of the steps run since the previous call (one synchronisation): a list of
        StepMetrics, and the number of older records the device ring overwrote."""
        arr = (_lib.StepRecord * cap)()
        n, dropped = C.c_int(), C.c_int64()
        _lib.call("aic_lm_step_history", self._h, arr, cap, C.byref(n), C.byref(dropped))
        out = [StepMetrics(r.loss, r.grad_norm, bool(r.found_inf), r.loss_scale, int(r.step), r.aux_loss)
               for r in arr[:n.value]]
        return out, int(dropped.value)

    def snapshot(self) -> None:
        """Keep a device copy of the parameters, AdamW moments and optimiser state."""
        _lib.call("aic_lm_snapshot", self._h)

    def restore(self) -> None:
        """Roll back to the last snapshot."""
        _lib.call("aic_lm_restore", self._h)

    def forward_step(self, ids, start_pos: int = 0) -> np.ndarray:
        """TransformerLM::forward_step: ids [B, S] (host) at positions start_pos..; returns the fp32
        logits [B, S, V] and appends the tokens' keys / values to the cache."""
        ids = np.ascontiguousarray(ids, np.int64)
        if ids.ndim == 1:
            ids = ids[None]
        B, S = ids.shape
        out = np.empty((B, S, self.cfg.vocab_size), np.float32)
        _lib.call("aic_lm_forward_step", self._h, ids.ctypes.data, B, S, start_pos, 0, out.ctypes.data)
        return out

    def generate(self, prompt, max_new_tokens: int, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
                 eos_token_id: int = -1, seed: int = 42) -> list[int]:
        """TransformerLM::generate (src/models/transformer_lm.cpp:89-233)."""
        p = np.ascontiguousarray(prompt, np.int64)
        out = np.empty(max(1, p.size) + max_new_tokens, np.int64)
        n = C.c_int64()
        _lib.call("aic_lm_generate", self._h, p.ctypes.data if p.size else None, p.size, max_new_tokens,
                  temperature, top_k, top_p, eos_token_id, C.c_uint64(seed), out.ctypes.data, C.byref(n))
        return [int(v) for v in out[:n.value]]

    def save_checkpoint(self, path: str, meta: "CheckpointMetadata | None" = None,
                        with_optimizer: bool = False) -> None:
        """save_checkpoint (src/train/checkpoint.cpp:30-95): the .aic file of every parameter;
        with_optimizer adds the AdamW moments, step and loss-scaler state."""
        meta = meta or CheckpointMetadata()
        _lib.call("aic_lm_save_checkpoint", self._h, path.encode(), meta.step, meta.epoch, meta.best_val_loss,
                  meta.description.encode(), 1 if with_optimizer else 0)

    def load_checkpoint(self, path: str) -> "CheckpointMetadata":
        """load_checkpoint (src/train/checkpoint.cpp:97-186); `has_optimizer` on the result says
        whether AdamW state was restored."""
        step, epoch, loss = C.c_int64(), C.c_int64(), C.c_float()
        desc = C.create_string_buffer(4096)
        has = C.c_int()
        _lib.call("aic_lm_load_checkpoint", self._h, path.encode(), C.byref(step), C.byref(epoch), C.byref(loss),
                  desc, 4096, C.byref(has))
        return CheckpointMetadata(int(step.value), int(epoch.value), float(loss.value), desc.value.decode(),
                                  bool(has.value))

    def synchronize(self) -> None:
        _lib.call("aic_lm_synchronize", self._h)

    def last_stats(self) -> StepMetrics:
        st = _lib.StepStats()
        _lib.call("aic_lm_last_stats", self._h, C.byref(st))
        return StepMetrics(st.loss, st.grad_norm, bool(st.found_inf), st.loss_scale, int(st.step), float(st.aux_loss))

    def fused_grad_norm(self, on: bool) -> bool:
        """Form the step's gradient norm from the producers' partial sums (True, the default
        where the model allows it) or from a pass over every gradient (False); returns whether
        the fused form is now used."""
        used = C.c_int(0)
        _lib.call("aic_lm_fused_grad_norm", self._h, 1 if on else 0, C.byref(used))
        return bool(used.value)

    def set_profiling(self, on: bool, classes=None) -> None:
        """Time the kernel launches of the following steps with HIP events (resets); `classes`
        (names) restricts the timing to those kernel classes."""
        if classes is None:
            _lib.call("aic_lm_profile", self._h, 1 if on else 0)
            return
        mask = 0
        for name in classes:
            c = _lib.load().aic_lm_profile_class_index(name.encode())
            if c < 0:
                raise ValueError(f"unknown kernel class {name}")
            mask |= 1 << c
        _lib.call("aic_lm_profile_classes", self._h, C.c_uint32(mask if on else 0))

    def profile_stats(self) -> list[dict]:
        """Per kernel class: launches, total_ms, algorithmic flops/bytes, mfma_bound."""
        arr = (_lib.KernelStat * 32)()
        n = C.c_int()
        _lib.call("aic_lm_profile_stats", self._h, arr, 32, C.byref(n))
        return [dict(name=arr[i].name.decode(), launches=int(arr[i].launches), total_ms=float(arr[i].total_ms),
                     flops=float(arr[i].flops), bytes=float(arr[i].bytes), mfma_bound=bool(arr[i].mfma_bound))
                for i in range(n.value)]

    @property
    def stream(self) -> int:
        s = C.c_void_p()
        _lib.call("aic_lm_stream", self._h, C.byref(s))
        return s.value or 0


# ----------------------------------------------------------------------------- synthetic data
def uniform_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.int64)
    _lib.call("aic_synth_uniform_ids", C.c_uint64(seed), n, vocab, out.ctypes.data)
    return out


def zipf_ids(seed: int, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    out = np.empty(n, np.int64)
    _lib.call("aic_synth_zipf_ids", C.c_uint64(seed), n, vocab, s, out.ctypes.data)
    return out


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    _lib.call("aic_synth_normal", C.c_uint64(seed), n, mean, std, out.ctypes.data)
    return out


def batch(seed: int, B: int, S: int, vocab: int, dist: str = "uniform", s: float = 1.1):
    """Draw [B, S+1] ids and return (ids [B,S], targets [B,S]) -- targets are ids shifted by
    one, as BinaryTokenDataset::get_item builds them (src/data/dataset.cpp:189-202)."""
    n = B * (S + 1)
    seq = (uniform_ids(seed, n, vocab) if dist == "uniform" else zipf_ids(seed, n, vocab, s)).reshape(B, S + 1)
    return np.ascontiguousarray(seq[:, :S]), np.ascontiguousarray(seq[:, 1:])
