"""ctypes binding of the native library libaic_hip.so (include/aic_hip.h).

Loading never compiles and never falls back: if the library is missing, `load()` raises
with the command that builds it.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaic_hip.so")

AIC_F32, AIC_F16, AIC_BF16, AIC_I32, AIC_I64, AIC_U8, AIC_U16 = 0, 1, 2, 3, 4, 5, 6

vp = C.c_void_p
i64 = C.c_int64
f32 = C.c_float
i32 = C.c_int
i64p = C.POINTER(C.c_int64)
f32p = C.POINTER(C.c_float)


class OptimCtl(C.Structure):
    _fields_ = [("scale", f32), ("good_steps", i32), ("skipped_steps", i32), ("use_scaler", i32),
                ("growth_factor", f32), ("backoff_factor", f32), ("growth_interval", i32), ("min_scale", f32),
                ("max_scale", f32), ("max_grad_norm", f32), ("grad_norm", f32), ("grad_mult", f32), ("skip", i32),
                ("step", i32)]


class StepRecord(C.Structure):
    _fields_ = [("step", i64), ("loss", f32), ("aux_loss", f32), ("grad_norm", f32), ("loss_scale", f32),
                ("found_inf", i32), ("pad", i32)]


class TelemetrySnapshot(C.Structure):
    _fields_ = [("step", i64), ("loss", f32), ("loss_ema_short", f32), ("loss_ema_long", f32),
                ("loss_variance", f32), ("grad_norm", f32), ("grad_norm_ema", f32), ("lr", f32),
                ("tokens_per_sec", f32), ("estimated_tflops", f32), ("host_total_bytes", C.c_uint64),
                ("host_free_bytes", C.c_uint64), ("gpu_total_bytes", C.c_uint64), ("gpu_free_bytes", C.c_uint64),
                ("anomaly", i32), ("pad", i32)]


class GemmDesc(C.Structure):
    _fields_ = [("transA", i32), ("transB", i32), ("M", i64), ("N", i64), ("K", i64), ("A", vp), ("lda", i64),
                ("B", vp), ("ldb", i64), ("C", vp), ("ldc", i64)]


class LMConfig(C.Structure):
    _fields_ = [("vocab", i64), ("d_model", i64), ("n_layers", i64), ("n_heads", i64), ("d_ffn", i64),
                ("max_seq_len", i64), ("norm_eps", f32), ("rope_base", f32), ("tied", i32), ("compute", i32),
                ("n_experts", i64), ("top_k", i64), ("aux_loss_coef", f32), ("lora_rank", i64),
                ("lora_alpha", f32), ("quant_group", i64)]


class TrainConfig(C.Structure):
    _fields_ = [("lr", f32), ("beta1", f32), ("beta2", f32), ("eps", f32), ("weight_decay", f32),
                ("max_grad_norm", f32), ("use_loss_scaler", i32), ("init_scale", f32), ("growth_factor", f32),
                ("backoff_factor", f32), ("growth_interval", i32), ("min_scale", f32), ("max_scale", f32)]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", i64), ("total_ms", C.c_double), ("flops", C.c_double),
                ("bytes", C.c_double), ("mfma_bound", i32)]


class StepStats(C.Structure):
    _fields_ = [("loss", f32), ("grad_norm", f32), ("found_inf", i32), ("loss_scale", f32), ("step", i64),
                ("aux_loss", f32)]


# name -> (restype, argtypes)
SIGNATURES = {
    "aic_hip_last_error": (C.c_char_p, []),
    "aic_hip_device_count": (i32, []),
    "aic_hip_version": (C.c_char_p, []),
    "aic_hip_mem_alloc_async": (i32, [C.POINTER(vp), C.c_size_t, vp]),
    "aic_hip_mem_free_async": (i32, [vp, vp]),
    "aic_hip_mem_stats": (i32, [i64p, i64p]),
    "aic_hip_mem_release_stream": (i32, [vp]),
    "aic_hip_gemm": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64, vp, i64, i32, i32, vp]),
    "aic_hip_gemm_grouped": (i32, [i32, C.POINTER(GemmDesc), f32, f32, i32, i32, vp]),
    "aic_hip_gemm_ragged": (i32, [i32, i64, i64, i64, f32, vp, i64, vp, i64, i64, vp, i64, vp, i32, i64, vp, i64, vp,
                                  vp, i64, i32, vp]),
    "aic_hip_gemm_lowrank": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, vp, i64, vp, i64, i64, i64, i32,
                                   f32, vp, i64, vp, i64, i32, i32, vp]),
    "aic_hip_rmsnorm_fwd": (i32, [vp, i64, vp, vp, i64, vp, i64, i64, f32, i32, vp]),
    "aic_hip_rmsnorm_bwd": (i32, [vp, i64, vp, i64, vp, vp, vp, i64, vp, i64, vp, i32, i64, i64, i32, vp]),
    "aic_hip_rope": (i32, [vp, i64, i64, i64, i64, i64, i64, vp, vp, i32, i32, vp]),
    "aic_hip_rope_tables": (i32, [vp, vp, i64, i64, f32]),
    "aic_hip_attn_fwd": (i32, [vp, vp, vp, i64, vp, i64, vp, i64, i64, i64, i64, i32, f32, i32, vp]),
    "aic_hip_attn_bwd": (i32, [vp, vp, vp, i64, vp, vp, i64, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, f32, i32,
                               vp]),
    "aic_hip_gemm_rope": (i32, [i64, i64, i64, vp, i64, vp, i64, vp, i64, i64, i64, i64, i64, vp, vp, vp]),
    "aic_hip_gemm_swiglu": (i32, [i64, i64, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp]),
    "aic_hip_gemm_swiglu_bwd": (i32, [i64, i64, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, vp]),
    "aic_hip_int4_gemm_swiglu": (i32, [i64, i64, i64, vp, i64, vp, vp, i64, vp, i64, vp, i64, i64, i64, vp, i64, vp,
                                       i64, vp]),
    "aic_hip_lora_skinny": (i32, [vp, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64, f32, vp, i64, vp, i64, i64, i32,
                                  vp]),
    "aic_hip_attn_bwd_rope": (i32, [vp, vp, vp, i64, vp, vp, i64, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, f32,
                                    vp, vp, i32, vp]),
    "aic_hip_swiglu_fwd": (i32, [vp, vp, i64, vp, i64, i64, i64, i32, vp]),
    "aic_hip_swiglu_bwd": (i32, [vp, vp, i64, vp, i64, vp, vp, i64, i64, i64, i32, vp]),
    "aic_hip_ce_fwd": (i32, [vp, i64, vp, i64, i64, i64, vp, vp, vp, vp, i32, vp]),
    "aic_hip_ce_bwd": (i32, [vp, i64, vp, vp, i64, i64, i64, vp, vp, vp, i64, i32, vp]),
    "aic_hip_ce_bwd_rows": (i32, [vp, i64, vp, vp, i64, i64, i64, vp, i32, f32, vp, i64, i32, vp]),
    "aic_hip_ce_fwd_bwd": (i32, [vp, i64, vp, i64, i64, i64, vp, vp, vp, vp, vp, i32, vp]),
    "aic_hip_ce_fwd_soft": (i32, [vp, i64, vp, i64, i64, i64, vp, vp, vp, i32, vp]),
    "aic_hip_ce_bwd_soft": (i32, [vp, i64, vp, i64, vp, i64, i64, vp, i32, f32, vp, i64, i32, vp]),
    "aic_hip_memcpy_sync": (i32, [vp, vp, C.c_size_t, vp]),
    "aic_hip_embed_fwd": (i32, [vp, i64, vp, i64, i64, vp, i32, vp]),
    "aic_hip_embed_bwd": (i32, [vp, i64, vp, i64, i64, vp, i32, i32, vp]),
    "aic_hip_grad_sqnorm_multi": (i32, [C.POINTER(vp), i64p, i32, vp, vp, vp]),
    "aic_hip_grad_sqnorm_multi_noalloc": (i32, [C.POINTER(vp), i64p, i32, vp, vp, vp]),
    "aic_hip_scale_multi": (i32, [C.POINTER(vp), i64p, i32, vp, vp]),
    "aic_hip_optim_finalize": (i32, [vp, vp, vp, vp]),
    "aic_hip_adamw_multi": (i32, [C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), i64p,
                                  i32, f32, f32, f32, f32, f32, i64, vp, vp]),
    "aic_hip_adamw_step": (i32, [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, f32, f32, vp]),
    "aic_hip_cast_f32_bf16": (i32, [vp, vp, i64, vp]),
    "aic_hip_stream_probe": (i32, [C.POINTER(vp), i32, C.POINTER(vp), i32, vp, vp, i64, i32, vp]),
    "aic_hip_moe_route": (i32, [vp, i64, i64, i64, f32, vp, vp, vp, vp, vp, vp, vp, vp]),
    "aic_hip_moe_max_rows": (i64, [i64, i64, i64]),
    "aic_hip_moe_permute": (i32, [vp, vp, i64, i64, i64, vp, vp, vp, vp]),
    "aic_hip_moe_gather": (i32, [vp, i64, vp, i64, i64, i64, vp, i32, vp]),
    "aic_hip_moe_combine": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, i64, vp, i64, i32, vp]),
    "aic_moe_ffn_create": (i32, [i64, i64, i64, i64, f32, i32, C.POINTER(vp)]),
    "aic_moe_ffn_destroy": (i32, [vp]),
    "aic_moe_ffn_forward": (i32, [vp, vp, i64, vp, vp, vp, vp, vp, vp]),
    "aic_moe_ffn_backward": (i32, [vp, vp, f32, vp, vp, vp, vp]),
    "aic_moe_ffn_routing": (i32, [vp, vp, vp, vp]),
    "aic_hip_int4_quantize": (i32, [vp, i64, i64, vp, vp, i32, vp]),
    "aic_hip_int4_dequantize": (i32, [vp, vp, i32, i64, i64, vp, i32, vp]),
    "aic_hip_int4_dequantize_zp": (i32, [vp, vp, vp, i32, i64, i64, vp, vp]),
    "aic_hip_int4_gemm_rope": (i32, [i64, i64, i64, vp, i64, vp, vp, i64, vp, i64, vp, i64, i64, i64, vp, i64, i64,
                                      i64, i64, i64, vp, vp, vp]),
    "aic_hip_int4_dequant_gemm": (i32, [i32, i64, i64, i64, f32, vp, i64, vp, vp, i32, i64, f32, vp, i64, vp, i64,
                                        i32, i32, vp]),
    "aic_hip_lora_merge": (i32, [vp, vp, vp, i64, i64, i64, f32, i32, i32, vp]),
    "aic_qlora_linear_create": (i32, [i64, i64, i64, f32, i64, i32, i32, vp]),
    "aic_qlora_linear_destroy": (i32, [vp]),
    "aic_qlora_linear_forward": (i32, [vp, vp, i64, vp, vp, vp, vp, vp, vp, vp]),
    "aic_qlora_linear_backward": (i32, [vp, vp, vp, vp, vp, i32, vp]),
    "aic_hip_strided_copy": (i32, [vp, i64, i32, i64p, i64p, i64, vp, vp]),
    "aic_hip_cast": (i32, [vp, i32, vp, i32, i64, vp]),
    "aic_hip_binary": (i32, [i32, vp, i64, i32, i64p, i64p, vp, i64, i32, i64p, i64p, vp, vp]),
    "aic_hip_unary": (i32, [i32, vp, vp, i64, vp]),
    "aic_hip_reduce_all": (i32, [i32, vp, i64, vp, vp]),
    "aic_hip_reduce_dim": (i32, [i32, vp, i32, i64p, i32, vp, vp]),
    "aic_hip_cat": (i32, [C.POINTER(vp), i64p, i32, i64, i64, i64, vp, vp]),
    "aic_hip_sum_to_shape": (i32, [vp, i32, i64p, i32, i64p, vp, vp]),
    "aic_lm_create": (i32, [C.POINTER(LMConfig), C.POINTER(TrainConfig), C.POINTER(vp)]),
    "aic_lm_destroy": (i32, [vp]),
    "aic_lm_num_params": (i64, [vp]),
    "aic_lm_num_tensors": (i32, [vp]),
    "aic_lm_tensor_info": (i32, [vp, i32, C.c_char_p, i32, C.POINTER(i32), i64p, i64p]),
    "aic_lm_num_base_params": (i64, [vp]),
    "aic_lm_num_base_tensors": (i32, [vp]),
    "aic_lm_base_tensor_info": (i32, [vp, i32, C.c_char_p, i32, C.POINTER(i32), i64p, i64p]),
    "aic_lm_set_base_params": (i32, [vp, vp]),
    "aic_lm_get_base_params": (i32, [vp, vp]),
    "aic_lm_set_params": (i32, [vp, vp]),
    "aic_lm_step_history": (i32, [vp, C.POINTER(StepRecord), i32, C.POINTER(i32), i64p]),
    "aic_lm_snapshot": (i32, [vp]),
    "aic_lm_restore": (i32, [vp]),
    "aic_telemetry_create": (i32, [i64, f32, f32, C.POINTER(vp)]),
    "aic_telemetry_destroy": (i32, [vp]),
    "aic_telemetry_record": (i32, [vp, i64, f32, f32, f32, f32, C.c_double, i64, i64, i32,
                                   C.POINTER(TelemetrySnapshot)]),
    "aic_telemetry_count": (i64, [vp]),
    "aic_telemetry_is_nan_or_inf": (i32, [vp]),
    "aic_telemetry_is_diverging": (i32, [vp, f32, i32]),
    "aic_telemetry_is_gradient_exploding": (i32, [vp, f32]),
    "aic_telemetry_is_gradient_vanishing": (i32, [vp, f32]),
    "aic_telemetry_reset": (i32, [vp]),
    "aic_telemetry_latest_json": (i32, [vp, C.c_char_p, i32]),
    "aic_lm_forward_step": (i32, [vp, vp, i64, i64, i64, i32, vp]),
    "aic_sample_tokens": (i32, [vp, i64, f32, i32, f32, C.c_uint64, i64, vp]),
    "aic_lm_generate": (i32, [vp, vp, i64, i64, f32, i32, f32, i64, C.c_uint64, vp, i64p]),
    "aic_lm_save_checkpoint": (i32, [vp, C.c_char_p, i64, i64, f32, C.c_char_p, i32]),
    "aic_lm_load_checkpoint": (i32, [vp, C.c_char_p, i64p, i64p, f32p, C.c_char_p, i32, C.POINTER(i32)]),
    "aic_checkpoint_write": (i32, [C.c_char_p, i64, i64, f32, C.c_char_p, i64, C.POINTER(C.c_char_p),
                                   C.POINTER(i32), i64p, C.POINTER(i32), C.POINTER(vp), C.POINTER(C.c_uint64)]),
    "aic_checkpoint_verify": (i32, [C.c_char_p, i64p, i64p, i64p, f32p]),
    "aic_checkpoint_module_order": (i32, [i64, C.POINTER(C.c_char_p), i64p]),
    "aic_lm_get_params": (i32, [vp, vp]),
    "aic_lm_get_grads": (i32, [vp, vp]),
    "aic_hip_attn_fwd_qk": (i32, [vp, i64, vp, vp, i64, vp, i64, vp, i64, i64, i64, i64, i64, i32, f32, i32, vp]),
    "aic_hip_attn_bwd_qk": (i32, [vp, i64, vp, vp, i64, vp, vp, i64, vp, vp, i64, vp, vp, i64, i64, i64, i64, i64, i64,
                                  i32, f32, i32, vp]),
    "aic_lm_moe_routing": (i32, [vp, i64, vp, i64, i64p]),
    "aic_lm_get_adam_state": (i32, [vp, vp, vp, i64p]),
    "aic_lm_init_normal": (i32, [vp, C.c_uint64, f32, i32]),
    "aic_lm_train_step": (i32, [vp, vp, vp, i64, i64, i32, C.POINTER(StepStats)]),
    "aic_lm_eval_loss": (i32, [vp, vp, vp, i64, i64, i32, f32p]),
    "aic_lm_stream": (i32, [vp, C.POINTER(vp)]),
    "aic_lm_synchronize": (i32, [vp]),
    "aic_lm_last_stats": (i32, [vp, C.POINTER(StepStats)]),
    "aic_lm_profile": (i32, [vp, i32]),
    "aic_lm_fused_grad_norm": (i32, [vp, i32, C.POINTER(i32)]),
    "aic_lm_profile_classes": (i32, [vp, C.c_uint32]),
    "aic_lm_profile_class_index": (i32, [C.c_char_p]),
    "aic_lm_profile_stats": (i32, [vp, C.POINTER(KernelStat), i32, C.POINTER(i32)]),
    "aic_dataset_open": (i32, [C.c_char_p, i64, i64, C.POINTER(vp)]),
    "aic_dataset_from_tokens": (i32, [vp, i64, i64, i64, C.POINTER(vp)]),
    "aic_dataset_destroy": (i32, [vp]),
    "aic_dataset_size": (i64, [vp]),
    "aic_dataset_total_tokens": (i64, [vp]),
    "aic_dataset_get_item": (i32, [vp, i64, vp, vp]),
    "aic_dataset_write_binary_file": (i32, [C.c_char_p, vp, i64]),
    "aic_loader_create": (i32, [vp, i64, i32, i32, C.c_uint64, i32, C.POINTER(vp)]),
    "aic_loader_destroy": (i32, [vp]),
    "aic_loader_num_batches": (i64, [vp]),
    "aic_loader_has_next": (i32, [vp]),
    "aic_loader_reset": (i32, [vp]),
    "aic_loader_next_host": (i32, [vp, vp, vp, i64p]),
    "aic_loader_next_device": (i32, [vp, vp, vp, i64p, vp]),
    "aic_synth_uniform_ids": (i32, [C.c_uint64, i64, i64, vp]),
    "aic_synth_zipf_ids": (i32, [C.c_uint64, i64, i64, C.c_double, vp]),
    "aic_synth_normal": (i32, [C.c_uint64, i64, f32, f32, vp]),
}


class AicError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"aic error {code}: {message}")
        self.code = code


_lib = None


def load():
    """Load libaic_hip.so (built by `python -m autonomousaicore_amd.build`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m autonomousaicore_amd.build` "
                           "(or __graft_entry__.build()); there is no fallback path")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().aic_hip_last_error()
        raise AicError(rc, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
