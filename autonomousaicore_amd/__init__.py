"""autonomousaicore_amd: MI355X (gfx950) native backend for the AutonomousAICore
TransformerLM training step.  The compute lives in libaic_hip.so (HIP kernels + C-ABI,
include/aic_hip.h); this package is its Python front end."""
from . import _lib
from ._lib import AicError, load
from .lm import (AdamWOptions, CheckpointMetadata, DynamicLossScalerOptions, MoETransformerLMConfig, QLoRATransformerLMConfig, StepMetrics,
                 TrainingConfig, TransformerLM, TransformerLMConfig, batch, normal, uniform_ids, zipf_ids)

__all__ = ["AicError", "load", "AdamWOptions", "CheckpointMetadata", "DynamicLossScalerOptions", "MoETransformerLMConfig",
           "QLoRATransformerLMConfig", "StepMetrics", "TrainingConfig",
           "TransformerLM", "TransformerLMConfig", "batch", "normal", "uniform_ids", "zipf_ids"]
