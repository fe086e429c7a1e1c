"""qwentts-turbo for MI355X: Qwen3-TTS decode (backbone + code predictor) as persistent gfx950 kernels.

Public surface mirrors the reference package (/root/reference/qwentts_turbo/__init__.py:3-4):
``NativeTTSGenerator`` plus the two kernel wrappers. Import name: ``qwentts_turbo_amd``.
"""
from .batched import BatchedTTSDecoder
from .generator import NativeTTSGenerator
from .megakernel_backbone import TTSMegakernelGenerator
from .megakernel_code_predictor import CodePredictorMegakernelGenerator
from .weights import load_local as load_model, synthetic_state_dict, SyntheticConfig

__all__ = ["BatchedTTSDecoder", "NativeTTSGenerator", "TTSMegakernelGenerator", "CodePredictorMegakernelGenerator", "load_model",
           "synthetic_state_dict", "SyntheticConfig"]
