"""Code-predictor decode on MI355X: the reference's ``CodePredictorMegakernelGenerator`` interface.

Mirrors /root/reference/qwentts_turbo/megakernel_code_predictor.py:319-350 (wrapper) and
:265-316 (weight extraction; RoPE theta 1e6, bf16 tables). Besides the reference's
single-step decoder it binds the 15 lm-heads and codebook embeddings so a whole frame (the
2-token prefill, 14 decode steps, 15 heads with on-device selection and the embedding
combine) runs in one launch (``MegakernelCodePredictorDecoder.frame``).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _ext
from .weights import (BB_PREFIX, CP_PREFIX, HEAD_DIM, HIDDEN_SIZE, INTERMEDIATE_SIZE, NUM_KV_HEADS, NUM_Q_HEADS,
                      ROPE_THETA, as_state_dict, count_groups, count_layers, layer_list, load_local, rope_tables)

CP_HIDDEN_SIZE = HIDDEN_SIZE
CP_INTERMEDIATE_SIZE = INTERMEDIATE_SIZE
CP_NUM_Q_HEADS = NUM_Q_HEADS
CP_NUM_KV_HEADS = NUM_KV_HEADS
CP_HEAD_DIM = HEAD_DIM
CP_NUM_LAYERS = 5


def extract_code_predictor_weights(model, max_seq_len: int = 4096, device="cuda") -> dict:
    """Code-predictor weights in the kernel's order (megakernel_code_predictor.py:265-316)."""
    if isinstance(model, str):
        model = load_local(model)
    sd = as_state_dict(model)
    n = count_layers(sd, CP_PREFIX)
    if n == 0:
        raise KeyError(f"no '{CP_PREFIX}layers.*' tensors in the model")
    ng = count_groups(sd)
    cos_t, sin_t = rope_tables(max_seq_len, ROPE_THETA, device=device)
    bf = torch.bfloat16
    return {
        "layer_weights": layer_list(sd, CP_PREFIX, n, device),
        "final_norm_weight": sd[CP_PREFIX + "norm.weight"].to(device, bf).contiguous(),
        "cos_table": cos_t,
        "sin_table": sin_t,
        "num_layers": n,
        "lm_heads": [sd[f"talker.code_predictor.lm_head.{g}.weight"].to(device, bf).contiguous() for g in range(ng)],
        "codec_embeddings": [sd[f"{CP_PREFIX}codec_embedding.{g}.weight"].to(device, bf).contiguous() for g in range(ng)],
        "bb_codec_embedding": sd[BB_PREFIX + "codec_embedding.weight"].to(device, bf).contiguous(),
    }


class CodePredictorMegakernelGenerator:
    """High-level code-predictor decoder (megakernel_code_predictor.py:319-350)."""

    def __init__(self, model_path: Optional[str] = None, max_seq_len: int = 256, model=None, device="cuda"):
        if model is None:
            if model_path is None:
                raise ValueError("pass model (state dict / module) or a local model_path")
            model = load_local(model_path)
        self.weights = extract_code_predictor_weights(model, device=device)
        kernel = _ext.load()
        w = self.weights
        self.decoder = kernel.MegakernelCodePredictorDecoder(
            w["layer_weights"], w["final_norm_weight"], w["cos_table"], w["sin_table"], w["num_layers"], max_seq_len)
        if w["lm_heads"]:
            self.decoder.set_heads(w["lm_heads"], w["codec_embeddings"], w["bb_codec_embedding"])
        self.max_seq_len = max_seq_len
        self.n_groups = len(w["lm_heads"])

    def decode_step_with_embedding(self, input_embedding: torch.Tensor) -> torch.Tensor:
        """One decode step at the running position; returns the final-norm hidden (f32 [1024])."""
        return self.decoder.decode_step_with_embedding(input_embedding)

    def reset(self):
        self.decoder.reset()

    def check_error(self):
        self.decoder.check_error()

    @property
    def position(self) -> int:
        return self.decoder.position()
