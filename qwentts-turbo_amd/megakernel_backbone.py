"""Backbone (talker) decode on MI355X: the reference's ``TTSMegakernelGenerator`` interface.

Mirrors /root/reference/qwentts_turbo/megakernel_backbone.py:412-488 (wrapper) and :358-409
(weight extraction). The kernel is the persistent gfx950 backbone kernel of
``csrc/qtts_decode.hip`` reached through ``_qwentts_amd_C.MegakernelTTSDecoder``.
Differences from the reference: weights come from a state dict / module / local safetensors
path (no download by model name), the extension is prebuilt (no JIT), and a decode step may
use distinct (t, h, w) rotary positions (interleaved mRoPE).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _ext
from .weights import (BB_PREFIX, HEAD_DIM, HIDDEN_SIZE, INTERMEDIATE_SIZE, NUM_KV_HEADS, NUM_Q_HEADS, ROPE_THETA,
                      as_state_dict, count_layers, layer_list, load_local, rope_tables)

Q_SIZE = NUM_Q_HEADS * HEAD_DIM
KV_SIZE = NUM_KV_HEADS * HEAD_DIM


def _extract_tts_backbone_weights(model, max_seq_len: int = 4096, rope_theta: float = ROPE_THETA,
                                  device="cuda") -> dict:
    """Weights of the talker backbone in the kernel's order (megakernel_backbone.py:358-409)."""
    sd = as_state_dict(model)
    n = count_layers(sd, BB_PREFIX)
    if n == 0:
        raise KeyError(f"no '{BB_PREFIX}layers.*' tensors in the model")
    embed = sd[BB_PREFIX + "codec_embedding.weight"].to(device, torch.bfloat16).contiguous()
    cos_t, sin_t = rope_tables(max_seq_len, rope_theta, device=device)
    return {
        "embed_weight": embed,
        "layer_weights": layer_list(sd, BB_PREFIX, n, device),
        "final_norm_weight": sd[BB_PREFIX + "norm.weight"].to(device, torch.bfloat16).contiguous(),
        "codec_head_weight": sd["talker.codec_head.weight"].to(device, torch.bfloat16).contiguous(),
        "cos_table": cos_t,
        "sin_table": sin_t,
        "num_layers": n,
        "vocab_size": embed.shape[0],
    }


class TTSMegakernelGenerator:
    """High-level backbone decoder (megakernel_backbone.py:412-488)."""

    def __init__(self, model_path: Optional[str] = None, model=None, max_seq_len: int = 4096,
                 rope_theta: float = ROPE_THETA, device="cuda", shared_weights: Optional[dict] = None):
        """``shared_weights``: the ``weights`` of another generator built with the same
        ``max_seq_len``, reused instead of extracting a copy (the decoders of a batch share one
        copy, which one multi-stream launch requires)."""
        if shared_weights is not None:
            if shared_weights["cos_table"].shape[0] < max_seq_len:
                raise ValueError("shared_weights were built for a shorter max_seq_len")
            w = shared_weights
        else:
            if model is None:
                if model_path is None:
                    raise ValueError("pass model (state dict / module) or a local model_path")
                model = load_local(model_path)
            w = _extract_tts_backbone_weights(model, max_seq_len, rope_theta, device)
        kernel = _ext.load()
        self.decoder = kernel.MegakernelTTSDecoder(
            w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["codec_head_weight"],
            w["cos_table"], w["sin_table"], w["num_layers"], max_seq_len)
        self.weights = w
        self.max_seq_len = max_seq_len
        self.vocab_size = w["vocab_size"]
        self.num_layers = w["num_layers"]

    def decode_step(self, input_token_id: int) -> torch.Tensor:
        """One decode step from a token id; returns the final-norm hidden (f32 [1024])."""
        return self.decoder.decode_step(input_token_id)

    def decode_step_with_argmax(self, input_token_id: int) -> int:
        """One decode step plus codec-head argmax (no suppression), as the reference."""
        return self.decoder.decode_step_with_argmax(input_token_id)

    def decode_step_with_embedding(self, input_embedding: torch.Tensor,
                                   pos3: Optional[Sequence[int]] = None) -> torch.Tensor:
        """One decode step from a [1024] / [1, 1024] embedding; returns f32 [1024].

        ``pos3`` optionally gives distinct (t, h, w) rotary positions for this step."""
        if pos3 is None:
            return self.decoder.decode_step_with_embedding(input_embedding)
        return self.decoder.decode_step_3d(input_embedding, [int(p) for p in pos3])

    def prefill(self, embeds: torch.Tensor, pos3=None) -> torch.Tensor:
        """All prompt embeddings ([S, 1024] or [1, S, 1024]) in one call at positions
        position .. position + S - 1: the transformers bf16 forward on MFMA with K/V written into
        this decoder's cache (replaces generator.py:209-225 plus the KV handoff :245-257).
        Returns the last token's final-norm hidden (f32 [1024]). ``pos3``: optional [3, S]
        rotary (t, h, w) positions."""
        return self.decoder.prefill(embeds, pos3=pos3)

    def reset(self):
        self.decoder.reset()

    def set_position(self, pos: int):
        self.decoder.set_position(pos)

    def set_kv_cache(self, k_cache: torch.Tensor, v_cache: torch.Tensor):
        """Prefix copy of [num_layers, 8, seq, 128] K/V into the cache."""
        self.decoder.set_kv_cache(k_cache, v_cache)

    def get_k_cache(self) -> torch.Tensor:
        return self.decoder.get_k_cache()

    def get_v_cache(self) -> torch.Tensor:
        return self.decoder.get_v_cache()

    def check_error(self):
        """Raise if a device-side wait timed out since the last check (synchronises)."""
        self.decoder.check_error()

    @property
    def position(self) -> int:
        return self.decoder.position()
