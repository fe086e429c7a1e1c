"""Weight handling for the decode path: state-dict access, seeded synthetic weights, RoPE tables.

Key names follow the Qwen3-TTS checkpoint layout the reference reads through qwen_tts
(``talker.model.*``, ``talker.codec_head``, ``talker.code_predictor.*``; see
/root/reference/qwentts_turbo/megakernel_backbone.py:358-409,
/root/reference/qwentts_turbo/megakernel_code_predictor.py:265-316 and
/root/reference/qwentts_turbo/generator.py:55-69).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Mapping, Optional

import torch

HIDDEN_SIZE = 1024
INTERMEDIATE_SIZE = 3072
NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
ROPE_THETA = 1e6

# 11 tensors per layer, in the order of the reference's TTSLayerWeights struct
LAYER_KEYS = (
    "input_layernorm.weight",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.q_norm.weight",
    "self_attn.k_norm.weight",
    "self_attn.o_proj.weight",
    "post_attention_layernorm.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)

BB_PREFIX = "talker.model."
CP_PREFIX = "talker.code_predictor.model."


def as_state_dict(model) -> Mapping[str, torch.Tensor]:
    """Accept a state dict, an nn.Module (``state_dict()``) or any object exposing one."""
    if isinstance(model, Mapping):
        return model
    if hasattr(model, "state_dict"):
        return model.state_dict()
    raise TypeError("model must be a state dict or a module with state_dict()")


def count_layers(sd: Mapping[str, torch.Tensor], prefix: str) -> int:
    n = 0
    while f"{prefix}layers.{n}.input_layernorm.weight" in sd:
        n += 1
    return n


def count_groups(sd: Mapping[str, torch.Tensor]) -> int:
    n = 0
    while f"talker.code_predictor.lm_head.{n}.weight" in sd:
        n += 1
    return n


def layer_list(sd: Mapping[str, torch.Tensor], prefix: str, n_layers: int, device=None) -> List[torch.Tensor]:
    out = []
    for i in range(n_layers):
        for k in LAYER_KEYS:
            t = sd[f"{prefix}layers.{i}.{k}"]
            if device is not None:
                t = t.to(device)
            out.append(t.to(torch.bfloat16).contiguous())
    return out


def rope_tables(max_seq_len: int, theta: float = ROPE_THETA, head_dim: int = HEAD_DIM, device="cuda"):
    """bf16 cos/sin [max_seq_len, head_dim]: cat(freqs, freqs) with inv_freq = theta^(-i/half),
    computed in f32 then cast (megakernel_backbone.py:392-398)."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    pos = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return (torch.cos(emb).to(torch.bfloat16).to(device).contiguous(),
            torch.sin(emb).to(torch.bfloat16).to(device).contiguous())


@dataclass
class SyntheticConfig:
    n_bb_layers: int = 28
    n_cp_layers: int = 5
    vocab: int = 3072
    cp_vocab: int = 2048
    n_groups: int = 15
    std: float = 0.02
    norm_mean: float = 1.0   # RMSNorm gains ~ N(norm_mean, std); 0.0 gives the literal N(0, 0.02)


def synthetic_state_dict(seed: int = 1234, cfg: Optional[SyntheticConfig] = None, device="cpu") -> Dict[str, torch.Tensor]:
    """Seeded random-init bf16 weights with the Qwen3-TTS 0.6B talker layout.

    Every tensor is drawn in a fixed key order from one ``torch.Generator`` on ``device``
    (CPU generation is reproducible across machines with the same torch build)."""
    cfg = cfg or SyntheticConfig()
    g = torch.Generator(device=device).manual_seed(seed)
    H, I, QS, KS = HIDDEN_SIZE, INTERMEDIATE_SIZE, NUM_Q_HEADS * HEAD_DIM, NUM_KV_HEADS * HEAD_DIM
    shapes = {
        "input_layernorm.weight": (H,), "self_attn.q_proj.weight": (QS, H), "self_attn.k_proj.weight": (KS, H),
        "self_attn.v_proj.weight": (KS, H), "self_attn.q_norm.weight": (HEAD_DIM,), "self_attn.k_norm.weight": (HEAD_DIM,),
        "self_attn.o_proj.weight": (H, QS), "post_attention_layernorm.weight": (H,), "mlp.gate_proj.weight": (I, H),
        "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I),
    }

    def draw(shape, is_norm=False):
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * cfg.std
        if is_norm:
            t = t + cfg.norm_mean
        return t.to(torch.bfloat16)

    sd: Dict[str, torch.Tensor] = {}
    sd[BB_PREFIX + "codec_embedding.weight"] = draw((cfg.vocab, H))
    for i in range(cfg.n_bb_layers):
        for k in LAYER_KEYS:
            sd[f"{BB_PREFIX}layers.{i}.{k}"] = draw(shapes[k], "norm" in k)
    sd[BB_PREFIX + "norm.weight"] = draw((H,), True)
    sd["talker.codec_head.weight"] = draw((cfg.vocab, H))
    for i in range(cfg.n_cp_layers):
        for k in LAYER_KEYS:
            sd[f"{CP_PREFIX}layers.{i}.{k}"] = draw(shapes[k], "norm" in k)
    sd[CP_PREFIX + "norm.weight"] = draw((H,), True)
    for gi in range(cfg.n_groups):
        sd[f"{CP_PREFIX}codec_embedding.{gi}.weight"] = draw((cfg.cp_vocab, H))
    for gi in range(cfg.n_groups):
        sd[f"talker.code_predictor.lm_head.{gi}.weight"] = draw((cfg.cp_vocab, H))
    return sd


def to_device(sd: Mapping[str, torch.Tensor], device="cuda") -> Dict[str, torch.Tensor]:
    return {k: v.to(device).contiguous() for k, v in sd.items()}


def load_local(model_path: str) -> Dict[str, torch.Tensor]:
    """Load ``*.safetensors`` from a local directory (no network access, nothing executed)."""
    from pathlib import Path
    from safetensors.torch import load_file
    p = Path(model_path)
    files = sorted(p.glob("*.safetensors")) if p.is_dir() else [p]
    if not files or not all(f.exists() for f in files):
        raise FileNotFoundError(f"no safetensors weights at {model_path!r} (only local paths are supported)")
    sd: Dict[str, torch.Tensor] = {}
    for f in files:
        sd.update(load_file(str(f)))
    return sd
