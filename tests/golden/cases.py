"""Seeded inputs of the golden cases, shared by the fixture writer
``make_golden.py`` and the tests that read the fixtures. Everything is drawn on the CPU with
``torch.Generator`` so the GPU tests rebuild the same tensors before moving them to the device.

  c0  backbone step: 28 layers, KV prefilled by 128 tokens, decode at position 128 (L=129)
  c1  code-predictor frame: 15 greedy groups from a backbone hidden and a group-0 id
  c2  frame loop: 128-token prefill, 64 greedy frames; 32 sampled frames (top-k 50, T 0.9);
      12 frames with every head sampled (code predictor too, cp_do_sample)
  c3  long context: KV of 2044 tokens, 4 decode steps with distinct monotone (t, h, w)
  c4  batch of 8 streams with ragged attended lengths in [128, 1024]: one backbone step
      (codec head, suppress mask, greedy g0) and one code-predictor frame per stream
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
SEEDS = {"c0": 1234, "c1": 1235, "c2": 1236, "c3": 1237, "c4": 1238}
C4_STREAMS = 8
EOS_ID = 2150
C2_GREEDY_FRAMES = 64
C2_SAMPLED_FRAMES = 32
C2_SAMPLING = dict(do_sample=True, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05, seed=7)
# sampled backbone and sampled code predictor (generate(cp_do_sample=True)): every head samples
C2_CP_SAMPLED_FRAMES = 12
C2_CP_SAMPLING = dict(do_sample=True, temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.05, seed=11,
                      cp_do_sample=True, cp_temperature=0.8, cp_top_k=40)
C3_KV = 2044
C3_STEPS = 4


def weights(pkg, case: str, norm_mean: float = 1.0):
    return pkg.synthetic_state_dict(seed=SEEDS[case], cfg=pkg.SyntheticConfig(norm_mean=norm_mean))


def weight_digest(sd) -> str:
    """sha256 over a few tensors' bytes: detects any drift of the seeded weight generator."""
    h = hashlib.sha256()
    for k in ("talker.model.layers.0.self_attn.q_proj.weight", "talker.model.layers.27.mlp.down_proj.weight",
              "talker.codec_head.weight", "talker.code_predictor.lm_head.14.weight",
              "talker.model.layers.5.input_layernorm.weight"):
        h.update(sd[k].contiguous().view(torch.int16).numpy().tobytes())
    return h.hexdigest()


def _gen(case: str, salt: int = 100) -> torch.Generator:
    return torch.Generator().manual_seed(SEEDS[case] + salt)


def c0_inputs():
    g = _gen("c0")
    prefill = torch.randn(128, 1024, generator=g).to(torch.bfloat16)
    x = torch.randn(1024, generator=g).to(torch.bfloat16)
    return prefill, x


def c1_inputs():
    g = _gen("c1")
    hidden = torch.randn(1024, generator=g)
    g0 = int(torch.randint(0, 2048, (1,), generator=g))
    text = torch.randn(1024, generator=g).to(torch.bfloat16)
    return hidden, g0, text


def c2_inputs():
    g = _gen("c2")
    prefill = torch.randn(1, 128, 1024, generator=g).to(torch.bfloat16)
    trailing = torch.randn(1, 32, 1024, generator=g).to(torch.bfloat16)
    pad = torch.randn(1, 1, 1024, generator=g).to(torch.bfloat16)
    return prefill, trailing, pad


def c3_pos3(i: int):
    """Distinct monotone (t, h, w) sequences: t = i, h = i // 2 + 5, w = i // 3 + 11."""
    return (i, i // 2 + 5, i // 3 + 11)


def c3_inputs():
    g = _gen("c3")
    k = torch.randn(28, 8, C3_KV, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(28, 8, C3_KV, 128, generator=g).to(torch.bfloat16)
    xs = torch.randn(C3_STEPS, 1024, generator=g).to(torch.bfloat16)
    return k, v, xs


def c4_lengths():
    """Ragged attended KV lengths of the 8 streams, uniform in [128, 1024]."""
    g = _gen("c4")
    return [int(x) for x in torch.randint(128, 1025, (C4_STREAMS,), generator=g)]


def c4_stream_inputs(s: int, L: int):
    """Stream s: KV of L - 1 cached tokens, the decode input, the text row of its frame."""
    g = _gen("c4", 200 + s)
    k = torch.randn(28, 8, L - 1, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(28, 8, L - 1, 128, generator=g).to(torch.bfloat16)
    x = torch.randn(1024, generator=g).to(torch.bfloat16)
    text = torch.randn(1024, generator=g).to(torch.bfloat16)
    return k, v, x, text


def load(name: str):
    import numpy as np
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
