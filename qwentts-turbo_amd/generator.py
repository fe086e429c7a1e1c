"""NativeTTSGenerator: the reference's generation loop with every per-token step on MI355X.

Mirrors /root/reference/qwentts_turbo/generator.py:21-362 and keeps ``generate()``'s signature
(:77-81). What moved on-device, per codec frame:
  * the whole code-predictor loop (:309-354) -- 2-token prefill, 14 decode steps, 15 lm-heads
    with token selection and embedding gathers -- plus the 16-codebook embedding combine and
    the text/pad add (:143-149, :356-362): one ``qtts_cp_frame`` launch;
  * the backbone step, codec head, suppress mask, repetition penalty, EOS suppression and
    group-0 selection (:152-172): one ``qtts_backbone_step`` launch.
The host enqueues frames without waiting and checks the EOS flag every ``sync_every`` frames
(the reference synchronises 16 times per frame through ``.item()``).

Differences (by design):
  * sampling draws with Gumbel-max over Philox-4x64-10 noise instead of torch.multinomial
    (same distribution; reproducible on device). Greedy decoding is unchanged.
  * the prefill (:209-225) and the KV handoff (:245-257) are one ``qtts_backbone_prefill`` call:
    the transformers bf16 forward of the whole prompt on MFMA, K/V written straight into the
    decode cache, and the first group-0 token selected from its codec-head logits on device
    (``prefill="mfma"``, default). ``prefill="steps"`` instead steps the decode kernel token by
    token (kernel precision). ``attention_mask`` must be all ones (batch 1, no padding).
  * only the megakernel backends exist (``backend="pytorch"`` needs qwen_tts, which this
    build does not ship).
"""
from __future__ import annotations

from typing import List, Optional

import torch

from .megakernel_backbone import TTSMegakernelGenerator
from .megakernel_code_predictor import CodePredictorMegakernelGenerator
from .weights import as_state_dict, load_local


def _config_value(model, *names):
    cfg = getattr(model, "config", None)
    for n in names:
        cur = cfg
        for part in n.split("."):
            cur = getattr(cur, part, None) if cur is not None else None
        if cur is not None:
            return cur
    return None


class NativeTTSGenerator:
    """Native TTS generation loop (generator.py:21-75)."""

    def __init__(self, model_path: Optional[str] = None, model=None, backend: str = "megakernel",
                 cp_backend: str = "megakernel", *, eos_token_id: Optional[int] = None,
                 vocab_size: Optional[int] = None, max_seq_len: int = 4096, device="cuda"):
        for name, b in (("backend", backend), ("cp_backend", cp_backend)):
            if b != "megakernel":
                raise ValueError(f"{name}={b!r}: only the 'megakernel' backend is available on MI355X "
                                 "(the reference's 'pytorch' backend needs the qwen_tts package)")
        self.backend, self.cp_backend = backend, cp_backend
        if model is None:
            if model_path is None:
                raise ValueError("pass model (state dict / module) or a local model_path")
            model = load_local(model_path)
        eos = eos_token_id if eos_token_id is not None else _config_value(model, "talker_config.codec_eos_token_id")
        if eos is None:
            raise ValueError("eos_token_id is required (not found in model.config.talker_config)")
        sd = as_state_dict(model)
        self.backbone_mega = TTSMegakernelGenerator(model=sd, max_seq_len=max_seq_len, device=device)
        self.cp_mega = CodePredictorMegakernelGenerator(model=sd, max_seq_len=32, device=device)
        if self.cp_mega.n_groups == 0:
            raise KeyError("model has no code-predictor lm-heads")
        self.eos_token_id = int(eos)
        self.vocab_size = int(vocab_size if vocab_size is not None else self.backbone_mega.vocab_size)
        self.device = torch.device(device)
        self.n_groups = self.cp_mega.n_groups
        # suppress mask of generator.py:71-75 (applied in-kernel; kept for inspection)
        self.suppress_mask = torch.zeros(self.vocab_size, dtype=torch.bool, device=self.device)
        self.suppress_mask[max(self.vocab_size - 1024, 0):] = True
        if 0 <= self.eos_token_id < self.vocab_size:
            self.suppress_mask[self.eos_token_id] = False

    def generate(self, talker_input_embeds, attention_mask, trailing_text_hidden, tts_pad_embed, max_tokens=500,
                 do_sample=False, temperature=0.9, top_k=50, top_p=1.0, cp_do_sample=False, cp_temperature=0.9,
                 cp_top_k=50, min_new_tokens=2, repetition_penalty=1.0, *, seed: int = 0,
                 sync_every: int = 8, prefill: str = "mfma") -> List[List[int]]:
        """Run the generation loop; returns one [16] codec id list per frame (generator.py:77-176)."""
        if prefill not in ("mfma", "steps"):
            raise ValueError(f"prefill={prefill!r}: 'mfma' or 'steps'")
        dev = self.device
        bb, cp = self.backbone_mega.decoder, self.cp_mega.decoder
        emb = talker_input_embeds
        if emb.dim() != 3 or emb.shape[0] != 1 or emb.shape[2] != 1024:
            raise ValueError(f"talker_input_embeds must be [1, seq, 1024], got {tuple(emb.shape)}")
        if attention_mask is not None and not bool((attention_mask != 0).all()):
            raise ValueError("attention_mask must be all ones (batch-1 prefill without padding)")
        seq = emb.shape[1]
        max_tokens = int(max_tokens)
        if seq < 1 or seq + max_tokens > self.backbone_mega.max_seq_len:
            raise ValueError(f"prefill {seq} + max_tokens {max_tokens} exceeds max_seq_len {self.backbone_mega.max_seq_len}")
        emb = emb[0].to(dev, torch.bfloat16).contiguous()
        text = trailing_text_hidden[0].to(dev, torch.bfloat16).contiguous()
        pad = tts_pad_embed.reshape(-1).to(dev, torch.bfloat16).contiguous()
        i32 = dict(dtype=torch.int32, device=dev)
        g0 = torch.zeros(1, **i32)
        done = torch.zeros(1, **i32)
        hist = torch.zeros(max(max_tokens, 1), **i32)
        records = torch.full((max(max_tokens, 1), 16), -1, **i32)
        combined = torch.empty(1024, dtype=torch.bfloat16, device=dev)

        # 1. prefill (positions 0..seq-1) and the first group-0 token
        bb.reset()
        if prefill == "mfma":
            bb.prefill(emb, g0, self.eos_token_id, min_new_tokens > 0, bool(do_sample), float(temperature),
                       int(top_k), float(top_p), int(seed))
        else:
            for i in range(seq - 1):
                bb.decode_step_with_embedding(emb[i])
            bb.decode_step_select(emb[seq - 1], g0, hist, 0, float(repetition_penalty), self.eos_token_id,
                                  min_new_tokens > 0, bool(do_sample), float(temperature), int(top_k), float(top_p),
                                  int(seed), 0)
        hidden = bb.hidden_state_buffer()

        # 2. frame loop, queued on the device; EOS checked every sync_every frames
        n_text = text.shape[0]
        for step in range(max_tokens):
            row = text[step] if step < n_text else pad
            cp.frame(hidden, g0, row, records[step], combined, self.eos_token_id, done, bool(cp_do_sample),
                     float(cp_temperature), int(cp_top_k), 1.0, int(seed), step, hist[step:step + 1])
            bb.decode_step_select(combined, g0, hist, step + 1, float(repetition_penalty), self.eos_token_id,
                                  step + 1 < min_new_tokens, bool(do_sample), float(temperature), int(top_k),
                                  float(top_p), int(seed), step + 1, None, done)
            if (step + 1) % sync_every == 0 and int(done.item()) != 0:
                break
        rec = records.cpu()
        bb.check_error()
        out = []
        for r in rec.tolist():
            if r[0] < 0:
                break
            out.append(r[: 1 + self.n_groups])
        return out
