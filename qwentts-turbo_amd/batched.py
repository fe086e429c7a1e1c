"""Decode of several independent streams (batch 8, ragged KV lengths).

Each stream keeps its own backbone KV cache and position; all streams share one copy of the
weights and one code-predictor decoder. A frame of the batch is two launches per 8 streams: the
backbone steps (codec head + selection) and the code-predictor frames. In both, stream s runs
on XCD s alone, its 32 workgroups acting as the 8 virtual XCDs of the batch-1 decomposition,
so every exchange stays in that XCD's L2. Everything is queued on
the current stream with no host sync, and every stream's results are bit-identical to its
batch-1 results.

The reference has no batched decode (its megakernels are batch 1, fused_decode_tts.cu:728-831).
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from .megakernel_backbone import TTSMegakernelGenerator
from .megakernel_code_predictor import CodePredictorMegakernelGenerator


class BatchedTTSDecoder:
    """``n_streams`` backbone decoders over shared weights plus one code predictor."""

    MAX_PER_LAUNCH = 8   # streams per launch: one per XCD

    def __init__(self, model, n_streams: int, max_seq_len: int = 4096, cp_max_seq_len: int = 32,
                 device="cuda"):
        if n_streams < 1:
            raise ValueError("n_streams must be >= 1")
        first = TTSMegakernelGenerator(model=model, max_seq_len=max_seq_len, device=device)
        self.streams: List[TTSMegakernelGenerator] = [first] + [
            TTSMegakernelGenerator(max_seq_len=max_seq_len, device=device, shared_weights=first.weights)
            for _ in range(n_streams - 1)]
        self.cp = CodePredictorMegakernelGenerator(model=model, max_seq_len=cp_max_seq_len, device=device)
        self.n_streams = n_streams
        self.device = torch.device(device)
        self.vocab_size = self.streams[0].vocab_size

    def set_kv_cache(self, stream: int, k: torch.Tensor, v: torch.Tensor):
        """Prefix KV of one stream ([layers, 8, S, 128]); the stream continues at position S."""
        dec = self.streams[stream]
        dec.set_kv_cache(k, v)
        dec.set_position(int(k.shape[2]))

    def positions(self) -> List[int]:
        return [s.position for s in self.streams]

    def step_select(self, embeds: torch.Tensor, tokens_out: torch.Tensor, eos_id: int,
                    history: Optional[torch.Tensor] = None, n_history: Sequence[int] = (),
                    repetition_penalty: float = 1.0, suppress_eos: bool = False, do_sample: bool = False,
                    temperature: float = 0.9, top_k: int = 50, top_p: float = 1.0, seed: int = 0,
                    frame_step: int = 0) -> torch.Tensor:
        """One backbone step per stream at its own position, codec head, suppress mask (ids
        [V-1024, V) except EOS), optional repetition penalty over ``history[s][:n_history[s]]``
        and selection of each stream's group-0 token into ``tokens_out[s]`` (device int32), with
        sampling key ``seed + s``. Up to 8 streams share one launch, stream s on XCD s
        (``decode_steps_streams``). Returns the final-norm hiddens (f32 [n_streams, 1024], device)."""
        if embeds.shape != (self.n_streams, 1024):
            raise ValueError(f"embeds must be [{self.n_streams}, 1024], got {tuple(embeds.shape)}")
        if tokens_out.dtype != torch.int32 or tokens_out.numel() < self.n_streams:
            raise ValueError("tokens_out must be a device int32 tensor with one entry per stream")
        emb = embeds.to(self.device, torch.bfloat16).contiguous()
        hist = history.to(self.device, torch.int32).contiguous() if history is not None else None
        nh = [int(x) for x in n_history] if n_history else [0] * self.n_streams
        hidden = torch.empty(self.n_streams, 1024, dtype=torch.float32, device=self.device)
        lead = self.streams[0].decoder
        for b in range(0, self.n_streams, self.MAX_PER_LAUNCH):
            e = min(self.n_streams, b + self.MAX_PER_LAUNCH)
            lead.decode_steps_streams([d.decoder for d in self.streams[b:e]], emb[b:e], tokens_out[b:e],
                                      hidden[b:e], hist[b:e] if hist is not None else None, nh[b:e],
                                      float(repetition_penalty), int(eos_id), bool(suppress_eos), bool(do_sample),
                                      float(temperature), int(top_k), float(top_p), int(seed) + b, int(frame_step))
        return hidden

    def cp_frames(self, hidden: torch.Tensor, g0: torch.Tensor, text_rows: Optional[torch.Tensor],
                  tokens_out: torch.Tensor, combined_out: torch.Tensor, eos_id: int = -1,
                  do_sample: bool = False, temperature: float = 0.9, top_k: int = 50, seed: int = 0,
                  frame_step: int = 0) -> None:
        """A code-predictor frame per stream: ``tokens_out[s]`` (int32 [16]) gets g0 and the 15
        group ids, ``combined_out[s]`` (bf16 [1024]) the embedding sum plus ``text_rows[s]``.
        Up to 8 streams share one launch, stream s on XCD s (``frames_streams``); stream s draws
        with key ``seed + s``."""
        n = self.n_streams
        done = torch.zeros(n, dtype=torch.int32, device=self.device)
        hid = hidden.to(self.device, torch.float32).contiguous()
        g = g0.to(self.device, torch.int32).contiguous()
        tr = text_rows.to(self.device, torch.bfloat16).contiguous() if text_rows is not None else None
        for b in range(0, n, self.MAX_PER_LAUNCH):
            e = min(n, b + self.MAX_PER_LAUNCH)
            self.cp.decoder.frames_streams(hid[b:e], g[b:e], tr[b:e] if tr is not None else None, tokens_out[b:e],
                                           combined_out[b:e], int(eos_id), done[b:e], bool(do_sample),
                                           float(temperature), int(top_k), 1.0, int(seed) + b, int(frame_step))

    def check_error(self):
        for dec in self.streams:
            dec.check_error()
        self.streams[0].decoder.check_error_streams()
        self.cp.check_error()
        self.cp.decoder.check_error_streams()
