"""Decode of several independent streams (batch 8, ragged KV lengths).

Each stream keeps its own backbone KV cache and position; all streams share one copy of the
weights and one code-predictor decoder. A frame of the batch is two launches per 8 streams: the
backbone steps (codec head + selection) and the code-predictor frames, queued on the current
stream with no host sync. Two kernels serve them:

* ``mode="shared"`` (default): the weight-shared kernels. Every weight byte is read once per
  launch for all streams: each workgroup applies its weight tile to the 8 streams' inputs at once
  on bf16 MFMA (each f32 input split exactly into three bf16 pieces, f32 sums), and wave s of
  every workgroup does stream s's vector work. Results agree with batch 1 to f32 rounding.
* ``mode="per_xcd"``: stream s runs on XCD s alone, its 32 workgroups acting as the 8 virtual
  XCDs of the batch-1 decomposition (every exchange in that XCD's L2), and every stream's results
  are bit-identical to its batch-1 results; each XCD reads the whole weight set for its stream.

The reference has no batched decode (its megakernels are batch 1, fused_decode_tts.cu:728-831).
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from .megakernel_backbone import TTSMegakernelGenerator
from .megakernel_code_predictor import CodePredictorMegakernelGenerator


class BatchedTTSDecoder:
    """``n_streams`` backbone decoders over shared weights plus one code predictor."""

    MAX_PER_LAUNCH = 8   # streams per launch (one per wave, or one per XCD)
    MODES = ("shared", "per_xcd")

    def __init__(self, model, n_streams: int, max_seq_len: int = 4096, cp_max_seq_len: int = 32,
                 device="cuda", mode: str = "shared"):
        if n_streams < 1:
            raise ValueError("n_streams must be >= 1")
        if mode not in self.MODES:
            raise ValueError(f"mode={mode!r}: one of {self.MODES}")
        self.mode = mode
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
                    frame_step: int = 0, skip: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One backbone step per stream at its own position, codec head, suppress mask (ids
        [V-1024, V) except EOS), optional repetition penalty over ``history[s][:n_history[s]]``
        and selection of each stream's group-0 token into ``tokens_out[s]`` (device int32), with
        sampling key ``seed + s``. Up to 8 streams share one launch (``decode_steps_streams``).

        ``skip`` (device int32 [n]) marks finished streams, and skipping is terminal: a stream
        whose ``skip[s]`` is nonzero computes nothing, writes no KV entry and leaves its token,
        logits and residual as they were, but its position still advances (the host does not
        read the flag, so no launch waits on the device), so its cache holds an unwritten slot
        and the stream must not be resumed. Its row of the returned hiddens is zero. Returns the
        final-norm hiddens (f32 [n_streams, 1024], device)."""
        if skip is not None and (skip.dtype != torch.int32 or skip.numel() != self.n_streams or not skip.is_contiguous()):
            raise ValueError("skip must be a contiguous device int32 tensor with one entry per stream")
        if embeds.shape != (self.n_streams, 1024):
            raise ValueError(f"embeds must be [{self.n_streams}, 1024], got {tuple(embeds.shape)}")
        if tokens_out.dtype != torch.int32 or tokens_out.numel() < self.n_streams:
            raise ValueError("tokens_out must be a device int32 tensor with one entry per stream")
        emb = embeds.to(self.device, torch.bfloat16).contiguous()
        hist = history.to(self.device, torch.int32).contiguous() if history is not None else None
        nh = [int(x) for x in n_history] if n_history else [0] * self.n_streams
        # zeros: a skipped stream's row is not written by the kernel
        hidden = torch.zeros(self.n_streams, 1024, dtype=torch.float32, device=self.device)
        lead = self.streams[0].decoder
        for b in range(0, self.n_streams, self.MAX_PER_LAUNCH):
            e = min(self.n_streams, b + self.MAX_PER_LAUNCH)
            lead.decode_steps_streams([d.decoder for d in self.streams[b:e]], emb[b:e], tokens_out[b:e],
                                      hidden[b:e], hist[b:e] if hist is not None else None, nh[b:e],
                                      float(repetition_penalty), int(eos_id), bool(suppress_eos), bool(do_sample),
                                      float(temperature), int(top_k), float(top_p), int(seed) + b, int(frame_step),
                                      skip[b:e] if skip is not None else None, self.mode == "shared")
        return hidden

    def cp_frames(self, hidden: torch.Tensor, g0: torch.Tensor, text_rows: Optional[torch.Tensor],
                  tokens_out: torch.Tensor, combined_out: torch.Tensor, eos_id: int = -1,
                  do_sample: bool = False, temperature: float = 0.9, top_k: int = 50, seed: int = 0,
                  frame_step: int = 0, done: Optional[torch.Tensor] = None) -> None:
        """A code-predictor frame per stream: ``tokens_out[s]`` (int32 [16]) gets g0 and the 15
        group ids, ``combined_out[s]`` (bf16 [1024]) the embedding sum plus ``text_rows[s]``.
        A stream whose g0 is ``eos_id`` writes nothing and sets ``done[s]`` (device int32 [n],
        kept by the caller across frames; a fresh one when None). Up to 8 streams share one
        launch (``frames_streams``); stream s draws with key ``seed + s``."""
        n = self.n_streams
        if done is None:
            done = torch.zeros(n, dtype=torch.int32, device=self.device)
        elif done.dtype != torch.int32 or done.numel() != n or not done.is_contiguous():
            raise ValueError("done must be a contiguous device int32 tensor with one entry per stream")
        hid = hidden.to(self.device, torch.float32).contiguous()
        g = g0.to(self.device, torch.int32).contiguous()
        tr = text_rows.to(self.device, torch.bfloat16).contiguous() if text_rows is not None else None
        for b in range(0, n, self.MAX_PER_LAUNCH):
            e = min(n, b + self.MAX_PER_LAUNCH)
            self.cp.decoder.frames_streams(hid[b:e], g[b:e], tr[b:e] if tr is not None else None, tokens_out[b:e],
                                           combined_out[b:e], int(eos_id), done[b:e], bool(do_sample),
                                           float(temperature), int(top_k), 1.0, int(seed) + b, int(frame_step),
                                           self.mode == "shared")

    def generate(self, talker_input_embeds: Sequence[torch.Tensor], trailing_text_hidden: Sequence[torch.Tensor],
                 tts_pad_embed: torch.Tensor, eos_token_id: int, max_tokens: int = 500, do_sample: bool = False,
                 temperature: float = 0.9, top_k: int = 50, top_p: float = 1.0, cp_do_sample: bool = False,
                 cp_temperature: float = 0.9, cp_top_k: int = 50, min_new_tokens: int = 2,
                 repetition_penalty: float = 1.0, *, seed: int = 0, sync_every: int = 8,
                 prefill: str = "mfma") -> List[List[List[int]]]:
        """``NativeTTSGenerator.generate`` (generator.py:77-176) for ``n_streams`` utterances at
        once: one prompt ``[1, seq_s, 1024]`` and one trailing text ``[1, T_s, 1024]`` per stream
        (ragged lengths), a shared pad row. Each stream is prefilled on its own, then every frame
        is one code-predictor launch and one backbone launch for all streams, queued with no host
        sync; the host checks the EOS flags every ``sync_every`` frames and stops when every
        stream has ended. Stream s samples with key ``seed + s``; in ``per_xcd`` mode it returns
        exactly what a single-stream ``generate(..., seed=seed + s)`` returns for its inputs, in
        ``shared`` mode the same up to choices that f32 rounding can tip (near-ties)."""
        n = self.n_streams
        if len(talker_input_embeds) != n or len(trailing_text_hidden) != n:
            raise ValueError(f"one prompt and one trailing text per stream ({n}) expected")
        if prefill not in ("mfma", "steps"):
            raise ValueError(f"prefill={prefill!r}: 'mfma' or 'steps'")
        dev = self.device
        max_tokens = int(max_tokens)
        groups = self.cp.n_groups
        i32 = dict(dtype=torch.int32, device=dev)
        g0 = torch.zeros(n, **i32)
        done = torch.zeros(n, **i32)
        hist = torch.zeros(n, max(max_tokens, 1), **i32)
        records = torch.full((max(max_tokens, 1), n, groups + 1), -1, **i32)
        combined = torch.empty(n, 1024, dtype=torch.bfloat16, device=dev)
        pad = tts_pad_embed.reshape(-1).to(dev, torch.bfloat16)
        # per-stream text rows for every frame (the trailing text, then the pad row)
        rows = pad.expand(n, max(max_tokens, 1), 1024).clone()
        hidden = torch.empty(n, 1024, dtype=torch.float32, device=dev)
        # every stream's arguments are checked before any stream is touched
        for s in range(n):
            emb, txt = talker_input_embeds[s], trailing_text_hidden[s]
            if emb.dim() != 3 or emb.shape[0] != 1 or emb.shape[2] != 1024:
                raise ValueError(f"prompt {s} must be [1, seq, 1024], got {tuple(emb.shape)}")
            if txt.dim() != 3 or txt.shape[0] != 1 or txt.shape[2] != 1024:
                raise ValueError(f"trailing text {s} must be [1, T, 1024], got {tuple(txt.shape)}")
            seq = emb.shape[1]
            if seq < 1 or seq + max_tokens > self.streams[s].max_seq_len:
                raise ValueError(f"stream {s}: prefill {seq} + max_tokens {max_tokens} exceeds max_seq_len "
                                 f"{self.streams[s].max_seq_len}")
        for s in range(n):
            emb = talker_input_embeds[s]
            seq = emb.shape[1]
            dec = self.streams[s]
            text = trailing_text_hidden[s][0].to(dev, torch.bfloat16)
            t = min(int(text.shape[0]), max_tokens)
            rows[s, :t] = text[:t]
            e = emb[0].to(dev, torch.bfloat16).contiguous()
            bb = dec.decoder
            bb.reset()
            if prefill == "mfma":
                bb.prefill(e, g0[s:s + 1], int(eos_token_id), min_new_tokens > 0, bool(do_sample),
                           float(temperature), int(top_k), float(top_p), int(seed) + s)
            else:
                for i in range(seq - 1):
                    bb.decode_step_with_embedding(e[i])
                bb.decode_step_select(e[seq - 1], g0[s:s + 1], hist[s], 0, float(repetition_penalty),
                                      int(eos_token_id), min_new_tokens > 0, bool(do_sample), float(temperature),
                                      int(top_k), float(top_p), int(seed) + s, 0)
            hidden[s] = bb.hidden_state_buffer()
        for step in range(max_tokens):
            self.cp_frames(hidden, g0, rows[:, step].contiguous(), records[step], combined, int(eos_token_id),
                           bool(cp_do_sample), float(cp_temperature), int(cp_top_k), int(seed), step, done)
            hist[:, step] = g0          # this frame's group 0 joins the penalty history
            hidden = self.step_select(combined, g0, int(eos_token_id), hist, [step + 1] * n,
                                      float(repetition_penalty), step + 1 < min_new_tokens, bool(do_sample),
                                      float(temperature), int(top_k), float(top_p), int(seed), step + 1,
                                      skip=done)   # streams that reached EOS compute nothing
            if (step + 1) % sync_every == 0 and bool(done.all()):
                break
        rec = records.cpu()
        self.check_error()
        out = []
        for s in range(n):
            frames = []
            for r in rec[:, s].tolist():
                if r[0] < 0:
                    break
                frames.append(r)
            out.append(frames)
        return out

    def check_error(self):
        for dec in self.streams:
            dec.check_error()
        self.streams[0].decoder.check_error_streams()
        self.cp.check_error()
        self.cp.decoder.check_error_streams()
