"""CPU restatement of qwenTTS-turbo's dual-megakernel decode path (PyTorch on CPU).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the checker. The
product package (``qwentts-turbo_amd/``) never imports it; its decode path runs the HIP
kernels and raises when they are not built.

What it restates (reference file:line):
  * backbone decode step  -- /root/reference/qwentts_turbo/csrc/fused_decode_tts.cu:728-831
    (phases :56-157 QKV+RMSNorm, :163-276 q/k-norm+RoPE+KV write, :282-385 attention,
    :391-547 O-proj/post-norm/SwiGLU/down, :796-830 final norm)
  * code-predictor step   -- /root/reference/qwentts_turbo/csrc/fused_decode_code_predictor.cu:565-668
  * RoPE tables           -- /root/reference/qwentts_turbo/megakernel_backbone.py:392-398,
                             /root/reference/qwentts_turbo/megakernel_code_predictor.py:297-308
  * interleaved 3D mRoPE  -- /root/reference/qwentts_turbo/csrc/rope_multimodal.cuh:9-54 (intent);
                             index map from transformers qwen3_vl ``apply_interleaved_mrope``
  * frame loop, combine, suppress mask, repetition penalty, sampling
                          -- /root/reference/qwentts_turbo/generator.py:71-75, 77-176, 178-207,
                             309-362; /root/reference/tests/test_audio.py:64-184

Precision policies (``policy=``):
  * ``"kernel"``  -- the arithmetic the HIP kernels implement: every dot product, norm and
    softmax accumulates in f64; values are stored as f32 where the reference stores f32
    (q/k/v, attention output, intermediates; here also the per-chunk attention partials and
    the 8 per-XCD partial sums of the O and down projections, which are added to the residual
    in a fixed order in f64) and as bf16 where the reference stores bf16: the backbone residual
    between layers (fused_decode_tts.cu:541) and backbone KV (fused_decode_tts.cu:270-271).
    The code predictor keeps f32 residuals and KV (fused_decode_code_predictor.cu:288-289,
    :553). cos/sin come from the bf16 tables. Logits are ``W_bf16 . bf16(h)`` in f64, rounded
    to bf16 as the reference's bf16 ``torch.mv`` returns them. With f64 accumulation on both sides every f32/bf16 rounding agrees except with
    ~1e-8 probability per value, so greedy tokens are reproducible.
  * ``"exact"``   -- the same formulas in f64 with no storage rounding and f32 cos/sin (the
    values transformers' rotary embedding produces); used to pin the math against
    transformers' Qwen3 modules run in float64.
  * ``"hf_bf16"`` -- the HF PyTorch bf16 path (transformers Qwen3DecoderLayer op order in bf16),
    i.e. what the reference's ``backend="pytorch"`` and its prefill (generator.py:209-225)
    compute. ``hf_sums="f64"`` keeps every bf16 rounding point but forms the projection sums in
    f64 instead of torch's f32 order: the spread between the two is this path's sensitivity to
    summation order alone (a 1-ulp bf16 flip in one op perturbs the next op's sums and flips a
    few percent of its outputs, so the spread grows with depth), the floor any bf16
    implementation with its own summation order (cuBLAS, MFMA) sits at.

Pinning (see tests/test_oracle_*.py): layer math against transformers ``Qwen3DecoderLayer``
(fp32 and bf16), interleaved mRoPE against transformers ``Qwen3VLTextRotaryEmbedding``,
t=h=w reduction to 1D RoPE, GQA against repeated-KV attention, Philox against numpy, sampler
distribution against softmax by exact enumeration. The frame loop (the 2-token CP prefill
``[bf16(h), emb_bb[g0]]`` at positions 0 and 1, ``lm_head[g]`` / ``emb[g-1]`` per group, the
embedding combine plus the text or pad row; generator.py:309-362) against transformers'
Qwen3-Omni talker ``prepare_inputs_for_generation`` and its code predictor's ``generate``, in the
``"exact"`` policy (tests/test_oracle_frame_loop.py). The GPU's code predictor accumulates in f32
(the reference CP kernel's arithmetic) where this policy sums in f64; the two agree to f32
rounding.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .philox import sampler_uniform


@dataclass(frozen=True)
class Dims:
    """Model dimensions; defaults are config.cuh:33-40 of the reference."""
    hidden: int = 1024
    inter: int = 3072
    n_q: int = 16
    n_kv: int = 8
    head_dim: int = 128
    eps: float = 1e-6
    theta: float = 1e6
    mrope_sections: Tuple[int, int, int] = (24, 20, 20)


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


def rb(x: torch.Tensor) -> torch.Tensor:
    """Round an f32 tensor to bf16 and back (round-to-nearest-even)."""
    return x.to(torch.bfloat16).to(torch.float32)


def rope_tables(max_seq: int, head_dim: int, theta: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 cos/sin tables [max_seq, head_dim]: cat(freqs, freqs), inv_freq = theta^(-i/half).

    Follows megakernel_backbone.py:392-398 (and megakernel_code_predictor.py:299-308).
    """
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    pos = torch.arange(max_seq, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return torch.cos(emb).to(torch.bfloat16), torch.sin(emb).to(torch.bfloat16)


def mrope_section_of_channel(head_dim: int, sections: Sequence[int]) -> torch.Tensor:
    """For channel i of the rotary half (i < head_dim/2): 0=T, 1=H, 2=W (interleaved layout).

    H takes ``slice(1, 3*sections[1], 3)``, W takes ``slice(2, 3*sections[2], 3)``, T keeps the
    rest -- the index map of transformers qwen3_vl ``apply_interleaved_mrope`` that the reference
    documents in rope_multimodal.cuh:9-54 (whose 22/21/21 count comment is for unrestricted
    interleaving; with sections [24,20,20] the T section holds 24 channels).
    """
    half = head_dim // 2
    sec = torch.zeros(half, dtype=torch.long)
    for s, off in ((1, 1), (2, 2)):
        sec[off: sections[s] * 3: 3] = s
    return sec


def mrope_cos_sin(cos_t: torch.Tensor, sin_t: torch.Tensor, pos3: Sequence[int],
                  sections: Sequence[int]) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [head_dim] (f32 values of bf16 table entries) for a token at (t, h, w).

    Channel c (and its twin c+half) reads table row pos3[section(c)]; since the 1D table entry
    at row p and channel c is cos(p * inv_freq[c % half]), this equals the interleaved mRoPE
    frequency layout evaluated at the section's position. With t == h == w it is the 1D row.
    """
    head_dim = cos_t.shape[1]
    sec = mrope_section_of_channel(head_dim, sections)
    sec = torch.cat((sec, sec))
    rows = torch.tensor([pos3[int(s)] for s in sec])
    ch = torch.arange(head_dim)
    return cos_t[rows, ch].float(), sin_t[rows, ch].float()


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin on the last dim (fused_decode_tts.cu:211-225)."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


EPS_F32 = float(torch.tensor(1e-6, dtype=torch.float32))   # the reference's 1e-6f
SCALE_F32 = float(torch.tensor(1.0 / math.sqrt(128.0), dtype=torch.float32))  # attn_scale (f32)
MAX_CHUNKS = 16     # attention chunks per KV head in the kernels
SUB_BB, SUB_CP = 64, 2   # chunking granularity (positions per chunk before the chunk cap)
PASS_BB, PASS_CP = 64, 16  # contexts up to this length are attended whole by every workgroup


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """(x * (1 / sqrt(mean(x^2) + eps))) * w (fused_decode_tts.cu:79-108), in x's dtype."""
    var = (x * x).sum(-1, keepdim=True) / x.shape[-1]
    return (x * (1.0 / torch.sqrt(var + eps))) * w


def chunking(L: int, sub: int) -> Tuple[int, int]:
    """Attention split of the kernels: C chunks of P positions ([cP, min((c+1)P, L)))."""
    c0 = min(max((L + sub - 1) // sub, 1), MAX_CHUNKS)
    P = (L + c0 - 1) // c0
    return (L + P - 1) // P, P


def r32(x: torch.Tensor) -> torch.Tensor:
    """Round an f64 tensor to f32 and back."""
    return x.to(torch.float32).to(torch.float64)


def local_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, scale: float, R=lambda t: t) -> torch.Tensor:
    """Decode attention over the whole context in one workgroup (contexts up to one pass of the
    kernels' math waves): f32 scores, out = (sum_p exp(s_p - M) v_p) * (1 / sum_p exp(s_p - M))
    in f64, rounded once (R) at the output -- no per-chunk rounding."""
    scores = R(torch.einsum("hd,hpd->hp", q, K) * scale)
    M = scores.max(dim=-1).values
    p = torch.exp(scores - M[:, None])
    return R(torch.einsum("hp,hpd->hd", p, V) * (1.0 / p.sum(-1))[:, None])


def split_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, scale: float, sub: int,
                    R=lambda t: t) -> torch.Tensor:
    """Decode attention split over sequence chunks and merged (split-K softmax).

    q [h, d], K/V [h, L, d] (f64). The sequence is cut as ``chunking(L, sub)``; chunk c keeps
    its max m_c, its sum l_c = sum exp(s - m_c) and its unnormalised output acc_c; the merge
    rescales by exp(m_c - M) with M the global max (the LDS split-K combine of
    fused_decode_tts.cu:282-385, here over up to MAX_CHUNKS chunks): out = (sum_c acc_c w_c) * (1 / Z),
    Z = sum_c l_c w_c. ``R`` is applied where the kernels store f32: the scores, l_c, acc_c and
    the merged output.
    """
    L = K.shape[1]
    scores = R(torch.einsum("hd,hpd->hp", q, K) * scale)
    C, P = chunking(L, sub)
    ms, ls, accs = [], [], []
    for c in range(C):
        sl = slice(c * P, min((c + 1) * P, L))
        m_c = scores[:, sl].max(dim=-1).values
        p = torch.exp(scores[:, sl] - m_c[:, None])
        ms.append(m_c)
        ls.append(R(p.sum(-1)))
        accs.append(R(torch.einsum("hp,hpd->hd", p, V[:, sl])))
    M = torch.stack(ms).max(dim=0).values
    wts = [torch.exp(m - M) for m in ms]
    Z = sum(lc * wc for wc, lc in zip(wts, ls))
    return R(sum(ac * wc[:, None] for wc, ac in zip(wts, accs)) * (1.0 / Z)[:, None])


def r16(x: torch.Tensor) -> torch.Tensor:
    """Round an f64 tensor to f32, then to bf16 (the kernels' double rounding), back to f64."""
    return x.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def rms_norm_hf(x_bf16: torch.Tensor, w_bf16: torch.Tensor, eps: float) -> torch.Tensor:
    """transformers Qwen3RMSNorm in bf16: f32 normalize, cast to bf16, multiply by bf16 gain."""
    h = x_bf16.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return w_bf16 * h.to(torch.bfloat16)


def silu(x: torch.Tensor) -> torch.Tensor:
    """x / (1 + exp(-x)) (fused_decode_tts.cu:48-50)."""
    return x / (1.0 + torch.exp(-x))


@dataclass
class LayerW:
    ln_in: torch.Tensor
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    qn: torch.Tensor
    kn: torch.Tensor
    o: torch.Tensor
    ln_post: torch.Tensor
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor

    @staticmethod
    def from_list(ts: Sequence[torch.Tensor], dtype) -> "LayerW":
        return LayerW(*[t.detach().to("cpu", dtype).contiguous() for t in ts])


class DecoderOracle:
    """A stack of Qwen3 decoder layers stepped one token at a time with an explicit KV cache.

    ``kind="backbone"``: bf16 residual between layers and bf16 KV under the kernel policy;
    3D mRoPE positions. ``kind="cp"``: f32 residual and f32 KV; 1D RoPE.
    KV layout is [layers, kv_heads, max_seq, head_dim] as in megakernel_backbone.py:156-159.
    """

    def __init__(self, layer_weights: Sequence[Sequence[torch.Tensor]], final_norm: torch.Tensor,
                 max_seq: int, kind: str = "backbone", policy: str = "kernel",
                 dims: Dims = Dims(), hf_sums: str = "torch"):
        assert kind in ("backbone", "cp") and policy in ("kernel", "exact", "hf_bf16")
        assert hf_sums in ("torch", "f64")
        self.kind, self.policy, self.d = kind, policy, dims
        self.hf_sums = hf_sums
        wdt = torch.bfloat16 if policy == "hf_bf16" else torch.float64
        self.layers = [LayerW.from_list(lw, wdt) for lw in layer_weights]
        self.final_norm = final_norm.detach().to("cpu", wdt)
        self.n_layers = len(self.layers)
        self.max_seq = max_seq
        self.cos_t, self.sin_t = rope_tables(max(max_seq, 4096), dims.head_dim, dims.theta)
        if policy == "kernel":
            kv_dtype = torch.bfloat16 if kind == "backbone" else torch.float32
        elif policy == "hf_bf16":
            kv_dtype = torch.bfloat16
        else:
            kv_dtype = torch.float64
        shape = (self.n_layers, dims.n_kv, max_seq, dims.head_dim)
        self.k = torch.zeros(shape, dtype=kv_dtype)
        self.v = torch.zeros(shape, dtype=kv_dtype)
        self.position = 0

    def reset(self):
        self.k.zero_()
        self.v.zero_()
        self.position = 0

    # -- cos/sin for one token -------------------------------------------------------------
    def _cos_sin(self, pos: int, pos3: Optional[Sequence[int]]):
        if self.kind == "backbone" and pos3 is not None:
            c, s = mrope_cos_sin(self.cos_t, self.sin_t, pos3, self.d.mrope_sections)
        else:
            c, s = self.cos_t[pos].float(), self.sin_t[pos].float()
        if self.policy == "exact":
            # f32 cos/sin without the bf16 table rounding, as transformers' rotary embedding
            half = self.d.head_dim // 2
            inv = 1.0 / (self.d.theta ** (torch.arange(0, half, dtype=torch.float32) / half))
            p3 = pos3 if (self.kind == "backbone" and pos3 is not None) else (pos, pos, pos)
            sec = mrope_section_of_channel(self.d.head_dim, self.d.mrope_sections)
            p = torch.tensor([float(p3[int(x)]) for x in sec])
            f = p * inv
            e = torch.cat((f, f))
            c, s = torch.cos(e), torch.sin(e)
        return c, s

    # -- one layer, kernel / exact policy -----------------------------------------------------
    def _layer_f64(self, li: int, r: torch.Tensor, pos: int, cos, sin, trace: Optional[dict]):
        """One decoder layer; ``r`` is the f64 layer input. Returns the layer output (f64)."""
        d, w = self.d, self.layers[li]
        kern = self.policy == "kernel"
        R = r32 if kern else (lambda t: t)
        eps = EPS_F32 if kern else d.eps
        cos, sin = cos.double(), sin.double()
        xn = R(rms_norm(r, w.ln_in, eps))
        q = R(w.q @ xn).view(d.n_q, d.head_dim)
        k = R(w.k @ xn).view(d.n_kv, d.head_dim)
        v = R(w.v @ xn).view(d.n_kv, d.head_dim)
        q = R(rope_apply(rms_norm(q, w.qn, eps), cos, sin))
        k = R(rope_apply(rms_norm(k, w.kn, eps), cos, sin))
        if kern and self.kind == "backbone":
            k, v = r16(k), r16(v)
        self.k[li, :, pos] = k.to(self.k.dtype)
        self.v[li, :, pos] = v.to(self.v.dtype)
        L = pos + 1
        K = self.k[li, :, :L].double()                    # the new token is read back from the cache
        V = self.v[li, :, :L].double()
        grp = d.n_q // d.n_kv
        kv_of_q = torch.arange(d.n_q) // grp               # GQA: q head h uses kv head h // grp
        if not kern:
            scores = torch.einsum("hd,hpd->hp", q, K[kv_of_q]) * (d.head_dim ** -0.5)
            attn = torch.einsum("hp,hpd->hd", torch.softmax(scores, dim=-1), V[kv_of_q]).reshape(-1)
            h1 = r + w.o @ attn
        else:
            if L <= (PASS_BB if self.kind == "backbone" else PASS_CP):
                attn = local_attention(q, K[kv_of_q], V[kv_of_q], SCALE_F32, r32).reshape(-1)
            else:
                attn = split_attention(q, K[kv_of_q], V[kv_of_q], SCALE_F32,
                                       SUB_BB if self.kind == "backbone" else SUB_CP, r32).reshape(-1)
            # O projection as 8 per-XCD partials (XCD x: heads 2x, 2x+1 = columns [256x, 256x+256))
            cols = attn.numel() // 8
            h1 = r.clone()
            for x in range(8):
                h1 = h1 + R(w.o[:, cols * x: cols * (x + 1)] @ attn[cols * x: cols * (x + 1)])
            h1 = R(h1)
        hn = R(rms_norm(h1, w.ln_post, eps))
        g = w.gate @ hn
        a = R(g / (1.0 + torch.exp(-g)) * (w.up @ hn))
        if not kern:
            out = h1 + w.down @ a
        else:
            cols = a.numel() // 8
            out = h1.clone()
            for x in range(8):
                out = out + R(w.down[:, cols * x: cols * (x + 1)] @ a[cols * x: cols * (x + 1)])
            out = R(out)
            if self.kind == "backbone":
                out = r16(out)
        if trace is not None:
            trace.setdefault("attn", []).append(attn.clone())
            trace.setdefault("h1", []).append(h1.clone())
        return out

    # -- one layer, HF bf16 policy (transformers Qwen3DecoderLayer op order) ----------------
    def _linear(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """bf16 projection: torch's own (f32 sums in its order), or f64 sums rounded once."""
        if self.hf_sums == "torch":
            return torch.nn.functional.linear(x, w)
        return (x.double() @ w.double().t()).to(torch.float32).to(x.dtype)

    def _layer_hf(self, li: int, x: torch.Tensor, pos: int, cos, sin, trace):
        d, w = self.d, self.layers[li]
        lin = self._linear
        bf = torch.bfloat16
        cos_b, sin_b = cos.to(bf), sin.to(bf)
        h = rms_norm_hf(x, w.ln_in, d.eps)
        q = lin(h, w.q).view(d.n_q, d.head_dim)
        k = lin(h, w.k).view(d.n_kv, d.head_dim)
        v = lin(h, w.v).view(d.n_kv, d.head_dim)
        q = rms_norm_hf(q, w.qn, d.eps)
        k = rms_norm_hf(k, w.kn, d.eps)
        half = d.head_dim // 2
        q = (q * cos_b) + (torch.cat((-q[..., half:], q[..., :half]), -1) * sin_b)
        k = (k * cos_b) + (torch.cat((-k[..., half:], k[..., :half]), -1) * sin_b)
        self.k[li, :, pos] = k
        self.v[li, :, pos] = v
        K = self.k[li, :, : pos + 1]
        V = self.v[li, :, : pos + 1]
        grp = d.n_q // d.n_kv
        kv_of_q = torch.arange(d.n_q) // grp
        scale = d.head_dim ** -0.5
        qb = q.unsqueeze(1)                                          # [16,1,128]
        sc = torch.matmul(qb, K[kv_of_q].transpose(1, 2).contiguous()) * scale
        p = torch.softmax(sc, dim=-1, dtype=torch.float32).to(bf)
        attn = torch.matmul(p, V[kv_of_q]).reshape(-1)
        o = lin(attn, w.o)
        h1 = x + o
        hn = rms_norm_hf(h1, w.ln_post, d.eps)
        g = lin(hn, w.gate)
        a = torch.nn.functional.silu(g) * lin(hn, w.up)
        out = h1 + lin(a, w.down)
        if trace is not None:
            trace.setdefault("attn", []).append(attn.float().clone())
            trace.setdefault("h1", []).append(h1.float().clone())
        return out

    def step(self, emb: torch.Tensor, pos: Optional[int] = None,
             pos3: Optional[Sequence[int]] = None, trace: Optional[dict] = None):
        """Run one token through all layers; returns (final hidden f32 [H], per-layer outputs).

        ``emb`` is the bf16 input embedding (or any tensor, which is cast to bf16 first, as
        megakernel_backbone.py:235 does). ``pos`` defaults to the running position (the cache
        slot written); ``pos3`` gives (t, h, w) rotary positions for the backbone (default:
        all equal to ``pos``).
        """
        if pos is None:
            pos = self.position
        if pos >= self.max_seq:
            raise ValueError(f"position {pos} >= max_seq {self.max_seq}")
        e = emb.detach().reshape(-1).to("cpu", torch.bfloat16)
        cos, sin = self._cos_sin(pos, pos3)
        outs = []
        if self.policy == "hf_bf16":
            x = e
            for li in range(self.n_layers):
                x = self._layer_hf(li, x, pos, cos, sin, trace)
                outs.append(x.float())
            hidden = rms_norm_hf(x, self.final_norm, self.d.eps).float()
        else:
            r = e.double()
            for li in range(self.n_layers):
                r = self._layer_f64(li, r, pos, cos, sin, trace)
                outs.append(r.float())
            if self.policy == "kernel":
                hidden = rms_norm(r, self.final_norm, EPS_F32).float()
            else:
                hidden = rms_norm(r, self.final_norm, self.d.eps)
        self.position = pos + 1
        return hidden, outs

    def set_kv(self, k: torch.Tensor, v: torch.Tensor):
        """Prefix copy [L, kv, S, hd] into [:, :, :S] with a cast (megakernel_backbone.py:285-294)."""
        s = k.shape[2]
        self.k[:, :, :s] = k.to(self.k.dtype)
        self.v[:, :, :s] = v.to(self.v.dtype)


# ------------------------------------------------------------------------------------------
# Heads, masks and sampling
# ------------------------------------------------------------------------------------------

def head_logits(w: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """W_bf16 . bf16(hidden) accumulated in f64, rounded to f32 and then to bf16, returned as
    f32 tensor of bf16 values: the reference's ``torch.mv`` over bf16 operands returns bf16
    logits (generator.py:158, :351), so greedy ties (lowest id wins, as torch.argmax) are
    those of the reference."""
    wd = w.detach().to("cpu", torch.float64)
    h = hidden.detach().to("cpu", torch.float32).reshape(-1).to(torch.bfloat16).to(torch.float64)
    return rb((wd @ h).to(torch.float32))


def suppress_mask(vocab: int, eos_id: int) -> torch.Tensor:
    """Ids [vocab-1024, vocab) except EOS are suppressed (generator.py:71-75)."""
    m = torch.zeros(vocab, dtype=torch.bool)
    m[max(vocab - 1024, 0):] = True
    if 0 <= eos_id < vocab:
        m[eos_id] = False
    return m


def apply_repetition_penalty(logits: torch.Tensor, history: Sequence[int], penalty: float) -> torch.Tensor:
    """s>0 ? s/p : s*p on each previously generated id, once per distinct id (generator.py:161-167)."""
    if penalty == 1.0 or not history:
        return logits
    out = logits.clone()
    prev = torch.tensor(sorted(set(int(h) for h in history)), dtype=torch.long)
    s = logits[prev]
    # the reference computes on bf16 logits, so each penalised value is rounded to bf16
    out[prev] = rb(torch.where(s > 0, s / penalty, s * penalty))
    return out


def filter_logits(logits: torch.Tensor, temperature: float, top_k: int, top_p: float) -> torch.Tensor:
    """Temperature, top-k and top-p filtering (generator.py:189-204); dropped ids become -inf.

    * temperature: f32 division rounded to bf16, as ``logits / temperature`` on the
      reference's bf16 logits (generator.py:189).
    * top-k keeps every value >= the k-th largest, ties included (generator.py:192-194).
    * top-p keeps x when the softmax mass of the strictly larger kept values is <= top_p,
      with probabilities exp(s - max) summed in f64. On distinct values this is the
      reference's sort / cumsum / shift-by-one rule (generator.py:197-204: position i of the
      descending order survives iff cumprobs[i-1] <= top_p); on exact ties it keeps every
      tied value, which makes the kept set independent of sort order.
    """
    scaled = rb(logits.to(torch.float32) / temperature)
    if top_k > 0 and top_k < scaled.numel():
        kth = torch.topk(scaled, top_k)[0][-1]
        scaled = torch.where(scaled < kth, torch.full_like(scaled, float("-inf")), scaled)
    if top_p < 1.0:
        s = scaled.double()
        fin = torch.isfinite(s)
        m = s[fin].max()
        p = torch.where(fin, torch.exp(s - m), torch.zeros_like(s))
        z = float(p.sum())
        order = torch.argsort(s, descending=True, stable=True)
        sv, pv = s[order], p[order]
        keep = torch.zeros_like(fin)
        acc, i, n = 0.0, 0, s.numel()
        while i < n and torch.isfinite(sv[i]):
            j = i
            while j < n and sv[j] == sv[i]:
                j += 1
            if acc <= float(torch.tensor(top_p, dtype=torch.float32).double()) * z:
                keep[order[i:j]] = True
            acc += float(pv[i:j].sum())
            i = j
        scaled = torch.where(keep, scaled, torch.full_like(scaled, float("-inf")))
    return scaled


def sample_token(logits: torch.Tensor, do_sample: bool, temperature: float, top_k: int,
                 top_p: float, suppress_eos_id: Optional[int] = None, *, seed: int = 0,
                 frame_step: int = 0, group: int = 0) -> int:
    """Greedy argmax (lowest index on ties) or Gumbel-max sampling over the filtered logits.

    Mirrors generator.py:178-207. The reference draws with ``torch.multinomial(softmax(.))``;
    here the draw is ``argmax_i(filtered_i + G_i)`` with ``G_i = -log(-log(U_i))`` and
    ``U_i`` from Philox-4x64-10 at (seed, frame_step, group, i) -- the same distribution, and
    reproducible on the GPU. Scores are compared in float64.
    """
    lg = logits.to(torch.float32).clone()
    if suppress_eos_id is not None:
        lg[suppress_eos_id] = float("-inf")
    if not do_sample:
        m = lg.max()
        return int(torch.nonzero(lg == m)[0, 0]) if torch.isfinite(m) else int(torch.argmax(lg))
    scaled = filter_logits(lg, temperature, top_k, top_p)
    best, best_i = -math.inf, -1
    for i in torch.nonzero(torch.isfinite(scaled)).reshape(-1).tolist():
        u = sampler_uniform(seed, frame_step, group, i)
        score = float(scaled[i]) - math.log(-math.log(u))
        if score > best:
            best, best_i = score, i
    return best_i


# ------------------------------------------------------------------------------------------
# Whole-model oracle: frame loop
# ------------------------------------------------------------------------------------------

@dataclass
class TalkerWeights:
    """The tensors of the decode path, in the reference's extraction order
    (megakernel_backbone.py:358-409, megakernel_code_predictor.py:265-316, generator.py:55-69)."""
    bb_layers: List[List[torch.Tensor]]
    bb_norm: torch.Tensor
    codec_head: torch.Tensor          # [V, H]
    codec_embedding: torch.Tensor     # [V, H]
    cp_layers: List[List[torch.Tensor]]
    cp_norm: torch.Tensor
    cp_heads: List[torch.Tensor]      # 15 x [Vc, H]
    cp_embeddings: List[torch.Tensor]  # 15 x [Vc, H]

    @staticmethod
    def from_state_dict(sd: Dict[str, torch.Tensor], n_bb: int, n_cp: int) -> "TalkerWeights":
        pre, cpre = "talker.model.", "talker.code_predictor.model."
        bb = [[sd[f"{pre}layers.{i}.{k}"] for k in LAYER_KEYS] for i in range(n_bb)]
        cp = [[sd[f"{cpre}layers.{i}.{k}"] for k in LAYER_KEYS] for i in range(n_cp)]
        ngroups = sum(1 for k in sd if k.startswith("talker.code_predictor.lm_head."))
        return TalkerWeights(
            bb, sd[pre + "norm.weight"], sd["talker.codec_head.weight"], sd[pre + "codec_embedding.weight"],
            cp, sd[cpre + "norm.weight"],
            [sd[f"talker.code_predictor.lm_head.{g}.weight"] for g in range(ngroups)],
            [sd[f"{cpre}codec_embedding.{g}.weight"] for g in range(ngroups)])


class TalkerOracle:
    """Backbone + code predictor + frame glue (generator.py:77-176, test_audio.py:104-184)."""

    def __init__(self, w: TalkerWeights, max_seq: int = 1024, policy: str = "kernel", dims: Dims = Dims()):
        self.w, self.d, self.policy = w, dims, policy
        self.bb = DecoderOracle(w.bb_layers, w.bb_norm, max_seq, "backbone", policy, dims)
        self.cp = DecoderOracle(w.cp_layers, w.cp_norm, 16 + 1, "cp", policy, dims)
        self.cp_emb = [e.detach().to("cpu", torch.bfloat16) for e in w.cp_embeddings]
        self.bb_emb = w.codec_embedding.detach().to("cpu", torch.bfloat16)

    def cp_frame(self, bb_hidden: torch.Tensor, g0: int, do_sample=False, temperature=0.9, top_k=50,
                 seed: int = 0, frame_step: int = 0, trace: Optional[dict] = None) -> List[int]:
        """15 code-predictor groups for one frame (generator.py:309-354), 2-token prefill in the
        kernel policy at positions 0 and 1, then 14 decode steps; greedy unless do_sample."""
        self.cp.reset()
        self.cp.step(rb(bb_hidden.float()).to(torch.bfloat16), pos=0)
        h, _ = self.cp.step(self.bb_emb[g0], pos=1)
        toks = []
        for g in range(len(self.w.cp_heads)):
            if g > 0:
                h, _ = self.cp.step(self.cp_emb[g - 1][toks[-1]], pos=g + 1)
            lg = head_logits(self.w.cp_heads[g], h)
            if trace is not None:
                trace.setdefault("cp_logits", []).append(lg)
            toks.append(sample_token(lg, do_sample, temperature, top_k, 1.0, None, seed=seed,
                                     frame_step=frame_step, group=g + 1))
        return toks

    def combine(self, groups: Sequence[int], text_row: torch.Tensor) -> torch.Tensor:
        """bf16 running sum of the 16 codebook embeddings, then + text/pad (generator.py:143-149, 356-362)."""
        acc = self.bb_emb[groups[0]].clone()
        for i in range(len(self.cp_emb)):
            acc = acc + self.cp_emb[i][groups[i + 1]]
        return acc + text_row.detach().to("cpu", torch.bfloat16).reshape(-1)

    def prefill(self, embeds: torch.Tensor) -> torch.Tensor:
        """Prefill by stepping the backbone token by token (positions 0..S-1, t=h=w)."""
        self.bb.reset()
        h = None
        for i in range(embeds.shape[-2]):
            h, _ = self.bb.step(embeds.reshape(-1, embeds.shape[-1])[i], pos=i)
        return h

    def generate(self, talker_input_embeds, trailing_text_hidden, tts_pad_embed, eos_id: int,
                 max_tokens=500, do_sample=False, temperature=0.9, top_k=50, top_p=1.0,
                 cp_do_sample=False, cp_temperature=0.9, cp_top_k=50, min_new_tokens=2,
                 repetition_penalty=1.0, seed: int = 0, trace: Optional[dict] = None) -> List[List[int]]:
        """generator.py:77-176 with the in-repo sampler; returns one [16] id list per frame."""
        vocab = self.w.codec_head.shape[0]
        mask = suppress_mask(vocab, eos_id)
        hidden = self.prefill(talker_input_embeds)
        lg = head_logits(self.w.codec_head, hidden)
        lg[mask] = float("-inf")
        g0 = sample_token(lg, do_sample, temperature, top_k, top_p,
                          eos_id if min_new_tokens > 0 else None, seed=seed, frame_step=0, group=0)
        return self.decode_frames(hidden, g0, trailing_text_hidden, tts_pad_embed, eos_id, max_tokens, do_sample,
                                  temperature, top_k, top_p, cp_do_sample, cp_temperature, cp_top_k, min_new_tokens,
                                  repetition_penalty, seed, trace)

    def decode_frames(self, hidden, g0: int, trailing_text_hidden, tts_pad_embed, eos_id: int, max_tokens=500,
                      do_sample=False, temperature=0.9, top_k=50, top_p=1.0, cp_do_sample=False, cp_temperature=0.9,
                      cp_top_k=50, min_new_tokens=2, repetition_penalty=1.0, seed: int = 0,
                      trace: Optional[dict] = None, on_frame=None) -> List[List[int]]:
        """The frame loop of generator.py:122-174 after the prefill: ``hidden`` is the backbone's
        final-norm hidden of the last prompt token, ``g0`` the group-0 id selected from it, and the
        backbone cache (``self.bb``) holds the prompt at positions 0 .. position - 1."""
        vocab = self.w.codec_head.shape[0]
        mask = suppress_mask(vocab, eos_id)
        frames, hist = [], []
        n_text = trailing_text_hidden.shape[1]
        for step in range(max_tokens):
            if g0 == eos_id:
                break
            hist.append(g0)
            groups = [g0] + self.cp_frame(hidden, g0, cp_do_sample, cp_temperature, cp_top_k,
                                          seed=seed, frame_step=step, trace=trace)
            frames.append(groups)
            text = trailing_text_hidden[0, step] if step < n_text else tts_pad_embed[0, 0]
            x = self.combine(groups, text)
            hidden, _ = self.bb.step(x)
            lg = head_logits(self.w.codec_head, hidden)
            lg[mask] = float("-inf")
            lg = apply_repetition_penalty(lg, hist, repetition_penalty)
            if trace is not None:
                trace.setdefault("bb_hidden", []).append(hidden.clone())
                trace.setdefault("bb_logits", []).append(lg.clone())
            g0 = sample_token(lg, do_sample, temperature, top_k, top_p,
                              eos_id if step + 1 < min_new_tokens else None,
                              seed=seed, frame_step=step + 1, group=0)
            if on_frame is not None:
                on_frame(step, frames)
        return frames


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().reshape(-1).cpu()
    b = b.detach().double().reshape(-1).cpu()
    return float(torch.linalg.vector_norm(a - b) / max(float(torch.linalg.vector_norm(b)), 1e-30))
