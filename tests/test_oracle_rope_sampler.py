"""Pin the oracle's RoPE tables, interleaved 3D mRoPE, Philox stream, sampler and frame-glue
rules (CPU only).

* mRoPE: against transformers ``Qwen3VLTextRotaryEmbedding`` (its ``apply_interleaved_mrope``
  is the index map /root/reference/qwentts_turbo/csrc/rope_multimodal.cuh:9-54 describes),
  evaluated in f32 and cast to bf16, which must equal the oracle's gather from the 1D bf16
  tables bit for bit; and the reduction t == h == w -> 1D row.
* 1D RoPE tables: against transformers ``Qwen3RotaryEmbedding`` cast to bf16.
* Philox-4x64-10: against ``numpy.random.Philox`` (library known answers).
* Sampler: Gumbel-max over Philox noise has the softmax distribution (chi-square over 40k
  seeded draws on a 6-way categorical); top-k keeps ties; top-p equals the reference's
  sort / cumsum / shift rule (generator.py:197-204) on distinct values.
* Suppress mask and repetition penalty: generator.py:71-75 and :161-167 on hand-made cases.
"""
import math

import numpy as np
import pytest
import torch

from oracle.philox import KEY_TAG, philox4x64_10, sampler_uniform, uniform_from_word
from oracle.qtts_oracle import (apply_repetition_penalty, filter_logits, mrope_cos_sin, rope_tables,
                                sample_token, suppress_mask)


# ---------------------------------------------------------------- RoPE -----------------------

def test_rope_tables_match_transformers_qwen3_rotary():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, head_dim=128,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    r = Qwen3RotaryEmbedding(cfg)
    pos = torch.arange(0, 4096, 37)
    c, s = r(torch.zeros(1, dtype=torch.bfloat16), pos[None])
    ct, st = rope_tables(4096, 128, 1e6)
    assert torch.equal(c[0], ct[pos]) and torch.equal(s[0], st[pos])


@pytest.mark.parametrize("pos3", [(300, 157, 111), (0, 0, 0), (5, 4095, 17), (2047, 1023, 682), (9, 9, 9)])
def test_interleaved_mrope_matches_transformers_qwen3_vl(pos3):
    from transformers.models.qwen3_vl import modeling_qwen3_vl as v
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    cfg = Qwen3VLTextConfig(hidden_size=2048, num_attention_heads=16, head_dim=128,
                            rope_parameters={"rope_type": "default", "rope_theta": 1e6,
                                             "mrope_section": [24, 20, 20], "mrope_interleaved": True})
    r = v.Qwen3VLTextRotaryEmbedding(cfg)
    c, s = r(torch.zeros(1, dtype=torch.bfloat16), torch.tensor(pos3).view(3, 1, 1))
    ct, st = rope_tables(4096, 128, 1e6)
    mc, ms = mrope_cos_sin(ct, st, pos3, (24, 20, 20))
    assert torch.equal(c[0, 0].float(), mc) and torch.equal(s[0, 0].float(), ms)
    if pos3[0] == pos3[1] == pos3[2]:
        assert torch.equal(mc, ct[pos3[0]].float())


def test_mrope_sections_are_interleaved_not_chunked():
    """Distinct (t, h, w): channel 1 follows h, channel 2 follows w, channel 0 and 60..63
    follow t (a chunked [T*24, H*20, W*20] layout would put channel 1 on t)."""
    ct, st = rope_tables(4096, 128, 1e6)
    mc, _ = mrope_cos_sin(ct, st, (100, 200, 300), (24, 20, 20))
    for ch, row in ((0, 100), (1, 200), (2, 300), (3, 100), (58, 200), (59, 300), (60, 100), (63, 100)):
        assert mc[ch] == ct[row, ch].float() and mc[ch + 64] == ct[row, ch + 64].float(), ch


# ---------------------------------------------------------------- Philox ---------------------

@pytest.mark.parametrize("ctr,key", [((0, 0, 0, 0), (0, 0)), ((1, 2, 3, 4), (5, 6)),
                                     ((2**64 - 1, 7, 2**63, 11), (0xDEADBEEF, KEY_TAG)),
                                     ((767, 255, 15, 0), (77, KEY_TAG))])
def test_philox4x64_10_matches_numpy(ctr, key):
    c = ctr[0] | (ctr[1] << 64) | (ctr[2] << 128) | (ctr[3] << 192)
    k = key[0] | (key[1] << 64)
    bg = np.random.Philox(counter=c, key=k)
    ref = [int(x) for x in bg.random_raw(4)]
    # numpy increments the 256-bit counter before producing a block
    c1 = (c + 1) % (1 << 256)
    mine = philox4x64_10([(c1 >> (64 * i)) & (2**64 - 1) for i in range(4)], key)
    assert mine == ref


def test_uniform_open_interval_and_mapping():
    assert uniform_from_word(0) == 0.5 * 2.0**-52
    assert uniform_from_word(2**64 - 1) == 1.0 - 0.5 * 2.0**-52 < 1.0
    # every word maps to k + 0.5 exactly: the map is strictly monotone in the top 52 bits
    ks = [0, 1, 2**51, 2**52 - 2, 2**52 - 1]
    us = [uniform_from_word(k << 12) for k in ks]
    assert all(a < b for a, b in zip(us, us[1:]))
    assert all((u * 2.0**52 - 0.5) == k for u, k in zip(us, ks))
    u = [sampler_uniform(3, 4, 5, i) for i in range(8)]
    assert len(set(u)) == 8 and all(0.0 < x < 1.0 for x in u)


# ---------------------------------------------------------------- sampler --------------------

def test_gumbel_max_sampler_has_softmax_distribution():
    logits = torch.tensor([1.0, 0.5, 0.0, -0.5, 2.0, -3.0])
    n = 40000
    counts = np.zeros(6)
    for t in range(n):
        counts[sample_token(logits, True, 1.0, 0, 1.0, seed=t % 97, frame_step=t // 97, group=3)] += 1
    p = torch.softmax(logits.double(), 0).numpy()
    chi2 = float(((counts - n * p) ** 2 / (n * p)).sum())
    # 5 degrees of freedom: P(chi2 > 25) ~ 1.4e-4
    assert chi2 < 25.0, (counts / n, p)


def test_greedy_lowest_index_on_ties_and_eos_suppression():
    lg = torch.tensor([0.0, 3.0, 1.0, 3.0, 2.0])
    assert sample_token(lg, False, 1.0, 0, 1.0) == 1
    assert sample_token(lg, False, 1.0, 0, 1.0, suppress_eos_id=1) == 3


def _reference_rule(logits, temperature, top_k, top_p):
    """generator.py:189-204 as written there, on the reference's bf16 logits: topk threshold,
    then sort / cumsum / shift."""
    scaled = logits.to(torch.bfloat16) / temperature
    if top_k > 0:
        kth = torch.topk(scaled, min(top_k, scaled.size(-1)))[0][-1]
        scaled = scaled.clone()
        scaled[scaled < kth] = float("-inf")
    if top_p < 1.0:
        sl, si = torch.sort(scaled, descending=True)
        cp = torch.cumsum(torch.softmax(sl.double(), dim=-1), dim=-1)
        rm = cp > top_p
        rm[1:] = rm[:-1].clone()
        rm[0] = False
        sl[rm] = float("-inf")
        scaled = scaled.clone().scatter_(0, si, sl)
    return scaled


def _distinct_bf16(n, seed):
    """n distinct bf16 values: a random choice among all bf16 values of magnitude in
    [2^-10, 32) (both signs; 3840 of them), in random order."""
    g = torch.Generator().manual_seed(seed)
    mag = torch.arange((127 - 10) << 7, (127 + 5) << 7, dtype=torch.int32)     # exponent and mantissa bits
    bits = torch.cat([mag, mag | 0x8000]).to(torch.int16)
    vals = bits.view(torch.bfloat16).float()
    assert vals.numel() >= n
    return vals[torch.randperm(vals.numel(), generator=g)[:n]]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("top_k,top_p", [(50, 1.0), (0, 0.8), (20, 0.5), (0, 0.05), (7, 0.95)])
def test_filter_matches_reference_rule_on_distinct_values(seed, top_k, top_p):
    lg = _distinct_bf16(3072, seed)
    # temperature 0.5 scales bf16 values exactly, so the scaled values stay distinct
    a = torch.isfinite(filter_logits(lg, 0.5, top_k, top_p))
    b = torch.isfinite(_reference_rule(lg, 0.5, top_k, top_p))
    assert torch.equal(a, b)


def test_temperature_scaling_rounds_to_bf16_like_the_reference():
    """logits / temperature on bf16 logits is a bf16 tensor in the reference (generator.py:189)."""
    lg = _distinct_bf16(3072, 9)
    a = filter_logits(lg, 0.9, 0, 1.0)
    b = (lg.to(torch.bfloat16) / 0.9).float()
    assert torch.equal(a, b)


def test_top_k_keeps_ties():
    lg = torch.tensor([5.0, 4.0, 4.0, 4.0, 1.0])
    kept = torch.isfinite(filter_logits(lg, 1.0, 2, 1.0))
    assert kept.tolist() == [True, True, True, True, False]


def test_top_p_keeps_first_token_and_boundary():
    lg = torch.log(torch.tensor([0.5, 0.3, 0.15, 0.05]))
    assert torch.isfinite(filter_logits(lg, 1.0, 0, 0.1)).tolist() == [True, False, False, False]
    # mass strictly above the 3rd value is 0.8 <= 0.85: kept; above the 4th 0.95 > 0.85
    assert torch.isfinite(filter_logits(lg, 1.0, 0, 0.85)).tolist() == [True, True, True, False]


def test_suppress_mask_and_repetition_penalty():
    m = suppress_mask(3072, 2150)
    assert not m[:2048].any() and m[2048:].sum() == 1023 and not m[2150]
    lg = torch.tensor([2.0, -2.0, 1.0, -1.0])
    out = apply_repetition_penalty(lg, [0, 1, 1], 2.0)
    assert out.tolist() == [1.0, -4.0, 1.0, -1.0]
    assert torch.equal(apply_repetition_penalty(lg, [0], 1.0), lg)
