"""Pin the oracle's decoder math against transformers' Qwen3 modules (CPU only).

The reference's PyTorch decode path is transformers' Qwen3 decoder layer (the talker of
qwen_tts, run by /root/reference/qwentts_turbo/generator.py:227-243 and
/root/reference/tests/test_audio.py:104-184). transformers is importable here, so its
``Qwen3Model`` -- RMSNorm, q/k-norm, rotate_half RoPE, GQA with repeat_kv, SwiGLU, eager
attention -- is the library routine the oracle's layer is checked against:

* ``policy="exact"`` (f64, f32 cos/sin) vs ``Qwen3Model`` in float64: agreement to f32
  rounding (transformers' Qwen3RMSNorm and rotary tables compute in f32 even for f64 models)
  pins every formula -- a dropped term, a wrong sign in rotate_half, a transposed operand or
  a wrong GQA head map all fail by orders of magnitude.
* ``policy="hf_bf16"`` vs ``Qwen3Model`` in bfloat16: the op order of the HF path.
* ``policy="kernel"`` (f64 accumulation, f32/bf16 storage) vs ``hf_bf16`` at the config-0
  shapes (28 layers, L=129): the north-star bar rel-L2 <= 1e-2 per layer and on the logits.
"""
import math

import pytest
import torch

from oracle.qtts_oracle import (DecoderOracle, TalkerWeights, head_logits, rel_l2, split_attention, chunking,
                                local_attention, MAX_CHUNKS, SUB_BB, SUB_CP)

transformers = pytest.importorskip("transformers")
from transformers import Qwen3Config  # noqa: E402
from transformers.models.qwen3.modeling_qwen3 import Qwen3Model  # noqa: E402


def _hf_model(sd, n_layers, dtype, attn="eager"):
    cfg = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=n_layers,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6,
                      vocab_size=16, max_position_embeddings=4096,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    cfg._attn_implementation = attn
    m = Qwen3Model(cfg)
    hsd = {"embed_tokens.weight": torch.zeros(16, 1024), "norm.weight": sd["talker.model.norm.weight"].float()}
    for k, v in sd.items():
        if k.startswith("talker.model.layers."):
            hsd[k[len("talker.model."):]] = v.float()
    m.load_state_dict(hsd)
    return m.to(dtype).eval()


@pytest.fixture(scope="module")
def small(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=1, n_groups=1)
    sd = pkg.synthetic_state_dict(seed=1234, cfg=cfg)
    return sd, TalkerWeights.from_state_dict(sd, 2, 1)


def _prefill_inputs(T, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(T, 1024, generator=g).to(torch.bfloat16)


def test_exact_policy_matches_transformers_qwen3_f64(small):
    sd, tw = small
    T = 12
    x = _prefill_inputs(T, 3)
    # sdpa keeps the softmax in f64 (the eager path rounds probabilities to f32)
    m = _hf_model(sd, 2, torch.float64, attn="sdpa")
    with torch.no_grad():
        ref = m(inputs_embeds=x.double()[None], position_ids=torch.arange(T)[None], use_cache=False,
                output_hidden_states=True)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "exact")
    worst = 0.0
    for i in range(T):
        h, layers = orc.step(x[i], pos=i)
        worst = max(worst, rel_l2(h, ref.last_hidden_state[0, i]))
        # per-layer output of layer 0 (hidden_states[1] is the output of the first layer)
        worst = max(worst, rel_l2(layers[0].double(), ref.hidden_states[1][0, i]))
    assert worst < 1e-6, worst


def test_exact_policy_mrope_equal_positions_is_1d(small):
    sd, tw = small
    x = _prefill_inputs(4, 4)
    a = DecoderOracle(tw.bb_layers, tw.bb_norm, 16, "backbone", "exact")
    b = DecoderOracle(tw.bb_layers, tw.bb_norm, 16, "backbone", "exact")
    for i in range(4):
        ha, _ = a.step(x[i], pos=i, pos3=(i, i, i))
        hb, _ = b.step(x[i], pos=i)
    assert torch.equal(ha, hb)


def test_hf_bf16_policy_matches_transformers_bf16(small):
    sd, tw = small
    T = 12
    x = _prefill_inputs(T, 5)
    m = _hf_model(sd, 2, torch.bfloat16)
    with torch.no_grad():
        ref = m(inputs_embeds=x[None], position_ids=torch.arange(T)[None], use_cache=False)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "hf_bf16")
    worst = 0.0
    for i in range(T):
        h, _ = orc.step(x[i], pos=i)
        worst = max(worst, rel_l2(h, ref.last_hidden_state[0, i].float()))
    # one-token decode vs full-sequence prefill in bf16: same ops, GEMM shapes differ
    assert worst < 1e-2, worst


def test_hf_bf16_f64_sums_keep_the_rounding_points(small):
    """``hf_sums="f64"`` changes only the order of the projection sums: one projection rounds to
    the same bf16 values almost everywhere (an f32 sum of 1024 products rarely crosses a bf16
    boundary), and 2 layers over 12 tokens stay within the 2-layer prefill bar (1e-2)."""
    from oracle.qtts_oracle import rms_norm_hf
    sd, tw = small
    x = _prefill_inputs(12, 6)
    a = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "hf_bf16")
    b = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "hf_bf16", hf_sums="f64")
    w = a.layers[0]
    h = rms_norm_hf(x[0], w.ln_in, 1e-6)
    la, lb = a._linear(h, w.q), b._linear(h, w.q)
    assert la.dtype == lb.dtype == torch.bfloat16
    assert float((la != lb).float().mean()) < 0.01
    for i in range(12):
        ha, _ = a.step(x[i], pos=i)
        hb, _ = b.step(x[i], pos=i)
    assert rel_l2(ha, hb) < 1e-2
    assert rel_l2(a.k[:, :, :12].float(), b.k[:, :, :12].float()) < 1e-2


def test_kernel_policy_matches_exact_small(small):
    sd, tw = small
    x = _prefill_inputs(40, 6)
    k = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "kernel")
    e = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "exact")
    worst = 0.0
    for i in range(40):
        hk, _ = k.step(x[i], pos=i)
        he, _ = e.step(x[i], pos=i)
        worst = max(worst, rel_l2(hk, he))
    assert worst < 1e-2, worst


@pytest.mark.parametrize("norm_mean", [0.0, 1.0])
def test_kernel_policy_vs_hf_bf16_config0_per_layer(pkg, norm_mean):
    """Config 0 shapes: 28 layers, KV of 128 tokens, decode at position 128 (L=129).

    Gains N(0, 0.02) (BASELINE's literal init): per-layer hidden states, final hidden and
    codec-head logits within rel-L2 1e-2 of the HF bf16 path.
    Gains N(1, 0.02) (layers not inert): the bf16 residual between layers, a storage point of
    the reference kernel (fused_decode_tts.cu:541), alone puts ~1% of rounding noise on layer
    28, and the HF bf16 path carries ~1.7%; there the kernel policy must stay closer to the f64
    ``exact`` path than the HF path is, on every layer, and within 2.5e-2 of the HF path.
    """
    sd = pkg.synthetic_state_dict(seed=1234, cfg=pkg.SyntheticConfig(n_cp_layers=1, n_groups=1,
                                                                     norm_mean=norm_mean))
    tw = TalkerWeights.from_state_dict(sd, 28, 1)
    g = torch.Generator().manual_seed(21)
    kv_k = torch.randn(28, 8, 128, 128, generator=g).to(torch.bfloat16)
    kv_v = torch.randn(28, 8, 128, 128, generator=g).to(torch.bfloat16)
    x = torch.randn(1024, generator=g).to(torch.bfloat16)
    out = {}
    for pol in ("kernel", "hf_bf16", "exact"):
        o = DecoderOracle(tw.bb_layers, tw.bb_norm, 136, "backbone", pol)
        o.set_kv(kv_k, kv_v)
        out[pol] = o.step(x, pos=128)
        del o
    (hk, lk), (hh, lh), (he, le) = out["kernel"], out["hf_bf16"], out["exact"]
    per_layer = [rel_l2(a, b) for a, b in zip(lk, lh)]
    logit_err = rel_l2(head_logits(tw.codec_head, hk), head_logits(tw.codec_head, hh))
    print(f"gains N({norm_mean},0.02): kernel vs hf_bf16 per layer max {max(per_layer):.4f}, "
          f"final {rel_l2(hk, hh):.4f}, logits {logit_err:.4f}")
    if norm_mean == 0.0:
        assert max(per_layer) < 1e-2, per_layer
        assert rel_l2(hk, hh) < 1e-2
        assert logit_err < 1e-2, logit_err
    else:
        assert max(per_layer) < 2.5e-2, per_layer
        for a, b, c in zip(lk, lh, le):
            assert rel_l2(a, c) < rel_l2(b, c)


@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 64, 65, 129, 511, 512, 513, 2048, 4096])
@pytest.mark.parametrize("sub", [SUB_BB, SUB_CP])
def test_split_attention_equals_single_pass_softmax(L, sub):
    g = torch.Generator().manual_seed(L * 7 + sub)
    q = torch.randn(4, 128, generator=g, dtype=torch.float64)
    K = torch.randn(4, L, 128, generator=g, dtype=torch.float64) * 3
    V = torch.randn(4, L, 128, generator=g, dtype=torch.float64)
    scale = 1 / math.sqrt(128)
    ref = torch.softmax(torch.einsum("hd,hpd->hp", q, K) * scale, -1)
    ref = torch.einsum("hp,hpd->hd", ref, V)
    C, P = chunking(L, sub)
    assert 1 <= C <= MAX_CHUNKS and (C - 1) * P < L <= C * P
    assert rel_l2(split_attention(q, K, V, scale, sub), ref) < 1e-13
    assert rel_l2(local_attention(q, K, V, scale), ref) < 1e-13


def test_gqa_head_map_uses_kv_head_h_div_2(small):
    """Swapping the two q heads that share a KV head leaves attention per head consistent;
    swapping KV heads changes it (the map h -> h // 2 of repeat_kv, not h % 8)."""
    sd, tw = small
    orc = DecoderOracle(tw.bb_layers[:1], tw.bb_norm, 8, "backbone", "exact")
    g = torch.Generator().manual_seed(9)
    k = torch.randn(1, 8, 3, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 8, 3, 128, generator=g).to(torch.bfloat16)
    orc.set_kv(k, v)
    tr = {}
    orc.step(torch.randn(1024, generator=g), pos=3, trace=tr)
    attn = tr["attn"][0].view(16, 128)
    # attention output of q head h is a convex combination of V rows of kv head h // 2
    V = orc.v[0].double()
    for h in range(16):
        basis = V[h // 2, :4]                                   # [4, 128]
        coef = torch.linalg.lstsq(basis.T, attn[h][:, None]).solution
        resid = basis.T @ coef - attn[h][:, None]
        assert float(resid.norm()) < 1e-8 * float(attn[h].norm()) + 1e-12
        assert abs(float(coef.sum()) - 1.0) < 1e-9
