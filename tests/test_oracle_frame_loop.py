"""Pin the oracle's frame-loop recursion against transformers' Qwen3-Omni talker (CPU only).

The code-predictor loop of one codec frame and the embedding combine are restated by the
oracle from /root/reference/qwentts_turbo/generator.py:309-354 (2-token prefill
``[bf16(h), emb_bb[g0]]`` at positions 0 and 1, then ``lm_head[g]`` on the last hidden and
``emb[g-1](token)`` as the next input) and :356-362 plus :143-149 (sum of the 16 codebook
embeddings, then the trailing-text row of the frame or the pad row). transformers in this
container ships the same talker/code-predictor recurrence as library code:

* ``Qwen3OmniMoeTalkerCodePredictorModelForConditionalGeneration.forward`` / ``generate``
  (``modeling_qwen3_omni_moe.py``: prefill of two inputs selects with ``lm_head[0]``, every
  later step embeds the previous id with ``codec_embedding[generation_steps - 1]`` and selects
  with ``lm_head[generation_steps]``);
* ``Qwen3OmniMoeTalkerForConditionalGeneration.prepare_inputs_for_generation``, which runs that
  ``generate`` from ``cat(hidden, codec_embedding(g0))`` and returns the residual codes and the
  next talker input ``sum(16 codebook embeddings) + trailing_text_hidden[step]`` (pad row once
  the text is exhausted).

The test builds a small talker (2 code-predictor layers with the 0.6B shapes, 15 heads) holding
the synthetic weights in float64, calls that function, and requires the oracle's ids to be
identical and its bf16 running-sum combine to lie within the bf16 rounding bound of
transformers' sum. The lm-heads are wrapped to round their input to bf16 first, as the
reference does before ``torch.mv`` (generator.py:351). Mutations planted in the oracle (the
embedding-table index or the head index shifted by one, the text row dropped) must fail.
"""
import copy
import math

import pytest
import torch

from oracle.qtts_oracle import TalkerOracle, TalkerWeights, rb

transformers = pytest.importorskip("transformers")
from transformers import DynamicCache  # noqa: E402

try:
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import Qwen3OmniMoeTalkerConfig
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import Qwen3OmniMoeTalkerForConditionalGeneration
except ImportError:  # pragma: no cover
    pytest.skip("transformers without qwen3_omni_moe", allow_module_level=True)

N_CP_LAYERS = 2
N_GROUPS = 15
N_TEXT = 4


class _Bf16InputHead(torch.nn.Module):
    """lm_head applied to bf16(hidden) (generator.py:351 casts the hidden before torch.mv)."""

    def __init__(self, lin):
        super().__init__()
        self.lin = lin

    def forward(self, x):
        return self.lin(x.to(torch.bfloat16).to(x.dtype))


@pytest.fixture(scope="module")
def talker(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=N_CP_LAYERS, n_groups=N_GROUPS)
    sd = pkg.synthetic_state_dict(seed=4321, cfg=cfg)
    cp_cfg = dict(hidden_size=1024, intermediate_size=3072, num_hidden_layers=N_CP_LAYERS, num_attention_heads=16,
                  num_key_value_heads=8, head_dim=128, vocab_size=2048, num_code_groups=N_GROUPS + 1,
                  rms_norm_eps=1e-6, rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    # the talker's own text model is never run here (only its codec embedding is used); keep it tiny
    text_cfg = dict(hidden_size=1024, intermediate_size=64, moe_intermediate_size=16, num_hidden_layers=1,
                    num_attention_heads=16, num_key_value_heads=8, head_dim=128, vocab_size=3072, num_experts=2,
                    num_experts_per_tok=1, shared_expert_intermediate_size=16)
    tcfg = Qwen3OmniMoeTalkerConfig(code_predictor_config=cp_cfg, text_config=text_cfg, num_code_groups=N_GROUPS + 1,
                                    thinker_hidden_size=64, spatial_merge_size=2)
    m = Qwen3OmniMoeTalkerForConditionalGeneration(tcfg)
    msd = m.state_dict()
    new = {}
    for k, v in msd.items():
        if k.startswith("code_predictor."):
            new[k] = sd["talker." + k].double()
        elif k == "model.codec_embedding.weight":
            new[k] = sd["talker.model.codec_embedding.weight"].double()
        else:
            new[k] = v.double()
    m = m.double()
    m.load_state_dict(new)
    m.eval()
    for g in range(N_GROUPS):
        m.code_predictor.lm_head[g] = _Bf16InputHead(m.code_predictor.lm_head[g])
    m.code_predictor.generation_config.do_sample = False
    tw = TalkerWeights.from_state_dict(sd, 1, N_CP_LAYERS)
    return m, tw


def _inputs(seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(1024, generator=g)
    g0 = int(torch.randint(0, 2048, (1,), generator=g))
    text = torch.randn(1, N_TEXT, 1024, generator=g).to(torch.bfloat16)
    pad = torch.randn(1, 1, 1024, generator=g).to(torch.bfloat16)
    return h, g0, text, pad


def _transformers_frame(m, h, g0, text, pad, step):
    """Residual codes [g0, g1..g15] and the next talker input from transformers' talker."""
    hs = ((rb(h).double().reshape(1, 1, 1024),),)   # the backbone hidden, bf16 as generator.py:130-131 passes it
    with torch.no_grad():
        inp = m.prepare_inputs_for_generation(
            torch.tensor([[g0]]), past_key_values=DynamicCache(config=m.config.text_config),
            attention_mask=torch.ones(1, step + 2, dtype=torch.long), hidden_states=hs, generation_step=step,
            trailing_text_hidden=text.double(), tts_pad_embed=pad.double(), is_first_iteration=False,
            use_cache=True, cache_position=torch.tensor([step + 1]))
    return inp["residual_codes"][0].tolist(), inp["inputs_embeds"].reshape(-1)


def _bf16_sum_bound(terms):
    """Per-element bound on |bf16 running sum - exact sum| for terms added left to right:
    half a bf16 ulp of every partial sum (taken from the exact partials, with slack 2)."""
    part = torch.cumsum(torch.stack([t.double() for t in terms]), 0)[1:]
    e = torch.floor(torch.log2(part.abs().clamp_min(1e-30)))
    return 2.0 * 0.5 * torch.pow(2.0, e - 7).sum(0)


def _oracle_frame(orc, h, g0, text, pad, step, trace=None):
    toks = orc.cp_frame(h, g0, trace=trace)
    row = text[0, step] if step < text.shape[1] else pad[0, 0]
    return [g0] + toks, orc.combine([g0] + toks, row), row


def _check(orc, m, seed, step):
    h, g0, text, pad = _inputs(seed)
    codes_tf, x_tf = _transformers_frame(m, h, g0, text, pad, step)
    tr = {}
    codes, x, row = _oracle_frame(orc, h, g0, text, pad, step, tr)
    terms = [orc.bb_emb[codes[0]]] + [orc.cp_emb[i][codes[i + 1]] for i in range(N_GROUPS)] + [row]
    bound = _bf16_sum_bound(terms)
    err = (x.double() - x_tf).abs()
    # top-2 margin of every head's logits (how far each greedy choice is from a tie)
    margins = [float(torch.topk(lg.double(), 2)[0].diff().abs()) for lg in tr["cp_logits"]]
    return codes, codes_tf, bool((err <= bound).all()), float((err / bound).max()), min(margins)


@pytest.mark.parametrize("seed,step", [(11, 0), (12, 2), (13, N_TEXT + 1)])
def test_cp_frame_and_combine_match_transformers_talker(talker, seed, step):
    m, tw = talker
    orc = TalkerOracle(tw, max_seq=16, policy="exact")
    codes, codes_tf, ok, ratio, margin = _check(orc, m, seed, step)
    print(f"seed {seed} step {step}: codes {codes[:5]}..., combine err / bound {ratio:.2f}, min top-2 margin {margin:.3e}")
    assert codes == codes_tf
    assert ok, ratio


def test_kernel_policy_cp_frame_ids_match_exact_policy(talker):
    """The fixtures are written in the kernel policy (f32/bf16 storage points, f64 sums): on the
    same inputs its 15 ids equal the exact policy's, which the test above ties to transformers."""
    _, tw = talker
    for seed in (11, 12, 13):
        h, g0, _, _ = _inputs(seed)
        a = TalkerOracle(tw, max_seq=16, policy="exact").cp_frame(h, g0)
        b = TalkerOracle(tw, max_seq=16, policy="kernel").cp_frame(h, g0)
        assert a == b


def _rotate(lst):
    return lst[1:] + lst[:1]


@pytest.mark.parametrize("mutation", ["embedding_index", "head_index", "text_dropped"])
def test_planted_frame_loop_mistakes_fail(talker, mutation):
    """Each planted mistake in the oracle must be caught by the comparison above."""
    m, tw = talker
    seed, step = 12, 2
    if mutation == "head_index":
        tw = copy.copy(tw)
        tw.cp_heads = _rotate(list(tw.cp_heads))          # lm_head[g + 1] used for group g + 1
    orc = TalkerOracle(tw, max_seq=16, policy="exact")
    if mutation == "embedding_index":
        orc.cp_emb = _rotate(list(orc.cp_emb))            # emb[g] instead of emb[g - 1]
    h, g0, text, pad = _inputs(seed)
    codes_tf, x_tf = _transformers_frame(m, h, g0, text, pad, step)
    codes, x, row = _oracle_frame(orc, h, g0, text, pad, step)
    if mutation == "text_dropped":
        x = orc.combine(codes, torch.zeros(1024, dtype=torch.bfloat16))
    terms = [orc.bb_emb[codes[0]]] + [orc.cp_emb[i][codes[i + 1]] for i in range(N_GROUPS)] + [row]
    ok = codes == codes_tf and bool(((x.double() - x_tf).abs() <= _bf16_sum_bound(terms)).all())
    assert not ok, f"mutation {mutation} was not detected"
