"""GPU parity of the MFMA prefill (qtts_backbone_prefill) against the oracle's transformers-bf16
policy (``hf_bf16``, the reference's PyTorch prefill, generator.py:209-225) stepped token by token:
the K/V cache entries of every prompt position and the last token's final-norm hidden.

Tolerance: both sides store bf16 after every op; the GPU's f32 sums run in MFMA order, so a sum
occasionally rounds to the neighbouring bf16 value, and each such flip perturbs the next op's
sums and flips a few percent of its outputs. The spread therefore grows with depth. The bar is
the north star's rel-L2 <= 1e-2 (TOL) for the 2-layer cases. For 28 layers the oracle's own
spread between torch's f32 sums and f64 sums (same rounding points, ``hf_sums="f64"``) is
already above 1e-2, so there the GPU is held to max(TOL, FLOOR_X x that spread): no further
from the oracle than a second valid summation order is.
"""
import pytest
import torch

from oracle.qtts_oracle import DecoderOracle, TalkerWeights, rel_l2, suppress_mask

pytestmark = pytest.mark.gpu

TOL = 1e-2
FLOOR_X = 2.0
EOS = 2150


def _print(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def small(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=1, n_groups=1)
    sd = pkg.synthetic_state_dict(seed=21, cfg=cfg)
    return {k: v.cuda() for k, v in sd.items()}, TalkerWeights.from_state_dict(sd, 2, 1)


def _compare(bb, orc, p0, S, hidden, hidden_ref, label, bars=(TOL, TOL, TOL)):
    L = p0 + S
    ek = rel_l2(bb.get_k_cache()[:, :, p0:L].float().cpu(), orc.k[:, :, p0:L].float())
    ev = rel_l2(bb.get_v_cache()[:, :, p0:L].float().cpu(), orc.v[:, :, p0:L].float())
    eh = rel_l2(hidden.cpu(), hidden_ref)
    _print(f"{label}: K rel_l2 {ek:.2e}, V {ev:.2e}, hidden {eh:.2e} (bars {bars[0]:.2e} {bars[1]:.2e} {bars[2]:.2e})")
    assert ek < bars[0] and ev < bars[1] and eh < bars[2]
    return eh


@pytest.mark.parametrize("S", [1, 7, 64, 128, 130, 256, 333, 1100])
def test_prefill_two_layers(pkg, small, S):
    """Prompt lengths across the tile edges and GEMM forms: one token and 7 (a partial 32-query
    block; the row GEMM's partial 16-row block), 64 (two query blocks; 4 whole row blocks), 128
    (the row GEMM's largest prompt, all 8 row blocks), 130 (the 64-column tile, a partial 128-row
    tile), 256 (the smallest prompt of the DMA-fed 128 x 128 GEMM), several tiles with a ragged
    last one, and a long prompt (the widest split-K target, 35 query blocks, a ragged last
    block)."""
    dsd, tw = small
    ms = 512 if S <= 512 else 2048
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=ms)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, ms, "backbone", "hf_bf16")
    x = torch.randn(S, 1024, generator=torch.Generator().manual_seed(100 + S)).to(torch.bfloat16)
    _print(f"prefill 2 layers S={S}: launching")
    h = bb.prefill(x.cuda())
    torch.cuda.synchronize()
    hr = None
    for i in range(S):
        hr, _ = orc.step(x[i], pos=i)
    _compare(bb, orc, 0, S, h, hr, f"prefill 2 layers S={S}")
    assert bb.position == S


@pytest.mark.parametrize("S", [100, 1100])
def test_prefill_after_prefix_and_distinct_mrope(pkg, small, S):
    """A prompt continuing a cached prefix (positions 50..50 + S - 1 attend 0..50 + S - 1) with
    distinct (t, h, w) rotary rows per token. At 1100 tokens the QKV GEMM is unsplit on 128-column
    tiles and finishes each head (q/k-norm, RoPE, K/V write) in its own epilogue."""
    dsd, tw = small
    p0 = 50
    ms = 512 if p0 + S <= 512 else 2048
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=ms)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, ms, "backbone", "hf_bf16")
    g = torch.Generator().manual_seed(77)
    k = torch.randn(2, 8, p0, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, p0, 128, generator=g).to(torch.bfloat16)
    bb.set_kv_cache(k.cuda(), v.cuda())
    bb.set_position(p0)
    orc.set_kv(k, v)
    x = torch.randn(S, 1024, generator=g).to(torch.bfloat16)
    pos = torch.arange(p0, p0 + S)
    pos3 = torch.stack([pos, pos // 2 + 7, pos // 3 + 11]).to(torch.int32)
    _print("prefill after a 50-position prefix, distinct mRoPE rows: launching")
    h = bb.prefill(x.cuda(), pos3=pos3.cuda())
    torch.cuda.synchronize()
    hr = None
    for i in range(S):
        hr, _ = orc.step(x[i], pos=p0 + i, pos3=[int(pos3[j, i]) for j in range(3)])
    _compare(bb, orc, p0, S, h, hr, f"prefill after prefix, mRoPE, S={S}")
    assert bb.position == p0 + S


def test_prefill_full_model_and_first_token(pkg):
    """All 28 layers at a 40-token prompt, then the first group-0 token (greedy, suppress mask,
    EOS removed) from the bf16 codec-head logits, as generate() uses it."""
    sd = pkg.synthetic_state_dict(seed=1234)
    dsd = {k: v.cuda() for k, v in sd.items()}
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    S = 40
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=256)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "hf_bf16")
    x = torch.randn(S, 1024, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    _print("prefill 28 layers S=40: launching")
    h = bb.decoder.prefill(x.cuda(), tok, EOS, True)
    torch.cuda.synchronize()
    hr = None
    for i in range(S):
        hr, _ = orc.step(x[i], pos=i)
    # the oracle's own summation-order spread over the same 28 layers
    alt = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "hf_bf16", hf_sums="f64")
    ha = None
    for i in range(S):
        ha, _ = alt.step(x[i], pos=i)
    fk = rel_l2(alt.k[:, :, :S].float(), orc.k[:, :, :S].float())
    fv = rel_l2(alt.v[:, :, :S].float(), orc.v[:, :, :S].float())
    fh = rel_l2(ha, hr)
    _print(f"oracle f32-vs-f64 sums spread: K {fk:.2e}, V {fv:.2e}, hidden {fh:.2e}")
    bars = tuple(max(TOL, FLOOR_X * f) for f in (fk, fv, fh))
    _compare(bb, orc, 0, S, h, hr, "prefill 28 layers S=40", bars)
    # logits: bf16(W_head . bf16 hidden) (generator.py:116), against the oracle's hidden
    lref = torch.nn.functional.linear(hr.to(torch.bfloat16), tw.codec_head.to(torch.bfloat16)).float()
    lg = bb.decoder.logits_buffer().cpu()
    el = rel_l2(lg, lref)
    _print(f"logits rel_l2 {el:.2e}")
    assert el < bars[2]
    # selection on the GPU's logits: suppress mask (generator.py:71-75) and EOS removed (:117),
    # greedy argmax with the lowest index on ties -- exact
    m = lg.clone()
    m[suppress_mask(m.numel(), EOS)] = -float("inf")
    m[EOS] = -float("inf")
    t = int(tok.item())
    _print(f"first token {t} (argmax of the masked GPU logits {int(m.argmax())})")
    assert t == int(m.argmax())


def test_prefill_per_layer_teacher_forced(pkg):
    """Every one of the 28 layers on its own, from the oracle's own input to that layer: the GPU
    prefill runs a one-layer model holding layer l's weights on the hf_bf16 oracle's residual
    stream entering layer l (40 tokens), and its K/V entries and the last token's output (through
    the final norm) must be within the north star's rel-L2 1e-2 of the oracle's layer l. This
    holds each layer to the bar without the depth-compounded rounding spread of the 28-layer run."""
    from oracle.qtts_oracle import rms_norm_hf
    sd = pkg.synthetic_state_dict(seed=1234)
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    S = 40
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 64, "backbone", "hf_bf16")
    x = torch.randn(S, 1024, generator=torch.Generator().manual_seed(19)).to(torch.bfloat16)
    outs = []
    for i in range(S):
        _, o = orc.step(x[i], pos=i)
        outs.append(o)
    prefix = "talker.model.layers."
    worst = [0.0, 0.0, 0.0]
    for l in range(28):
        sd1 = {}
        for k, v in sd.items():
            if k.startswith(prefix):
                if k.startswith(f"{prefix}{l}."):
                    sd1[prefix + "0." + k[len(f"{prefix}{l}."):]] = v.cuda()
            else:
                sd1[k] = v.cuda()
        x_in = x if l == 0 else torch.stack([outs[i][l - 1] for i in range(S)]).to(torch.bfloat16)
        bb = pkg.TTSMegakernelGenerator(model=sd1, max_seq_len=64)
        h = bb.prefill(x_in.cuda())
        torch.cuda.synchronize()
        ek = rel_l2(bb.get_k_cache()[0, :, :S].float().cpu(), orc.k[l, :, :S].float())
        ev = rel_l2(bb.get_v_cache()[0, :, :S].float().cpu(), orc.v[l, :, :S].float())
        href = rms_norm_hf(outs[S - 1][l].to(torch.bfloat16), tw.bb_norm.to(torch.bfloat16), 1e-6).float()
        eh = rel_l2(h.cpu(), href)
        worst = [max(worst[0], ek), max(worst[1], ev), max(worst[2], eh)]
        assert ek < TOL and ev < TOL and eh < TOL, (l, ek, ev, eh)
        del bb, sd1
    _print(f"per-layer teacher-forced prefill, 28 layers, S={S}: worst K {worst[0]:.2e}, V {worst[1]:.2e}, "
           f"output {worst[2]:.2e} (bar {TOL:.0e})")


def test_prefill_rejects_bad_arguments(pkg, small):
    """Host-side validation before any launch: an empty prompt, a prompt past max_seq_len, a
    wrong embedding width, a pos3 of the wrong shape; the decoder's position is left unchanged."""
    dsd, _ = small
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=64)
    bb.set_position(60)
    with pytest.raises(RuntimeError, match=r"embeds must be \[S, 1024\], got \[0, 1024\]"):
        bb.prefill(torch.zeros(0, 1024, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError, match="max_seq_len"):
        bb.prefill(torch.zeros(5, 1024, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError, match="embeds"):
        bb.prefill(torch.zeros(2, 512, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError, match="pos3"):
        bb.prefill(torch.zeros(2, 1024, dtype=torch.bfloat16, device="cuda"),
                   pos3=torch.zeros(3, 3, dtype=torch.int32, device="cuda"))
    assert bb.position == 60


def test_prefill_then_decode_handoff(pkg, small):
    """The decode kernel continues from the cache the prefill wrote (generator.py:104-119 then
    :152-172): a 100-token prompt, then 3 backbone decode steps with the codec head. The oracle
    does the same, prefilling with its bf16 policy and handing that KV to its kernel policy. The
    decode hidden states agree within the prefill's tolerance, since the two caches differ only
    at bf16 rounding level."""
    dsd, tw = small
    S = 100
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=256)
    pf = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "hf_bf16")
    g = torch.Generator().manual_seed(31)
    x = torch.randn(S + 3, 1024, generator=g).to(torch.bfloat16)
    print("prefill + decode handoff: launching", flush=True)
    bb.prefill(x[:S].cuda())
    for i in range(S):
        pf.step(x[i], pos=i)
    dec = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "kernel")
    dec.set_kv(pf.k[:, :, :S], pf.v[:, :, :S])
    worst = 0.0
    for j in range(3):
        h = bb.decode_step_with_embedding(x[S + j].cuda())
        hr, _ = dec.step(x[S + j], pos=S + j)
        worst = max(worst, rel_l2(h.cpu(), hr))
    bb.check_error()
    print(f"prefill + decode handoff: worst decode hidden rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
    assert bb.position == S + 3


def test_prefill_fills_the_cache_in_one_or_two_calls(pkg, small):
    """Maximum size: a 4096-token prompt fills the whole cache (max_seq_len 4096) in one call,
    and again as two 2048-token calls, the second continuing from the first one's cache. Causal
    attention makes the two equivalent; they differ only in summation order (the GEMMs split K
    differently at 4096 and 2048 rows), so K, V and the last hidden agree within TOL. (The
    oracle is too slow at this size; the 2-layer cases above pin the arithmetic.)"""
    dsd, _ = small
    S = 4096
    x = torch.randn(S, 1024, generator=torch.Generator().manual_seed(4096)).to(torch.bfloat16).cuda()
    one = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=S)
    _print("prefill 2 layers S=4096 in one call: launching")
    h1 = one.prefill(x)
    two = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=S)
    _print("prefill 2 layers S=4096 as 2 x 2048: launching")
    two.prefill(x[:2048])
    h2 = two.prefill(x[2048:])
    torch.cuda.synchronize()
    one.check_error()
    two.check_error()
    ek = rel_l2(one.get_k_cache().float().cpu(), two.get_k_cache().float().cpu())
    ev = rel_l2(one.get_v_cache().float().cpu(), two.get_v_cache().float().cpu())
    eh = rel_l2(h1.cpu(), h2.cpu())
    _print(f"S=4096 one call vs two: K rel_l2 {ek:.2e}, V {ev:.2e}, hidden {eh:.2e}")
    assert ek < TOL and ev < TOL and eh < TOL
    assert one.position == S and two.position == S
