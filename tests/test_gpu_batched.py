"""GPU: BASELINE config 4 -- a batch of 8 independent streams with ragged attended KV lengths
in [128, 1024] (per-stream positions and attention lengths), one backbone step with codec head,
suppress mask and greedy g0, then one code-predictor frame per stream, against the committed
oracle fixture tests/golden/c4_batched.npz; and both multi-stream kernels against batch 1.

Two kernels serve several streams (BatchedTTSDecoder ``mode``):
* ``per_xcd``: stream s on XCD s, the batch-1 arithmetic; held bit-identical to batch 1.
* ``shared``: one weight read for all streams, projections on bf16 MFMA with the f32 inputs split
  exactly into three bf16 pieces and f32 sums (the reference kernels' f32 arithmetic). Its sums
  differ from the f64 ones of batch 1 and the oracle by f32 rounding. The stored values hide most
  of that (f32 q/k/v and partials, bf16 backbone residual and KV, bf16 logits): with BASELINE's
  literal N(0, 0.02) norm gains all 8 streams of 28 layers come out bit-identical to batch 1.
  Now and then the difference tips a bf16 rounding of the backbone residual by one ulp (0.4% of
  one element); with N(1, 0.02) gains (the fixtures' non-inert layers) later layers spread such a
  flip to ~5e-3 - 9e-3 rel-L2 of the final hidden, as they spread an f32-level perturbation of the
  f64 oracle itself. So the shared backbone is held to rel-L2 1e-3 at literal gains and to
  north_star's 1e-2 at N(1, 0.02), with the group-0 ids identical (their top-2 gaps logged). The
  code predictor (f32 in both kernels, summed in different orders) is held to identical ids and
  combine, except where a decision is tipped by a last-bit difference (the oracle's own choice
  under a one-ulp move of one logit, checked when it occurs).
"""
import json
import math

import numpy as np
import pytest
import torch

from golden import cases
from oracle.qtts_oracle import TalkerOracle, TalkerWeights, head_logits, rb, rel_l2, sample_token

pytestmark = pytest.mark.gpu
TOL = 1e-5
TOL_SHARED_BB = 2e-3      # 2-layer models: a flip has few layers to spread through
TOL_SHARED_LITERAL = 1e-3  # 28 layers, N(0, 0.02) gains
TOL_NORTH_STAR = 1e-2      # 28 layers, N(1, 0.02) gains
MODES = ["per_xcd", "shared"]


def _gap(logits: torch.Tensor) -> float:
    """Top-2 gap of a logit vector (how far its greedy choice is from a tie)."""
    v = torch.topk(logits[torch.isfinite(logits)].double(), 2)[0]
    return float(v[0] - v[1])


@pytest.mark.parametrize("mode", MODES)
def test_c4_batch8_ragged(pkg, mode):
    manifest = json.loads((cases.HERE / "manifest.json").read_text())["cases"]["c4"]
    sd = cases.weights(pkg, "c4")
    assert cases.weight_digest(sd) == manifest["weights"], "seeded weight generator drifted"
    dsd = {k: v.cuda() for k, v in sd.items()}
    fx = cases.load("c4_batched")
    lengths = cases.c4_lengths()
    assert lengths == fx["lengths"].tolist()
    n = len(lengths)
    dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=max(lengths) + 8, mode=mode)
    xs, texts = [], []
    print(f"c4 ({mode}): lengths {lengths}", flush=True)
    for s, L in enumerate(lengths):
        k, v, x, text = cases.c4_stream_inputs(s, L)
        dec.set_kv_cache(s, k.cuda(), v.cuda())
        xs.append(x)
        texts.append(text)
    assert dec.positions() == [L - 1 for L in lengths]
    i32 = dict(dtype=torch.int32, device="cuda")
    g0 = torch.zeros(n, **i32)
    hidden = dec.step_select(torch.stack(xs).cuda(), g0, cases.EOS_ID)
    toks = torch.full((n, 16), -1, **i32)
    comb = torch.empty(n, 1024, dtype=torch.bfloat16, device="cuda")
    dec.cp_frames(hidden, g0, torch.stack(texts).cuda(), toks, comb)
    torch.cuda.synchronize()
    dec.check_error()
    errs = [rel_l2(hidden[s].cpu(), torch.from_numpy(fx["hidden"][s])) for s in range(n)]
    print(f"c4 batch {n} ({mode}), lengths {lengths}: hidden rel_l2 per stream {[f'{e:.1e}' for e in errs]}", flush=True)
    assert dec.positions() == lengths
    if mode == "per_xcd":
        assert max(errs) < TOL
        assert np.array_equal(toks.cpu().numpy(), fx["tokens"])
        assert np.array_equal(comb.float().cpu().numpy(), fx["combined"])
        return
    assert max(errs) < TOL_NORTH_STAR
    gaps = [_gap(d.decoder.logits_buffer()) for d in dec.streams]
    print(f"  g0 {toks[:, 0].tolist()}, top-2 gaps {[f'{g:.3f}' for g in gaps]}", flush=True)
    assert np.array_equal(toks[:, 0].cpu().numpy(), fx["tokens"][:, 0])
    # the weight-shared code-predictor frame against the oracle (kernel policy, 5 layers) run from
    # each stream's own GPU backbone hidden, as read back after step_select; ids and combine
    # identical, or at the first differing group a decision that a last-bit difference tips
    orc = _cp_oracle(sd, 5)
    toks_h, comb_h = toks.cpu(), comb.cpu()
    for s in range(n):
        got = toks_h[s].tolist()
        ids = [got[0]] + orc.cp_frame(hidden[s].cpu(), got[0])
        if got != ids:
            _explain_cp_difference(orc, hidden[s], got[0], ids, got, False, {}, 0, f"stream {s}")
            continue
        assert torch.equal(comb_h[s], orc.combine(ids, texts[s])), f"stream {s}: combined input differs from the oracle"
        print(f"  stream {s}: 15 code-predictor ids and the combine equal to the oracle's", flush=True)


def test_shared_28_layers_literal_gains(pkg):
    """The weight-shared backbone step and code-predictor frame of 8 streams at the c4 lengths,
    28 + 5 layers with BASELINE's literal N(0, 0.02) norm gains, against the per-XCD kernels
    (bit-identical to batch 1): hidden and logits within TOL_SHARED_LITERAL (observed 0 and ~1e-7:
    a logit can round to the next bf16 value), every id identical, top-2 gaps logged."""
    sd = pkg.synthetic_state_dict(seed=cases.SEEDS["c4"], cfg=pkg.SyntheticConfig(norm_mean=0.0))
    dsd = {k: v.cuda() for k, v in sd.items()}
    lengths = cases.c4_lengths()
    n = len(lengths)
    i32 = dict(dtype=torch.int32, device="cuda")
    out = {}
    for mode in ("shared", "per_xcd"):
        dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=max(lengths) + 8, mode=mode)
        xs, texts = [], []
        for s, L in enumerate(lengths):
            k, v, x, text = cases.c4_stream_inputs(s, L)
            dec.set_kv_cache(s, k.cuda(), v.cuda())
            xs.append(x)
            texts.append(text)
        print(f"literal gains ({mode}): launching", flush=True)
        g0 = torch.zeros(n, **i32)
        hidden = dec.step_select(torch.stack(xs).cuda(), g0, cases.EOS_ID)
        toks = torch.full((n, 16), -1, **i32)
        comb = torch.empty(n, 1024, dtype=torch.bfloat16, device="cuda")
        dec.cp_frames(hidden, g0, torch.stack(texts).cuda(), toks, comb)
        torch.cuda.synchronize()
        dec.check_error()
        out[mode] = (hidden.cpu(), [d.decoder.logits_buffer().cpu() for d in dec.streams], toks.cpu(), comb.cpu())
    (hs, ls, ts, cs), (hp, lp, tp, cp_) = out["shared"], out["per_xcd"]
    for s in range(n):
        eh, el = rel_l2(hs[s], hp[s]), rel_l2(ls[s], lp[s])
        print(f"  stream {s} (L={lengths[s]}): hidden {eh:.1e} logits {el:.1e} top-2 gap {_gap(lp[s]):.2e}", flush=True)
        assert eh < TOL_SHARED_LITERAL and el < TOL_SHARED_LITERAL
    assert torch.equal(ts, tp), f"ids differ: {ts.tolist()} vs {tp.tolist()}"
    assert torch.equal(cs, cp_)


def _batched_pair(pkg, lengths, seed, mode="per_xcd"):
    """Two BatchedTTSDecoders over one 2-layer synthetic model with identical per-stream KV
    prefixes: stream s attends lengths[s] positions (its new entry at slot lengths[s] - 1). The
    first runs in `mode`; the second's streams serve as batch-1 references."""
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=1, n_groups=1)
    dsd = {k: v.cuda() for k, v in pkg.synthetic_state_dict(seed=seed, cfg=cfg).items()}
    n, S = len(lengths), max(lengths)
    decs = [pkg.BatchedTTSDecoder(dsd, n, max_seq_len=S, mode=m) for m in (mode, "per_xcd")]
    g = torch.Generator().manual_seed(seed)
    for s, L in enumerate(lengths):
        k = torch.randn(2, 8, L - 1, 128, generator=g).to(torch.bfloat16).cuda()
        v = torch.randn(2, 8, L - 1, 128, generator=g).to(torch.bfloat16).cuda()
        for d in decs:
            if L > 1:
                d.set_kv_cache(s, k, v)
            else:
                d.streams[s].set_position(0)
    return decs


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("lengths,sample", [
    ([1, 33, 64, 65, 577, 4096, 200, 2, 1500], False),
    ([4096, 129, 1000], True),
], ids=["greedy9", "sampled3"])
def test_backbone_streams_match_batch1(pkg, lengths, sample, mode):
    """One launch of up to 8 backbone streams (decode_steps_streams) against batch-1
    decode_step_select on a copy of each stream. per_xcd (stream s on XCD s): token, final-norm
    hidden, residual, logits and the new KV entry bit-identical. shared: token identical, the
    states within rel-L2 TOL_SHARED_BB. Lengths mix the batch-1 one-pass local attention (<= 64)
    and its chunked split up to 32 (chunk, head) units (4096: 8 per workgroup), and give the
    shared kernel's length-proportional units (1 .. 8 per stream); 9 streams take two launches
    (8 + 1); the sampled case adds top-k / top-p, temperature and a repetition penalty over
    per-stream histories of different lengths."""
    n = len(lengths)
    xl, ref = _batched_pair(pkg, lengths, 70 + n, mode)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, 1024, generator=g).to(torch.bfloat16).cuda()
    vocab = xl.vocab_size
    hist = torch.randint(0, vocab, (n, 24), generator=g, dtype=torch.int32).cuda()
    n_hist = [24, 0, 7][:n] if sample else []
    kw = dict(repetition_penalty=1.3 if sample else 1.0, suppress_eos=False, do_sample=sample, temperature=0.8,
              top_k=40, top_p=0.9, frame_step=3)
    i32 = dict(dtype=torch.int32, device="cuda")
    tok = torch.full((n,), -1, **i32)
    print(f"backbone streams {lengths} sample={sample} ({mode}): launching", flush=True)
    hidden = xl.step_select(x, tok, cases.EOS_ID, history=hist if sample else None, n_history=n_hist, seed=5, **kw)
    for s, dec in enumerate(ref.streams):
        t1 = torch.full((1,), -1, **i32)
        dec.decoder.decode_step_select(x[s], t1, hist[s], n_hist[s] if sample else 0, kw["repetition_penalty"],
                                       cases.EOS_ID, False, sample, kw["temperature"], kw["top_k"], kw["top_p"], 5 + s,
                                       kw["frame_step"])
        torch.cuda.synchronize()
        xd = xl.streams[s].decoder
        L = lengths[s]
        if mode == "per_xcd":
            assert torch.equal(tok[s:s + 1], t1), f"stream {s} (L={L}): token {tok[s].item()} vs {t1.item()}"
            assert torch.equal(hidden[s], dec.decoder.hidden_state_buffer()), f"stream {s}: hidden differs"
            assert torch.equal(xd.residual_buffer(), dec.decoder.residual_buffer()), f"stream {s}: residual differs"
            assert torch.equal(xd.logits_buffer(), dec.decoder.logits_buffer()), f"stream {s}: logits differ"
            assert torch.equal(xd.get_k_cache()[:, :, L - 1], dec.decoder.get_k_cache()[:, :, L - 1])
            assert torch.equal(xd.get_v_cache()[:, :, L - 1], dec.decoder.get_v_cache()[:, :, L - 1])
        else:
            eh = rel_l2(hidden[s], dec.decoder.hidden_state_buffer())
            el = rel_l2(xd.logits_buffer(), dec.decoder.logits_buffer())
            ek = rel_l2(xd.get_k_cache()[:, :, L - 1].float(), dec.decoder.get_k_cache()[:, :, L - 1].float())
            ev = rel_l2(xd.get_v_cache()[:, :, L - 1].float(), dec.decoder.get_v_cache()[:, :, L - 1].float())
            print(f"  stream {s} (L={L}): hidden {eh:.1e} logits {el:.1e} K {ek:.1e} V {ev:.1e}, "
                  f"top-2 gap {_gap(dec.decoder.logits_buffer()):.3e}", flush=True)
            assert max(eh, el, ek, ev) < TOL_SHARED_BB, f"stream {s} (L={L})"
            assert torch.equal(tok[s:s + 1], t1), f"stream {s} (L={L}): token {tok[s].item()} vs {t1.item()}"
    xl.check_error()
    ref.check_error()
    assert xl.positions() == ref.positions() == lengths
    print(f"backbone streams {lengths}: tokens {tok.tolist()}", flush=True)


def test_backbone_streams_reject_bad_arguments(pkg):
    """decode_steps_streams validates before launching: more than 8 decoders, a decoder listed
    twice, a decoder over other weight tensors, a full KV cache; positions stay unchanged."""
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=1, n_groups=1)
    dsd = {k: v.cuda() for k, v in pkg.synthetic_state_dict(seed=5, cfg=cfg).items()}
    bd = pkg.BatchedTTSDecoder(dsd, 2, max_seq_len=16)
    lead, other = bd.streams[0].decoder, bd.streams[1].decoder
    i32 = dict(dtype=torch.int32, device="cuda")
    x2 = torch.zeros(2, 1024, dtype=torch.bfloat16, device="cuda")
    h2 = torch.empty(2, 1024, device="cuda")
    args = (None, [], 1.0, -1, False, False, 1.0, 0, 1.0, 0, 0)
    with pytest.raises(RuntimeError, match="1..8"):
        lead.decode_steps_streams([lead] * 9, torch.zeros(9, 1024, dtype=torch.bfloat16, device="cuda"),
                                  torch.zeros(9, **i32), torch.empty(9, 1024, device="cuda"), *args)
    with pytest.raises(RuntimeError, match="twice"):
        lead.decode_steps_streams([lead, lead], x2, torch.zeros(2, **i32), h2, *args)
    alien = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=16).decoder   # its own weight copy
    with pytest.raises(RuntimeError, match="share"):
        lead.decode_steps_streams([lead, alien], x2, torch.zeros(2, **i32), h2, *args)
    other.set_position(16)
    with pytest.raises(RuntimeError, match="KV cache full"):
        lead.decode_steps_streams([lead, other], x2, torch.zeros(2, **i32), h2, *args)
    assert lead.position() == 0 and other.position() == 16


def _bf16_step(v: float, up: bool) -> float:
    """The neighbouring bf16 value of the bf16 value v (towards +inf when up)."""
    b = int(torch.tensor([v], dtype=torch.bfloat16).view(torch.int16)[0]) & 0xFFFF
    b = b + (1 if (up == (b < 0x8000)) else -1) if v != 0.0 else (0x0001 if up else 0x8001)
    return float(torch.tensor([b if b < 0x8000 else b - 0x10000], dtype=torch.int16).view(torch.bfloat16)[0])


def _cp_oracle(sd, n_cp):
    """The oracle (kernel policy) over the n_cp code-predictor layers of sd (one backbone layer,
    unused)."""
    return TalkerOracle(TalkerWeights.from_state_dict(sd, 1, n_cp), max_seq=64, policy="kernel")


def _cp_last_bit_choice(orc, hid, g0, ids_ref, ids_got, j, sample, kw, seed):
    """Group j (1..15) of a code-predictor frame, where two computations chose ids_ref[j] and
    ids_got[j] after agreeing on groups 1..j-1. The oracle (kernel policy, f64 sums), teacher-forced
    with the agreed ids, must choose ids_ref[j] from its bf16 logits, and ids_got[j] once one logit
    moves by one bf16 ulp (ids_got[j] up or ids_ref[j] down): a decision that a last-bit difference
    of one sum tips, through the top-2 order, the top-k boundary or a greedy tie. Returns the move."""
    tw = orc.w
    orc.cp.reset()
    orc.cp.step(rb(hid.float().cpu()).to(torch.bfloat16), pos=0)
    h, _ = orc.cp.step(orc.bb_emb[g0], pos=1)
    for g in range(j - 1):
        h, _ = orc.cp.step(orc.cp_emb[g][ids_ref[g + 1]], pos=g + 2)
    lg = head_logits(tw.cp_heads[j - 1], h).float()

    def pick(x):
        return sample_token(x, sample, kw.get("temperature", 1.0), kw.get("top_k", 0), 1.0, None, seed=seed,
                            frame_step=kw.get("frame_step", 0), group=j)

    assert pick(lg) == ids_ref[j], f"group {j}: the oracle picks {pick(lg)}, the reference side {ids_ref[j]}"
    for idx, up, label in ((ids_got[j], True, "kernel's id one ulp up"), (ids_ref[j], False, "reference side's id one ulp down")):
        moved = lg.clone()
        moved[idx] = _bf16_step(float(lg[idx]), up)
        if pick(moved) == ids_got[j]:
            return label
    raise AssertionError(f"group {j}: {ids_got[j]} is not the oracle's choice under a one-ulp move of either logit")


def _explain_cp_difference(orc, hid, g0, ids_ref, ids_got, sample, kw, seed, label):
    """ids_got differs from ids_ref (group 0 equal): the first differing group must be a decision
    that a last-bit difference tips (_cp_last_bit_choice); later groups start from different inputs
    and are not compared."""
    j = next(k for k in range(16) if ids_ref[k] != ids_got[k])
    assert j >= 1, f"{label}: group 0 id is the input and must be equal"
    how = _cp_last_bit_choice(orc, hid, g0, ids_ref, ids_got, j, sample, kw, seed)
    print(f"{label}: first difference at group {j} ({ids_ref[j]} vs {ids_got[j]}): the oracle's choice with the "
          f"{how}", flush=True)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n,sample", [(3, False), (9, True), (8, False)], ids=["greedy3", "sampled9", "greedy8"])
def test_cp_frames_streams_match_batch1(pkg, n, sample, mode):
    """Code-predictor frames of n streams through BatchedTTSDecoder.cp_frames (up to 8 per launch)
    against the batch-1 frame() of each stream with the same key (seed + s); 9 streams take two
    launches; the sampled case draws every group with temperature and top-k.

    per_xcd: the 15 group ids and the combined next input identical (the batch-1 arithmetic).
    shared: the same, except where the two kernels' f32 sums (different summation orders) tip a
    last-bit decision: at the first differing group the oracle, teacher-forced with the agreed
    earlier ids, must choose batch 1's id, and the shared kernel's once one bf16 logit moves by one
    ulp (every later group of that frame starts from different inputs and is not compared)."""
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=2, n_groups=15)
    sd = pkg.synthetic_state_dict(seed=40 + n, cfg=cfg)
    dsd = {k: v.cuda() for k, v in sd.items()}
    dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=16, mode=mode)
    g = torch.Generator().manual_seed(n)
    hid = torch.randn(n, 1024, generator=g).cuda()
    i32 = dict(dtype=torch.int32, device="cuda")
    g0 = torch.randint(0, 2048, (n,), generator=g, dtype=torch.int32).cuda()
    text = torch.randn(n, 1024, generator=g).to(torch.bfloat16).cuda()
    toks = torch.full((n, 16), -1, **i32)
    comb = torch.empty(n, 1024, dtype=torch.bfloat16, device="cuda")
    kw = dict(do_sample=sample, temperature=0.8, top_k=30, seed=11, frame_step=5)
    print(f"cp frames {n} streams sample={sample} ({mode}): launching", flush=True)
    dec.cp_frames(hid, g0, text, toks, comb, **kw)
    cp = dec.cp.decoder
    orc = _cp_oracle(sd, 2)
    for s in range(n):
        t1 = torch.full((16,), -1, **i32)
        c1 = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
        cp.frame(hid[s].contiguous(), g0[s:s + 1], text[s].contiguous(), t1, c1, -1, torch.zeros(1, **i32), sample,
                 kw["temperature"], kw["top_k"], 1.0, kw["seed"] + s, kw["frame_step"])
        torch.cuda.synchronize()
        if mode == "shared":
            # against the oracle from the same hidden, then against batch 1
            got = toks[s].tolist()
            ids = [got[0]] + orc.cp_frame(hid[s].cpu(), got[0], sample, kw["temperature"], kw["top_k"],
                                          seed=kw["seed"] + s, frame_step=kw["frame_step"])
            if got != ids:
                _explain_cp_difference(orc, hid[s], got[0], ids, got, sample, kw, kw["seed"] + s,
                                       f"stream {s} (oracle)")
            else:
                assert torch.equal(comb[s].cpu(), orc.combine(ids, text[s].cpu())), f"stream {s}: combine vs oracle"
            if not torch.equal(toks[s], t1):
                _explain_cp_difference(orc, hid[s], got[0], t1.tolist(), got, sample, kw, kw["seed"] + s,
                                       f"stream {s} (batch 1)")
                continue
        assert torch.equal(toks[s], t1), f"stream {s}: {toks[s].tolist()} vs {t1.tolist()}"
        assert torch.equal(comb[s], c1), f"stream {s}: combined input differs"
    dec.check_error()
    print(f"cp frames {n} streams: first stream groups {toks[0, 1:6].tolist()}...", flush=True)


@pytest.mark.parametrize("n_cp_layers,n_groups", [(1, 1), (1, 15), (2, 2), (3, 15)])
def test_shared_cp_two_column_pass(pkg, n_cp_layers, n_groups):
    """The weight-shared code-predictor frame runs positions 0 and 1 of every stream as one
    two-column pass (16 input columns: 8 streams x 2 positions); the second column publishes into
    the exchange buffers of the other parity. Odd and even layer counts, a one-layer pass (its
    only layer is position 0's last, which writes only the K/V entry) and frames of 1, 2 and 15
    groups (a frame of 1 group ends with the pass's head). 5 streams, greedy and sampled: ids and
    combine against the oracle (kernel policy) from the same hidden, under the last-bit rule."""
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=n_cp_layers, n_groups=n_groups)
    sd = pkg.synthetic_state_dict(seed=600 + 7 * n_cp_layers + n_groups, cfg=cfg)
    dsd = {k: v.cuda() for k, v in sd.items()}
    n = 5
    dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=16, mode="shared")
    orc = _cp_oracle(sd, n_cp_layers)
    g = torch.Generator().manual_seed(n_cp_layers * 100 + n_groups)
    i32 = dict(dtype=torch.int32, device="cuda")
    for sample in (False, True):
        hid = torch.randn(n, 1024, generator=g).cuda()
        g0 = torch.randint(0, 2048, (n,), generator=g, dtype=torch.int32).cuda()
        text = torch.randn(n, 1024, generator=g).to(torch.bfloat16).cuda()
        toks = torch.full((n, n_groups + 1), -1, **i32)
        comb = torch.empty(n, 1024, dtype=torch.bfloat16, device="cuda")
        kw = dict(do_sample=sample, temperature=0.8, top_k=30, seed=21, frame_step=3)
        print(f"shared cp frame, {n_cp_layers} layers, {n_groups} groups, sample={sample}: launching", flush=True)
        dec.cp_frames(hid, g0, text, toks, comb, **kw)
        torch.cuda.synchronize()
        dec.check_error()
        for s in range(n):
            got = toks[s].tolist()
            ids = [got[0]] + orc.cp_frame(hid[s].cpu(), got[0], sample, kw["temperature"], kw["top_k"],
                                          seed=kw["seed"] + s, frame_step=kw["frame_step"])
            assert got[0] == int(g0[s])
            if got != ids:
                _explain_cp_difference(orc, hid[s], got[0], ids, got, sample, kw, kw["seed"] + s, f"stream {s}")
                continue
            assert torch.equal(comb[s].cpu(), orc.combine(ids, text[s].cpu())), f"stream {s}: combine vs oracle"
        print(f"  stream 0: {toks[0, 1:].tolist()[:6]}", flush=True)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("sample", [False, True], ids=["greedy", "sampled"])
def test_batched_generate_matches_single_stream(pkg, sample, mode):
    """BatchedTTSDecoder.generate() -- per-stream prefill, then one code-predictor launch and one
    backbone launch per frame for all streams -- against NativeTTSGenerator.generate() of each
    stream with key seed + s, frame for frame and id for id: 3 streams with ragged prompts (40,
    97, 160 tokens) and trailing texts (5, 1, 30 rows). The EOS id is a group-0 token that
    stream 0 first chooses at a frame k >= 5 (not a multiple of sync_every) in a run with EOS
    suppressed, so stream 0 ends there while the others may run on; suppressing that id earlier
    changes no earlier choice, since it was never chosen before. The shared mode runs at BASELINE's
    literal N(0, 0.02) gains (see the module docstring)."""
    # shared mode: BASELINE's literal gains, where the f32 sums tip no stored rounding
    cfg = pkg.SyntheticConfig(n_bb_layers=4, n_cp_layers=2, n_groups=15, norm_mean=1.0 if mode == "per_xcd" else 0.0)
    dsd = {k: v.cuda() for k, v in pkg.synthetic_state_dict(seed=77, cfg=cfg).items()}
    g = torch.Generator().manual_seed(78)
    prompts = [torch.randn(1, S, 1024, generator=g).to(torch.bfloat16) for S in (40, 97, 160)]
    texts = [torch.randn(1, T, 1024, generator=g).to(torch.bfloat16) for T in (5, 1, 30)]
    pad = torch.randn(1, 1, 1024, generator=g).to(torch.bfloat16)
    n, frames_max = 3, 24
    kw = dict(do_sample=sample, temperature=0.9, top_k=40, top_p=0.9, cp_do_sample=sample, cp_temperature=0.8,
              cp_top_k=30, repetition_penalty=1.1, seed=5)
    dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=256, mode=mode)
    print(f"batched generate sample={sample} ({mode}): EOS suppressed run", flush=True)
    free = dec.generate(prompts, texts, pad, 3000, max_tokens=frames_max, min_new_tokens=frames_max, **kw)
    assert [len(f) for f in free] == [frames_max] * n
    g0 = [f[0] for f in free[0]]
    k = next(i for i in range(5, frames_max - 2) if g0[i] not in g0[:i] and i % 8 != 0)
    eos = g0[k]
    print(f"batched generate sample={sample}: EOS = {eos} (stream 0, frame {k})", flush=True)
    out = dec.generate(prompts, texts, pad, eos, max_tokens=frames_max, min_new_tokens=2, **kw)
    assert len(out[0]) == k and out[0] == free[0][:k]
    gen = pkg.NativeTTSGenerator(model=dsd, eos_token_id=eos, max_seq_len=256)
    for s in range(n):
        kws = dict(kw, seed=kw["seed"] + s)
        ref = gen.generate(prompts[s], None, texts[s], pad, max_tokens=frames_max, min_new_tokens=2, **kws)
        print(f"stream {s}: batched {len(out[s])} frames, single-stream {len(ref)}", flush=True)
        assert out[s] == ref, f"stream {s} differs"


def test_batched_generate_rejects_bad_arguments(pkg):
    """Argument checks of BatchedTTSDecoder.generate run for every stream before any stream is
    prefilled: a wrong prompt shape, a wrong trailing-text shape, a prompt too long for
    max_seq_len, or a prompt count different from n_streams raise ValueError and leave every
    stream's position untouched."""
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=1, n_groups=15)
    dsd = {k: v.cuda() for k, v in pkg.synthetic_state_dict(seed=5, cfg=cfg).items()}
    dec = pkg.BatchedTTSDecoder(dsd, 2, max_seq_len=64)
    with pytest.raises(ValueError, match="mode"):
        pkg.BatchedTTSDecoder(dsd, 2, max_seq_len=64, mode="xcd")
    for s in range(2):
        dec.streams[s].set_position(7)
    ok = torch.zeros(1, 10, 1024, dtype=torch.bfloat16)
    txt = torch.zeros(1, 3, 1024, dtype=torch.bfloat16)
    pad = torch.zeros(1, 1, 1024, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="prompt 1"):
        dec.generate([ok, torch.zeros(10, 1024)], [txt, txt], pad, 2150, max_tokens=4)
    with pytest.raises(ValueError, match="trailing text 1"):
        dec.generate([ok, ok], [txt, torch.zeros(3, 1024)], pad, 2150, max_tokens=4)
    with pytest.raises(ValueError, match="stream 1"):
        dec.generate([ok, torch.zeros(1, 60, 1024, dtype=torch.bfloat16)], [txt, txt], pad, 2150, max_tokens=8)
    with pytest.raises(ValueError, match="one prompt"):
        dec.generate([ok], [txt], pad, 2150, max_tokens=4)
    assert dec.positions() == [7, 7]
