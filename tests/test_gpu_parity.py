"""GPU parity: the HIP decode kernels against the CPU oracle on the same seeded inputs.

The oracle's kernel policy accumulates in f64 and rounds to f32 / bf16 at the reference's
storage points. The backbone kernel does the same (f64 sums), so its states agree bit for bit
in practice; the code-predictor kernel accumulates in f32, as the reference's CP kernel does,
so its states agree to f32 rounding. Both are held to rel-L2 <= 1e-5 (the north-star bar
against the reference's PyTorch path is 1e-2, checked in test_gpu_golden.py), and greedy
tokens must be identical.
"""
import math

import pytest
import torch

from oracle.qtts_oracle import (DecoderOracle, TalkerOracle, TalkerWeights, head_logits, rel_l2, sample_token,
                                suppress_mask, apply_repetition_penalty)

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _print(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def full(pkg):
    sd = pkg.synthetic_state_dict(seed=1234)
    dsd = {k: v.to("cuda") for k, v in sd.items()}
    return sd, dsd, TalkerWeights.from_state_dict(sd, 28, 5)


def _rand_kv(n_layers, L, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n_layers, 8, L, 128, generator=g).to(dtype)
    v = torch.randn(n_layers, 8, L, 128, generator=g).to(dtype)
    return k, v


def test_backbone_two_layers_prefill_steps(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=1, n_groups=1)
    sd = pkg.synthetic_state_dict(seed=11, cfg=cfg)
    bb = pkg.TTSMegakernelGenerator(model={k: v.cuda() for k, v in sd.items()}, max_seq_len=256)
    tw = TalkerWeights.from_state_dict(sd, 2, 1)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "kernel")
    g = torch.Generator().manual_seed(5)
    xs = torch.randn(70, 1024, generator=g).to(torch.bfloat16)
    worst = 0.0
    for i in range(70):
        h = bb.decode_step_with_embedding(xs[i].cuda())
        hr, _ = orc.step(xs[i], pos=i)
        worst = max(worst, rel_l2(h.cpu(), hr))
    bb.check_error()
    _print(f"2-layer backbone, 70 steps: worst rel_l2 {worst:.2e}")
    assert worst < TOL
    # KV written by the kernel equals the oracle's within bf16 rounding
    k = bb.get_k_cache()[:, :, :70].float().cpu()
    assert rel_l2(k, orc.k[:, :, :70].float()) < TOL


def test_backbone_28_layers_L129(full, pkg):
    sd, dsd, tw = full
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=512)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 512, "backbone", "kernel")
    k, v = _rand_kv(28, 128, 21, torch.bfloat16)
    bb.set_kv_cache(k.cuda(), v.cuda())
    bb.set_position(128)
    orc.set_kv(k, v)
    x = torch.randn(1024, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    h = bb.decode_step_with_embedding(x.cuda())
    hr, layers = orc.step(x, pos=128)
    e = rel_l2(h.cpu(), hr)
    res = bb.decoder.residual_buffer().float().cpu()
    e_res = rel_l2(res, layers[-1])
    lg = head_logits(tw.codec_head, h.cpu())
    lr = head_logits(tw.codec_head, hr)
    _print(f"28-layer backbone L=129: hidden rel_l2 {e:.2e}, residual {e_res:.2e}, logits {rel_l2(lg, lr):.2e}")
    bb.check_error()
    assert e < TOL and e_res < TOL


def test_backbone_long_context_2048(full, pkg):
    sd, dsd, tw = full
    n = 4
    orc = DecoderOracle(tw.bb_layers[:n], tw.bb_norm, 2048, "backbone", "kernel")
    # 4-layer model so the oracle stays fast; exercises 16 chunks x 2 sub-blocks of attention
    sd4 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bbn = pkg.TTSMegakernelGenerator(model=sd4, max_seq_len=2048)
    k, v = _rand_kv(n, 2047, 31, torch.bfloat16)
    bbn.set_kv_cache(k.cuda(), v.cuda())
    bbn.set_position(2047)
    orc.set_kv(k, v)
    x = torch.randn(1024, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    h = bbn.decode_step_with_embedding(x.cuda())
    hr, _ = orc.step(x, pos=2047)
    e = rel_l2(h.cpu(), hr)
    _print(f"4-layer backbone L=2048: hidden rel_l2 {e:.2e}")
    bbn.check_error()
    assert e < TOL


@pytest.mark.parametrize("L", [65, 513, 577, 961, 4096])
def test_backbone_context_edges(full, pkg, L):
    """Attended lengths at the edges of the attention paths: just past the one-pass local path (65:
    2 chunks of 33), the first context past 8 chunks (513: 9 chunks of 57, the poller's second read
    covering one chunk), a ragged chunk split (577: 10 chunks of 58, the last of 55), the first
    context with 16 chunks (961: 16 chunks of 61, the last of 46), and the maximum context (4096 =
    max_seq_len: 16 chunks of 256, 4 sub-blocks each)."""
    sd, dsd, tw = full
    n = 2
    orc = DecoderOracle(tw.bb_layers[:n], tw.bb_norm, L, "backbone", "kernel")
    sd2 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bb = pkg.TTSMegakernelGenerator(model=sd2, max_seq_len=L)
    k, v = _rand_kv(n, L - 1, 40 + L, torch.bfloat16)
    bb.set_kv_cache(k.cuda(), v.cuda())
    bb.set_position(L - 1)
    orc.set_kv(k, v)
    x = torch.randn(1024, generator=torch.Generator().manual_seed(L)).to(torch.bfloat16)
    _print(f"2-layer backbone L={L}: launching")
    h = bb.decode_step_with_embedding(x.cuda())
    hr, _ = orc.step(x, pos=L - 1)
    e = rel_l2(h.cpu(), hr)
    _print(f"2-layer backbone L={L}: hidden rel_l2 {e:.2e}")
    bb.check_error()
    assert e < TOL
    # the new entry landed at the last cache slot
    kc = bb.get_k_cache()[:, :, L - 1].float().cpu()
    assert rel_l2(kc, orc.k[:, :, L - 1].float()) < TOL


def test_backbone_mrope_distinct_positions(full, pkg):
    sd, dsd, tw = full
    n = 2
    sd2 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bb = pkg.TTSMegakernelGenerator(model=sd2, max_seq_len=600)
    orc = DecoderOracle(tw.bb_layers[:n], tw.bb_norm, 600, "backbone", "kernel")
    k, v = _rand_kv(n, 300, 41, torch.bfloat16)
    bb.set_kv_cache(k.cuda(), v.cuda())
    bb.set_position(300)
    orc.set_kv(k, v)
    x = torch.randn(1024, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    pos3 = (300, 157, 111)
    h = bb.decode_step_with_embedding(x.cuda(), pos3=pos3)
    hr, _ = orc.step(x, pos=300, pos3=pos3)
    h1d, _ = DecoderOracle(tw.bb_layers[:n], tw.bb_norm, 600, "backbone", "kernel").step(x, pos=300)
    e = rel_l2(h.cpu(), hr)
    _print(f"mRoPE (300,157,111): rel_l2 {e:.2e} (vs 1D-RoPE oracle {rel_l2(h.cpu(), h1d):.2e})")
    assert e < TOL


def test_cp_reference_steps(full, pkg):
    sd, dsd, tw = full
    cp = pkg.CodePredictorMegakernelGenerator(model=dsd, max_seq_len=256)
    orc = DecoderOracle(tw.cp_layers, tw.cp_norm, 256, "cp", "kernel")
    g = torch.Generator().manual_seed(6)
    worst = 0.0
    for i in range(6):
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        h = cp.decode_step_with_embedding(x.cuda())
        hr, _ = orc.step(x, pos=i)
        worst = max(worst, rel_l2(h.cpu(), hr))
    cp.check_error()
    _print(f"CP 6 steps: worst rel_l2 {worst:.2e}")
    assert worst < TOL


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_cp_frame_greedy_tokens(full, pkg, seed):
    sd, dsd, tw = full
    cp = pkg.CodePredictorMegakernelGenerator(model=dsd, max_seq_len=32)
    talker = TalkerOracle(tw, max_seq=64)
    g = torch.Generator().manual_seed(100 + seed)
    hid = torch.randn(1024, generator=g)
    g0 = int(torch.randint(0, 3072, (1,), generator=g))
    trace = {}
    ref = talker.cp_frame(hid, g0, trace=trace)
    i32 = dict(dtype=torch.int32, device="cuda")
    out = torch.full((16,), -1, **i32)
    comb = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    text = torch.randn(1024, generator=g).to(torch.bfloat16)
    cp.decoder.frame(hid.cuda(), torch.tensor([g0], **i32), text.cuda(), out, comb, -1, torch.zeros(1, **i32),
                     False, 1.0, 0, 1.0, 0, 0)
    torch.cuda.synchronize()
    cp.check_error()
    toks = out.cpu().tolist()
    margins = [float(torch.topk(l, 2)[0][0] - torch.topk(l, 2)[0][1]) for l in trace["cp_logits"]]
    _print(f"CP frame seed {seed}: gpu {toks[1:]} oracle {ref} min top-2 margin {min(margins):.3g}")
    assert toks[0] == g0
    assert toks[1:] == ref
    comb_ref = talker.combine([g0] + ref, text)
    assert torch.equal(comb.cpu(), comb_ref)


@pytest.mark.parametrize("n_cp_layers", [1, 2, 3])
def test_cp_frame_two_column_pass_layer_counts(pkg, n_cp_layers):
    """The frame's positions 0 and 1 run as one two-column pass whose second column publishes into
    the exchange buffers of the other parity; with an even layer count both columns' layer-pass
    numbers have the same parity, with one layer the pass's only layer is position 0's last. Ids,
    combine and the cache entries of positions 0 and 1 against the oracle at 1, 2 and 3 layers."""
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=n_cp_layers, n_groups=15)
    sd = pkg.synthetic_state_dict(seed=77 + n_cp_layers, cfg=cfg)
    dsd = {k: v.to("cuda") for k, v in sd.items()}
    tw = TalkerWeights.from_state_dict(sd, 1, n_cp_layers)
    cp = pkg.CodePredictorMegakernelGenerator(model=dsd, max_seq_len=32)
    talker = TalkerOracle(tw, max_seq=64)
    g = torch.Generator().manual_seed(500 + n_cp_layers)
    i32 = dict(dtype=torch.int32, device="cuda")
    for rep in range(2):
        hid = torch.randn(1024, generator=g)
        g0 = int(torch.randint(0, 3072, (1,), generator=g))
        text = torch.randn(1024, generator=g).to(torch.bfloat16)
        ref = talker.cp_frame(hid, g0)
        out = torch.full((16,), -1, **i32)
        comb = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
        cp.decoder.frame(hid.cuda(), torch.tensor([g0], **i32), text.cuda(), out, comb, -1, torch.zeros(1, **i32),
                         False, 1.0, 0, 1.0, 0, rep)
        torch.cuda.synchronize()
        cp.check_error()
        toks = out.cpu().tolist()
        _print(f"CP {n_cp_layers} layers, frame {rep}: gpu {toks[1:]} oracle {ref}")
        assert toks[0] == g0
        assert toks[1:] == ref
        assert torch.equal(comb.cpu(), talker.combine([g0] + ref, text))
        # the K/V entries the pass wrote for positions 0 and 1, every layer
        kc, vc = cp.decoder.get_k_cache(), cp.decoder.get_v_cache()
        okk, ovv = talker.cp.k, talker.cp.v
        for l in range(n_cp_layers):
            for pos in (0, 1):
                assert rel_l2(kc[l, :, pos].float().cpu(), okk[l, :, pos].float()) < TOL
                assert rel_l2(vc[l, :, pos].float().cpu(), ovv[l, :, pos].float()) < TOL


def test_backbone_head_select_greedy_and_penalty(full, pkg):
    sd, dsd, tw = full
    n = 2
    sd2 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bb = pkg.TTSMegakernelGenerator(model=sd2, max_seq_len=64)
    x = torch.randn(1024, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    i32 = dict(dtype=torch.int32, device="cuda")
    tok = torch.zeros(1, **i32)
    hist = torch.tensor([5, 7, 5, 3000, 12], **i32)
    eos = 2150
    for pen, sup in ((1.0, False), (1.3, True)):
        bb.reset()
        bb.decoder.decode_step_select(x.cuda(), tok, hist, 5, pen, eos, sup, False, 1.0, 50, 1.0, 0, 1)
        torch.cuda.synchronize()
        logits = bb.decoder.logits_buffer().cpu()
        lg = logits.clone()
        lg[suppress_mask(3072, eos)] = float("-inf")
        lg = apply_repetition_penalty(lg, hist.cpu().tolist(), pen)
        ref = sample_token(lg, False, 1.0, 50, 1.0, eos if sup else None)
        _print(f"head select pen={pen} sup={sup}: gpu {int(tok.item())} oracle {ref}")
        assert int(tok.item()) == ref
    bb.check_error()


@pytest.mark.parametrize("top_k,top_p", [(50, 1.0), (0, 0.8), (20, 0.5)])
def test_backbone_sampling_matches_oracle(full, pkg, top_k, top_p):
    sd, dsd, tw = full
    n = 1
    sd1 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bb = pkg.TTSMegakernelGenerator(model=sd1, max_seq_len=64)
    i32 = dict(dtype=torch.int32, device="cuda")
    tok = torch.zeros(1, **i32)
    hist = torch.zeros(1, **i32)
    eos = 2150
    agree = 0
    for trial in range(6):
        x = torch.randn(1024, generator=torch.Generator().manual_seed(50 + trial)).to(torch.bfloat16)
        bb.reset()
        bb.decoder.decode_step_select(x.cuda(), tok, hist, 0, 1.0, eos, False, True, 0.9, top_k, top_p, 77, trial)
        torch.cuda.synchronize()
        lg = bb.decoder.logits_buffer().cpu().clone()
        lg[suppress_mask(3072, eos)] = float("-inf")
        ref = sample_token(lg, True, 0.9, top_k, top_p, None, seed=77, frame_step=trial, group=0)
        agree += int(int(tok.item()) == ref)
    _print(f"sampling top_k={top_k} top_p={top_p}: {agree}/6 identical draws")
    bb.check_error()
    assert agree == 6


def test_reference_kv_roundtrip(full, pkg):
    sd, dsd, tw = full
    sd1 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < 1}
    bb = pkg.TTSMegakernelGenerator(model=sd1, max_seq_len=64)
    k, v = _rand_kv(1, 17, 3, torch.bfloat16)
    bb.set_kv_cache(k.cuda(), v.cuda())
    assert torch.equal(bb.get_k_cache()[:, :, :17].cpu(), k)
    assert torch.equal(bb.get_v_cache()[:, :, :17].cpu(), v)
    assert int(bb.get_k_cache()[:, :, 17:].abs().sum()) == 0


def test_decode_step_token_id_and_argmax(full, pkg):
    """The reference's token-id entry points (megakernel_backbone.py:218-227): decode_step(id)
    gathers the codec embedding row and returns the final hidden; decode_step_with_argmax(id)
    returns argmax(bf16(codec_head . bf16(h))) with no suppress mask, lowest id on ties."""
    sd, dsd, tw = full
    n = 2
    sd2 = {k: v for k, v in dsd.items() if not k.startswith("talker.model.layers.") or int(k.split(".")[3]) < n}
    bb = pkg.TTSMegakernelGenerator(model=sd2, max_seq_len=64)
    orc = DecoderOracle(tw.bb_layers[:n], tw.bb_norm, 64, "backbone", "kernel")
    emb = tw.codec_embedding.to(torch.bfloat16)
    ids = [17, 2900, 1024, 3071, 0, 555]
    worst = 0.0
    for i, t in enumerate(ids):
        if i % 2 == 0:
            h = bb.decoder.decode_step(t).cpu()
            hr, _ = orc.step(emb[t], pos=i)
            worst = max(worst, rel_l2(h, hr))
        else:
            got = bb.decoder.decode_step_with_argmax(t)
            hr, _ = orc.step(emb[t], pos=i)
            lg = head_logits(tw.codec_head, hr)
            ref = int(torch.nonzero(lg == lg.max())[0, 0])
            _print(f"decode_step_with_argmax({t}): gpu {got} oracle {ref}")
            assert got == ref
    bb.check_error()
    _print(f"decode_step(id): worst hidden rel_l2 {worst:.2e}")
    assert worst < TOL
    assert bb.decoder.position() == len(ids)
