"""Write the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py            # all cases (about 3 minutes on 8 cores)
    python tests/golden/make_golden.py c4         # selected cases only (manifest entries merged)

The reference ships no golden vectors for this path (its tests check audio RMS and duration
on real weights), so the fixtures are the oracle's outputs on the seeded cases of
``cases.py``; the oracle itself is pinned against transformers and numpy by
tests/test_oracle_*.py. Each fixture is an ``.npz`` of plain arrays (no pickles) and
``manifest.json`` records the seeds, the weight digest and the shapes.
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE.parent))

import __graft_entry__  # noqa: E402
from golden import cases  # noqa: E402
from oracle.qtts_oracle import (DecoderOracle, TalkerOracle, TalkerWeights, head_logits, sample_token,  # noqa: E402
                                suppress_mask)


def log(*a):
    print(f"[{time.strftime('%H:%M:%S')}]", *a, flush=True)


def f32(t):
    return t.detach().float().cpu().numpy().astype(np.float32)


def main(selected):
    torch.set_num_threads(8)
    pkg = __graft_entry__.import_package()
    mpath = HERE / "manifest.json"
    manifest = {"generator": "tests/golden/make_golden.py", "oracle": "oracle/qtts_oracle.py",
                "torch": torch.__version__, "cases": {}}
    if selected and mpath.exists():
        manifest["cases"] = json.loads(mpath.read_text())["cases"]
    want = lambda c: not selected or c in selected

    if want("c0"):
        c0(pkg, manifest)
    if want("c1"):
        c1(pkg, manifest)
    if want("c2"):
        c2(pkg, manifest)
    if want("c3"):
        c3(pkg, manifest)
    if want("c4"):
        c4(pkg, manifest)
    mpath.write_text(json.dumps(manifest, indent=1) + "\n")
    log("done")


def c0(pkg, manifest):
    """Config-0 backbone step, both gain variants, kernel and HF-bf16 policies."""
    prefill, x = cases.c0_inputs()
    out = {}
    for nm in (0.0, 1.0):
        sd = cases.weights(pkg, "c0", nm)
        tw = TalkerWeights.from_state_dict(sd, 28, 5)
        tag = "g0" if nm == 0.0 else "g1"
        manifest["cases"][f"c0_{tag}"] = {"seed": cases.SEEDS["c0"], "norm_mean": nm, "weights": cases.weight_digest(sd)}
        for pol in ("kernel", "hf_bf16"):
            o = DecoderOracle(tw.bb_layers, tw.bb_norm, 136, "backbone", pol)
            for i in range(128):
                o.step(prefill[i], pos=i)
            h, layers = o.step(x, pos=128)
            out[f"{tag}_{pol}_hidden"] = f32(h)
            out[f"{tag}_{pol}_logits"] = f32(head_logits(tw.codec_head, h))
            log(f"c0 gains N({nm},0.02) {pol}: argmax {int(out[f'{tag}_{pol}_logits'].argmax())}")
            del o
    np.savez_compressed(HERE / "c0_backbone.npz", **out)


def c1(pkg, manifest):
    """One code-predictor frame (greedy)."""
    sd = cases.weights(pkg, "c1")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    hidden, g0, text = cases.c1_inputs()
    talker = TalkerOracle(tw, max_seq=64)
    toks = talker.cp_frame(hidden, g0)
    comb = talker.combine([g0] + toks, text)
    np.savez_compressed(HERE / "c1_cp_frame.npz", tokens=np.array([g0] + toks, dtype=np.int32), combined=f32(comb))
    manifest["cases"]["c1"] = {"seed": cases.SEEDS["c1"], "norm_mean": 1.0, "weights": cases.weight_digest(sd), "g0": g0}
    log("c1 tokens", [g0] + toks)


def c2(pkg, manifest):
    """Frame loop from one 128-token prefill: greedy, sampled, and sampled with a sampled code
    predictor (cp_do_sample)."""
    sd = cases.weights(pkg, "c2")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    prefill, trailing, pad = cases.c2_inputs()
    talker = TalkerOracle(tw, max_seq=4096)
    hidden = talker.prefill(prefill)
    k0, v0, pos0 = talker.bb.k.clone(), talker.bb.v.clone(), talker.bb.position
    lg0 = head_logits(tw.codec_head, hidden)
    lg0[suppress_mask(tw.codec_head.shape[0], cases.EOS_ID)] = float("-inf")

    def run(n, sampling):
        talker.bb.k.copy_(k0)
        talker.bb.v.copy_(v0)
        talker.bb.position = pos0
        s = dict(do_sample=False, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.0, seed=0,
                 cp_do_sample=False, cp_temperature=0.9, cp_top_k=50)
        s.update(sampling)
        g0 = sample_token(lg0, s["do_sample"], s["temperature"], s["top_k"], s["top_p"], cases.EOS_ID,
                          seed=s["seed"], frame_step=0, group=0)
        return talker.decode_frames(hidden, g0, trailing, pad, cases.EOS_ID, max_tokens=n, min_new_tokens=n, **s)

    greedy = run(cases.C2_GREEDY_FRAMES, {})
    log("c2 greedy frames", len(greedy), greedy[0], greedy[-1])
    sampled = run(cases.C2_SAMPLED_FRAMES, cases.C2_SAMPLING)
    log("c2 sampled frames", len(sampled), sampled[0], sampled[-1])
    cp_sampled = run(cases.C2_CP_SAMPLED_FRAMES, cases.C2_CP_SAMPLING)
    log("c2 cp-sampled frames", len(cp_sampled), cp_sampled[0], cp_sampled[-1])
    np.savez_compressed(HERE / "c2_frames.npz", greedy=np.array(greedy, dtype=np.int32),
                        sampled=np.array(sampled, dtype=np.int32), cp_sampled=np.array(cp_sampled, dtype=np.int32))
    manifest["cases"]["c2"] = {"seed": cases.SEEDS["c2"], "norm_mean": 1.0, "weights": cases.weight_digest(sd),
                               "eos_id": cases.EOS_ID, "greedy_frames": len(greedy), "sampled_frames": len(sampled),
                               "sampling": cases.C2_SAMPLING, "cp_sampled_frames": len(cp_sampled),
                               "cp_sampling": cases.C2_CP_SAMPLING}


def c3(pkg, manifest):
    """Long context, distinct monotone (t, h, w)."""
    sd = cases.weights(pkg, "c3")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    k, v, xs = cases.c3_inputs()
    o = DecoderOracle(tw.bb_layers, tw.bb_norm, cases.C3_KV + cases.C3_STEPS, "backbone", "kernel")
    o.set_kv(k, v)
    hs, lgs = [], []
    for j in range(cases.C3_STEPS):
        pos = cases.C3_KV + j
        h, _ = o.step(xs[j], pos=pos, pos3=cases.c3_pos3(pos))
        hs.append(f32(h))
        lgs.append(f32(head_logits(tw.codec_head, h)))
    np.savez_compressed(HERE / "c3_long.npz", hidden=np.stack(hs), logits=np.stack(lgs))
    manifest["cases"]["c3"] = {"seed": cases.SEEDS["c3"], "norm_mean": 1.0, "weights": cases.weight_digest(sd),
                               "kv_len": cases.C3_KV, "steps": cases.C3_STEPS,
                               "pos3": [cases.c3_pos3(cases.C3_KV + j) for j in range(cases.C3_STEPS)]}
    log("c3 argmax", [int(l.argmax()) for l in lgs])


def c4(pkg, manifest):
    """Batch of 8 streams with ragged attended lengths: per stream one backbone step at its
    position (codec head, suppress mask, greedy g0) and one greedy code-predictor frame."""
    sd = cases.weights(pkg, "c4")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    lengths = cases.c4_lengths()
    talker = TalkerOracle(tw, max_seq=max(lengths) + 1)
    mask = suppress_mask(tw.codec_head.shape[0], cases.EOS_ID)
    hid, toks, comb = [], [], []
    for s, L in enumerate(lengths):
        k, v, x, text = cases.c4_stream_inputs(s, L)
        talker.bb.reset()
        talker.bb.set_kv(k, v)
        h, _ = talker.bb.step(x, pos=L - 1)
        lg = head_logits(tw.codec_head, h)
        lg[mask] = float("-inf")
        g0 = sample_token(lg, False, 1.0, 0, 1.0)
        groups = [g0] + talker.cp_frame(h, g0)
        hid.append(f32(h))
        toks.append(groups)
        comb.append(f32(talker.combine(groups, text)))
        log(f"c4 stream {s} L={L}: {groups[:4]}...")
    np.savez_compressed(HERE / "c4_batched.npz", lengths=np.array(lengths, dtype=np.int32), hidden=np.stack(hid),
                        tokens=np.array(toks, dtype=np.int32), combined=np.stack(comb))
    manifest["cases"]["c4"] = {"seed": cases.SEEDS["c4"], "norm_mean": 1.0, "weights": cases.weight_digest(sd),
                               "streams": len(lengths), "lengths": lengths, "eos_id": cases.EOS_ID}


if __name__ == "__main__":
    main(sys.argv[1:])
