"""Write the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py            # all cases (about 2 minutes on 8 cores)

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
from oracle.qtts_oracle import DecoderOracle, TalkerOracle, TalkerWeights, head_logits  # noqa: E402


def log(*a):
    print(f"[{time.strftime('%H:%M:%S')}]", *a, flush=True)


def f32(t):
    return t.detach().float().cpu().numpy().astype(np.float32)


def main():
    torch.set_num_threads(8)
    pkg = __graft_entry__.import_package()
    manifest = {"generator": "tests/golden/make_golden.py", "oracle": "oracle/qtts_oracle.py",
                "torch": torch.__version__, "cases": {}}

    # c0: config-0 backbone step, both gain variants, kernel and HF-bf16 policies
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

    # c1: one code-predictor frame (greedy)
    sd = cases.weights(pkg, "c1")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    hidden, g0, text = cases.c1_inputs()
    talker = TalkerOracle(tw, max_seq=64)
    toks = talker.cp_frame(hidden, g0)
    comb = talker.combine([g0] + toks, text)
    np.savez_compressed(HERE / "c1_cp_frame.npz", tokens=np.array([g0] + toks, dtype=np.int32), combined=f32(comb))
    manifest["cases"]["c1"] = {"seed": cases.SEEDS["c1"], "norm_mean": 1.0, "weights": cases.weight_digest(sd), "g0": g0}
    log("c1 tokens", [g0] + toks)

    # c2: frame loop, greedy and sampled
    sd = cases.weights(pkg, "c2")
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    prefill, trailing, pad = cases.c2_inputs()
    talker = TalkerOracle(tw, max_seq=4096)
    greedy = talker.generate(prefill, trailing, pad, cases.EOS_ID, max_tokens=cases.C2_GREEDY_FRAMES,
                             min_new_tokens=cases.C2_GREEDY_FRAMES)
    log("c2 greedy frames", len(greedy), greedy[0], greedy[-1])
    s = cases.C2_SAMPLING
    sampled = talker.generate(prefill, trailing, pad, cases.EOS_ID, max_tokens=cases.C2_SAMPLED_FRAMES,
                              do_sample=s["do_sample"], temperature=s["temperature"], top_k=s["top_k"],
                              top_p=s["top_p"], repetition_penalty=s["repetition_penalty"], seed=s["seed"],
                              min_new_tokens=cases.C2_SAMPLED_FRAMES)
    log("c2 sampled frames", len(sampled), sampled[0], sampled[-1])
    np.savez_compressed(HERE / "c2_frames.npz", greedy=np.array(greedy, dtype=np.int32), sampled=np.array(sampled, dtype=np.int32))
    manifest["cases"]["c2"] = {"seed": cases.SEEDS["c2"], "norm_mean": 1.0, "weights": cases.weight_digest(sd),
                               "eos_id": cases.EOS_ID, "greedy_frames": len(greedy), "sampled_frames": len(sampled),
                               "sampling": s}

    # c3: long context, distinct monotone (t, h, w)
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

    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    log("done")


if __name__ == "__main__":
    main()
