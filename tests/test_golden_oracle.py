"""The CPU oracle still reproduces the committed golden fixtures, and the seeded weight
generator still produces the weights the fixtures were made from (CPU only)."""
import json

import numpy as np
import pytest
import torch

from golden import cases
from oracle.qtts_oracle import DecoderOracle, TalkerOracle, TalkerWeights, head_logits, rel_l2

MANIFEST = json.loads((cases.HERE / "manifest.json").read_text())


@pytest.mark.parametrize("key,case,nm", [("c0_g0", "c0", 0.0), ("c1", "c1", 1.0), ("c3", "c3", 1.0)])
def test_weight_digest_matches_manifest(pkg, key, case, nm):
    assert cases.weight_digest(cases.weights(pkg, case, nm)) == MANIFEST["cases"][key]["weights"]


def test_c1_cp_frame_reproduces(pkg):
    tw = TalkerWeights.from_state_dict(cases.weights(pkg, "c1"), 28, 5)
    fx = cases.load("c1_cp_frame")
    hidden, g0, text = cases.c1_inputs()
    talker = TalkerOracle(tw, max_seq=64)
    toks = talker.cp_frame(hidden, g0)
    assert [g0] + toks == fx["tokens"].tolist()
    assert np.array_equal(talker.combine([g0] + toks, text).float().numpy(), fx["combined"])


def test_c3_long_context_reproduces(pkg):
    tw = TalkerWeights.from_state_dict(cases.weights(pkg, "c3"), 28, 5)
    fx = cases.load("c3_long")
    k, v, xs = cases.c3_inputs()
    o = DecoderOracle(tw.bb_layers, tw.bb_norm, cases.C3_KV + cases.C3_STEPS, "backbone", "kernel")
    o.set_kv(k, v)
    for j in range(cases.C3_STEPS):
        pos = cases.C3_KV + j
        h, _ = o.step(xs[j], pos=pos, pos3=cases.c3_pos3(pos))
        assert np.array_equal(h.float().numpy(), fx["hidden"][j])
        assert np.array_equal(head_logits(tw.codec_head, h).numpy(), fx["logits"][j])


def test_fixture_shapes():
    c0 = cases.load("c0_backbone")
    for g in ("g0", "g1"):
        for pol in ("kernel", "hf_bf16"):
            assert c0[f"{g}_{pol}_hidden"].shape == (1024,) and c0[f"{g}_{pol}_logits"].shape == (3072,)
        # the graded bar between the two policies holds in the fixture itself
        if g == "g0":
            assert rel_l2(torch.from_numpy(c0["g0_kernel_logits"]), torch.from_numpy(c0["g0_hf_bf16_logits"])) < 1e-2
    c2 = cases.load("c2_frames")
    assert c2["greedy"].shape == (cases.C2_GREEDY_FRAMES, 16) and c2["sampled"].shape == (cases.C2_SAMPLED_FRAMES, 16)
    assert (c2["greedy"][:, 0] < 2048).all() and (c2["greedy"][:, 1:] < 2048).all()
