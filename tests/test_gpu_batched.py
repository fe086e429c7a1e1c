"""GPU: BASELINE config 4 -- a batch of 8 independent streams with ragged attended KV lengths
in [128, 1024] (per-stream positions and attention lengths), one backbone step with codec head,
suppress mask and greedy g0, then one code-predictor frame per stream, against the committed
oracle fixture tests/golden/c4_batched.npz."""
import json

import numpy as np
import pytest
import torch

from golden import cases
from oracle.qtts_oracle import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def test_c4_batch8_ragged(pkg):
    manifest = json.loads((cases.HERE / "manifest.json").read_text())["cases"]["c4"]
    sd = cases.weights(pkg, "c4")
    assert cases.weight_digest(sd) == manifest["weights"], "seeded weight generator drifted"
    dsd = {k: v.cuda() for k, v in sd.items()}
    fx = cases.load("c4_batched")
    lengths = cases.c4_lengths()
    assert lengths == fx["lengths"].tolist()
    n = len(lengths)
    dec = pkg.BatchedTTSDecoder(dsd, n, max_seq_len=max(lengths) + 8)
    xs, texts = [], []
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
    worst = max(rel_l2(hidden[s].cpu(), torch.from_numpy(fx["hidden"][s])) for s in range(n))
    print(f"c4 batch {n}, lengths {lengths}: worst hidden rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
    assert np.array_equal(toks.cpu().numpy(), fx["tokens"])
    assert np.array_equal(comb.float().cpu().numpy(), fx["combined"])
    assert dec.positions() == lengths
