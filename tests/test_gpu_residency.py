"""GPU: failure handling of the persistent launches, forced from the host. No kernel faults, traps
or hangs here: every workgroup of every launch runs to its end.

The launches are plain (not cooperative), so residency of all 256 workgroups is not promised by
the runtime. Every in-kernel wait is bounded; a wait that gives up latches the workspace's error
word, every later wait of the launch sees the word at its next check and gives up too, and the
host's check_error() raises. The waits of a launch's first layer pass, which complete only once
every workgroup has started, run under a short cap (2^15 poll rounds, about 30 ms, against 2^22
for later waits): the arrival check.

* A pre-set error word (the state a timed-out wait leaves) ends every wait of the next launch at
  its first check: the launch returns, check_error() raises, and the launch after it is clean and
  bit-identical to a clean one.
* With the entry cap 128 times below its default, co-resident launches still complete without
  error and bit-identical: the first exchanges finish well inside the cap.
"""
import ctypes

import pytest
import torch

from oracle.qtts_oracle import DecoderOracle, TalkerOracle, TalkerWeights, rel_l2

pytestmark = pytest.mark.gpu
I32 = dict(dtype=torch.int32, device="cuda")


@pytest.fixture(scope="module")
def small(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=2, n_groups=15)
    sd = pkg.synthetic_state_dict(seed=91, cfg=cfg)
    return sd, {k: v.cuda() for k, v in sd.items()}, TalkerWeights.from_state_dict(sd, 2, 2)


def _backbone_step(bb, x, L):
    bb.decoder.set_position(L - 1)
    tok = torch.full((1,), -1, **I32)
    bb.decoder.decode_step_select(x, tok, torch.zeros(1, **I32), 0, 1.0, -1, False, False, 1.0, 0, 1.0, 0, 0)
    torch.cuda.synchronize()
    return bb.decoder.hidden_state_buffer().clone(), int(tok.item())


def _cp_frame(cp, hid, g0, text):
    out = torch.full((16,), -1, **I32)
    comb = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    cp.decoder.frame(hid, torch.tensor([g0], **I32), text, out, comb, -1, torch.zeros(1, **I32), False, 1.0, 0, 1.0,
                     0, 0)
    torch.cuda.synchronize()
    return out.clone(), comb.clone()


def _setup(pkg, small):
    sd, dsd, tw = small
    L = 150   # chunked attention (3 chunks)
    bb = pkg.TTSMegakernelGenerator(model=dsd, max_seq_len=256)
    g = torch.Generator().manual_seed(3)
    k = torch.randn(2, 8, L - 1, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, L - 1, 128, generator=g).to(torch.bfloat16)
    bb.decoder.set_kv_cache(k.cuda(), v.cuda())
    x = torch.randn(1024, generator=g).to(torch.bfloat16)
    cp = pkg.CodePredictorMegakernelGenerator(model=dsd, max_seq_len=32)
    hid = torch.randn(1024, generator=g)
    text = torch.randn(1024, generator=g).to(torch.bfloat16)
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, 256, "backbone", "kernel")
    orc.set_kv(k, v)
    href, _ = orc.step(x, pos=L - 1)
    ids_ref = TalkerOracle(tw, max_seq=64).cp_frame(hid, 17)
    return bb, cp, L, x.cuda(), hid.cuda(), text.cuda(), href, ids_ref


def test_preset_error_word_ends_every_wait(pkg, small):
    bb, cp, L, x, hid, text, href, ids_ref = _setup(pkg, small)
    h0, t0 = _backbone_step(bb, x, L)
    bb.check_error()
    assert rel_l2(h0.cpu(), href) < 1e-5
    o0, c0 = _cp_frame(cp, hid, 17, text)
    cp.check_error()
    assert o0[1:].tolist() == ids_ref
    print("clean launches equal the oracle; pre-setting the error words", flush=True)
    bb.decoder.debug_set_error(1)
    _backbone_step(bb, x, L)           # returns: every wait gives up at its first check
    with pytest.raises(RuntimeError):
        bb.check_error()
    cp.decoder.debug_set_error(1)
    _cp_frame(cp, hid, 17, text)
    with pytest.raises(RuntimeError):
        cp.check_error()
    print("launches with the error word set ended and check_error raised", flush=True)
    # check_error cleared the words: the next launches are clean and bit-identical
    h1, t1 = _backbone_step(bb, x, L)
    bb.check_error()
    assert torch.equal(h0, h1) and t0 == t1
    o1, c1 = _cp_frame(cp, hid, 17, text)
    cp.check_error()
    assert torch.equal(o0, o1) and torch.equal(c0, c1)


def test_short_entry_cap_keeps_resident_launches(pkg, small):
    lib = ctypes.CDLL(str(pkg._ext.library_path()))
    lib.qtts_debug_entry_spin_cap.argtypes = [ctypes.c_uint]
    bb, cp, L, x, hid, text, href, ids_ref = _setup(pkg, small)
    h0, t0 = _backbone_step(bb, x, L)
    o0, c0 = _cp_frame(cp, hid, 17, text)
    bb.check_error()
    cp.check_error()
    assert lib.qtts_debug_entry_spin_cap(256) == 0
    try:
        for rep in range(3):
            h1, t1 = _backbone_step(bb, x, L)
            o1, c1 = _cp_frame(cp, hid, 17, text)
            bb.check_error()
            cp.check_error()
            assert torch.equal(h0, h1) and t0 == t1
            assert torch.equal(o0, o1) and torch.equal(c0, c1)
    finally:
        assert lib.qtts_debug_entry_spin_cap(0) == 0
    print("entry cap 256 poll rounds: 3 backbone steps and 3 frames clean and bit-identical", flush=True)
