"""GPU: the reference-compatible C launchers called through ctypes (no torch extension), the way
the reference's Python side would bind them, checked against the CPU oracle.

launch_tts_decode_with_embedding  <- fused_decode_tts.cu:834-857
launch_tts_decode                 <- fused_decode_tts.cu:664-688 (token-id gather)
launch_cp_decode_with_embedding   <- fused_decode_code_predictor.cu:674-697

and the extended entry points (no reference counterpart): qtts_backbone_step_streams (several
streams in one launch) and qtts_backbone_prefill (the prompt prefill, generator.py:209-225).
"""
import ctypes
import struct

import pytest
import torch

from oracle.qtts_oracle import DecoderOracle, TalkerWeights, rel_l2, rope_tables

pytestmark = pytest.mark.gpu
TOL = 1e-5
P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


@pytest.fixture(scope="module")
def lib(pkg):
    lib = ctypes.CDLL(str(pkg._ext.library_path()))
    for name in ("launch_tts_decode_with_embedding", "launch_cp_decode_with_embedding"):
        fn = getattr(lib, name)
        fn.argtypes = [P] * 16 + [I] * 4 + [F, P]
        fn.restype = I
    lib.launch_tts_decode.argtypes = [I, P] + [P] * 15 + [I] * 4 + [F, P]
    lib.launch_tts_decode.restype = I
    return lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _layer_table(layers):
    """num_layers x 11 device pointers (TTSLayerWeights), as megakernel_backbone.py:148-151 builds it."""
    raw = b"".join(struct.pack("<Q", t.data_ptr()) for lw in layers for t in lw)
    return torch.frombuffer(bytearray(raw), dtype=torch.uint8).cuda()


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def model(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=2, n_cp_layers=2, n_groups=1)
    sd = pkg.synthetic_state_dict(seed=77, cfg=cfg)
    return sd, TalkerWeights.from_state_dict(sd, 2, 2)


def test_launch_tts_decode_with_embedding(lib, model):
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq = 64
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    res = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    hid = torch.empty(1024, dtype=torch.float32, device="cuda")
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "kernel")
    g = torch.Generator().manual_seed(1)
    worst = 0.0
    for pos in range(10):
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        xd = x.cuda()
        err = lib.launch_tts_decode_with_embedding(
            _ptr(xd), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res),
            None, None, None, None, None, None, None, _ptr(hid), 2, pos, pos + 1, max_seq, 128 ** -0.5, _stream())
        assert err == 0
        torch.cuda.synchronize()
        hr, outs = orc.step(x, pos=pos)
        worst = max(worst, rel_l2(hid.cpu(), hr), rel_l2(res.float().cpu(), outs[-1]))
    print(f"launch_tts_decode_with_embedding, 10 steps: worst rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
    # invalid arguments are rejected before any launch
    assert lib.launch_tts_decode_with_embedding(
        _ptr(xd), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res),
        None, None, None, None, None, None, None, _ptr(hid), 2, 5, 7, max_seq, 128 ** -0.5, _stream()) != 0
    assert lib.launch_tts_decode_with_embedding(
        _ptr(xd), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res),
        None, None, None, None, None, None, None, _ptr(hid), 2, max_seq, max_seq + 1, max_seq, 128 ** -0.5,
        _stream()) != 0


def test_launch_tts_decode_token_id(lib, model):
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    emb = tw.codec_embedding.cuda()
    norm = tw.bb_norm.cuda()
    max_seq = 16
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    res = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    hid = torch.empty(1024, dtype=torch.float32, device="cuda")
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "kernel")
    for pos, tok in enumerate([5, 3071, 0, 1234]):
        assert lib.launch_tts_decode(tok, _ptr(emb), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc),
                                     _ptr(vc), _ptr(res), None, None, None, None, None, None, None, _ptr(hid),
                                     2, pos, pos + 1, max_seq, 128 ** -0.5, _stream()) == 0
        torch.cuda.synchronize()
        hr, _ = orc.step(tw.codec_embedding[tok], pos=pos)
        assert rel_l2(hid.cpu(), hr) < TOL


def test_launch_cp_decode_with_embedding(lib, model):
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.cp_layers]
    table = _layer_table(layers)
    norm = tw.cp_norm.cuda()
    max_seq = 32
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.float32, device="cuda")
    vc = torch.zeros_like(kc)
    res = torch.empty(1024, dtype=torch.float32, device="cuda")
    hid = torch.empty(1024, dtype=torch.float32, device="cuda")
    orc = DecoderOracle(tw.cp_layers, tw.cp_norm, max_seq, "cp", "kernel")
    g = torch.Generator().manual_seed(2)
    worst = 0.0
    for pos in range(16):
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        assert lib.launch_cp_decode_with_embedding(
            _ptr(x.cuda()), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res),
            None, None, None, None, None, None, None, _ptr(hid), 2, pos, pos + 1, max_seq, 128 ** -0.5,
            _stream()) == 0
        torch.cuda.synchronize()
        hr, outs = orc.step(x, pos=pos)
        worst = max(worst, rel_l2(hid.cpu(), hr), rel_l2(res.cpu(), outs[-1]))
    print(f"launch_cp_decode_with_embedding, 16 steps: worst rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
    # the code predictor accumulates in f32 (the reference's CP arithmetic) against the f64
    # oracle: its f32 cache agrees to f32 rounding
    assert rel_l2(kc[:, :, :16].cpu(), orc.k[:, :, :16]) < TOL


# ---- the extended entry points, bound the same way ------------------------------------------

class QttsBackboneStream(ctypes.Structure):
    """include/qwentts_amd.h QttsBackboneStream."""
    _fields_ = [("k_cache", P), ("v_cache", P), ("position", I), ("pos3", I * 3), ("input_embedding", P),
                ("out_hidden", P), ("out_residual", P), ("out_logits", P), ("out_token", P), ("history", P),
                ("n_history", I), ("seed", ctypes.c_ulonglong), ("skip_if", P)]


def test_qtts_backbone_step_streams(lib, model):
    """Three streams at positions 0, 9 and 40 of their own caches in one launch, each against the
    oracle stepping that stream alone (kernel policy, f64 sums: rel-L2 < 1e-5)."""
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq = 64
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    lib.qtts_workspace_bytes.restype = ctypes.c_size_t
    wsb = lib.qtts_workspace_bytes()
    ws = torch.zeros(3 * wsb, dtype=torch.uint8, device="cuda")
    lib.qtts_workspace_init.argtypes = [P, I]
    lib.qtts_workspace_init.restype = I
    assert lib.qtts_workspace_init(_ptr(ws), torch.cuda.current_device()) == 0
    fn = lib.qtts_backbone_step_streams
    fn.argtypes = [I, P, P, I, P, P, P, I, ctypes.POINTER(QttsBackboneStream), P, I, I, F, I, I, P, I, P]
    fn.restype = I
    g = torch.Generator().manual_seed(8)
    positions = [0, 9, 40]
    bufs, orcs, xs = [], [], []
    arr = (QttsBackboneStream * 3)()
    for s, pos in enumerate(positions):
        kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        kc[:, :, :pos] = torch.randn(2, 8, pos, 128, generator=g).to(torch.bfloat16)
        vc[:, :, :pos] = torch.randn(2, 8, pos, 128, generator=g).to(torch.bfloat16)
        orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "kernel")
        orc.set_kv(kc[:, :, :pos], vc[:, :, :pos])
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        b = dict(kc=kc.cuda(), vc=vc.cuda(), x=x.cuda(), hid=torch.empty(1024, device="cuda"),
                 res=torch.empty(1024, dtype=torch.bfloat16, device="cuda"))
        bufs.append(b); orcs.append(orc); xs.append(x)
        st = arr[s]
        st.k_cache, st.v_cache, st.position = b["kc"].data_ptr(), b["vc"].data_ptr(), pos
        st.pos3[0] = st.pos3[1] = st.pos3[2] = pos
        st.input_embedding, st.out_hidden, st.out_residual = b["x"].data_ptr(), b["hid"].data_ptr(), b["res"].data_ptr()
    assert fn(3, _ptr(ws), _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), max_seq, arr, None, 0, 0, 1.0, -1, 0,
              None, 0, _stream()) == 0
    torch.cuda.synchronize()
    worst = 0.0
    for s, pos in enumerate(positions):
        hr, outs = orcs[s].step(xs[s], pos=pos)
        worst = max(worst, rel_l2(bufs[s]["hid"].cpu(), hr), rel_l2(bufs[s]["res"].float().cpu(), outs[-1]))
        assert rel_l2(bufs[s]["kc"][:, :, pos].float().cpu(), orcs[s].k[:, :, pos].float()) < TOL
    print(f"qtts_backbone_step_streams, 3 streams: worst rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
    # a stream whose skip flag is set computes nothing and writes nothing (streams that ended)
    flags = torch.tensor([0, 1, 0], dtype=torch.int32, device="cuda")
    marker = torch.full((1024,), 7.0, device="cuda")
    bufs[1]["hid"].copy_(marker)
    for s in range(3):
        arr[s].skip_if = flags.data_ptr() + 4 * s
        arr[s].position = positions[s] + 1
        arr[s].pos3[0] = arr[s].pos3[1] = arr[s].pos3[2] = positions[s] + 1
    assert fn(3, _ptr(ws), _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), max_seq, arr, None, 0, 0, 1.0, -1, 0,
              None, 0, _stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(bufs[1]["hid"], marker)
    assert int(bufs[1]["kc"][:, :, positions[1] + 1].float().abs().sum()) == 0
    for s in (0, 2):
        hr, _ = orcs[s].step(xs[s], pos=positions[s] + 1)
        assert rel_l2(bufs[s]["hid"].cpu(), hr) < TOL
    # a stream position outside the cache is rejected before any launch
    arr[2].position = max_seq
    assert fn(3, _ptr(ws), _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), max_seq, arr, None, 0, 0, 1.0, -1, 0,
              None, 0, _stream()) != 0


def test_qtts_backbone_step_shared_skip(lib, model):
    """The weight-shared launch (qtts_backbone_step_shared, the default batched mode) over three
    streams at positions 0, 9 and 40: each within the shared kernel's bar (f32 MFMA sums against
    the f64 oracle, 2 layers: rel-L2 < 2e-3). Then its skip flags: with flags [0, 1, 0] stream 1
    keeps a marker in its hidden and its KV slot stays zero while the others step; a launch with
    every stream skipped (its early return) writes nothing; the launch after it on the same
    workspace is again equal to the oracle."""
    sd, tw = model
    tol = 2e-3
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq = 64
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    lib.qtts_shared_workspace_bytes.restype = ctypes.c_size_t
    ws = torch.zeros(lib.qtts_shared_workspace_bytes(), dtype=torch.uint8, device="cuda")
    lib.qtts_shared_workspace_check.argtypes = [P, ctypes.POINTER(ctypes.c_uint), P]
    lib.qtts_shared_workspace_check.restype = I
    fn = lib.qtts_backbone_step_shared
    fn.argtypes = [I, P, P, I, P, P, P, I, ctypes.POINTER(QttsBackboneStream), P, I, I, F, I, I, P, I, P]
    fn.restype = I
    g = torch.Generator().manual_seed(9)
    positions = [0, 9, 40]
    bufs, orcs, xs = [], [], []
    arr = (QttsBackboneStream * 3)()
    for s, pos in enumerate(positions):
        kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        kc[:, :, :pos] = torch.randn(2, 8, pos, 128, generator=g).to(torch.bfloat16)
        vc[:, :, :pos] = torch.randn(2, 8, pos, 128, generator=g).to(torch.bfloat16)
        orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "kernel")
        orc.set_kv(kc[:, :, :pos], vc[:, :, :pos])
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        b = dict(kc=kc.cuda(), vc=vc.cuda(), x=x.cuda(), hid=torch.empty(1024, device="cuda"),
                 res=torch.empty(1024, dtype=torch.bfloat16, device="cuda"))
        bufs.append(b); orcs.append(orc); xs.append(x)
        st = arr[s]
        st.k_cache, st.v_cache = b["kc"].data_ptr(), b["vc"].data_ptr()
        st.input_embedding, st.out_hidden, st.out_residual = b["x"].data_ptr(), b["hid"].data_ptr(), b["res"].data_ptr()

    def launch(step, flags):
        for s in range(3):
            arr[s].position = positions[s] + step
            arr[s].pos3[0] = arr[s].pos3[1] = arr[s].pos3[2] = positions[s] + step
            arr[s].skip_if = flags.data_ptr() + 4 * s if flags is not None else None
        assert fn(3, _ptr(ws), _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), max_seq, arr, None, 0, 0, 1.0, -1,
                  0, None, 0, _stream()) == 0
        torch.cuda.synchronize()
        code = ctypes.c_uint(0)
        assert lib.qtts_shared_workspace_check(_ptr(ws), ctypes.byref(code), _stream()) == 0 and code.value == 0

    def check(s, step):
        hr, _ = orcs[s].step(xs[s], pos=positions[s] + step)
        e = rel_l2(bufs[s]["hid"].cpu(), hr)
        ek = rel_l2(bufs[s]["kc"][:, :, positions[s] + step].float().cpu(), orcs[s].k[:, :, positions[s] + step].float())
        assert e < tol and ek < tol, (s, step, e, ek)
        return e

    print("qtts_backbone_step_shared, 3 streams: launching", flush=True)
    launch(0, None)
    worst = max(check(s, 0) for s in range(3))
    print(f"qtts_backbone_step_shared, 3 streams: worst rel_l2 {worst:.2e}", flush=True)
    marker = torch.full((1024,), 7.0, device="cuda")
    bufs[1]["hid"].copy_(marker)
    launch(1, torch.tensor([0, 1, 0], dtype=torch.int32, device="cuda"))
    assert torch.equal(bufs[1]["hid"], marker)
    assert int(bufs[1]["kc"][:, :, positions[1] + 1].float().abs().sum()) == 0
    assert int(bufs[1]["vc"][:, :, positions[1] + 1].float().abs().sum()) == 0
    for s in (0, 2):
        check(s, 1)
    # every stream skipped: the launch returns early and writes nothing
    hid_before = [b["hid"].clone() for b in bufs]
    launch(2, torch.ones(3, dtype=torch.int32, device="cuda"))
    for s in range(3):
        assert torch.equal(bufs[s]["hid"], hid_before[s])
        assert int(bufs[s]["kc"][:, :, positions[s] + 2].float().abs().sum()) == 0
    # the next launch on the same workspace; stream 1's slot of step 1 was never written and stays
    # zero, in its cache and in the oracle's (a skipped stream's position still advances)
    launch(2, None)
    for s in range(3):
        check(s, 2)
    print("qtts_backbone_step_shared: skip [0, 1, 0], all skipped, then a normal launch: all as expected", flush=True)


def test_qtts_backbone_prefill(lib, model):
    """A 20-token prompt in one call, K/V straight into the cache, against the oracle's
    transformers-bf16 policy stepped token by token (2 layers: rel-L2 <= 1e-2)."""
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq, S = 64, 20
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    lib.qtts_prefill_workspace_bytes.argtypes = [I, I]
    lib.qtts_prefill_workspace_bytes.restype = ctypes.c_size_t
    wsb = lib.qtts_prefill_workspace_bytes(S, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    fn = lib.qtts_backbone_prefill
    fn.argtypes = [P, ctypes.c_size_t, P, I, P, P, P, P, P, I, I, I, P, P, P, P, I, P, P, I, I, I, P, I, P]
    fn.restype = I
    kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    x = torch.randn(S, 1024, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    xd = x.cuda()
    hid = torch.empty(1024, device="cuda")
    assert fn(_ptr(ws), wsb, _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), max_seq, 0, S,
              None, _ptr(xd), _ptr(hid), None, 0, None, None, 0, -1, 0, None, 0, _stream()) == 0
    torch.cuda.synchronize()
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "hf_bf16")
    hr = None
    for i in range(S):
        hr, _ = orc.step(x[i], pos=i)
    e = (rel_l2(hid.cpu(), hr), rel_l2(kc[:, :, :S].float().cpu(), orc.k[:, :, :S].float()),
         rel_l2(vc[:, :, :S].float().cpu(), orc.v[:, :, :S].float()))
    print(f"qtts_backbone_prefill S={S}: hidden / K / V rel_l2 {e[0]:.2e} {e[1]:.2e} {e[2]:.2e}", flush=True)
    assert max(e) < 1e-2
    # too small a workspace, or a prompt past the cache, is rejected before any launch
    assert fn(_ptr(ws), wsb - 256, _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), max_seq, 0,
              S, None, _ptr(xd), _ptr(hid), None, 0, None, None, 0, -1, 0, None, 0, _stream()) != 0
    assert fn(_ptr(ws), wsb, _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), max_seq, 50, S,
              None, _ptr(xd), _ptr(hid), None, 0, None, None, 0, -1, 0, None, 0, _stream()) != 0
    # an empty prompt is rejected too (and has no workspace size)
    assert fn(_ptr(ws), wsb, _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), max_seq, 0, 0,
              None, _ptr(xd), _ptr(hid), None, 0, None, None, 0, -1, 0, None, 0, _stream()) != 0
    assert lib.qtts_prefill_workspace_bytes(0, 0) == 0


def _bb_step_args(b, table, norm, cos, sin, max_seq, pos):
    return (_ptr(b["x"][pos]), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(b["kc"]), _ptr(b["vc"]),
            _ptr(b["res"][pos]), None, None, None, None, None, None, None, _ptr(b["hid"][pos]), 2, pos, pos + 1,
            max_seq, 128 ** -0.5)


def test_reference_launchers_on_two_streams(lib, model):
    """A backbone decoder on one HIP stream and a code-predictor decoder on another, their
    launches queued alternately with no synchronisation in between (the reference gives every
    decoder object its own scratch). The library keeps one workspace per (device, stream) and
    orders its launches across streams, so every step equals the oracle's."""
    sd, tw = model
    steps, max_seq = 6, 32
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    g = torch.Generator().manual_seed(21)
    dec = {}
    for kind, lw, nrm, kv_dt in (("backbone", tw.bb_layers, tw.bb_norm, torch.bfloat16),
                                  ("cp", tw.cp_layers, tw.cp_norm, torch.float32)):
        layers = [[t.cuda().contiguous() for t in l] for l in lw]
        x = torch.randn(steps, 1024, generator=g).to(torch.bfloat16)
        dec[kind] = dict(layers=layers, table=_layer_table(layers), norm=nrm.cuda(), xh=x, x=x.cuda(),
                         kc=torch.zeros(2, 8, max_seq, 128, dtype=kv_dt, device="cuda"),
                         vc=torch.zeros(2, 8, max_seq, 128, dtype=kv_dt, device="cuda"),
                         res=torch.zeros(steps, 1024, dtype=kv_dt, device="cuda"),
                         hid=torch.zeros(steps, 1024, device="cuda"),
                         orc=DecoderOracle(lw, nrm, max_seq, kind, "kernel"))
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for pos in range(steps):
        for kind, st, fn in (("backbone", sa, lib.launch_tts_decode_with_embedding),
                             ("cp", sb, lib.launch_cp_decode_with_embedding)):
            b = dec[kind]
            assert fn(*_bb_step_args(b, b["table"], b["norm"], cos, sin, max_seq, pos), ctypes.c_void_p(st.cuda_stream)) == 0
    torch.cuda.synchronize()
    worst = 0.0
    for kind, b in dec.items():
        for pos in range(steps):
            hr, outs = b["orc"].step(b["xh"][pos], pos=pos)
            worst = max(worst, rel_l2(b["hid"][pos].cpu(), hr), rel_l2(b["res"][pos].float().cpu(), outs[-1]))
    print(f"reference launchers on two streams, {steps} steps each: worst rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL


def test_sequence_wrap_keeps_results(lib, model):
    """The tag sequence of a workspace runs out after 2^20 - 2 launches; the launch that finds it
    used up zero-fills the workspace and restarts. Steps on either side of that point (set
    through the test hook) equal the oracle's."""
    sd, tw = model
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq = 16
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    lib.qtts_workspace_bytes.restype = ctypes.c_size_t
    ws = torch.zeros(lib.qtts_workspace_bytes(), dtype=torch.uint8, device="cuda")
    lib.qtts_workspace_init.argtypes = [P, I]
    lib.qtts_workspace_init.restype = I
    lib.qtts_debug_set_sequence.argtypes = [P, ctypes.c_uint]
    lib.qtts_debug_set_sequence.restype = I
    assert lib.qtts_workspace_init(_ptr(ws), torch.cuda.current_device()) == 0
    fn = lib.qtts_backbone_step
    fn.argtypes = [P, P, I, P, P, P, P, P, I, I, P, P, P, I, P, P, P, I, P, P, I, P, I, F, I, I, P, I, P, P]
    fn.restype = I
    kc = torch.zeros(2, 8, max_seq, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    hid = torch.empty(1024, device="cuda")
    orc = DecoderOracle(tw.bb_layers, tw.bb_norm, max_seq, "backbone", "kernel")
    g = torch.Generator().manual_seed(31)
    worst = 0.0
    for pos in range(6):
        if pos == 2:
            assert lib.qtts_debug_set_sequence(_ptr(ws), (1 << 20) - 3) == 0   # two launches before the wrap
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        xd = x.cuda()
        assert fn(_ptr(ws), _ptr(table), 2, _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), max_seq, pos, None,
                  _ptr(xd), None, 0, _ptr(hid), None, None, 0, None, None, 0, None, 0, 1.0, -1, 0, None, 0, None,
                  _stream()) == 0
        torch.cuda.synchronize()
        hr, _ = orc.step(x, pos=pos)
        worst = max(worst, rel_l2(hid.cpu(), hr))
    assert lib.qtts_debug_set_sequence(_ptr(ws), 0) != 0 and lib.qtts_debug_set_sequence(_ptr(ws), 1 << 20) != 0
    print(f"sequence wrap: 6 steps across it, worst rel_l2 {worst:.2e}", flush=True)
    assert worst < TOL
