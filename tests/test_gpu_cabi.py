"""GPU: the reference-compatible C launchers called through ctypes (no torch extension), the way
the reference's Python side would bind them, checked against the CPU oracle.

launch_tts_decode_with_embedding  <- fused_decode_tts.cu:834-857
launch_tts_decode                 <- fused_decode_tts.cu:664-688 (token-id gather)
launch_cp_decode_with_embedding   <- fused_decode_code_predictor.cu:674-697
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
    assert rel_l2(kc[:, :, :16].cpu(), orc.k[:, :, :16]) == 0.0
