"""GPU: launch_tts_decode_with_embedding_static, the entry point that allocates nothing (its
exchange workspace is a static device array), against launch_tts_decode_with_embedding on the
same inputs, through the C ABI: two calls in a row, the second over a shorter context, each
bit-identical to the allocating entry point (same kernel, same arithmetic)."""
import ctypes
import struct

import pytest
import torch

from oracle.qtts_oracle import TalkerWeights, rope_tables

pytestmark = pytest.mark.gpu
P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _layer_table(layers):
    raw = b"".join(struct.pack("<Q", t.data_ptr()) for lw in layers for t in lw)
    return torch.frombuffer(bytearray(raw), dtype=torch.uint8).cuda()


def test_static_scratch_entry_matches_allocating_entry(pkg):
    lib = ctypes.CDLL(str(pkg._ext.library_path()))
    for name in ("launch_tts_decode_with_embedding", "launch_tts_decode_with_embedding_static"):
        fn = getattr(lib, name)
        fn.argtypes = [P] * 16 + [I] * 4 + [F, P]
        fn.restype = I
    cfg = pkg.SyntheticConfig(n_bb_layers=3, n_cp_layers=1, n_groups=1)
    sd = pkg.synthetic_state_dict(seed=99, cfg=cfg)
    tw = TalkerWeights.from_state_dict(sd, 3, 1)
    layers = [[t.cuda().contiguous() for t in lw] for lw in tw.bb_layers]
    table = _layer_table(layers)
    norm = tw.bb_norm.cuda()
    max_seq = 256
    cos, sin = (t.cuda() for t in rope_tables(max_seq, 128, 1e6))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator().manual_seed(4)
    # call 1 attends to 161 positions (chunked attention), call 2 to 9 (one pass): a smaller input
    for L in (161, 9):
        pos = L - 1
        k0 = torch.randn(3, 8, max_seq, 128, generator=g).to(torch.bfloat16)
        v0 = torch.randn(3, 8, max_seq, 128, generator=g).to(torch.bfloat16)
        x = torch.randn(1024, generator=g).to(torch.bfloat16).cuda()
        out = {}
        for name in ("launch_tts_decode_with_embedding", "launch_tts_decode_with_embedding_static"):
            kc, vc = k0.cuda(), v0.cuda()
            res = torch.full((1024,), float("nan"), device="cuda").to(torch.bfloat16)
            hid = torch.full((1024,), float("nan"), device="cuda")
            print(f"{name}: L={L}", flush=True)
            err = getattr(lib, name)(_ptr(x), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc),
                                     _ptr(res), None, None, None, None, None, None, None, _ptr(hid), 3, pos, pos + 1,
                                     max_seq, 128 ** -0.5, stream)
            assert err == 0, err
            torch.cuda.synchronize()
            out[name] = (hid.cpu(), res.cpu(), kc[:, :, pos].cpu(), vc[:, :, pos].cpu())
        a, b = out["launch_tts_decode_with_embedding"], out["launch_tts_decode_with_embedding_static"]
        for ta, tb in zip(a, b):
            assert torch.equal(ta, tb)
        assert torch.isfinite(a[0]).all()
    # the layer count the static workspace's tags cover is the limit
    assert lib.launch_tts_decode_with_embedding_static(
        _ptr(x), _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res), None, None, None,
        None, None, None, None, _ptr(hid), 441, 3, 4, max_seq, 128 ** -0.5, stream) != 0
    assert lib.launch_tts_decode_with_embedding_static(
        None, _ptr(table), _ptr(norm), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc), _ptr(res), None, None, None,
        None, None, None, None, _ptr(hid), 3, 3, 4, max_seq, 128 ** -0.5, stream) != 0
