"""The C-ABI library and the torch extension load, and export every entry point the public
header declares (CPU only: nothing is launched)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qwentts_amd.h"
LIB = ROOT / "qwentts-turbo_amd" / "lib" / "libqwentts_amd.so"


def declared_functions():
    text = HEADER.read_text()
    body = text[text.index('extern "C" {'):]
    return re.findall(r"^(?:hipError_t|size_t|void|int)\s+(\w+)\s*\(", body, flags=re.M)


def test_header_declares_reference_launchers():
    names = declared_functions()
    for ref in ("launch_tts_decode", "launch_tts_decode_with_embedding", "launch_cp_decode_with_embedding"):
        assert ref in names
    assert len(names) == len(set(names)) >= 9


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.skip("libqwentts_amd.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_workspace_bytes_is_callable_without_a_gpu():
    """qtts_workspace_bytes is a pure size query (no HIP call)."""
    if not LIB.exists():
        pytest.skip("libqwentts_amd.so is not built")
    lib = ctypes.CDLL(str(LIB))
    lib.qtts_workspace_bytes.restype = ctypes.c_size_t
    n = lib.qtts_workspace_bytes()
    assert 0 < n < 8 << 20 and n % 256 == 0


def test_prefill_workspace_bytes_without_a_gpu():
    """qtts_prefill_workspace_bytes is a host-only size query: 0 for an empty prompt or an
    out-of-range vocabulary; otherwise at least the bf16 activations of every prompt row
    (hidden, normed, q|k|v, attention, SwiGLU: 1024 + 1024 + 4096 + 2048 + 3072 per row) plus the
    head logits. Not monotone in the prompt length (the split-K factor, and so the partials
    buffer, changes with the row count)."""
    lib = ctypes.CDLL(str(LIB))
    f = lib.qtts_prefill_workspace_bytes
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int, ctypes.c_int]
    assert f(0, 0) == 0 and f(-1, 0) == 0 and f(128, -1) == 0 and f(128, 3073) == 0
    for n in (1, 7, 40, 127, 128, 129, 255, 256, 333, 511, 512, 1100, 2048, 4096):
        lower = n * (1024 + 1024 + 4096 + 2048 + 3072) * 2 + 3072 * 2
        assert f(n, 0) >= lower, n
        assert f(n, 3072) >= f(n, 0), n


def test_torch_extension_exposes_reference_classes(pkg):
    ext = pkg._ext.load()
    for cls, methods in {
        "MegakernelTTSDecoder": ("decode_step", "decode_step_with_argmax", "decode_step_with_embedding", "reset",
                                 "position", "set_position", "get_hidden_states", "get_k_cache", "get_v_cache",
                                 "set_kv_cache"),
        "MegakernelCodePredictorDecoder": ("decode_step_with_embedding", "reset", "position", "set_position",
                                           "get_hidden_states", "set_kv_cache"),
    }.items():
        c = getattr(ext, cls)
        for m in methods:
            assert hasattr(c, m), (cls, m)


def test_workspace_hooks_validate_arguments_without_a_gpu():
    """The host-only workspace hooks reject bad arguments; qtts_shutdown with nothing on any
    device makes no HIP call and succeeds."""
    lib = ctypes.CDLL(str(LIB))
    P = ctypes.c_void_p
    lib.qtts_workspace_release.argtypes = [P, ctypes.c_int]
    lib.qtts_debug_set_sequence.argtypes = [P, ctypes.c_uint]
    assert lib.qtts_workspace_release(None, 1) != 0
    assert lib.qtts_workspace_release(P(4096), 0) != 0
    assert lib.qtts_workspace_release(P(4096), 2) == 0
    assert lib.qtts_debug_set_sequence(None, 5) != 0
    assert lib.qtts_debug_set_sequence(P(4096), 0) != 0 and lib.qtts_debug_set_sequence(P(4096), 1 << 20) != 0
    assert lib.qtts_debug_set_sequence(P(4096), 5) == 0
    assert lib.qtts_workspace_release(P(4096), 1) == 0
    # the error-word hook rejects a null workspace and a zero code before any HIP call; the
    # entry-cap hook is host-only (0 restores the default)
    lib.qtts_debug_set_error.argtypes = [P, ctypes.c_uint, P]
    assert lib.qtts_debug_set_error(None, 1, None) != 0 and lib.qtts_debug_set_error(P(4096), 0, None) != 0
    lib.qtts_debug_entry_spin_cap.argtypes = [ctypes.c_uint]
    assert lib.qtts_debug_entry_spin_cap(64) == 0 and lib.qtts_debug_entry_spin_cap(0) == 0
    assert lib.qtts_shutdown() == 0
