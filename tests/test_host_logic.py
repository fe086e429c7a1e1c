"""Host-side logic of the package that runs before any GPU call (CPU only): backend and
argument validation of the generator, weight-layout helpers, seeded synthetic weights,
RoPE tables, and the loud failure when the HIP extension is missing."""
import importlib

import pytest
import torch


def test_generator_rejects_pytorch_backend(pkg):
    for kw in ({"backend": "pytorch"}, {"cp_backend": "pytorch"}):
        with pytest.raises(ValueError, match="megakernel"):
            pkg.NativeTTSGenerator(model={}, eos_token_id=1, **kw)


def test_generator_requires_model_and_eos(pkg):
    with pytest.raises(ValueError, match="model"):
        pkg.NativeTTSGenerator()
    with pytest.raises(ValueError, match="eos_token_id"):
        pkg.NativeTTSGenerator(model={})


def test_generator_reads_eos_from_model_config(pkg):
    class Cfg:
        class talker_config:
            codec_eos_token_id = 2150

    class Model(dict):
        config = Cfg

    # the eos lookup happens before any device work; construction then fails for lack of
    # weights (KeyError) rather than for the eos id
    with pytest.raises(KeyError):
        pkg.NativeTTSGenerator(model=Model())


def test_batched_decoder_rejects_empty_batch(pkg):
    with pytest.raises(ValueError, match="n_streams"):
        pkg.BatchedTTSDecoder({}, 0)


def test_load_local_refuses_missing_path(pkg, tmp_path):
    with pytest.raises(FileNotFoundError):
        pkg.load_model(str(tmp_path / "nothing"))


def test_synthetic_weights_layout_and_determinism(pkg):
    cfg = pkg.SyntheticConfig(n_bb_layers=1, n_cp_layers=1, n_groups=2)
    a = pkg.synthetic_state_dict(seed=3, cfg=cfg)
    b = pkg.synthetic_state_dict(seed=3, cfg=cfg)
    assert a.keys() == b.keys() and all(torch.equal(a[k], b[k]) for k in a)
    w = importlib.import_module("qwentts_turbo_amd.weights")
    assert w.count_layers(a, w.BB_PREFIX) == 1 and w.count_layers(a, w.CP_PREFIX) == 1
    assert w.count_groups(a) == 2
    assert a["talker.model.layers.0.self_attn.q_proj.weight"].shape == (2048, 1024)
    assert a["talker.model.layers.0.mlp.down_proj.weight"].shape == (1024, 3072)
    assert a["talker.code_predictor.lm_head.1.weight"].shape == (2048, 1024)
    assert all(t.dtype == torch.bfloat16 for t in a.values())
    # norm gains centred on norm_mean, matrices on 0
    assert abs(float(a["talker.model.norm.weight"].float().mean()) - 1.0) < 0.01
    assert abs(float(a["talker.codec_head.weight"].float().mean())) < 0.01
    lst = w.layer_list(a, w.BB_PREFIX, 1)
    assert len(lst) == 11 and lst[1].shape == (2048, 1024)


def test_package_rope_tables_match_oracle(pkg):
    from oracle.qtts_oracle import rope_tables as oracle_tables
    w = importlib.import_module("qwentts_turbo_amd.weights")
    c, s = w.rope_tables(256, device="cpu")
    oc, os_ = oracle_tables(256, 128, 1e6)
    assert torch.equal(c, oc) and torch.equal(s, os_)


def test_extension_loader_fails_loudly_when_not_built(pkg, monkeypatch, tmp_path):
    ext = importlib.import_module("qwentts_turbo_amd._ext")
    monkeypatch.setattr(ext, "_MOD", None)
    monkeypatch.setattr(ext, "_PKG", tmp_path)
    with pytest.raises(ImportError, match="not built"):
        ext.load()
