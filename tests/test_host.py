"""Host-side logic that needs no GPU: model structure, HF config mapping, op API
argument checks (the reference's asserts), loader, random init."""

from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch

from mamba_metal_amd import MambaConfig, MambaModel, init_weights_, selective_scan
from mamba_metal_amd.load_hf import _config_from_hf, _convert_key

# experiments/13-mamba-model/test_model.py:15-31
HF_EXPECTED_LAYER_NAMES = {
    "norm.weight", "mixer.A_log", "mixer.D", "mixer.conv1d.bias", "mixer.conv1d.weight",
    "mixer.dt_proj.bias", "mixer.dt_proj.weight", "mixer.in_proj.weight", "mixer.out_proj.weight",
    "mixer.x_proj.weight",
}
HF_EXPECTED_TOP_NAMES = {"embeddings.weight", "norm_f.weight"}


def test_parameter_names_match_hf():
    model = MambaModel(MambaConfig(d_model=64, n_layer=1, vocab_size=128))
    names = {n for n, _ in model.named_parameters()}
    layer = {n.removeprefix("layers.0.") for n in names if n.startswith("layers.0.")}
    assert layer == HF_EXPECTED_LAYER_NAMES
    assert {n for n in names if "layers." not in n} == HF_EXPECTED_TOP_NAMES


def test_parameter_shapes_and_130m_count():
    cfg = MambaConfig(d_model=768, n_layer=24, vocab_size=50280, dt_rank=48)
    with torch.device("meta"):
        model = MambaModel(cfg)
    sd = dict(model.named_parameters())
    assert sd["layers.0.mixer.conv1d.weight"].shape == (1536, 1, 4)      # HF/torch order
    assert sd["layers.0.mixer.in_proj.weight"].shape == (3072, 768)
    assert sd["layers.0.mixer.x_proj.weight"].shape == (48 + 32, 1536)
    assert sd["layers.0.mixer.dt_proj.weight"].shape == (1536, 48)
    assert sd["layers.0.mixer.A_log"].shape == (1536, 16)
    total = sum(p.numel() for p in model.parameters())
    assert 125e6 < total < 135e6, total                                  # "~130M"


def test_dt_rank_auto():
    assert MambaModel(MambaConfig(d_model=100, n_layer=1, vocab_size=8)).layers[0].mixer.dt_rank == 7


def test_config_from_hf(tmp_path):
    # transformers-style fields; a stale d_model must lose to hidden_size (mamba-790m-hf)
    (tmp_path / "config.json").write_text(json.dumps({
        "hidden_size": 1536, "d_model": 1024, "intermediate_size": 3072, "num_hidden_layers": 48,
        "vocab_size": 50280, "state_size": 16, "conv_kernel": 4, "time_step_rank": 96,
        "layer_norm_epsilon": 1e-5}))
    c = _config_from_hf(tmp_path)
    assert (c.d_model, c.n_layer, c.expand, c.dt_rank, c.d_state, c.d_conv) == (1536, 48, 2, 96, 16, 4)
    # legacy state-spaces aliases
    (tmp_path / "config.json").write_text(json.dumps({
        "d_model": 768, "n_layer": 24, "vocab_size": 50277}))
    c = _config_from_hf(tmp_path)
    assert (c.d_model, c.n_layer, c.expand, c.d_state, c.d_conv, c.dt_rank) == (768, 24, 2, 16, 4, None)
    assert _convert_key("backbone.layers.3.mixer.D") == "layers.3.mixer.D"
    assert _convert_key("lm_head.weight") == "lm_head.weight"


def test_load_mamba_hf_cpu(tmp_path):
    from safetensors.torch import save_file

    from mamba_metal_amd import load_mamba_hf

    cfg = MambaConfig(d_model=32, n_layer=2, vocab_size=64)
    model = init_weights_(MambaModel(cfg), seed=1)
    sd = {"backbone." + k: v.detach().clone() for k, v in model.state_dict().items()}
    sd["lm_head.weight"] = sd["backbone.embeddings.weight"].clone()
    save_file(sd, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"d_model": 32, "n_layer": 2, "vocab_size": 64}))
    m2, _ = load_mamba_hf(tmp_path, device="cpu", dtype=torch.float16)
    for k, v in model.state_dict().items():
        v2 = m2.state_dict()[k]
        if k.endswith(("A_log", "mixer.D")):
            assert v2.dtype == torch.float32 and torch.equal(v2, v)
        else:
            assert v2.dtype == torch.float16 and torch.equal(v2, v.half())
    with pytest.raises(FileNotFoundError):
        load_mamba_hf(tmp_path / "nope", device="cpu")


def test_init_weights():
    model = init_weights_(MambaModel(MambaConfig(d_model=64, n_layer=2, vocab_size=100)), seed=3)
    mix = model.layers[1].mixer
    assert torch.allclose(mix.A_log, torch.log(torch.arange(1, 17.0)).expand(128, 16))
    dt = torch.nn.functional.softplus(mix.dt_proj.bias.float())
    assert dt.min() >= 1e-3 - 1e-6 and dt.max() <= 1e-1 + 1e-6
    assert torch.all(mix.D == 1) and torch.all(model.norm_f.weight == 1)
    assert abs(float(mix.in_proj.weight.std()) - 0.02) < 2e-3
    again = init_weights_(MambaModel(MambaConfig(d_model=64, n_layer=2, vocab_size=100)), seed=3)
    assert all(torch.equal(a, b) for a, b in zip(model.parameters(), again.parameters()))


def test_selective_scan_shape_asserts_before_device_checks():
    """The reference's asserts (selective_scan.py:46-50) fire first, AssertionError."""
    u = torch.zeros((1, 4, 8))
    A = torch.zeros((4, 16))
    B = torch.zeros((1, 16, 8))
    with pytest.raises(AssertionError):
        selective_scan(u, torch.zeros((1, 4, 7)), A, B, B)
    with pytest.raises(AssertionError):
        selective_scan(u, u, A, B, torch.zeros((1, 16, 9)))
    with pytest.raises(AssertionError):
        selective_scan(u, u, torch.zeros((4, 65)), torch.zeros((1, 65, 8)), torch.zeros((1, 65, 8)))
    # valid shapes on CPU tensors: no fallback, a clear error
    with pytest.raises(ValueError, match="no CPU fallback"):
        selective_scan(u, u, A, B, B)


def test_load_kernel_names():
    from mamba_metal_amd import load_kernel
    from mamba_metal_amd._loader import read_kernel_source

    assert read_kernel_source("selective_scan_chunked") == "mm_selective_scan_fwd"
    k = load_kernel("selective_scan_chunked",
                    ["u", "delta", "A", "B", "C", "D", "z", "batch", "dim", "dstate", "seqlen",
                     "apply_softplus", "use_D", "use_z"], ["y", "ssm_state_out"])
    assert k.name == "selective_scan_chunked"
    with pytest.raises(FileNotFoundError):
        load_kernel("conv1d_tg", [], [])


def test_bench_byte_formulas():
    import bench

    assert bench.scan_bytes(4, 5120, 16, 32768) == 5_378_756_608       # config 4
    assert bench.scan_bytes(8, 1536, 16, 8192) == 810_391_552          # config 2
    assert bench.scan_bytes(1, 16, 16, 4096, xs=4, bcs=4) == 1_574_976  # config 0
    assert bench.decode_roofline_bytes(2560, 64, 50280, 16, 4, 160, 64) == pytest.approx(
        8_556_590_080, rel=2e-3)


def test_packed_weight_cache(monkeypatch):
    """The packed-weight cache: one pack per weight, a repack after an in-place
    update, and the entry dropped with the weight."""
    import gc

    import torch

    from mamba_metal_amd import linear

    made = []
    monkeypatch.setattr(linear, "_make_packed", lambda w: made.append(1) or w.clone())
    w = torch.ones(4, 64)
    p1 = linear.packed_weight(w)
    assert linear.packed_weight(w) is p1 and len(made) == 1
    w.mul_(2)
    p2 = linear.packed_weight(w)
    assert p2 is not p1 and len(made) == 2 and float(p2[0, 0]) == 2.0
    n = len(linear._PACKED)
    del w
    gc.collect()
    assert len(linear._PACKED) == n - 1
