"""Config 3 (Mamba-2.8b shape, batch 64 decode, fp16) on the MI355X.

  * 2.8b width (d_model 2560, d_inner 5120, dt_rank 160, vocab 50280), batch 64,
    2 layers: 64-token prompts, then 4 teacher-forced decode steps against the float64
    CPU oracle -- the decode kernels at the configuration's real shapes (the fused
    in_proj + conv + x_proj at 64 x 10240 x 2560, the MFMA SSM step at 64 x 5120, the
    split-K out_proj with the residual + RMSNorm reduce, the LM head), and the prefill
    scan's channel-contiguous path at 64 x 5120.
  * the full 64-layer model at batch 64 through properties that hold at any size:
    finite logits, prefill(L) then step == prefill(L + 1) at position L
    (experiments/17-incremental/test_step.py:31-41), and the HIP-graph decode equal to
    the eager decode, token for token.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, check_greedy

pytestmark = pytest.mark.gpu

C3 = dict(d_model=2560, vocab_size=50280, dt_rank=160)


def make_model(dev, n_layer, seed):
    from mamba_metal_amd import MambaConfig, MambaModel, init_weights_

    cfg = MambaConfig(n_layer=n_layer, **C3)
    model = init_weights_(MambaModel(cfg, device=dev, dtype=torch.float16), seed=seed).eval()
    return model, cfg


def test_config3_width_two_layers_against_oracle(dev):
    from oracle.model_ref import RefConfig, RefModel

    from mamba_metal_amd.selective_scan import reset_scan_status, scan_status

    model, cfg = make_model(dev, 2, seed=41)
    ref = RefModel(RefConfig(cfg.d_model, cfg.n_layer, cfg.vocab_size, cfg.d_state, cfg.d_conv,
                             cfg.expand, cfg.dt_rank, cfg.rms_norm_eps),
                   {k: v.detach().float().cpu() for k, v in model.state_dict().items()})
    rng = np.random.default_rng(41)
    ids = rng.integers(0, cfg.vocab_size, (64, 64))
    teacher = rng.integers(0, cfg.vocab_size, (64, 4))
    reset_scan_status(dev)
    with torch.inference_mode():
        lg, convs, ssms = model.prefill(torch.as_tensor(ids, device=dev), last_only=True)
        gl = [lg[:, -1].float()]
        for s in range(3):
            lg, convs, ssms = model.step(torch.as_tensor(teacher[:, s:s + 1], device=dev), convs,
                                         ssms, inplace=True)
            gl.append(lg[:, 0].float())
    assert scan_status(dev) == 0
    _, ref_logits = ref.generate_fast_ids(ids, 4, teacher=teacher)
    got = np.stack([g.argmax(-1).cpu().numpy() for g in gl], 1)
    # the logits of 64 rows x 50280 tokens span about +-35 here: 3e-2 absolute is ~1e-3 of that
    check_greedy(got, gl, ref_logits, 4, "config-3 width, 2 layers, batch 64", tol=3e-2)


@pytest.fixture(scope="module")
def full_c3(dev):
    model, cfg = make_model(dev, 64, seed=43)
    return model, cfg


def test_config3_full_depth_prefill_step_invariant(dev, full_c3):
    from mamba_metal_amd.selective_scan import reset_scan_status, scan_status

    model, cfg = full_c3
    rng = np.random.default_rng(43)
    ids = torch.as_tensor(rng.integers(0, cfg.vocab_size, (64, 513)), device=dev)
    reset_scan_status(dev)
    with torch.inference_mode():
        full, _, _ = model.prefill(ids, last_only=True)
        _, convs, ssms = model.prefill(ids[:, :512], last_only=True)
        st, _, _ = model.step(ids[:, 512:], convs, ssms, inplace=True)
    assert scan_status(dev) == 0
    full, st = full[:, -1].float(), st[:, 0].float()
    assert torch.isfinite(full).all() and torch.isfinite(st).all()
    err = float((full - st).abs().max())
    scale = float(full.abs().max())
    agree = float((full.argmax(-1) == st.argmax(-1)).float().mean())
    print(f"[config3 64 layers] prefill(513) vs prefill(512)+step: max |d logit| {err:.3e}, "
          f"max |logit| {scale:.3f}, argmax agreement {agree:.3f}")
    assert err < 0.03 * scale
    assert agree >= 0.9


def test_config3_full_depth_graph_equals_eager(dev, full_c3):
    from mamba_metal_amd import generate_fast_ids

    model, cfg = full_c3
    rng = np.random.default_rng(44)
    ids = torch.as_tensor(rng.integers(0, cfg.vocab_size, (64, 128)), device=dev)
    eager = generate_fast_ids(model, ids, 8)
    graph = generate_fast_ids(model, ids, 8, use_graph=True)
    assert torch.equal(eager, graph)
