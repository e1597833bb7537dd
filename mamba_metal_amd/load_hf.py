"""Load ``state-spaces/mamba-*-hf`` checkpoints into a MambaModel (mamba_metal/load_hf.py).

Same entry point and config mapping as the reference:
  - ``_config_from_hf`` prefers the HF transformers fields (hidden_size,
    intermediate_size, num_hidden_layers, state_size, conv_kernel, time_step_rank,
    layer_norm_epsilon) and falls back to the legacy state-spaces aliases; a stale
    ``d_model`` (mamba-790m-hf) loses to ``hidden_size`` (load_hf.py:22-39);
  - every key loses its ``backbone.`` prefix (load_hf.py:42-43);
  - conv1d.weight keeps the torch/HF (d_inner, 1, d_conv) order -- the model is
    torch, so the reference's transpose to MLX order (load_hf.py:46-50) is not needed.

Differences, both forced by the environment: there is no network, so ``repo_id``
must be a local directory or a repo already in the local HF cache
(``snapshot_download(..., local_files_only=True)``); and ``dtype``/``device``
arguments place the weights (A_log and D stay float32).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from mamba_metal_amd.mamba_model import MambaConfig, MambaModel

_FP32_KEYS = ("mixer.A_log", "mixer.D")


def _config_from_hf(local_dir: Path) -> MambaConfig:
    cfg = json.loads((Path(local_dir) / "config.json").read_text())
    d_model = cfg.get("hidden_size") or cfg["d_model"]
    d_inner = cfg.get("intermediate_size") or cfg.get("d_inner")
    expand = d_inner // d_model if d_inner else cfg.get("expand", 2)
    return MambaConfig(
        d_model=d_model,
        n_layer=cfg.get("num_hidden_layers") or cfg["n_layer"],
        vocab_size=cfg["vocab_size"],
        d_state=cfg.get("state_size") or cfg.get("d_state", 16),
        d_conv=cfg.get("conv_kernel") or cfg.get("d_conv", 4),
        expand=expand,
        dt_rank=cfg.get("time_step_rank") or cfg.get("dt_rank"),
        rms_norm_eps=cfg.get("layer_norm_epsilon", 1e-5),
    )


def _convert_key(key: str) -> str:
    return key.removeprefix("backbone.")


def _resolve(repo_id: str | Path) -> Path:
    p = Path(repo_id)
    if p.is_dir():
        return p
    try:
        from huggingface_hub import snapshot_download

        return Path(snapshot_download(
            repo_id=str(repo_id),
            allow_patterns=["*.json", "*.safetensors", "tokenizer*", "special_tokens*"],
            local_files_only=True))
    except Exception as e:  # not cached and no network
        raise FileNotFoundError(
            f"{repo_id!r} is neither a local directory nor a repo in the local HF cache "
            "(downloads are not available)") from e


def load_mamba_hf(repo_id: str | Path = "state-spaces/mamba-130m-hf", *,
                  device="cuda", dtype: torch.dtype | None = None):
    """Returns (MambaModel, MambaConfig) loaded from a local HF-format directory."""
    from safetensors import safe_open

    local_dir = _resolve(repo_id)
    cfg = _config_from_hf(local_dir)
    files = sorted(local_dir.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors under {local_dir}")
    weights = {}
    for st in files:
        with safe_open(str(st), framework="pt") as f:
            for hf_key in f.keys():
                weights[_convert_key(hf_key)] = f.get_tensor(hf_key)
    # Tied head: a stored lm_head.weight duplicates embeddings.weight.
    head = weights.pop("lm_head.weight", None)
    if head is not None and "embeddings.weight" not in weights:
        weights["embeddings.weight"] = head
    if dtype is None:
        dtype = weights["embeddings.weight"].dtype
    with torch.device("meta"):
        model = MambaModel(cfg, dtype=dtype)
    model = model.to_empty(device=device)
    for k, v in list(weights.items()):
        weights[k] = v.float() if k.endswith(_FP32_KEYS) else v.to(dtype)
    missing, unexpected = model.load_state_dict(weights, strict=False)
    if missing or unexpected:
        raise ValueError(f"checkpoint mismatch: missing={sorted(missing)} "
                         f"unexpected={sorted(unexpected)}")
    model.eval()
    return model, cfg
