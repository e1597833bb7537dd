"""Full Mamba causal LM on the MI355X kernels (mamba_metal/mamba_model.py:23-127).

Stack of (RMSNorm -> MambaBlock + residual) layers, final RMSNorm and a tied LM
head (logits = x @ embeddings.weight.T).  Attribute layout mirrors HF's
``state-spaces/mamba-*-hf`` with the ``backbone.`` prefix stripped:

    embeddings.weight, layers.{i}.norm.weight, layers.{i}.mixer.<X>, norm_f.weight
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from mamba_metal_amd.mamba_block import NORM_PENDING, MambaBlock
from mamba_metal_amd.linear import decode_head_argmax, decode_linear, decode_linear_ok
from mamba_metal_amd.norm import add_rmsnorm
from mamba_metal_amd.sample import argmax_rows


@dataclass
class MambaConfig:
    d_model: int = 768
    n_layer: int = 24
    vocab_size: int = 50280
    d_state: int = 16
    d_conv: int = 4
    expand: int = 2
    dt_rank: int | None = None  # auto = ceil(d_model / 16) if None
    rms_norm_eps: float = 1e-5


class MambaResidualBlock(nn.Module):
    """Pre-norm + residual wrapper around a MambaBlock (mamba_model.py:35-58)."""

    def __init__(self, cfg: MambaConfig, device=None, dtype=None):
        super().__init__()
        self.norm = nn.RMSNorm(cfg.d_model, eps=cfg.rms_norm_eps, device=device, dtype=dtype)
        self.mixer = MambaBlock(d_model=cfg.d_model, d_state=cfg.d_state, d_conv=cfg.d_conv,
                                expand=cfg.expand, dt_rank=cfg.dt_rank, device=device, dtype=dtype)

    def forward(self, x):
        return x + self.mixer(self.norm(x))

    def prefill(self, x):
        y, conv_state, ssm_state = self.mixer.prefill(self.norm(x))
        return x + y, conv_state, ssm_state

    def step(self, x_token, conv_state, ssm_state, inplace: bool = False):
        """Functional by default, as the reference's step: the given states are left
        untouched and fresh ones returned; ``inplace=True`` updates them in place."""
        y, new_conv, new_ssm = self.mixer.step(self.norm(x_token), conv_state, ssm_state,
                                               inplace=inplace)
        return x_token + y, new_conv, new_ssm


class MambaModel(nn.Module):
    """Stack of MambaResidualBlocks with a tied LM head (mamba_model.py:61-127)."""

    def __init__(self, cfg: MambaConfig, device=None, dtype=None):
        super().__init__()
        self.cfg = cfg
        self.embeddings = nn.Embedding(cfg.vocab_size, cfg.d_model, device=device, dtype=dtype)
        self.layers = nn.ModuleList(
            [MambaResidualBlock(cfg, device=device, dtype=dtype) for _ in range(cfg.n_layer)])
        self.norm_f = nn.RMSNorm(cfg.d_model, eps=cfg.rms_norm_eps, device=device, dtype=dtype)

    @property
    def d_inner(self) -> int:
        return self.cfg.expand * self.cfg.d_model

    def _head(self, h):
        """Tied LM head on normalised rows: logits = h @ E^T (mamba_model.py:78).
        Decode-sized row blocks run on the weight-streaming GEMM."""
        E = self.embeddings.weight
        if h.dim() == 2 and decode_linear_ok(h, E):
            return decode_linear(h, E)
        return F.linear(h, E)

    def _run(self, input_ids, mix, defer_norm: bool = False, resid=None):
        """Layer chain with the residual add fused into the next layer's RMSNorm:
        resid += y_prev; h = RMSNorm(resid) (one kernel per layer boundary).
        ``mix(mixer, h, resid, norm, next_norm)`` returns either ``(y, None)`` -- the
        mixer output, added here -- or ``(None, h_next)`` when it has already added its
        output into ``resid`` and applied ``next_norm`` itself.  With ``defer_norm`` the
        first norm is not applied here (h = NORM_PENDING: the mixer applies ``norm`` to
        ``resid`` itself, in its first projection), and a mixer may return
        ``(None, NORM_PENDING)`` to leave ``next_norm`` to the next one.  ``resid``, when
        given, already holds the embedding rows of input_ids and becomes the residual
        stream (updated in place)."""
        if resid is None:
            resid = self.embeddings(input_ids)
        norms = [layer.norm for layer in self.layers] + [self.norm_f]
        h = NORM_PENDING if defer_norm else add_rmsnorm(resid, None, norms[0].weight,
                                                        norms[0].eps)
        for i, layer in enumerate(self.layers):
            y, h_next = mix(layer.mixer, h, resid, norms[i], norms[i + 1])
            h = h_next if h_next is not None else add_rmsnorm(resid, y, norms[i + 1].weight,
                                                              norms[i + 1].eps)
        if h is NORM_PENDING:
            h = add_rmsnorm(resid, None, norms[-1].weight, norms[-1].eps)
        return h

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """input_ids (B, L) -> logits (B, L, vocab_size)."""
        return self._head(self._run(input_ids, lambda m, h, resid, nrm, nxt: (m(h), None)))

    def init_state(self, batch_size: int = 1):
        """Zero conv and SSM states (float32, as mamba_model.py:80-91)."""
        dev = self.embeddings.weight.device
        convs = [torch.zeros((batch_size, self.d_inner, self.cfg.d_conv), dtype=torch.float32,
                             device=dev) for _ in self.layers]
        ssms = [torch.zeros((batch_size, self.d_inner, self.cfg.d_state), dtype=torch.float32,
                            device=dev) for _ in self.layers]
        return convs, ssms

    def prefill(self, input_ids: torch.Tensor, last_only: bool = False):
        """Process a (B, L) prompt in parallel (mamba_model.py:93-110).

        Returns (logits (B, L, vocab) -- (B, 1, vocab) with last_only=True --,
        conv_states, ssm_states)."""
        convs, ssms = [], []

        def mix(m, h, resid, nrm, nxt):
            y, cs, ss = m.prefill(h)
            convs.append(cs)
            ssms.append(ss)
            return y, None

        h = self._run(input_ids, mix)
        if last_only:
            # (B, d_model) rows: decode-sized row blocks take the weight-streaming head
            return self._head(h[:, -1, :])[:, None, :], convs, ssms
        return self._head(h), convs, ssms

    def step_greedy(self, input_ids: torch.Tensor, conv_states, ssm_states, ids_out: torch.Tensor,
                    hidden: torch.Tensor | None = None):
        """``step(input_ids, conv_states, ssm_states, inplace=True)`` followed by the greedy
        choice ids_out = argmax(logits[:, 0, :]) (generate.py:91-93), the head and the argmax
        in one call (mm_decode_head_argmax) where the decode GEMM takes the head.  The
        states are updated in place; ids_out may be input_ids (the embedding reads it
        first).  ``hidden`` (B, d_model), when given, holds the embedding rows of input_ids
        on entry (the step uses it as its residual stream instead of looking them up) and
        the embedding rows of ids_out on return, written by the argmax's kernel
        (mm_decode_head_argmax_embed): consecutive steps then run no embedding lookup.
        Returns the logits (B, 1, vocab)."""
        it = iter(zip(conv_states, ssm_states))

        def mix(m, h, resid, nrm, nxt):
            cs, ss = next(it)
            if h is NORM_PENDING:
                return m.step_2d(resid, cs, ss, resid=resid, next_norm=nxt, x_norm=nrm,
                                 defer_norm=True)
            return m.step_2d(h, cs, ss, resid=resid, next_norm=nxt, defer_norm=True)

        h = self._run(input_ids.reshape(-1), mix, defer_norm=True, resid=hidden)
        E = self.embeddings.weight
        if h.dim() == 2 and decode_linear_ok(h, E):
            return decode_head_argmax(h, E, ids_out, embed_out=hidden)[:, None, :]
        logits = self._head(h)
        argmax_rows(logits if logits.stride(-1) == 1 else logits.contiguous(), out=ids_out)
        if hidden is not None:
            hidden.copy_(self.embeddings(ids_out))
        return logits[:, None, :]

    def step(self, input_ids: torch.Tensor, conv_states, ssm_states, inplace: bool = False):
        """One new token per sequence (B, 1) -> (logits (B, 1, vocab), states).

        Functional by default, as the reference's step (mamba_model.py:112-127): the
        given state lists are left untouched and new state tensors are returned.  With
        ``inplace=True`` the decode kernels update the given tensors in place (no copy;
        what generate_fast and GraphDecoder use) and the same tensors are returned."""
        if not inplace:
            conv_states = [t.clone() for t in conv_states]
            ssm_states = [t.clone() for t in ssm_states]
        it = iter(zip(conv_states, ssm_states))

        def mix(m, h, resid, nrm, nxt):
            cs, ss = next(it)
            if h is NORM_PENDING:
                return m.step_2d(resid, cs, ss, resid=resid, next_norm=nxt, x_norm=nrm,
                                 defer_norm=True)
            return m.step_2d(h, cs, ss, resid=resid, next_norm=nxt, defer_norm=True)

        h = self._run(input_ids.reshape(-1), mix, defer_norm=True)
        return self._head(h)[:, None, :], list(conv_states), list(ssm_states)


@torch.no_grad()
def init_weights_(model: MambaModel, seed: int = 0, std: float = 0.02,
                  dt_min: float = 1e-3, dt_max: float = 1e-1) -> MambaModel:
    """Random init used for the synthetic benchmark models.

    Linear / conv / embedding weights ~ N(0, std); A_log = log(1..d_state);
    dt_proj.bias = softplus^-1(U(dt_min, dt_max)) = log(expm1(dt)); D = 1;
    norm weights = 1; conv bias = 0.  Drawn on the model's device from one
    seeded generator, in a fixed parameter order, so a run is reproducible."""
    dev = model.embeddings.weight.device
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("A_log"):
            n = p.shape[-1]
            p.copy_(torch.log(torch.arange(1, n + 1, dtype=torch.float32, device=dev)).expand_as(p))
        elif name.endswith("mixer.D") or name.endswith("norm.weight") or name == "norm_f.weight":
            p.fill_(1.0)
        elif name.endswith("dt_proj.bias"):
            dt = torch.empty(p.shape, dtype=torch.float32, device=dev)
            dt.uniform_(dt_min, dt_max, generator=g)
            p.copy_(torch.log(torch.expm1(dt)).to(p.dtype))
        elif name.endswith("conv1d.bias"):
            p.zero_()
        else:
            w = torch.empty(p.shape, dtype=torch.float32, device=dev)
            w.normal_(0.0, std, generator=g)
            p.copy_(w.to(p.dtype))
    return model
