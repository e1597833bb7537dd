"""torch-CPU restatement of the reference Mamba model -- TEST INFRASTRUCTURE ONLY.

Restates, in float64 (or float32) on the CPU:
  MambaBlock.__call__ / prefill / step   mamba_metal/mamba_block.py:68-198
  MambaResidualBlock                      mamba_metal/mamba_model.py:35-58
  MambaModel.__call__ / prefill / step    mamba_metal/mamba_model.py:71-127
  generate (O(L^2) greedy) / generate_fast (prefill + O(1) step)
                                          mamba_metal/generate.py:16-110 (token-id form)

Weights come as a dict keyed by the HF parameter names with the ``backbone.``
prefix stripped (mamba_metal/load_hf.py:42-43), conv1d.weight in torch/HF order
(d_inner, 1, d_conv).  The scan uses the float64 sequential recurrence of
``numpy_ref.selective_scan``; prefill's softplus uses the kernel's cutoff form,
step's softplus MLX's logaddexp form (mamba_block.py:184), as the reference does.

Pinning: the building blocks are pinned in tests/test_oracle.py; the model
composition is pinned by the reference's own invariants -- prefill(L) then
step == prefill(L+1) (experiments/17-incremental/test_step.py:31-41), causality
(experiments/11-mamba-block/test_block.py:42-61) and the parameter-name set
(experiments/13-mamba-model/test_model.py:15-31).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import numpy_ref


class RefConfig:
    def __init__(self, d_model, n_layer, vocab_size, d_state=16, d_conv=4, expand=2,
                 dt_rank=None, rms_norm_eps=1e-5):
        self.d_model = d_model
        self.n_layer = n_layer
        self.vocab_size = vocab_size
        self.d_state = d_state
        self.d_conv = d_conv
        self.expand = expand
        self.d_inner = expand * d_model
        self.dt_rank = math.ceil(d_model / 16) if dt_rank is None else dt_rank
        self.rms_norm_eps = rms_norm_eps


def _t(x, dtype):
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu", dtype)
    return torch.as_tensor(np.asarray(x), dtype=dtype)


class RefModel:
    def __init__(self, cfg: RefConfig, weights: dict, dtype=torch.float64):
        self.cfg = cfg
        self.dtype = dtype
        self.w = {k: _t(v, dtype) for k, v in weights.items()}

    # -- helpers ------------------------------------------------------------
    def _rms(self, x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + self.cfg.rms_norm_eps) * w

    def _lw(self, i, name):
        return self.w[f"layers.{i}.{name}"]

    def _mixer_prefill(self, i, x):
        cfg = self.cfg
        Bsz, L, _ = x.shape
        xz = x @ self._lw(i, "mixer.in_proj.weight").T
        xpre, z = xz[..., : cfg.d_inner], xz[..., cfg.d_inner:]
        w = self._lw(i, "mixer.conv1d.weight")                  # (d_inner, 1, K)
        xc = F.conv1d(xpre.transpose(1, 2), w, self._lw(i, "mixer.conv1d.bias"),
                      padding=cfg.d_conv - 1, groups=cfg.d_inner)[..., :L]
        xc = F.silu(xc).transpose(1, 2)                          # (B, L, d_inner)
        xpad = torch.cat([xpre.new_zeros(Bsz, cfg.d_conv, cfg.d_inner), xpre], 1)
        conv_state = xpad[:, -cfg.d_conv:, :].transpose(1, 2).contiguous()
        xdbl = xc @ self._lw(i, "mixer.x_proj.weight").T
        r, n = cfg.dt_rank, cfg.d_state
        dt = xdbl[..., :r] @ self._lw(i, "mixer.dt_proj.weight").T + self._lw(i, "mixer.dt_proj.bias")
        Bm, Cm = xdbl[..., r:r + n], xdbl[..., r + n:]
        A = -torch.exp(self._lw(i, "mixer.A_log"))
        y, h = numpy_ref.selective_scan(
            xc.transpose(1, 2).numpy(), dt.transpose(1, 2).numpy(), A.numpy(),
            Bm.transpose(1, 2).numpy(), Cm.transpose(1, 2).numpy(),
            D=self._lw(i, "mixer.D").numpy(), z=z.transpose(1, 2).numpy(), delta_softplus=True)
        y = torch.as_tensor(y, dtype=self.dtype).transpose(1, 2)
        out = y @ self._lw(i, "mixer.out_proj.weight").T
        return out, conv_state, torch.as_tensor(h, dtype=self.dtype)

    def _mixer_step(self, i, x, conv_state, ssm_state):
        cfg = self.cfg
        xz = x @ self._lw(i, "mixer.in_proj.weight").T             # (B, 2*d_inner)
        xm, z = xz[:, : cfg.d_inner], xz[:, cfg.d_inner:]
        w = self._lw(i, "mixer.conv1d.weight")[:, 0, :]
        xc, new_conv = numpy_ref.decode_conv_step(conv_state.numpy(), xm.numpy(), w.numpy(),
                                                  self._lw(i, "mixer.conv1d.bias").numpy())
        xc = torch.as_tensor(xc, dtype=self.dtype)
        xdbl = xc @ self._lw(i, "mixer.x_proj.weight").T
        r, n = cfg.dt_rank, cfg.d_state
        dt = xdbl[:, :r] @ self._lw(i, "mixer.dt_proj.weight").T + self._lw(i, "mixer.dt_proj.bias")
        A = -torch.exp(self._lw(i, "mixer.A_log"))
        y, h = numpy_ref.decode_ssm_step(ssm_state.numpy(), xc.numpy(), dt.numpy(), A.numpy(),
                                         xdbl[:, r:r + n].numpy(), xdbl[:, r + n:].numpy(),
                                         D=self._lw(i, "mixer.D").numpy(), z=z.numpy())
        y = torch.as_tensor(y, dtype=self.dtype)
        out = y @ self._lw(i, "mixer.out_proj.weight").T
        return out, torch.as_tensor(new_conv, dtype=self.dtype), torch.as_tensor(h, dtype=self.dtype)

    # -- public API (mamba_model.py:71-127) ----------------------------------
    def prefill(self, input_ids, last_only=False):
        ids = torch.as_tensor(np.asarray(input_ids), dtype=torch.long)
        x = self.w["embeddings.weight"][ids]
        convs, ssms = [], []
        for i in range(self.cfg.n_layer):
            y, cs, ss = self._mixer_prefill(i, self._rms(x, self._lw(i, "norm.weight")))
            x = x + y
            convs.append(cs)
            ssms.append(ss)
        x = self._rms(x, self.w["norm_f.weight"])
        if last_only:
            x = x[:, -1:]
        return x @ self.w["embeddings.weight"].T, convs, ssms

    def forward(self, input_ids):
        return self.prefill(input_ids)[0]

    def step(self, ids, convs, ssms):
        ids = torch.as_tensor(np.asarray(ids), dtype=torch.long).reshape(-1)
        x = self.w["embeddings.weight"][ids]
        new_c, new_s = [], []
        for i in range(self.cfg.n_layer):
            y, cs, ss = self._mixer_step(i, self._rms(x, self._lw(i, "norm.weight")), convs[i], ssms[i])
            x = x + y
            new_c.append(cs)
            new_s.append(ss)
        x = self._rms(x, self.w["norm_f.weight"])
        return (x @ self.w["embeddings.weight"].T)[:, None, :], new_c, new_s

    def generate_fast_ids(self, input_ids, max_new_tokens, teacher=None):
        """Greedy prefill + step decode.  Returns (tokens (B, n), logits list).

        teacher: optional (B, n) token ids fed instead of the argmax (teacher
        forcing), so the per-step logits can be compared with another
        implementation without divergence cascades."""
        logits, convs, ssms = self.prefill(input_ids, last_only=True)
        nxt = logits[:, -1]
        toks, all_logits = [], []
        for s in range(max_new_tokens):
            all_logits.append(nxt.clone())
            tok = torch.argmax(nxt, -1)
            toks.append(tok)
            feed = tok if teacher is None else torch.as_tensor(np.asarray(teacher))[:, s]
            lg, convs, ssms = self.step(feed, convs, ssms)
            nxt = lg[:, 0]
        return torch.stack(toks, 1), all_logits
