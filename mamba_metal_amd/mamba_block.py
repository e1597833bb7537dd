"""One Mamba block on the MI355X kernels (mamba_metal/mamba_block.py:27-198).

Layout (single layer, inference only), as in the reference:

    x (B, L, d_model) -> in_proj -> [x_main, z] -> causal depthwise conv1d -> SiLU
      -> x_proj -> (dt_pre, B, C) -> dt_proj -> selective scan(A=-exp(A_log), D, z,
      delta_softplus) -> out_proj

Parameter names and shapes follow the HF checkpoints (and the reference's
attribute names): in_proj.weight, conv1d.weight (d_inner, 1, d_conv) -- torch/HF
order, so no transpose is needed (the reference transposes to MLX order,
load_hf.py:46-50) --, conv1d.bias, x_proj.weight, dt_proj.weight/bias, A_log, D,
out_proj.weight.  A_log and D stay float32 whatever the model dtype.

Where the reference transposes activations to (B, dim, L) contiguous copies
before the scan (mamba_block.py:90-100), this block hands the kernel strided
(B, L, dim) views: the scan reads channel-contiguous tiles directly.

The prefill's in/x/out projections run on torch (hipBLASLt) and its dt projection
(K = dt_rank, with bias) on the library's short-K matrix-core GEMM (mm_prefill_linear);
the conv, the scan and every decode-step op -- including the projections at decode
batch <= 64, on the weight-streaming GEMM -- are libmamba_mi355x kernels.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from mamba_metal_amd.conv1d import causal_conv1d, conv_step
from mamba_metal_amd.decode import ssm_step_dtproj
from mamba_metal_amd.linear import (NORM_IN_MAX_M, decode_in_proj_conv, decode_in_proj_conv_xproj,
                                    decode_linear, decode_linear_ok, decode_linear_resid_,
                                    decode_linear_resid_norm_, in_proj_conv_ok, norm_in_ok,
                                    prefill_linear, prefill_linear_ok, split_k, xproj_weight_ok)
from mamba_metal_amd.norm import add_rmsnorm
from mamba_metal_amd.selective_scan import selective_scan_into

# step_2d's marker for "resid updated, next norm not applied yet" (see step_2d).
NORM_PENDING = object()



class MambaBlock(nn.Module):
    def __init__(self, d_model: int, d_state: int = 16, d_conv: int = 4, expand: int = 2,
                 dt_rank: int | None = None, device=None, dtype=None):
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        self.d_model = d_model
        self.d_state = d_state
        self.d_conv = d_conv
        self.d_inner = expand * d_model
        self.dt_rank = math.ceil(d_model / 16) if dt_rank is None else dt_rank

        self.in_proj = nn.Linear(d_model, self.d_inner * 2, bias=False, **fk)
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, kernel_size=d_conv,
                                groups=self.d_inner, padding=d_conv - 1, bias=True, **fk)
        self.x_proj = nn.Linear(self.d_inner, self.dt_rank + 2 * d_state, bias=False, **fk)
        self.dt_proj = nn.Linear(self.dt_rank, self.d_inner, bias=True, **fk)
        # A = -exp(A_log); init A[d, n] = n + 1 (mamba_block.py:57-63).
        A_init = torch.arange(1, d_state + 1, dtype=torch.float32, device=device)
        self.A_log = nn.Parameter(torch.log(A_init).expand(self.d_inner, d_state).contiguous(),
                                  requires_grad=False)
        self.D = nn.Parameter(torch.ones(self.d_inner, dtype=torch.float32, device=device),
                              requires_grad=False)
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False, **fk)

    # ------------------------------------------------------------------ helpers
    def _A(self) -> torch.Tensor:
        """A = -exp(A_log) (float32), cached until A_log changes (decode would
        otherwise spend two kernel launches per layer per token recomputing it)."""
        key = (self.A_log.data_ptr(), self.A_log._version, self.A_log.device)
        cache = getattr(self, "_A_cache", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                A = -torch.exp(self.A_log.detach().float())
            self._A_cache = (key, A)
            return A
        return cache[1]

    def _split_xdbl(self, x_dbl):
        r, n = self.dt_rank, self.d_state
        return x_dbl[..., :r], x_dbl[..., r:r + n], x_dbl[..., r + n:]

    def _mix(self, x, conv_state=None, ssm_state=None):
        """Shared body of __call__ / prefill.  x: (B, L, d_model)."""
        Bsz, L, _ = x.shape
        di = self.d_inner
        xz = self.in_proj(x)                                   # (B, L, 2*d_inner)
        x_pre, z = xz[..., :di], xz[..., di:]                  # strided views
        x_main = causal_conv1d(x_pre, self.conv1d.weight, self.conv1d.bias, apply_silu=True,
                               conv_state_out=conv_state)      # (B, L, d_inner)
        x_dbl = self.x_proj(x_main)                            # (B, L, dt_rank + 2N)
        dt_pre, Bm, Cm = self._split_xdbl(x_dbl)
        # dt_proj as one 2-D GEMM on the strided dt slice (leading dims merge into a view
        # with row stride dt_rank + 2N), bias in the GEMM epilogue: F.linear on the
        # non-contiguous 3-D slice added the bias in a separate pass over (B, L, d_inner).
        dt_2d = dt_pre.reshape(Bsz * L, -1)
        if prefill_linear_ok(dt_2d, self.dt_proj.weight, self.dt_proj.bias):
            dt = prefill_linear(dt_2d, self.dt_proj.weight, self.dt_proj.bias).view(Bsz, L, di)
        else:
            W_dt = self.dt_proj.weight.t()
            dt = (torch.addmm(self.dt_proj.bias, dt_2d, W_dt) if self.dt_proj.bias is not None
                  else dt_2d @ W_dt).view(Bsz, L, di)
        y = torch.empty_like(x_main)
        selective_scan_into(x_main.transpose(1, 2), dt.transpose(1, 2), self._A(),
                            Bm.transpose(1, 2), Cm.transpose(1, 2), y.transpose(1, 2),
                            D=self.D, z=z.transpose(1, 2), delta_softplus=True,
                            state_out=ssm_state)
        return self.out_proj(y)

    # --------------------------------------------------------------- public API
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Full forward without state (mamba_block.py:68-102)."""
        return self._mix(x)

    def prefill(self, x: torch.Tensor):
        """Parallel prefill (mamba_block.py:104-153).

        Returns (y (B, L, d_model), conv_state (B, d_inner, d_conv) in x's dtype,
        ssm_state (B, d_inner, d_state) float32)."""
        Bsz = x.shape[0]
        conv_state = torch.empty((Bsz, self.d_inner, self.d_conv), dtype=x.dtype, device=x.device)
        ssm_state = torch.empty((Bsz, self.d_inner, self.d_state), dtype=torch.float32,
                                device=x.device)
        y = self._mix(x, conv_state, ssm_state)
        return y, conv_state, ssm_state

    def step(self, x_token: torch.Tensor, conv_state: torch.Tensor, ssm_state: torch.Tensor,
             inplace: bool = False):
        """O(1) per-token forward (mamba_block.py:155-198).

        x_token (B, 1, d_model).  Functional by default, as the reference (which returns
        fresh arrays): the given states are left untouched and new ones returned.  With
        inplace=True the decode kernels update the given states in place and return them."""
        if not inplace:
            conv_state = conv_state.clone()
            ssm_state = ssm_state.clone()
        return self.step_2d(x_token[:, 0, :], conv_state, ssm_state)[:, None, :], \
            conv_state, ssm_state

    def step_2d(self, x: torch.Tensor, conv_state: torch.Tensor, ssm_state: torch.Tensor,
                resid: torch.Tensor | None = None, next_norm: nn.Module | None = None,
                x_norm: nn.Module | None = None, defer_norm: bool = False):
        """The decode step on a (B, d_model) row block, states updated in place.

        in_proj GEMM + conv-window step -> x_proj GEMM -> fused dt_proj + softplus +
        SSM update + C contraction + D skip + SiLU(z) -> out_proj GEMM.  For f16/bf16
        at B <= 64 the GEMMs are the weight-streaming decode kernel with the conv
        step folded into in_proj and, when ``resid`` is given, the residual add (and
        ``next_norm``, an RMSNorm, when given) folded into out_proj.

        Without ``resid`` returns out_proj(y).  With ``resid`` returns a pair: ``(y,
        None)`` when the caller still has to add y; ``(None, None)`` when ``resid``
        already holds x + out_proj(y); ``(None, h)`` when in addition h =
        next_norm(resid); with ``defer_norm``, ``(None, NORM_PENDING)`` when ``resid``
        holds x + out_proj(y) and next_norm is left to the next in_proj.

        ``x_norm`` (an RMSNorm): x holds the raw residual rows and the block's input is
        x_norm(x) -- folded into in_proj's operand load at small batch (bit-identical
        to the separate norm), applied by ``add_rmsnorm`` first otherwise."""
        di = self.d_inner
        W_in = self.in_proj.weight
        conv_ok = in_proj_conv_ok(x, W_in, conv_state, self.conv1d.weight, self.conv1d.bias)
        fold = None
        if x_norm is not None:
            if conv_ok and norm_in_ok(x, W_in, x_norm.weight):
                fold = (x_norm.weight, x_norm.eps)
            else:
                x = add_rmsnorm(x, None, x_norm.weight, x_norm.eps)
        W_x = self.x_proj.weight
        if conv_ok and xproj_weight_ok(x, W_x, di):
            # in_proj + conv window + x_proj in one call (x_proj inside in_proj's epilogue
            # where the shape allows)
            x_conv, z, x_dbl = decode_in_proj_conv_xproj(x, W_in, conv_state, self.conv1d.weight,
                                                         self.conv1d.bias, W_x, x_norm=fold)
        else:
            if conv_ok:
                x_conv, z = decode_in_proj_conv(x, W_in, conv_state, self.conv1d.weight,
                                                self.conv1d.bias, x_norm=fold)
            else:
                xz = self.in_proj(x)                           # (B, 2*d_inner)
                x_main, z = xz[:, :di], xz[:, di:]
                x_conv = conv_step(conv_state, x_main, self.conv1d.weight, self.conv1d.bias,
                                   apply_silu=True)            # (B, d_inner)
            x_dbl = (decode_linear(x_conv, W_x) if decode_linear_ok(x_conv, W_x)
                     else self.x_proj(x_conv))
        dt_pre, Bm, Cm = self._split_xdbl(x_dbl)
        y = ssm_step_dtproj(ssm_state, x_conv, dt_pre, self.dt_proj.weight, self._A(), Bm, Cm,
                            dt_bias=self.dt_proj.bias, D=self.D, z=z)
        W_out = self.out_proj.weight
        fused = decode_linear_ok(y, W_out)
        if resid is None:
            return decode_linear(y, W_out) if fused else self.out_proj(y)
        if not (fused and resid.dtype == y.dtype and resid.stride(-1) == 1):
            return self.out_proj(y), None
        if next_norm is not None and next_norm.weight.dtype == y.dtype:
            if defer_norm and y.shape[0] <= NORM_IN_MAX_M and not split_k(y.shape[0], W_out):
                # no split-K reduce to carry the norm: leave it to the next in_proj
                decode_linear_resid_(resid, y, W_out)
                return None, NORM_PENDING
            return None, decode_linear_resid_norm_(resid, y, W_out, next_norm.weight, next_norm.eps)
        decode_linear_resid_(resid, y, W_out)
        return None, None
