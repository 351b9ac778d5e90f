"""Triangle attention (AlphaFold2 Algorithms 13 and 14).

Drop-in for ``src/genie_tk/triangle_attention.py`` of the reference: same
classes, constructor arguments, parameter names and ``forward(x, mask=None)``
returning the update (no residual).

Kernel path (``use_fused_kernel=True``, GPU tensor):
``genie_tk._C.tri_attn_forward`` — a gfx950 prologue (LN, q/k/v/gate and
triangle-bias projections on the matrix cores) and a flash-style kernel
(online softmax, bias streamed from HBM, gate and output projection fused).
When autograd needs gradients the same forward runs inside
``_TriAttnFunction``, whose backward is ``genie_tk._C.tri_attn_backward``.
PyTorch path: ``_forward_pytorch``, the reference fallback semantics
(triangle_attention.py:100-143).

Mask semantics of the kernel path: the reference's additive bias
``inf * (mask - 1)`` (triangle_attention.py:118) with the module's ``inf``,
in fp32.  A key with mask 1 takes no bias; a row whose keys are all masked
follows the fp32 arithmetic of the reference, which with the default
``inf=1e9`` makes it uniform (every logit rounds to -1e9 while |logit| < 32).
The backward kernels implement the default ``inf=1e9`` with a binary mask; a
module with another ``inf``, or a call with mask values other than 0 and 1,
trains through autograd of its PyTorch path.
"""
from __future__ import annotations

import math
from functools import partialmethod
from typing import Optional

import torch
import torch.nn as nn
from torch import Tensor

from genie_tk import _dispatch, _ext
from genie_tk.primitives import Attention, Linear
from genie_tk.utils import has_cuda_kernels, permute_final_dims

_CUDA_AVAILABLE = has_cuda_kernels()


# The backward kernels' head shape: four heads of HD_BWD channels.
H_BWD, HD_BWD = 4, 32


def _pad_heads(params, H: int, ch: int):
    """The module's parameters for the backward kernels' four heads of 32:
    head h's d = ch / H channels go to padded channels 32 h .. 32 h + d - 1,
    every other row of W_q, W_k, W_v, W_g and b_g and column of W_o is zero,
    and so are the triangle-bias rows of heads H .. 3.  W_q is scaled by
    sqrt(32 / d), so that the kernels' score scale 1/sqrt(32) is the module's
    1/sqrt(d).  The zero channels and heads add nothing to the output (their
    v and their W_o columns are zero), so the padded module's gradients
    restricted to the real parameters are the module's own.  Returns the
    padded list and the channel index of the real ones."""
    ln_w, ln_b, tri_w, q_w, k_w, v_w, g_w, g_b, o_w, o_b = params
    d = ch // H
    idx = (torch.arange(H, device=q_w.device)[:, None] * HD_BWD
           + torch.arange(d, device=q_w.device)[None, :]).reshape(-1)
    cp = H_BWD * HD_BWD
    scale = math.sqrt(HD_BWD / d)

    def rows(w, s=1.0):
        out = w.new_zeros((cp,) + tuple(w.shape[1:]))
        out[idx] = w * s if s != 1.0 else w
        return out

    o_p = o_w.new_zeros(o_w.shape[0], cp)
    o_p[:, idx] = o_w
    tri_p = tri_w.new_zeros(H_BWD, tri_w.shape[1])
    tri_p[:H] = tri_w
    return [ln_w, ln_b, tri_p, rows(q_w, scale), rows(k_w), rows(v_w), rows(g_w), rows(g_b), o_p,
            o_b], idx, scale


class _TriAttnFunction(torch.autograd.Function):
    """The update on the HIP kernels, forward and backward.

    The reference trains through torch autograd of its PyTorch path
    (triangle_attention.py:100-143, primitives.py:114-178); this computes the
    same gradients on the kernels.  Activations are recomputed in the backward
    from x (only x, the mask and the parameters are saved).  Modules with
    fewer than four heads, or heads narrower than 32 channels, run the
    backward on their weights padded to four heads of 32 (_pad_heads)."""

    @staticmethod
    def forward(ctx, module, x, mask, chunk_size, *params):
        ctx.module = module
        ctx.save_for_backward(x, mask, *params)
        return module._forward_cuda(x, mask, chunk_size=chunk_size)

    @staticmethod
    def backward(ctx, dy):
        x, mask, *params = ctx.saved_tensors
        mod = ctx.module
        xb, mb, lead = _dispatch.flatten_batch(x, mask)
        padded = (mod.no_heads, mod.c_hidden) != (H_BWD, H_BWD * HD_BWD)
        bparams = list(params)
        if padded:
            with torch.no_grad():
                bparams, idx, scale = _pad_heads(params, mod.no_heads, mod.c_hidden)
        res = _ext.require().tri_attn_backward(
            xb, mb, dy.reshape(xb.shape).to(x.dtype), bparams, mod.c_in, H_BWD * HD_BWD,
            H_BWD, mod.starting, mod.layer_norm.eps)
        dx = res[0].reshape(x.shape) if ctx.needs_input_grad[1] else None
        g, flat = list(res[1:-1]), res[-1]
        if padded:
            flat = None
            # back to the module's parameters (order of _PARAMS)
            g[2] = g[2][:mod.no_heads]
            g[3] = g[3][idx] * scale
            for k in (4, 5, 6, 7):
                g[k] = g[k][idx]
            g[8] = g[8][:, idx]
        g = _dispatch.grads_as_params(g, flat, params)
        grads = [gk if ctx.needs_input_grad[4 + k] else None for k, gk in enumerate(g)]
        return (None, dx, None, None, *grads)


class TriangleAttention(nn.Module):
    """Row-wise (starting) or column-wise (ending) gated attention with a
    triangle bias tri[h, q, k] = linear(LN(x))[q, k, h] shared by every row."""

    def __init__(self, c_in: int, c_hidden: int, no_heads: int, starting: bool = True,
                 inf: float = 1e9, use_fused_kernel: bool = True):
        super().__init__()
        self.c_in = c_in
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.starting = starting
        self.inf = inf
        self._fused_requested = use_fused_kernel
        self.use_fused_kernel = use_fused_kernel and _CUDA_AVAILABLE
        self.layer_norm = nn.LayerNorm(c_in)
        self.linear = Linear(c_in, no_heads, bias=False, init="normal")
        self.mha = Attention(c_q=c_in, c_k=c_in, c_v=c_in, c_hidden=c_hidden, no_heads=no_heads)
        self._packed = _dispatch.PackedWeights()

    # -- reference fallback -------------------------------------------------
    def _compute_triangle_bias(self, x: Tensor) -> Tensor:
        """[*, I, J, C] normalised input -> [*, H, I, J]."""
        return permute_final_dims(self.linear(x), 2, 0, 1)

    def _forward_pytorch(self, x: Tensor, mask: Optional[Tensor] = None,
                         chunk_size: Optional[int] = None) -> Tensor:
        # the mask in the input's dtype: the reference's own path (its mask
        # bias added to the scores) accepts only that pairing, and gives this
        # result for a mask passed in the input's dtype
        mask = x.new_ones(x.shape[:-1]) if mask is None else mask.to(x.dtype)
        if not self.starting:
            x = x.transpose(-2, -3)
            mask = mask.transpose(-1, -2)
        x = self.layer_norm(x)
        # [*, I, 1, 1, J]: added to the scores of every head and query of row I
        mask_bias = (self.inf * (mask - 1))[..., :, None, None, :]
        # [*, 1, H, Q, K]: the same triangle bias for every row
        tri = self._compute_triangle_bias(x).unsqueeze(-4)
        rows = x.shape[-3]
        if chunk_size is None or chunk_size >= rows:
            x = self.mha(q_x=x, k_x=x, v_x=x, biases=[mask_bias, tri])
        else:
            # rows are independent once the shared triangle bias exists: the
            # row axis is split and re-joined as chunk_layer does
            # (utils.py:78-123), bounding the [*, rows, H, Q, K] scores
            parts = []
            for s0 in range(0, rows, chunk_size):
                xs = x[..., s0:s0 + chunk_size, :, :]
                parts.append(self.mha(q_x=xs, k_x=xs, v_x=xs,
                                      biases=[mask_bias[..., s0:s0 + chunk_size, :, :, :], tri]))
            x = torch.cat(parts, dim=-3)
        if not self.starting:
            x = x.transpose(-2, -3)
        return x

    # -- HIP kernel path ----------------------------------------------------
    def _kernel_supported(self, x: Tensor) -> bool:
        """Forward kernels: c_in in {32, 64, 128}, 1, 2 or 4 heads of at most
        32 channels (the reference layer's default c_hidden=32 with 4 heads
        is d=8)."""
        h, ch = self.no_heads, self.c_hidden
        return (x.dim() >= 3 and x.shape[-2] == x.shape[-3] and x.shape[-1] == self.c_in
                and self.c_in in (32, 64, 128) and h in (1, 2, 4) and ch % h == 0
                and 1 <= ch // h <= 32 and self.mha.gating
                and x.dtype in _dispatch.SUPPORTED_DTYPES and self.layer_norm.elementwise_affine)

    def _backward_supported(self) -> bool:
        """The backward kernels: c_in in {32, 64, 128}; every head shape of the
        forward kernels (1, 2 or 4 heads of at most 32 channels) runs padded
        to four heads of 32."""
        return self.c_in in (32, 64, 128)

    def _pack(self, params, fp32: bool) -> Tensor:
        return _ext.require().tri_attn_pack(params, self.c_in, self.c_hidden, self.no_heads, fp32)

    # the parameters in the order of tri_attn_pack / gtk_tri_attn_weights
    _PARAMS = (("layer_norm", "weight"), ("layer_norm", "bias"), ("linear", "weight"),
               ("mha", "linear_q", "weight"), ("mha", "linear_k", "weight"),
               ("mha", "linear_v", "weight"), ("mha", "linear_g", "weight"),
               ("mha", "linear_g", "bias"), ("mha", "linear_o", "weight"),
               ("mha", "linear_o", "bias"))

    def _param_list(self):
        return _dispatch.params_at(self, self._PARAMS)

    def _packed_params(self, fp32: bool) -> Tensor:
        return self._packed.get(self._param_list(), fp32, self._pack)

    def _forward_cuda(self, x: Tensor, mask: Optional[Tensor] = None,
                      residual: bool = False, chunk_size: Optional[int] = None) -> Tensor:
        """HIP path; returns the update (plus x when ``residual``).  With
        ``chunk_size`` the attention rows run that many at a time in a
        workspace of that many rows (bit-identical output)."""
        C = _ext.require()
        xb, mb, lead = _dispatch.flatten_batch(x, mask)
        packed = self._packed_params(x.dtype == torch.float32)
        out = C.tri_attn_forward(xb, mb, packed, self.c_in, self.c_hidden, self.no_heads,
                                 self.starting, residual, self.layer_norm.eps,
                                 int(chunk_size or 0), float(self.inf))
        return out.reshape(*lead, *out.shape[1:])

    def forward_residual(self, x: Tensor, mask: Optional[Tensor] = None) -> Tensor:
        """x + forward(x, mask), with the add fused into the kernel's output."""
        if (x.is_cuda and self._fused_requested and self.use_fused_kernel
                and self._kernel_supported(x) and not _dispatch.needs_autograd(x, self)):
            return self._forward_cuda(x, mask, residual=True)
        return x + self.forward(x, mask)

    def forward(self, x: Tensor, mask: Optional[Tensor] = None,
                chunk_size: Optional[int] = None) -> Tensor:
        """x: [*, N, N, c_in], mask: [*, N, N] -> update [*, N, N, c_in].

        ``chunk_size`` (an addition to the reference's signature, default off)
        bounds memory: the attention rows are processed that many at a time,
        with the same result, on the kernels (every kernel shape and dtype, in
        inference) and on the PyTorch path (which also serves chunked calls
        that need gradients)."""
        if chunk_size is not None and chunk_size < 1:
            raise ValueError(f"chunk_size must be >= 1, got {chunk_size}")
        if x.is_cuda and self._fused_requested:
            if not _CUDA_AVAILABLE:
                _ext.missing(type(self).__name__)
            elif self.use_fused_kernel and self._kernel_supported(x):
                if not _dispatch.needs_autograd(x, self):
                    return self._forward_cuda(x, mask, chunk_size=chunk_size)
                # the backward kernels: their shapes, inf = 1e9 and a binary
                # mask (they model no other mask bias than 0 or -inf)
                if (self.inf == 1e9 and self._backward_supported()
                        and _dispatch.binary_mask(mask)):
                    return _TriAttnFunction.apply(self, x, mask, chunk_size, *self._param_list())
        return self._forward_pytorch(x, mask, chunk_size)


class TriangleAttentionStartingNode(TriangleAttention):
    """Algorithm 13: attention along j within each row i."""

    __init__ = partialmethod(TriangleAttention.__init__, starting=True)


class TriangleAttentionEndingNode(TriangleAttention):
    """Algorithm 14: attention along i within each column j."""

    __init__ = partialmethod(TriangleAttention.__init__, starting=False)
