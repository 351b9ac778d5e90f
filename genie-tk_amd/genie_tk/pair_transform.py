"""Pair transform stack: the caller of the triangle operators.

API of ``src/genie_tk/pair_transform.py`` in the reference (DropoutRowwise
:26-42, DropoutColumnwise :45-61, PairTransition :64-84, PairTransformLayer
:87-195, PairTransformNet :198-258).  Update order per layer (:180-193):
tri-mul out, tri-mul in, tri-attn start, tri-attn end (each added to p with
row/column-shared dropout), pair transition, then p * mask.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from genie_tk import _dispatch, _ext

from genie_tk.primitives import Linear
from genie_tk.triangle_attention import TriangleAttentionEndingNode, TriangleAttentionStartingNode
from genie_tk.triangle_mul import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing


class _SharedDropout(nn.Module):
    """Dropout whose mask is shared along one spatial axis of [*, L, L, C]."""

    def __init__(self, p: float, shared_dim: int):
        super().__init__()
        self.p = p
        self.dropout = nn.Dropout(p)
        self._shared_dim = shared_dim

    def forward(self, x: Tensor) -> Tensor:
        if not self.training or self.p == 0:
            return x
        shape = list(x.shape)
        shape[self._shared_dim] = 1
        return x * self.dropout(x.new_ones(shape))


class DropoutRowwise(_SharedDropout):
    """Same dropout mask for every row (broadcast over dim -3)."""

    def __init__(self, p: float):
        super().__init__(p, -3)


class DropoutColumnwise(_SharedDropout):
    """Same dropout mask for every column (broadcast over dim -2)."""

    def __init__(self, p: float):
        super().__init__(p, -2)


class _PairTransitionFunction(torch.autograd.Function):
    """PairTransition on the HIP kernels, forward and backward.

    The reference trains through torch autograd of its PyTorch path
    (pair_transform.py:79-84); this computes the same gradients with
    ``genie_tk._C.pair_transition_backward`` (the hidden activation is
    recomputed from p; only p and the parameters are saved)."""

    @staticmethod
    def forward(ctx, module, p, *params):
        ctx.module = module
        ctx.save_for_backward(p, *params)
        return module._run_kernel(p, None, False)

    @staticmethod
    def backward(ctx, dy):
        p, *params = ctx.saved_tensors
        mod = ctx.module
        res = _ext.require().pair_transition_backward(
            p, dy.reshape(p.shape).to(p.dtype), list(params), mod.c_p, mod.n, mod.layer_norm.eps)
        dp = res[0] if ctx.needs_input_grad[1] else None
        g = _dispatch.grads_as_params(list(res[1:-1]), res[-1], params)
        grads = [gk if ctx.needs_input_grad[2 + k] else None for k, gk in enumerate(g)]
        return (None, dp, *grads)


class PairTransition(nn.Module):
    """LN -> Linear(c_p, n*c_p) -> ReLU -> Linear(n*c_p, c_p) (final init).

    Kernel path (``use_fused_kernel``, bf16 or fp32 GPU tensor, c_p in
    {64, 128}, n == 4): ``genie_tk._C.pair_transition_forward``, one gfx950
    kernel for the whole MLP; when autograd needs gradients the same forward
    runs inside ``_PairTransitionFunction``, whose backward is
    ``genie_tk._C.pair_transition_backward``.  ``forward_residual_masked``
    computes the pair-stack update ``(p + transition(p)) * mask`` in the same
    kernel (inference).
    """

    def __init__(self, c_p: int, n: int = 4, use_fused_kernel: bool = True):
        super().__init__()
        self.c_p = c_p
        self.n = n
        self._fused_requested = use_fused_kernel
        self.layer_norm = nn.LayerNorm(c_p)
        self.linear_1 = Linear(c_p, c_p * n)
        self.relu = nn.ReLU()
        self.linear_2 = Linear(c_p * n, c_p, init="final")
        self._packed = _dispatch.PackedWeights()

    def _forward_pytorch(self, p: Tensor) -> Tensor:
        return self.linear_2(self.relu(self.linear_1(self.layer_norm(p))))

    def _kernel_supported(self, p: Tensor) -> bool:
        """Kernel shapes: c_p in {64, 128}, n == 4, bf16 or fp32."""
        if not (p.is_cuda and self._fused_requested):
            return False
        if _ext.C is None or not torch.cuda.is_available():
            _ext.missing(type(self).__name__)
            return False
        return (p.dtype in (torch.bfloat16, torch.float32) and p.dim() >= 1
                and p.shape[-1] == self.c_p and self.c_p in (64, 128) and self.n == 4
                and self.layer_norm.elementwise_affine)

    def _use_kernel(self, p: Tensor) -> bool:
        """Inference on the kernels (no gradient needed)."""
        return self._kernel_supported(p) and not _dispatch.needs_autograd(p, self)

    # the parameters in the order of pair_transition_pack
    _PARAMS = tuple((m, w) for m in ("layer_norm", "linear_1", "linear_2") for w in ("weight", "bias"))

    def _param_list(self):
        return _dispatch.params_at(self, self._PARAMS)

    def _run_kernel(self, p: Tensor, mask: Optional[Tensor], residual: bool) -> Tensor:
        C = _ext.require()
        fp32 = p.dtype == torch.float32
        packed = self._packed.get(self._param_list(), fp32,
                                  lambda prm, f: C.pair_transition_pack(prm, self.c_p, self.n, f))
        m = None if mask is None else mask.expand(p.shape[:-1])
        return C.pair_transition_forward(p, m, packed, self.c_p, self.n, residual,
                                         self.layer_norm.eps)

    def forward(self, p: Tensor, mask: Optional[Tensor] = None) -> Tensor:
        if self._kernel_supported(p):
            if not _dispatch.needs_autograd(p, self):
                return self._run_kernel(p, None, False)
            return _PairTransitionFunction.apply(self, p, *self._param_list())
        return self._forward_pytorch(p)

    def forward_residual_masked(self, p: Tensor, mask: Tensor) -> Tensor:
        """(p + transition(p)) * mask[..., None] (pair_transform.py:192-193)."""
        if self._use_kernel(p):
            return self._run_kernel(p, mask, True)
        return (p + self.forward(p)) * mask.unsqueeze(-1)


class PairTransformLayer(nn.Module):
    """One pair-stack block; forward((p, p_mask)) -> (p, p_mask)."""

    def __init__(self, c_p: int, include_mul_update: bool = True, include_tri_att: bool = True,
                 c_hidden_mul: int = 128, c_hidden_tri_att: int = 32, n_head_tri: int = 4,
                 tri_dropout: float = 0.25, pair_transition_n: int = 4,
                 use_fused_kernel: bool = True):
        super().__init__()
        self.include_mul_update = include_mul_update
        self.include_tri_att = include_tri_att
        if include_mul_update:
            self.tri_mul_out = TriangleMultiplicationOutgoing(
                c_z=c_p, c_hidden=c_hidden_mul, use_fused_kernel=use_fused_kernel)
            self.tri_mul_in = TriangleMultiplicationIncoming(
                c_z=c_p, c_hidden=c_hidden_mul, use_fused_kernel=use_fused_kernel)
        if include_tri_att:
            self.tri_att_start = TriangleAttentionStartingNode(
                c_in=c_p, c_hidden=c_hidden_tri_att, no_heads=n_head_tri,
                use_fused_kernel=use_fused_kernel)
            self.tri_att_end = TriangleAttentionEndingNode(
                c_in=c_p, c_hidden=c_hidden_tri_att, no_heads=n_head_tri,
                use_fused_kernel=use_fused_kernel)
        self.pair_transition = PairTransition(c_p, pair_transition_n,
                                              use_fused_kernel=use_fused_kernel)
        self.dropout_row = DropoutRowwise(tri_dropout)
        self.dropout_col = DropoutColumnwise(tri_dropout)

    def forward(self, inputs: Tuple[Tensor, Tensor]) -> Tuple[Tensor, Tensor]:
        p, p_mask = inputs
        if not self.training or self.dropout_row.p == 0:
            # dropout is the identity: every residual add and the final mask
            # fold into the operators' kernels
            if self.include_mul_update:
                p = self.tri_mul_out.forward_residual(p, p_mask)
                p = self.tri_mul_in.forward_residual(p, p_mask)
            if self.include_tri_att:
                p = self.tri_att_start.forward_residual(p, p_mask)
                p = self.tri_att_end.forward_residual(p, p_mask)
            return self.pair_transition.forward_residual_masked(p, p_mask), p_mask
        if self.include_mul_update:
            p = p + self.dropout_row(self.tri_mul_out(p, p_mask))
            p = p + self.dropout_row(self.tri_mul_in(p, p_mask))
        if self.include_tri_att:
            p = p + self.dropout_row(self.tri_att_start(p, p_mask))
            p = p + self.dropout_col(self.tri_att_end(p, p_mask))
        p = p + self.pair_transition(p, p_mask)
        p = p * p_mask.unsqueeze(-1)
        return p, p_mask


class PairTransformNet(nn.Module):
    """``n_layers`` PairTransformLayers applied in sequence."""

    def __init__(self, c_p: int, n_layers: int, include_mul_update: bool = True,
                 include_tri_att: bool = True, c_hidden_mul: int = 128,
                 c_hidden_tri_att: int = 32, n_head_tri: int = 4, tri_dropout: float = 0.25,
                 pair_transition_n: int = 4, use_fused_kernel: bool = True):
        super().__init__()
        self.layers = nn.ModuleList([
            PairTransformLayer(c_p=c_p, include_mul_update=include_mul_update,
                               include_tri_att=include_tri_att, c_hidden_mul=c_hidden_mul,
                               c_hidden_tri_att=c_hidden_tri_att, n_head_tri=n_head_tri,
                               tri_dropout=tri_dropout, pair_transition_n=pair_transition_n,
                               use_fused_kernel=use_fused_kernel)
            for _ in range(n_layers)
        ])

    def forward(self, p: Tensor, p_mask: Tensor) -> Tensor:
        for layer in self.layers:
            p, p_mask = layer((p, p_mask))
        return p
