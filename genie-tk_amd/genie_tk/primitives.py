"""Linear layer with AlphaFold-style initialisers and gated multi-head attention.

API and semantics of ``src/genie_tk/primitives.py`` in the reference:
``_init_weights`` (:17-40), ``Linear`` (:43-62), ``Attention`` (:65-178).
"""
from __future__ import annotations

import math
from typing import List, Optional

import torch
import torch.nn as nn
from torch import Tensor


def _init_weights(linear: nn.Linear, init: str = "default", std: float = 0.02) -> None:
    """In-place initialisation of an ``nn.Linear``.

    default: kaiming-uniform(a=sqrt(5)) weight, U(+-1/sqrt(fan_in)) bias (the
    nn.Linear default); final: zeros; gating: zero weight, unit bias;
    normal: N(0, std^2) weight, zero bias.
    """
    w, b = linear.weight, linear.bias
    if init == "default":
        nn.init.kaiming_uniform_(w, a=math.sqrt(5))
        if b is not None:
            fan_in = w.shape[1]
            bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
            nn.init.uniform_(b, -bound, bound)
    elif init == "final":
        nn.init.zeros_(w)
        if b is not None:
            nn.init.zeros_(b)
    elif init == "gating":
        nn.init.zeros_(w)
        if b is not None:
            nn.init.ones_(b)
    elif init == "normal":
        nn.init.normal_(w, std=std)
        if b is not None:
            nn.init.zeros_(b)


class _DenseMatmul(torch.autograd.Function):
    """a @ b over equal leading (batch) dims, every operand made contiguous
    first, in the forward and in the backward (dA = G B^T, dB = A^T G).

    torch.matmul over batches on a transposed or permuted view makes a strided
    batched product, and so does its autograd backward by itself; in bfloat16
    that form has faulted gfx950 devices.  The products here are the same ones
    on contiguous copies."""

    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor) -> Tensor:
        a, b = a.contiguous(), b.contiguous()
        ctx.save_for_backward(a, b)
        return torch.matmul(a, b)

    @staticmethod
    def backward(ctx, g: Tensor):
        a, b = ctx.saved_tensors
        g = g.contiguous()
        ga = gb = None
        if ctx.needs_input_grad[0]:
            ga = torch.matmul(g, b.transpose(-1, -2).contiguous())
        if ctx.needs_input_grad[1]:
            gb = torch.matmul(a.transpose(-1, -2).contiguous(), g)
        return ga, gb


def dense_matmul(a: Tensor, b: Tensor) -> Tensor:
    """``torch.matmul(a, b)`` for operands of equal leading dims, computed on
    contiguous operands in the forward and the backward."""
    assert a.shape[:-2] == b.shape[:-2], (a.shape, b.shape)
    return _DenseMatmul.apply(a, b)


class Linear(nn.Linear):
    """``nn.Linear`` whose parameters are initialised by ``_init_weights(init)``."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 init: str = "default"):
        super().__init__(in_features, out_features, bias=bias)
        _init_weights(self, init)


class Attention(nn.Module):
    """Gated multi-head attention with additive score biases.

    ``c_hidden`` is the total width over heads (head_dim = c_hidden / no_heads).
    forward: q, k, v projections without bias; scores = q k^T / sqrt(head_dim)
    plus every tensor in ``biases`` (added in list order); softmax over keys;
    o = attn v; o *= sigmoid(linear_g(q_x)) when gating; linear_o(o).
    """

    def __init__(self, c_q: int, c_k: int, c_v: int, c_hidden: int, no_heads: int,
                 gating: bool = True):
        super().__init__()
        assert c_hidden % no_heads == 0
        self.c_q, self.c_k, self.c_v = c_q, c_k, c_v
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.gating = gating
        self.head_dim = c_hidden // no_heads
        self.linear_q = Linear(c_q, c_hidden, bias=False)
        self.linear_k = Linear(c_k, c_hidden, bias=False)
        self.linear_v = Linear(c_v, c_hidden, bias=False)
        self.linear_o = Linear(c_hidden, c_q, init="final")
        if gating:
            self.linear_g = Linear(c_q, c_hidden, init="gating")
        self.sigmoid = nn.Sigmoid()
        self.softmax = nn.Softmax(dim=-1)

    def _heads(self, t: Tensor) -> Tensor:
        # [*, L, H*D] -> [*, H, L, D]
        return t.unflatten(-1, (self.no_heads, self.head_dim)).transpose(-2, -3)

    def forward(self, q_x: Tensor, k_x: Tensor, v_x: Tensor,
                biases: Optional[List[Tensor]] = None) -> Tensor:
        q = self._heads(self.linear_q(q_x))
        k = self._heads(self.linear_k(k_x))
        v = self._heads(self.linear_v(v_x))
        scores = dense_matmul(q, k.transpose(-1, -2)) * (1.0 / math.sqrt(self.head_dim))
        for extra in biases or ():
            scores = scores + extra
        o = dense_matmul(self.softmax(scores), v)           # [*, H, Q, D]
        o = o.transpose(-2, -3).flatten(-2)                 # [*, Q, H*D]
        if self.gating:
            o = o * self.sigmoid(self.linear_g(q_x))
        return self.linear_o(o)
