"""Triangle multiplicative update (AlphaFold2 Algorithms 11 and 12).

Drop-in for ``src/genie_tk/triangle_mul.py`` of the reference: same classes,
constructor arguments, parameter names (state_dict keys) and ``forward(z,
mask=None)`` returning the update (no residual).

Kernel path (``use_fused_kernel=True``, GPU tensor):
``genie_tk._C.tri_mul_forward``, three gfx950 kernels (prologue
LN + gated projections + mask, matrix-core contraction per channel, epilogue
LN + output projection + gate).  When autograd needs gradients the same
forward runs inside ``_TriMulFunction``, whose backward is
``genie_tk._C.tri_mul_backward`` (gradients of z and every parameter).
PyTorch path: ``_forward_pytorch``, the reference fallback semantics
(triangle_mul.py:103-132).

Memory-bounded mode (``forward(z, mask, chunk_size=R)``, an addition to the
reference's signature): the output rows i run R at a time, the row chunking of
``chunk_layer`` (utils.py:78-123) applied to the update.  On the kernels
(inference) the workspace shrinks from three to one full set of c planes plus
two R-row sets, with a bit-identical output; the PyTorch path holds x and its
output projection for one chunk at a time.
"""
from __future__ import annotations

from functools import partialmethod
from typing import Optional

import torch
import torch.nn as nn
from torch import Tensor

from genie_tk import _dispatch, _ext
from genie_tk.primitives import Linear, dense_matmul
from genie_tk.utils import has_cuda_kernels, permute_final_dims

_CUDA_AVAILABLE = has_cuda_kernels()

# hidden widths below the kernels' 32-channel tile run as 32 channels, each
# real channel repeated 32 / c_hidden times (_repeat_channels)
_NARROW = (8, 16)
# parameter positions (_PARAMS order) whose leading axis is the hidden channel
_HIDDEN_ROWS = (2, 3, 4, 5, 6, 7, 8, 9, 12, 13)


def _repeat_channels(params, r: int):
    """The module's parameters for r copies of every hidden channel (c_hidden
    c -> r c, copy k of channel j at r-channel index k c + j): the a/b
    projection and gate rows and biases and the LN_out affine repeated, the
    columns of W_z repeated and scaled by 1/r (exact: r is 2 or 4).  The
    copies of a and b are equal, so are the copies of x; LN_out over the r c
    channels has the mean and variance of x's c; and the scaled W_z adds the
    r equal copies back to one.  The update is the module's own."""
    out = list(params)
    for k in _HIDDEN_ROWS:
        out[k] = params[k].repeat(r, *([1] * (params[k].dim() - 1)))
    out[14] = params[14].repeat(1, r) * (1.0 / r)
    return out


def _fold_channel_grads(grads, c: int, r: int):
    """Gradients of the repeated parameters back to the module's: the sum
    over the r copies (the chain rule through the repetition), and 1/r of it
    for W_z's columns."""
    out = list(grads)
    for k in _HIDDEN_ROWS:
        g = grads[k]
        out[k] = g.reshape(r, c, *g.shape[1:]).sum(0)
    gz = grads[14]
    out[14] = gz.reshape(gz.shape[0], r, c).sum(1) * (1.0 / r)
    return out


class _TriMulFunction(torch.autograd.Function):
    """The update on the HIP kernels, forward and backward.

    The reference trains through torch autograd of its PyTorch path
    (triangle_mul.py:103-132); this computes the same gradients on the
    kernels.  Activations are recomputed in the backward from z (only z, the
    mask and the parameters are saved)."""

    @staticmethod
    def forward(ctx, module, z, mask, *params):
        ctx.module = module
        ctx.save_for_backward(z, mask, *params)
        return module._forward_cuda(z, mask)

    @staticmethod
    def backward(ctx, dy):
        z, mask, *params = ctx.saved_tensors
        mod = ctx.module
        zb, mb, lead = _dispatch.flatten_batch(z, mask)
        r = mod._repeats()
        bparams = list(params)
        if r > 1:
            with torch.no_grad():
                bparams = _repeat_channels(bparams, r)
        res = _ext.require().tri_mul_backward(
            zb, mb, dy.reshape(zb.shape).to(z.dtype), bparams, mod.c_z, mod.c_hidden * r,
            mod._outgoing, mod.layer_norm_in.eps, mod.layer_norm_out.eps)
        dz = res[0].reshape(z.shape) if ctx.needs_input_grad[1] else None
        g, flat = list(res[1:-1]), res[-1]
        if r > 1:
            g, flat = _fold_channel_grads(g, mod.c_hidden, r), None
        g = _dispatch.grads_as_params(g, flat, params)
        grads = [gk if ctx.needs_input_grad[3 + k] else None for k, gk in enumerate(g)]
        return (None, dz, None, *grads)


class TriangleMultiplicativeUpdate(nn.Module):
    """Triangle multiplicative update over a pair representation ``z [*, N, N, c_z]``.

    outgoing: x[i,j,c] = sum_k a[i,k,c] b[j,k,c];  incoming: x[i,j,c] = sum_k a[k,i,c] b[k,j,c]
    with a, b the sigmoid-gated, masked projections of LN_in(z); the result is
    LN_out(x) -> linear_z, gated by sigmoid(linear_g(LN_in(z))).
    """

    def __init__(self, c_z: int, c_hidden: int, _outgoing: bool = True,
                 use_fused_kernel: bool = True):
        super().__init__()
        self.c_z = c_z
        self.c_hidden = c_hidden
        self._outgoing = _outgoing
        self._fused_requested = use_fused_kernel
        self.use_fused_kernel = use_fused_kernel and _CUDA_AVAILABLE

        self.linear_a_p = Linear(c_z, c_hidden)
        self.linear_a_g = Linear(c_z, c_hidden, init="gating")
        self.linear_b_p = Linear(c_z, c_hidden)
        self.linear_b_g = Linear(c_z, c_hidden, init="gating")
        self.linear_g = Linear(c_z, c_z, init="gating")
        self.linear_z = Linear(c_hidden, c_z, init="final")
        self.layer_norm_in = nn.LayerNorm(c_z)
        self.layer_norm_out = nn.LayerNorm(c_hidden)
        self.sigmoid = nn.Sigmoid()
        self._packed = _dispatch.PackedWeights()

    # -- reference fallback -------------------------------------------------
    def _outgoing_matmul(self, a: Tensor, b: Tensor) -> Tensor:
        """x[*, i, j, c] = sum_k a[*, i, k, c] b[*, j, k, c] as a batched [c] matmul."""
        x = dense_matmul(permute_final_dims(a, 2, 0, 1), permute_final_dims(b, 2, 1, 0))
        return permute_final_dims(x, 1, 2, 0)

    def _incoming_matmul(self, a: Tensor, b: Tensor) -> Tensor:
        """x[*, i, j, c] = sum_k a[*, k, i, c] b[*, k, j, c] as a batched [c] matmul."""
        x = dense_matmul(permute_final_dims(a, 2, 1, 0), permute_final_dims(b, 2, 0, 1))
        return permute_final_dims(x, 1, 2, 0)

    def _forward_pytorch(self, z: Tensor, mask: Optional[Tensor] = None,
                         chunk_size: Optional[int] = None) -> Tensor:
        # the mask in the input's dtype (the reference's own path multiplies
        # in that dtype; a float32 mask on a bf16 input would promote a and b)
        mask = z.new_ones(z.shape[:-1]) if mask is None else mask.to(z.dtype)
        m = mask.unsqueeze(-1)
        zn = self.layer_norm_in(z)
        a = self.linear_a_p(zn) * self.sigmoid(self.linear_a_g(zn)) * m
        b = self.linear_b_p(zn) * self.sigmoid(self.linear_b_g(zn)) * m
        n = z.shape[-3]
        if chunk_size is None or chunk_size >= n:
            x = self._outgoing_matmul(a, b) if self._outgoing else self._incoming_matmul(a, b)
            x = self.linear_z(self.layer_norm_out(x))
            return x * self.sigmoid(self.linear_g(zn))
        # output rows i in chunks: x[i, j] needs row i of a (outgoing: a[i, k];
        # incoming: a[k, i]) against every row of b
        outs = []
        for s0 in range(0, n, chunk_size):
            rows = slice(s0, s0 + chunk_size)
            if self._outgoing:
                x = self._outgoing_matmul(a[..., rows, :, :], b)
            else:
                x = self._incoming_matmul(a[..., :, rows, :], b)
            x = self.linear_z(self.layer_norm_out(x))
            outs.append(x * self.sigmoid(self.linear_g(zn[..., rows, :, :])))
        return torch.cat(outs, dim=-3)

    # -- HIP kernel path ----------------------------------------------------
    def _kernel_supported(self, z: Tensor) -> bool:
        """Forward kernels: c_z in {32, 64, 128}, c_hidden in {32, 64, 128,
        256}, and 8 or 16 run as 32 (_repeat_channels)."""
        return (z.dim() >= 3 and z.shape[-2] == z.shape[-3] and z.shape[-1] == self.c_z
                and self.c_z in (32, 64, 128) and self.c_hidden in (*_NARROW, 32, 64, 128, 256)
                and z.dtype in _dispatch.SUPPORTED_DTYPES
                and self.layer_norm_in.elementwise_affine and self.layer_norm_out.elementwise_affine)

    def _backward_supported(self) -> bool:
        """The shapes the backward kernels are built for: c_z and c_hidden in
        {32, 64, 128}, and c_hidden 8 or 16 run as 32."""
        return self.c_z in (32, 64, 128) and self.c_hidden in (*_NARROW, 32, 64, 128)

    def _repeats(self) -> int:
        """Copies of each hidden channel on the kernels: 32 / c_hidden for the
        narrow widths, else 1."""
        return 32 // self.c_hidden if self.c_hidden in _NARROW else 1

    def _pack(self, params, fp32: bool) -> Tensor:
        r = self._repeats()
        if r > 1:
            params = _repeat_channels(params, r)
        return _ext.require().tri_mul_pack(params, self.c_z, self.c_hidden * r, fp32)

    # the parameters in the order of tri_mul_pack / gtk_tri_mul_weights
    _PARAMS = tuple((m, w) for m in ("layer_norm_in", "linear_a_p", "linear_a_g", "linear_b_p",
                                     "linear_b_g", "linear_g", "layer_norm_out", "linear_z")
                    for w in ("weight", "bias"))

    def _param_list(self):
        return _dispatch.params_at(self, self._PARAMS)

    def _packed_params(self, fp32: bool) -> Tensor:
        return self._packed.get(self._param_list(), fp32, self._pack)

    def _forward_cuda(self, z: Tensor, mask: Optional[Tensor] = None,
                      residual: bool = False, chunk_size: Optional[int] = None) -> Tensor:
        """HIP path; returns the update (plus z when ``residual``).  With
        ``chunk_size`` the output rows run that many at a time (the
        memory-bounded mode, bit-identical output)."""
        C = _ext.require()
        zb, mb, lead = _dispatch.flatten_batch(z, mask)
        packed = self._packed_params(z.dtype == torch.float32)
        out = C.tri_mul_forward(zb, mb, packed, self.c_z, self.c_hidden * self._repeats(),
                                self._outgoing, residual, self.layer_norm_in.eps,
                                self.layer_norm_out.eps, int(chunk_size or 0))
        return out.reshape(*lead, *out.shape[1:])

    @staticmethod
    def _check_chunk(chunk_size: Optional[int]) -> None:
        if chunk_size is not None and chunk_size < 1:
            raise ValueError(f"chunk_size must be >= 1, got {chunk_size}")

    def forward_residual(self, z: Tensor, mask: Optional[Tensor] = None,
                         chunk_size: Optional[int] = None) -> Tensor:
        """z + forward(z, mask), with the add fused into the kernel's output."""
        self._check_chunk(chunk_size)
        if (z.is_cuda and self._fused_requested and self.use_fused_kernel and _CUDA_AVAILABLE
                and self._kernel_supported(z) and not _dispatch.needs_autograd(z, self)):
            return self._forward_cuda(z, mask, residual=True, chunk_size=chunk_size)
        return z + self.forward(z, mask, chunk_size=chunk_size)

    def forward(self, z: Tensor, mask: Optional[Tensor] = None,
                chunk_size: Optional[int] = None) -> Tensor:
        """z: [*, N, N, c_z], mask: [*, N, N] -> update [*, N, N, c_z].

        ``chunk_size`` (an addition to the reference's signature, default off)
        runs the output rows that many at a time.  On the kernels it applies
        to inference; when autograd needs gradients a chunked call runs the
        PyTorch path."""
        self._check_chunk(chunk_size)
        if z.is_cuda and self._fused_requested:
            if not _CUDA_AVAILABLE:
                _ext.missing(type(self).__name__)
            elif self.use_fused_kernel and self._kernel_supported(z):
                if not _dispatch.needs_autograd(z, self):
                    return self._forward_cuda(z, mask, chunk_size=chunk_size)
                if self._backward_supported() and chunk_size is None:
                    return _TriMulFunction.apply(self, z, mask, *self._param_list())
        return self._forward_pytorch(z, mask, chunk_size)


class TriangleMultiplicationOutgoing(TriangleMultiplicativeUpdate):
    """Algorithm 11: x[i,j] = sum_k a[i,k] * b[j,k]."""

    __init__ = partialmethod(TriangleMultiplicativeUpdate.__init__, _outgoing=True)


class TriangleMultiplicationIncoming(TriangleMultiplicativeUpdate):
    """Algorithm 12: x[i,j] = sum_k a[k,i] * b[k,j]."""

    __init__ = partialmethod(TriangleMultiplicativeUpdate.__init__, _outgoing=False)
