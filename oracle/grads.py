"""numpy backward of the pair hot path (test oracle for the backward kernels).

Analytic gradients of the functions in pair_ops.py, restated from the chain
rule over the same operation sequence as the reference fallback:
  * TriangleMultiplicativeUpdate._forward_pytorch, triangle_mul.py:103-132
    (contractions :77-101);
  * TriangleAttention._forward_pytorch, triangle_attention.py:100-143, with
    Attention.forward, primitives.py:114-178.
The reference has no backward of its own: its gradients are torch autograd
over those lines.  These functions are pinned against central finite
differences (float64) and against torch autograd of the PyTorch path in
tests/test_oracle_grads.py.

Test infrastructure only: the product path never imports this module.
Every function returns (d_input, {state_dict key: gradient}), with the
gradients of a loss L for a given dL/dy.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import numpy as np

from oracle.pair_ops import Params, _p, contract, sigmoid

Grads = Dict[str, np.ndarray]


def layer_norm_fwd(x: np.ndarray, eps: float):
    """Normalised x (no affine) and 1/sqrt(var + eps), over the last axis."""
    mu = x.mean(axis=-1, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    return (x - mu) * rstd, rstd


def layer_norm_bwd(xhat: np.ndarray, rstd: np.ndarray, w: np.ndarray, dy: np.ndarray):
    """y = xhat * w + b with xhat = (x - mean) * rstd: returns dx, dw, db."""
    red = tuple(range(dy.ndim - 1))
    dw = (dy * xhat).sum(axis=red)
    db = dy.sum(axis=red)
    dxh = dy * w
    dx = rstd * (dxh - dxh.mean(axis=-1, keepdims=True)
                 - xhat * (dxh * xhat).mean(axis=-1, keepdims=True))
    return dx, dw, db


def linear_bwd(x: np.ndarray, w: np.ndarray, dy: np.ndarray):
    """y = x w^T + b: returns dx, dw (summed over every leading axis), db."""
    dx = dy @ w
    c_out, c_in = w.shape
    dw = dy.reshape(-1, c_out).T @ x.reshape(-1, c_in)
    db = dy.reshape(-1, c_out).sum(axis=0)
    return dx, dw, db


def contract_bwd(a: np.ndarray, b: np.ndarray, dx: np.ndarray, outgoing: bool):
    """Gradients of pair_ops.contract for dL/dx: (da, db).

    outgoing x_ijc = sum_k a_ikc b_jkc:  da_ikc = sum_j dx_ijc b_jkc,
                                          db_jkc = sum_i dx_ijc a_ikc.
    incoming x_ijc = sum_k a_kic b_kjc:  da_kic = sum_j dx_ijc b_kjc,
                                          db_kjc = sum_i dx_ijc a_kic.
    """
    dxc = dx.transpose(0, 3, 1, 2)  # [B, C, I, J]
    if outgoing:
        ac = a.transpose(0, 3, 1, 2)  # [B, C, I, K]
        bc = b.transpose(0, 3, 1, 2)  # [B, C, J, K]
        da = dxc @ bc                  # [B, C, I, K]
        db = dxc.swapaxes(-1, -2) @ ac  # [B, C, J, K]
    else:
        ac = a.transpose(0, 3, 2, 1)  # [B, C, I, K] = a[k, i]
        bc = b.transpose(0, 3, 2, 1)  # [B, C, J, K] = b[k, j]
        da = (dxc @ bc).swapaxes(-1, -2)                 # [B, C, K, I]
        db = (dxc.swapaxes(-1, -2) @ ac).swapaxes(-1, -2)  # [B, C, K, J]
    return da.transpose(0, 2, 3, 1), db.transpose(0, 2, 3, 1)


def tri_mul_grad(z: np.ndarray, mask: Optional[np.ndarray], params: Params, outgoing: bool,
                 dy: np.ndarray, dtype=np.float64, eps: float = 1e-5) -> Tuple[np.ndarray, Grads]:
    """Backward of pair_ops.tri_mul (triangle_mul.py:103-132) for dL/dy."""
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    z = np.asarray(z, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    m = (np.ones(z.shape[:-1], dtype=dtype) if mask is None
         else np.asarray(mask, dtype=dtype))[..., None]
    # forward, keeping what the backward needs
    zh, zr = layer_norm_fwd(z, eps)
    zn = zh * P("layer_norm_in.weight") + P("layer_norm_in.bias")
    lin = lambda x, k: x @ P(k + ".weight").T + P(k + ".bias")  # noqa: E731
    ap, ag = lin(zn, "linear_a_p"), lin(zn, "linear_a_g")
    bp, bg = lin(zn, "linear_b_p"), lin(zn, "linear_b_g")
    sa, sb = sigmoid(ag), sigmoid(bg)
    a, b = ap * sa * m, bp * sb * m
    x = contract(a, b, outgoing)
    xh, xr = layer_norm_fwd(x, eps)
    xn = xh * P("layer_norm_out.weight") + P("layer_norm_out.bias")
    p = lin(xn, "linear_z")
    g = sigmoid(lin(zn, "linear_g"))
    # backward
    grads: Grads = {}
    dp = dy * g
    dgp = dy * p * g * (1 - g)
    dxn, grads["linear_z.weight"], grads["linear_z.bias"] = linear_bwd(xn, P("linear_z.weight"), dp)
    dx, grads["layer_norm_out.weight"], grads["layer_norm_out.bias"] = layer_norm_bwd(
        xh, xr, P("layer_norm_out.weight"), dxn)
    da, db = contract_bwd(a, b, dx, outgoing)
    dzn, grads["linear_g.weight"], grads["linear_g.bias"] = linear_bwd(zn, P("linear_g.weight"), dgp)
    for name, d_pre in (("linear_a_p", da * sa * m), ("linear_a_g", da * ap * m * sa * (1 - sa)),
                        ("linear_b_p", db * sb * m), ("linear_b_g", db * bp * m * sb * (1 - sb))):
        dzi, grads[name + ".weight"], grads[name + ".bias"] = linear_bwd(zn, P(name + ".weight"), d_pre)
        dzn = dzn + dzi
    dz, grads["layer_norm_in.weight"], grads["layer_norm_in.bias"] = layer_norm_bwd(
        zh, zr, P("layer_norm_in.weight"), dzn)
    return dz, grads
