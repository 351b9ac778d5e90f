"""numpy backward of the pair hot path (test oracle for the backward kernels).

Analytic gradients of the functions in pair_ops.py, restated from the chain
rule over the same operation sequence as the reference fallback:
  * TriangleMultiplicativeUpdate._forward_pytorch, triangle_mul.py:103-132
    (contractions :77-101);
  * TriangleAttention._forward_pytorch, triangle_attention.py:100-143, with
    Attention.forward, primitives.py:114-178;
  * PairTransition.forward, pair_transform.py:79-84.
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

from oracle.pair_ops import Params, _masked_scores, _p, _softmax_rows, contract, sigmoid

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


def tri_attn_grad(x: np.ndarray, mask: Optional[np.ndarray], params: Params, starting: bool,
                  no_heads: int, dy: np.ndarray, inf: float = 1e9, dtype=np.float64,
                  eps: float = 1e-5) -> Tuple[np.ndarray, Grads]:
    """Backward of pair_ops.tri_attn (triangle_attention.py:100-143,
    primitives.py:114-178) for dL/dy.

    The softmax gradient ds = p (dp - sum_k p dp) flows into q.k and the
    triangle bias with derivative one, also for a row whose keys are all
    masked: there the forward's scores are the constant -inf (absorbed in
    fp32, primitives.py:156-158) and p is uniform, but torch autograd of the
    reference still differentiates the sum qk + mask_bias + tri term by term.
    That is the reference's gradient, and the one restated here.
    """
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    x = np.asarray(x, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    m = np.ones(x.shape[:-1], dtype=dtype) if mask is None else np.asarray(mask, dtype=dtype)
    if not starting:
        x, m, dy = x.swapaxes(1, 2), m.swapaxes(1, 2), dy.swapaxes(1, 2)
    B, N, _, C = x.shape
    H = no_heads
    Wq, Wk, Wv = P("mha.linear_q.weight"), P("mha.linear_k.weight"), P("mha.linear_v.weight")
    Wg, bg = P("mha.linear_g.weight"), P("mha.linear_g.bias")
    Wo, bo = P("mha.linear_o.weight"), P("mha.linear_o.bias")
    Wb = P("linear.weight")
    ch = Wq.shape[0]
    d = ch // H
    scale = dtype(1.0 / np.sqrt(d))
    xh, xr = layer_norm_fwd(x, eps)
    xn = xh * P("layer_norm.weight") + P("layer_norm.bias")
    tri = (xn @ Wb.T).transpose(0, 3, 1, 2)  # [B, H, Q, K]
    g = {k: np.zeros_like(v, dtype=dtype) for k, v in params.items()}
    dxn = np.zeros_like(xn)
    dtri = np.zeros_like(tri)
    heads = lambda t: t.reshape(N, H, d).transpose(1, 0, 2)  # noqa: E731  [J, ch] -> [H, J, d]
    flat = lambda t: t.transpose(1, 0, 2).reshape(N, ch)    # noqa: E731
    for b in range(B):
        for i in range(N):
            if not dy[b, i].any():
                continue  # every term of this row is a product with dy[b, i]: all zero
            xi = xn[b, i]
            q, k, v = heads(xi @ Wq.T), heads(xi @ Wk.T), heads(xi @ Wv.T)
            s = _masked_scores((q @ k.transpose(0, 2, 1)) * scale, m[b, i][None, None, :],
                               tri[b], inf, dtype)
            p = _softmax_rows(s)
            of = flat(p @ v)
            gt = sigmoid(xi @ Wg.T + bg)
            dyi = dy[b, i]
            g["mha.linear_o.weight"] += dyi.T @ (of * gt)
            g["mha.linear_o.bias"] += dyi.sum(axis=0)
            dog = dyi @ Wo
            dgpre = dog * of * gt * (1 - gt)
            g["mha.linear_g.weight"] += dgpre.T @ xi
            g["mha.linear_g.bias"] += dgpre.sum(axis=0)
            do = heads(dog * gt)
            dp = do @ v.transpose(0, 2, 1)                        # [H, Q, K]
            dv = p.transpose(0, 2, 1) @ do                        # [H, K, d]
            ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True))
            dtri[b] += ds
            dq = (ds @ k) * scale
            dk = (ds.transpose(0, 2, 1) @ q) * scale
            for name, dt_, W in (("q", dq, Wq), ("k", dk, Wk), ("v", dv, Wv)):
                g[f"mha.linear_{name}.weight"] += flat(dt_).T @ xi
            dxn[b, i] += dgpre @ Wg + flat(dq) @ Wq + flat(dk) @ Wk + flat(dv) @ Wv
    dtp = dtri.transpose(0, 2, 3, 1)                              # [B, Q, K, H]
    dxn += dtp @ Wb
    g["linear.weight"] = dtp.reshape(-1, H).T @ xn.reshape(-1, C)
    dx, g["layer_norm.weight"], g["layer_norm.bias"] = layer_norm_bwd(
        xh, xr, P("layer_norm.weight"), dxn)
    if not starting:
        dx = dx.swapaxes(1, 2)
    return dx, g


def relu_bwd(h: np.ndarray, da: np.ndarray) -> np.ndarray:
    """Gradient through relu(h): passed where h > 0 (torch's convention at 0)."""
    return da * (h > 0)


def pair_transition_grad(p: np.ndarray, params: Params, dy: np.ndarray, dtype=np.float64,
                         eps: float = 1e-5,
                         gate: Optional[np.ndarray] = None) -> Tuple[np.ndarray, Grads]:
    """Backward of pair_ops.pair_transition (PairTransition.forward,
    pair_transform.py:79-84: LayerNorm -> linear_1 -> ReLU -> linear_2) for
    dL/dy over every leading axis.  The ReLU passes the gradient where its
    input is > 0 (torch's convention at 0).

    ``gate`` (boolean, the shape of the hidden activation) replaces the ReLU's
    pass pattern h > 0, for comparing with an implementation whose h is
    rounded differently: the derivative of ReLU is discontinuous, so a unit
    with h within rounding distance of 0 passes its gradient in one and not
    in the other."""
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    x = np.asarray(p, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    xh, rstd = layer_norm_fwd(x, eps)
    xn = xh * P("layer_norm.weight") + P("layer_norm.bias")
    h = xn @ P("linear_1.weight").T + P("linear_1.bias")
    a = np.maximum(h, 0)
    g: Grads = {}
    da, g["linear_2.weight"], g["linear_2.bias"] = linear_bwd(a, P("linear_2.weight"), dy)
    dh = relu_bwd(h, da) if gate is None else da * gate
    dxn, g["linear_1.weight"], g["linear_1.bias"] = linear_bwd(xn, P("linear_1.weight"), dh)
    dx, g["layer_norm.weight"], g["layer_norm.bias"] = layer_norm_bwd(
        xh, rstd, P("layer_norm.weight"), dxn)
    return dx, g
