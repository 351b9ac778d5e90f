"""numpy restatement of the reference fallback for the pair hot path (test oracle).

Parameters are dicts keyed by the reference modules' state_dict names, with
numpy arrays in nn.Linear layout ([out, in]).  ``dtype`` selects the working
precision: float32 reproduces the reference's default fp32 arithmetic,
float64 is used to pin the restatement against the scalar loops in brute.py.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional

import numpy as np

Params = Dict[str, np.ndarray]

# |inf| from which the fp32 rounding of a masked key's score is modelled in
# float64 (ulp(2^29) = 64 in fp32: the mask term absorbs |logits| below 32).
_ABSORB_INF = 2.0 ** 29


def _p(params: Params, key: str, dtype) -> np.ndarray:
    return np.asarray(params[key], dtype=dtype)


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """torch.nn.LayerNorm over the last axis: biased variance, eps inside the root."""
    mu = x.mean(axis=-1, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def linear(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray] = None) -> np.ndarray:
    """nn.Linear: x @ w^T + b (primitives.py:43-62)."""
    y = x @ w.T
    return y if b is None else y + b


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------
# Triangle multiplicative update — triangle_mul.py:77-132
# ---------------------------------------------------------------------------
def contract(a: np.ndarray, b: np.ndarray, outgoing: bool,
             rows: Optional[Iterable[int]] = None) -> np.ndarray:
    """outgoing x[.., i, j, c] = sum_k a[.., i, k, c] b[.., j, k, c]   (triangle_mul.py:77-89)
    incoming x[.., i, j, c] = sum_k a[.., k, i, c] b[.., k, j, c]   (triangle_mul.py:91-101)

    a, b: [B, N, N, C].  ``rows`` restricts the output to those i (x: [B, R, N, C]).
    """
    if not outgoing:
        a = a.swapaxes(1, 2)
        b = b.swapaxes(1, 2)
    if rows is not None:
        a = a[:, list(rows)]
    # per channel: X_c = A_c B_c^T with A_c[i, k] = a[i, k, c]; contiguous
    # operands keep np.matmul on its BLAS path
    ac = np.ascontiguousarray(a.transpose(0, 3, 1, 2))
    bc = np.ascontiguousarray(b.transpose(0, 3, 1, 2))
    x = np.matmul(ac, bc.swapaxes(-1, -2))  # [B, C, I, J]
    return x.transpose(0, 2, 3, 1)


def tri_mul(z: np.ndarray, mask: Optional[np.ndarray], params: Params, outgoing: bool,
            dtype=np.float32, eps: float = 1e-5,
            rows: Optional[Iterable[int]] = None) -> np.ndarray:
    """TriangleMultiplicativeUpdate._forward_pytorch (triangle_mul.py:103-132).

    z: [B, N, N, c_z], mask: [B, N, N] or None -> update [B, N, N, c_z]
    (or [B, R, N, c_z] for the output rows ``rows``).
    """
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    z = np.asarray(z, dtype=dtype)
    m = (np.ones(z.shape[:-1], dtype=dtype) if mask is None else np.asarray(mask, dtype=dtype))[..., None]
    zn = layer_norm(z, P("layer_norm_in.weight"), P("layer_norm_in.bias"), eps)
    # Output rows i need a at pairs (i, k) (outgoing) or (k, i) (incoming)
    # only, and b everywhere: with ``rows`` a is projected for those rows
    # alone and enters the contraction already restricted.
    if rows is None:
        za, ma = zn, m
    else:
        sel = (slice(None), list(rows)) if outgoing else (slice(None), slice(None), list(rows))
        za, ma = zn[sel], m[sel]
    a = linear(za, P("linear_a_p.weight"), P("linear_a_p.bias")) * sigmoid(
        linear(za, P("linear_a_g.weight"), P("linear_a_g.bias"))) * ma
    b = linear(zn, P("linear_b_p.weight"), P("linear_b_p.bias")) * sigmoid(
        linear(zn, P("linear_b_g.weight"), P("linear_b_g.bias"))) * m
    x = contract(a, b, outgoing)
    zr = zn if rows is None else zn[:, list(rows)]
    x = linear(layer_norm(x, P("layer_norm_out.weight"), P("layer_norm_out.bias"), eps),
               P("linear_z.weight"), P("linear_z.bias"))
    g = sigmoid(linear(zr, P("linear_g.weight"), P("linear_g.bias")))
    return x * g


# ---------------------------------------------------------------------------
# Triangle attention — triangle_attention.py:84-143, primitives.py:114-178
# ---------------------------------------------------------------------------
def _softmax_rows(s: np.ndarray) -> np.ndarray:
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def _masked_scores(qk: np.ndarray, keymask: np.ndarray, tri: np.ndarray, inf: float,
                   dtype) -> np.ndarray:
    """scores = (qk + inf*(m-1)) + tri, in the reference's order (primitives.py:156-158;
    mask bias triangle_attention.py:118).

    In float32 this is the literal reference arithmetic.  In float64, for
    |inf| >= 2^29, a masked key's score takes the reference's two fp32
    roundings, fl32(fl32(qk + fl32(inf*(m-1))) + tri), on the float64 values
    of qk and tri (each float64 sum is exact or within 2^-29 of exact, far
    inside the fp32 rounding step).  With inf = 1e9 and |qk| < 32 the scores
    are -1e9 plus multiples of 64: a row whose keys are all masked with mask 0
    is uniform when its bias values round to one multiple (|tri| < 32, or a
    per-head constant with small variation), and otherwise puts its weight on
    the keys whose fl32(-1e9 + tri) is largest, as the fp32 reference does.
    For smaller |inf| the float64 sum is used as it stands.
    """
    mb = (inf * (keymask - 1)).astype(dtype)
    if dtype == np.float32:
        return (qk + mb) + tri
    s = qk + tri
    masked = np.broadcast_to(keymask != 1, s.shape)
    if abs(inf) >= _ABSORB_INF and masked.any():
        mb32 = np.broadcast_to((inf * (keymask - 1)).astype(np.float32).astype(dtype), s.shape)
        f32 = lambda a: a.astype(np.float32).astype(dtype)  # noqa: E731
        masked_s = f32(f32(qk + mb32) + np.broadcast_to(tri, s.shape))
        return np.where(masked, masked_s, s)
    return (qk + mb) + tri


def tri_attn(x: np.ndarray, mask: Optional[np.ndarray], params: Params, starting: bool,
             no_heads: int, inf: float = 1e9, dtype=np.float32, eps: float = 1e-5,
             rows: Optional[Iterable[int]] = None) -> np.ndarray:
    """TriangleAttention._forward_pytorch (triangle_attention.py:100-143).

    x: [B, N, N, c_in], mask: [B, N, N] or None.  Ending node works on the
    transposed problem and transposes back (:110-112, :140-141).  ``rows``
    restricts the output to those attention rows (starting: rows i of the
    output; ending: columns j of the output); rows are independent problems.
    """
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    x = np.asarray(x, dtype=dtype)
    m = np.ones(x.shape[:-1], dtype=dtype) if mask is None else np.asarray(mask, dtype=dtype)
    if not starting:
        x = x.swapaxes(1, 2)
        m = m.swapaxes(1, 2)
    B, N, _, _ = x.shape
    xn = layer_norm(x, P("layer_norm.weight"), P("layer_norm.bias"), eps)
    tri = linear(xn, P("linear.weight")).transpose(0, 3, 1, 2)  # [B, H, Q, K]
    ch = P("mha.linear_q.weight").shape[0]
    d = ch // no_heads
    scale = 1.0 / np.sqrt(d)
    row_ids = list(range(N)) if rows is None else list(rows)
    out = np.empty((B, len(row_ids), N, x.shape[-1]), dtype=dtype)
    for b in range(B):
        for ri, i in enumerate(row_ids):
            xi = xn[b, i]                                           # [J, C]
            q = linear(xi, P("mha.linear_q.weight")).reshape(N, no_heads, d).transpose(1, 0, 2)
            k = linear(xi, P("mha.linear_k.weight")).reshape(N, no_heads, d).transpose(1, 0, 2)
            v = linear(xi, P("mha.linear_v.weight")).reshape(N, no_heads, d).transpose(1, 0, 2)
            qk = (q @ k.transpose(0, 2, 1)) * dtype(scale)          # [H, Q, K]
            s = _masked_scores(qk, m[b, i][None, None, :], tri[b], inf, dtype)
            o = (_softmax_rows(s) @ v).transpose(1, 0, 2).reshape(N, ch)
            o = o * sigmoid(linear(xi, P("mha.linear_g.weight"), P("mha.linear_g.bias")))
            out[b, ri] = linear(o, P("mha.linear_o.weight"), P("mha.linear_o.bias"))
    if not starting:
        out = out.swapaxes(1, 2)
    return out


def attention_core(q: np.ndarray, k: np.ndarray, v: np.ndarray, bias: np.ndarray,
                   mask: np.ndarray, scale: float, starting: bool, inf: float = 1e9,
                   dtype=np.float32) -> np.ndarray:
    """Semantics of _C.triangle_attention_starting/ending (kernels/bindings.cpp:82-90).

    q, k, v: [B, H, N, N, D]; bias: [B, H, N, N] indexed [query, key];
    mask: [B, N, N].  starting: rows = axis 2, positions = axis 3; ending:
    rows = axis 3, positions = axis 2 (the transposed problem).  Returns
    [B, N, N, H*D] in the input's spatial order.
    """
    q, k, v = (np.asarray(t, dtype=dtype) for t in (q, k, v))
    bias = np.asarray(bias, dtype=dtype)
    m = np.asarray(mask, dtype=dtype)
    if not starting:
        q, k, v = (t.swapaxes(2, 3) for t in (q, k, v))
        m = m.swapaxes(1, 2)
    B, H, N, _, D = q.shape
    out = np.empty((B, N, N, H * D), dtype=dtype)
    for b in range(B):
        for i in range(N):
            qk = (q[b, :, i] @ k[b, :, i].transpose(0, 2, 1)) * dtype(scale)   # [H, Q, K]
            s = _masked_scores(qk, m[b, i][None, None, :], bias[b], inf, dtype)
            o = _softmax_rows(s) @ v[b, :, i]                                  # [H, Q, D]
            out[b, i] = o.transpose(1, 0, 2).reshape(N, H * D)
    if not starting:
        out = out.swapaxes(1, 2)
    return out


# ---------------------------------------------------------------------------
# Pair-stack block (eval mode) — pair_transform.py:162-195
# ---------------------------------------------------------------------------
def pair_transition(p: np.ndarray, params: Params, dtype=np.float32, eps: float = 1e-5) -> np.ndarray:
    """PairTransition (pair_transform.py:64-84): LN -> linear_1 -> ReLU -> linear_2."""
    P = lambda k: _p(params, k, dtype)  # noqa: E731
    h = linear(layer_norm(p, P("layer_norm.weight"), P("layer_norm.bias"), eps),
               P("linear_1.weight"), P("linear_1.bias"))
    return linear(np.maximum(h, 0), P("linear_2.weight"), P("linear_2.bias"))


def sub_params(params: Params, prefix: str) -> Params:
    return {k[len(prefix):]: v for k, v in params.items() if k.startswith(prefix)}


def pair_block(p: np.ndarray, mask: np.ndarray, params: Params, no_heads: int,
               dtype=np.float32, include_transition: bool = True) -> np.ndarray:
    """PairTransformLayer.forward in eval mode (dropout is the identity).

    ``params`` uses the layer's state_dict names (tri_mul_out.*, tri_mul_in.*,
    tri_att_start.*, tri_att_end.*, pair_transition.*).
    """
    p = np.asarray(p, dtype=dtype)
    p = p + tri_mul(p, mask, sub_params(params, "tri_mul_out."), True, dtype)
    p = p + tri_mul(p, mask, sub_params(params, "tri_mul_in."), False, dtype)
    p = p + tri_attn(p, mask, sub_params(params, "tri_att_start."), True, no_heads, dtype=dtype)
    p = p + tri_attn(p, mask, sub_params(params, "tri_att_end."), False, no_heads, dtype=dtype)
    if include_transition:
        p = p + pair_transition(p, sub_params(params, "pair_transition."), dtype)
        p = p * np.asarray(mask, dtype=dtype)[..., None]
    return p
