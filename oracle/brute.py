"""Scalar-loop restatement of the pair hot path for tiny inputs (float64).

Written index-by-index from the equations (AlphaFold2 Algorithms 11-14 as
used by src/genie_tk/triangle_mul.py:103-132 and
src/genie_tk/triangle_attention.py:100-143 / primitives.py:114-178) without
matmuls, transposes or broadcasting, so that it shares no code path with
pair_ops.  Sizes: N <= 12, channels <= 32.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import numpy as np


def _ln(v: List[float], w, b, eps: float) -> List[float]:
    n = len(v)
    mu = sum(v) / n
    var = sum((t - mu) ** 2 for t in v) / n
    r = 1.0 / math.sqrt(var + eps)
    return [(v[c] - mu) * r * float(w[c]) + float(b[c]) for c in range(n)]


def _lin(v: List[float], W, b=None) -> List[float]:
    out = []
    for o in range(W.shape[0]):
        s = 0.0 if b is None else float(b[o])
        for c in range(W.shape[1]):
            s += float(W[o, c]) * v[c]
        out.append(s)
    return out


def _sig(t: float) -> float:
    return 1.0 / (1.0 + math.exp(-t))


def _score(sqk: float, tri: float, m: float, inf: float) -> float:
    """The reference's score (qk*scale + inf*(m - 1)) + tri (primitives.py:156-158,
    triangle_attention.py:118).  For m != 1 and |inf| >= 2^29 the score takes
    the fp32 reference's roundings of both sums, fl32(fl32(qk + fl32(mb)) +
    tri); with |qk| below half an ulp of mb the first is mb itself, and a row
    whose keys are all masked with mask 0 is uniform while its bias values
    round to one value."""
    if m == 1.0:
        return sqk + tri
    mb = inf * (m - 1.0)
    if abs(inf) >= 2.0 ** 29:
        f32 = lambda t: float(np.float32(t))  # noqa: E731
        return f32(f32(sqk + f32(mb)) + tri)
    return (sqk + mb) + tri


def tri_mul(z: np.ndarray, mask: Optional[np.ndarray], P: Dict[str, np.ndarray],
            outgoing: bool, eps: float = 1e-5) -> np.ndarray:
    B, N, _, cz = z.shape
    c = P["linear_a_p.weight"].shape[0]
    out = np.zeros((B, N, N, cz))
    for bb in range(B):
        zn = [[_ln([float(t) for t in z[bb, i, j]], P["layer_norm_in.weight"],
                   P["layer_norm_in.bias"], eps) for j in range(N)] for i in range(N)]
        a = [[None] * N for _ in range(N)]
        bv = [[None] * N for _ in range(N)]
        for i in range(N):
            for j in range(N):
                mij = 1.0 if mask is None else float(mask[bb, i, j])
                ap = _lin(zn[i][j], P["linear_a_p.weight"], P["linear_a_p.bias"])
                ag = _lin(zn[i][j], P["linear_a_g.weight"], P["linear_a_g.bias"])
                bp = _lin(zn[i][j], P["linear_b_p.weight"], P["linear_b_p.bias"])
                bg = _lin(zn[i][j], P["linear_b_g.weight"], P["linear_b_g.bias"])
                a[i][j] = [ap[t] * _sig(ag[t]) * mij for t in range(c)]
                bv[i][j] = [bp[t] * _sig(bg[t]) * mij for t in range(c)]
        for i in range(N):
            for j in range(N):
                x = []
                for ch in range(c):
                    s = 0.0
                    for k in range(N):
                        if outgoing:
                            s += a[i][k][ch] * bv[j][k][ch]
                        else:
                            s += a[k][i][ch] * bv[k][j][ch]
                    x.append(s)
                y = _lin(_ln(x, P["layer_norm_out.weight"], P["layer_norm_out.bias"], eps),
                         P["linear_z.weight"], P["linear_z.bias"])
                g = _lin(zn[i][j], P["linear_g.weight"], P["linear_g.bias"])
                for o in range(cz):
                    out[bb, i, j, o] = y[o] * _sig(g[o])
    return out


def tri_attn(x: np.ndarray, mask: Optional[np.ndarray], P: Dict[str, np.ndarray],
             starting: bool, no_heads: int, inf: float = 1e9, eps: float = 1e-5) -> np.ndarray:
    """Attention over positions of each row; ending node indexes columns directly.

    Scores follow _score: a masked key's score takes the fp32 reference's
    roundings when |inf| >= 2^29, so a row whose keys are all masked with
    mask 0 gets uniform weights while its bias values round to one value.
    """
    B, N, _, cin = x.shape
    ch = P["mha.linear_q.weight"].shape[0]
    d = ch // no_heads
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((B, N, N, cin))

    def at(bb, r, j):  # pair of row r, position j in the input's coordinates
        return (bb, r, j) if starting else (bb, j, r)

    for bb in range(B):
        xn = {}
        for r in range(N):
            for j in range(N):
                xn[(r, j)] = _ln([float(t) for t in x[at(bb, r, j)]], P["layer_norm.weight"],
                                 P["layer_norm.bias"], eps)
        tri = {(q, k): _lin(xn[(q, k)], P["linear.weight"]) for q in range(N) for k in range(N)}
        for r in range(N):
            valid = [1.0 if mask is None else float(mask[at(bb, r, k)]) for k in range(N)]
            qv = [_lin(xn[(r, j)], P["mha.linear_q.weight"]) for j in range(N)]
            kv = [_lin(xn[(r, j)], P["mha.linear_k.weight"]) for j in range(N)]
            vv = [_lin(xn[(r, j)], P["mha.linear_v.weight"]) for j in range(N)]
            for q in range(N):
                o = [0.0] * ch
                for h in range(no_heads):
                    logits = []
                    for k in range(N):
                        s = sum(qv[q][h * d + t] * kv[k][h * d + t] for t in range(d)) * scale
                        logits.append(_score(s, tri[(q, k)][h], valid[k], inf))
                    mx = max(logits)
                    w = [math.exp(t - mx) for t in logits]
                    tot = sum(w)
                    for t in range(d):
                        o[h * d + t] = sum(w[k] * vv[k][h * d + t] for k in range(N)) / tot
                g = _lin(xn[(r, q)], P["mha.linear_g.weight"], P["mha.linear_g.bias"])
                o = [o[t] * _sig(g[t]) for t in range(ch)]
                y = _lin(o, P["mha.linear_o.weight"], P["mha.linear_o.bias"])
                for c in range(cin):
                    out[at(bb, r, q) + (c,)] = y[c]
    return out


def pair_transition(p: np.ndarray, P: Dict[str, np.ndarray], eps: float = 1e-5) -> np.ndarray:
    """PairTransition.forward (pair_transform.py:79-84) pair by pair: LayerNorm,
    linear_1 (c -> n c), ReLU, linear_2 (n c -> c)."""
    out = np.zeros(p.shape)
    flat = p.reshape(-1, p.shape[-1])
    of = out.reshape(-1, p.shape[-1])
    for r in range(flat.shape[0]):
        v = _ln([float(t) for t in flat[r]], P["layer_norm.weight"], P["layer_norm.bias"], eps)
        h = [max(t, 0.0) for t in _lin(v, P["linear_1.weight"], P["linear_1.bias"])]
        of[r] = _lin(h, P["linear_2.weight"], P["linear_2.bias"])
    return out


def pair_block(p: np.ndarray, mask: np.ndarray, P: Dict[str, np.ndarray], no_heads: int) -> np.ndarray:
    """PairTransformLayer.forward in eval mode (pair_transform.py:180-193): each
    update added to p in turn (dropout is the identity), then p * mask."""
    def sub(prefix):
        return {k[len(prefix):]: v for k, v in P.items() if k.startswith(prefix)}

    p = np.asarray(p, dtype=np.float64)
    p = p + tri_mul(p, mask, sub("tri_mul_out."), True)
    p = p + tri_mul(p, mask, sub("tri_mul_in."), False)
    p = p + tri_attn(p, mask, sub("tri_att_start."), True, no_heads)
    p = p + tri_attn(p, mask, sub("tri_att_end."), False, no_heads)
    p = p + pair_transition(p, sub("pair_transition."))
    out = np.zeros(p.shape)
    B, N = p.shape[0], p.shape[1]
    for bb in range(B):
        for i in range(N):
            for j in range(N):
                for c in range(p.shape[-1]):
                    out[bb, i, j, c] = p[bb, i, j, c] * float(mask[bb, i, j])
    return out


def layer_norm(x: np.ndarray, w, b, eps: float = 1e-5) -> np.ndarray:
    out = np.zeros(x.shape)
    flat = x.reshape(-1, x.shape[-1])
    of = out.reshape(-1, x.shape[-1])
    for r in range(flat.shape[0]):
        of[r] = _ln([float(t) for t in flat[r]], w, b, eps)
    return out


def contract(a: np.ndarray, b: np.ndarray, outgoing: bool) -> np.ndarray:
    """x[b,i,j,c] = sum_k a[b,i,k,c] b[b,j,k,c] (outgoing, triangle_mul.py:77-89) or
    sum_k a[b,k,i,c] b[b,k,j,c] (incoming, triangle_mul.py:91-101), element by element."""
    B, N, _, C = a.shape
    out = np.zeros((B, N, N, C))
    for bb in range(B):
        for i in range(N):
            for j in range(N):
                for c in range(C):
                    s = 0.0
                    for k in range(N):
                        if outgoing:
                            s += float(a[bb, i, k, c]) * float(b[bb, j, k, c])
                        else:
                            s += float(a[bb, k, i, c]) * float(b[bb, k, j, c])
                    out[bb, i, j, c] = s
    return out


def attention_core(q, k, v, bias, mask, scale: float, starting: bool, inf: float = 1e9) -> np.ndarray:
    """_C.triangle_attention_starting/ending semantics (kernels/bindings.cpp:82-90):
    q, k, v [B,H,N,N,D]; bias [B,H,N,N] indexed (query, key); mask [B,N,N].
    Starting: row i = axis 2, positions along axis 3; ending: row j = axis 3,
    positions along axis 2.  Scores follow _score with the reference's
    default inf = 1e9.  Returns [B,N,N,H*D]."""
    B, H, N, _, D = q.shape
    out = np.zeros((B, N, N, H * D))

    def at(r, j):
        return (r, j) if starting else (j, r)

    for bb in range(B):
        for r in range(N):
            for h in range(H):
                for qi in range(N):
                    logits = []
                    for ki in range(N):
                        s = sum(float(q[(bb, h) + at(r, qi) + (t,)]) * float(k[(bb, h) + at(r, ki) + (t,)])
                                for t in range(D)) * scale
                        logits.append(_score(s, float(bias[bb, h, qi, ki]),
                                             float(mask[(bb,) + at(r, ki)]), inf))
                    mx = max(logits)
                    w = [math.exp(t - mx) for t in logits]
                    tot = sum(w)
                    for t in range(D):
                        o = sum(w[ki] * float(v[(bb, h) + at(r, ki) + (t,)]) for ki in range(N)) / tot
                        out[(bb,) + at(r, qi) + (h * D + t,)] = o
    return out
