"""Pins of the CPU oracle (oracle/pair_ops.py) — CPU only.

Each check is chosen so that a plausible restatement mistake (a transposed
operand, a wrong index, a dropped bias term, the mask applied in the wrong
place) fails at least one of them:
  * float64 agreement with the scalar loops in oracle/brute.py;
  * agreement with library routines (torch layer_norm, einsum, SDPA);
  * identities (incoming vs transposed outgoing, ending vs transposed starting);
  * closed forms (zero output under default init, constant gate, padded
    tri-mul rows, uniform attention on fully masked rows);
  * planted mistakes in a copy of the oracle are detected.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute, pair_ops
from tests import helpers as H

F64 = np.float64


def _tm_params(cz=16, c=8, seed=0, **kw):
    kw.setdefault("ln_random", True)
    kw.setdefault("bias_random", True)
    return H.draw_params(H.tri_mul_shapes(cz, c), seed, **kw)


def _ta_params(cin=16, ch=8, nh=2, seed=0, **kw):
    kw.setdefault("ln_random", True)
    kw.setdefault("bias_random", True)
    return H.draw_params(H.tri_attn_shapes(cin, ch, nh), seed, **kw)


def _partial_mask(B, N, seed=3):
    rng = np.random.default_rng(seed)
    m = (rng.random((B, N, N)) > 0.3).astype(np.float32)
    return m


# ---------------------------------------------------------------- LayerNorm
def test_layer_norm_matches_torch_and_loops():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7, 24)) * 3 + 1.5
    w = rng.standard_normal(24)
    b = rng.standard_normal(24)
    ref = F.layer_norm(torch.from_numpy(x), (24,), torch.from_numpy(w), torch.from_numpy(b), 1e-5)
    got = pair_ops.layer_norm(x, w, b, 1e-5)
    np.testing.assert_allclose(got, ref.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(brute.layer_norm(x, w, b, 1e-5), got, rtol=0, atol=1e-12)


# -------------------------------------------------------------- contraction
@pytest.mark.parametrize("outgoing", [True, False])
def test_contract_matches_einsum(outgoing):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((2, 9, 9, 5))
    b = rng.standard_normal((2, 9, 9, 5))
    eq = "bikc,bjkc->bijc" if outgoing else "bkic,bkjc->bijc"
    ref = torch.einsum(eq, torch.from_numpy(a), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(pair_ops.contract(a, b, outgoing), ref, atol=1e-12)
    rows = [0, 4, 8]
    np.testing.assert_allclose(pair_ops.contract(a, b, outgoing, rows), ref[:, rows], atol=1e-12)


# ------------------------------------------------------------------ tri-mul
@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_matches_loops(outgoing):
    P = _tm_params()
    z = H.pair_input(2, 6, 16, seed=4).astype(F64)
    m = _partial_mask(2, 6)
    ref = brute.tri_mul(z, m, P, outgoing)
    got = pair_ops.tri_mul(z, m, P, outgoing, dtype=F64)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-11)
    rows = [1, 5]
    got_r = pair_ops.tri_mul(z, m, P, outgoing, dtype=F64, rows=rows)
    np.testing.assert_allclose(got_r, ref[:, rows], rtol=0, atol=1e-11)


def test_tri_mul_incoming_is_transposed_outgoing():
    P = _tm_params(seed=5)
    swapped = dict(P)
    for part in ("weight", "bias"):
        swapped[f"linear_a_p.{part}"], swapped[f"linear_b_p.{part}"] = P[f"linear_b_p.{part}"], P[f"linear_a_p.{part}"]
        swapped[f"linear_a_g.{part}"], swapped[f"linear_b_g.{part}"] = P[f"linear_b_g.{part}"], P[f"linear_a_g.{part}"]
    z = H.pair_input(1, 10, 16, seed=6).astype(F64)
    m = _partial_mask(1, 10, seed=7)
    inc = pair_ops.tri_mul(z, m, P, False, dtype=F64)
    out_t = pair_ops.tri_mul(z.swapaxes(1, 2), m.swapaxes(1, 2), swapped, True, dtype=F64)
    np.testing.assert_allclose(inc, out_t.swapaxes(1, 2), atol=1e-11)


def test_tri_mul_closed_forms():
    cz, c = 16, 8
    z = H.pair_input(1, 8, cz, seed=8).astype(F64)
    # default init of the reference: linear_z is zero ("final") -> exactly zero output
    P = _tm_params(cz, c, seed=9)
    P["linear_z.weight"][:] = 0
    P["linear_z.bias"][:] = 0
    assert np.all(pair_ops.tri_mul(z, None, P, True, dtype=F64) == 0)
    # gating init (W_g = 0, b_g = 1) and constant output bias -> t * sigmoid(1)
    P = _tm_params(cz, c, seed=10)
    P["linear_z.weight"][:] = 0
    P["linear_z.bias"][:] = np.linspace(-1, 1, cz)
    P["linear_g.weight"][:] = 0
    P["linear_g.bias"][:] = 1
    got = pair_ops.tri_mul(z, None, P, False, dtype=F64)
    np.testing.assert_allclose(got, np.broadcast_to(P["linear_z.bias"] * 0.7310585786300049, got.shape),
                               atol=1e-12)
    # padded rows (mask 0 for i >= L): x = 0 -> LN_out(0) = beta_out
    P = _tm_params(cz, c, seed=11)
    L = 5
    m = H.tail_mask(1, 8, [L])
    got = pair_ops.tri_mul(z, m, P, True, dtype=F64)
    zn = pair_ops.layer_norm(z, P["layer_norm_in.weight"].astype(F64), P["layer_norm_in.bias"].astype(F64))
    gate = pair_ops.sigmoid(zn @ P["linear_g.weight"].T.astype(F64) + P["linear_g.bias"])
    const = P["linear_z.weight"].astype(F64) @ P["layer_norm_out.bias"] + P["linear_z.bias"]
    np.testing.assert_allclose(got[0, L:], (const * gate)[0, L:], atol=1e-10)


# ----------------------------------------------------------------- tri-attn
@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_matches_loops(starting):
    P = _ta_params()
    x = H.pair_input(2, 6, 16, seed=12).astype(F64)
    m = _partial_mask(2, 6, seed=13)
    m[0, 2, :] = 0  # a row (starting) / column (ending) with every key masked
    m[1, :, 3] = 0
    ref = brute.tri_attn(x, m, P, starting, 2)
    got = pair_ops.tri_attn(x, m, P, starting, 2, dtype=F64)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-11)
    rows = [0, 2, 5]
    got_r = pair_ops.tri_attn(x, m, P, starting, 2, dtype=F64, rows=rows)
    sel = ref[:, rows] if starting else ref[:, :, rows]
    np.testing.assert_allclose(got_r, sel, rtol=0, atol=1e-11)


def test_tri_attn_ending_is_transposed_starting():
    P = _ta_params(seed=14)
    x = H.pair_input(1, 9, 16, seed=15).astype(F64)
    m = _partial_mask(1, 9, seed=16)
    end = pair_ops.tri_attn(x, m, P, False, 2, dtype=F64)
    start_t = pair_ops.tri_attn(x.swapaxes(1, 2), m.swapaxes(1, 2), P, True, 2, dtype=F64)
    np.testing.assert_allclose(end, start_t.swapaxes(1, 2), atol=1e-12)


def test_tri_attn_fully_masked_row_is_uniform():
    P = _ta_params(seed=17)
    N, cin, ch, nh = 7, 16, 8, 2
    x = H.pair_input(1, N, cin, seed=18).astype(F64)
    m = np.ones((1, N, N), np.float32)
    m[0, 4, :] = 0
    for dt in (F64, np.float32):
        got = pair_ops.tri_attn(x, m, P, True, nh, dtype=dt)
        xn = pair_ops.layer_norm(x[0, 4], P["layer_norm.weight"].astype(F64), P["layer_norm.bias"].astype(F64))
        v = xn @ P["mha.linear_v.weight"].T.astype(F64)
        o = np.broadcast_to(v.mean(axis=0), (N, ch))
        o = o * pair_ops.sigmoid(xn @ P["mha.linear_g.weight"].T.astype(F64) + P["mha.linear_g.bias"])
        want = o @ P["mha.linear_o.weight"].T.astype(F64) + P["mha.linear_o.bias"]
        np.testing.assert_allclose(got[0, 4], want, atol=1e-5 if dt == np.float32 else 1e-12)


def _head_constant_params(const: float, seed: int):
    """Small tri-attn parameters whose triangle bias carries the per-head
    constant `const`: channels 8..15 are the constant const/8 after the
    LayerNorm (weight 0, bias const/8) and feed only the bias (weight 1
    there, no q/k/v/gate weight); channels 0..7 form an ordinary module."""
    P = _ta_params(seed=seed)
    hi = slice(8, 16)
    P["layer_norm.weight"][hi] = 0.0
    P["layer_norm.bias"][hi] = const / 8
    P["linear.weight"][:, hi] = 1.0
    for k in ("mha.linear_q.weight", "mha.linear_k.weight", "mha.linear_v.weight", "mha.linear_g.weight"):
        P[k][:, hi] = 0.0
    return P


@pytest.mark.parametrize("const,uniform", [(200.0, True), (224.0, False)])
def test_fully_masked_row_with_bias_constant(const, uniform):
    """A row whose keys are all masked (inf = 1e9) under a triangle bias with
    a per-head constant.  The fp32 reference's scores fl32(fl32(qk - 1e9) +
    tri) are -1e9 plus multiples of 64.  A constant of 200 (bias values
    200 +- 1) rounds every score of the row to -1e9 + 192: uniform, as with
    no constant.  224 sits on a rounding boundary: keys with tri > 224 take
    -1e9 + 256 and all the weight.  The float64 oracle and the scalar loops
    model both roundings and match the literal fp32 arithmetic."""
    P = _head_constant_params(const, seed=47)
    N = 7
    x = H.pair_input(1, N, 16, seed=48).astype(F64)
    m = np.ones((1, N, N), np.float32)
    m[0, 4, :] = 0
    xn = pair_ops.layer_norm(x[0, 4], P["layer_norm.weight"].astype(F64), P["layer_norm.bias"].astype(F64))
    tri = xn @ P["linear.weight"].T.astype(F64)  # [K, H] of row 4
    assert np.abs(tri - const).max() < 8
    if not uniform:  # the precondition of the split: bias values on both sides of 224
        assert (tri > 224).any() and (tri < 224).any()
    got = pair_ops.tri_attn(x, m, P, True, 2, dtype=F64)
    np.testing.assert_allclose(brute.tri_attn(x, m, P, True, 2), got, rtol=0, atol=1e-11)
    np.testing.assert_allclose(pair_ops.tri_attn(x, m, P, True, 2, dtype=np.float32), got,
                               rtol=0, atol=2e-5)
    v = xn @ P["mha.linear_v.weight"].T.astype(F64)
    o = np.broadcast_to(v.mean(axis=0), (N, 8))
    o = o * pair_ops.sigmoid(xn @ P["mha.linear_g.weight"].T.astype(F64) + P["mha.linear_g.bias"])
    want = o @ P["mha.linear_o.weight"].T.astype(F64) + P["mha.linear_o.bias"]
    if uniform:
        np.testing.assert_allclose(got[0, 4], want, atol=1e-12)
    else:
        assert np.abs(got[0, 4] - want).max() > 1e-2
    # rows with a valid key do not see the constant: softmax cancels it
    np.testing.assert_allclose(np.delete(got[0], 4, axis=0),
                               np.delete(pair_ops.tri_attn(x, m, _head_constant_params(0.0, 47), True, 2,
                                                           dtype=F64)[0], 4, axis=0), atol=1e-9)


@pytest.mark.parametrize("starting", [True, False])
def test_attention_core_matches_sdpa(starting):
    rng = np.random.default_rng(19)
    B, Hh, N, D = 1, 3, 8, 4
    q, k, v = (rng.standard_normal((B, Hh, N, N, D)) for _ in range(3))
    bias = rng.standard_normal((B, Hh, N, N))
    m = _partial_mask(B, N, seed=20)
    m[:, :, 0] = 1  # every row keeps a valid key
    m[:, 0, :] = 1
    scale = 0.37
    got = pair_ops.attention_core(q, k, v, bias, m, scale, starting, dtype=F64)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    qq, kk, vv, mm = (q, k, v, m) if starting else (q.swapaxes(2, 3), k.swapaxes(2, 3), v.swapaxes(2, 3), m.swapaxes(1, 2))
    # rows -> batch: [B, H, R, N, D] -> [B, R, H, N, D]
    qq, kk, vv = (t(a).transpose(1, 2) for a in (qq, kk, vv))
    addm = t(1e9 * (mm - 1))[:, :, None, None, :] + t(bias)[:, None]
    o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=addm, scale=scale)  # [B, R, H, N, D]
    want = o.transpose(2, 3).reshape(B, N, N, Hh * D).numpy()
    if not starting:
        want = want.swapaxes(1, 2)
    np.testing.assert_allclose(got, want, atol=1e-10)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("inf", [2.5, 30.0, 1e4])
def test_tri_attn_general_inf_and_fractional_mask(starting, inf):
    """The mask bias inf * (mask - 1) with a non-default inf and fractional mask
    values, where the reference's sum does not absorb: pair_ops (float64)
    against the scalar loops and against SDPA with the additive mask
    inf * (m - 1) + tri, in float64 (no fp32 absorption anywhere)."""
    P = _ta_params(seed=40)
    N, nh = 7, 2
    x = H.pair_input(2, N, 16, seed=41).astype(F64)
    m = _partial_mask(2, N, seed=42)
    m[0, 1, :] = 0            # every key masked
    m[1, 2, :3] = 0.5         # fractional values
    m[1, 4, :] = 0.25         # every key fractional
    m = m if starting else m.swapaxes(1, 2).copy()
    got = pair_ops.tri_attn(x, m, P, starting, nh, inf=inf, dtype=F64)
    np.testing.assert_allclose(brute.tri_attn(x, m, P, starting, nh, inf=inf), got, rtol=0, atol=1e-11)
    # the same through torch: LN, projections, SDPA with the additive mask
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=F64))  # noqa: E731
    xs, ms = (x, m) if starting else (x.swapaxes(1, 2), m.swapaxes(1, 2))
    xn = F.layer_norm(t(xs), (16,), t(P["layer_norm.weight"]), t(P["layer_norm.bias"]), 1e-5)
    tri = F.linear(xn, t(P["linear.weight"])).permute(0, 3, 1, 2)           # [B, H, Q, K]
    heads = lambda a: a.reshape(2, N, N, nh, 4).permute(0, 1, 3, 2, 4)     # noqa: E731 [B, I, H, J, d]
    q, k, v = (heads(F.linear(xn, t(P[f"mha.linear_{n}.weight"]))) for n in "qkv")
    addm = inf * (t(ms) - 1)[:, :, None, None, :] + tri[:, None]
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=addm, scale=0.5)  # d = 4
    o = o.permute(0, 1, 3, 2, 4).reshape(2, N, N, 8)
    o = o * torch.sigmoid(F.linear(xn, t(P["mha.linear_g.weight"]), t(P["mha.linear_g.bias"])))
    want = F.linear(o, t(P["mha.linear_o.weight"]), t(P["mha.linear_o.bias"])).numpy()
    if not starting:
        want = want.swapaxes(1, 2)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-10)
    # float32 literal arithmetic stays within the fp32 rounding of s - inf
    got32 = pair_ops.tri_attn(x, m, P, starting, nh, inf=inf, dtype=np.float32)
    np.testing.assert_allclose(got32, got, rtol=0, atol=4e-3 if inf > 100 else 1e-4)


def test_fractional_mask_absorbed_default_inf():
    """inf = 1e9 with fractional mask values: float64 uses the fp32-absorbed
    score of every key with mask != 1; the float32 literal reference agrees,
    also for a row whose keys are all fractional (the largest mask wins)."""
    P = _ta_params(seed=43)
    N = 6
    x = H.pair_input(1, N, 16, seed=44).astype(F64)
    m = np.ones((1, N, N), np.float32)
    m[0, 0, :2] = 0.5
    m[0, 3, :] = 0.0
    m[0, 3, 4] = 0.75         # row 3: every key masked, key 4 the least
    got = pair_ops.tri_attn(x, m, P, True, 2, dtype=F64)
    np.testing.assert_allclose(brute.tri_attn(x, m, P, True, 2), got, rtol=0, atol=1e-11)
    np.testing.assert_allclose(pair_ops.tri_attn(x, m, P, True, 2, dtype=np.float32), got,
                               rtol=0, atol=1e-5)
    # row 3 attends only to key 4: its output is that key's value path
    xn = pair_ops.layer_norm(x[0, 3], P["layer_norm.weight"].astype(F64), P["layer_norm.bias"].astype(F64))
    v = xn @ P["mha.linear_v.weight"].T.astype(F64)
    o = np.broadcast_to(v[4], (N, 8)) * pair_ops.sigmoid(
        xn @ P["mha.linear_g.weight"].T.astype(F64) + P["mha.linear_g.bias"])
    np.testing.assert_allclose(got[0, 3], o @ P["mha.linear_o.weight"].T.astype(F64) + P["mha.linear_o.bias"],
                               atol=1e-12)


# ------------------------------------------------------- pair transition
def test_pair_transition_matches_torch_and_loops():
    """PairTransition (pair_transform.py:79-84): LayerNorm, linear_1, ReLU,
    linear_2, against torch.nn.functional in float64 and the scalar loops."""
    P = H.draw_params(H.pair_transition_shapes(16, 4), seed=45, ln_random=True, bias_random=True)
    p = H.pair_input(2, 5, 16, seed=46).astype(F64) * 1.5 + 0.2
    got = pair_ops.pair_transition(p, P, dtype=F64)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=F64))  # noqa: E731
    h = F.linear(F.layer_norm(t(p), (16,), t(P["layer_norm.weight"]), t(P["layer_norm.bias"]), 1e-5),
                 t(P["linear_1.weight"]), t(P["linear_1.bias"]))
    want = F.linear(F.relu(h), t(P["linear_2.weight"]), t(P["linear_2.bias"])).numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    np.testing.assert_allclose(brute.pair_transition(p, P), got, rtol=0, atol=1e-12)
    # a good share of the hidden units is clipped by the ReLU, so dropping it shows
    assert (h.numpy() < 0).mean() > 0.2


def test_pair_block_matches_loops():
    """PairTransformLayer in eval (pair_transform.py:180-193): the four
    residual updates, the transition and the final mask, against the scalar
    loops' composition, with a ragged mask (a row and a column fully masked)."""
    P = H.draw_params(H.pair_layer_shapes(16, 8, 8, 2), seed=47, ln_random=True, bias_random=True)
    p = H.pair_input(1, 5, 16, seed=48).astype(F64)
    m = H.tail_mask(1, 5, [4])
    got = pair_ops.pair_block(p, m, P, 2, dtype=F64)
    np.testing.assert_allclose(brute.pair_block(p, m, P, 2), got, rtol=0, atol=1e-10)
    assert np.all(got[0, 4] == 0) and np.all(got[0, :, 4] == 0)
    assert np.abs(got[0, :4, :4]).min() > 0


# ------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_detected(monkeypatch):
    """A transposed contraction operand, a dropped mask bias and a gate taken from
    the raw input each break one of the pins above."""
    P = _tm_params()
    z = H.pair_input(1, 5, 16, seed=21).astype(F64)
    m = _partial_mask(1, 5, seed=22)
    ref = brute.tri_mul(z, m, P, True)

    orig_contract = pair_ops.contract
    monkeypatch.setattr(pair_ops, "contract", lambda a, b, o, rows=None: orig_contract(b, a, o, rows))
    assert np.abs(pair_ops.tri_mul(z, m, P, True, dtype=F64) - ref).max() > 1e-3
    monkeypatch.undo()

    orig_ln = pair_ops.layer_norm
    calls = {"n": 0}

    def ln_skip_first(x, w, b, eps=1e-5):  # LN_in dropped: gate and projections see raw z
        calls["n"] += 1
        return x if calls["n"] == 1 else orig_ln(x, w, b, eps)

    monkeypatch.setattr(pair_ops, "layer_norm", ln_skip_first)
    assert np.abs(pair_ops.tri_mul(z, m, P, True, dtype=F64) - ref).max() > 1e-3
    monkeypatch.undo()

    PA = _ta_params()
    x = H.pair_input(1, 5, 16, seed=23).astype(F64)
    ma = _partial_mask(1, 5, seed=24)
    ref_a = brute.tri_attn(x, ma, PA, True, 2)
    monkeypatch.setattr(pair_ops, "_masked_scores", lambda qk, km, tri, inf, dt: qk + tri)
    assert np.abs(pair_ops.tri_attn(x, ma, PA, True, 2, dtype=F64) - ref_a).max() > 1e-3
    monkeypatch.undo()

    # transition: the ReLU dropped, or the residual order changed
    PT = H.draw_params(H.pair_transition_shapes(16, 4), seed=49, ln_random=True, bias_random=True)
    pt = H.pair_input(1, 4, 16, seed=50).astype(F64)
    ref_t = brute.pair_transition(pt, PT)
    monkeypatch.setattr(pair_ops.np, "maximum", lambda a, b: a)
    assert np.abs(pair_ops.pair_transition(pt, PT, dtype=F64) - ref_t).max() > 1e-3
    monkeypatch.undo()
    PB = H.draw_params(H.pair_layer_shapes(16, 8, 8, 2), seed=51, ln_random=True, bias_random=True)
    pb = H.pair_input(1, 4, 16, seed=52).astype(F64)
    mb = H.tail_mask(1, 4, [3])
    ref_b = brute.pair_block(pb, mb, PB, 2)
    orig_tm = pair_ops.tri_mul
    monkeypatch.setattr(pair_ops, "tri_mul", lambda z, m, P, o, dt=np.float32, *a, **k: orig_tm(z, m, P, not o, dt))
    assert np.abs(pair_ops.pair_block(pb, mb, PB, 2, dtype=F64) - ref_b).max() > 1e-3
