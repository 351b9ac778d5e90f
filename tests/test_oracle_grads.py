"""Pins of the backward oracle (oracle/grads.py) — CPU only.

* Every gradient (input and each parameter, every element) against central
  finite differences of the float64 forward oracle on tiny shapes.  A wrong
  sign, a dropped term, a transposed contraction operand or a gradient routed
  to the wrong parameter fails here.
* The same gradients against torch autograd of the genie_tk PyTorch path in
  float64, a second, independent derivation of the reference's graph.
* A planted mistake in a copy of the backward (the incoming contraction's
  operands swapped) is caught by the finite differences.
* PairTransition (pair_transform.py:79-84): the same two pins, and a
  dropped ReLU gate in the backward is caught.
"""
import numpy as np
import pytest
import torch

from oracle import grads, pair_ops
from tests import helpers as H

F64 = np.float64


def _fd_check(f, x, analytic, h=1e-6, tol=1e-6):
    """Central differences of the scalar function f at every element of x."""
    x = x.copy()
    flat = x.reshape(-1)
    num = np.empty_like(flat)
    for idx in range(flat.size):
        old = flat[idx]
        flat[idx] = old + h
        fp = f(x)
        flat[idx] = old - h
        fm = f(x)
        flat[idx] = old
        num[idx] = (fp - fm) / (2 * h)
    num = num.reshape(x.shape)
    scale = max(1.0, np.abs(num).max())
    err = np.abs(num - analytic).max() / scale
    assert err < tol, f"finite-difference mismatch {err:.3e}"


def _tri_mul_case(outgoing, seed=0):
    P = H.draw_params(H.tri_mul_shapes(6, 4), seed, ln_random=True, bias_random=True)
    P = {k: v.astype(F64) for k, v in P.items()}
    z = H.pair_input(2, 4, 6, seed + 1).astype(F64)
    mask = H.tail_mask(2, 4, [4, 3])
    dy = np.random.default_rng(seed + 2).standard_normal(z.shape)
    return P, z, mask, dy


@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_grad_finite_differences(outgoing):
    P, z, mask, dy = _tri_mul_case(outgoing)
    dz, g = grads.tri_mul_grad(z, mask, P, outgoing, dy)
    loss = lambda zz, PP: float((pair_ops.tri_mul(zz, mask, PP, outgoing, dtype=F64) * dy).sum())  # noqa: E731
    _fd_check(lambda zz: loss(zz, P), z, dz)
    assert set(g) == set(P)
    for key in P:
        def f(v, key=key):
            PP = dict(P)
            PP[key] = v
            return loss(z, PP)
        _fd_check(f, P[key], g[key])


@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_grad_matches_torch_autograd(outgoing):
    from genie_tk import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    P = H.draw_params(H.tri_mul_shapes(16, 8), 3, ln_random=True, bias_random=True)
    z = H.pair_input(2, 7, 16, 4)
    mask = H.tail_mask(2, 7, [7, 5])
    dy = np.random.default_rng(5).standard_normal(z.shape)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = cls(16, 8, use_fused_kernel=False).double()
    mod.load_state_dict(H.to_state_dict(P, dtype=torch.float64))
    zt = torch.from_numpy(z.astype(F64)).requires_grad_(True)
    y = mod(zt, torch.from_numpy(mask).double())
    (y * torch.from_numpy(dy)).sum().backward()
    dz, g = grads.tri_mul_grad(z, mask, P, outgoing, dy)
    np.testing.assert_allclose(zt.grad.numpy(), dz, rtol=1e-9, atol=1e-10)
    for name, prm in mod.named_parameters():
        np.testing.assert_allclose(prm.grad.numpy(), g[name], rtol=1e-9, atol=1e-10, err_msg=name)


def test_planted_contraction_mistake_is_caught():
    P, z, mask, dy = _tri_mul_case(False, seed=7)

    orig = grads.contract_bwd

    def wrong_bwd(a, b, dx, outgoing):
        return orig(a, b, dx, not outgoing)

    grads.contract_bwd = wrong_bwd
    try:
        dz, _ = grads.tri_mul_grad(z, mask, P, False, dy)
    finally:
        grads.contract_bwd = orig
    with pytest.raises(AssertionError):
        _fd_check(lambda zz: float((pair_ops.tri_mul(zz, mask, P, False, dtype=F64) * dy).sum()), z, dz)


def _tri_attn_case(seed=0, B=2, N=4, C=6, ch=4, H=2):
    P = H_.draw_params(H_.tri_attn_shapes(C, ch, H), seed, ln_random=True, bias_random=True)
    P = {k: v.astype(F64) for k, v in P.items()}
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((B, N, N, C))
    # every row keeps at least one key (the diagonal), some keys masked
    mask = (rng.random((B, N, N)) > 0.3).astype(np.float32)
    mask[:, np.arange(N), np.arange(N)] = 1.0
    dy = rng.standard_normal(x.shape)
    return P, x, mask, dy


H_ = H


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_grad_finite_differences(starting):
    P, x, mask, dy = _tri_attn_case()
    dx, g = grads.tri_attn_grad(x, mask, P, starting, 2, dy)
    loss = lambda xx, PP: float((pair_ops.tri_attn(xx, mask, PP, starting, 2, dtype=F64) * dy).sum())  # noqa: E731
    _fd_check(lambda xx: loss(xx, P), x, dx)
    assert set(g) == set(P)
    for key in P:
        def f(v, key=key):
            PP = dict(P)
            PP[key] = v
            return loss(x, PP)
        _fd_check(f, P[key], g[key])


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_tri_attn_grad_matches_torch_autograd(starting, dtype):
    """float64 autograd without fully masked rows; float32 autograd with a
    tail mask, whose padded rows are fully masked: there the fp32 reference's
    scores absorb -inf and the softmax is uniform, and autograd still passes
    its gradient to q.k and the triangle bias (the oracle's convention)."""
    from genie_tk import TriangleAttentionEndingNode, TriangleAttentionStartingNode

    P = H.draw_params(H.tri_attn_shapes(16, 8, 2), 3, ln_random=True, bias_random=True)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 7, 7, 16))
    dy = rng.standard_normal(x.shape)
    if dtype == torch.float64:
        mask = (rng.random((2, 7, 7)) > 0.3).astype(np.float32)
        mask[:, np.arange(7), np.arange(7)] = 1.0
    else:
        mask = H.tail_mask(2, 7, [7, 4])
        x, dy = x.astype(np.float32), dy.astype(np.float32)
    cls = TriangleAttentionStartingNode if starting else TriangleAttentionEndingNode
    mod = cls(16, 8, 2, use_fused_kernel=False).to(dtype)
    mod.load_state_dict(H.to_state_dict(P, dtype=dtype))
    xt = torch.from_numpy(x).to(dtype).requires_grad_(True)
    y = mod(xt, torch.from_numpy(mask).to(dtype))
    (y * torch.from_numpy(dy).to(dtype)).sum().backward()
    dx, g = grads.tri_attn_grad(x, mask, P, starting, 2, dy)
    tol = dict(rtol=1e-9, atol=1e-10) if dtype == torch.float64 else dict(rtol=2e-4, atol=2e-4)
    np.testing.assert_allclose(xt.grad.double().numpy(), dx, **tol)
    for name, prm in mod.named_parameters():
        np.testing.assert_allclose(prm.grad.double().numpy(), g[name], err_msg=name, **tol)


def _pt_case(seed=0, c=6, n=4):
    P = H.draw_params(H.pair_transition_shapes(c, n), seed, ln_random=True, bias_random=True)
    P = {k: v.astype(F64) for k, v in P.items()}
    p = H.pair_input(2, 3, c, seed + 1).astype(F64) * 1.5 + 0.2
    dy = np.random.default_rng(seed + 2).standard_normal(p.shape)
    return P, p, dy


def test_pair_transition_grad_finite_differences():
    P, p, dy = _pt_case()
    dp, g = grads.pair_transition_grad(p, P, dy)
    loss = lambda pp, PP: float((pair_ops.pair_transition(pp, PP, dtype=F64) * dy).sum())  # noqa: E731
    _fd_check(lambda pp: loss(pp, P), p, dp)
    assert set(g) == set(P)
    for key in P:
        def f(v, key=key):
            PP = dict(P)
            PP[key] = v
            return loss(p, PP)
        _fd_check(f, P[key], g[key])


def test_pair_transition_grad_matches_torch_autograd():
    from genie_tk.pair_transform import PairTransition

    P = H.draw_params(H.pair_transition_shapes(16, 4), 8, ln_random=True, bias_random=True)
    p = H.pair_input(2, 5, 16, 9).astype(F64)
    dy = np.random.default_rng(10).standard_normal(p.shape)
    mod = PairTransition(16, 4, use_fused_kernel=False).double()
    mod.load_state_dict(H.to_state_dict(P, dtype=torch.float64))
    pt = torch.from_numpy(p).requires_grad_(True)
    (mod(pt) * torch.from_numpy(dy)).sum().backward()
    dp, g = grads.pair_transition_grad(p, P, dy)
    np.testing.assert_allclose(pt.grad.numpy(), dp, rtol=1e-9, atol=1e-10)
    for name, prm in mod.named_parameters():
        np.testing.assert_allclose(prm.grad.numpy(), g[name], rtol=1e-9, atol=1e-10, err_msg=name)


def test_planted_relu_gate_mistake_is_caught(monkeypatch):
    """The backward with the ReLU gate dropped (dh = da) fails the finite
    differences: the case has clipped hidden units."""
    P, p, dy = _pt_case(seed=11)
    xn = pair_ops.layer_norm(p, P["layer_norm.weight"], P["layer_norm.bias"])
    assert (xn @ P["linear_1.weight"].T + P["linear_1.bias"] < 0).mean() > 0.2
    monkeypatch.setattr(grads, "relu_bwd", lambda h, da: da)
    dp, _ = grads.pair_transition_grad(p, P, dy)
    monkeypatch.undo()
    with pytest.raises(AssertionError):
        _fd_check(lambda pp: float((pair_ops.pair_transition(pp, P, dtype=F64) * dy).sum()), p, dp)
