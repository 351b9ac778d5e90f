"""Pins of the backward oracle (oracle/grads.py) — CPU only.

* Every gradient (input and each parameter, every element) against central
  finite differences of the float64 forward oracle on tiny shapes.  A wrong
  sign, a dropped term, a transposed contraction operand or a gradient routed
  to the wrong parameter fails here.
* The same gradients against torch autograd of the genie_tk PyTorch path in
  float64, a second, independent derivation of the reference's graph.
* A planted mistake in a copy of the backward (the incoming contraction's
  operands swapped) is caught by the finite differences.
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
