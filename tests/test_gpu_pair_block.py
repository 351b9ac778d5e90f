"""GPU parity of the pair-stack block on the kernels: the fused PairTransition
kernel (pair_transform.py:64-84) alone and with the layer's residual and mask
(:180-193), its fp32 kernel and its backward, and a whole PairTransformLayer
(eval mode) whose four triangle operators run with the residual add fused into
their kernels.
bf16 tolerance per operator: |y - y_ref| <= 2e-2 + 1e-2 |y_ref| against the fp32
oracle on bf16-rounded inputs and weights; fp32: max abs error <= 1e-4 against
the float64 oracle.  Gradients: the tolerances of test_gpu_grads."""
import numpy as np
import pytest
import torch

from genie_tk import PairTransformLayer
from genie_tk.pair_transform import PairTransition
from oracle import grads, pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, check_fp32, log, to_np
from tests.test_gpu_grads import _check_grad

pytestmark = pytest.mark.gpu


def _dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


@pytest.mark.parametrize("c", [128, 64])
def test_pair_transition_kernel(c):
    log(f"pair transition kernel c={c}")
    P = H.bf16_params(H.draw_params(H.pair_transition_shapes(c), 70 + c, ln_random=True, bias_random=True))
    p = H.bf16_round(H.pair_input(2, 45, c, seed=c))  # 4050 rows: a ragged last tile and batch
    mod = PairTransition(c, 4)
    mod.load_state_dict(H.to_state_dict(P))
    mod = mod.to("cuda", torch.bfloat16).eval()
    pt = _dev(p)
    with torch.no_grad():
        assert mod._use_kernel(pt)
        y = mod(pt)
        m = H.tail_mask(2, 45, [45, 31])
        m[1, 3, 5] = 0.5  # a fractional mask value is applied as a factor
        y2 = mod.forward_residual_masked(pt, _dev(m, torch.float32))
    ref = pair_ops.pair_transition(p, P)
    check_bf16(to_np(y), ref, f"pair transition c={c}")
    check_bf16(to_np(y2), (p + ref) * m[..., None], f"pair transition residual+mask c={c}")


@pytest.mark.parametrize("c", [128, 64])
def test_pair_transition_fp32_kernel(c):
    """The fp32 kernel (generic: one wave per 32-row tile) against the float64
    oracle, alone and with the layer's residual and a fractional mask."""
    log(f"pair transition fp32 kernel c={c}")
    P = H.draw_params(H.pair_transition_shapes(c), 80 + c, ln_random=True, bias_random=True)
    p = H.pair_input(2, 45, c, seed=c + 1)
    mod = PairTransition(c, 4)
    mod.load_state_dict(H.to_state_dict(P))
    mod = mod.to("cuda").eval()
    mod._forward_pytorch = lambda *a, **k: (_ for _ in ()).throw(AssertionError("PyTorch path"))
    pt = _dev(p, torch.float32)
    m = H.tail_mask(2, 45, [45, 31])
    m[1, 3, 5] = 0.5
    with torch.no_grad():
        y = mod(pt)
        y2 = mod.forward_residual_masked(pt, _dev(m, torch.float32))
    ref = pair_ops.pair_transition(p, P, dtype=np.float64)
    check_fp32(to_np(y), ref, f"pair transition fp32 c={c}")
    check_fp32(to_np(y2), (p + ref) * m[..., None], f"pair transition fp32 residual+mask c={c}")


def _hidden(p, P, bf16: bool, eps=1e-5):
    """The pre-activation h of linear_1 in float64; with bf16, formed as the
    bf16 kernels form it: bf16(x_hat) against bf16(W1 diag(gamma)), plus
    b1 + W1 beta."""
    x = p.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    xh = (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
    w1 = P["linear_1.weight"].astype(np.float64)
    g, b = P["layer_norm.weight"].astype(np.float64), P["layer_norm.bias"].astype(np.float64)
    if not bf16:
        return (xh * g + b) @ w1.T + P["linear_1.bias"]
    return H.bf16_round(xh.astype(np.float32)).astype(np.float64) @ H.bf16_round(
        (w1 * g).astype(np.float32)).astype(np.float64).T + (P["linear_1.bias"] + w1 @ b)


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("c", [128, 64])
def test_pair_transition_backward(dname, c):
    """Training through the kernels: dL/dp and every parameter gradient of
    PairTransition against the float64 gradient oracle (oracle/grads.py,
    pinned by finite differences and torch autograd), 4050 rows (a ragged
    last tile); the PyTorch path is made to raise.

    The ReLU's derivative jumps at 0: a hidden unit whose h lies within
    rounding distance of 0 passes its gradient in one computation and not in
    the other.  So rows with some |h| < 1e-4 get dy = 0 (their gradients are
    then exactly 0 everywhere), and for bf16 the oracle takes the pass pattern
    of h as the bf16 kernels form it (x_hat and W1 diag(gamma) in bf16)."""
    log(f"pair transition backward {dname} c={c}")
    dt = torch.bfloat16 if dname == "bf16" else torch.float32
    P = H.draw_params(H.pair_transition_shapes(c), 90 + c, ln_random=True, bias_random=True)
    p = H.pair_input(2, 45, c, seed=c + 2)
    dy = np.random.default_rng(c + 3).standard_normal(p.shape).astype(np.float32)
    if dname == "bf16":
        P, p, dy = H.bf16_params(P), H.bf16_round(p), H.bf16_round(dy)
    h = _hidden(p, P, dname == "bf16")
    ambiguous = (np.abs(h) < 1e-4).any(axis=-1)
    dy[ambiguous] = 0.0
    log(f"  {ambiguous.sum()} of {ambiguous.size} rows with |h| < 1e-4 take dy = 0")
    mod = PairTransition(c, 4)
    mod.load_state_dict(H.to_state_dict(P))
    mod = mod.to("cuda", dt)
    mod._forward_pytorch = lambda *a, **k: (_ for _ in ()).throw(AssertionError("PyTorch path"))
    pt = _dev(p, dt).requires_grad_(True)
    y = mod(pt)
    y.backward(_dev(dy, dt))
    torch.cuda.synchronize()
    check = check_fp32 if dname == "fp32" else check_bf16
    ref_y = pair_ops.pair_transition(p, P, dtype=np.float64 if dname == "fp32" else np.float32)
    check(to_np(y), ref_y, f"pair transition forward under autograd {dname} c={c}")
    gate = h > 0 if dname == "bf16" else None
    dp_ref, g_ref = grads.pair_transition_grad(p, P, dy, gate=gate)
    worst = [(_check_grad(to_np(pt.grad), dp_ref, dname, "dp"), "dp")]
    for name, prm in mod.named_parameters():
        assert prm.grad is not None and prm.grad.dtype == dt, name
        worst.append((_check_grad(to_np(prm.grad), g_ref[name], dname, name), name))
    log(f"  worst max|g - r| / max|r|: {max(worst)[0]:.2e} ({max(worst)[1]})")


def test_pair_layer_kernel_path():
    """One PairTransformLayer (eval) on the kernels vs the oracle's block.  The
    layer composes five bf16 operators over a bf16 residual stream, so the check
    allows 2.5x the per-operator tolerance."""
    log("pair layer kernel path B=2 N=64")
    B, N, c = 2, 64, 128
    P = H.bf16_params(H.draw_params(H.pair_layer_shapes(c, 128, 128, 4), 90, ln_random=True,
                                    bias_random=True, tri_std=1.0 / np.sqrt(128)))
    layer = PairTransformLayer(c_p=c, c_hidden_mul=128, c_hidden_tri_att=128, n_head_tri=4,
                               tri_dropout=0.25)
    layer.load_state_dict(H.to_state_dict(P))
    layer = layer.to("cuda", torch.bfloat16).eval()
    p = H.bf16_round(H.pair_input(B, N, c, seed=91))
    m = H.tail_mask(B, N, [N, 50])
    with torch.no_grad():
        out, _ = layer((_dev(p), _dev(m, torch.float32)))
    ref = pair_ops.pair_block(p, m, P, 4, dtype=np.float32)
    got = to_np(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    bound = 2.5 * (2e-2 + 1e-2 * np.abs(ref))
    log(f"pair layer: max abs err {err.max():.3e}, worst err/bound {(err / bound).max():.2f}")
    assert (err <= bound).all(), f"pair layer: max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"
    assert np.all(got[1, 50:] == 0) and np.all(got[1, :, 50:] == 0)  # masked pairs are zero


@pytest.mark.parametrize("c,c_mul,c_att,heads", [(128, 128, 32, 4), (64, 32, 16, 2)])
def test_pair_layer_reference_shapes(c, c_mul, c_att, heads, monkeypatch):
    """The reference layer's default shape (c_hidden_tri_att=32 with 4 heads:
    head dim 8; pair_transform.py:116-117) and its test's small shape
    (tests/test_triangle_attention.py:131-136: c_hidden_mul=32,
    c_hidden_tri_att=16, head dim 8 over 2 heads) run every triangle operator
    on the kernels (their PyTorch paths are made to raise) and match the
    oracle's block."""
    log(f"pair layer reference shape c={c} c_mul={c_mul} c_att={c_att} heads={heads}")
    B, N = 2, 40
    P = H.bf16_params(H.draw_params(H.pair_layer_shapes(c, c_mul, c_att, heads), 92 + c,
                                    ln_random=True, bias_random=True,
                                    tri_std=1.0 / np.sqrt(c)))
    layer = PairTransformLayer(c_p=c, c_hidden_mul=c_mul, c_hidden_tri_att=c_att, n_head_tri=heads,
                               tri_dropout=0.25)
    layer.load_state_dict(H.to_state_dict(P))
    layer = layer.to("cuda", torch.bfloat16).eval()
    for name in ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end"):
        monkeypatch.setattr(getattr(layer, name), "_forward_pytorch",
                            lambda *a, **k: (_ for _ in ()).throw(AssertionError("PyTorch path")))
    p = H.bf16_round(H.pair_input(B, N, c, seed=93))
    m = H.tail_mask(B, N, [N, 33])
    with torch.no_grad():
        out, _ = layer((_dev(p), _dev(m, torch.float32)))
    ref = pair_ops.pair_block(p, m, P, heads, dtype=np.float32)
    got = to_np(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    bound = 2.5 * (2e-2 + 1e-2 * np.abs(ref))
    log(f"  max abs err {err.max():.3e}, worst err/bound {(err / bound).max():.2f}")
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"
