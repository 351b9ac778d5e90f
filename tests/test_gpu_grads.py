"""Backward kernels against the float64 backward oracle (oracle/grads.py).

The modules run forward on the kernels inside their autograd Function and
backward through genie_tk._C.*_backward (the C ABI's gtk_*_backward).  The
oracle is evaluated on the same (bf16-rounded, for bf16) inputs, parameters
and upstream gradient.

Tolerances, per gradient tensor g against the oracle's r:
  * fp32: max|g - r| <= 1e-4 * max(1, max|r|);
  * bf16: max|g - r| <= 3e-2 * max|r| and ||g - r||_2 <= 1e-2 * ||r||_2.  The
    bf16 backward rounds its intermediate planes (dX, dA, dB and the
    per-pair operands of the weight-gradient products) to bf16, so errors
    are relative to the tensor's scale rather than per element.  A tensor
    over the normwise bound passes if its error is at most 1.25 times that
    of the reference's bf16 computation on the same case (autograd of the
    module's PyTorch path, the reference's operation sequence op for op, in
    bf16 on the CPU): a bias gradient is a sum over
    every pair with cancellation, whose bf16 error can exceed 1e-2 of its
    norm in the reference too (the gate bias of one head of 8: 1.06e-2).
"""
import numpy as np
import pytest
import torch

from oracle import grads
from tests import helpers as H
from tests.gpu_common import log, triattn_module, trimul_module

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def _normwise(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def _check_grad(got: np.ndarray, ref: np.ndarray, dname: str, what: str, floor: float = 0.0) -> float:
    """Asserts the tolerance (``floor``: the reference bf16 path's normwise
    error on this tensor, when measured); returns max|g - r| / max|r|."""
    assert np.isfinite(got).all(), f"{what}: non-finite gradient"
    err = np.abs(got - ref)
    scale = np.abs(ref).max()
    if dname == "fp32":
        assert err.max() <= 1e-4 * max(1.0, scale), f"{what}: max err {err.max():.3e} (scale {scale:.3e})"
    else:
        rel = _normwise(got, ref)
        assert err.max() <= 3e-2 * scale, f"{what}: max err {err.max():.3e} > 3e-2 * {scale:.3e}"
        assert rel <= max(1e-2, 1.25 * floor), \
            f"{what}: normwise relative error {rel:.3e} (reference bf16 path: {floor:.3e})"
    return float(err.max() / max(scale, 1e-30))


def _reference_bf16_errors(module, P, x, m, dy, dx_ref, g_ref) -> dict:
    """Normwise errors of the reference's bf16 computation against the
    oracle: ``module`` is a fresh PyTorch-path module (the reference's
    operation sequence op for op), run with autograd in bf16 on the CPU."""
    module.load_state_dict(H.to_state_dict(P))
    module = module.bfloat16()
    xt = torch.from_numpy(x).bfloat16().requires_grad_(True)
    module(xt, torch.from_numpy(m)).backward(torch.from_numpy(dy).bfloat16())
    out = {"dx": _normwise(_np(xt.grad), dx_ref)}
    for name, prm in module.named_parameters():
        out[name] = _normwise(_np(prm.grad), g_ref[name])
    return out


def _check_all(dname, got: dict, refs: dict, reference_module) -> list:
    """Checks every gradient; for bf16 tensors over the fixed normwise bound,
    measures the reference bf16 path once (``reference_module()`` returns its
    errors) and allows 1.25 times its error."""
    floors = {}
    if dname == "bf16" and any(_normwise(got[k], refs[k]) > 1e-2 for k in got):
        floors = reference_module()
        log("  reference bf16 path normwise errors: "
            + ", ".join(f"{k} {v:.2e}" for k, v in floors.items() if _normwise(got[k], refs[k]) > 1e-2))
    return [(_check_grad(got[k], refs[k], dname, k, floors.get(k, 0.0)), k) for k in got]


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("N,c", [(64, 128), (37, 64), (130, 128), (100, 128)])
def test_tri_mul_backward(dname, outgoing, N, c):
    """N = 100 (planes of 128): the bf16 contraction backward reads the
    operands that enter transposed straight from the planes."""
    _tri_mul_backward_case(dname, outgoing, N, c)


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("B,N", [(1, 512), (2, 100)])
def test_tri_mul_backward_transposed_operands_bit_exact(monkeypatch, outgoing, B, N):
    """The contraction backward with the transposed operands read from the
    planes (256 x 256 tiles at N = 512, 128 x 128 at N = 100) gives the same
    bits as transposing the planes first (GENIE_TK_TRANSPOSE_PLANES=1): the
    same products are summed in the same order."""
    log(f"tri_mul backward transposed operands B={B} N={N} outgoing={outgoing}")
    P = H.bf16_params(H.draw_params(H.tri_mul_shapes(128, 128), seed=N + 3, ln_random=True,
                                    bias_random=True))
    z = H.bf16_round(H.pair_input(B, N, 128, seed=N + 4))
    m = H.tail_mask(B, N, [N - 9] * B)
    dy = H.bf16_round(H.pair_input(B, N, 128, seed=N + 5))
    mod = trimul_module(P, outgoing, torch.bfloat16)
    runs = []
    for force in ("0", "1"):
        monkeypatch.setenv("GENIE_TK_TRANSPOSE_PLANES", force)
        mod.zero_grad(set_to_none=True)
        zt = torch.from_numpy(z).to("cuda", torch.bfloat16).requires_grad_(True)
        y = mod(zt, torch.from_numpy(m).to("cuda"))
        y.backward(torch.from_numpy(dy).to("cuda", torch.bfloat16))
        torch.cuda.synchronize()
        g = {"dx": zt.grad.clone()}
        for name, prm in mod.named_parameters():
            g[name] = prm.grad.clone()
        runs.append(g)
    for name in runs[0]:
        assert torch.equal(runs[0][name], runs[1][name]), f"{name} differs between the two forms"


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("N", [64, 37])
def test_tri_mul_backward_element_paths(monkeypatch, outgoing, N):
    """bf16 through the element-pointer kernels, the path taken where the
    buffers' byte offsets exceed 32 bits (N above about 2900), selected here
    at a small N by GENIE_TK_ELEMENT_PATHS."""
    monkeypatch.setenv("GENIE_TK_ELEMENT_PATHS", "1")
    _tri_mul_backward_case("bf16", outgoing, N, 128)


def _tri_mul_backward_case(dname, outgoing, N, c):
    log(f"tri_mul backward {dname} outgoing={outgoing} N={N} c={c}")
    dt = DT[dname]
    P = H.draw_params(H.tri_mul_shapes(128, c), seed=N + c, ln_random=True, bias_random=True)
    z = H.pair_input(2, N, 128, seed=N + 1)
    m = H.tail_mask(2, N, [N, N - 5])
    dy = H.pair_input(2, N, 128, seed=N + 2)
    if dname == "bf16":
        P, z, dy = H.bf16_params(P), H.bf16_round(z), H.bf16_round(dy)
    mod = trimul_module(P, outgoing, dt)
    zt = torch.from_numpy(z).to("cuda", dt).requires_grad_(True)
    mt = torch.from_numpy(m).to("cuda")
    y = mod(zt, mt)
    y.backward(torch.from_numpy(dy).to("cuda", dt))
    torch.cuda.synchronize()
    dz_ref, g_ref = grads.tri_mul_grad(z, m, P, outgoing, dy)
    got, refs = {"dx": _np(zt.grad)}, {"dx": dz_ref}
    for name, prm in mod.named_parameters():
        assert prm.grad is not None and prm.grad.dtype == dt, name
        got[name], refs[name] = _np(prm.grad), g_ref[name]
    cls = type(mod)
    worst = _check_all(dname, got, refs, lambda: _reference_bf16_errors(
        cls(128, c, use_fused_kernel=False), P, z, m, dy, dz_ref, g_ref))
    log(f"  worst max|g - r| / max|r|: {max(worst)[0]:.2e} ({max(worst)[1]})")


def test_tri_mul_backward_runs_the_kernels(monkeypatch):
    """With gradients required, forward and backward go through the kernels
    (the PyTorch path is made to raise), for leading batch dimensions too."""
    P = H.draw_params(H.tri_mul_shapes(128, 128), seed=9, bias_random=True)
    mod = trimul_module(P, True, torch.bfloat16)
    monkeypatch.setattr(mod, "_forward_pytorch",
                        lambda *a, **k: (_ for _ in ()).throw(AssertionError("fallback")))
    z = torch.randn(2, 1, 40, 40, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = mod(z)
    y.float().square().sum().backward()
    assert z.grad is not None and z.grad.shape == z.shape and torch.isfinite(z.grad).all()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in mod.parameters())


def _tri_attn_backward_case(dname, starting, N, lengths, inner_mask=0.0, cin=128, ch=128, heads=4):
    log(f"tri_attn backward {dname} starting={starting} N={N} lengths={lengths} c_in={cin} c_h={ch} H={heads}")
    dt = DT[dname]
    B = len(lengths)
    P = H.draw_params(H.tri_attn_shapes(cin, ch, heads), seed=N + 7, ln_random=True, bias_random=True)
    x = H.pair_input(B, N, cin, seed=N + 8)
    m = H.tail_mask(B, N, lengths)
    if inner_mask > 0:
        # scattered masked pairs inside the valid block (no row loses every key)
        rng = np.random.default_rng(N)
        m = m * (rng.random(m.shape) >= inner_mask).astype(np.float32)
        m[:, np.arange(N), np.arange(N)] = H.tail_mask(B, N, lengths)[:, np.arange(N), np.arange(N)]
    dy = H.pair_input(B, N, cin, seed=N + 9)
    if dname == "bf16":
        P, x, dy = H.bf16_params(P), H.bf16_round(x), H.bf16_round(dy)
    mod = triattn_module(P, starting, heads, dt)
    mod._forward_pytorch = lambda *a, **k: (_ for _ in ()).throw(AssertionError("PyTorch path"))
    xt = torch.from_numpy(x).to("cuda", dt).requires_grad_(True)
    y = mod(xt, torch.from_numpy(m).to("cuda"))
    y.backward(torch.from_numpy(dy).to("cuda", dt))
    torch.cuda.synchronize()
    dx_ref, g_ref = grads.tri_attn_grad(x, m, P, starting, heads, dy)
    got, refs = {"dx": _np(xt.grad)}, {"dx": dx_ref}
    for name, prm in mod.named_parameters():
        assert prm.grad is not None and prm.grad.dtype == dt, name
        got[name], refs[name] = _np(prm.grad), g_ref[name]
    cls = type(mod)
    worst = _check_all(dname, got, refs, lambda: _reference_bf16_errors(
        cls(cin, ch, heads, use_fused_kernel=False), P, x, m, dy, dx_ref, g_ref))
    log(f"  worst max|g - r| / max|r|: {max(worst)[0]:.2e} ({max(worst)[1]})")


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [40, 77, 130])
def test_tri_attn_backward(dname, starting, N):
    """Includes fully masked rows (the padded rows of the second batch
    element), whose uniform softmax passes its gradient to q, k and the
    triangle bias as torch autograd of the reference does."""
    _tri_attn_backward_case(dname, starting, N, [N, N - 6])


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_backward_n264(starting):
    """bf16 at N = 264 (288 padded positions, 9 key tiles): the (row, head)
    backward kernels with 512-position LDS buffers, a dL/dbias wave owning two
    key tiles (0 and 8), fully masked rows (the last 6) and scattered masked
    pairs."""
    _tri_attn_backward_case("bf16", starting, 264, [258], inner_mask=0.05)


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_backward_exact_recompute(monkeypatch, starting):
    """bf16 with the forward recompute's exact online softmax for every query
    tile (GENIE_TK_EXACT_SOFTMAX=1).  The kernel takes it where the pass
    without a running maximum leaves l's safe range: scores beyond about 60
    log2 units, where bf16 inputs are too coarse for a well-conditioned
    gradient check."""
    monkeypatch.setenv("GENIE_TK_EXACT_SOFTMAX", "1")
    _tri_attn_backward_case("bf16", starting, 77, [77, 71], inner_mask=0.05)


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_backward_element_paths(monkeypatch, starting):
    """bf16 with the prologue backward's element-pointer kernel, the path
    taken where the channel-major buffers' byte offsets exceed 32 bits (N
    above about 1440), selected here at a small N by GENIE_TK_ELEMENT_PATHS."""
    monkeypatch.setenv("GENIE_TK_ELEMENT_PATHS", "1")
    _tri_attn_backward_case("bf16", starting, 77, [77, 71])


def test_tri_attn_backward_runs_the_kernels(monkeypatch):
    P = H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=11, bias_random=True)
    mod = triattn_module(P, False, 4, torch.bfloat16)
    monkeypatch.setattr(mod, "_forward_pytorch",
                        lambda *a, **k: (_ for _ in ()).throw(AssertionError("fallback")))
    x = torch.randn(1, 2, 33, 33, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = mod(x)
    y.float().square().sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape and torch.isfinite(x.grad).all()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in mod.parameters())


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("cin,ch,heads", [(128, 32, 4), (64, 32, 4), (32, 16, 2), (32, 8, 1)])
def test_tri_attn_backward_other_shapes(dname, starting, cin, ch, heads):
    """The reference layer's default attention (c_in = 128, four heads of 8;
    pair_transform.py:116-117), its tests' shapes (c_in = 64 with four heads
    of 8, tests/test_triangle_attention.py:36; c_in = 32 with two heads of 8,
    :74) and one head of 8: the backward kernels of c_in 32 / 64 / 128, on
    the weights padded to four heads of 32, with fully masked rows."""
    _tri_attn_backward_case(dname, starting, 40, [40, 33], cin=cin, ch=ch, heads=heads)


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("cz,c,N", [(64, 32, 40), (32, 32, 37), (64, 64, 33), (32, 128, 24),
                                    (32, 16, 16), (64, 8, 30), (64, 32, 32), (32, 64, 64)])
def test_tri_mul_backward_other_shapes(dname, outgoing, cz, c, N):
    """The backward kernels of c_z in {32, 64} and c in {32, 64, 128} (the
    reference tests' c_z = 64, c = 32, tests/test_triangle_mul.py:37), whose
    forward packing leaves the LayerNorm affine to the kernels; and c = 16
    (the reference's gradient test, c_z = 32, N = 16, :73) and 8, which run
    as 32 repeated channels.  N = 32 and 64 take the whole-tile path of the
    bf16 prologue backward (channel-major blocks staged through LDS)."""
    log(f"tri_mul backward {dname} outgoing={outgoing} c_z={cz} c={c} N={N}")
    dt = DT[dname]
    P = H.draw_params(H.tri_mul_shapes(cz, c), seed=N + c + cz, ln_random=True, bias_random=True)
    z = H.pair_input(2, N, cz, seed=N + 1)
    m = H.tail_mask(2, N, [N, N - 5])
    dy = H.pair_input(2, N, cz, seed=N + 2)
    if dname == "bf16":
        P, z, dy = H.bf16_params(P), H.bf16_round(z), H.bf16_round(dy)
    mod = trimul_module(P, outgoing, dt)
    mod._forward_pytorch = lambda *a, **k: (_ for _ in ()).throw(AssertionError("PyTorch path"))
    zt = torch.from_numpy(z).to("cuda", dt).requires_grad_(True)
    y = mod(zt, torch.from_numpy(m).to("cuda"))
    y.backward(torch.from_numpy(dy).to("cuda", dt))
    torch.cuda.synchronize()
    dz_ref, g_ref = grads.tri_mul_grad(z, m, P, outgoing, dy)
    got, refs = {"dx": _np(zt.grad)}, {"dx": dz_ref}
    for name, prm in mod.named_parameters():
        assert prm.grad is not None and prm.grad.dtype == dt, name
        got[name], refs[name] = _np(prm.grad), g_ref[name]
    cls = type(mod)
    worst = _check_all(dname, got, refs, lambda: _reference_bf16_errors(
        cls(cz, c, use_fused_kernel=False), P, z, m, dy, dz_ref, g_ref))
    log(f"  worst max|g - r| / max|r|: {max(worst)[0]:.2e} ({max(worst)[1]})")
