"""GPU parity at corners of the reference's semantics that the benchmark
workload tests do not reach.

* Tri-mul with fractional mask values: the reference multiplies a and b by
  the mask value itself (src/genie_tk/triangle_mul.py:115,117), so 0.25,
  0.5 and 0.75 scale the projections; both directions, fp32 and bf16, the
  padded-plane layout (N not a multiple of 64), row chunks, and a shape of
  the generic kernels.
* Triangle attention rows whose keys are all masked, under a triangle bias
  with a per-head constant of 200 (natural units): the reference's fp32
  scores fl32(fl32(qk - 1e9) + tri) all round to -1e9 + 192, so those rows
  are uniform; every kernel path must give that result.
* Training with a mask that is not binary: the backward kernels model only
  0/1 masks, so the module must run autograd of its PyTorch path, and its
  gradients match the float64 oracle.
* The pair block (B=2, N=512, lengths 384 / 512) through ``forward_residual``,
  the fused-residual path a PairTransformLayer takes in eval, each operator
  on the previous one's output, against the oracle on sampled rows.

Tolerances: fp32 max abs error <= 1e-4 against the float64 oracle; bf16
|y - y_ref| <= 2e-2 + 1e-2 |y_ref| against the fp32 oracle on bf16-rounded
inputs and weights; gradients as in test_gpu_grads.
"""
import numpy as np
import pytest
import torch

from genie_tk import triangle_attention as ta_mod
from oracle import grads, pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, check_fp32, log, to_np, triattn_module, trimul_module
from tests.test_gpu_grads import _check_grad
from tests.test_gpu_kernels import logit_offset_params

pytestmark = pytest.mark.gpu


def _dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _fractional_mask(B, N, seed):
    """Values 0, 0.25, 0.5, 0.75 and 1 at random, plus a fully masked tail row
    and column in the second batch element."""
    rng = np.random.default_rng(seed)
    m = rng.choice(np.array([0.0, 0.25, 0.5, 0.75, 1.0], np.float32), size=(B, N, N))
    if B > 1:
        m[1, N - 3:, :] = 0
        m[1, :, N - 3:] = 0
    return m.astype(np.float32)


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("c_z,c,N", [(128, 128, 70), (128, 64, 130), (64, 32, 45)])
def test_tri_mul_fractional_mask(dname, outgoing, c_z, c, N):
    log(f"tri_mul fractional mask {dname} outgoing={outgoing} c_z={c_z} c={c} N={N}")
    dt = torch.float32 if dname == "fp32" else torch.bfloat16
    # LayerNorm affine at its default (gamma 1, beta 0): the variable here is
    # the mask value; random affines are test_gpu_kernels.test_tri_mul_module's
    P = H.draw_params(H.tri_mul_shapes(c_z, c), seed=N + c, bias_random=True)
    z = H.pair_input(2, N, c_z, seed=N + 3)
    m = _fractional_mask(2, N, seed=N + 4)
    if dname == "bf16":
        P, z = H.bf16_params(P), H.bf16_round(z)
    mod = trimul_module(P, outgoing, dt)
    zt, mt = _dev(z, dt), _dev(m, torch.float32)
    with torch.no_grad():
        y = mod(zt, mt)
        y_chunk = mod(zt, mt, chunk_size=32)
    torch.cuda.synchronize()
    assert torch.equal(y, y_chunk), "row chunks differ from the unchunked output"
    if dname == "fp32":
        check_fp32(to_np(y), pair_ops.tri_mul(z, m, P, outgoing, dtype=np.float64),
                   f"tri_mul fractional mask fp32 outgoing={outgoing}")
    else:
        check_bf16(to_np(y), pair_ops.tri_mul(z, m, P, outgoing, dtype=np.float32),
                   f"tri_mul fractional mask bf16 outgoing={outgoing}")


@pytest.mark.parametrize("dname", ["fp32", "bf16"])
@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_fully_masked_rows_head_constant(dname, starting):
    """Rows with no valid key (the masked tail and row/column 7) under a
    triangle bias whose per-head constant is 200: the fp32 reference's row is
    uniform there, and so is every kernel's (the bf16 fast path drops the
    constant; the fp32 kernels keep it, in log2 units, where -1e9 log2(e)
    rounds the constant with the rest)."""
    log(f"tri_attn fully masked rows, head constant 200, {dname} starting={starting}")
    dt = torch.float32 if dname == "fp32" else torch.bfloat16
    N = 64
    P = logit_offset_params(200.0)
    x = H.bf16_round(H.pair_input(1, N, 128, seed=21))
    m = H.tail_mask(1, N, [52])
    m[0, 7, :] = 0
    m[0, :, 7] = 0
    m[0, 3, 5] = 0  # an isolated masked key in a valid row
    mod = triattn_module(P, starting, 4, dt)
    with torch.no_grad():
        y = mod(_dev(x, dt), _dev(m, torch.float32))
    torch.cuda.synchronize()
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float64)
    # the regime: the reference's fully masked rows equal those without the constant
    ref0 = pair_ops.tri_attn(x, m, logit_offset_params(0.0), starting, 4, dtype=np.float64)
    full = [7] + list(range(52, N))
    sel = (lambda a: a[:, full]) if starting else (lambda a: a[:, :, full])
    np.testing.assert_allclose(sel(ref), sel(ref0), atol=1e-9)
    if dname == "fp32":
        check_fp32(to_np(y), ref, "fully masked rows fp32")
    else:
        check_bf16(to_np(y), pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float32),
                   "fully masked rows bf16")


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_backward_nonbinary_mask(starting, monkeypatch):
    """A row of fractional mask values with no 1 among them, and a value
    above 1: the forward's bias inf * (mask - 1) then decides the weights,
    which the backward kernels do not model.  The module must train through
    autograd of its PyTorch path (the kernels' Function is made to raise),
    with gradients matching the float64 oracle (fp32 tolerance)."""
    log(f"tri_attn backward, non-binary mask, starting={starting}")
    monkeypatch.setattr(ta_mod._TriAttnFunction, "apply",
                        lambda *a, **k: (_ for _ in ()).throw(AssertionError("backward kernels")))
    N = 24
    P = H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=51, bias_random=True)
    x = H.pair_input(1, N, 128, seed=52)
    m = H.tail_mask(1, N, [N - 3])
    m[0, 2, :] = np.resize(np.array([0.25, 0.5, 0.75], np.float32), N)  # no key with mask 1
    m[0, 5, 7] = 1.5
    dy = H.pair_input(1, N, 128, seed=53)
    mod = triattn_module(P, starting, 4, torch.float32)
    xt = _dev(x, torch.float32).requires_grad_(True)
    y = mod(xt, _dev(m, torch.float32))
    y.backward(_dev(dy, torch.float32))
    torch.cuda.synchronize()
    dx_ref, g_ref = grads.tri_attn_grad(x, m, P, starting, 4, dy)
    _check_grad(to_np(xt.grad), dx_ref, "fp32", "dx")
    for name, prm in mod.named_parameters():
        _check_grad(to_np(prm.grad), g_ref[name], "fp32", name)


def test_tri_attn_backward_binary_mask_uses_kernels(monkeypatch):
    """The same call with a binary mask still takes the backward kernels."""
    calls = []
    real = ta_mod._TriAttnFunction.apply
    monkeypatch.setattr(ta_mod._TriAttnFunction, "apply", lambda *a: calls.append(1) or real(*a))
    P = H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=54, bias_random=True)
    mod = triattn_module(P, True, 4, torch.bfloat16)
    x = torch.randn(1, 24, 24, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    m = torch.from_numpy(H.tail_mask(1, 24, [20])).cuda()
    mod(x, m).float().sum().backward()
    assert calls == [1] and x.grad is not None


def test_pair_block_b2_n512_forward_residual():
    """The pair block (B=2, N=512, lengths 384 / 512, bf16) through the modules'
    forward_residual (residual add fused into the last kernel of each
    operator), chained tri-mul out -> in -> tri-attn start -> end: each
    operator's output p + update against the GPU's own input p plus the
    oracle's update, on sampled rows."""
    log("pair block via forward_residual: B=2 N=512 lengths (384, 512)")
    B, N = 2, 512
    m = H.tail_mask(B, N, [384, 512])
    tm = lambda s: H.bf16_params(H.draw_params(H.tri_mul_shapes(128, 128), s))  # noqa: E731
    tap = lambda s: H.bf16_params(H.draw_params(H.tri_attn_shapes(128, 128, 4), s,  # noqa: E731
                                                tri_std=1.0 / np.sqrt(128)))
    params = [tm(40), tm(41), tap(42), tap(43)]
    mods = [trimul_module(params[0], True, torch.bfloat16), trimul_module(params[1], False, torch.bfloat16),
            triattn_module(params[2], True, 4, torch.bfloat16),
            triattn_module(params[3], False, 4, torch.bfloat16)]
    mt = _dev(m, torch.float32)
    p = _dev(H.pair_input(B, N, 128, seed=4), torch.bfloat16)
    rows = [0, 1, 200, 383, 384, 511]
    for idx, mod in enumerate(mods):
        with torch.no_grad():
            p_next = mod.forward_residual(p, mt)
        torch.cuda.synchronize()
        p_in = to_np(p)
        if idx < 2:
            upd = pair_ops.tri_mul(p_in, m, params[idx], idx == 0, dtype=np.float32, rows=rows)
            got, base = to_np(p_next)[:, rows], p_in[:, rows]
        else:
            starting = idx == 2
            upd = pair_ops.tri_attn(p_in, m, params[idx], starting, 4, dtype=np.float32, rows=rows)
            sel = (lambda a: a[:, rows]) if starting else (lambda a: a[:, :, rows])
            got, base = sel(to_np(p_next)), sel(p_in)
        check_bf16(got, base + upd, f"pair block forward_residual op {idx}")
        p = p_next
    assert torch.isfinite(p).all()
