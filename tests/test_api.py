"""The genie_tk Python API on the CPU: names, constructors, parameters,
PyTorch-path numerics against the oracle, the kernel/fallback switch and the
utilities.  Mirrors the reference's tests/test_triangle_mul.py:26-111 and
tests/test_triangle_attention.py:25-175 (shape, gradient flow, mask, pair
transform) and adds value checks, since the reference's own checks pass on
all-zero outputs.
"""
import numpy as np
import pytest
import torch

import genie_tk
from genie_tk import (PairTransformLayer, PairTransformNet, TriangleAttention,
                      TriangleAttentionEndingNode, TriangleAttentionStartingNode,
                      TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing,
                      TriangleMultiplicativeUpdate)
from genie_tk import utils
from oracle import pair_ops
from tests import helpers as H

REFERENCE_ALL = [
    "TriangleMultiplicativeUpdate", "TriangleMultiplicationOutgoing",
    "TriangleMultiplicationIncoming", "TriangleAttention", "TriangleAttentionStartingNode",
    "TriangleAttentionEndingNode", "PairTransformLayer", "PairTransformNet",
    "has_cuda_kernels", "get_device_info",
]


def _load(module, params):
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}
    missing, unexpected = module.load_state_dict(sd, strict=True)
    assert not missing and not unexpected
    return module


def _pair(B, N, C, seed):
    return torch.from_numpy(H.pair_input(B, N, C, seed))


def test_public_names_match_reference():
    assert sorted(genie_tk.__all__) == sorted(REFERENCE_ALL)
    for name in REFERENCE_ALL:
        assert hasattr(genie_tk, name)


def test_tri_mul_state_dict_layout():
    m = TriangleMultiplicationOutgoing(c_z=32, c_hidden=16, use_fused_kernel=False)
    got = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert got == H.tri_mul_shapes(32, 16)
    # AlphaFold initialisers: gates W=0 b=1, final projection zero
    for g in ("linear_a_g", "linear_b_g", "linear_g"):
        assert torch.all(getattr(m, g).weight == 0) and torch.all(getattr(m, g).bias == 1)
    assert torch.all(m.linear_z.weight == 0) and torch.all(m.linear_z.bias == 0)


def test_tri_attn_state_dict_layout():
    m = TriangleAttentionStartingNode(c_in=32, c_hidden=16, no_heads=2, use_fused_kernel=False)
    got = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert got == H.tri_attn_shapes(32, 16, 2)
    assert m.linear.bias is None and m.mha.linear_q.bias is None
    assert m.inf == 1e9 and m.starting
    assert not TriangleAttentionEndingNode(32, 16, 2).starting


def test_default_init_outputs_zero():
    """The final-init output projections make a fresh module's update exactly 0."""
    z = _pair(1, 8, 32, 0)
    assert torch.count_nonzero(TriangleMultiplicationOutgoing(32, 16)(z)) == 0
    assert torch.count_nonzero(TriangleAttentionStartingNode(32, 16, 2)(z)) == 0


@pytest.mark.parametrize("cls,outgoing", [(TriangleMultiplicationOutgoing, True),
                                          (TriangleMultiplicationIncoming, False)])
def test_tri_mul_pytorch_path_matches_oracle(cls, outgoing):
    P = H.draw_params(H.tri_mul_shapes(32, 16), 3, ln_random=True, bias_random=True)
    z = H.pair_input(2, 12, 32, seed=3)
    mask = H.tail_mask(2, 12, [12, 9])
    mod = _load(cls(c_z=32, c_hidden=16, use_fused_kernel=False), P)
    with torch.no_grad():
        y = mod(torch.from_numpy(z), torch.from_numpy(mask)).numpy()
    ref = pair_ops.tri_mul(z, mask, P, outgoing, dtype=np.float64)
    np.testing.assert_allclose(y, ref, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("cls,starting", [(TriangleAttentionStartingNode, True),
                                          (TriangleAttentionEndingNode, False)])
def test_tri_attn_pytorch_path_matches_oracle(cls, starting):
    P = H.draw_params(H.tri_attn_shapes(32, 16, 2), 4, ln_random=True, bias_random=True)
    x = H.pair_input(2, 10, 32, seed=4)
    mask = H.tail_mask(2, 10, [10, 7])
    mod = _load(cls(c_in=32, c_hidden=16, no_heads=2, use_fused_kernel=False), P)
    with torch.no_grad():
        y = mod(torch.from_numpy(x), torch.from_numpy(mask)).numpy()
    ref = pair_ops.tri_attn(x, mask, P, starting, 2, dtype=np.float64)
    np.testing.assert_allclose(y, ref, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("chunk", [1, 3, 4, 10, 64])
def test_tri_attn_row_chunks_pytorch_path(starting, chunk):
    """forward(chunk_size=...) attends rows a chunk at a time with the triangle
    bias of the whole pair map: same values as without chunks (and the oracle)."""
    P = H.draw_params(H.tri_attn_shapes(32, 16, 2), 6, ln_random=True, bias_random=True)
    x = H.pair_input(2, 10, 32, seed=6)
    mask = H.tail_mask(2, 10, [10, 6])
    cls = TriangleAttentionStartingNode if starting else TriangleAttentionEndingNode
    mod = _load(cls(c_in=32, c_hidden=16, no_heads=2, use_fused_kernel=False), P)
    with torch.no_grad():
        y = mod(torch.from_numpy(x), torch.from_numpy(mask), chunk_size=chunk).numpy()
        y0 = mod(torch.from_numpy(x), torch.from_numpy(mask)).numpy()
    np.testing.assert_allclose(y, y0, atol=1e-6, rtol=1e-6)
    ref = pair_ops.tri_attn(x, mask, P, starting, 2, dtype=np.float64)
    np.testing.assert_allclose(y, ref, atol=2e-5, rtol=1e-4)
    with pytest.raises(ValueError):
        mod(torch.from_numpy(x), chunk_size=0)


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("chunk", [1, 3, 4, 64])
def test_tri_mul_row_chunks_pytorch_path(outgoing, chunk):
    """forward(chunk_size=R) runs the output rows R at a time and equals the
    unchunked update (and the oracle)."""
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    P = H.draw_params(H.tri_mul_shapes(16, 8), seed=31, ln_random=True, bias_random=True)
    mod = _load(cls(16, 8), P)
    z = _pair(2, 7, 16, seed=32)
    m = torch.from_numpy(H.tail_mask(2, 7, [7, 5]))
    with torch.no_grad():
        full = mod(z, m)
        got = mod(z, m, chunk_size=chunk)
        res = mod.forward_residual(z, m, chunk_size=chunk)
    torch.testing.assert_close(got, full, rtol=0, atol=1e-6)
    torch.testing.assert_close(res, z + full, rtol=0, atol=1e-6)
    ref = pair_ops.tri_mul(z.numpy(), m.numpy(), P, outgoing, dtype=np.float64)
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-5)
    with pytest.raises(ValueError):
        mod(z, m, chunk_size=0)


def test_mask_default_is_all_ones():
    P = H.draw_params(H.tri_mul_shapes(16, 8), 5, bias_random=True)
    mod = _load(TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=False), P)
    z = _pair(1, 6, 16, 5)
    with torch.no_grad():
        assert torch.equal(mod(z), mod(z, torch.ones(1, 6, 6)))


@pytest.mark.parametrize("kind", ["mul", "attn"])
def test_gradient_flow(kind):
    """Gradients reach the input and every parameter (PyTorch path)."""
    if kind == "mul":
        mod = TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=True)
        _load(mod, H.draw_params(H.tri_mul_shapes(16, 8), 6, bias_random=True))
    else:
        mod = TriangleAttentionStartingNode(16, 8, 2, use_fused_kernel=True)
        _load(mod, H.draw_params(H.tri_attn_shapes(16, 8, 2), 6, bias_random=True))
    z = _pair(1, 8, 16, 6).requires_grad_(True)
    mod(z, torch.ones(1, 8, 8)).square().sum().backward()
    assert z.grad is not None and torch.isfinite(z.grad).all() and z.grad.abs().sum() > 0
    for name, p in mod.named_parameters():
        assert p.grad is not None, name


def test_masked_pairs_do_not_contribute():
    """Tri-mul outgoing: changing z on masked pairs (i, k) with k masked leaves rows
    whose contraction only sees masked k unchanged except through the gate."""
    P = H.draw_params(H.tri_mul_shapes(16, 8), 7, bias_random=True)
    mod = _load(TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=False), P)
    mask = torch.ones(1, 8, 8)
    mask[:, :, 5:] = 0
    z1 = _pair(1, 8, 16, 7)
    z2 = z1.clone()
    # pairs (i, k>=5) are masked in a and b: perturbing them must not change
    # x[i, j] for any (i, j) with j < 5, whose gate reads z[i, j] only
    z2[:, :, 5:] += 3.0
    with torch.no_grad():
        y1, y2 = mod(z1, mask), mod(z2, mask)
    assert torch.allclose(y1[:, :, :5], y2[:, :, :5], atol=1e-6)


def test_tri_attn_masked_keys_are_ignored():
    P = H.draw_params(H.tri_attn_shapes(16, 8, 2), 8, bias_random=True)
    mod = _load(TriangleAttentionStartingNode(16, 8, 2, use_fused_kernel=False), P)
    mask = torch.ones(1, 8, 8)
    mask[:, :, 6:] = 0
    x1 = _pair(1, 8, 16, 8)
    x2 = x1.clone()
    x2[:, :, 6:] += 2.0  # masked keys; their own query outputs change, others must not
    with torch.no_grad():
        y1, y2 = mod(x1, mask), mod(x2, mask)
    # the triangle bias tri[q, k] is read from pair (q, k): masked keys k>=6 feed
    # only through -inf scores, so queries q<6 of every row are unchanged
    assert torch.allclose(y1[:, :, :6], y2[:, :, :6], atol=1e-5)


def test_batch_dims_are_flattened():
    P = H.draw_params(H.tri_mul_shapes(16, 8), 9, bias_random=True)
    mod = _load(TriangleMultiplicationIncoming(16, 8, use_fused_kernel=False), P)
    z = torch.from_numpy(H.pair_input(6, 5, 16, 9)).reshape(2, 3, 5, 5, 16)
    with torch.no_grad():
        y = mod(z)
        y0 = mod(z[1, 2])
    assert y.shape == z.shape
    assert torch.allclose(y[1, 2], y0, atol=1e-6)


def test_cpu_host_switch():
    """No GPU here: the kernel switch is off and CPU tensors use the PyTorch path."""
    assert utils.has_cuda_kernels() is False or torch.cuda.is_available()
    m = TriangleMultiplicationOutgoing(128, 128, use_fused_kernel=True)
    assert m.use_fused_kernel == (m._fused_requested and utils.has_cuda_kernels())
    assert m._kernel_supported(torch.zeros(1, 4, 4, 128))
    assert not m._kernel_supported(torch.zeros(1, 4, 5, 128))
    assert not m._kernel_supported(torch.zeros(1, 4, 4, 128, dtype=torch.float16))
    # the reference tests' and layer's shapes have forward kernels
    for cz, c in ((64, 32), (32, 32), (128, 256), (64, 64)):
        assert TriangleMultiplicationOutgoing(cz, c)._kernel_supported(torch.zeros(1, 4, 4, cz))
    assert not TriangleMultiplicationOutgoing(96, 32)._kernel_supported(torch.zeros(1, 4, 4, 96))
    assert not TriangleMultiplicationOutgoing(64, 48)._kernel_supported(torch.zeros(1, 4, 4, 64))
    # backward kernels: c_z and c in {32, 64, 128}
    for cz, c in ((128, 64), (64, 32), (32, 32), (128, 128)):
        assert TriangleMultiplicationOutgoing(cz, c)._backward_supported(), (cz, c)
    assert not TriangleMultiplicationOutgoing(128, 256)._backward_supported()
    a = TriangleAttentionEndingNode(128, 128, 4)
    assert a._kernel_supported(torch.zeros(2, 4, 4, 128, dtype=torch.bfloat16))
    assert a._backward_supported()
    # every forward head shape trains on the backward kernels (heads padded to 4 x 32)
    for cin, ch, h in ((128, 32, 4), (64, 32, 4), (32, 16, 2), (128, 64, 4), (64, 64, 2), (32, 8, 1)):
        t = TriangleAttentionEndingNode(cin, ch, h)
        assert t._kernel_supported(torch.zeros(1, 4, 4, cin)), (cin, ch, h)
        assert t._backward_supported(), (cin, ch, h)
    assert not TriangleAttentionEndingNode(128, 128, 8)._kernel_supported(torch.zeros(1, 4, 4, 128))
    assert not TriangleAttentionEndingNode(128, 256, 4)._kernel_supported(torch.zeros(1, 4, 4, 128))
    assert not TriangleAttentionEndingNode(96, 32, 4)._kernel_supported(torch.zeros(1, 4, 4, 96))


def test_device_info_keys():
    info = genie_tk.get_device_info()
    assert set(info) == {"cuda_available", "cuda_kernels_available", "device_count", "devices"}
    assert info["device_count"] == len(info["devices"])
    for d in info["devices"]:
        assert set(d) == {"name", "total_memory", "major", "minor", "multi_processor_count"}


def test_layout_helpers():
    t = torch.arange(2 * 3 * 4 * 5).reshape(2, 3, 4, 5)
    assert torch.equal(utils.permute_final_dims(t, 2, 0, 1), t.permute(0, 3, 1, 2))
    assert utils.flatten_final_dims(t, 2).shape == (2, 3, 20)

    def layer(x, y):
        return x * 2 + y

    x = torch.randn(4, 6, 3)
    y = torch.randn(4, 6, 3)
    out = utils.chunk_layer(layer, {"x": x, "y": y}, chunk_size=5, no_batch_dims=2)
    assert torch.equal(out, layer(x, y))


def test_pair_transform_layer_and_net():
    """Reference tests/test_triangle_attention.py:123-165, plus block semantics."""
    torch.manual_seed(0)
    p = torch.randn(1, 12, 12, 32)
    m = torch.ones(1, 12, 12)
    m[:, 10:, :] = 0
    m[:, :, 10:] = 0
    layer = PairTransformLayer(c_p=32, c_hidden_mul=16, c_hidden_tri_att=16, n_head_tri=4,
                               tri_dropout=0.0, use_fused_kernel=False).eval()
    for mod in layer.modules():  # non-trivial weights so every branch contributes
        if isinstance(mod, torch.nn.Linear):
            torch.nn.init.normal_(mod.weight, std=mod.in_features ** -0.5)
    with torch.no_grad():
        out, out_m = layer((p, m))
        q = p
        for name in ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end"):
            q = q + getattr(layer, name)(q, m)
        q = q + layer.pair_transition(q, m)
        q = q * m.unsqueeze(-1)
    assert out.shape == p.shape and out_m is m
    assert torch.allclose(out, q, atol=1e-6)
    assert torch.all(out[:, 10:] == 0)
    net = PairTransformNet(c_p=32, n_layers=2, c_hidden_mul=16, c_hidden_tri_att=16,
                           n_head_tri=4, tri_dropout=0.0, use_fused_kernel=False)
    with torch.no_grad():
        y = net(p, m)
    assert y.shape == p.shape and torch.isfinite(y).all()


def test_shared_dropout_broadcasts():
    from genie_tk.pair_transform import DropoutColumnwise, DropoutRowwise
    x = torch.ones(2, 6, 6, 4)
    torch.manual_seed(1)
    r = DropoutRowwise(0.5).train()(x)
    assert torch.all(r == r[:, :1])          # same mask for every row
    c = DropoutColumnwise(0.5).train()(x)
    assert torch.all(c == c[:, :, :1])       # same mask for every column
    assert torch.equal(DropoutRowwise(0.5).eval()(x), x)


@pytest.fixture
def no_extension(monkeypatch):
    """genie_tk._C made unimportable (sys.modules entry None) and the loader
    re-run, as in a tree where the extension was never built; restored after."""
    import importlib
    import sys

    import genie_tk
    from genie_tk import _ext, triangle_attention, triangle_mul

    saved_mod = sys.modules.get("genie_tk._C", None)
    had_attr = hasattr(genie_tk, "_C")
    saved_attr = getattr(genie_tk, "_C", None)
    saved = (_ext.C, _ext.IMPORT_ERROR)
    sys.modules["genie_tk._C"] = None
    if had_attr:
        delattr(genie_tk, "_C")
    try:
        importlib.reload(_ext)
        assert _ext.C is None and isinstance(_ext.IMPORT_ERROR, ImportError)
        monkeypatch.setattr(triangle_mul, "_CUDA_AVAILABLE", False)
        monkeypatch.setattr(triangle_attention, "_CUDA_AVAILABLE", False)
        _ext._warned.clear()
        yield _ext
    finally:
        if saved_mod is None:
            sys.modules.pop("genie_tk._C", None)
        else:
            sys.modules["genie_tk._C"] = saved_mod
        if had_attr:
            genie_tk._C = saved_attr
        _ext.C, _ext.IMPORT_ERROR = saved
        _ext._warned.clear()


class _FakeCuda(torch.Tensor):
    """A CPU tensor that reports is_cuda, to reach the kernel switch without a GPU."""

    @property
    def is_cuda(self):
        return True


def test_missing_extension_falls_back_with_warning(no_extension, monkeypatch):
    """The reference's switch (triangle_mul.py:24-30,61; triangle_attention.py:25-31,67):
    with genie_tk._C missing, a GPU tensor with use_fused_kernel=True runs the
    PyTorch path.  This build also warns, once per module class."""
    monkeypatch.delenv(no_extension.STRICT_ENV, raising=False)
    torch.manual_seed(0)
    mod = TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=True)
    att = TriangleAttentionStartingNode(16, 8, 2, use_fused_kernel=True)
    for m in (mod, att):
        for p in m.parameters():
            torch.nn.init.normal_(p, std=0.3)
    assert not mod.use_fused_kernel and not att.use_fused_kernel
    z = torch.randn(1, 5, 5, 16)
    with pytest.warns(RuntimeWarning, match="not available"):
        y = mod(z.as_subclass(_FakeCuda))
    assert torch.equal(y.as_subclass(torch.Tensor), mod._forward_pytorch(z))
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # once per class: no second warning
        mod(z.as_subclass(_FakeCuda))
    with pytest.warns(RuntimeWarning, match="TriangleAttentionStartingNode"):
        ya = att(z.as_subclass(_FakeCuda))
    assert torch.equal(ya.as_subclass(torch.Tensor), att._forward_pytorch(z))


def test_missing_extension_strict_raises(no_extension, monkeypatch):
    """GENIE_TK_STRICT=1 (this repository's tests, smoke and bench) turns the
    fallback into ImportError, so an unbuilt library never passes for a working one."""
    monkeypatch.setenv(no_extension.STRICT_ENV, "1")
    mod = TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=True)
    with pytest.raises(ImportError):
        mod(torch.zeros(1, 4, 4, 16).as_subclass(_FakeCuda))
    att = TriangleAttentionEndingNode(16, 8, 2, use_fused_kernel=True)
    with pytest.raises(ImportError):
        att(torch.zeros(1, 4, 4, 16).as_subclass(_FakeCuda))
    # explicitly disabled: the PyTorch path is the documented behaviour
    mod2 = TriangleMultiplicationOutgoing(16, 8, use_fused_kernel=False)
    assert mod2(torch.zeros(1, 4, 4, 16)).shape == (1, 4, 4, 16)


def test_generic_class_direction_flag():
    assert TriangleMultiplicativeUpdate(16, 8)._outgoing
    assert not TriangleMultiplicationIncoming(16, 8)._outgoing
    assert TriangleAttention(16, 8, 2).starting


def test_head_padding_for_the_backward_kernels():
    """The attention backward kernels take four heads of 32 channels; a module
    with fewer or narrower heads runs them on its weights padded with zero
    channels and heads (triangle_attention._pad_heads), W_q scaled by
    sqrt(32 / d).  The padded module computes the same function: checked
    here in float64 on the PyTorch path, with the gradient of the real
    parameters recovered as the backward does."""
    from genie_tk import triangle_attention as ta

    torch.manual_seed(0)
    for cin, ch, h in ((32, 16, 2), (64, 32, 4), (32, 8, 1)):
        mod = TriangleAttentionStartingNode(cin, ch, h, use_fused_kernel=False).double()
        for p in mod.parameters():
            with torch.no_grad():
                p.copy_(torch.randn_like(p) * 0.3)
        params = mod._param_list()
        padded, idx, scale = ta._pad_heads([p.detach() for p in params], h, ch)
        big = TriangleAttentionStartingNode(cin, 128, 4, use_fused_kernel=False).double()
        with torch.no_grad():
            for p, v in zip(big._param_list(), padded):
                p.copy_(v)
        x = torch.randn(2, 6, 6, cin, dtype=torch.float64)
        m = (torch.rand(2, 6, 6) > 0.2).double()
        torch.testing.assert_close(big(x, m), mod(x, m), rtol=0, atol=1e-12)
        dy = torch.randn(2, 6, 6, cin, dtype=torch.float64)
        g_small = torch.autograd.grad((mod(x, m) * dy).sum(), params)
        g_big = list(torch.autograd.grad((big(x, m) * dy).sum(), big._param_list()))
        g_big[2] = g_big[2][:h]
        g_big[3] = g_big[3][idx] * scale
        for k in (4, 5, 6, 7):
            g_big[k] = g_big[k][idx]
        g_big[8] = g_big[8][:, idx]
        for a, b in zip(g_big, g_small):
            torch.testing.assert_close(a, b, rtol=0, atol=1e-10)


def test_dense_matmul_gradients():
    """primitives.dense_matmul (the PyTorch path's batched products, taken on
    contiguous operands with its own backward) against torch.autograd's
    numerical Jacobian, on the permuted views the modules pass it."""
    from genie_tk.primitives import dense_matmul
    g = torch.Generator().manual_seed(3)
    a = torch.randn(2, 5, 3, 4, dtype=torch.float64, generator=g).requires_grad_(True)
    b = torch.randn(2, 6, 3, 4, dtype=torch.float64, generator=g).requires_grad_(True)
    f = lambda a, b: dense_matmul(a.permute(0, 3, 1, 2), b.permute(0, 3, 2, 1))  # noqa: E731
    assert torch.autograd.gradcheck(f, (a, b))
    ref = torch.matmul(a.permute(0, 3, 1, 2), b.permute(0, 3, 2, 1))
    assert torch.equal(f(a, b), ref)


@pytest.mark.parametrize("cls", [TriangleMultiplicationOutgoing, TriangleMultiplicationIncoming,
                                 TriangleAttentionStartingNode, TriangleAttentionEndingNode])
def test_float32_mask_on_bf16_input(cls):
    """The PyTorch path takes a float32 mask with a bf16 input (the kernel path
    does): the mask is converted to the input's dtype, which gives the result
    the reference's path gives for the mask passed in that dtype."""
    mod = cls(32, 16) if "Multiplication" in cls.__name__ else cls(32, 8, 1)
    mod = mod.bfloat16()
    z = _pair(1, 10, 32, 7).bfloat16().requires_grad_(True)
    m = torch.ones(1, 10, 10)
    m[0, :, 8:] = 0.25
    y = mod(z, m)
    assert y.dtype == torch.bfloat16
    assert torch.equal(y, mod(z, m.bfloat16()))
    y.float().sum().backward()
    assert z.grad is not None and torch.isfinite(z.grad.float()).all()


@pytest.mark.parametrize("c,outgoing", [(16, True), (16, False), (8, True)])
def test_channel_repetition_for_narrow_hidden_widths(c, outgoing):
    """Tri-mul with c_hidden 8 or 16 runs on the kernels as 32 channels, each
    repeated 32 / c times (triangle_mul._repeat_channels).  The repeated
    module computes the same update, and summing its gradients over the
    copies (_fold_channel_grads) gives the module's own: float64, PyTorch
    path.  A plain zero padding would not: LN_out's mean and variance run
    over every hidden channel (checked too)."""
    from genie_tk import triangle_mul as tm

    torch.manual_seed(c)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = cls(32, c, use_fused_kernel=False).double()
    for p in mod.parameters():
        with torch.no_grad():
            p.copy_(torch.randn_like(p) * 0.3)
    r = 32 // c
    params = mod._param_list()
    big = cls(32, 32, use_fused_kernel=False).double()
    with torch.no_grad():
        for p, v in zip(big._param_list(), tm._repeat_channels([p.detach() for p in params], r)):
            p.copy_(v)
    z = torch.randn(2, 7, 7, 32, dtype=torch.float64)
    m = (torch.rand(2, 7, 7) > 0.2).double()
    torch.testing.assert_close(big(z, m), mod(z, m), rtol=0, atol=1e-12)
    dy = torch.randn(2, 7, 7, 32, dtype=torch.float64)
    g_small = torch.autograd.grad((mod(z, m) * dy).sum(), params)
    g_big = tm._fold_channel_grads(torch.autograd.grad((big(z, m) * dy).sum(), big._param_list()), c, r)
    for a, b in zip(g_big, g_small):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-10)
    # zero channels instead of copies change LN_out's statistics
    with torch.no_grad():
        for k in tm._HIDDEN_ROWS:
            p = big._param_list()[k]
            p[c:] = 0
        big.layer_norm_out.weight[c:] = 0
        big.linear_z.weight.zero_()
        big.linear_z.weight[:, :c] = mod.linear_z.weight
    assert (big(z, m) - mod(z, m)).abs().max() > 1e-3


def test_binary_mask_check_is_remembered_per_tensor():
    """The training path's binary-mask check (a reduction and a host
    synchronisation) runs once per mask tensor: again after an in-place
    change, and its entry goes with the tensor."""
    from genie_tk import _dispatch as D
    m = torch.ones(2, 5, 5)
    calls = []
    orig = torch.Tensor.all

    def counting_all(self, *a, **k):
        calls.append(1)
        return orig(self, *a, **k)

    torch.Tensor.all = counting_all
    try:
        assert D.binary_mask(m) and D.binary_mask(m)
        assert len(calls) == 1
        m[0, 1, 2] = 0.5
        assert not D.binary_mask(m)
        assert len(calls) == 2
        other = torch.zeros(3)
        assert D.binary_mask(other)
        n = len(D._binary_seen)
        del other
        assert len(D._binary_seen) == n - 1
        assert D.binary_mask(None)
    finally:
        torch.Tensor.all = orig
