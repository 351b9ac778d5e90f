"""Large-N parity: the attention kernels that only run past N = 1024 (forward),
the backward kernels between N = 512 and N = 1024 and beyond, and the
triangle update's row chunks at N = 2048, against the oracle on sampled rows.

A row of triangle attention is an independent problem once the shared
triangle bias exists, so the oracle evaluates only the sampled rows
(pair_ops.tri_attn(..., rows=...)); the backward oracle gets an upstream
gradient that is zero outside the sampled rows, whose other rows then
contribute exactly zero (grads.tri_attn_grad skips them).

Masks: a tail mask (the last rows and columns fully masked), one fully
masked row and one fully masked column inside the valid block, and 5 % of
scattered masked pairs.  Tolerances as in gpu_common / test_gpu_grads.
"""
import numpy as np
import pytest
import torch

from oracle import grads, pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, log, to_np, triattn_module, trimul_module
from tests.test_gpu_grads import _check_grad

pytestmark = pytest.mark.gpu


def _mask(N: int, L: int, seed: int) -> np.ndarray:
    m = H.tail_mask(1, N, [L])
    rng = np.random.default_rng(seed)
    m *= (rng.random(m.shape) >= 0.05).astype(np.float32)
    m[0, 100, :] = 0.0   # a fully masked row (starting node) ...
    m[0, :, 200] = 0.0   # ... and column (ending node)
    return m


def _rows(N: int, L: int) -> list:
    return sorted({0, 1, 100, 200, 517, L - 1, L, N - 1})


_cache = {}


def _inputs(N: int):
    """bf16-rounded input, mask and parameters for size N (built once per N)."""
    if N not in _cache:
        _cache.clear()
        L = N - 37
        P = H.bf16_params(H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=N + 3,
                                        ln_random=True, bias_random=True))
        x = H.bf16_round(H.pair_input(1, N, 128, seed=N + 4))
        _cache[N] = (x, _mask(N, L, N + 5), P, L)
    return _cache[N]


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [1152, 2048])
def test_tri_attn_forward_beyond_1024(starting, N):
    """bf16 forward for Np > 1024 (the streaming flash kernel with the K/V ring,
    the bf16 bias through the identity MFMA and W_o fused), sampled rows
    against the oracle: fp32 arithmetic on the bf16-rounded inputs (float64
    at N = 1152)."""
    log(f"tri_attn forward N={N} starting={starting}")
    x, m, P, L = _inputs(N)
    rows = _rows(N, L)
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    xd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        y = mod(xd, md)
        y_res = mod.forward_residual(xd, md)
    torch.cuda.synchronize()
    sel = (lambda a: a[:, rows]) if starting else (lambda a: a[:, :, rows])
    got = to_np(sel(y))
    got_res = to_np(sel(y_res))
    del y, y_res
    dt = np.float64 if N <= 1152 else np.float32
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=dt, rows=rows)
    check_bf16(got, ref, f"tri_attn N={N} starting={starting}")
    check_bf16(got_res, ref + sel(x), f"tri_attn residual N={N} starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [600, 1024])
def test_tri_attn_forward_np1024(starting, N):
    """bf16 forward for 512 < Np <= 1024: the (row, head) flash kernel with
    1024-position K^T/V^T buffers (128 KiB of LDS) in 16-wave blocks, sampled
    rows against the float64 oracle, plus row chunks bit-identical to the
    unchunked output."""
    log(f"tri_attn forward (row, head) Np<=1024 N={N} starting={starting}")
    x, m, P, L = _inputs(N)
    rows = _rows(N, L)
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    xd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        y = mod(xd, md)
        y_chunk = mod(xd, md, chunk_size=250)
    torch.cuda.synchronize()
    assert torch.equal(y_chunk, y), "row chunks of 250 differ from the unchunked output"
    sel = (lambda a: a[:, rows]) if starting else (lambda a: a[:, :, rows])
    got = to_np(sel(y))
    del y, y_chunk
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float64, rows=rows)
    check_bf16(got, ref, f"tri_attn N={N} starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
def test_tri_attn_row_chunks_beyond_1024(starting):
    """Row chunks on the Np > 1024 path: bit-identical to the unchunked
    output (chunk sizes that do and do not divide N)."""
    N = 1152
    log(f"tri_attn row chunks N={N} starting={starting}")
    x, m, P, L = _inputs(N)
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    xd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        full = mod(xd, md)
        for c in (128, 500):
            y = mod(xd, md, chunk_size=c)
            torch.cuda.synchronize()
            assert torch.equal(y, full), f"chunk {c}: differs from the unchunked output"


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [600, 1024, 1100])
def test_tri_attn_backward_large(starting, N):
    """bf16 backward at N = 600 (Np between 512 and 1024: the (row, head)
    kernels with 1024-position buffers and the first dL/dbias kernel), N =
    1024 (the largest (row, head) size) and N = 1100 (Np > 1024: the
    one-wave-per-tile kernels), upstream gradient on sampled rows only."""
    log(f"tri_attn backward N={N} starting={starting}")
    x, m, P, L = _inputs(N)
    rows = _rows(N, L)
    rng = np.random.default_rng(N + 6)
    dy = np.zeros_like(x)
    if starting:
        dy[:, rows] = H.bf16_round(rng.standard_normal(dy[:, rows].shape).astype(np.float32))
    else:
        dy[:, :, rows] = H.bf16_round(rng.standard_normal(dy[:, :, rows].shape).astype(np.float32))
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    xt = torch.from_numpy(x).to("cuda", torch.bfloat16).requires_grad_(True)
    y = mod(xt, torch.from_numpy(m).to("cuda"))
    y.backward(torch.from_numpy(dy).to("cuda", torch.bfloat16))
    torch.cuda.synchronize()
    dx_ref, g_ref = grads.tri_attn_grad(x, m, P, starting, 4, dy)
    worst = [(_check_grad(to_np(xt.grad), dx_ref, "bf16", "dx"), "dx")]
    for name, prm in mod.named_parameters():
        assert prm.grad is not None and prm.grad.dtype == torch.bfloat16, name
        worst.append((_check_grad(to_np(prm.grad), g_ref[name], "bf16", name), name))
    log(f"  worst max|g - r| / max|r|: {max(worst)[0]:.2e} ({max(worst)[1]})")


@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_row_chunks_2048(outgoing):
    """The memory-bounded mode at N = 2048 (bf16, c_z = c = 128): 512-row
    chunks (workspace 1.5 GiB instead of 3 GiB) bit-identical to the unchunked
    update, sampled rows against the oracle (fp32 arithmetic on the
    bf16-rounded inputs)."""
    N = 2048
    log(f"tri_mul row chunks N={N} outgoing={outgoing}")
    x, m, _, L = _inputs(N)
    P = H.bf16_params(H.draw_params(H.tri_mul_shapes(128, 128), seed=N + 7, ln_random=True,
                                    bias_random=True))
    rows = _rows(N, L)
    mod = trimul_module(P, outgoing, torch.bfloat16)
    zd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        y = mod(zd, md, chunk_size=512)
        full = mod(zd, md)
        torch.cuda.synchronize()
        assert torch.equal(y, full), "512-row chunks differ from the unchunked update"
        del full
        got = to_np(y[:, rows])
    del y
    ref = pair_ops.tri_mul(x, m, P, outgoing, dtype=np.float32, rows=rows)
    check_bf16(got, ref, f"tri_mul chunks N={N} outgoing={outgoing}")
