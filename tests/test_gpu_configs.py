"""GPU parity at the benchmark workloads:

tri-mul outgoing, fp32, B=1 N=64, LN gamma=1 beta=0, biases 0   (max abs err <= 1e-4)
tri-mul outgoing + incoming, bf16, B=1 N=256, tail mask (224), gate biases 1
tri-attn starting + ending, bf16, B=1 N=256, H=4 d=32, tail mask (224)
pair block (tri-mul out -> in -> tri-attn start -> end, residual each),
    bf16, B=2 N=512, lengths (384, 512): each operator checked on the GPU's
    own input to it; tri-attn on sampled rows (rows are independent)
B=1 N=1024, mask ones: tri-mul outgoing and tri-attn starting on sampled
    output rows, LayerNorm in full
plus size-independent properties at N=512 (incoming = transposed outgoing with
swapped a/b projections; ending = transposed starting).
bf16 tolerance: |y - y_ref| <= 2e-2 + 1e-2 |y_ref|, y_ref = fp32/fp64 oracle on
the bf16-rounded inputs and weights.
"""
import numpy as np
import pytest
import torch

from oracle import pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, check_fp32, ext, log, to_np, trimul_module, triattn_module

pytestmark = pytest.mark.gpu


def _dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _trimul_params(seed, gates=False):
    kw = dict(gate_bias=1.0, gate_keys=H.TRI_MUL_GATES) if gates else {}
    return H.draw_params(H.tri_mul_shapes(128, 128), seed, **kw)


def _triattn_params(seed):
    return H.draw_params(H.tri_attn_shapes(128, 128, 4), seed, tri_std=1.0 / np.sqrt(128))


def test_trimul_fp32_n64():
    log("tri-mul outgoing fp32 N=64")
    P = _trimul_params(0)
    z = H.pair_input(1, 64, 128, seed=0)
    m = np.ones((1, 64, 64), np.float32)
    mod = trimul_module(P, True, torch.float32)
    with torch.no_grad():
        y = mod(_dev(z, torch.float32), _dev(m, torch.float32))
    ref = pair_ops.tri_mul(z, m, P, True, dtype=np.float64)
    check_fp32(to_np(y), ref, "tri-mul fp32 N=64")


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_bf16_n256(outgoing):
    log(f"tri-mul bf16 N=256 outgoing={outgoing}")
    P = H.bf16_params(_trimul_params(1, gates=True))
    z = H.bf16_round(H.pair_input(1, 256, 128, seed=1))
    m = H.tail_mask(1, 256, [224])
    mod = trimul_module(P, outgoing, torch.bfloat16)
    with torch.no_grad():
        y = mod(_dev(z, torch.bfloat16), _dev(m, torch.float32))
    ref = pair_ops.tri_mul(z, m, P, outgoing, dtype=np.float32)
    check_bf16(to_np(y), ref, f"tri-mul bf16 N=256 outgoing={outgoing}")


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_bf16_n256(starting):
    log(f"tri-attn bf16 N=256 starting={starting}")
    P = H.bf16_params(_triattn_params(2))
    x = H.bf16_round(H.pair_input(1, 256, 128, seed=2))
    m = H.tail_mask(1, 256, [224])
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    with torch.no_grad():
        y = mod(_dev(x, torch.bfloat16), _dev(m, torch.float32))
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float32)
    check_bf16(to_np(y), ref, f"tri-attn bf16 N=256 starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [200, 130])
def test_triattn_multi_block_ragged(starting, N):
    log(f"tri-attn bf16 multi query block N={N} starting={starting}")
    P = H.bf16_params(H.draw_params(H.tri_attn_shapes(128, 128, 4), N, ln_random=True, bias_random=True))
    x = H.bf16_round(H.pair_input(2, N, 128, seed=N))
    m = H.tail_mask(2, N, [N, N - 37])
    m[0, 5, 7] = 0  # isolated masked keys inside a valid row
    m[0, 9, :] = 0
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    with torch.no_grad():
        y = mod(_dev(x, torch.bfloat16), _dev(m, torch.float32))
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float32)
    check_bf16(to_np(y), ref, f"tri-attn N={N}")


def test_pair_block_b2_n512():
    log("pair block bf16 B=2 N=512 lengths (384, 512)")
    B, N = 2, 512
    m = H.tail_mask(B, N, [384, 512])
    Pm_out = H.bf16_params(_trimul_params(40))
    Pm_in = H.bf16_params(_trimul_params(41))
    Pa_s = H.bf16_params(_triattn_params(42))
    Pa_e = H.bf16_params(_triattn_params(43))
    mods = [trimul_module(Pm_out, True, torch.bfloat16), trimul_module(Pm_in, False, torch.bfloat16),
            triattn_module(Pa_s, True, 4, torch.bfloat16), triattn_module(Pa_e, False, 4, torch.bfloat16)]
    mt = _dev(m, torch.float32)
    p = _dev(H.pair_input(B, N, 128, seed=4), torch.bfloat16)
    rows = [0, 1, 200, 383, 384, 511]
    for idx, mod in enumerate(mods):
        with torch.no_grad():
            upd = mod(p, mt)
        p_in = to_np(p)
        got = to_np(upd)
        if idx < 2:
            P = (Pm_out, Pm_in)[idx]
            ref = pair_ops.tri_mul(p_in, m, P, idx == 0, dtype=np.float32)
            check_bf16(got, ref, f"pair block op {idx}")
        else:
            P = (Pa_s, Pa_e)[idx - 2]
            starting = idx == 2
            ref = pair_ops.tri_attn(p_in, m, P, starting, 4, dtype=np.float32, rows=rows)
            sel = got[:, rows] if starting else got[:, :, rows]
            check_bf16(sel, ref, f"pair block op {idx}")
        p = p + upd
    assert torch.isfinite(p).all()


def test_trimul_triattn_layernorm_n1024():
    log("N=1024 tri-mul outgoing, tri-attn starting (sampled rows), LayerNorm")
    N = 1024
    z = H.bf16_round(H.pair_input(1, N, 128, seed=5))
    zt = _dev(z, torch.bfloat16)
    rows = [0, 333, 1023]
    Pm = H.bf16_params(_trimul_params(50))
    with torch.no_grad():
        y = trimul_module(Pm, True, torch.bfloat16)(zt)
    ref = pair_ops.tri_mul(z, None, Pm, True, dtype=np.float32, rows=rows)
    check_bf16(to_np(y)[:, rows], ref, "N=1024 tri-mul")
    Pa = H.bf16_params(_triattn_params(51))
    with torch.no_grad():
        y = triattn_module(Pa, True, 4, torch.bfloat16)(zt)
    ref = pair_ops.tri_attn(z, None, Pa, True, 4, dtype=np.float32, rows=rows)
    check_bf16(to_np(y)[:, rows], ref, "N=1024 tri-attn")
    w = np.ones(128, np.float32)
    bb = np.zeros(128, np.float32)
    y = ext().layernorm(zt, _dev(w, torch.float32), _dev(bb, torch.float32), 1e-5)
    check_bf16(to_np(y), pair_ops.layer_norm(z, w, bb), "N=1024 layernorm")


def test_transpose_identities_n512():
    """incoming(z; a<->b swapped) == outgoing(z^T)^T and ending(x) == starting(x^T)^T
    on the GPU at N=512 (no oracle involved)."""
    log("identities at N=512")
    N = 512
    P = H.bf16_params(_trimul_params(60))
    swapped = dict(P)
    for part in ("weight", "bias"):
        for a, b in (("linear_a_p", "linear_b_p"), ("linear_a_g", "linear_b_g")):
            swapped[f"{a}.{part}"], swapped[f"{b}.{part}"] = P[f"{b}.{part}"], P[f"{a}.{part}"]
    z = _dev(H.pair_input(1, N, 128, seed=6), torch.bfloat16)
    m = _dev(H.tail_mask(1, N, [500]), torch.float32)
    with torch.no_grad():
        inc = trimul_module(P, False, torch.bfloat16)(z, m)
        out_t = trimul_module(swapped, True, torch.bfloat16)(z.transpose(1, 2).contiguous(),
                                                            m.transpose(1, 2).contiguous())
    assert torch.equal(inc, out_t.transpose(1, 2))
    Pa = H.bf16_params(_triattn_params(61))
    with torch.no_grad():
        end = triattn_module(Pa, False, 4, torch.bfloat16)(z, m)
        st_t = triattn_module(Pa, True, 4, torch.bfloat16)(z.transpose(1, 2).contiguous(),
                                                           m.transpose(1, 2).contiguous())
    assert torch.equal(end, st_t.transpose(1, 2))
