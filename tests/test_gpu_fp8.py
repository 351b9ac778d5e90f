"""The fp8 a/b storage experiment (memory-bounded mode, outside the bf16
parity contract): the triangle update with its gated projections a and b
stored as OCP fp8 E4M3 and contracted on the fp8 matrix cores.

* The fp8 contraction alone against float64 products of the decoded bytes:
  pins the operand pairing of v_mfma_f32_32x32x64_f8f6f4 and the E4M3
  decoding.
* The whole fp8 forward against the oracle whose contraction takes a and b
  as the bf16 prologue forms them (x_hat in bf16, the LayerNorm affine and
  the gate's -log2(e) folded into bf16 weights), rounded to E4M3
  (tests/helpers.py e4m3_round), at the bf16 tolerance.  With a and b taken
  from the oracle itself, a value that lies within its bf16-level difference
  of an E4M3 rounding midpoint rounds the other way, about 3 % of them, and
  each such step is 6-12 % of the value.  The distance from the unrounded
  oracle (the experiment's accuracy) is logged, not asserted.
"""
import numpy as np
import pytest
import torch

from oracle import pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, ext, log, to_np, trimul_module

pytestmark = pytest.mark.gpu


def _fp8_bytes(rng, shape):
    """Random E4M3 codes with |value| < 4 (exponent field <= 8): normals and
    subnormals, no NaN codes."""
    sign = rng.integers(0, 2, size=shape, dtype=np.uint8) << 7
    exp = rng.integers(0, 9, size=shape, dtype=np.uint8) << 3
    man = rng.integers(0, 8, size=shape, dtype=np.uint8)
    return sign | exp | man


@pytest.mark.parametrize("P,Np", [(3, 256), (2, 512)])
def test_fp8_contraction_matches_decoded_products(P, Np):
    log(f"fp8 contraction P={P} Np={Np}")
    rng = np.random.default_rng(Np + P)
    a, b = _fp8_bytes(rng, (P, Np, Np)), _fp8_bytes(rng, (P, Np, Np))
    x = ext().tri_mul_contract_fp8(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    da, db = H.e4m3_decode(a), H.e4m3_decode(b)
    ref = da @ db.transpose(0, 2, 1)
    mag = np.abs(da) @ np.abs(db).transpose(0, 2, 1)
    err = np.abs(to_np(x).astype(np.float64) - ref)
    # bf16 rounding of the result (at most 2^-8 relative) plus the matrix
    # cores' accumulation, which is coarser than fp32 for this instruction:
    # about 97 % of the outputs equal bf16(exact sum) and the rest stay within
    # 2.2e-5 of the sum of |products| (measured on MI355X, 2 x 256^2 random
    # outputs); fp32 accumulation of exact 64-term partial sums does not
    # reproduce them.  The bound allows 6e-5.
    bound = 2.0 ** -8 * np.abs(ref) + 6e-5 * mag
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst err/bound {(err / bound).max():.2f}"


def _prologue_ab(z, m, P, eps=1e-5):
    """a and b [B, N, N, c] (pair-major, before any transpose) as the bf16
    prologue computes them before its E4M3 rounding, in float64."""
    zf = z.astype(np.float64)
    mu = zf.mean(-1, keepdims=True)
    var = ((zf - mu) ** 2).mean(-1, keepdims=True)
    xh = H.bf16_round(((zf - mu) / np.sqrt(var + eps)).astype(np.float32)).astype(np.float64)
    g = P["layer_norm_in.weight"].astype(np.float64)
    beta = P["layer_norm_in.bias"].astype(np.float64)

    def proj(name, scale):
        w = P[f"{name}.weight"].astype(np.float64)
        wf = H.bf16_round((w * g * scale).astype(np.float32)).astype(np.float64)
        return xh @ wf.T + scale * (P[f"{name}.bias"] + w @ beta)

    l2e = np.log2(np.e)
    gate = lambda name: 1.0 / (1.0 + 2.0 ** proj(name, -l2e))  # noqa: E731
    mk = m[..., None].astype(np.float64)
    a = proj("linear_a_p", 1.0) * gate("linear_a_g") * mk
    b = proj("linear_b_p", 1.0) * gate("linear_b_g") * mk
    return a, b


@pytest.mark.parametrize("outgoing", [True, False])
def test_fp8ab_forward_matches_fp8_emulation(outgoing, monkeypatch):
    B, N = 1, 300  # planes padded to 512
    log(f"fp8 a/b forward N={N} outgoing={outgoing}")
    P = H.bf16_params(H.draw_params(H.tri_mul_shapes(128, 128), seed=N + 11, ln_random=True,
                                    bias_random=True))
    z = H.bf16_round(H.pair_input(B, N, 128, seed=N + 12))
    m = H.tail_mask(B, N, [N - 20])
    mod = trimul_module(P, outgoing, torch.bfloat16)
    zd = torch.from_numpy(z).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        y = ext().tri_mul_forward_fp8ab(zd, md, mod._packed_params(False), 128, 128, outgoing)
        y_res = ext().tri_mul_forward_fp8ab(zd, md, mod._packed_params(False), 128, 128, outgoing,
                                            True)
    torch.cuda.synchronize()
    got = to_np(y)
    plain = pair_ops.tri_mul(z, m, P, outgoing, dtype=np.float32)
    a8, b8 = (H.e4m3_round(v).astype(np.float32) for v in _prologue_ab(z, m, P))
    orig = pair_ops.contract
    monkeypatch.setattr(pair_ops, "contract", lambda a, b, o, rows=None: orig(a8, b8, o, rows))
    ref = pair_ops.tri_mul(z, m, P, outgoing, dtype=np.float32)
    check_bf16(got, ref, f"fp8 a/b forward outgoing={outgoing}")
    check_bf16(to_np(y_res), ref + z, f"fp8 a/b forward + residual outgoing={outgoing}")
    rel = np.linalg.norm(got - plain) / np.linalg.norm(plain)
    log(f"  fp8 a/b against the unrounded oracle: max abs err {np.abs(got - plain).max():.3e}, "
        f"normwise relative {rel:.3e}")
