"""GPU parity against the golden fixtures (float64 scalar-loop results): the
fp32 HIP path, through the genie_tk modules and the reference-surface _C
operators, within max abs error 1e-4."""
import numpy as np
import pytest
import torch

from tests.gpu_common import check_fp32, ext, log, to_np, trimul_module, triattn_module
from tests.test_golden import load, params

pytestmark = pytest.mark.gpu


def _dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


@pytest.mark.parametrize("outgoing", [True, False])
def test_golden_tri_mul_fp32(outgoing):
    log(f"golden tri-mul fp32 N=8 c=64 outgoing={outgoing}")
    g = load("tri_mul_n8.npz")
    mod = trimul_module(params(g), outgoing, torch.float32)
    with torch.no_grad():
        y = mod(_dev(g["z"]), _dev(g["mask"]))
    check_fp32(to_np(y), g["outgoing" if outgoing else "incoming"], f"golden tri-mul {outgoing}")


@pytest.mark.parametrize("starting", [True, False])
def test_golden_tri_attn_fp32(starting):
    log(f"golden tri-attn fp32 N=8 starting={starting}")
    g = load("tri_attn_n8.npz")
    mod = triattn_module(params(g), starting, 4, torch.float32)
    with torch.no_grad():
        y = mod(_dev(g["x"]), _dev(g["mask"]))
    check_fp32(to_np(y), g["starting" if starting else "ending"], f"golden tri-attn {starting}")


def test_golden_raw_operators_fp32():
    log("golden raw operators fp32 N=8")
    C = ext()
    g = load("raw_ops_n8.npz")
    a, b, m = _dev(g["a"]), _dev(g["b"]), _dev(g["mask"])
    check_fp32(to_np(C.triangle_mul_outgoing(a, b, m)), g["contract_outgoing"], "contract out")
    check_fp32(to_np(C.triangle_mul_incoming(a, b, m)), g["contract_incoming"], "contract in")
    q, k, v, bias = (_dev(g[n]) for n in ("q", "k", "v", "bias"))
    s = float(g["scale"])
    check_fp32(to_np(C.triangle_attention_starting(q, k, v, bias, m, s)), g["attention_starting"],
               "attention starting")
    check_fp32(to_np(C.triangle_attention_ending(q, k, v, bias, m, s)), g["attention_ending"],
               "attention ending")
    y = C.layernorm(_dev(g["ln_x"]), _dev(g["ln_w"]), _dev(g["ln_b"]), 1e-5)
    check_fp32(to_np(y), g["layer_norm"], "layernorm")
