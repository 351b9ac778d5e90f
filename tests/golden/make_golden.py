"""Write the golden fixtures of the pair hot path (run from the repo root:
``python tests/golden/make_golden.py``).

Every expected output is computed by oracle/brute.py's scalar loops in float64
from float32 inputs drawn with numpy's PCG64 generator (tests/helpers.py).
The reference ships no golden vectors of its own, so these fixtures pin the
oracle and the kernels to the equations of src/genie_tk/triangle_mul.py:77-132,
src/genie_tk/triangle_attention.py:84-143 and src/genie_tk/primitives.py:114-178,
at the channel sizes the kernels are built for (c_z = c_in = 128, c in {64},
H = 4, d = 32) and a ragged N = 8.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402
from tests import helpers as H  # noqa: E402

N = 8


def _mask():
    m = H.tail_mask(1, N, [6])
    m[0, 2, 4] = 0.0  # an isolated masked pair inside the valid block
    return m


def tri_mul():
    P = H.draw_params(H.tri_mul_shapes(128, 64), 100, ln_random=True, bias_random=True)
    z = H.pair_input(1, N, 128, seed=100)
    m = _mask()
    out = {f"param.{k}": v for k, v in P.items()}
    out.update(z=z, mask=m,
               outgoing=brute.tri_mul(z, m, P, True),
               incoming=brute.tri_mul(z, m, P, False))
    return out


def tri_attn():
    P = H.draw_params(H.tri_attn_shapes(128, 128, 4), 101, ln_random=True, bias_random=True,
                      tri_std=1.0 / np.sqrt(128))
    x = H.pair_input(1, N, 128, seed=101)
    m = _mask()
    m[0, 7, :] = 0.0  # row 7 has no valid key in the starting direction
    out = {f"param.{k}": v for k, v in P.items()}
    out.update(x=x, mask=m,
               starting=brute.tri_attn(x, m, P, True, 4),
               ending=brute.tri_attn(x, m, P, False, 4))
    return out


def raw_ops():
    rng = np.random.default_rng(102)
    a = rng.standard_normal((1, N, N, 16)).astype(np.float32)
    b = rng.standard_normal((1, N, N, 16)).astype(np.float32)
    q = rng.standard_normal((1, 4, N, N, 32)).astype(np.float32)
    k = rng.standard_normal((1, 4, N, N, 32)).astype(np.float32)
    v = rng.standard_normal((1, 4, N, N, 32)).astype(np.float32)
    bias = rng.standard_normal((1, 4, N, N)).astype(np.float32)
    m = _mask()
    scale = float(np.float32(1.0 / np.sqrt(32)))
    rows = rng.standard_normal((16, 128)).astype(np.float32) * 2 + 0.5
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    beta = (0.2 * rng.standard_normal(128)).astype(np.float32)
    return dict(a=a, b=b, contract_outgoing=brute.contract(a, b, True),
                contract_incoming=brute.contract(a, b, False),
                q=q, k=k, v=v, bias=bias, mask=m, scale=np.float64(scale),
                attention_starting=brute.attention_core(q, k, v, bias, m, scale, True),
                attention_ending=brute.attention_core(q, k, v, bias, m, scale, False),
                ln_x=rows, ln_w=w, ln_b=beta, layer_norm=brute.layer_norm(rows, w, beta))


FIXTURES = {"tri_mul_n8.npz": tri_mul, "tri_attn_n8.npz": tri_attn, "raw_ops_n8.npz": raw_ops}


def main():
    for name, fn in FIXTURES.items():
        np.savez_compressed(os.path.join(HERE, name), **fn())
        print("wrote", name)


if __name__ == "__main__":
    main()
