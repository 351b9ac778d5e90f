"""GPU parity of the (row, head) attention walk at Np = 512 and of the online
softmax after key tiles that hold only masked keys.

(row, head) flash kernel at Np = 512 (bf16, c_in = 128, four heads of 32,
384 < N <= 512):

* B = 2 (blocks of both batch elements), starting and ending node;
* N = 390: 13 query tiles, the last key tiles all padding;
* masks: a tail (fully masked rows: the exact pass), a fully masked row and
  column inside the valid block, 5 % scattered masked pairs, and a row with
  fractional mask values (the exact pass with the mask value's bias), so that
  blocks on the max-free pass and on the exact pass run side by side;
* row chunks (a walk starting at row r0 > 0), bit-equal to the unchunked
  output, and the fused residual.

Leading masked keys (every attention kernel): rows whose first key tiles
hold only masked keys while later keys are valid.  An online softmax that
subtracts its running reference before taking a tile's maximum would, after
such tiles, hold a reference near -inf log2 e and round the valid keys'
logits to multiples of its fp32 ulp.

Checked against the oracle on sampled rows (fp32 arithmetic on the
bf16-rounded inputs; bf16 tolerance |y - y_ref| <= 2e-2 + 1e-2 |y_ref|).
"""
import numpy as np
import pytest
import torch

from oracle import pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, log, to_np, triattn_module

pytestmark = pytest.mark.gpu


def _mask(B: int, N: int, seed: int) -> np.ndarray:
    L = [N - 29, N]
    m = H.tail_mask(B, N, L)
    rng = np.random.default_rng(seed)
    m *= (rng.random(m.shape) >= 0.05).astype(np.float32)
    m[0, 100, :] = 0.0                 # a fully masked row (starting node) ...
    m[0, :, 200] = 0.0                 # ... and column (ending node)
    m[1, 37, :40] = 0.5                # fractional values in one row ...
    m[1, :40, 41] = 0.25               # ... and one column
    return m


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [390, 512])
def test_flash_np512(starting, N):
    log(f"(row, head) flash Np=512 N={N} starting={starting}")
    B = 2
    P = H.bf16_params(H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=N + 61,
                                    ln_random=True, bias_random=True))
    x = H.bf16_round(H.pair_input(B, N, 128, seed=N + 62))
    m = _mask(B, N, N + 63)
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    xd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    md = torch.from_numpy(m).to("cuda")
    with torch.no_grad():
        y = mod(xd, md)
        y_res = mod.forward_residual(xd, md)
        y_chunk = mod(xd, md, chunk_size=100)
    torch.cuda.synchronize()
    assert torch.equal(y, y_chunk), "row chunks differ from the unchunked output"
    rows = sorted({0, 1, 37, 41, 100, 200, N - 30, N - 29, N - 1})
    sel = (lambda a: a[:, rows]) if starting else (lambda a: a[:, :, rows])
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float32, rows=rows)
    check_bf16(to_np(sel(y)), ref, f"flash Np=512 N={N} starting={starting}")
    check_bf16(to_np(sel(y_res)), ref + sel(x), f"flash Np=512 residual N={N}")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [200, 600, 1152])
def test_leading_masked_keys(starting, N):
    """Rows whose first key tiles hold only masked keys while later keys are
    valid.  The online softmax of the exact pass (fractional mask values) and
    of the kernel past N = 1024 (every row) then sets its running reference
    from masked keys (about -inf log2 e) before it meets a valid key; the
    valid keys' logits must keep their precision.  Rows: 40 leading keys
    with mask 0.5 (exact pass), 40 leading keys with mask 0, and a row of
    mask 0 up to its last 5 keys."""
    log(f"leading masked keys N={N} starting={starting}")
    P = H.bf16_params(H.draw_params(H.tri_attn_shapes(128, 128, 4), seed=N + 71,
                                    ln_random=True, bias_random=True))
    x = H.bf16_round(H.pair_input(1, N, 128, seed=N + 72))
    m = np.ones((1, N, N), np.float32)
    m[0, 3, :40] = 0.5
    m[0, 9, :40] = 0.0
    m[0, 17, :N - 5] = 0.0
    if not starting:
        m = m.transpose(0, 2, 1).copy()
    mod = triattn_module(P, starting, 4, torch.bfloat16)
    with torch.no_grad():
        y = mod(torch.from_numpy(x).to("cuda", torch.bfloat16), torch.from_numpy(m).to("cuda"))
    torch.cuda.synchronize()
    rows = [0, 3, 9, 17]
    sel = (lambda a: a[:, rows]) if starting else (lambda a: a[:, :, rows])
    ref = pair_ops.tri_attn(x, m, P, starting, 4, dtype=np.float32, rows=rows)
    check_bf16(to_np(sel(y)), ref, f"leading masked keys N={N} starting={starting}")
