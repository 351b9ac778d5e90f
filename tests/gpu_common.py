"""Helpers for the GPU parity tests: module builders and the bf16 tolerance."""
from __future__ import annotations

import numpy as np
import torch

from tests import helpers as H

BF16_ATOL, BF16_RTOL = 2e-2, 1e-2
FP32_ATOL = 1e-4


def ext():
    from genie_tk import _ext

    assert _ext.C is not None, f"genie_tk._C not loaded: {_ext.IMPORT_ERROR!r}"
    return _ext.C


def trimul_module(params, outgoing: bool, dtype, device="cuda"):
    from genie_tk import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    c_z = params["linear_z.weight"].shape[0]
    c = params["linear_a_p.weight"].shape[0]
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    m = cls(c_z, c, use_fused_kernel=True)
    m.load_state_dict(H.to_state_dict(params))
    m = m.to(device=device, dtype=dtype).eval()
    assert m.use_fused_kernel
    return m


def triattn_module(params, starting: bool, no_heads: int, dtype, device="cuda"):
    from genie_tk import TriangleAttentionEndingNode, TriangleAttentionStartingNode

    c_in = params["layer_norm.weight"].shape[0]
    c_h = params["mha.linear_q.weight"].shape[0]
    cls = TriangleAttentionStartingNode if starting else TriangleAttentionEndingNode
    m = cls(c_in, c_h, no_heads, use_fused_kernel=True)
    m.load_state_dict(H.to_state_dict(params))
    m = m.to(device=device, dtype=dtype).eval()
    assert m.use_fused_kernel
    return m


def check_bf16(got: np.ndarray, ref: np.ndarray, what: str) -> None:
    """|got - ref| <= 2e-2 + 1e-2 |ref| elementwise (ref: fp32 on bf16-rounded inputs)."""
    err = np.abs(got - ref)
    bound = BF16_ATOL + BF16_RTOL * np.abs(ref)
    bad = err > bound
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} elements out of tolerance; "
                           f"max err {err.max():.3e}, worst excess {(err - bound).max():.3e}")


def check_fp32(got: np.ndarray, ref: np.ndarray, what: str, atol: float = FP32_ATOL) -> None:
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref).max()
    assert err <= atol, f"{what}: max abs err {err:.3e} > {atol}"


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def log(msg: str) -> None:
    print(msg, flush=True)
