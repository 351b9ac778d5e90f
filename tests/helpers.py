"""Seeded parameter/input builders shared by the tests, bench.py and smoke().

Parameters are numpy float32 arrays keyed by the reference modules'
state_dict names, drawn with numpy's PCG64 generator in sorted-key order so
that a (shape, seed) pair always yields the same weights.
"""
from __future__ import annotations

from typing import Dict, Optional, Sequence

import numpy as np

TRI_MUL_LINEARS = ["linear_a_p", "linear_a_g", "linear_b_p", "linear_b_g", "linear_g", "linear_z"]
TRI_MUL_GATES = ("linear_a_g", "linear_b_g", "linear_g")


def tri_mul_shapes(c_z: int, c: int) -> Dict[str, tuple]:
    return {
        "layer_norm_in.weight": (c_z,), "layer_norm_in.bias": (c_z,),
        "linear_a_p.weight": (c, c_z), "linear_a_p.bias": (c,),
        "linear_a_g.weight": (c, c_z), "linear_a_g.bias": (c,),
        "linear_b_p.weight": (c, c_z), "linear_b_p.bias": (c,),
        "linear_b_g.weight": (c, c_z), "linear_b_g.bias": (c,),
        "linear_g.weight": (c_z, c_z), "linear_g.bias": (c_z,),
        "layer_norm_out.weight": (c,), "layer_norm_out.bias": (c,),
        "linear_z.weight": (c_z, c), "linear_z.bias": (c_z,),
    }


def tri_attn_shapes(c_in: int, c_h: int, H: int) -> Dict[str, tuple]:
    return {
        "layer_norm.weight": (c_in,), "layer_norm.bias": (c_in,),
        "linear.weight": (H, c_in),
        "mha.linear_q.weight": (c_h, c_in), "mha.linear_k.weight": (c_h, c_in),
        "mha.linear_v.weight": (c_h, c_in),
        "mha.linear_o.weight": (c_in, c_h), "mha.linear_o.bias": (c_in,),
        "mha.linear_g.weight": (c_h, c_in), "mha.linear_g.bias": (c_h,),
    }


def pair_transition_shapes(c: int, n: int = 4) -> Dict[str, tuple]:
    return {
        "layer_norm.weight": (c,), "layer_norm.bias": (c,),
        "linear_1.weight": (n * c, c), "linear_1.bias": (n * c,),
        "linear_2.weight": (c, n * c), "linear_2.bias": (c,),
    }


def pair_layer_shapes(c: int, c_mul: int, c_att: int, heads: int, n: int = 4) -> Dict[str, tuple]:
    """state_dict shapes of PairTransformLayer (pair_transform.py:87-178)."""
    out = {}
    for name, sub in (("tri_mul_out", tri_mul_shapes(c, c_mul)), ("tri_mul_in", tri_mul_shapes(c, c_mul)),
                      ("tri_att_start", tri_attn_shapes(c, c_att, heads)),
                      ("tri_att_end", tri_attn_shapes(c, c_att, heads)),
                      ("pair_transition", pair_transition_shapes(c, n))):
        out.update({f"{name}.{k}": v for k, v in sub.items()})
    return out


def draw_params(shapes: Dict[str, tuple], seed: int, *, ln_random: bool = False,
                bias_random: bool = False, gate_bias: Optional[float] = None,
                gate_keys: Sequence[str] = (), tri_std: Optional[float] = None) -> Dict[str, np.ndarray]:
    """Weights ~ N(0, 1/fan_in); LN gamma=1, beta=0 and biases 0 unless randomised.

    gate_bias sets the bias of every Linear named in ``gate_keys``;
    tri_std overrides the std of the triangle-bias projection ``linear.weight``.
    """
    rng = np.random.default_rng(seed)
    out = {}
    for key in sorted(shapes):
        shape = shapes[key]
        if key.endswith(".weight") and len(shape) == 2:
            std = 1.0 / np.sqrt(shape[1])
            if key == "linear.weight" and tri_std is not None:
                std = tri_std
            v = rng.standard_normal(shape) * std
        elif "layer_norm" in key:
            if ln_random:
                base = 1.0 if key.endswith("weight") else 0.0
                v = base + 0.2 * rng.standard_normal(shape)
            else:
                v = np.ones(shape) if key.endswith("weight") else np.zeros(shape)
        else:  # Linear bias
            mod = key.rsplit(".", 1)[0]
            if gate_bias is not None and mod in gate_keys:
                v = np.full(shape, gate_bias)
            elif bias_random:
                v = 0.3 * rng.standard_normal(shape)
            else:
                v = np.zeros(shape)
        out[key] = np.asarray(v, dtype=np.float32)
    return out


def pair_input(B: int, N: int, C: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((B, N, N, C)).astype(np.float32)


def tail_mask(B: int, N: int, lengths: Sequence[int]) -> np.ndarray:
    """m[b, i, j] = [i < len_b][j < len_b]."""
    m = np.zeros((B, N, N), dtype=np.float32)
    for b, L in enumerate(lengths):
        m[b, :L, :L] = 1.0
    return m


def to_state_dict(params: Dict[str, np.ndarray], dtype=None, device="cpu"):
    import torch

    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}
    return {k: v.to(device=device, dtype=dtype or v.dtype) for k, v in sd.items()}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return rounded.astype(np.uint32).view(np.float32)


def bf16_params(params: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    return {k: bf16_round(v) for k, v in params.items()}


# ---------------------------------------------------------------------------
# OCP fp8 E4M3 (the "fn" variant: bias 7, 3 mantissa bits, no infinity,
# S.1111.111 = NaN, largest finite 448), for the fp8 a/b storage experiment.
# ---------------------------------------------------------------------------
def e4m3_decode(b: np.ndarray) -> np.ndarray:
    """Bytes -> float64 values (NaN codes give NaN)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    return np.where((b & 0x7F) == 0x7F, np.nan, s * val)


def e4m3_round(x: np.ndarray) -> np.ndarray:
    """Nearest E4M3 value (ties to even), after clamping to +-448; float64."""
    x = np.clip(np.asarray(x, dtype=np.float64), -448.0, 448.0)
    a = np.abs(x)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -6)))  # subnormals share the 2^-6 binade's step
    q = 2.0 ** (e - 3)                                # spacing of the values in that binade
    return np.sign(x) * np.round(a / q) * q           # np.round: ties to even
