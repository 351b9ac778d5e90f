"""Shared plumbing of the modules' kernel path: capability checks, the packed
weight cache and the autograd rule.

A call on a GPU tensor with ``use_fused_kernel=True`` runs the HIP kernels.
When it must produce gradients (autograd enabled and the input or a
parameter requires grad), the triangle modules run their kernel forward
inside an autograd Function whose backward is the kernels' backward; the
modules without backward kernels (PairTransition) run their PyTorch path
then.
"""
from __future__ import annotations

import warnings
import weakref
from typing import Callable, Dict, List, Optional, Tuple

import torch
from torch import Tensor, nn

SUPPORTED_DTYPES = (torch.float32, torch.bfloat16)

_warned: set = set()


def needs_autograd(x: Tensor, module: nn.Module) -> bool:
    if not torch.is_grad_enabled():
        return False
    return x.requires_grad or any(p.requires_grad for p in module.parameters())


# binary_mask results per live mask tensor: id -> (weak reference, version, result)
_binary_seen: Dict[int, Tuple["weakref.ref", int, bool]] = {}


def binary_mask(mask: Optional[Tensor]) -> bool:
    """True when every mask value is 0 or 1 (or there is no mask).  One
    reduction and a host synchronisation, used only on the training path and
    remembered for the tensor until it is modified in place or freed: the
    layers of a network share one mask, which then costs one synchronisation
    instead of one per attention call."""
    if mask is None:
        return True
    key = id(mask)
    seen = _binary_seen.get(key)
    if seen is not None and seen[0]() is mask and seen[1] == mask._version:
        return seen[2]
    result = bool(((mask == 0) | (mask == 1)).all())
    if len(_binary_seen) >= 64:
        _binary_seen.clear()
    # the entry goes when the tensor does, before its id can be reused
    _binary_seen[key] = (weakref.ref(mask, lambda _, k=key: _binary_seen.pop(k, None)),
                         mask._version, result)
    return result


def warn_once(key: str, msg: str) -> None:
    if key not in _warned:
        _warned.add(key)
        warnings.warn(msg, stacklevel=3)


def params_at(module: nn.Module, paths: Tuple[Tuple[str, ...], ...]) -> List[Tensor]:
    """The parameters of ``module`` at ``paths`` (("linear_a_p", "weight"),
    ("mha", "linear_q", "weight"), ...), read through the submodules'
    ``_modules`` and ``_parameters`` dicts: an attribute lookup through
    nn.Module.__getattr__ costs about half a microsecond, and the kernel path
    reads 6-16 parameters on every call.  A replaced submodule or parameter
    is seen at once (nothing is cached here)."""
    out = []
    for path in paths:
        mod = module
        for name in path[:-1]:
            mod = mod._modules[name]
        out.append(mod._parameters[path[-1]])
    return out


class PackedWeights:
    """Device copy of a module's parameters in the kernels' fragment order.

    Rebuilt when any parameter is replaced or moved (its data pointer),
    modified in place (its version counter), or when the compute precision
    changes.
    """

    def __init__(self) -> None:
        self._key: Optional[Tuple] = None
        self._packed: Optional[Tensor] = None

    def get(self, params: List[Tensor], fp32: bool,
            pack: Callable[[List[Tensor], bool], Tensor]) -> Tensor:
        p0 = params[0]
        key = [fp32, p0.device, p0.dtype]
        for p in params:
            key.append(p.data_ptr())
            key.append(p._version)
        if key != self._key or self._packed is None:
            with torch.no_grad():
                self._packed = pack([p.detach() for p in params], fp32)
            self._key = key
        return self._packed


def grads_as_params(grads: List[Tensor], flat: Optional[Tensor], params: List[Tensor]) -> List[Tensor]:
    """Parameter gradients in their parameters' dtypes.  ``grads`` are fp32;
    when ``flat`` is given they are views of it (the backward bindings'
    layout) and, if every parameter has one non-fp32 dtype, one cast of
    ``flat`` replaces a cast per gradient."""
    dt = params[0].dtype
    if flat is not None and dt != torch.float32 and all(p.dtype == dt for p in params):
        fc = flat.to(dt)
        return [fc.as_strided(g.shape, g.stride(), g.storage_offset()) for g in grads]
    return [g.to(p.dtype) for g, p in zip(grads, params)]


def flatten_batch(x: Tensor, mask: Optional[Tensor]) -> Tuple[Tensor, Optional[Tensor], Tuple]:
    """[*, N, N, C] -> [B, N, N, C] (and the mask likewise); returns the leading shape."""
    if x.dim() == 4 and (mask is None or mask.shape == x.shape[:-1]):
        return x, mask, (x.shape[0],)  # already [B, N, N, C] (the common call)
    lead = tuple(x.shape[:-3])
    n, c = x.shape[-2], x.shape[-1]
    xb = x.reshape(-1, n, n, c)
    mb = None if mask is None else mask.expand(*lead, n, n).reshape(-1, n, n)
    return xb, mb, lead

