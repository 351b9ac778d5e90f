"""Device probes and tensor-layout helpers.

API of ``src/genie_tk/utils.py`` in the reference (has_cuda_kernels :12-18,
get_device_info :21-42, permute_final_dims :45-60, flatten_final_dims,
chunk_layer :78-123).
"""
from __future__ import annotations

from typing import Any, Callable, Dict

import torch
from torch import Tensor

from genie_tk import _ext


def has_cuda_kernels() -> bool:
    """True when the gfx950 extension ``genie_tk._C`` is loaded and a GPU is visible.

    On ROCm builds of PyTorch the AMD GPU is exposed through the ``torch.cuda``
    namespace, so the name is kept from the reference.
    """
    return _ext.C is not None and torch.cuda.is_available()


def get_device_info() -> Dict[str, Any]:
    """Summary of the visible GPUs, with the keys of the reference's version."""
    avail = torch.cuda.is_available()
    info: Dict[str, Any] = {
        "cuda_available": avail,
        "cuda_kernels_available": has_cuda_kernels(),
        "device_count": torch.cuda.device_count() if avail else 0,
        "devices": [],
    }
    for idx in range(info["device_count"]):
        p = torch.cuda.get_device_properties(idx)
        info["devices"].append({
            "name": p.name,
            "total_memory": p.total_memory,
            "major": p.major,
            "minor": p.minor,
            "multi_processor_count": p.multi_processor_count,
        })
    return info


def permute_final_dims(tensor: Tensor, *order: int) -> Tensor:
    """Permute the trailing ``len(order)`` dimensions; ``order`` indexes them from 0."""
    lead = tensor.dim() - len(order)
    return tensor.permute(*range(lead), *(lead + o for o in order))


def flatten_final_dims(tensor: Tensor, num_dims: int) -> Tensor:
    """Merge the trailing ``num_dims`` dimensions into one."""
    return tensor.reshape(*tensor.shape[: tensor.dim() - num_dims], -1)


def chunk_layer(layer: Callable[..., Tensor], inputs: Dict[str, Tensor], chunk_size: int,
                no_batch_dims: int) -> Tensor:
    """Apply ``layer`` to slices of the flattened leading ``no_batch_dims`` dimensions.

    Every input shares those leading dimensions; outputs are concatenated and
    reshaped back.
    """
    first = next(iter(inputs.values()))
    batch_shape = first.shape[:no_batch_dims]
    flat = {k: v.reshape(-1, *v.shape[no_batch_dims:]) for k, v in inputs.items()}
    total = next(iter(flat.values())).shape[0]
    pieces = [layer(**{k: v[s:s + chunk_size] for k, v in flat.items()})
              for s in range(0, total, chunk_size)]
    out = torch.cat(pieces, dim=0)
    return out.reshape(*batch_shape, *out.shape[1:])
