"""Loader for the compiled extension ``genie_tk._C``.

``C`` is the module, or None when it is not built; ``IMPORT_ERROR`` keeps the
reason.  Modules asked to run their fused path on a GPU tensor call
``require()``, which raises instead of silently using the PyTorch path.
"""
from __future__ import annotations

import torch  # noqa: F401  (loads torch's HIP runtime before the extension)

C = None
IMPORT_ERROR: BaseException | None = None
try:
    from genie_tk import _C as C  # type: ignore[attr-defined]
except ImportError as exc:  # not built in this tree
    IMPORT_ERROR = exc


def require():
    """Return the extension module or raise ImportError naming the cause."""
    if C is None:
        raise ImportError(
            "genie_tk._C (the gfx950 HIP extension) is not available: "
            f"{IMPORT_ERROR!r}. Build it with `python genie-tk_amd/build.py`.")
    return C
