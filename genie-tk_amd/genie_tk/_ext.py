"""Loader for the compiled extension ``genie_tk._C``.

``C`` is the module, or None when it is not built; ``IMPORT_ERROR`` keeps the
reason.

A module asked for its fused path on a GPU tensor while ``_C`` is missing
behaves as the reference does (src/genie_tk/triangle_mul.py:24-30,61;
triangle_attention.py:25-31,67): it runs its PyTorch path.  Unlike the
reference it says so, once per module class, with a RuntimeWarning.  With the
environment variable ``GENIE_TK_STRICT=1`` (set by this repository's tests,
``smoke()`` and ``bench.py``) it raises ImportError instead, so that an
unbuilt library can never pass for a working one.
"""
from __future__ import annotations

import os
import warnings

import torch  # noqa: F401  (loads torch's HIP runtime before the extension)

C = None
IMPORT_ERROR: BaseException | None = None
try:
    from genie_tk import _C as C  # type: ignore[attr-defined]
except ImportError as exc:  # not built in this tree
    IMPORT_ERROR = exc

STRICT_ENV = "GENIE_TK_STRICT"
_warned: set = set()


def strict() -> bool:
    """True when a missing extension must raise (``GENIE_TK_STRICT`` set and not "0")."""
    return os.environ.get(STRICT_ENV, "") not in ("", "0")


def _missing_message() -> str:
    return ("genie_tk._C (the gfx950 HIP extension) is not available: "
            f"{IMPORT_ERROR!r}. Build it with `python genie-tk_amd/build.py`.")


def require():
    """Return the extension module or raise ImportError naming the cause."""
    if C is None:
        raise ImportError(_missing_message())
    return C


def missing(what: str) -> None:
    """Called when ``what`` was asked for its kernel path on a GPU tensor and
    the extension is missing: raises under strict mode, else warns once and
    lets the caller run its PyTorch path."""
    if strict():
        raise ImportError(_missing_message())
    if what not in _warned:
        _warned.add(what)
        warnings.warn(f"{what}: {_missing_message()} Running the PyTorch path.",
                      RuntimeWarning, stacklevel=3)
