"""Loader for the native extension ``cufk_amd._C`` (which links ``libcufk_hip.so``).

There is no fallback: if the in-tree build is missing, importing the package raises
ImportError naming the build command.
"""

from __future__ import annotations

from pathlib import Path

_PKG = Path(__file__).resolve().parent

try:
    from . import _C  # noqa: F401
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        f"cufk_amd native extension not built in {_PKG} ({exc}); run `python cufk_amd/_build.py`"
    ) from exc

HIP_LIBRARY = _PKG / "libcufk_hip.so"
