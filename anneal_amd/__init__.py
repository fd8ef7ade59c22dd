"""anneal_amd — MI355X (gfx950) backend for georgebuilds/anneal's training hot path.

The compute path is libanneal_hip.so (hand-written HIP kernels behind a C ABI, include/anneal_hip.h);
this package only binds it. Importing the package does not load the library; the first Device() does,
and raises if the library was not built.
"""
from . import data  # noqa: F401
from ._lib import AnnealHipError, load  # noqa: F401

__all__ = ["data", "load", "AnnealHipError"]
