"""graph_horizon_amd — MI355X (gfx950) numeric backend for graph_horizon_engine.

The product is libgh_hip.so (C ABI: include/gh_backend.h) plus its gfx950 code objects in
graph_horizon_amd/lib/. This package holds the Python mirror of the engine's Backend trait
(`backend.HipBackend`), the graph driver handle (`backend.HipModel`), GGUF files (`gguf`: the
native reader's binding and a writer), seeded synthetic GGUF tensors (`synth`) and the in-tree
build (`build`).
"""
from . import _ffi  # noqa: F401
from ._ffi import GhSampling  # noqa: F401
from .backend import GhError, HipBackend, HipModel, Yarn  # noqa: F401
