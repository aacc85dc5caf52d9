"""dl-inference on MI355X: graph engine bindings and the gfx950 operator plugin.

Same Python surface as the reference package (python/dli/__init__.py: Engine, Graph,
load_weights). torch is imported first so that the HIP runtime inside PyTorch is the one the
native libraries bind to.
"""
from __future__ import annotations

import os as _os

import torch as _torch  # noqa: F401  (must precede the native import)

from . import _dli_native
from ._dli_native import (GreedyDecoder, Graph, Node, ProfileSession, load_weights,
                          set_log_level)

_PACKAGE_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
LIB_DIR = _os.path.join(_PACKAGE_ROOT, "lib")


def plugin_path() -> str:
    """Path of the gfx950 operator plugin (exports dli_register_operators)."""
    return _os.path.join(LIB_DIR, "libdli_hip_ops.so")


def aten_plugin_path() -> str:
    """Path of the ATen CPU reference plugin (the same operator names on host tensors)."""
    return _os.path.join(LIB_DIR, "libdli_aten_ops.so")


def hip_library_path() -> str:
    """Path of the device C ABI library (include/dli_hip.h)."""
    return _os.path.join(LIB_DIR, "libdli_hip.so")


class Engine(_dli_native.Engine):
    """Graph engine. run() enqueues kernels on torch's current stream unless told otherwise."""

    def run(self, graph, inputs, stream=None, profile=None):  # noqa: D401
        """Runs graph on inputs; with profile (a ProfileSession) every node is timed."""
        if stream is None:
            stream = 0
            if _torch.cuda.is_available() and any(
                isinstance(t, _torch.Tensor) and t.is_cuda for t in inputs.values()
            ):
                stream = _torch.cuda.current_stream().cuda_stream
        return super().run(graph, inputs, int(stream), profile)

    def load_aten_plugin(self) -> "Engine":
        """Loads the ATen CPU reference plugin (graphs then run on host tensors)."""
        path = aten_plugin_path()
        if not _os.path.exists(path):
            raise RuntimeError(f"ATen CPU reference plugin is not built: {path}")
        self.load_library(path)
        return self

    def load_plugin(self) -> "Engine":
        """Loads the gfx950 plugin; raises if it was not built."""
        path = plugin_path()
        if not _os.path.exists(path):
            raise RuntimeError(f"gfx950 operator plugin is not built: {path}")
        self.load_library(path)
        return self


__all__ = ["Engine", "GreedyDecoder", "Graph", "Node", "ProfileSession", "load_weights", "plugin_path",
           "aten_plugin_path", "hip_library_path", "set_log_level"]
