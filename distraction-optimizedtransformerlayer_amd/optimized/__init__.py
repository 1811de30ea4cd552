"""The optimized transformer layer on MI355X (gfx950) kernels.

Same modules and public names as the reference's optimized/ package
(reference optimized/__init__.py:1-36), in reading order:

    config.py    runtime knobs, read at call time
    cli.py       command-line overrides for the knobs
    model.py     OptimizedTransformer, the whole forward pass
    layers.py    submodules with the baseline's parameter names
    kernels.py   dispatch into libdotl_hip.so through kernel_ext
    graphs.py    hipGraph capture and replay
    util.py      small shared helpers

A harness declares `class UserOptimizedTransformer(OptimizedTransformer,
BaselineTransformer)`, keeping the optimized model an instance of its
baseline class without this package importing the harness.
"""

from . import cli, config, graphs, kernels, layers, util
from .model import OptimizedTransformer

__all__ = ["OptimizedTransformer", "cli", "config", "graphs", "kernels", "layers", "util"]
