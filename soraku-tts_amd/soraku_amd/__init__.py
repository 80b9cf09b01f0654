"""MI355X (gfx950) per-frame CFG decode engine for soraku-TTS.

The compute runs in ``libsoraku_mi355x.so`` (hand-written HIP kernels behind
the C ABI of include/soraku_mi355x.h); this package is the host-side mirror of
the reference's engine API:

* ``GraphFrameEngine``  - acceleration/graph_frame.py:23-328
* ``FastGenerator``     - acceleration/fast_generate.py:28-569 (generate contract)
* ``ops``               - acceleration/tilelang_kernels.py operator factories
* ``load_release``      - runtime.py:14-44 (release directory -> shape + tensors)
"""

from ._lib import SkError, lib
from .checkpoint import Release, load_release
from .config import QWEN3_06B, QWEN3_17B, TINY, DecodeShape
from .engine import GraphFrameEngine
from .generate import FastGenerator

__all__ = ["DecodeShape", "FastGenerator", "GraphFrameEngine", "QWEN3_06B", "QWEN3_17B", "Release", "SkError",
           "TINY", "lib", "load_release"]
