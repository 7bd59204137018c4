"""Drop-in import path of the reference's lowrank.py (README.md:24-25, test.py:3-4).

    from lowrank import lowrank_dynamic_convolution

resolves to the MI355X implementation in dynamic-conv1d_amd/dynconv/lowrank.py.
"""

import os as _os
import sys as _sys

_PKG_DIR = _os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "dynamic-conv1d_amd")
if _PKG_DIR not in _sys.path:
    _sys.path.insert(0, _PKG_DIR)

from dynconv.lowrank import lowrank_dynamic_convolution  # noqa: E402,F401
from dynconv.lowrank import _LowrankDynamicConvolutionFn  # noqa: E402,F401
from dynconv.lowrank import lowrank_dynamic_convolution_grouped  # noqa: E402,F401
from dynconv.modules import LowRankDynamicShortConvolution, GroupedLowRankDynamicShortConvolution  # noqa: E402,F401
