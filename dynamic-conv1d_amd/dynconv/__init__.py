"""dynconv: MI355X-native dynamic short convolutions (headwise and lowrank).

Public API (same as the reference's headwise.py / lowrank.py):
    headwise_dynamic_convolution(x, weight, static_w=None, residual=False)
    lowrank_dynamic_convolution(x, z, U, static_w=None, residual=False)

Beyond the reference's operators: lowrank_dynamic_convolution_grouped (the
q / k / v convolutions of one layer in one launch per direction, README.md:57-110)
and the README's LowRankDynamicShortConvolution module, plus its grouped form.

Both are torch.autograd.Functions backed by hand-written gfx950 HIP kernels
in libdynconv.so, reached through a C ABI (include/dynconv.h).
"""

from .headwise import headwise_dynamic_convolution, _HeadwiseDynamicConvolutionFn  # noqa: F401
from .lowrank import lowrank_dynamic_convolution, _LowrankDynamicConvolutionFn  # noqa: F401
from .lowrank import lowrank_dynamic_convolution_grouped  # noqa: F401
from .modules import LowRankDynamicShortConvolution, GroupedLowRankDynamicShortConvolution  # noqa: F401
from ._capi import LIB_PATH, load as load_library  # noqa: F401

__all__ = [
    "headwise_dynamic_convolution",
    "lowrank_dynamic_convolution",
    "lowrank_dynamic_convolution_grouped",
    "LowRankDynamicShortConvolution",
    "GroupedLowRankDynamicShortConvolution",
    "load_library",
    "LIB_PATH",
]
