"""kanforge_amd — the fused KAN basis hot path of kanforge, MI355X-native.

The spline part of ``KANLinear`` (F/G/P primitives, edge derivatives) runs on
hand-written HIP kernels for gfx950 behind the C ABI of libkfhip.so
(include/kfhip.h)::

    from kanforge_amd.torch import KANLinear, KAN, GRKAN
"""

from . import bases
from .bases import *  # noqa: F401,F403
from .bases import __all__ as _bases_all

__version__ = "0.1.0"

__all__ = [*_bases_all, "bases", "__version__"]
