"""ictc_o3 on AMD MI355X: the equivariant operator hot path (channelwise CG tensor
product, graph message, symmetric contraction) on hand-written HIP kernels for
gfx950, behind the reference library's public operator API."""
from ictc_o3.operators import *  # noqa: F401,F403
from ictc_o3.operators import __all__  # noqa: F401
