"""tvdcn_amd: MI355X (gfx950) deformable convolution with tvdcn's Python API.

``import tvdcn_amd as tvdcn`` gives the same public names as ``import tvdcn``
(tvdcn/__init__.py): the functional ops, the modules, the mask activations and
the capability queries. The ops run on hand-written HIP kernels only; there is
no CPU path.
"""
from . import ops
from ._version import __version__
from .extension import _HAS_OPS, cuda_arch_list, cuda_version, has_ops, with_cuda
from .ops import *  # noqa: F401,F403
