"""tvdcn_amd: MI355X (gfx950) deformable convolution with tvdcn's Python API.

The implementation package behind ``import tvdcn`` (the top-level ``tvdcn`` package
re-exports it under the reference's module names). It has the same public names as
tvdcn/__init__.py: the functional ops, the modules, the mask activations and the
capability queries. The ops are the native ``torch.ops.tvdcn.*`` operators; their
GPU kernels are hand-written HIP only.
"""
from . import ops
from ._version import __version__
from .extension import _HAS_OPS, cuda_arch_list, cuda_version, has_ops, set_keep_channels_last_copy, with_cuda
from .ops import *  # noqa: F401,F403
