"""``import tvdcn``: the reference's package name for this MI355X (gfx950) build.

A drop-in for tvdcn 1.1.0's Python package (tvdcn/__init__.py:1-4): the same public
names (functional ops, modules, mask activations, capability queries) and the same
submodules (``tvdcn.ops``, ``tvdcn.ops.activations``, ``tvdcn.ops.deform_conv``,
``tvdcn.ops.deform_conv_transpose``, ``tvdcn.extension``, ``tvdcn.utils``), served by the
implementation package ``tvdcn_amd``, whose native library registers the ops as
``torch.ops.tvdcn.*`` with the reference's schemas.
"""
import sys as _sys

import tvdcn_amd as _impl
from tvdcn_amd import _version, extension, ops, utils  # noqa: F401
from tvdcn_amd._version import __version__  # noqa: F401
from tvdcn_amd.extension import (  # noqa: F401
    _HAS_OPS, cuda_arch_list, cuda_version, has_ops, set_keep_channels_last_copy, with_cuda)
from tvdcn_amd.ops import *  # noqa: F401,F403

for _name in ("ops", "ops.activations", "ops.activations.mask_sigmoid", "ops.activations.mask_softmax",
              "ops.deform_conv", "ops.deform_conv_transpose", "extension", "utils", "_version"):
    _sys.modules[f"{__name__}.{_name}"] = _sys.modules[f"{_impl.__name__}.{_name}"]
del _name
