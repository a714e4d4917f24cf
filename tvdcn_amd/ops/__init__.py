"""tvdcn_amd.ops -- same names as tvdcn.ops (tvdcn/ops/__init__.py)."""
from .activations import *  # noqa: F401,F403
from .deform_conv import *  # noqa: F401,F403
from .deform_conv_transpose import *  # noqa: F401,F403
