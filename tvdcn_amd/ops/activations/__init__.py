"""Mask activations, same names as tvdcn/ops/activations/__init__.py."""
from .mask_sigmoid import *  # noqa: F401,F403
from .mask_softmax import *  # noqa: F401,F403
