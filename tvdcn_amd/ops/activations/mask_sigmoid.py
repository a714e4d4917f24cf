"""``mask_sigmoid`` / ``MaskSigmoid``: ``scale * sigmoid(mask)`` (tvdcn/ops/activations/mask_sigmoid.py:11-39).

Plain torch operations, as in the reference. The packed modules do not run this
module when it is their mask activation: the kernels apply it in their mask load.
"""
import torch
from torch import Tensor, nn

__all__ = ["mask_sigmoid", "MaskSigmoid"]


def mask_sigmoid(mask: Tensor, scale: float = 2.0) -> Tensor:
    r"""``scale * sigmoid(mask)``; with the default scale 2, a zero-initialised mask generator yields 1."""
    if scale <= 0:
        raise ValueError("scale must be positive. Got scale={}".format(scale))
    return torch.sigmoid(mask) * scale


class MaskSigmoid(nn.Module):
    """See :func:`mask_sigmoid`."""

    def __init__(self, scale: float = 2.0):
        super().__init__()
        self.scale = float(scale)

    def forward(self, mask: Tensor) -> Tensor:
        return mask_sigmoid(mask, self.scale)
