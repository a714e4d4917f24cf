"""Mask activations: ``mask_softmax{1,2,3}d`` / ``MaskSoftmax{1,2,3}d`` and ``mask_sigmoid`` / ``MaskSigmoid``.

Same API as tvdcn/ops/activations/mask_softmax.py:19-184 and mask_sigmoid.py:11-39.
The softmax over the kernel taps of each mask group runs in the
``tvdcn_amd::mask_softmax`` HIP kernel (forward and backward), not in
``torch.softmax``.
"""
from typing import Optional, Tuple

import torch
from torch import Tensor, nn
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t, _size_any_t
from torch.nn.modules.utils import _pair, _single, _triple

from ..extension import _assert_has_ops

__all__ = [
    "mask_softmax1d", "mask_softmax2d", "mask_softmax3d",
    "MaskSoftmax1d", "MaskSoftmax2d", "MaskSoftmax3d",
    "mask_sigmoid", "MaskSigmoid",
]

_NTUPLE = {1: _single, 2: _pair, 3: _triple}


def _mask_softmax(mask: Tensor, kernel_size, dim: int) -> Tensor:
    kernel_size = _NTUPLE[dim](kernel_size)
    if mask.dim() != dim + 2:
        raise RuntimeError(f"mask_softmax{dim}d expects a batched mask of {dim + 2} dimensions, "
                           f"got {mask.dim()}")
    kernel_numel = 1
    for k in kernel_size:
        kernel_numel *= int(k)
    if mask.size(1) // kernel_numel == 0:
        names = " * ".join(f"kernel_size[{i}]" for i in range(dim))
        raise RuntimeError(
            "The shape of the mask tensor at dimension 1 is not valid. It should "
            f"be a multiple of {names}.\n"
            f"Got mask.size(1)={mask.size(1)}, while {names}={kernel_numel}")
    _assert_has_ops()
    return torch.ops.tvdcn_amd.mask_softmax(mask, kernel_numel)


def mask_softmax1d(mask: Tensor, kernel_size: Tuple[int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kernel_w, out_w) mask over the kernel taps of each group."""
    return _mask_softmax(mask, kernel_size, 1)


def mask_softmax2d(mask: Tensor, kernel_size: Tuple[int, int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kh * kw, out_h, out_w) mask over the kernel taps of each group
    (DCNv3, https://arxiv.org/abs/2211.05778)."""
    return _mask_softmax(mask, kernel_size, 2)


def mask_softmax3d(mask: Tensor, kernel_size: Tuple[int, int, int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kd * kh * kw, out_d, out_h, out_w) mask over the kernel taps."""
    return _mask_softmax(mask, kernel_size, 3)


class _MaskSoftmaxNd(nn.Module):
    _dim = 0

    def __init__(self, kernel_size: _size_any_t):
        super().__init__()
        self.kernel_size: Tuple[int, ...] = _NTUPLE[self._dim](kernel_size)

    def forward(self, mask: Tensor, kernel_size: Optional[_size_any_t] = None) -> Tensor:
        return _mask_softmax(mask, kernel_size if kernel_size is not None else self.kernel_size, self._dim)


class MaskSoftmax1d(_MaskSoftmaxNd):
    """See :func:`mask_softmax1d`."""
    _dim = 1

    def __init__(self, kernel_size: _size_1_t) -> None:
        super().__init__(kernel_size)


class MaskSoftmax2d(_MaskSoftmaxNd):
    """See :func:`mask_softmax2d`."""
    _dim = 2

    def __init__(self, kernel_size: _size_2_t) -> None:
        super().__init__(kernel_size)


class MaskSoftmax3d(_MaskSoftmaxNd):
    """See :func:`mask_softmax3d`."""
    _dim = 3

    def __init__(self, kernel_size: _size_3_t) -> None:
        super().__init__(kernel_size)


def mask_sigmoid(mask: Tensor, scale: float = 2.0) -> Tensor:
    r"""``scale * sigmoid(mask)``; with the default scale 2, a zero-initialised mask generator yields 1."""
    if scale <= 0:
        raise ValueError(f"scale must be positive. Got scale={scale}")
    return torch.sigmoid(mask) * scale


class MaskSigmoid(nn.Module):
    """See :func:`mask_sigmoid`."""

    def __init__(self, scale: float = 2.0):
        super().__init__()
        self.scale = float(scale)

    def forward(self, mask: Tensor) -> Tensor:
        return mask_sigmoid(mask, self.scale)
