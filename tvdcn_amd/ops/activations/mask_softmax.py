"""``mask_softmax{1,2,3}d`` / ``MaskSoftmax{1,2,3}d``: softmax of a mask over the kernel taps of each group.

Same API as tvdcn/ops/activations/mask_softmax.py:19-184: the mask
(batch, mask_groups * prod(kernel_size), *spatial) is viewed as
(batch, mask_groups, prod(kernel_size), *spatial) and normalised over the third axis.
On the GPU the softmax runs in the ``tvdcn::mask_softmax`` HIP kernel (forward and
backward); CPU tensors take the same definition through ATen. Written for TorchScript
(the modules script, as in tvdcn's examples).
"""
from typing import List, Optional, Tuple

import torch
from torch import Tensor, nn
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t, _size_any_t

from ...extension import _assert_has_ops
from ...utils import _ints1, _ints2, _ints3

__all__ = [
    "mask_softmax1d", "mask_softmax2d", "mask_softmax3d",
    "MaskSoftmax1d", "MaskSoftmax2d", "MaskSoftmax3d",
]


def _mask_softmax(mask: Tensor, kernel_size: List[int], dim: int) -> Tensor:
    if mask.dim() != dim + 2:
        raise RuntimeError("mask_softmax{}d expects a batched mask of {} dimensions, got {}".format(
            dim, dim + 2, mask.dim()))
    kernel_numel = 1
    for k in kernel_size:
        kernel_numel *= k
    if mask.size(1) // kernel_numel == 0:
        names: List[str] = []
        for i in range(dim):
            names.append("kernel_size[{}]".format(i))
        joined = " * ".join(names)
        raise RuntimeError(
            "The shape of the mask tensor at dimension 1 is not valid. It should be a multiple of {}.\n"
            "Got mask.size(1)={}, while {}={}".format(joined, mask.size(1), joined, kernel_numel))
    _assert_has_ops()
    return torch.ops.tvdcn.mask_softmax(mask, kernel_numel)


def mask_softmax1d(mask: Tensor, kernel_size: Tuple[int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kernel_w, out_w) mask over the kernel taps of each group."""
    return _mask_softmax(mask, _ints1(kernel_size), 1)


def mask_softmax2d(mask: Tensor, kernel_size: Tuple[int, int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kh * kw, out_h, out_w) mask over the kernel taps of each group
    (DCNv3, https://arxiv.org/abs/2211.05778)."""
    return _mask_softmax(mask, _ints2(kernel_size), 2)


def mask_softmax3d(mask: Tensor, kernel_size: Tuple[int, int, int]) -> Tensor:
    r"""Softmax of a (batch, mask_groups * kd * kh * kw, out_d, out_h, out_w) mask over the kernel taps."""
    return _mask_softmax(mask, _ints3(kernel_size), 3)


class _MaskSoftmaxNd(nn.Module):
    """Base of the mask softmax modules (tvdcn/ops/activations/mask_softmax.py:132-141)."""

    def __init__(self, kernel_size: _size_any_t):
        super().__init__()
        self.kernel_size = kernel_size

    def forward(self, mask: Tensor, kernel_size: Optional[_size_any_t] = None) -> Tensor:
        raise NotImplementedError


class MaskSoftmax1d(_MaskSoftmaxNd):
    """See :func:`mask_softmax1d`."""

    def __init__(self, kernel_size: _size_1_t) -> None:
        super().__init__(tuple(_ints1(kernel_size)))

    def forward(self, mask: Tensor, kernel_size: Optional[Tuple[int]] = None) -> Tensor:
        if kernel_size is None:
            return mask_softmax1d(mask, self.kernel_size)
        return mask_softmax1d(mask, kernel_size)


class MaskSoftmax2d(_MaskSoftmaxNd):
    """See :func:`mask_softmax2d`."""

    def __init__(self, kernel_size: _size_2_t) -> None:
        super().__init__(tuple(_ints2(kernel_size)))

    def forward(self, mask: Tensor, kernel_size: Optional[Tuple[int, int]] = None) -> Tensor:
        if kernel_size is None:
            return mask_softmax2d(mask, self.kernel_size)
        return mask_softmax2d(mask, kernel_size)


class MaskSoftmax3d(_MaskSoftmaxNd):
    """See :func:`mask_softmax3d`."""

    def __init__(self, kernel_size: _size_3_t) -> None:
        super().__init__(tuple(_ints3(kernel_size)))

    def forward(self, mask: Tensor, kernel_size: Optional[Tuple[int, int, int]] = None) -> Tensor:
        if kernel_size is None:
            return mask_softmax3d(mask, self.kernel_size)
        return mask_softmax3d(mask, kernel_size)
