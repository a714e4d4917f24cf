"""Transposed deformable convolution: ``deform_conv_transpose{1,2,3}d``, ``DeformConvTranspose{1,2,3}d``,
``PackedDeformConvTranspose{1,2,3}d``.

Same signatures, defaults and error behaviour as tvdcn/ops/deform_conv_transpose.py
(functions :29-196, modules :203-790). Offsets and masks live on the *input*
grid; the sampled/scattered side is the output. The GPU kernels are the fused
grad-columns + scatter kernel (forward) and the gather-GEMM / coordinate /
weight-gradient kernels (backward).
"""
from typing import Callable, List, Optional, Union

import torch
from torch import Tensor
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t, _size_any_t
from torch.nn.modules.utils import _pair, _single, _triple

from .deform_conv import _DeformConvNd, _PackedMixin, _deform_conv_sigmoid_mask
from ..extension import _assert_has_ops
from ..utils import _log_api_usage_once

__all__ = [
    "deform_conv_transpose1d", "deform_conv_transpose2d", "deform_conv_transpose3d",
    "DeformConvTranspose1d", "DeformConvTranspose2d", "DeformConvTranspose3d",
    "PackedDeformConvTranspose1d", "PackedDeformConvTranspose2d", "PackedDeformConvTranspose3d",
]

_NTUPLE = {1: _single, 2: _pair, 3: _triple}


def _call(dim: int, fn, input, weight, offset, mask, bias, stride, padding, output_padding, dilation,
          groups) -> Tensor:
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(fn)
    _assert_has_ops()
    op = getattr(torch.ops.tvdcn_amd, f"deform_conv_transpose{dim}d")
    nt = _NTUPLE[dim]
    return op(input, weight, offset, mask, bias, nt(stride), nt(padding), nt(output_padding), nt(dilation), groups)


def deform_conv_transpose1d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None, stride: _size_1_t = 1,
                            padding: _size_1_t = 0, output_padding: _size_1_t = 0, dilation: _size_1_t = 1,
                            groups: int = 1) -> Tensor:
    r"""1D transposed deformable convolution.

    input (B, Cin, W); weight (Cin, Cout // groups, kw); offset (B, offset_groups * kw, W) and
    mask (B, mask_groups * kw, W) on the input grid; bias (Cout,).
    """
    return _call(1, deform_conv_transpose1d, input, weight, offset, mask, bias, stride, padding, output_padding,
                 dilation, groups)


def deform_conv_transpose2d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None, stride: _size_2_t = 1,
                            padding: _size_2_t = 0, output_padding: _size_2_t = 0, dilation: _size_2_t = 1,
                            groups: int = 1) -> Tensor:
    r"""2D transposed deformable convolution.

    input (B, Cin, H, W); weight (Cin, Cout // groups, kh, kw); offset (B, 2 * offset_groups * kh * kw, H, W)
    and mask (B, mask_groups * kh * kw, H, W) on the input grid; bias (Cout,).
    Output size (H - 1) * stride - 2 * padding + dilation * (k - 1) + 1 + output_padding.
    """
    return _call(2, deform_conv_transpose2d, input, weight, offset, mask, bias, stride, padding, output_padding,
                 dilation, groups)


def deform_conv_transpose3d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None, stride: _size_3_t = 1,
                            padding: _size_3_t = 0, output_padding: _size_3_t = 0, dilation: _size_3_t = 1,
                            groups: int = 1) -> Tensor:
    r"""3D transposed deformable convolution (offsets (dz, dy, dx) on the input grid)."""
    return _call(3, deform_conv_transpose3d, input, weight, offset, mask, bias, stride, padding, output_padding,
                 dilation, groups)


_FUNCTIONAL = {1: deform_conv_transpose1d, 2: deform_conv_transpose2d, 3: deform_conv_transpose3d}


class _DeformConvTransposeNd(_DeformConvNd):
    """Base of the transposed modules (tvdcn/ops/deform_conv_transpose.py:203-285)."""

    def _output_padding(self, input: Tensor, output_size: Optional[List[int]], stride: List[int],
                        padding: List[int], kernel_size: List[int], num_spatial_dims: int,
                        dilation: Optional[List[int]] = None) -> List[int]:
        """output_padding that yields ``output_size`` (torch's ConvTranspose rule)."""
        if output_size is None:
            return list(_single(self.output_padding))
        has_batch_dim = input.dim() == num_spatial_dims + 2
        num_non_spatial = 2 if has_batch_dim else 1
        output_size = list(output_size)
        if len(output_size) == num_non_spatial + num_spatial_dims:
            output_size = output_size[num_non_spatial:]
        if len(output_size) != num_spatial_dims:
            raise ValueError(
                f"ConvTranspose{num_spatial_dims}D: for {input.dim()}D input, output_size must have "
                f"{num_spatial_dims} or {num_non_spatial + num_spatial_dims} elements (got {len(output_size)})")
        min_sizes, max_sizes = [], []
        for d in range(num_spatial_dims):
            dl = dilation[d] if dilation is not None else 1
            lo = (input.size(d + num_non_spatial) - 1) * stride[d] - 2 * padding[d] + dl * (kernel_size[d] - 1) + 1
            min_sizes.append(lo)
            max_sizes.append(lo + stride[d] - 1)
        for size, lo, hi in zip(output_size, min_sizes, max_sizes):
            if size < lo or size > hi:
                raise ValueError(
                    f"requested an output size of {output_size}, but valid sizes range from {min_sizes} to "
                    f"{max_sizes} (for an input of {input.size()[2:]})")
        return [output_size[d] - min_sizes[d] for d in range(num_spatial_dims)]

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None) -> Tensor:
        raise NotImplementedError

    def forward(self, input: Tensor, offset: Optional[Tensor], mask: Optional[Tensor] = None,
                output_size: Optional[List[int]] = None) -> Tensor:
        return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size)


class _DeformConvTransposeDim(_DeformConvTransposeNd):
    _dim = 0

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                 output_padding=0, groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None,
                 dtype=None) -> None:
        nt = _NTUPLE[self._dim]
        super().__init__(in_channels, out_channels, nt(kernel_size), nt(stride), nt(padding), nt(dilation), True,
                         nt(output_padding), groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None,
                                mask_sigmoid_scale: Optional[float] = None) -> Tensor:
        if self.padding_mode != "zeros":
            raise ValueError(f"Only `zeros` padding mode is supported for {type(self).__name__}.")
        output_padding = self._output_padding(input, output_size, list(self.stride), list(self.padding),
                                              list(self.kernel_size), self._dim, list(self.dilation))
        if mask_sigmoid_scale is not None:
            # mask holds logits: the sigmoid runs inside the kernels
            return _deform_conv_sigmoid_mask(self._dim, input, weight, offset, mask, bias, self.stride, self.padding,
                                             tuple(output_padding), self.dilation, self.groups, True,
                                             mask_sigmoid_scale)
        return _FUNCTIONAL[self._dim](input, weight, offset, mask, bias, self.stride, self.padding,
                                      tuple(output_padding), self.dilation, self.groups)


class DeformConvTranspose1d(_DeformConvTransposeDim):
    """See :func:`deform_conv_transpose1d`."""
    _dim = 1

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: _size_1_t = 0, dilation: _size_1_t = 1, output_padding: _size_1_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, output_padding, groups,
                         bias, padding_mode, device, dtype)


class DeformConvTranspose2d(_DeformConvTransposeDim):
    """See :func:`deform_conv_transpose2d`."""
    _dim = 2

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: _size_2_t = 0, dilation: _size_2_t = 1, output_padding: _size_2_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, output_padding, groups,
                         bias, padding_mode, device, dtype)


class DeformConvTranspose3d(_DeformConvTransposeDim):
    """See :func:`deform_conv_transpose3d`."""
    _dim = 3

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: _size_3_t = 0, dilation: _size_3_t = 1, output_padding: _size_3_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, output_padding, groups,
                         bias, padding_mode, device, dtype)


def _make_packed(base, dim: int, doc: str):
    class _Packed(_PackedMixin, base):
        __doc__ = doc

        def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                     output_padding=0, groups: int = 1, offset_groups: int = 1, mask_groups: int = 1,
                     bias: bool = True, generator_bias: bool = False, deformable: bool = True,
                     modulated: bool = False, offset_activation: Optional[Union[str, Callable]] = None,
                     mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                     device=None, dtype=None) -> None:
            base.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, output_padding,
                          groups, bias, padding_mode, device, dtype)
            # offsets/masks live on the input grid: 1x1 generators
            self._setup_generators(dim, offset_groups, mask_groups, generator_bias, deformable, modulated,
                                   offset_activation, mask_activation, dict(kernel_size=1), device, dtype)

        def reset_parameters(self) -> None:
            if not hasattr(self, "modulated"):
                return
            base.reset_parameters(self)
            self._reset_generators()

        def forward(self, input: Tensor, output_size: Optional[List[int]] = None) -> Tensor:
            offset, mask, scale = self._generate(input)
            return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size,
                                                mask_sigmoid_scale=scale)

    return _Packed


PackedDeformConvTranspose1d = _make_packed(DeformConvTranspose1d, 1,
                                           "Packed version of :class:`DeformConvTranspose1d`.")
PackedDeformConvTranspose1d.__name__ = PackedDeformConvTranspose1d.__qualname__ = "PackedDeformConvTranspose1d"
PackedDeformConvTranspose2d = _make_packed(DeformConvTranspose2d, 2,
                                           "Packed version of :class:`DeformConvTranspose2d`.")
PackedDeformConvTranspose2d.__name__ = PackedDeformConvTranspose2d.__qualname__ = "PackedDeformConvTranspose2d"
PackedDeformConvTranspose3d = _make_packed(DeformConvTranspose3d, 3,
                                           "Packed version of :class:`DeformConvTranspose3d`.")
PackedDeformConvTranspose3d.__name__ = PackedDeformConvTranspose3d.__qualname__ = "PackedDeformConvTranspose3d"
