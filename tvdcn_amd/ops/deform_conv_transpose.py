"""Transposed deformable convolution: ``deform_conv_transpose{1,2,3}d``, ``DeformConvTranspose{1,2,3}d``,
``PackedDeformConvTranspose{1,2,3}d``.

Same signatures, defaults and error behaviour as tvdcn/ops/deform_conv_transpose.py
(functions :29-196, modules :203-790). Offsets and masks live on the *input*
grid; the sampled/scattered side is the output. The GPU kernels are the fused
grad-columns + scatter kernel (forward) and the gather-GEMM / coordinate /
weight-gradient kernels (backward). The modules compile with ``torch.jit.script``.
"""
from typing import Callable, List, Optional, Tuple, Union

import torch
from torch import Tensor
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t
from torch.nn.modules.utils import _pair, _single, _triple

from .deform_conv import _DeformConvNd, _PackedGenerators, _deform_conv_mask_activation
from ..extension import _assert_has_ops
from ..utils import _ints1, _ints2, _ints3, _log_api_usage_once

__all__ = [
    "deform_conv_transpose1d", "deform_conv_transpose2d", "deform_conv_transpose3d",
    "DeformConvTranspose1d", "DeformConvTranspose2d", "DeformConvTranspose3d",
    "PackedDeformConvTranspose1d", "PackedDeformConvTranspose2d", "PackedDeformConvTranspose3d",
]


def deform_conv_transpose1d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None,
                            stride: Union[int, Tuple[int]] = 1, padding: Union[int, Tuple[int]] = 0,
                            output_padding: Union[int, Tuple[int]] = 0, dilation: Union[int, Tuple[int]] = 1,
                            groups: int = 1) -> Tensor:
    r"""1D transposed deformable convolution.

    input (B, Cin, W); weight (Cin, Cout // groups, kw); offset (B, offset_groups * kw, W) and
    mask (B, mask_groups * kw, W) on the input grid; bias (Cout,).
    """
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv_transpose1d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv_transpose1d(input, weight, offset, mask, bias, _ints1(stride),
                                                   _ints1(padding), _ints1(output_padding), _ints1(dilation),
                                                   groups)


def deform_conv_transpose2d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None,
                            stride: Union[int, Tuple[int, int]] = 1, padding: Union[int, Tuple[int, int]] = 0,
                            output_padding: Union[int, Tuple[int, int]] = 0,
                            dilation: Union[int, Tuple[int, int]] = 1, groups: int = 1) -> Tensor:
    r"""2D transposed deformable convolution.

    input (B, Cin, H, W); weight (Cin, Cout // groups, kh, kw); offset (B, 2 * offset_groups * kh * kw, H, W)
    and mask (B, mask_groups * kh * kw, H, W) on the input grid; bias (Cout,).
    Output size (H - 1) * stride - 2 * padding + dilation * (k - 1) + 1 + output_padding.
    """
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv_transpose2d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv_transpose2d(input, weight, offset, mask, bias, _ints2(stride),
                                                   _ints2(padding), _ints2(output_padding), _ints2(dilation),
                                                   groups)


def deform_conv_transpose3d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None,
                            mask: Optional[Tensor] = None, bias: Optional[Tensor] = None,
                            stride: Union[int, Tuple[int, int, int]] = 1,
                            padding: Union[int, Tuple[int, int, int]] = 0,
                            output_padding: Union[int, Tuple[int, int, int]] = 0,
                            dilation: Union[int, Tuple[int, int, int]] = 1, groups: int = 1) -> Tensor:
    r"""3D transposed deformable convolution (offsets (dz, dy, dx) on the input grid)."""
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv_transpose3d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv_transpose3d(input, weight, offset, mask, bias, _ints3(stride),
                                                   _ints3(padding), _ints3(output_padding), _ints3(dilation),
                                                   groups)


class _DeformConvTransposeNd(_DeformConvNd):
    """Base of the transposed modules (tvdcn/ops/deform_conv_transpose.py:203-285)."""

    def _output_padding(self, input: Tensor, output_size: Optional[List[int]], stride: List[int],
                        padding: List[int], kernel_size: List[int], num_spatial_dims: int,
                        dilation: Optional[List[int]] = None) -> List[int]:
        """output_padding that yields ``output_size`` (torch's ConvTranspose rule, as the reference)."""
        if output_size is None:
            return _single(self.output_padding)
        has_batch_dim = input.dim() == num_spatial_dims + 2
        num_non_spatial = 2 if has_batch_dim else 1
        if len(output_size) == num_non_spatial + num_spatial_dims:
            output_size = output_size[num_non_spatial:]
        if len(output_size) != num_spatial_dims:
            raise ValueError(
                "ConvTranspose{}D: for {}D input, output_size must have {} or {} elements (got {})".format(
                    num_spatial_dims, input.dim(), num_spatial_dims, num_non_spatial + num_spatial_dims,
                    len(output_size)))
        min_sizes = torch.jit.annotate(List[int], [])
        max_sizes = torch.jit.annotate(List[int], [])
        for d in range(num_spatial_dims):
            dl = dilation[d] if dilation is not None else 1
            lo = (input.size(d + num_non_spatial) - 1) * stride[d] - 2 * padding[d] + dl * (kernel_size[d] - 1) + 1
            min_sizes.append(lo)
            max_sizes.append(lo + stride[d] - 1)
        for d in range(num_spatial_dims):
            if output_size[d] < min_sizes[d] or output_size[d] > max_sizes[d]:
                raise ValueError(
                    "requested an output size of {}, but valid sizes range from {} to {} (for an input of {})".format(
                        output_size, min_sizes, max_sizes, input.size()[2:]))
        res = torch.jit.annotate(List[int], [])
        for d in range(num_spatial_dims):
            res.append(output_size[d] - min_sizes[d])
        return res

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None) -> Tensor:
        raise NotImplementedError

    def forward(self, input: Tensor, offset: Optional[Tensor], mask: Optional[Tensor] = None,
                output_size: Optional[List[int]] = None) -> Tensor:
        return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size)


class DeformConvTranspose1d(_DeformConvTransposeNd):
    """See :func:`deform_conv_transpose1d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: _size_1_t = 0, dilation: _size_1_t = 1, output_padding: _size_1_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _single(kernel_size), _single(stride), _single(padding),
                         _single(dilation), True, _single(output_padding), groups, bias, padding_mode,
                         device=device, dtype=dtype)

    def _padding_for(self, input: Tensor, output_size: Optional[List[int]]) -> List[int]:
        if self.padding_mode != "zeros":
            raise ValueError("Only `zeros` padding mode is supported for DeformConvTranspose1d.")
        return self._output_padding(input, output_size, _ints1(self.stride), _ints1(self.padding),
                                    _ints1(self.kernel_size), 1, _ints1(self.dilation))

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None) -> Tensor:
        op = self._padding_for(input, output_size)
        return deform_conv_transpose1d(input, weight, offset, mask, bias, self.stride, self.padding, (op[0],),
                                       self.dilation, self.groups)

    def _conv_transpose_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                                mask_logits: Tensor, bias: Optional[Tensor],
                                                output_size: Optional[List[int]], activation: int,
                                                scale: float) -> Tensor:
        op = self._padding_for(input, output_size)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints1(self.stride),
                                            _ints1(self.padding), op, _ints1(self.dilation), self.groups, True,
                                            activation, scale)


class DeformConvTranspose2d(_DeformConvTransposeNd):
    """See :func:`deform_conv_transpose2d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: _size_2_t = 0, dilation: _size_2_t = 1, output_padding: _size_2_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _pair(kernel_size), _pair(stride), _pair(padding),
                         _pair(dilation), True, _pair(output_padding), groups, bias, padding_mode,
                         device=device, dtype=dtype)

    def _padding_for(self, input: Tensor, output_size: Optional[List[int]]) -> List[int]:
        if self.padding_mode != "zeros":
            raise ValueError("Only `zeros` padding mode is supported for DeformConvTranspose2d.")
        return self._output_padding(input, output_size, _ints2(self.stride), _ints2(self.padding),
                                    _ints2(self.kernel_size), 2, _ints2(self.dilation))

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None) -> Tensor:
        op = self._padding_for(input, output_size)
        return deform_conv_transpose2d(input, weight, offset, mask, bias, self.stride, self.padding,
                                       (op[0], op[1]), self.dilation, self.groups)

    def _conv_transpose_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                                mask_logits: Tensor, bias: Optional[Tensor],
                                                output_size: Optional[List[int]], activation: int,
                                                scale: float) -> Tensor:
        op = self._padding_for(input, output_size)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints2(self.stride),
                                            _ints2(self.padding), op, _ints2(self.dilation), self.groups, True,
                                            activation, scale)


class DeformConvTranspose3d(_DeformConvTransposeNd):
    """See :func:`deform_conv_transpose3d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: _size_3_t = 0, dilation: _size_3_t = 1, output_padding: _size_3_t = 0,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _triple(kernel_size), _triple(stride), _triple(padding),
                         _triple(dilation), True, _triple(output_padding), groups, bias, padding_mode,
                         device=device, dtype=dtype)

    def _padding_for(self, input: Tensor, output_size: Optional[List[int]]) -> List[int]:
        if self.padding_mode != "zeros":
            raise ValueError("Only `zeros` padding mode is supported for DeformConvTranspose3d.")
        return self._output_padding(input, output_size, _ints3(self.stride), _ints3(self.padding),
                                    _ints3(self.kernel_size), 3, _ints3(self.dilation))

    def _conv_transpose_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                mask: Optional[Tensor], bias: Optional[Tensor],
                                output_size: Optional[List[int]] = None) -> Tensor:
        op = self._padding_for(input, output_size)
        return deform_conv_transpose3d(input, weight, offset, mask, bias, self.stride, self.padding,
                                       (op[0], op[1], op[2]), self.dilation, self.groups)

    def _conv_transpose_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                                mask_logits: Tensor, bias: Optional[Tensor],
                                                output_size: Optional[List[int]], activation: int,
                                                scale: float) -> Tensor:
        op = self._padding_for(input, output_size)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints3(self.stride),
                                            _ints3(self.padding), op, _ints3(self.dilation), self.groups, True,
                                            activation, scale)


def _packed_transposed_init(self, base, dim: int, in_channels, out_channels, kernel_size, stride, padding,
                            dilation, output_padding, groups, offset_groups, mask_groups, bias, generator_bias,
                            deformable, modulated, offset_activation, mask_activation, padding_mode, device,
                            dtype) -> None:
    base.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, output_padding, groups,
                  bias, padding_mode, device, dtype)
    # offsets / masks live on the input grid: 1x1 generators
    self._setup_generators(dim, offset_groups, mask_groups, generator_bias, deformable, modulated,
                           offset_activation, mask_activation, 1, 1, 0, 1, device, dtype)


class PackedDeformConvTranspose1d(_PackedGenerators, DeformConvTranspose1d):
    """Packed version of :class:`DeformConvTranspose1d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: _size_1_t = 0, dilation: _size_1_t = 1, output_padding: _size_1_t = 0,
                 groups: int = 1, offset_groups: int = 1, mask_groups: int = 1, bias: bool = True,
                 generator_bias: bool = False, deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        _packed_transposed_init(self, DeformConvTranspose1d, 1, in_channels, out_channels, kernel_size, stride,
                                padding, dilation, output_padding, groups, offset_groups, mask_groups, bias,
                                generator_bias, deformable, modulated, offset_activation, mask_activation,
                                padding_mode, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConvTranspose1d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor, output_size: Optional[List[int]] = None) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_transpose_forward_mask_activation(input, self.weight, offset, mask, self.bias,
                                                                output_size, fused, scale)
        return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size)


class PackedDeformConvTranspose2d(_PackedGenerators, DeformConvTranspose2d):
    """Packed version of :class:`DeformConvTranspose2d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: _size_2_t = 0, dilation: _size_2_t = 1, output_padding: _size_2_t = 0,
                 groups: int = 1, offset_groups: int = 1, mask_groups: int = 1, bias: bool = True,
                 generator_bias: bool = False, deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        _packed_transposed_init(self, DeformConvTranspose2d, 2, in_channels, out_channels, kernel_size, stride,
                                padding, dilation, output_padding, groups, offset_groups, mask_groups, bias,
                                generator_bias, deformable, modulated, offset_activation, mask_activation,
                                padding_mode, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConvTranspose2d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor, output_size: Optional[List[int]] = None) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_transpose_forward_mask_activation(input, self.weight, offset, mask, self.bias,
                                                                output_size, fused, scale)
        return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size)


class PackedDeformConvTranspose3d(_PackedGenerators, DeformConvTranspose3d):
    """Packed version of :class:`DeformConvTranspose3d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: _size_3_t = 0, dilation: _size_3_t = 1, output_padding: _size_3_t = 0,
                 groups: int = 1, offset_groups: int = 1, mask_groups: int = 1, bias: bool = True,
                 generator_bias: bool = False, deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        _packed_transposed_init(self, DeformConvTranspose3d, 3, in_channels, out_channels, kernel_size, stride,
                                padding, dilation, output_padding, groups, offset_groups, mask_groups, bias,
                                generator_bias, deformable, modulated, offset_activation, mask_activation,
                                padding_mode, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConvTranspose3d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor, output_size: Optional[List[int]] = None) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_transpose_forward_mask_activation(input, self.weight, offset, mask, self.bias,
                                                                output_size, fused, scale)
        return self._conv_transpose_forward(input, self.weight, offset, mask, self.bias, output_size)
