"""Deformable convolution: ``deform_conv{1,2,3}d``, ``DeformConv{1,2,3}d``, ``PackedDeformConv{1,2,3}d``.

Same signatures, defaults and error behaviour as tvdcn/ops/deform_conv.py
(functions :30-199, modules :206-751). The functions dispatch to
``torch.ops.tvdcn_amd.deform_conv{N}d`` whose GPU kernel is the fused gfx950
gather-GEMM (forward) and the fused grad-columns / scatter / weight-gradient
kernels (backward).
"""
from typing import Callable, Optional, Union

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.nn import init
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t, _size_any_t
from torch.nn.modules.conv import _ConvNd
from torch.nn.modules.utils import _pair, _single, _triple

from .activations import MaskSigmoid, MaskSoftmax1d, MaskSoftmax2d, MaskSoftmax3d
from ..extension import _assert_has_ops
from ..utils import _log_api_usage_once

__all__ = [
    "deform_conv1d", "deform_conv2d", "deform_conv3d",
    "DeformConv1d", "DeformConv2d", "DeformConv3d",
    "PackedDeformConv1d", "PackedDeformConv2d", "PackedDeformConv3d",
]

_NTUPLE = {1: _single, 2: _pair, 3: _triple}
_MASK_SOFTMAX = {1: MaskSoftmax1d, 2: MaskSoftmax2d, 3: MaskSoftmax3d}


def _call(dim: int, fn, input, weight, offset, mask, bias, stride, padding, dilation, groups) -> Tensor:
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(fn)
    _assert_has_ops()
    op = getattr(torch.ops.tvdcn_amd, f"deform_conv{dim}d")
    nt = _NTUPLE[dim]
    return op(input, weight, offset, mask, bias, nt(stride), nt(padding), nt(dilation), groups)


def deform_conv1d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: _size_1_t = 1, padding: _size_1_t = 0,
                  dilation: _size_1_t = 1, groups: int = 1) -> Tensor:
    r"""1D deformable convolution.

    input (B, Cin, W); weight (Cout, Cin // groups, kw); offset (B, offset_groups * kw, out_w);
    mask (B, mask_groups * kw, out_w); bias (Cout,). Returns (B, Cout, out_w).
    """
    return _call(1, deform_conv1d, input, weight, offset, mask, bias, stride, padding, dilation, groups)


def deform_conv2d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: _size_2_t = 1, padding: _size_2_t = 0,
                  dilation: _size_2_t = 1, groups: int = 1) -> Tensor:
    r"""2D deformable convolution (DCNv1 / DCNv2; https://arxiv.org/abs/1703.06211, https://arxiv.org/abs/1811.11168).

    input (B, Cin, H, W); weight (Cout, Cin // groups, kh, kw);
    offset (B, 2 * offset_groups * kh * kw, out_h, out_w), channel ((g * kh + i) * kw + j) * 2 + {0: dy, 1: dx};
    mask (B, mask_groups * kh * kw, out_h, out_w); bias (Cout,). Returns (B, Cout, out_h, out_w).
    """
    return _call(2, deform_conv2d, input, weight, offset, mask, bias, stride, padding, dilation, groups)


def deform_conv3d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: _size_3_t = 1, padding: _size_3_t = 0,
                  dilation: _size_3_t = 1, groups: int = 1) -> Tensor:
    r"""3D deformable convolution.

    input (B, Cin, D, H, W); weight (Cout, Cin // groups, kd, kh, kw);
    offset (B, 3 * offset_groups * kd * kh * kw, out_d, out_h, out_w) with directions (dz, dy, dx);
    mask (B, mask_groups * kd * kh * kw, out_d, out_h, out_w); bias (Cout,).
    """
    return _call(3, deform_conv3d, input, weight, offset, mask, bias, stride, padding, dilation, groups)


_FUNCTIONAL = {1: deform_conv1d, 2: deform_conv2d, 3: deform_conv3d}


def _deform_conv_sigmoid_mask(dim: int, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask_logits: Tensor,
                              bias: Optional[Tensor], stride, padding, output_padding, dilation, groups: int,
                              transposed: bool, mask_scale: float) -> Tensor:
    """Deformable (transposed) convolution whose mask is ``mask_scale * sigmoid(mask_logits)``, the
    activation applied in the kernels' mask load (the packed modules' default ``MaskSigmoid``,
    tvdcn/ops/deform_conv.py:502-505, without its separate passes). Gradients flow to the logits."""
    _assert_has_ops()
    nt = _NTUPLE[dim]
    return torch.ops.tvdcn_amd.deform_conv_sigmoid_mask(input, weight, offset, mask_logits, bias, nt(stride),
                                                        nt(padding), nt(output_padding), nt(dilation), groups,
                                                        transposed, float(mask_scale))


class _DeformConvNd(_ConvNd):
    """Base of the deformable convolution modules (tvdcn/ops/deform_conv.py:206-265)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_any_t, stride: _size_any_t,
                 padding: Union[str, _size_any_t], dilation: _size_any_t, transposed: bool,
                 output_padding: _size_any_t, groups: int, bias: bool, padding_mode: str, device=None,
                 dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, transposed,
                         output_padding, groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask: Optional[Tensor],
                      bias: Optional[Tensor]) -> Tensor:
        raise NotImplementedError

    def forward(self, input: Tensor, offset: Optional[Tensor], mask: Optional[Tensor] = None) -> Tensor:
        return self._conv_forward(input, self.weight, offset, mask, self.bias)

    def extra_repr(self):
        s = "{in_channels}, {out_channels}, kernel_size={kernel_size}, stride={stride}"
        if self.padding != (0,) * len(self.padding):
            s += ", padding={padding}"
        if self.dilation != (1,) * len(self.dilation):
            s += ", dilation={dilation}"
        if self.output_padding != (0,) * len(self.output_padding):
            s += ", output_padding={output_padding}"
        if self.groups != 1:
            s += ", groups={groups}"
        if getattr(self, "offset_groups", 1) != 1:
            s += ", offset_groups={offset_groups}"
        if getattr(self, "mask_groups", 1) != 1:
            s += ", mask_groups={mask_groups}"
        if self.bias is None:
            s += ", bias=False"
        if not getattr(self, "deformable", True):
            s += ", deformable=False"
        if not getattr(self, "modulated", True):
            s += ", modulated=False"
        if self.padding_mode != "zeros":
            s += ", padding_mode={padding_mode}"
        return s.format(**self.__dict__)


class _DeformConvDim(_DeformConvNd):
    """Rank-specific deformable convolution module; ``_dim`` is set by the subclasses."""
    _dim = 0

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                 groups: int = 1, bias: bool = True, padding_mode: str = "zeros", device=None, dtype=None) -> None:
        nt = _NTUPLE[self._dim]
        super().__init__(in_channels, out_channels, nt(kernel_size), nt(stride),
                         padding if isinstance(padding, str) else nt(padding), nt(dilation), False, nt(0),
                         groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask: Optional[Tensor],
                      bias: Optional[Tensor], mask_sigmoid_scale: Optional[float] = None) -> Tensor:
        if mask_sigmoid_scale is not None:
            # mask holds logits: the sigmoid runs inside the kernels
            padding = self.padding
            if self.padding_mode != "zeros":
                input = F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode)
                padding = (0,) * self._dim
            return _deform_conv_sigmoid_mask(self._dim, input, weight, offset, mask, bias, self.stride, padding,
                                             (0,) * self._dim, self.dilation, self.groups, False, mask_sigmoid_scale)
        fn = _FUNCTIONAL[self._dim]
        if self.padding_mode != "zeros":
            # non-zero padding modes: pad explicitly, then convolve without padding
            return fn(F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode), weight, offset,
                      mask, bias, self.stride, (0,) * self._dim, self.dilation, self.groups)
        return fn(input, weight, offset, mask, bias, self.stride, self.padding, self.dilation, self.groups)


class DeformConv1d(_DeformConvDim):
    """See :func:`deform_conv1d`."""
    _dim = 1

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: Union[str, _size_1_t] = 0, dilation: _size_1_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                         padding_mode, device, dtype)


class DeformConv2d(_DeformConvDim):
    """See :func:`deform_conv2d`."""
    _dim = 2

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: Union[str, _size_2_t] = 0, dilation: _size_2_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                         padding_mode, device, dtype)


class DeformConv3d(_DeformConvDim):
    """See :func:`deform_conv3d`."""
    _dim = 3

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: Union[str, _size_3_t] = 0, dilation: _size_3_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                         padding_mode, device, dtype)


def _check_packed_groups(in_channels: int, out_channels: int, offset_groups: int, mask_groups: int) -> None:
    for what, n in (("offset_groups", offset_groups), ("mask_groups", mask_groups)):
        if in_channels % n != 0:
            raise ValueError(f"in_channels must be divisible by {what}")
        if out_channels % n != 0:
            raise ValueError(f"out_channels must be divisible by {what}")


def _resolve_mask_activation(mask_activation, dim: int, kernel_size):
    if isinstance(mask_activation, str):
        if mask_activation == "sigmoid":
            return MaskSigmoid(scale=2.)
        if mask_activation == "softmax":
            return _MASK_SOFTMAX[dim](kernel_size)
        raise ValueError('only "sigmoid" and "softmax" activations are supported for mask')
    return mask_activation


class _PackedMixin:
    """Shared parts of the packed modules: zero-initialised offset/mask generators
    (tvdcn/ops/deform_conv.py:392-510 and twins)."""

    def _setup_generators(self, dim: int, offset_groups: int, mask_groups: int, generator_bias: bool,
                          deformable: bool, modulated: bool, offset_activation, mask_activation, conv_kwargs,
                          device, dtype) -> None:
        _check_packed_groups(self.in_channels, self.out_channels, offset_groups, mask_groups)
        if isinstance(offset_activation, str):
            raise ValueError("currently, no activation is supported for offset")
        mask_activation = _resolve_mask_activation(mask_activation, dim, self.kernel_size)
        self.offset_groups = offset_groups
        self.mask_groups = mask_groups
        self.deformable = deformable
        self.modulated = modulated
        conv_cls = {1: nn.Conv1d, 2: nn.Conv2d, 3: nn.Conv3d}[dim]
        taps = 1
        for k in self.kernel_size:
            taps *= k
        if deformable:
            self.offset_generator = conv_cls(self.in_channels, dim * taps * offset_groups, groups=offset_groups,
                                             bias=generator_bias, device=device, dtype=dtype, **conv_kwargs)
        else:
            self.register_module("offset_generator", None)
        if modulated:
            self.mask_generator = conv_cls(self.in_channels, taps * mask_groups, groups=mask_groups,
                                           bias=generator_bias, device=device, dtype=dtype, **conv_kwargs)
        else:
            self.register_module("mask_generator", None)
        self.offset_activation = offset_activation
        self.mask_activation = mask_activation
        self.reset_parameters()

    def _reset_generators(self) -> None:
        for gen in (self.offset_generator, self.mask_generator):
            if gen is not None:
                init.zeros_(gen.weight)
                if gen.bias is not None:
                    init.zeros_(gen.bias)

    def _generate(self, input: Tensor):
        """offset, mask and the mask's sigmoid scale: a ``MaskSigmoid`` activation (the default) is
        left to the kernels, which apply it in their mask load — the mask is then returned as
        logits with the scale; any other activation is applied here (scale None)."""
        offset = mask = scale = None
        if self.deformable and self.offset_generator is not None:
            offset = self.offset_generator(input)
            if self.offset_activation is not None:
                offset = self.offset_activation(offset)
        if self.modulated and self.mask_generator is not None:
            mask = self.mask_generator(input)
            if type(self.mask_activation) is MaskSigmoid:
                scale = self.mask_activation.scale
            elif self.mask_activation is not None:
                mask = self.mask_activation(mask)
        return offset, mask, scale


def _make_packed(base, dim: int, doc: str):
    class _Packed(_PackedMixin, base):
        __doc__ = doc

        def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                     groups: int = 1, offset_groups: int = 1, mask_groups: int = 1, bias: bool = True,
                     generator_bias: bool = False, deformable: bool = True, modulated: bool = False,
                     offset_activation: Optional[Union[str, Callable]] = None,
                     mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                     device=None, dtype=None) -> None:
            base.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                          padding_mode, device, dtype)
            # the generators see the same receptive field as the deformable conv
            conv_kwargs = dict(kernel_size=self.kernel_size, stride=self.stride, padding=self.padding,
                               dilation=self.dilation)
            self._setup_generators(dim, offset_groups, mask_groups, generator_bias, deformable, modulated,
                                   offset_activation, mask_activation, conv_kwargs, device, dtype)

        def reset_parameters(self) -> None:
            if not hasattr(self, "modulated"):
                return
            base.reset_parameters(self)
            self._reset_generators()

        def forward(self, input: Tensor) -> Tensor:
            offset, mask, scale = self._generate(input)
            return self._conv_forward(input, self.weight, offset, mask, self.bias, mask_sigmoid_scale=scale)

    return _Packed


PackedDeformConv1d = _make_packed(DeformConv1d, 1, "Packed version of :class:`DeformConv1d`.")
PackedDeformConv1d.__name__ = PackedDeformConv1d.__qualname__ = "PackedDeformConv1d"
PackedDeformConv2d = _make_packed(DeformConv2d, 2, "Packed version of :class:`DeformConv2d`.")
PackedDeformConv2d.__name__ = PackedDeformConv2d.__qualname__ = "PackedDeformConv2d"
PackedDeformConv3d = _make_packed(DeformConv3d, 3, "Packed version of :class:`DeformConv3d`.")
PackedDeformConv3d.__name__ = PackedDeformConv3d.__qualname__ = "PackedDeformConv3d"
