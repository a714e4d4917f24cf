"""Deformable convolution: ``deform_conv{1,2,3}d``, ``DeformConv{1,2,3}d``, ``PackedDeformConv{1,2,3}d``.

Same signatures, defaults and error behaviour as tvdcn/ops/deform_conv.py
(functions :30-199, modules :206-751). The functions dispatch to
``torch.ops.tvdcn.deform_conv{N}d`` whose GPU kernel is the fused gfx950
gather-GEMM (forward) and the fused grad-columns / scatter / weight-gradient
kernels (backward). The modules compile with ``torch.jit.script``.

The packed modules differ from the reference in one way that does not change
their results: when their mask activation is the default ``MaskSigmoid`` or a
``MaskSoftmax{N}d`` over the convolution's own taps, the activation runs inside the
kernels' mask load (op ``tvdcn::deform_conv_mask_activation``) instead of as
separate passes over the mask, and the gradient flows to the generator's logits.
"""
from typing import Callable, List, Optional, Tuple, Union

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.nn import init
from torch.nn.common_types import _size_1_t, _size_2_t, _size_3_t, _size_any_t
from torch.nn.modules.conv import _ConvNd
from torch.nn.modules.utils import _pair, _single, _triple

from .activations import MaskSigmoid, MaskSoftmax1d, MaskSoftmax2d, MaskSoftmax3d
from ..extension import _assert_has_ops
from ..utils import _ints1, _ints2, _ints3, _log_api_usage_once

__all__ = [
    "deform_conv1d", "deform_conv2d", "deform_conv3d",
    "DeformConv1d", "DeformConv2d", "DeformConv3d",
    "PackedDeformConv1d", "PackedDeformConv2d", "PackedDeformConv3d",
]


def deform_conv1d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: Union[int, Tuple[int]] = 1,
                  padding: Union[int, Tuple[int]] = 0, dilation: Union[int, Tuple[int]] = 1,
                  groups: int = 1) -> Tensor:
    r"""1D deformable convolution.

    input (B, Cin, W); weight (Cout, Cin // groups, kw); offset (B, offset_groups * kw, out_w);
    mask (B, mask_groups * kw, out_w); bias (Cout,). Returns (B, Cout, out_w).
    """
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv1d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv1d(input, weight, offset, mask, bias, _ints1(stride), _ints1(padding),
                                         _ints1(dilation), groups)


def deform_conv2d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: Union[int, Tuple[int, int]] = 1,
                  padding: Union[int, Tuple[int, int]] = 0, dilation: Union[int, Tuple[int, int]] = 1,
                  groups: int = 1) -> Tensor:
    r"""2D deformable convolution (DCNv1 / DCNv2; https://arxiv.org/abs/1703.06211, https://arxiv.org/abs/1811.11168).

    input (B, Cin, H, W); weight (Cout, Cin // groups, kh, kw);
    offset (B, 2 * offset_groups * kh * kw, out_h, out_w), channel ((g * kh + i) * kw + j) * 2 + {0: dy, 1: dx};
    mask (B, mask_groups * kh * kw, out_h, out_w); bias (Cout,). Returns (B, Cout, out_h, out_w).
    """
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv2d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv2d(input, weight, offset, mask, bias, _ints2(stride), _ints2(padding),
                                         _ints2(dilation), groups)


def deform_conv3d(input: Tensor, weight: Tensor, offset: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                  bias: Optional[Tensor] = None, stride: Union[int, Tuple[int, int, int]] = 1,
                  padding: Union[int, Tuple[int, int, int]] = 0, dilation: Union[int, Tuple[int, int, int]] = 1,
                  groups: int = 1) -> Tensor:
    r"""3D deformable convolution.

    input (B, Cin, D, H, W); weight (Cout, Cin // groups, kd, kh, kw);
    offset (B, 3 * offset_groups * kd * kh * kw, out_d, out_h, out_w) with directions (dz, dy, dx);
    mask (B, mask_groups * kd * kh * kw, out_d, out_h, out_w); bias (Cout,).
    """
    if not torch.jit.is_scripting() and not torch.jit.is_tracing():
        _log_api_usage_once(deform_conv3d)
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv3d(input, weight, offset, mask, bias, _ints3(stride), _ints3(padding),
                                         _ints3(dilation), groups)


# mask activations the kernels can apply in their mask load (codes of tvdcn::deform_conv_mask_activation;
# the scripted methods below write 0 for _FUSED_NONE: TorchScript reads no module-level ints)
_FUSED_NONE = 0
_FUSED_SIGMOID = 1
_FUSED_SOFTMAX = 2


def _deform_conv_mask_activation(input: Tensor, weight: Tensor, offset: Optional[Tensor], mask_logits: Tensor,
                                 bias: Optional[Tensor], stride: List[int], padding: List[int],
                                 output_padding: List[int], dilation: List[int], groups: int, transposed: bool,
                                 activation: int, scale: float) -> Tensor:
    """Deformable (transposed) convolution whose mask is an activation of ``mask_logits``, applied in the
    kernels' mask load: ``scale * sigmoid`` (activation 1, tvdcn's ``MaskSigmoid``) or the softmax over
    the kernel taps of each mask group (activation 2, ``MaskSoftmax{N}d``). Gradients flow to the logits."""
    _assert_has_ops()
    return torch.ops.tvdcn.deform_conv_mask_activation(input, weight, offset, mask_logits, bias, stride, padding,
                                                       output_padding, dilation, groups, transposed, activation,
                                                       scale)


def _has_forward_hooks(module: nn.Module) -> bool:
    """True when calling ``module`` would run forward (pre-)hooks: its own or torch's global ones."""
    from torch.nn.modules import module as _module
    return bool(module._forward_hooks or module._forward_pre_hooks or _module._global_forward_hooks or
                _module._global_forward_pre_hooks)


def _mask_fusion_of(activation: Optional[Callable], kernel_size: Tuple[int, ...]) -> Tuple[int, float]:
    """(code, scale) of a mask activation the kernels apply themselves; (0, 0.0) for any other.

    Only the exact classes qualify (a subclass may change ``forward``), and only while no forward
    hook or pre-hook would run on the call (the reference calls the module, so a hook that reads or
    edits the mask keeps running). A non-positive sigmoid scale is left to ``MaskSigmoid`` itself,
    which raises the reference's ``ValueError``."""
    if isinstance(activation, nn.Module) and _has_forward_hooks(activation):
        return _FUSED_NONE, 0.0
    if type(activation) is MaskSigmoid:
        if activation.scale > 0:
            return _FUSED_SIGMOID, float(activation.scale)
        return _FUSED_NONE, 0.0
    if type(activation) in (MaskSoftmax1d, MaskSoftmax2d, MaskSoftmax3d):
        if tuple(activation.kernel_size) == tuple(kernel_size):
            return _FUSED_SOFTMAX, 0.0
    return _FUSED_NONE, 0.0


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


class DeformConv1d(_DeformConvNd):
    """See :func:`deform_conv1d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: Union[str, _size_1_t] = 0, dilation: _size_1_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _single(kernel_size), _single(stride),
                         padding if isinstance(padding, str) else _single(padding), _single(dilation), False,
                         _single(0), groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask: Optional[Tensor],
                      bias: Optional[Tensor]) -> Tensor:
        if self.padding_mode != "zeros":
            # non-zero padding modes: pad explicitly, then convolve without padding
            return deform_conv1d(F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode),
                                 weight, offset, mask, bias, self.stride, (0,), self.dilation, self.groups)
        return deform_conv1d(input, weight, offset, mask, bias, self.stride, self.padding, self.dilation,
                             self.groups)

    def _conv_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                      mask_logits: Tensor, bias: Optional[Tensor], activation: int,
                                      scale: float) -> Tensor:
        padding = self.padding
        if self.padding_mode != "zeros":
            input = F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode)
            padding = (0,)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints1(self.stride),
                                            _ints1(padding), [0], _ints1(self.dilation), self.groups, False,
                                            activation, scale)


class DeformConv2d(_DeformConvNd):
    """See :func:`deform_conv2d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: Union[str, _size_2_t] = 0, dilation: _size_2_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _pair(kernel_size), _pair(stride),
                         padding if isinstance(padding, str) else _pair(padding), _pair(dilation), False,
                         _pair(0), groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask: Optional[Tensor],
                      bias: Optional[Tensor]) -> Tensor:
        if self.padding_mode != "zeros":
            return deform_conv2d(F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode),
                                 weight, offset, mask, bias, self.stride, (0, 0), self.dilation, self.groups)
        return deform_conv2d(input, weight, offset, mask, bias, self.stride, self.padding, self.dilation,
                             self.groups)

    def _conv_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                      mask_logits: Tensor, bias: Optional[Tensor], activation: int,
                                      scale: float) -> Tensor:
        padding = self.padding
        if self.padding_mode != "zeros":
            input = F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode)
            padding = (0, 0)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints2(self.stride),
                                            _ints2(padding), [0, 0], _ints2(self.dilation), self.groups, False,
                                            activation, scale)


class DeformConv3d(_DeformConvNd):
    """See :func:`deform_conv3d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: Union[str, _size_3_t] = 0, dilation: _size_3_t = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros", device=None, dtype=None) -> None:
        super().__init__(in_channels, out_channels, _triple(kernel_size), _triple(stride),
                         padding if isinstance(padding, str) else _triple(padding), _triple(dilation), False,
                         _triple(0), groups, bias, padding_mode, device=device, dtype=dtype)

    def _conv_forward(self, input: Tensor, weight: Tensor, offset: Optional[Tensor], mask: Optional[Tensor],
                      bias: Optional[Tensor]) -> Tensor:
        if self.padding_mode != "zeros":
            return deform_conv3d(F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode),
                                 weight, offset, mask, bias, self.stride, (0, 0, 0), self.dilation, self.groups)
        return deform_conv3d(input, weight, offset, mask, bias, self.stride, self.padding, self.dilation,
                             self.groups)

    def _conv_forward_mask_activation(self, input: Tensor, weight: Tensor, offset: Optional[Tensor],
                                      mask_logits: Tensor, bias: Optional[Tensor], activation: int,
                                      scale: float) -> Tensor:
        padding = self.padding
        if self.padding_mode != "zeros":
            input = F.pad(input, self._reversed_padding_repeated_twice, mode=self.padding_mode)
            padding = (0, 0, 0)
        return _deform_conv_mask_activation(input, weight, offset, mask_logits, bias, _ints3(self.stride),
                                            _ints3(padding), [0, 0, 0], _ints3(self.dilation), self.groups, False,
                                            activation, scale)


class _PackedGenerators:
    """What the packed modules share (tvdcn/ops/deform_conv.py:392-510 and twins): the zero-initialised
    offset / mask generator convolutions, the mask activation and its fusion into the kernels.

    ``_mask_fusion`` decides at every eager call from the current ``mask_activation``; a scripted module
    keeps the decision taken when it was scripted (``__prepare_scriptable__``), as it keeps every other
    attribute's value."""

    def _setup_generators(self, dim: int, offset_groups: int, mask_groups: int, generator_bias: bool,
                          deformable: bool, modulated: bool, offset_activation, mask_activation, kernel_size,
                          stride, padding, dilation, device, dtype) -> None:
        for what, n in (("offset_groups", offset_groups), ("mask_groups", mask_groups)):
            if self.in_channels % n != 0:
                raise ValueError(f"in_channels must be divisible by {what}")
            if self.out_channels % n != 0:
                raise ValueError(f"out_channels must be divisible by {what}")
        if isinstance(offset_activation, str):
            raise ValueError("currently, no activation is supported for offset")
        if isinstance(mask_activation, str):
            if mask_activation == "sigmoid":
                mask_activation = MaskSigmoid(scale=2.)
            elif mask_activation == "softmax":
                mask_activation = (MaskSoftmax1d, MaskSoftmax2d, MaskSoftmax3d)[dim - 1](self.kernel_size)
            else:
                raise ValueError('only "sigmoid" and "softmax" activations are supported for mask')
        self.offset_groups = offset_groups
        self.mask_groups = mask_groups
        self.deformable = deformable
        self.modulated = modulated
        conv = (nn.Conv1d, nn.Conv2d, nn.Conv3d)[dim - 1]
        taps = 1
        for k in self.kernel_size:
            taps *= k
        if deformable:
            self.offset_generator = conv(self.in_channels, dim * taps * offset_groups, kernel_size=kernel_size,
                                         stride=stride, padding=padding, dilation=dilation, groups=offset_groups,
                                         bias=generator_bias, device=device, dtype=dtype)
        else:
            self.register_module("offset_generator", None)
        if modulated:
            self.mask_generator = conv(self.in_channels, taps * mask_groups, kernel_size=kernel_size,
                                       stride=stride, padding=padding, dilation=dilation, groups=mask_groups,
                                       bias=generator_bias, device=device, dtype=dtype)
        else:
            self.register_module("mask_generator", None)
        self.offset_activation = offset_activation
        self.mask_activation = mask_activation
        self._fused_mask_activation, self._fused_mask_scale = _mask_fusion_of(mask_activation, self.kernel_size)
        self.reset_parameters()

    def _reset_generators(self) -> None:
        for gen in (self.offset_generator, self.mask_generator):
            if gen is not None:
                init.zeros_(gen.weight)
                if gen.bias is not None:
                    init.zeros_(gen.bias)

    def __prepare_scriptable__(self):
        self._fused_mask_activation, self._fused_mask_scale = _mask_fusion_of(self.mask_activation,
                                                                              self.kernel_size)
        return self

    def _mask_fusion(self) -> Tuple[int, float]:
        if not torch.jit.is_scripting():
            return _mask_fusion_of(self.mask_activation, self.kernel_size)
        return self._fused_mask_activation, self._fused_mask_scale

    def _generate(self, input: Tensor) -> Tuple[Optional[Tensor], Optional[Tensor], int, float]:
        """(offset, mask, fused activation code, scale); with a non-zero code the mask holds the logits."""
        offset: Optional[Tensor] = None
        if self.deformable and self.offset_generator is not None:
            offset = self.offset_generator(input)
            if self.offset_activation is not None:
                offset = self.offset_activation(offset)
        mask: Optional[Tensor] = None
        if self.modulated and self.mask_generator is not None:
            mask = self.mask_generator(input)
            fused, scale = self._mask_fusion()
            if fused != 0:
                return offset, mask, fused, scale
            if self.mask_activation is not None:
                mask = self.mask_activation(mask)
        return offset, mask, 0, 0.0


class PackedDeformConv1d(_PackedGenerators, DeformConv1d):
    """Packed version of :class:`DeformConv1d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_1_t, stride: _size_1_t = 1,
                 padding: Union[str, _size_1_t] = 0, dilation: _size_1_t = 1, groups: int = 1,
                 offset_groups: int = 1, mask_groups: int = 1, bias: bool = True, generator_bias: bool = False,
                 deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        DeformConv1d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                              padding_mode, device, dtype)
        # the generators see the same receptive field as the deformable convolution
        self._setup_generators(1, offset_groups, mask_groups, generator_bias, deformable, modulated,
                               offset_activation, mask_activation, self.kernel_size, self.stride, self.padding,
                               self.dilation, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConv1d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_forward_mask_activation(input, self.weight, offset, mask, self.bias, fused, scale)
        return self._conv_forward(input, self.weight, offset, mask, self.bias)


class PackedDeformConv2d(_PackedGenerators, DeformConv2d):
    """Packed version of :class:`DeformConv2d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_2_t, stride: _size_2_t = 1,
                 padding: Union[str, _size_2_t] = 0, dilation: _size_2_t = 1, groups: int = 1,
                 offset_groups: int = 1, mask_groups: int = 1, bias: bool = True, generator_bias: bool = False,
                 deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        DeformConv2d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                              padding_mode, device, dtype)
        self._setup_generators(2, offset_groups, mask_groups, generator_bias, deformable, modulated,
                               offset_activation, mask_activation, self.kernel_size, self.stride, self.padding,
                               self.dilation, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConv2d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_forward_mask_activation(input, self.weight, offset, mask, self.bias, fused, scale)
        return self._conv_forward(input, self.weight, offset, mask, self.bias)


class PackedDeformConv3d(_PackedGenerators, DeformConv3d):
    """Packed version of :class:`DeformConv3d`."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: _size_3_t, stride: _size_3_t = 1,
                 padding: Union[str, _size_3_t] = 0, dilation: _size_3_t = 1, groups: int = 1,
                 offset_groups: int = 1, mask_groups: int = 1, bias: bool = True, generator_bias: bool = False,
                 deformable: bool = True, modulated: bool = False,
                 offset_activation: Optional[Union[str, Callable]] = None,
                 mask_activation: Optional[Union[str, Callable]] = "sigmoid", padding_mode: str = "zeros",
                 device=None, dtype=None) -> None:
        DeformConv3d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
                              padding_mode, device, dtype)
        self._setup_generators(3, offset_groups, mask_groups, generator_bias, deformable, modulated,
                               offset_activation, mask_activation, self.kernel_size, self.stride, self.padding,
                               self.dilation, device, dtype)

    def reset_parameters(self) -> None:
        if not hasattr(self, "modulated"):
            return
        DeformConv3d.reset_parameters(self)
        self._reset_generators()

    def forward(self, input: Tensor) -> Tensor:
        offset, mask, fused, scale = self._generate(input)
        if fused != 0 and mask is not None:
            return self._conv_forward_mask_activation(input, self.weight, offset, mask, self.bias, fused, scale)
        return self._conv_forward(input, self.weight, offset, mask, self.bias)
