/*
 * tvdcn_ops.h -- C++ API of the tvdcn operator library (tvdcn_amd/_C.so), for C++ callers that link
 * against the library instead of going through Python. Same namespace, names, signatures and default
 * arguments as the reference's C++ API, so code written against it compiles and links unchanged:
 *   tvdcn::ops::deform_conv{1,2,3}d, deform_conv{1,2,3}d_symint,
 *   tvdcn::ops::detail::_deform_conv{1,2,3}d_backward(_symint)
 *       reference: tvdcn/csrc/ops/deform_conv{1,2,3}d.h (e.g. deform_conv2d.h:9-58)
 *   tvdcn::ops::deform_conv_transpose{1,2,3}d(_symint), detail::_deform_conv_transpose{1,2,3}d_backward(_symint)
 *       reference: tvdcn/csrc/ops/deform_conv_transpose{1,2,3}d.h (e.g. deform_conv_transpose2d.h:9-62)
 *   tvdcn::cuda_version, tvdcn::cuda_arch_flags
 *       reference: tvdcn/csrc/tvdcn.h:6-9 (here: the HIP runtime version and "gfx950")
 * Each function calls the registered `tvdcn::` operator through the dispatcher, so tensors on a GPU
 * run the HIP kernels, host tensors the CPU kernels, and autograd / autocast apply as from Python.
 * The transposed ops take output_padding after padding, as the reference's do.
 */
#pragma once

#include <ATen/Tensor.h>

#include <cstdint>
#include <string>
#include <tuple>

#define TVDCN_API __attribute__((visibility("default")))

namespace tvdcn {

TVDCN_API int64_t cuda_version();
TVDCN_API std::string cuda_arch_flags();

namespace ops {

using Grads5 = std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor>;

// ---- deform_conv{1,2,3}d ---------------------------------------------------------------------
TVDCN_API at::Tensor deform_conv1d(const at::Tensor &input, const at::Tensor &weight,
                                   const at::optional<at::Tensor> &offset = {},
                                   const at::optional<at::Tensor> &mask = {},
                                   const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                   at::IntArrayRef padding = 0, at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv1d_symint(const at::Tensor &input, const at::Tensor &weight,
                                          const at::optional<at::Tensor> &offset = {},
                                          const at::optional<at::Tensor> &mask = {},
                                          const at::optional<at::Tensor> &bias = {},
                                          at::SymIntArrayRef stride = c10::SymInt(1),
                                          at::SymIntArrayRef padding = c10::SymInt(0),
                                          at::SymIntArrayRef dilation = c10::SymInt(1), c10::SymInt groups = 1);

TVDCN_API at::Tensor deform_conv2d(const at::Tensor &input, const at::Tensor &weight,
                                   const at::optional<at::Tensor> &offset = {},
                                   const at::optional<at::Tensor> &mask = {},
                                   const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                   at::IntArrayRef padding = 0, at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv2d_symint(const at::Tensor &input, const at::Tensor &weight,
                                          const at::optional<at::Tensor> &offset = {},
                                          const at::optional<at::Tensor> &mask = {},
                                          const at::optional<at::Tensor> &bias = {},
                                          at::SymIntArrayRef stride = c10::SymInt(1),
                                          at::SymIntArrayRef padding = c10::SymInt(0),
                                          at::SymIntArrayRef dilation = c10::SymInt(1), c10::SymInt groups = 1);

TVDCN_API at::Tensor deform_conv3d(const at::Tensor &input, const at::Tensor &weight,
                                   const at::optional<at::Tensor> &offset = {},
                                   const at::optional<at::Tensor> &mask = {},
                                   const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                   at::IntArrayRef padding = 0, at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv3d_symint(const at::Tensor &input, const at::Tensor &weight,
                                          const at::optional<at::Tensor> &offset = {},
                                          const at::optional<at::Tensor> &mask = {},
                                          const at::optional<at::Tensor> &bias = {},
                                          at::SymIntArrayRef stride = c10::SymInt(1),
                                          at::SymIntArrayRef padding = c10::SymInt(0),
                                          at::SymIntArrayRef dilation = c10::SymInt(1), c10::SymInt groups = 1);

// ---- deform_conv_transpose{1,2,3}d -------------------------------------------------------------
TVDCN_API at::Tensor deform_conv_transpose1d(const at::Tensor &input, const at::Tensor &weight,
                                             const at::optional<at::Tensor> &offset = {},
                                             const at::optional<at::Tensor> &mask = {},
                                             const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                             at::IntArrayRef padding = 0, at::IntArrayRef output_padding = 0,
                                             at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv_transpose1d_symint(
    const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset = {},
    const at::optional<at::Tensor> &mask = {}, const at::optional<at::Tensor> &bias = {},
    at::SymIntArrayRef stride = c10::SymInt(1), at::SymIntArrayRef padding = c10::SymInt(0),
    at::SymIntArrayRef output_padding = c10::SymInt(0), at::SymIntArrayRef dilation = c10::SymInt(1),
    c10::SymInt groups = 1);

TVDCN_API at::Tensor deform_conv_transpose2d(const at::Tensor &input, const at::Tensor &weight,
                                             const at::optional<at::Tensor> &offset = {},
                                             const at::optional<at::Tensor> &mask = {},
                                             const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                             at::IntArrayRef padding = 0, at::IntArrayRef output_padding = 0,
                                             at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv_transpose2d_symint(
    const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset = {},
    const at::optional<at::Tensor> &mask = {}, const at::optional<at::Tensor> &bias = {},
    at::SymIntArrayRef stride = c10::SymInt(1), at::SymIntArrayRef padding = c10::SymInt(0),
    at::SymIntArrayRef output_padding = c10::SymInt(0), at::SymIntArrayRef dilation = c10::SymInt(1),
    c10::SymInt groups = 1);

TVDCN_API at::Tensor deform_conv_transpose3d(const at::Tensor &input, const at::Tensor &weight,
                                             const at::optional<at::Tensor> &offset = {},
                                             const at::optional<at::Tensor> &mask = {},
                                             const at::optional<at::Tensor> &bias = {}, at::IntArrayRef stride = 1,
                                             at::IntArrayRef padding = 0, at::IntArrayRef output_padding = 0,
                                             at::IntArrayRef dilation = 1, int64_t groups = 1);
TVDCN_API at::Tensor deform_conv_transpose3d_symint(
    const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset = {},
    const at::optional<at::Tensor> &mask = {}, const at::optional<at::Tensor> &bias = {},
    at::SymIntArrayRef stride = c10::SymInt(1), at::SymIntArrayRef padding = c10::SymInt(0),
    at::SymIntArrayRef output_padding = c10::SymInt(0), at::SymIntArrayRef dilation = c10::SymInt(1),
    c10::SymInt groups = 1);

// ---- the backward schemas (what the autograd nodes call): grad_input, grad_weight, grad_offset,
//      grad_mask, grad_bias --------------------------------------------------------------------------
namespace detail {
Grads5 _deform_conv1d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                               const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                               const at::optional<at::Tensor> &bias, at::IntArrayRef stride, at::IntArrayRef padding,
                               at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv1d_backward_symint(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                      const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                      const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
                                      at::SymIntArrayRef padding, at::SymIntArrayRef dilation, c10::SymInt groups);
Grads5 _deform_conv2d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                               const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                               const at::optional<at::Tensor> &bias, at::IntArrayRef stride, at::IntArrayRef padding,
                               at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv2d_backward_symint(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                      const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                      const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
                                      at::SymIntArrayRef padding, at::SymIntArrayRef dilation, c10::SymInt groups);
Grads5 _deform_conv3d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                               const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                               const at::optional<at::Tensor> &bias, at::IntArrayRef stride, at::IntArrayRef padding,
                               at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv3d_backward_symint(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                      const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                      const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
                                      at::SymIntArrayRef padding, at::SymIntArrayRef dilation, c10::SymInt groups);

Grads5 _deform_conv_transpose1d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                         const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                         const at::optional<at::Tensor> &bias, at::IntArrayRef stride,
                                         at::IntArrayRef padding, at::IntArrayRef output_padding,
                                         at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv_transpose1d_backward_symint(
    const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset,
    const at::optional<at::Tensor> &mask, const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
    at::SymIntArrayRef padding, at::SymIntArrayRef output_padding, at::SymIntArrayRef dilation, c10::SymInt groups);
Grads5 _deform_conv_transpose2d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                         const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                         const at::optional<at::Tensor> &bias, at::IntArrayRef stride,
                                         at::IntArrayRef padding, at::IntArrayRef output_padding,
                                         at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv_transpose2d_backward_symint(
    const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset,
    const at::optional<at::Tensor> &mask, const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
    at::SymIntArrayRef padding, at::SymIntArrayRef output_padding, at::SymIntArrayRef dilation, c10::SymInt groups);
Grads5 _deform_conv_transpose3d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight,
                                         const at::optional<at::Tensor> &offset, const at::optional<at::Tensor> &mask,
                                         const at::optional<at::Tensor> &bias, at::IntArrayRef stride,
                                         at::IntArrayRef padding, at::IntArrayRef output_padding,
                                         at::IntArrayRef dilation, int64_t groups);
Grads5 _deform_conv_transpose3d_backward_symint(
    const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight, const at::optional<at::Tensor> &offset,
    const at::optional<at::Tensor> &mask, const at::optional<at::Tensor> &bias, at::SymIntArrayRef stride,
    at::SymIntArrayRef padding, at::SymIntArrayRef output_padding, at::SymIntArrayRef dilation, c10::SymInt groups);
}  // namespace detail

}  // namespace ops
}  // namespace tvdcn
