// C++ API of the operator library (include/tvdcn_ops.h): each function forwards to the registered
// `tvdcn::` operator through the dispatcher (one operator-handle lookup per function, on its first
// call), so device selection, autograd and autocast apply as they do for Python callers.
//
// Reference interface mirrored (paths relative to tvdcn/csrc/): ops/deform_conv{1,2,3}d.h and
// ops/deform_conv_transpose{1,2,3}d.h (declarations; e.g. deform_conv2d.h:9-58), whose definitions in
// the matching .cpp files call the operators the same way; tvdcn.h:6-9 (cuda_version, cuda_arch_flags).
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/util/Logging.h>

#include "tvdcn_hip.h"
#include "tvdcn_ops.h"

namespace tvdcn {

int64_t cuda_version() { return tvdcn_hip_version(); }
std::string cuda_arch_flags() { return tvdcn_arch_flags(); }

namespace ops {
namespace {

template <typename Fn>
c10::TypedOperatorHandle<Fn> typed_op(const char *name) {
    return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<Fn>();
}

using Opt = at::optional<at::Tensor>;

}  // namespace

// forward and backward of one conv rank: int and SymInt argument forms, same operator
#define TVDCN_CONV_API(D)                                                                                        \
    at::Tensor deform_conv##D##d(const at::Tensor &input, const at::Tensor &weight, const Opt &offset,           \
                                 const Opt &mask, const Opt &bias, at::IntArrayRef stride, at::IntArrayRef padding, \
                                 at::IntArrayRef dilation, int64_t groups) {                                     \
        C10_LOG_API_USAGE_ONCE("tvdcn_amd.cpp_api.deform_conv" #D "d");                                           \
        static const auto op = typed_op<decltype(deform_conv##D##d)>("tvdcn::deform_conv" #D "d");               \
        return op.call(input, weight, offset, mask, bias, stride, padding, dilation, groups);                    \
    }                                                                                                            \
    at::Tensor deform_conv##D##d_symint(const at::Tensor &input, const at::Tensor &weight, const Opt &offset,    \
                                        const Opt &mask, const Opt &bias, at::SymIntArrayRef stride,             \
                                        at::SymIntArrayRef padding, at::SymIntArrayRef dilation,                 \
                                        c10::SymInt groups) {                                                    \
        C10_LOG_API_USAGE_ONCE("tvdcn_amd.cpp_api.deform_conv" #D "d");                                           \
        static const auto op = typed_op<decltype(deform_conv##D##d_symint)>("tvdcn::deform_conv" #D "d");        \
        return op.call(input, weight, offset, mask, bias, stride, padding, dilation, std::move(groups));         \
    }                                                                                                            \
    namespace detail {                                                                                           \
    Grads5 _deform_conv##D##d_backward(const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight, \
                                       const Opt &offset, const Opt &mask, const Opt &bias,                      \
                                       at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef dilation, \
                                       int64_t groups) {                                                         \
        static const auto op =                                                                                   \
            typed_op<decltype(_deform_conv##D##d_backward)>("tvdcn::_deform_conv" #D "d_backward");              \
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, dilation, groups);              \
    }                                                                                                            \
    Grads5 _deform_conv##D##d_backward_symint(const at::Tensor &grad, const at::Tensor &input,                  \
                                              const at::Tensor &weight, const Opt &offset, const Opt &mask,      \
                                              const Opt &bias, at::SymIntArrayRef stride,                        \
                                              at::SymIntArrayRef padding, at::SymIntArrayRef dilation,           \
                                              c10::SymInt groups) {                                              \
        static const auto op =                                                                                   \
            typed_op<decltype(_deform_conv##D##d_backward_symint)>("tvdcn::_deform_conv" #D "d_backward");       \
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, dilation, std::move(groups));   \
    }                                                                                                            \
    }

// the transposed ops: output_padding after padding
#define TVDCN_TRANSPOSE_API(D)                                                                                   \
    at::Tensor deform_conv_transpose##D##d(const at::Tensor &input, const at::Tensor &weight, const Opt &offset, \
                                           const Opt &mask, const Opt &bias, at::IntArrayRef stride,             \
                                           at::IntArrayRef padding, at::IntArrayRef output_padding,              \
                                           at::IntArrayRef dilation, int64_t groups) {                           \
        C10_LOG_API_USAGE_ONCE("tvdcn_amd.cpp_api.deform_conv_transpose" #D "d");                                 \
        static const auto op =                                                                                   \
            typed_op<decltype(deform_conv_transpose##D##d)>("tvdcn::deform_conv_transpose" #D "d");              \
        return op.call(input, weight, offset, mask, bias, stride, padding, output_padding, dilation, groups);    \
    }                                                                                                            \
    at::Tensor deform_conv_transpose##D##d_symint(const at::Tensor &input, const at::Tensor &weight,            \
                                                  const Opt &offset, const Opt &mask, const Opt &bias,           \
                                                  at::SymIntArrayRef stride, at::SymIntArrayRef padding,         \
                                                  at::SymIntArrayRef output_padding, at::SymIntArrayRef dilation, \
                                                  c10::SymInt groups) {                                          \
        C10_LOG_API_USAGE_ONCE("tvdcn_amd.cpp_api.deform_conv_transpose" #D "d");                                 \
        static const auto op =                                                                                   \
            typed_op<decltype(deform_conv_transpose##D##d_symint)>("tvdcn::deform_conv_transpose" #D "d");       \
        return op.call(input, weight, offset, mask, bias, stride, padding, output_padding, dilation,             \
                       std::move(groups));                                                                       \
    }                                                                                                            \
    namespace detail {                                                                                           \
    Grads5 _deform_conv_transpose##D##d_backward(const at::Tensor &grad, const at::Tensor &input,               \
                                                 const at::Tensor &weight, const Opt &offset, const Opt &mask,   \
                                                 const Opt &bias, at::IntArrayRef stride, at::IntArrayRef padding, \
                                                 at::IntArrayRef output_padding, at::IntArrayRef dilation,       \
                                                 int64_t groups) {                                               \
        static const auto op = typed_op<decltype(_deform_conv_transpose##D##d_backward)>(                        \
            "tvdcn::_deform_conv_transpose" #D "d_backward");                                                    \
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, output_padding, dilation,       \
                       groups);                                                                                  \
    }                                                                                                            \
    Grads5 _deform_conv_transpose##D##d_backward_symint(                                                         \
        const at::Tensor &grad, const at::Tensor &input, const at::Tensor &weight, const Opt &offset,            \
        const Opt &mask, const Opt &bias, at::SymIntArrayRef stride, at::SymIntArrayRef padding,                 \
        at::SymIntArrayRef output_padding, at::SymIntArrayRef dilation, c10::SymInt groups) {                    \
        static const auto op = typed_op<decltype(_deform_conv_transpose##D##d_backward_symint)>(                 \
            "tvdcn::_deform_conv_transpose" #D "d_backward");                                                    \
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, output_padding, dilation,       \
                       std::move(groups));                                                                       \
    }                                                                                                            \
    }

TVDCN_CONV_API(1)
TVDCN_CONV_API(2)
TVDCN_CONV_API(3)
TVDCN_TRANSPOSE_API(1)
TVDCN_TRANSPOSE_API(2)
TVDCN_TRANSPOSE_API(3)

#undef TVDCN_CONV_API
#undef TVDCN_TRANSPOSE_API

}  // namespace ops
}  // namespace tvdcn
