// CPU kernels of the tvdcn operators (host tensors). The reference registers CPU twins of its
// CUDA drivers under the CPU dispatch key (tvdcn/csrc/ops/cpu/deform_conv2d_kernel.cpp:645 and
// the 1D / 3D / transposed files); these are the CPU-key bodies of this library's schemas.
#pragma once

#include <ATen/ATen.h>

#include <tuple>
#include <vector>

#include "tvdcn_hip.h"

namespace tvdcn_amd {
namespace cpu {

// One validated problem: the descriptor (rank, transposed flag, sizes, groups, flags and mask
// activation), the spatial size of the result, and batched NC<spatial>-contiguous tensors of one
// floating type (offset / mask / bias undefined when absent; with TVDCN_FLAG_MASK_SIGMOID or
// TVDCN_FLAG_MASK_SOFTMAX the mask holds logits).
struct Operands {
    tvdcn_conv_desc desc;
    std::vector<int64_t> out_size;
    at::Tensor input, weight, offset, mask, bias;
};

// Forward: (batch, out_channels, *out_size).
at::Tensor forward(const Operands &op);

// Backward: grad_input, grad_weight, grad_offset, grad_mask (with respect to the logits when the
// mask is activated), grad_bias; the last three undefined when the operand is absent.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> backward(const Operands &op,
                                                                                 const at::Tensor &grad);

// mask_softmax over the K taps of each group: x viewed as (B, G, K, S).
at::Tensor mask_softmax(const at::Tensor &x, int64_t B, int64_t G, int64_t K, int64_t S);
at::Tensor mask_softmax_backward(const at::Tensor &grad, const at::Tensor &y, int64_t B, int64_t G, int64_t K,
                                 int64_t S);

}  // namespace cpu
}  // namespace tvdcn_amd
