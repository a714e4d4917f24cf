// Test program for include/tvdcn_ops.h: a C++ caller of the operator library, built and run by
// tests/test_api_cpu.py::test_cpp_api_caller. It links tvdcn_amd/_C.so, calls the tvdcn::ops API on host
// tensors with inputs that the test rebuilds in Python, and prints every result value (one tensor
// per line: name then values) for the test to compare with the Python API's.
#include <ATen/ATen.h>

#include <cstdio>
#include <vector>

#include "tvdcn_ops.h"

namespace {

// deterministic input: sin(0.37 * k + phase) over the tensor's elements, k = 0, 1, ...
at::Tensor filled(at::IntArrayRef shape, double phase) {
    int64_t n = 1;
    for (const int64_t v : shape) n *= v;
    return at::sin(at::arange(n, at::kFloat) * 0.37 + phase).reshape(shape);
}

void print(const char *name, const at::Tensor &t) {
    const at::Tensor c = t.contiguous().to(at::kDouble);
    std::printf("%s", name);
    const double *p = c.data_ptr<double>();
    for (int64_t i = 0; i < c.numel(); ++i) std::printf(" %.17g", p[i]);
    std::printf("\n");
}

}  // namespace

int main() {
    std::printf("cuda_version %lld\n", (long long)tvdcn::cuda_version());
    std::printf("cuda_arch_flags %s\n", tvdcn::cuda_arch_flags().c_str());

    // 2D conv: stride 1, padding 1, dilation 1, 2 offset groups, 1 mask group
    const at::Tensor x = filled({2, 4, 5, 6}, 0.1), w = filled({3, 4, 3, 3}, 0.2), b = filled({3}, 0.3);
    const at::Tensor off = filled({2, 36, 5, 6}, 0.4) * 1.5, msk = filled({2, 9, 5, 6}, 0.5).abs();
    const at::Tensor y = tvdcn::ops::deform_conv2d(x, w, off, msk, b, {1, 1}, {1, 1}, {1, 1}, 1);
    print("conv2d", y);
    const std::vector<c10::SymInt> one{c10::SymInt(1), c10::SymInt(1)};
    print("conv2d_symint", tvdcn::ops::deform_conv2d_symint(x, w, off, msk, b, one, one, one, c10::SymInt(1)));
    const at::Tensor gy = filled(y.sizes(), 0.6);
    const auto g = tvdcn::ops::detail::_deform_conv2d_backward(gy, x, w, off, msk, b, {1, 1}, {1, 1}, {1, 1}, 1);
    print("conv2d_grad_input", std::get<0>(g));
    print("conv2d_grad_weight", std::get<1>(g));
    print("conv2d_grad_offset", std::get<2>(g));
    print("conv2d_grad_mask", std::get<3>(g));
    print("conv2d_grad_bias", std::get<4>(g));

    // 1D transposed: stride 2, padding 1, output_padding 1, no mask
    const at::Tensor x1 = filled({2, 4, 7}, 0.7), w1 = filled({4, 2, 3}, 0.8), off1 = filled({2, 3, 7}, 0.9);
    print("transpose1d", tvdcn::ops::deform_conv_transpose1d(x1, w1, off1, {}, {}, 2, 1, 1, 1, 1));

    // 3D conv with the default arguments (offset only)
    const at::Tensor x3 = filled({1, 2, 3, 4, 4}, 1.0), w3 = filled({2, 2, 2, 2, 2}, 1.1);
    const at::Tensor off3 = filled({1, 24, 2, 3, 3}, 1.2);
    print("conv3d_defaults", tvdcn::ops::deform_conv3d(x3, w3, off3));
    return 0;
}
