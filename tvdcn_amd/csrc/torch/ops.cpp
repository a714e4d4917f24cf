// PyTorch-ROCm operator layer of tvdcn_amd: the reference's twelve operator
// schemas (plus mask_softmax), registered under the reference's `tvdcn` namespace with
// CUDA (= HIP on ROCm), CPU, Meta, Autograd and Autocast kernels. The CUDA kernels
// validate, allocate outputs and workspace from the caching allocator, and call
// the C ABI of libtvdcn_hip.so on the current HIP stream. The CPU kernels
// (host tensors only; cpu_kernels.cpp) run the same validation and compute on the
// host, as the reference's CPU key does (ops/cpu/deform_conv2d_kernel.cpp:645).
//
// Reference interface mirrored (paths relative to tvdcn/csrc/):
//   schemas        ops/deform_conv{1,2,3}d.cpp, ops/deform_conv_transpose{1,2,3}d.cpp
//                  (e.g. ops/deform_conv2d.cpp:117-126, ops/deform_conv_transpose2d.cpp:125-136)
//   validation     ops/cuda/deform_conv2d_kernel.cpp:100-268,
//                  ops/cuda/deform_conv_transpose2d_kernel.cpp:100-275 and 1D/3D twins
//   autograd       ops/autograd/deform_conv2d_kernel.cpp:9-203 (saved tensors, returned
//                  grads, double-backward error) and twins
//   autocast       ops/autocast/deform_conv2d_kernel.cpp:9-38 and twins
//   library info   tvdcn.cpp:24-53 (_cuda_version, _cuda_arch_flags)
#include <ATen/ATen.h>
#include <ATen/FunctionalTensorWrapper.h>
#include <ATen/autocast_mode.h>
#include <c10/core/DeviceGuard.h>
#include <c10/core/impl/TorchDispatchModeTLS.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <atomic>
#include <cmath>
#include <sstream>
#include <string>
#include <vector>

#include "cpu_kernels.h"
#include "tvdcn_hip.h"

namespace tvdcn_amd {
namespace {

using at::Tensor;
using c10::optional;

const char *axis_name(int dim, int i) {
    static const char *n3[] = {"d", "h", "w"};
    return n3[3 - dim + i];
}

std::vector<int64_t> ntuple(at::IntArrayRef v, int dim, const char *what) {
    TORCH_CHECK(v.size() == 1 || (int)v.size() == dim, "Expected a sequence of ", dim, " elements for ", what,
                ", got ", v.size());
    std::vector<int64_t> r(dim);
    for (int i = 0; i < dim; ++i) r[i] = v.size() == 1 ? v[0] : v[i];
    return r;
}

std::string join(const std::vector<int64_t> &v) {
    std::ostringstream os;
    for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
    return os.str();
}

int32_t dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return TVDCN_DTYPE_FLOAT32;
        case at::kDouble: return TVDCN_DTYPE_FLOAT64;
        case at::kHalf: return TVDCN_DTYPE_FLOAT16;
        case at::kBFloat16: return TVDCN_DTYPE_BFLOAT16;
        default: TORCH_CHECK(false, "tvdcn_amd: unsupported dtype ", t, " (expected float32/64, float16, bfloat16)");
    }
    return -1;
}

// Parsed and validated problem.
struct Problem {
    int dim;
    bool transposed;
    bool unbatched;
    bool channels_last;   // conv input kept in channels-last order (TVDCN_FLAG_CHANNELS_LAST)
    tvdcn_conv_desc desc;
    std::vector<int64_t> out_size;
    // batched, contiguous (input: channels-last when channels_last); offset/mask/bias may be undefined
    Tensor input, weight, offset, mask, bias;
};

// Dense channels-last order (batch, *spatial, channels) of a batched conv input: torch's
// channels_last / channels_last_3d formats in 2D / 3D; in 1D (no torch format) a (B, C, L)
// tensor with strides (L * C, 1, C), as a permuted (B, L, C) tensor has.
bool is_channels_last(const Tensor &x, int dim) {
    if (x.dim() != dim + 2) return false;
    if (dim == 2) return x.is_contiguous(at::MemoryFormat::ChannelsLast);
    if (dim == 3) return x.is_contiguous(at::MemoryFormat::ChannelsLast3d);
    const int64_t C = x.size(1), L = x.size(2);
    return (C == 1 || x.stride(1) == 1) && (L == 1 || x.stride(2) == C) && (x.size(0) == 1 || x.stride(0) == C * L);
}

// Shape checks of the reference forward drivers, in the same order and with the
// same wording (rank-generic).
Problem make_problem(int dim, bool transposed, const Tensor &input, const Tensor &weight,
                     const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
                     at::IntArrayRef stride_, at::IntArrayRef padding_, at::IntArrayRef output_padding_,
                     at::IntArrayRef dilation_, int64_t groups, const char *name) {
    Problem pr;
    pr.dim = dim;
    pr.transposed = transposed;
    const bool deformable = offset.has_value() && offset->defined();
    const bool modulated = mask.has_value() && mask->defined();
    const bool with_bias = bias.has_value() && bias->defined();

    at::CheckedFrom c = name;
    std::vector<at::TensorArg> args;
    args.emplace_back(input, "input", 1);
    args.emplace_back(weight, "weight", 2);
    if (deformable) args.emplace_back(offset.value(), "offset", 3);
    if (modulated) args.emplace_back(mask.value(), "mask", 4);
    if (with_bias) args.emplace_back(bias.value(), "bias", 5);
    at::checkAllSameType(c, args);
    for (auto &a : args)
        TORCH_CHECK(a->device() == input.device(), name, ": expected all tensors on ", input.device(), ", but ",
                    a.name, " is on ", a->device());

    pr.unbatched = input.dim() == dim + 1;
    TORCH_CHECK(pr.unbatched || input.dim() == dim + 2, "Expected ", dim + 1, "D (unbatched) or ", dim + 2,
                "D (batched) input to ", transposed ? "deform_conv_transpose" : "deform_conv", dim,
                "d, but got input of size: ", input.sizes());
    TORCH_CHECK(weight.dim() == dim + 2, "Expected ", dim + 2, "D weight");
    TORCH_CHECK(!deformable || offset->dim() == input.dim(), "Expected ", dim + 1, "D (unbatched) or ", dim + 2,
                "D (batched) offset, but got offset of size: ", deformable ? offset->sizes() : at::IntArrayRef());
    TORCH_CHECK(!modulated || mask->dim() == input.dim(), "Expected ", dim + 1, "D (unbatched) or ", dim + 2,
                "D (batched) mask, but got mask of size: ", modulated ? mask->sizes() : at::IntArrayRef());

    // a batched conv input that is channels-last (and not also plain contiguous) is handed over
    // as it is: the kernels sample channels-last data, so no layout copy is needed
    pr.channels_last = !transposed && !pr.unbatched && is_channels_last(input, dim) && !input.is_contiguous();
    pr.input = pr.channels_last ? input : input.contiguous();
    pr.weight = weight.contiguous();
    pr.offset = deformable ? offset->contiguous() : Tensor();
    pr.mask = modulated ? mask->contiguous() : Tensor();
    pr.bias = with_bias ? bias->contiguous() : Tensor();
    if (pr.unbatched) {
        pr.input = pr.input.unsqueeze(0);
        if (deformable) pr.offset = pr.offset.unsqueeze(0);
        if (modulated) pr.mask = pr.mask.unsqueeze(0);
    }

    const auto stride = ntuple(stride_, dim, "stride");
    const auto padding = ntuple(padding_, dim, "padding");
    const auto dilation = ntuple(dilation_, dim, "dilation");
    const auto out_pad = transposed ? ntuple(output_padding_, dim, "output_padding") : std::vector<int64_t>(dim, 0);

    const int64_t B = pr.input.size(0), Cin = pr.input.size(1);
    std::vector<int64_t> ksz(dim), in_size(dim);
    int64_t kn = 1;
    for (int i = 0; i < dim; ++i) {
        ksz[i] = pr.weight.size(2 + i);
        in_size[i] = pr.input.size(2 + i);
        kn *= ksz[i];
    }
    auto check_pos = [&](const std::vector<int64_t> &v, const char *what, bool allow_zero) {
        bool ok = true;
        for (auto x : v) ok = ok && (allow_zero ? x >= 0 : x > 0);
        if (!ok) {
            std::ostringstream os;
            for (int i = 0; i < dim; ++i) os << (i ? " " : "") << what << "_" << axis_name(dim, i) << ": " << v[i];
            TORCH_CHECK(false, os.str());
        }
    };
    check_pos(ksz, "weight", false);
    check_pos(stride, "stride", false);
    check_pos(padding, "pad", true);
    check_pos(dilation, "dilation", false);

    int64_t Cout;
    if (!transposed) {
        Cout = pr.weight.size(0);
        TORCH_CHECK(pr.weight.size(1) * groups == Cin, "Expected weight.size(1) * groups == in_channels (",
                    pr.weight.size(1), " * ", groups, " != ", Cin, ")");
        TORCH_CHECK(pr.weight.size(0) % groups == 0, "Expected weight.size(0) % groups == 0");
    } else {
        Cout = pr.weight.size(1) * groups;
        TORCH_CHECK(pr.weight.size(0) == Cin, "Expected weight.size(0) == in_channels (", pr.weight.size(0),
                    " != ", Cin, ")");
        TORCH_CHECK(pr.weight.size(0) % groups == 0, "Expected weight.size(0) % groups == 0");
    }

    std::vector<int64_t> out(dim);
    for (int i = 0; i < dim; ++i)
        out[i] = transposed ? (in_size[i] - 1) * stride[i] - 2 * padding[i] + dilation[i] * (ksz[i] - 1) + 1 + out_pad[i]
                            : (in_size[i] + 2 * padding[i] - (dilation[i] * (ksz[i] - 1) + 1)) / stride[i] + 1;
    // offsets / masks live on the column grid: conv output grid, transposed input grid
    const std::vector<int64_t> &grid = transposed ? in_size : out;
    const char *grid_name = transposed ? "input" : "output";
    std::string kprod;
    for (int i = 0; i < dim; ++i) kprod += std::string(i ? " * " : "") + "weight.size(" + std::to_string(2 + i) + ")";

    int64_t og = 0, mg = 0;
    if (deformable) {
        og = pr.offset.size(1) / (dim * kn);
        TORCH_CHECK(pr.offset.size(0) == B, "invalid batch size of offset");
        TORCH_CHECK(og > 0, "The shape of the offset tensor at dimension 1 is not valid. It should be a multiple of ",
                    dim, " * ", kprod, ".\nGot offset.size(1)=", pr.offset.size(1), ", while ", dim, " * ", kprod, "=",
                    dim * kn);
        TORCH_CHECK(Cin % og == 0, "Expected in_channels % offset_groups == 0");
        TORCH_CHECK(pr.offset.size(1) == og * dim * kn, "offset.shape[1] is not valid. got: ", pr.offset.size(1),
                    " expected: ", og * dim * kn);
        std::vector<int64_t> got(pr.offset.sizes().begin() + 2, pr.offset.sizes().end());
        TORCH_CHECK(got == grid, "offset ", grid_name, " dims: (", join(got), ") - computed ", grid_name, " dims: (",
                    join(grid), ")");
        if (transposed)
            TORCH_CHECK(Cout % og == 0, "Expected out_channels % offset_groups == 0 (offset groups partition the ",
                        "output channels of a transposed deformable convolution)");
    }
    if (modulated) {
        mg = pr.mask.size(1) / kn;
        TORCH_CHECK(pr.mask.size(0) == B, "invalid batch size of mask");
        TORCH_CHECK(mg > 0, "The shape of the mask tensor at dimension 1 is not valid. It should be a multiple of ",
                    kprod, ".\nGot mask.size(1)=", pr.mask.size(1), ", while ", kprod, "=", kn);
        TORCH_CHECK(Cin % mg == 0, "Expected in_channels % mask_groups == 0");
        TORCH_CHECK(pr.mask.size(1) == mg * kn, "mask.shape[1] is not valid. got: ", pr.mask.size(1), " expected: ",
                    mg * kn);
        std::vector<int64_t> got(pr.mask.sizes().begin() + 2, pr.mask.sizes().end());
        TORCH_CHECK(got == grid, "mask ", grid_name, " dims: (", join(got), ") - computed ", grid_name, " dims: (",
                    join(grid), ")");
        if (transposed)
            TORCH_CHECK(Cout % mg == 0, "Expected out_channels % mask_groups == 0 (mask groups partition the ",
                        "output channels of a transposed deformable convolution)");
    }
    {
        bool ok = true;
        std::ostringstream os;
        for (int i = 0; i < dim; ++i) {
            ok = ok && out[i] > 0;
            os << (i ? " " : "") << "out_" << axis_name(dim, i) << ": " << out[i];
        }
        TORCH_CHECK(ok, "Calculated output size too small - ", os.str());
    }
    if (with_bias) TORCH_CHECK(pr.bias.numel() == Cout, "Expected bias of ", Cout, " elements");

    tvdcn_conv_desc &d = pr.desc;
    std::memset(&d, 0, sizeof(d));
    d.dim = dim;
    d.transposed = transposed;
    d.flags = pr.channels_last ? TVDCN_FLAG_CHANNELS_LAST : 0;
    d.dtype = -1;
    d.batch = B;
    d.in_channels = Cin;
    d.out_channels = Cout;
    d.groups = groups;
    d.offset_groups = og;
    d.mask_groups = mg;
    for (int i = 0; i < 3; ++i) {
        d.kernel[i] = d.stride[i] = d.dilation[i] = d.in_size[i] = 1;
        d.padding[i] = d.output_padding[i] = 0;
    }
    for (int i = 0; i < dim; ++i) {
        d.in_size[i] = in_size[i];
        d.kernel[i] = ksz[i];
        d.stride[i] = stride[i];
        d.padding[i] = padding[i];
        d.dilation[i] = dilation[i];
        d.output_padding[i] = out_pad[i];
    }
    pr.out_size = out;
    return pr;
}

std::vector<int64_t> out_shape(const Problem &pr) {
    std::vector<int64_t> s = {pr.desc.batch, pr.desc.out_channels};
    s.insert(s.end(), pr.out_size.begin(), pr.out_size.end());
    return s;
}

void check_status(tvdcn_status st, const char *what) {
    TORCH_CHECK(st == TVDCN_STATUS_SUCCESS, what, " failed (status ", (int)st, "): ", tvdcn_last_error());
}

const void *ptr_or_null(const Tensor &t) { return t.defined() ? t.data_ptr() : nullptr; }
void *mut_ptr_or_null(const Tensor &t) { return t.defined() ? t.data_ptr() : nullptr; }

// The C ABI wants 16-byte aligned operands; tensors that are contiguous views at
// an odd offset are copied.
Tensor aligned(const Tensor &t) {
    if (!t.defined()) return t;
    if ((reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0) return t;
    return t.clone(at::MemoryFormat::Preserve);   // keeps a channels-last input channels-last
}

// activation 1 / 2: the mask holds logits, activated in the kernels as mask_scale * sigmoid /
// as the softmax over the kernel taps of each mask group (0: the mask is used as it is)
void set_mask_activation(Problem &pr, int64_t activation, double mask_scale) {
    if (activation == 0) return;
    TORCH_CHECK(pr.mask.defined(), "an activated mask needs a mask tensor");
    if (activation == 1) {
        TORCH_CHECK(mask_scale > 0.0 && std::isfinite(mask_scale), "mask_scale must be a positive finite number");
        pr.desc.flags |= TVDCN_FLAG_MASK_SIGMOID;
        pr.desc.mask_scale = mask_scale;
    } else {
        TORCH_CHECK(activation == 2, "unknown mask activation ", activation);
        pr.desc.flags |= TVDCN_FLAG_MASK_SOFTMAX;
    }
}

hipStream_t current_stream(const Tensor &t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// ---------------------------------------------------------------------------
// One image above the kernels' 32-bit indexing (the C ABI refuses it with
// TVDCN_STATUS_NOT_SUPPORTED; the reference indexes such images in 64 bits,
// tvdcn/csrc/ops/utils/dispatch.h:52-60): the problem runs as sub-problems over channel ranges,
// each of whose tensors fits. A sub-problem is one conv group's range of s sampled-side channels
// (conv: input channels; transposed: output channels) times a range of t GEMM-side channels
// (conv: output; transposed: input), with the offset / mask groups of its sampled channels. The
// results that sum over ranges — the output over the ranges it contracts (conv: sampled side;
// transposed: GEMM side), grad_input over the other side's, grad_offset / grad_mask over all — are
// added in float32 (float64 for float64) in a fixed order; the weight gradient is written block by
// block; the bias and its gradient go with the first range of the contracted side.
// ---------------------------------------------------------------------------
struct ChannelSplit {
    int64_t G, Cg, Mg;   // groups, sampled / GEMM-side channels per group
    int64_t cpo, cpm;    // sampled channels per offset / mask group (0: no offset / mask)
    int64_t kn;          // kernel taps
    int64_t s, t;        // channels per sampled / GEMM-side range
};

bool image_too_large(const tvdcn_conv_desc &d) {
    int64_t images = 0;
    return d.batch > 0 && tvdcn_conv_batch_block(&d, &images) == TVDCN_STATUS_NOT_SUPPORTED;
}

// first offset / mask group of sampled channels [c0, c0 + s) and their count (a range lies inside one
// group or covers whole groups)
void range_groups(int64_t c0, int64_t s, int64_t per, int64_t &first, int64_t &count) {
    first = c0 / per;
    count = s > per ? s / per : 1;
}

tvdcn_conv_desc range_desc(const Problem &pr, const ChannelSplit &sp, int64_t c0) {
    tvdcn_conv_desc d = pr.desc;
    d.flags &= ~TVDCN_FLAG_CHANNELS_LAST;   // the ranges are copied to NC<spatial> order
    d.groups = 1;
    d.in_channels = pr.transposed ? sp.t : sp.s;
    d.out_channels = pr.transposed ? sp.s : sp.t;
    int64_t first = 0, count = 0;
    if (sp.cpo) {
        range_groups(c0, sp.s, sp.cpo, first, count);
        d.offset_groups = count;
    }
    if (sp.cpm) {
        range_groups(c0, sp.s, sp.cpm, first, count);
        d.mask_groups = count;
    }
    return d;
}

// a range size s of the sampled side is usable when it divides the group's channels and each range
// lies inside one offset (mask) group or covers whole ones that do not straddle conv groups
bool range_fits_groups(int64_t s, int64_t Cg, int64_t per) {
    if (Cg % s) return false;
    if (per == 0) return true;
    return per % s == 0 || (s % per == 0 && Cg % per == 0);
}

ChannelSplit plan_channel_split(const Problem &pr, const char *name) {
    const tvdcn_conv_desc &d = pr.desc;
    ChannelSplit sp{};
    sp.G = d.groups;
    const int64_t Cs = pr.transposed ? d.out_channels : d.in_channels;
    const int64_t Cm = pr.transposed ? d.in_channels : d.out_channels;
    sp.Cg = Cs / sp.G;
    sp.Mg = Cm / sp.G;
    sp.cpo = d.offset_groups ? Cs / d.offset_groups : 0;
    sp.cpm = d.mask_groups ? Cs / d.mask_groups : 0;
    sp.kn = 1;
    for (int i = 0; i < d.dim; ++i) sp.kn *= d.kernel[i];
    // the largest usable sampled-side range with a one-channel GEMM-side range, then the largest
    // GEMM-side range beside it
    auto fits = [&](int64_t s, int64_t t) {
        ChannelSplit c = sp;
        c.s = s;
        c.t = t;
        int64_t images = 0;
        const tvdcn_conv_desc rd = range_desc(pr, c, 0);
        return tvdcn_conv_batch_block(&rd, &images) == TVDCN_STATUS_SUCCESS;
    };
    for (int64_t s = sp.Cg; s >= 1 && sp.s == 0; --s)
        if (range_fits_groups(s, sp.Cg, sp.cpo) && range_fits_groups(s, sp.Cg, sp.cpm) && fits(s, 1)) sp.s = s;
    TORCH_CHECK(sp.s > 0, name, ": one image's tensors exceed 2^31 - 1 elements even for one channel (its offset, ",
                "mask or spatial extent alone is too large for the kernels' 32-bit indexing)");
    for (int64_t t = sp.Mg; t >= 1 && sp.t == 0; --t)
        if (sp.Mg % t == 0 && fits(sp.s, t)) sp.t = t;
    TORCH_CHECK(sp.t > 0, name, ": one image's tensors exceed 2^31 - 1 elements even for one channel");
    return sp;
}

// the tensors of range (g, i, j): sampled channels c0 = g * Cg + i * s, GEMM-side m0 = g * Mg + j * t
struct RangeOperands {
    int64_t c0, m0;
    bool first;   // the first range of the contracted side: takes the bias
    tvdcn_conv_desc desc;
    Tensor input, weight, offset, mask, bias;
};

RangeOperands range_operands(const Problem &pr, const ChannelSplit &sp, int64_t g, int64_t i, int64_t j) {
    RangeOperands r;
    r.c0 = g * sp.Cg + i * sp.s;
    r.m0 = g * sp.Mg + j * sp.t;
    r.first = pr.transposed ? j == 0 : i == 0;
    r.desc = range_desc(pr, sp, r.c0);
    r.input = aligned((pr.transposed ? pr.input.narrow(1, r.m0, sp.t) : pr.input.narrow(1, r.c0, sp.s)).contiguous());
    // conv weight (Cout, Cin / G, k...), transposed weight (Cin, Cout / G, k...): GEMM-side rows, the
    // group's sampled channels as columns in both
    r.weight = aligned(pr.weight.narrow(0, r.m0, sp.t).narrow(1, i * sp.s, sp.s).contiguous());
    int64_t first = 0, count = 0;
    if (sp.cpo) {
        range_groups(r.c0, sp.s, sp.cpo, first, count);
        const int64_t per = sp.kn * pr.dim;
        r.offset = aligned(pr.offset.narrow(1, first * per, count * per).contiguous());
    }
    if (sp.cpm) {
        range_groups(r.c0, sp.s, sp.cpm, first, count);
        r.mask = aligned(pr.mask.narrow(1, first * sp.kn, count * sp.kn).contiguous());
    }
    if (pr.bias.defined() && r.first)
        r.bias = aligned((pr.transposed ? pr.bias.narrow(0, r.c0, sp.s) : pr.bias.narrow(0, r.m0, sp.t)).contiguous());
    return r;
}

at::ScalarType sum_type(const Tensor &t) { return t.scalar_type() == at::kDouble ? at::kDouble : at::kFloat; }

Tensor forward_channel_split(const Problem &pr, const char *name) {
    const ChannelSplit sp = plan_channel_split(pr, name);
    Tensor acc = at::zeros(out_shape(pr), pr.input.options().dtype(sum_type(pr.input)));
    Tensor ws;
    for (int64_t g = 0; g < sp.G; ++g)
        for (int64_t i = 0; i < sp.Cg / sp.s; ++i)
            for (int64_t j = 0; j < sp.Mg / sp.t; ++j) {
                RangeOperands r = range_operands(pr, sp, g, i, j);
                Tensor part = pr.transposed ? acc.narrow(1, r.c0, sp.s) : acc.narrow(1, r.m0, sp.t);
                Tensor y = at::empty(part.sizes(), pr.input.options());
                const size_t ws_bytes = tvdcn_deform_conv_forward_workspace_size(&r.desc);
                TORCH_CHECK(ws_bytes > 0, name, ": ", tvdcn_last_error());
                if (!ws.defined() || (size_t)ws.numel() < ws_bytes)
                    ws = at::empty({(int64_t)ws_bytes}, pr.input.options().dtype(at::kByte));
                check_status(tvdcn_deform_conv_forward(&r.desc, r.input.data_ptr(), r.weight.data_ptr(),
                                                       ptr_or_null(r.offset), ptr_or_null(r.mask), ptr_or_null(r.bias),
                                                       y.data_ptr(), ws.data_ptr(), ws_bytes, current_stream(y)),
                             name);
                part.add_(y);
            }
    return acc.to(pr.input.scalar_type());
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_channel_split(const Problem &pr, const Tensor &grad,
                                                                          const char *name) {
    const ChannelSplit sp = plan_channel_split(pr, name);
    const auto sums = pr.input.options().dtype(sum_type(pr.input));
    Tensor gi = at::zeros(pr.input.sizes(), sums);
    Tensor gw = at::empty_like(pr.weight);
    Tensor go = pr.offset.defined() ? at::zeros(pr.offset.sizes(), sums) : Tensor();
    Tensor gm = pr.mask.defined() ? at::zeros(pr.mask.sizes(), sums) : Tensor();
    Tensor gb = pr.bias.defined() ? at::empty({pr.desc.out_channels}, pr.input.options()) : Tensor();
    Tensor ws;
    for (int64_t g = 0; g < sp.G; ++g)
        for (int64_t i = 0; i < sp.Cg / sp.s; ++i)
            for (int64_t j = 0; j < sp.Mg / sp.t; ++j) {
                RangeOperands r = range_operands(pr, sp, g, i, j);
                Tensor gr = aligned((pr.transposed ? grad.narrow(1, r.c0, sp.s) : grad.narrow(1, r.m0, sp.t)).contiguous());
                Tensor r_gi = at::empty_like(r.input), r_gw = at::empty_like(r.weight);
                Tensor r_go = r.offset.defined() ? at::empty_like(r.offset) : Tensor();
                Tensor r_gm = r.mask.defined() ? at::empty_like(r.mask) : Tensor();
                Tensor r_gb = r.bias.defined() ? at::empty_like(r.bias) : Tensor();
                const size_t ws_bytes = tvdcn_deform_conv_backward_workspace_size(&r.desc);
                TORCH_CHECK(ws_bytes > 0, name, ": ", tvdcn_last_error());
                if (!ws.defined() || (size_t)ws.numel() < ws_bytes)
                    ws = at::empty({(int64_t)ws_bytes}, pr.input.options().dtype(at::kByte));
                check_status(tvdcn_deform_conv_backward(&r.desc, gr.data_ptr(), r.input.data_ptr(), r.weight.data_ptr(),
                                                        ptr_or_null(r.offset), ptr_or_null(r.mask), r_gi.data_ptr(),
                                                        r_gw.data_ptr(), mut_ptr_or_null(r_go), mut_ptr_or_null(r_gm),
                                                        mut_ptr_or_null(r_gb), ws.data_ptr(), ws_bytes,
                                                        current_stream(r_gi)),
                             name);
                (pr.transposed ? gi.narrow(1, r.m0, sp.t) : gi.narrow(1, r.c0, sp.s)).add_(r_gi);
                gw.narrow(0, r.m0, sp.t).narrow(1, i * sp.s, sp.s).copy_(r_gw);
                int64_t first = 0, count = 0;
                if (r_go.defined()) {
                    range_groups(r.c0, sp.s, sp.cpo, first, count);
                    go.narrow(1, first * sp.kn * pr.dim, count * sp.kn * pr.dim).add_(r_go);
                }
                if (r_gm.defined()) {
                    range_groups(r.c0, sp.s, sp.cpm, first, count);
                    gm.narrow(1, first * sp.kn, count * sp.kn).add_(r_gm);
                }
                if (r_gb.defined())
                    (pr.transposed ? gb.narrow(0, r.c0, sp.s) : gb.narrow(0, r.m0, sp.t)).copy_(r_gb);
            }
    Tensor grad_input = at::empty_like(pr.input);   // (keeps a channels-last input's order)
    grad_input.copy_(gi);
    return {grad_input, gw, go.defined() ? go.to(pr.input.scalar_type()) : go,
            gm.defined() ? gm.to(pr.input.scalar_type()) : gm, gb};
}

// ---------------------------------------------------------------------------
// forward / backward, CUDA (HIP) key
// ---------------------------------------------------------------------------
Tensor forward_hip(int dim, bool transposed, const Tensor &input, const Tensor &weight,
                   const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
                   at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding,
                   at::IntArrayRef dilation, int64_t groups, const char *name, int64_t activation = 0,
                   double mask_scale = 0.0) {
    TORCH_CHECK(input.is_cuda(), name, ": expected a GPU (HIP) tensor");
    c10::DeviceGuard guard(input.device());
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    pr.desc.dtype = dtype_code(pr.input.scalar_type());
    set_mask_activation(pr, activation, mask_scale);
    Tensor output = at::empty(out_shape(pr), pr.input.options());
    if (output.numel() > 0 && image_too_large(pr.desc)) {
        output = forward_channel_split(pr, name);
    } else if (output.numel() > 0) {
        const size_t ws_bytes = tvdcn_deform_conv_forward_workspace_size(&pr.desc);
        TORCH_CHECK(ws_bytes > 0 || pr.desc.batch == 0, name, ": ", tvdcn_last_error());
        Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 1)}, pr.input.options().dtype(at::kByte));
        Tensor x = aligned(pr.input), w = aligned(pr.weight), o = aligned(pr.offset), m = aligned(pr.mask),
               b = aligned(pr.bias);
        check_status(tvdcn_deform_conv_forward(&pr.desc, x.data_ptr(), w.data_ptr(), ptr_or_null(o), ptr_or_null(m),
                                               ptr_or_null(b), output.data_ptr(), ws.data_ptr(), ws_bytes,
                                               current_stream(output)),
                     name);
    } else {
        output.zero_();
    }
    if (pr.unbatched) output = output.squeeze(0);
    return output;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_hip(
    int dim, bool transposed, const Tensor &grad, const Tensor &input, const Tensor &weight,
    const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
    at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding, at::IntArrayRef dilation,
    int64_t groups, const char *name, int64_t activation = 0, double mask_scale = 0.0) {
    TORCH_CHECK(input.is_cuda(), name, ": expected a GPU (HIP) tensor");
    c10::DeviceGuard guard(input.device());
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    pr.desc.dtype = dtype_code(pr.input.scalar_type());
    set_mask_activation(pr, activation, mask_scale);
    Tensor g = grad.contiguous();
    if (pr.unbatched) g = g.unsqueeze(0);
    TORCH_CHECK(g.sizes() == at::IntArrayRef(out_shape(pr)), name, ": grad has shape ", g.sizes(), ", expected ",
                at::IntArrayRef(out_shape(pr)));
    TORCH_CHECK(g.scalar_type() == pr.input.scalar_type(), name, ": grad dtype must match input dtype");

    if (image_too_large(pr.desc)) {
        auto [grad_input, grad_weight, grad_offset, grad_mask, grad_bias] = backward_channel_split(pr, g, name);
        if (pr.unbatched) {
            grad_input = grad_input.squeeze(0);
            if (grad_offset.defined()) grad_offset = grad_offset.squeeze(0);
            if (grad_mask.defined()) grad_mask = grad_mask.squeeze(0);
        }
        return {grad_input, grad_weight, grad_offset, grad_mask, grad_bias};
    }
    Tensor grad_input = at::empty_like(pr.input);
    Tensor grad_weight = at::empty_like(pr.weight);
    Tensor grad_offset = pr.offset.defined() ? at::empty_like(pr.offset) : Tensor();
    Tensor grad_mask = pr.mask.defined() ? at::empty_like(pr.mask) : Tensor();
    Tensor grad_bias = pr.bias.defined() ? at::empty({pr.desc.out_channels}, pr.input.options()) : Tensor();
    const size_t ws_bytes = tvdcn_deform_conv_backward_workspace_size(&pr.desc);
    TORCH_CHECK(ws_bytes > 0, name, ": ", tvdcn_last_error());
    Tensor ws = at::empty({(int64_t)ws_bytes}, pr.input.options().dtype(at::kByte));
    Tensor ga = aligned(g), x = aligned(pr.input), w = aligned(pr.weight), o = aligned(pr.offset),
           m = aligned(pr.mask);
    check_status(tvdcn_deform_conv_backward(&pr.desc, ga.data_ptr(), x.data_ptr(), w.data_ptr(), ptr_or_null(o),
                                            ptr_or_null(m), grad_input.data_ptr(), grad_weight.data_ptr(),
                                            mut_ptr_or_null(grad_offset), mut_ptr_or_null(grad_mask),
                                            mut_ptr_or_null(grad_bias), ws.data_ptr(), ws_bytes,
                                            current_stream(grad_input)),
                 name);
    if (pr.unbatched) {
        grad_input = grad_input.squeeze(0);
        if (grad_offset.defined()) grad_offset = grad_offset.squeeze(0);
        if (grad_mask.defined()) grad_mask = grad_mask.squeeze(0);
    }
    return {grad_input, grad_weight, grad_offset, grad_mask, grad_bias};
}

// ---------------------------------------------------------------------------
// Meta key: same validation, shapes only (no data, no compute)
// ---------------------------------------------------------------------------
Tensor forward_meta(int dim, bool transposed, const Tensor &input, const Tensor &weight,
                    const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
                    at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding,
                    at::IntArrayRef dilation, int64_t groups, const char *name) {
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    dtype_code(pr.input.scalar_type());
    Tensor output = at::empty(out_shape(pr), pr.input.options());
    if (pr.unbatched) output = output.squeeze(0);
    return output;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_meta(
    int dim, bool transposed, const Tensor &grad, const Tensor &input, const Tensor &weight,
    const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
    at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding, at::IntArrayRef dilation,
    int64_t groups, const char *name) {
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    (void)grad;
    return {at::empty_like(input), at::empty_like(weight),
            pr.offset.defined() ? at::empty_like(offset.value()) : Tensor(),
            pr.mask.defined() ? at::empty_like(mask.value()) : Tensor(),
            pr.bias.defined() ? at::empty({pr.desc.out_channels}, input.options()) : Tensor()};
}

// ---------------------------------------------------------------------------
// CPU key: same validation, host kernels (cpu_kernels.cpp); channels-last host inputs are
// made NC<spatial>-contiguous first, as the reference does (cpu/deform_conv2d_kernel.cpp:114)
// ---------------------------------------------------------------------------
cpu::Operands cpu_operands(Problem &pr) {
    dtype_code(pr.input.scalar_type());
    if (pr.channels_last) {
        pr.input = pr.input.contiguous();
        pr.channels_last = false;
        pr.desc.flags &= ~TVDCN_FLAG_CHANNELS_LAST;
    }
    return cpu::Operands{pr.desc, pr.out_size, pr.input, pr.weight, pr.offset, pr.mask, pr.bias};
}

Tensor forward_cpu(int dim, bool transposed, const Tensor &input, const Tensor &weight,
                   const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
                   at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding,
                   at::IntArrayRef dilation, int64_t groups, const char *name, int64_t activation = 0,
                   double mask_scale = 0.0) {
    TORCH_CHECK(input.device().is_cpu(), name, ": expected a CPU tensor");
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    set_mask_activation(pr, activation, mask_scale);
    Tensor output = cpu::forward(cpu_operands(pr));
    if (pr.unbatched) output = output.squeeze(0);
    return output;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_cpu(
    int dim, bool transposed, const Tensor &grad, const Tensor &input, const Tensor &weight,
    const optional<Tensor> &offset, const optional<Tensor> &mask, const optional<Tensor> &bias,
    at::IntArrayRef stride, at::IntArrayRef padding, at::IntArrayRef output_padding, at::IntArrayRef dilation,
    int64_t groups, const char *name, int64_t activation = 0, double mask_scale = 0.0) {
    TORCH_CHECK(input.device().is_cpu(), name, ": expected a CPU tensor");
    Problem pr = make_problem(dim, transposed, input, weight, offset, mask, bias, stride, padding, output_padding,
                              dilation, groups, name);
    set_mask_activation(pr, activation, mask_scale);
    Tensor g = grad.contiguous();
    if (pr.unbatched) g = g.unsqueeze(0);
    TORCH_CHECK(g.sizes() == at::IntArrayRef(out_shape(pr)), name, ": grad has shape ", g.sizes(), ", expected ",
                at::IntArrayRef(out_shape(pr)));
    TORCH_CHECK(g.scalar_type() == pr.input.scalar_type(), name, ": grad dtype must match input dtype");
    auto r = cpu::backward(cpu_operands(pr), g);
    if (pr.unbatched) {
        std::get<0>(r) = std::get<0>(r).squeeze(0);
        if (std::get<2>(r).defined()) std::get<2>(r) = std::get<2>(r).squeeze(0);
        if (std::get<3>(r).defined()) std::get<3>(r) = std::get<3>(r).squeeze(0);
    }
    return r;
}

// ---------------------------------------------------------------------------
// autograd (ops/autograd/deform_conv2d_kernel.cpp:9-203): save the five tensors,
// backward calls the `_..._backward` op, which itself refuses double backward.
// ---------------------------------------------------------------------------
struct OpNames {
    const char *fwd;
    const char *bwd;
};

template <int DIM, bool TR>
struct Names;
#define TVDCN_NAMES(D, TRV, F, Bw)                               \
    template <>                                                  \
    struct Names<D, TRV> {                                       \
        static constexpr const char *fwd = "tvdcn::" F;      \
        static constexpr const char *bwd = "tvdcn::" Bw;     \
        static constexpr const char *short_name = F;             \
    };
TVDCN_NAMES(1, false, "deform_conv1d", "_deform_conv1d_backward")
TVDCN_NAMES(2, false, "deform_conv2d", "_deform_conv2d_backward")
TVDCN_NAMES(3, false, "deform_conv3d", "_deform_conv3d_backward")
TVDCN_NAMES(1, true, "deform_conv_transpose1d", "_deform_conv_transpose1d_backward")
TVDCN_NAMES(2, true, "deform_conv_transpose2d", "_deform_conv_transpose2d_backward")
TVDCN_NAMES(3, true, "deform_conv_transpose3d", "_deform_conv_transpose3d_backward")
#undef TVDCN_NAMES

using FwdSig = Tensor(const Tensor &, const Tensor &, const optional<Tensor> &, const optional<Tensor> &,
                      const optional<Tensor> &, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef,
                      int64_t);
using BwdSig = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor>(
    const Tensor &, const Tensor &, const Tensor &, const optional<Tensor> &, const optional<Tensor> &,
    const optional<Tensor> &, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t);
// conv schemas have no output_padding: their typed signatures differ
using FwdSigC = Tensor(const Tensor &, const Tensor &, const optional<Tensor> &, const optional<Tensor> &,
                       const optional<Tensor> &, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t);
using BwdSigC = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor>(
    const Tensor &, const Tensor &, const Tensor &, const optional<Tensor> &, const optional<Tensor> &,
    const optional<Tensor> &, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t);

template <int DIM, bool TR>
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> call_backward(const Tensor &grad, const Tensor &input,
                                                                 const Tensor &weight, const optional<Tensor> &offset,
                                                                 const optional<Tensor> &mask,
                                                                 const optional<Tensor> &bias, at::IntArrayRef stride,
                                                                 at::IntArrayRef padding, at::IntArrayRef out_pad,
                                                                 at::IntArrayRef dilation, int64_t groups) {
    if constexpr (TR) {
        static auto op = c10::Dispatcher::singleton().findSchemaOrThrow(Names<DIM, TR>::bwd, "").template typed<BwdSig>();
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, out_pad, dilation, groups);
    } else {
        static auto op =
            c10::Dispatcher::singleton().findSchemaOrThrow(Names<DIM, TR>::bwd, "").template typed<BwdSigC>();
        return op.call(grad, input, weight, offset, mask, bias, stride, padding, dilation, groups);
    }
}

template <int DIM, bool TR>
Tensor call_forward(const Tensor &input, const Tensor &weight, const optional<Tensor> &offset,
                    const optional<Tensor> &mask, const optional<Tensor> &bias, at::IntArrayRef stride,
                    at::IntArrayRef padding, at::IntArrayRef out_pad, at::IntArrayRef dilation, int64_t groups) {
    if constexpr (TR) {
        static auto op = c10::Dispatcher::singleton().findSchemaOrThrow(Names<DIM, TR>::fwd, "").template typed<FwdSig>();
        return op.call(input, weight, offset, mask, bias, stride, padding, out_pad, dilation, groups);
    } else {
        static auto op =
            c10::Dispatcher::singleton().findSchemaOrThrow(Names<DIM, TR>::fwd, "").template typed<FwdSigC>();
        return op.call(input, weight, offset, mask, bias, stride, padding, dilation, groups);
    }
}

optional<Tensor> opt(const Tensor &t) { return t.defined() ? optional<Tensor>(t) : optional<Tensor>(); }

// Opt-in (tvdcn::_set_keep_input_copy): for float32 1D / 2D / 3D conv inputs in NC<spatial> order
// the forward makes the channels-last copy that the kernels sample (tvdcn_to_channels_last) and
// the autograd node saves it instead of the input, so that the backward skips its own copy; the
// backward writes grad_input channels-last and brings it back to NC<spatial>
// (tvdcn_from_channels_last). It costs one |input| of device memory per layer until the backward
// runs (the caller usually holds the input too), and an in-place change of the input after the
// forward is no longer detected; off by default, the node saves the input as the reference does
// (autograd/deform_conv2d_kernel.cpp:35).
std::atomic<bool> g_keep_input_copy{false};

bool set_keep_input_copy(bool enable) { return g_keep_input_copy.exchange(enable); }

bool keeps_cl_copy(const Tensor &x, int dim, bool transposed) {
    if (!g_keep_input_copy.load()) return false;
    if (transposed || dim < 1 || dim > 3 || !x.is_cuda() || x.scalar_type() != at::kFloat ||
        x.dim() != dim + 2 || !x.is_contiguous() || x.numel() == 0)
        return false;
    // traced calls (fake / functional tensors, dispatch modes) hold no device memory to copy
    // and record dispatcher ops only: they keep the plain path
    if (c10::impl::dispatch_mode_enabled() || x.key_set().has(c10::DispatchKey::Python) ||
        at::functionalization::impl::isFunctionalTensor(x))
        return false;
    // (the layout copy indexes in 32 bits; larger inputs keep the plain path, which batch-blocks)
    return x.size(1) > 1 && x.numel() > x.size(0) * x.size(1) && x.numel() <= INT32_MAX;   // else both orders coincide
}

Tensor cl_copy(const Tensor &x, int dim, bool to_cl) {
    TORCH_CHECK(to_cl ? x.is_contiguous() : is_channels_last(x, dim), "cl_copy: unexpected memory layout");
    c10::DeviceGuard guard(x.device());
    const int64_t B = x.size(0), C = x.size(1), S = x.numel() / (B * C);
    Tensor y;
    if (!to_cl)
        y = at::empty_like(x, at::MemoryFormat::Contiguous);
    else if (dim == 1)
        y = at::empty({B, x.size(2), C}, x.options()).permute({0, 2, 1});   // (B, C, L), strides (L * C, 1, C)
    else
        y = at::empty_like(x, dim == 2 ? at::MemoryFormat::ChannelsLast : at::MemoryFormat::ChannelsLast3d);
    const auto fn = to_cl ? tvdcn_to_channels_last : tvdcn_from_channels_last;
    check_status(fn(TVDCN_DTYPE_FLOAT32, B, C, S, x.data_ptr(), y.data_ptr(), current_stream(y)),
                 to_cl ? "to_channels_last" : "from_channels_last");
    return y;
}

template <int DIM, bool TR>
class DeformFunction : public torch::autograd::Function<DeformFunction<DIM, TR>> {
   public:
    static torch::autograd::Variable forward(torch::autograd::AutogradContext *ctx, const Tensor &input,
                                             const Tensor &weight, const optional<Tensor> &offset,
                                             const optional<Tensor> &mask, const optional<Tensor> &bias,
                                             at::IntArrayRef stride, at::IntArrayRef padding,
                                             at::IntArrayRef out_pad, at::IntArrayRef dilation, int64_t groups) {
        at::AutoDispatchBelowADInplaceOrView guard;
        const bool cl = keeps_cl_copy(input, DIM, TR);
        const Tensor x = cl ? cl_copy(input, DIM, true) : input;
        Tensor output = call_forward<DIM, TR>(x, weight, offset, mask, bias, stride, padding, out_pad, dilation, groups);
        ctx->save_for_backward({x, weight, offset.value_or(Tensor()), mask.value_or(Tensor()),
                                bias.value_or(Tensor())});
        ctx->saved_data["cl_copy"] = cl;
        ctx->saved_data["stride"] = stride.vec();
        ctx->saved_data["padding"] = padding.vec();
        ctx->saved_data["output_padding"] = out_pad.vec();
        ctx->saved_data["dilation"] = dilation.vec();
        ctx->saved_data["groups"] = groups;
        return output;
    }

    static torch::autograd::variable_list backward(torch::autograd::AutogradContext *ctx,
                                                   const torch::autograd::variable_list &grad_output) {
        auto saved = ctx->get_saved_variables();
        const auto stride = ctx->saved_data["stride"].toIntVector();
        const auto padding = ctx->saved_data["padding"].toIntVector();
        const auto out_pad = ctx->saved_data["output_padding"].toIntVector();
        const auto dilation = ctx->saved_data["dilation"].toIntVector();
        const int64_t groups = ctx->saved_data["groups"].toInt();
        auto grads = call_backward<DIM, TR>(grad_output[0], saved[0], saved[1], opt(saved[2]), opt(saved[3]),
                                            opt(saved[4]), stride, padding, out_pad, dilation, groups);
        if (ctx->saved_data["cl_copy"].toBool() && std::get<0>(grads).defined())
            std::get<0>(grads) = cl_copy(std::get<0>(grads), DIM, false);
        return {std::get<0>(grads), std::get<1>(grads), std::get<2>(grads), std::get<3>(grads), std::get<4>(grads),
                Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// Autograd kernel of the backward op: runs it below autograd; when any input
// still requires grad, the outputs get a node that raises on use
// (ops/autograd/deform_conv2d_kernel.cpp:96-144: "double backwards on ... not supported").
template <int DIM, bool TR>
class DeformBackwardFunction : public torch::autograd::Function<DeformBackwardFunction<DIM, TR>> {
   public:
    static torch::autograd::variable_list forward(torch::autograd::AutogradContext *ctx, const Tensor &grad,
                                                  const Tensor &input, const Tensor &weight,
                                                  const optional<Tensor> &offset, const optional<Tensor> &mask,
                                                  const optional<Tensor> &bias, at::IntArrayRef stride,
                                                  at::IntArrayRef padding, at::IntArrayRef out_pad,
                                                  at::IntArrayRef dilation, int64_t groups) {
        at::AutoDispatchBelowADInplaceOrView guard;
        auto r = call_backward<DIM, TR>(grad, input, weight, offset, mask, bias, stride, padding, out_pad, dilation,
                                        groups);
        // undefined gradients (absent offset / mask / bias) are returned as
        // empty placeholders here and turned back into undefined by the caller
        ctx->saved_data["defined"] = std::vector<int64_t>{std::get<2>(r).defined(), std::get<3>(r).defined(),
                                                          std::get<4>(r).defined()};
        auto ph = [&](const Tensor &t) { return t.defined() ? t : at::empty({0}, input.options()); };
        return {std::get<0>(r), std::get<1>(r), ph(std::get<2>(r)), ph(std::get<3>(r)), ph(std::get<4>(r))};
    }
    static torch::autograd::variable_list backward(torch::autograd::AutogradContext *,
                                                   const torch::autograd::variable_list &) {
        TORCH_CHECK(false, "double backwards on ", Names<DIM, TR>::short_name, " not supported");
        return {};
    }
};

template <int DIM, bool TR>
Tensor forward_autograd(const Tensor &input, const Tensor &weight, const optional<Tensor> &offset,
                        const optional<Tensor> &mask, const optional<Tensor> &bias, at::IntArrayRef stride,
                        at::IntArrayRef padding, at::IntArrayRef out_pad, at::IntArrayRef dilation, int64_t groups) {
    return DeformFunction<DIM, TR>::apply(input, weight, offset, mask, bias, stride, padding, out_pad, dilation,
                                          groups);
}

template <int DIM, bool TR>
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_autograd(
    const Tensor &grad, const Tensor &input, const Tensor &weight, const optional<Tensor> &offset,
    const optional<Tensor> &mask, const optional<Tensor> &bias, at::IntArrayRef stride, at::IntArrayRef padding,
    at::IntArrayRef out_pad, at::IntArrayRef dilation, int64_t groups) {
    auto r = DeformBackwardFunction<DIM, TR>::apply(grad, input, weight, offset, mask, bias, stride, padding, out_pad,
                                                    dilation, groups);
    const bool has_off = offset.has_value() && offset->defined();
    const bool has_mask = mask.has_value() && mask->defined();
    const bool has_bias = bias.has_value() && bias->defined();
    return {r[0], r[1], has_off ? r[2] : Tensor(), has_mask ? r[3] : Tensor(), has_bias ? r[4] : Tensor()};
}

// ---------------------------------------------------------------------------
// autocast (ops/autocast/deform_conv2d_kernel.cpp:9-38): run in fp32, cast back
// ---------------------------------------------------------------------------
template <int DIM, bool TR>
Tensor forward_autocast(const Tensor &input, const Tensor &weight, const optional<Tensor> &offset,
                        const optional<Tensor> &mask, const optional<Tensor> &bias, at::IntArrayRef stride,
                        at::IntArrayRef padding, at::IntArrayRef out_pad, at::IntArrayRef dilation, int64_t groups) {
    c10::impl::ExcludeDispatchKeyGuard no_autocast(c10::DispatchKey::Autocast);
    auto f32 = [](const optional<Tensor> &t) -> optional<Tensor> {
        if (!t.has_value() || !t->defined()) return t;
        return at::autocast::cached_cast(at::kFloat, *t, c10::DeviceType::CUDA);
    };
    return call_forward<DIM, TR>(at::autocast::cached_cast(at::kFloat, input, c10::DeviceType::CUDA),
                                 at::autocast::cached_cast(at::kFloat, weight, c10::DeviceType::CUDA), f32(offset),
                                 f32(mask), f32(bias), stride, padding, out_pad, dilation, groups)
        .to(input.scalar_type());
}

// ---------------------------------------------------------------------------
// kernel adapters with the exact schema signatures
// ---------------------------------------------------------------------------
template <int DIM, bool TR>
struct Kernels {
    // conv signature (no output_padding) adapters
    static Tensor fwd_hip_c(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                            const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef d,
                            int64_t g) {
        return forward_hip(DIM, TR, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_hip_t(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                            const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                            at::IntArrayRef d, int64_t g) {
        return forward_hip(DIM, TR, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_meta_c(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                             const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef d,
                             int64_t g) {
        return forward_meta(DIM, TR, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_meta_t(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                             const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                             at::IntArrayRef d, int64_t g) {
        return forward_meta(DIM, TR, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_cpu_c(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                            const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef d,
                            int64_t g) {
        return forward_cpu(DIM, TR, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_cpu_t(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                            const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                            at::IntArrayRef d, int64_t g) {
        return forward_cpu(DIM, TR, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    using G5 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor>;
    static G5 bwd_cpu_c(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                        const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                        at::IntArrayRef d, int64_t g) {
        return backward_cpu(DIM, TR, gr, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g, Names<DIM, TR>::short_name);
    }
    static G5 bwd_cpu_t(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                        const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                        at::IntArrayRef op, at::IntArrayRef d, int64_t g) {
        return backward_cpu(DIM, TR, gr, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    static G5 bwd_hip_c(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                        const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                        at::IntArrayRef d, int64_t g) {
        return backward_hip(DIM, TR, gr, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g, Names<DIM, TR>::short_name);
    }
    static G5 bwd_hip_t(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                        const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                        at::IntArrayRef op, at::IntArrayRef d, int64_t g) {
        return backward_hip(DIM, TR, gr, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    static G5 bwd_meta_c(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                         const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                         at::IntArrayRef d, int64_t g) {
        return backward_meta(DIM, TR, gr, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g,
                             Names<DIM, TR>::short_name);
    }
    static G5 bwd_meta_t(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                         const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                         at::IntArrayRef op, at::IntArrayRef d, int64_t g) {
        return backward_meta(DIM, TR, gr, i, w, o, m, b, s, p, op, d, g, Names<DIM, TR>::short_name);
    }
    static Tensor fwd_ag_c(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                           const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef d,
                           int64_t g) {
        return forward_autograd<DIM, TR>(i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g);
    }
    static Tensor fwd_ag_t(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                           const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                           at::IntArrayRef d, int64_t g) {
        return forward_autograd<DIM, TR>(i, w, o, m, b, s, p, op, d, g);
    }
    static G5 bwd_ag_c(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                       const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                       at::IntArrayRef d, int64_t g) {
        return backward_autograd<DIM, TR>(gr, i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g);
    }
    static G5 bwd_ag_t(const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o,
                       const optional<Tensor> &m, const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p,
                       at::IntArrayRef op, at::IntArrayRef d, int64_t g) {
        return backward_autograd<DIM, TR>(gr, i, w, o, m, b, s, p, op, d, g);
    }
    static Tensor fwd_ac_c(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                           const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef d,
                           int64_t g) {
        return forward_autocast<DIM, TR>(i, w, o, m, b, s, p, at::IntArrayRef({0}), d, g);
    }
    static Tensor fwd_ac_t(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const optional<Tensor> &m,
                           const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                           at::IntArrayRef d, int64_t g) {
        return forward_autocast<DIM, TR>(i, w, o, m, b, s, p, op, d, g);
    }
};

// ---------------------------------------------------------------------------
// mask_softmax: x viewed as (B, groups, K, S), softmax over K
// ---------------------------------------------------------------------------
void softmax_dims(const Tensor &x, int64_t K, int64_t &B, int64_t &G, int64_t &S) {
    TORCH_CHECK(x.dim() >= 2, "mask_softmax: expected a (batch, groups * kernel_numel, *spatial) tensor");
    TORCH_CHECK(K > 0, "mask_softmax: kernel_numel must be positive");
    B = x.size(0);
    G = x.size(1) / K;
    TORCH_CHECK(G > 0 && G * K == x.size(1), "The shape of the mask tensor at dimension 1 is not valid. It should ",
                "be a multiple of the kernel size.\nGot mask.size(1)=", x.size(1), ", while kernel_numel=", K);
    S = 1;
    for (int64_t i = 2; i < x.dim(); ++i) S *= x.size(i);
}

Tensor mask_softmax_hip(const Tensor &x, int64_t K) {
    TORCH_CHECK(x.is_cuda(), "mask_softmax: expected a GPU (HIP) tensor");
    c10::DeviceGuard guard(x.device());
    int64_t B, G, S;
    softmax_dims(x, K, B, G, S);
    Tensor xc = x.contiguous();
    Tensor y = at::empty_like(xc);
    check_status(tvdcn_mask_softmax_forward(dtype_code(xc.scalar_type()), B, G, K, S, xc.data_ptr(), y.data_ptr(),
                                            current_stream(y)),
                 "mask_softmax");
    return y;
}

Tensor mask_softmax_backward_hip(const Tensor &grad, const Tensor &y, int64_t K) {
    TORCH_CHECK(y.is_cuda(), "mask_softmax: expected a GPU (HIP) tensor");
    c10::DeviceGuard guard(y.device());
    int64_t B, G, S;
    softmax_dims(y, K, B, G, S);
    Tensor yc = y.contiguous(), gc = grad.contiguous();
    TORCH_CHECK(gc.sizes() == yc.sizes() && gc.scalar_type() == yc.scalar_type(),
                "mask_softmax backward: grad must match the output");
    Tensor gx = at::empty_like(yc);
    check_status(tvdcn_mask_softmax_backward(dtype_code(yc.scalar_type()), B, G, K, S, yc.data_ptr(), gc.data_ptr(),
                                             gx.data_ptr(), current_stream(gx)),
                 "mask_softmax backward");
    return gx;
}

Tensor mask_softmax_cpu(const Tensor &x, int64_t K) {
    TORCH_CHECK(x.device().is_cpu(), "mask_softmax: expected a CPU tensor");
    int64_t B, G, S;
    softmax_dims(x, K, B, G, S);
    dtype_code(x.scalar_type());
    return cpu::mask_softmax(x, B, G, K, S);
}

Tensor mask_softmax_backward_cpu(const Tensor &grad, const Tensor &y, int64_t K) {
    TORCH_CHECK(y.device().is_cpu(), "mask_softmax: expected a CPU tensor");
    int64_t B, G, S;
    softmax_dims(y, K, B, G, S);
    TORCH_CHECK(grad.sizes() == y.sizes() && grad.scalar_type() == y.scalar_type(),
                "mask_softmax backward: grad must match the output");
    return cpu::mask_softmax_backward(grad, y, B, G, K, S);
}

Tensor mask_softmax_meta(const Tensor &x, int64_t K) {
    int64_t B, G, S;
    softmax_dims(x, K, B, G, S);
    return at::empty_like(x, at::MemoryFormat::Contiguous);
}

Tensor mask_softmax_backward_meta(const Tensor &grad, const Tensor &y, int64_t K) {
    int64_t B, G, S;
    softmax_dims(y, K, B, G, S);
    (void)grad;
    return at::empty_like(y, at::MemoryFormat::Contiguous);
}

class MaskSoftmaxFunction : public torch::autograd::Function<MaskSoftmaxFunction> {
   public:
    static Tensor forward(torch::autograd::AutogradContext *ctx, const Tensor &x, int64_t K) {
        at::AutoDispatchBelowADInplaceOrView guard;
        static auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("tvdcn::mask_softmax", "")
                             .typed<Tensor(const Tensor &, int64_t)>();
        Tensor y = op.call(x, K);
        ctx->save_for_backward({y});
        ctx->saved_data["K"] = K;
        return y;
    }
    static torch::autograd::variable_list backward(torch::autograd::AutogradContext *ctx,
                                                   const torch::autograd::variable_list &g) {
        static auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("tvdcn::_mask_softmax_backward", "")
                             .typed<Tensor(const Tensor &, const Tensor &, int64_t)>();
        auto saved = ctx->get_saved_variables();
        return {op.call(g[0], saved[0], ctx->saved_data["K"].toInt()), Tensor()};
    }
};

Tensor mask_softmax_autograd(const Tensor &x, int64_t K) { return MaskSoftmaxFunction::apply(x, K); }

// ---------------------------------------------------------------------------
// deform_conv_mask_activation: conv / transposed conv (rank from len(stride)) whose mask
// tensor holds logits, activated in the kernels' mask load: activation 1 = mask_scale *
// sigmoid (tvdcn's MaskSigmoid), 2 = softmax over the kernel taps of each mask group
// (MaskSoftmax{N}d). The backward's mask gradient is with respect to the logits. Used by the
// packed modules for those two activations; no counterpart op in the reference, whose
// packed modules run the activation as separate passes (ops/deform_conv.py:623-626).
// ---------------------------------------------------------------------------
const char *kActName = "deform_conv_mask_activation";

int act_dim(at::IntArrayRef stride) {
    TORCH_CHECK(stride.size() >= 1 && stride.size() <= 3, kActName, ": stride must have 1 to 3 ",
                "elements (one per spatial axis)");
    return (int)stride.size();
}

void check_activation(int64_t activation, double scale) {
    TORCH_CHECK(activation == 1 || activation == 2, kActName, ": activation must be 1 (sigmoid) or 2 (softmax), got ",
                activation);
    TORCH_CHECK(activation != 1 || (scale > 0.0 && std::isfinite(scale)), "mask_scale must be a positive finite number");
}

Tensor act_fwd_hip(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                   const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                   at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    check_activation(act, scale);
    return forward_hip(act_dim(s), tr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName, act, scale);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> act_bwd_hip(const Tensor &gr, const Tensor &i, const Tensor &w,
                                                               const optional<Tensor> &o, const Tensor &m,
                                                               const optional<Tensor> &b, at::IntArrayRef s,
                                                               at::IntArrayRef p, at::IntArrayRef op,
                                                               at::IntArrayRef d, int64_t g, bool tr, int64_t act,
                                                               double scale) {
    check_activation(act, scale);
    return backward_hip(act_dim(s), tr, gr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName, act, scale);
}

Tensor act_fwd_cpu(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                   const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                   at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    check_activation(act, scale);
    return forward_cpu(act_dim(s), tr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName, act, scale);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> act_bwd_cpu(const Tensor &gr, const Tensor &i, const Tensor &w,
                                                               const optional<Tensor> &o, const Tensor &m,
                                                               const optional<Tensor> &b, at::IntArrayRef s,
                                                               at::IntArrayRef p, at::IntArrayRef op,
                                                               at::IntArrayRef d, int64_t g, bool tr, int64_t act,
                                                               double scale) {
    check_activation(act, scale);
    return backward_cpu(act_dim(s), tr, gr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName, act, scale);
}

Tensor act_fwd_meta(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                    const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                    at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    check_activation(act, scale);
    return forward_meta(act_dim(s), tr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> act_bwd_meta(const Tensor &gr, const Tensor &i, const Tensor &w,
                                                                const optional<Tensor> &o, const Tensor &m,
                                                                const optional<Tensor> &b, at::IntArrayRef s,
                                                                at::IntArrayRef p, at::IntArrayRef op,
                                                                at::IntArrayRef d, int64_t g, bool tr, int64_t act,
                                                                double scale) {
    check_activation(act, scale);
    return backward_meta(act_dim(s), tr, gr, i, w, o, optional<Tensor>(m), b, s, p, op, d, g, kActName);
}

using ActFwdSig = Tensor(const Tensor &, const Tensor &, const optional<Tensor> &, const Tensor &,
                         const optional<Tensor> &, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef,
                         int64_t, bool, int64_t, double);
using ActBwdSig = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor>(
    const Tensor &, const Tensor &, const Tensor &, const optional<Tensor> &, const Tensor &, const optional<Tensor> &,
    at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t, bool, int64_t, double);

Tensor act_call_forward(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                        const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                        at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    static auto fop =
        c10::Dispatcher::singleton().findSchemaOrThrow("tvdcn::deform_conv_mask_activation", "").typed<ActFwdSig>();
    return fop.call(i, w, o, m, b, s, p, op, d, g, tr, act, scale);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> act_call_backward(
    const Tensor &gr, const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
    const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op, at::IntArrayRef d, int64_t g,
    bool tr, int64_t act, double scale) {
    static auto bop = c10::Dispatcher::singleton()
                          .findSchemaOrThrow("tvdcn::_deform_conv_mask_activation_backward", "")
                          .typed<ActBwdSig>();
    return bop.call(gr, i, w, o, m, b, s, p, op, d, g, tr, act, scale);
}

class MaskActivationFunction : public torch::autograd::Function<MaskActivationFunction> {
   public:
    static torch::autograd::Variable forward(torch::autograd::AutogradContext *ctx, const Tensor &input,
                                             const Tensor &weight, const optional<Tensor> &offset,
                                             const Tensor &mask, const optional<Tensor> &bias, at::IntArrayRef stride,
                                             at::IntArrayRef padding, at::IntArrayRef out_pad,
                                             at::IntArrayRef dilation, int64_t groups, bool transposed,
                                             int64_t activation, double scale) {
        at::AutoDispatchBelowADInplaceOrView guard;
        const int dim = (int)stride.size();
        const bool cl = keeps_cl_copy(input, dim, transposed);
        const Tensor x = cl ? cl_copy(input, dim, true) : input;
        Tensor output = act_call_forward(x, weight, offset, mask, bias, stride, padding, out_pad, dilation, groups,
                                         transposed, activation, scale);
        ctx->save_for_backward({x, weight, offset.value_or(Tensor()), mask, bias.value_or(Tensor())});
        ctx->saved_data["cl_copy"] = cl;
        ctx->saved_data["stride"] = stride.vec();
        ctx->saved_data["padding"] = padding.vec();
        ctx->saved_data["output_padding"] = out_pad.vec();
        ctx->saved_data["dilation"] = dilation.vec();
        ctx->saved_data["groups"] = groups;
        ctx->saved_data["transposed"] = transposed;
        ctx->saved_data["activation"] = activation;
        ctx->saved_data["scale"] = scale;
        return output;
    }

    static torch::autograd::variable_list backward(torch::autograd::AutogradContext *ctx,
                                                   const torch::autograd::variable_list &grad_output) {
        auto saved = ctx->get_saved_variables();
        auto grads = act_call_backward(
            grad_output[0], saved[0], saved[1], opt(saved[2]), saved[3], opt(saved[4]),
            ctx->saved_data["stride"].toIntVector(), ctx->saved_data["padding"].toIntVector(),
            ctx->saved_data["output_padding"].toIntVector(), ctx->saved_data["dilation"].toIntVector(),
            ctx->saved_data["groups"].toInt(), ctx->saved_data["transposed"].toBool(),
            ctx->saved_data["activation"].toInt(), ctx->saved_data["scale"].toDouble());
        if (ctx->saved_data["cl_copy"].toBool() && std::get<0>(grads).defined())
            std::get<0>(grads) = cl_copy(std::get<0>(grads), (int)saved[0].dim() - 2, false);
        return {std::get<0>(grads), std::get<1>(grads), std::get<2>(grads), std::get<3>(grads), std::get<4>(grads),
                Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

class MaskActivationBackwardFunction : public torch::autograd::Function<MaskActivationBackwardFunction> {
   public:
    static torch::autograd::variable_list forward(torch::autograd::AutogradContext *, const Tensor &grad,
                                                  const Tensor &input, const Tensor &weight,
                                                  const optional<Tensor> &offset, const Tensor &mask,
                                                  const optional<Tensor> &bias, at::IntArrayRef stride,
                                                  at::IntArrayRef padding, at::IntArrayRef out_pad,
                                                  at::IntArrayRef dilation, int64_t groups, bool transposed,
                                                  int64_t activation, double scale) {
        at::AutoDispatchBelowADInplaceOrView guard;
        auto r = act_call_backward(grad, input, weight, offset, mask, bias, stride, padding, out_pad, dilation, groups,
                                   transposed, activation, scale);
        auto ph = [&](const Tensor &t) { return t.defined() ? t : at::empty({0}, input.options()); };
        return {std::get<0>(r), std::get<1>(r), ph(std::get<2>(r)), std::get<3>(r), ph(std::get<4>(r))};
    }
    static torch::autograd::variable_list backward(torch::autograd::AutogradContext *,
                                                   const torch::autograd::variable_list &) {
        TORCH_CHECK(false, "double backwards on ", kActName, " not supported");
        return {};
    }
};

Tensor act_fwd_autograd(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                        const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                        at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    return MaskActivationFunction::apply(i, w, o, m, b, s, p, op, d, g, tr, act, scale);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> act_bwd_autograd(const Tensor &gr, const Tensor &i,
                                                                    const Tensor &w, const optional<Tensor> &o,
                                                                    const Tensor &m, const optional<Tensor> &b,
                                                                    at::IntArrayRef s, at::IntArrayRef p,
                                                                    at::IntArrayRef op, at::IntArrayRef d, int64_t g,
                                                                    bool tr, int64_t act, double scale) {
    auto r = MaskActivationBackwardFunction::apply(gr, i, w, o, m, b, s, p, op, d, g, tr, act, scale);
    const bool has_off = o.has_value() && o->defined();
    const bool has_bias = b.has_value() && b->defined();
    return {r[0], r[1], has_off ? r[2] : Tensor(), r[3], has_bias ? r[4] : Tensor()};
}

Tensor act_fwd_autocast(const Tensor &i, const Tensor &w, const optional<Tensor> &o, const Tensor &m,
                        const optional<Tensor> &b, at::IntArrayRef s, at::IntArrayRef p, at::IntArrayRef op,
                        at::IntArrayRef d, int64_t g, bool tr, int64_t act, double scale) {
    c10::impl::ExcludeDispatchKeyGuard no_autocast(c10::DispatchKey::Autocast);
    auto f32 = [](const Tensor &t) { return at::autocast::cached_cast(at::kFloat, t, c10::DeviceType::CUDA); };
    auto f32o = [&](const optional<Tensor> &t) -> optional<Tensor> {
        if (!t.has_value() || !t->defined()) return t;
        return f32(*t);
    };
    return act_call_forward(f32(i), f32(w), f32o(o), f32(m), f32o(b), s, p, op, d, g, tr, act, scale)
        .to(i.scalar_type());
}

int64_t hip_version() { return tvdcn_hip_version(); }
std::string arch_flags() { return tvdcn_arch_flags(); }

}  // namespace
}  // namespace tvdcn_amd

// ---------------------------------------------------------------------------
// registration
// ---------------------------------------------------------------------------
#define TVDCN_CONV_SCHEMA(D)                                                                                   \
    "deform_conv" #D "d(Tensor input, Tensor weight, Tensor? offset=None, Tensor? mask=None, Tensor? bias=None, " \
    "SymInt[" #D "] stride=1, SymInt[" #D "] padding=0, SymInt[" #D "] dilation=1, SymInt groups=1) -> Tensor"
#define TVDCN_CONV_BWD_SCHEMA(D)                                                                                 \
    "_deform_conv" #D "d_backward(Tensor grad, Tensor input, Tensor weight, Tensor? offset=None, "               \
    "Tensor? mask=None, Tensor? bias=None, SymInt[" #D "] stride=1, SymInt[" #D "] padding=0, SymInt[" #D        \
    "] dilation=1, SymInt groups=1) -> (Tensor, Tensor, Tensor, Tensor, Tensor)"
#define TVDCN_TR_SCHEMA(D)                                                                                     \
    "deform_conv_transpose" #D "d(Tensor input, Tensor weight, Tensor? offset=None, Tensor? mask=None, "        \
    "Tensor? bias=None, SymInt[" #D "] stride=1, SymInt[" #D "] padding=0, SymInt[" #D "] output_padding=0, "   \
    "SymInt[" #D "] dilation=1, SymInt groups=1) -> Tensor"
#define TVDCN_TR_BWD_SCHEMA(D)                                                                                 \
    "_deform_conv_transpose" #D "d_backward(Tensor grad, Tensor input, Tensor weight, Tensor? offset=None, "    \
    "Tensor? mask=None, Tensor? bias=None, SymInt[" #D "] stride=1, SymInt[" #D "] padding=0, SymInt[" #D      \
    "] output_padding=0, SymInt[" #D "] dilation=1, SymInt groups=1) -> (Tensor, Tensor, Tensor, Tensor, Tensor)"

// a fragment (as the reference registers each op file, ops/deform_conv2d.cpp:117): other libraries
// may add operators to the namespace
TORCH_LIBRARY_FRAGMENT(tvdcn, m) {
    m.def(TVDCN_CONV_SCHEMA(1));
    m.def(TVDCN_CONV_BWD_SCHEMA(1));
    m.def(TVDCN_CONV_SCHEMA(2));
    m.def(TVDCN_CONV_BWD_SCHEMA(2));
    m.def(TVDCN_CONV_SCHEMA(3));
    m.def(TVDCN_CONV_BWD_SCHEMA(3));
    m.def(TVDCN_TR_SCHEMA(1));
    m.def(TVDCN_TR_BWD_SCHEMA(1));
    m.def(TVDCN_TR_SCHEMA(2));
    m.def(TVDCN_TR_BWD_SCHEMA(2));
    m.def(TVDCN_TR_SCHEMA(3));
    m.def(TVDCN_TR_BWD_SCHEMA(3));
    m.def("deform_conv_mask_activation(Tensor input, Tensor weight, Tensor? offset, Tensor mask, Tensor? bias, "
          "SymInt[] stride, SymInt[] padding, SymInt[] output_padding, SymInt[] dilation, SymInt groups, "
          "bool transposed, int activation, float mask_scale) -> Tensor");
    m.def("_deform_conv_mask_activation_backward(Tensor grad, Tensor input, Tensor weight, Tensor? offset, "
          "Tensor mask, Tensor? bias, SymInt[] stride, SymInt[] padding, SymInt[] output_padding, "
          "SymInt[] dilation, SymInt groups, bool transposed, int activation, float mask_scale) "
          "-> (Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def("mask_softmax(Tensor mask, int kernel_numel) -> Tensor");
    m.def("_mask_softmax_backward(Tensor grad, Tensor output, int kernel_numel) -> Tensor");
    m.def("_set_keep_input_copy", &tvdcn_amd::set_keep_input_copy);
    m.def("_cuda_version", &tvdcn_amd::hip_version);
    m.def("_cuda_arch_flags", &tvdcn_amd::arch_flags);
}

namespace tvdcn_amd {
using Conv1 = Kernels<1, false>;
using Conv2 = Kernels<2, false>;
using Conv3 = Kernels<3, false>;
using Tr1 = Kernels<1, true>;
using Tr2 = Kernels<2, true>;
using Tr3 = Kernels<3, true>;
}  // namespace tvdcn_amd

#define TVDCN_IMPL_CONV(D, KEYFN_F, KEYFN_B)                                                  \
    m.impl("deform_conv" #D "d", TORCH_FN(tvdcn_amd::Conv##D::KEYFN_F##_c));                  \
    m.impl("_deform_conv" #D "d_backward", TORCH_FN(tvdcn_amd::Conv##D::KEYFN_B##_c));        \
    m.impl("deform_conv_transpose" #D "d", TORCH_FN(tvdcn_amd::Tr##D::KEYFN_F##_t));          \
    m.impl("_deform_conv_transpose" #D "d_backward", TORCH_FN(tvdcn_amd::Tr##D::KEYFN_B##_t));

TORCH_LIBRARY_IMPL(tvdcn, CUDA, m) {
    TVDCN_IMPL_CONV(1, fwd_hip, bwd_hip)
    TVDCN_IMPL_CONV(2, fwd_hip, bwd_hip)
    TVDCN_IMPL_CONV(3, fwd_hip, bwd_hip)
    m.impl("deform_conv_mask_activation", TORCH_FN(tvdcn_amd::act_fwd_hip));
    m.impl("_deform_conv_mask_activation_backward", TORCH_FN(tvdcn_amd::act_bwd_hip));
    m.impl("mask_softmax", TORCH_FN(tvdcn_amd::mask_softmax_hip));
    m.impl("_mask_softmax_backward", TORCH_FN(tvdcn_amd::mask_softmax_backward_hip));
}

TORCH_LIBRARY_IMPL(tvdcn, CPU, m) {
    TVDCN_IMPL_CONV(1, fwd_cpu, bwd_cpu)
    TVDCN_IMPL_CONV(2, fwd_cpu, bwd_cpu)
    TVDCN_IMPL_CONV(3, fwd_cpu, bwd_cpu)
    m.impl("deform_conv_mask_activation", TORCH_FN(tvdcn_amd::act_fwd_cpu));
    m.impl("_deform_conv_mask_activation_backward", TORCH_FN(tvdcn_amd::act_bwd_cpu));
    m.impl("mask_softmax", TORCH_FN(tvdcn_amd::mask_softmax_cpu));
    m.impl("_mask_softmax_backward", TORCH_FN(tvdcn_amd::mask_softmax_backward_cpu));
}

TORCH_LIBRARY_IMPL(tvdcn, Meta, m) {
    TVDCN_IMPL_CONV(1, fwd_meta, bwd_meta)
    TVDCN_IMPL_CONV(2, fwd_meta, bwd_meta)
    TVDCN_IMPL_CONV(3, fwd_meta, bwd_meta)
    m.impl("deform_conv_mask_activation", TORCH_FN(tvdcn_amd::act_fwd_meta));
    m.impl("_deform_conv_mask_activation_backward", TORCH_FN(tvdcn_amd::act_bwd_meta));
    m.impl("mask_softmax", TORCH_FN(tvdcn_amd::mask_softmax_meta));
    m.impl("_mask_softmax_backward", TORCH_FN(tvdcn_amd::mask_softmax_backward_meta));
}

TORCH_LIBRARY_IMPL(tvdcn, Autograd, m) {
    TVDCN_IMPL_CONV(1, fwd_ag, bwd_ag)
    TVDCN_IMPL_CONV(2, fwd_ag, bwd_ag)
    TVDCN_IMPL_CONV(3, fwd_ag, bwd_ag)
    m.impl("deform_conv_mask_activation", TORCH_FN(tvdcn_amd::act_fwd_autograd));
    m.impl("_deform_conv_mask_activation_backward", TORCH_FN(tvdcn_amd::act_bwd_autograd));
    m.impl("mask_softmax", TORCH_FN(tvdcn_amd::mask_softmax_autograd));
}

TORCH_LIBRARY_IMPL(tvdcn, Autocast, m) {
    m.impl("deform_conv1d", TORCH_FN(tvdcn_amd::Conv1::fwd_ac_c));
    m.impl("deform_conv2d", TORCH_FN(tvdcn_amd::Conv2::fwd_ac_c));
    m.impl("deform_conv3d", TORCH_FN(tvdcn_amd::Conv3::fwd_ac_c));
    m.impl("deform_conv_transpose1d", TORCH_FN(tvdcn_amd::Tr1::fwd_ac_t));
    m.impl("deform_conv_transpose2d", TORCH_FN(tvdcn_amd::Tr2::fwd_ac_t));
    m.impl("deform_conv_transpose3d", TORCH_FN(tvdcn_amd::Tr3::fwd_ac_t));
    m.impl("deform_conv_mask_activation", TORCH_FN(tvdcn_amd::act_fwd_autocast));
}
