// CPU-key bodies of the tvdcn operators: deform_conv{1,2,3}d, deform_conv_transpose{1,2,3}d
// (forward and backward), the fused mask-activation op and mask_softmax, for host tensors.
//
// The reference registers CPU twins of its CUDA drivers (tvdcn/csrc/ops/cpu/
// deform_conv2d_kernel.cpp:85-645, deform_conv_transpose2d_kernel.cpp and the 1D / 3D files:
// im2col / col2im / coordinate-gradient loops + ATen addmm_ per batch block). This file is its
// own design, shared by all ranks and both directions:
//
//   * one unified view (the one the HIP kernels use): the "sampled" tensor on grid S (conv: the
//     input; transposed: the output), columns on the "column grid" P (conv: the output grid;
//     transposed: the input grid), the weight as W[m][c_local][tap] of shape (M, C/G, Kn); ranks
//     1 and 2 are embedded in rank 3 (unused leading axes of extent 1, which multiply every
//     weight by an exact 1);
//   * per image and chunk of column pixels, a sampling table per (offset group, tap, pixel) --
//     the 2^dim corner indices, bilinear weights and fractional positions -- built once and
//     shared by every channel of the group;
//   * gather (im2col), scatter (col2im) and the offset / mask gradients walk that table with
//     at::parallel_for; the scatter runs one channel per task (a channel only ever writes its
//     own plane of the result, so there are no atomics and the sums are deterministic), the
//     offset / mask gradients one (group, tap) row per task;
//   * the contractions are batched matrix products over the groups (at::bmm / baddbmm_).
//
// Numerics follow the reference's (tvdcn/csrc/ops/cpu/deform_conv2d_common_kernels.cpp:22-135):
// a sample is 0 when its point lies outside (-1, size) on any axis, the scatter and the
// coordinate weights have no such early-out, corners outside the grid are skipped; without
// offsets the sampling is integer (only the low corner, zero padding). float64 runs in float64;
// float32, float16 and bfloat16 run in float32, float16 sampling positions rounded once to half
// precision (the reference forms `y + offset` in c10::Half; the HIP kernels round the same way).
#include "cpu_kernels.h"

#include <ATen/Parallel.h>
#include <c10/util/Half.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

namespace tvdcn_amd {
namespace cpu {
namespace {

using at::Tensor;

// the unified view, ranks embedded in 3 axes (axis 0 = depth, 2 = width)
struct View {
    int dim;
    bool transposed, deformable, modulated, half_pos;
    int64_t B, C, M, G, Cg, Mg, og, mg, Kn, Sn, Pn;
    int64_t S[3], P[3], K[3], st[3], pad[3], dil[3];
};

View make_view(const Operands &op) {
    const tvdcn_conv_desc &d = op.desc;
    View v{};
    v.dim = d.dim;
    v.transposed = d.transposed != 0;
    v.deformable = op.offset.defined();
    v.modulated = op.mask.defined();
    v.half_pos = op.input.scalar_type() == at::kHalf;
    v.B = d.batch;
    v.C = v.transposed ? d.out_channels : d.in_channels;
    v.M = v.transposed ? d.in_channels : d.out_channels;
    v.G = d.groups;
    v.Cg = v.C / v.G;
    v.Mg = v.M / v.G;
    v.og = v.deformable ? d.offset_groups : 1;
    v.mg = v.modulated ? d.mask_groups : 1;
    for (int e = 0; e < 3; ++e) {
        v.S[e] = v.P[e] = v.K[e] = v.st[e] = v.dil[e] = 1;
        v.pad[e] = 0;
    }
    for (int a = 0; a < d.dim; ++a) {
        const int e = 3 - d.dim + a;
        v.S[e] = v.transposed ? op.out_size[a] : d.in_size[a];
        v.P[e] = v.transposed ? d.in_size[a] : op.out_size[a];
        v.K[e] = d.kernel[a];
        v.st[e] = d.stride[a];
        v.pad[e] = d.padding[a];
        v.dil[e] = d.dilation[a];
    }
    v.Kn = v.K[0] * v.K[1] * v.K[2];
    v.Sn = v.S[0] * v.S[1] * v.S[2];
    v.Pn = v.P[0] * v.P[1] * v.P[2];
    return v;
}

// Sampling geometry of one (offset group, tap, column pixel). Corner k selects the high
// corner on axis e when bit (2 - e) of k is set: the last axis varies fastest, the
// reference's corner order.
template <typename A>
struct Sample {
    int64_t idx[8];   // flat index into the sampled grid (valid corners only)
    A w[8];           // bilinear weight, 0 for corners outside the grid
    A fh[3];          // fractional position per axis: the high corner's factor
    uint8_t valid;    // bit k: corner k inside the grid
    bool inside;      // the point lies inside (-1, size) on every axis (sample early-out rule)
};

inline int corner_bit(int k, int e) { return (k >> (2 - e)) & 1; }

// the derivative of corner k's weight along axis d: that axis' factor is -1 (low) / +1 (high)
template <typename A>
inline A corner_dweight(const Sample<A> &s, int k, int d) {
    A r = A(1);
    for (int e = 0; e < 3; ++e) {
        const int hi = corner_bit(k, e);
        const A f = e == d ? (hi ? A(1) : A(-1)) : (hi ? s.fh[e] : A(1) - s.fh[e]);
        r = e == 0 ? f : r * f;
    }
    return r;
}

// table[(ogi * Kn + t) * n + j] for column pixels p0 .. p0 + n of image b (ogi < og when the
// problem is deformable; one group otherwise: integer sampling does not depend on it)
template <typename A>
void build_samples(const View &v, const A *offset, int64_t b, int64_t p0, int64_t n, std::vector<Sample<A>> &tab) {
    const int64_t rows = v.og * v.Kn;
    tab.resize((size_t)(rows * n));
    constexpr double kFar = 1099511627776.0;   // 2^40: positions beyond this are outside every grid
    at::parallel_for(0, rows * n, 256, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i) {
            const int64_t r = i / n, j = i % n, p = p0 + j;
            const int64_t ogi = r / v.Kn, t = r % v.Kn;
            const int64_t pp[3] = {p / (v.P[1] * v.P[2]), (p / v.P[2]) % v.P[1], p % v.P[2]};
            const int64_t kk[3] = {t / (v.K[1] * v.K[2]), (t / v.K[2]) % v.K[1], t % v.K[2]};
            Sample<A> &s = tab[(size_t)i];
            int64_t lo[3];
            bool vlo[3], vhi[3];
            s.inside = true;
            for (int e = 0; e < 3; ++e) {
                const int64_t base = pp[e] * v.st[e] - v.pad[e] + kk[e] * v.dil[e];
                const int64_t n_e = v.S[e];
                const int a = e - (3 - v.dim);
                if (v.deformable && a >= 0) {
                    A pos = static_cast<A>(base) +
                            offset[(((b * v.og + ogi) * v.Kn + t) * v.dim + a) * v.Pn + p];
                    if (v.half_pos) pos = static_cast<A>(static_cast<float>(c10::Half(static_cast<float>(pos))));
                    const A f = std::floor(pos);
                    const bool finite = std::fabs(static_cast<double>(f)) < kFar;
                    lo[e] = finite ? static_cast<int64_t>(f) : -(int64_t)kFar;
                    s.fh[e] = pos - f;
                    s.inside = s.inside && !(pos <= A(-1) || A(n_e) <= pos);
                    vhi[e] = 0 <= lo[e] + 1 && lo[e] + 1 < n_e;
                } else {
                    lo[e] = base;
                    s.fh[e] = A(0);
                    s.inside = s.inside && 0 <= base && base < n_e;
                    vhi[e] = false;
                }
                vlo[e] = 0 <= lo[e] && lo[e] < n_e;
            }
            s.valid = 0;
            for (int k = 0; k < 8; ++k) {
                bool ok = true;
                int64_t flat = 0;
                A wk = A(1);
                for (int e = 0; e < 3; ++e) {
                    const int hi = corner_bit(k, e);
                    ok = ok && (hi ? vhi[e] : vlo[e]);
                    flat = flat * v.S[e] + lo[e] + hi;
                    const A f = hi ? s.fh[e] : A(1) - s.fh[e];
                    wk = e == 0 ? f : wk * f;
                }
                s.idx[k] = ok ? flat : 0;
                s.w[k] = ok ? wk : A(0);
                if (ok) s.valid |= (uint8_t)(1u << k);
            }
        }
    });
}

// sampled value of one channel plane x at s (0 outside, the early-out rule)
template <typename A>
inline A sample_value(const Sample<A> &s, const A *x) {
    A val = A(0);
    if (!s.inside) return val;
    for (int k = 0; k < 8; ++k)
        if (s.valid & (1u << k)) val += s.w[k] * x[s.idx[k]];
    return val;
}

struct Chunk {
    int64_t b, p0, n;
};

// cols[c * Kn + t][j] = mask * sample(x[c], point(og(c), t, p0 + j))       (im2col)
template <typename A>
void gather(const View &v, const std::vector<Sample<A>> &tab, const Chunk &ch, const A *x_b, const A *m_b,
            A *cols) {
    const int64_t cpo = v.C / v.og, cpm = v.C / v.mg, n = ch.n;
    at::parallel_for(0, v.C * v.Kn, 1, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t c = r / v.Kn, t = r % v.Kn;
            const Sample<A> *s = tab.data() + ((c / cpo) * v.Kn + t) * n;
            const A *x = x_b + c * v.Sn;
            const A *m = m_b ? m_b + ((c / cpm) * v.Kn + t) * v.Pn + ch.p0 : nullptr;
            A *out = cols + r * n;
            for (int64_t j = 0; j < n; ++j) {
                const A val = sample_value(s[j], x);
                out[j] = m ? val * m[j] : val;
            }
        }
    });
}

// y[c][corner] += weight * mask * cols[c * Kn + t][j]                        (col2im)
template <typename A>
void scatter(const View &v, const std::vector<Sample<A>> &tab, const Chunk &ch, const A *cols, const A *m_b,
             A *y_b) {
    const int64_t cpo = v.C / v.og, cpm = v.C / v.mg, n = ch.n;
    at::parallel_for(0, v.C, 1, [&](int64_t c0, int64_t c1) {
        for (int64_t c = c0; c < c1; ++c) {
            A *y = y_b + c * v.Sn;
            for (int64_t t = 0; t < v.Kn; ++t) {
                const Sample<A> *s = tab.data() + ((c / cpo) * v.Kn + t) * n;
                const A *m = m_b ? m_b + ((c / cpm) * v.Kn + t) * v.Pn + ch.p0 : nullptr;
                const A *col = cols + (c * v.Kn + t) * n;
                for (int64_t j = 0; j < n; ++j) {
                    const A val = m ? m[j] * col[j] : col[j];
                    const Sample<A> &sj = s[j];
                    for (int k = 0; k < 8; ++k)
                        if (sj.valid & (1u << k)) y[sj.idx[k]] += sj.w[k] * val;
                }
            }
        }
    });
}

// grad_offset[b][ogi][t][a][p] = sum_{c in ogi} mask * cols * sum_k dweight_a(k) * x[c][corner k]
// grad_mask[b][mgi][t][p]      = sum_{c in mgi} cols * sample(x[c])                 (col2im_coord)
template <typename A>
void coordinate_grads(const View &v, const std::vector<Sample<A>> &tab, const Chunk &ch, const A *cols,
                      const A *x_b, const A *m_b, A *goff_b, A *gmask_b) {
    const int64_t cpo = v.C / v.og, cpm = v.C / v.mg, n = ch.n;
    if (goff_b != nullptr) {
        at::parallel_for(0, v.og * v.Kn, 1, [&](int64_t r0, int64_t r1) {
            for (int64_t r = r0; r < r1; ++r) {
                const int64_t ogi = r / v.Kn, t = r % v.Kn;
                const Sample<A> *s = tab.data() + r * n;
                for (int64_t j = 0; j < n; ++j) {
                    const Sample<A> &sj = s[j];
                    A dw[8][3];
                    for (int k = 0; k < 8; ++k)
                        for (int a = 0; a < v.dim; ++a) dw[k][a] = corner_dweight(sj, k, 3 - v.dim + a);
                    A acc[3] = {A(0), A(0), A(0)};
                    for (int64_t c = ogi * cpo; c < (ogi + 1) * cpo; ++c) {
                        A gm = cols[(c * v.Kn + t) * n + j];
                        if (m_b) gm *= m_b[((c / cpm) * v.Kn + t) * v.Pn + ch.p0 + j];
                        const A *x = x_b + c * v.Sn;
                        for (int k = 0; k < 8; ++k) {
                            if (!(sj.valid & (1u << k))) continue;
                            const A xv = x[sj.idx[k]] * gm;
                            for (int a = 0; a < v.dim; ++a) acc[a] += dw[k][a] * xv;
                        }
                    }
                    for (int a = 0; a < v.dim; ++a) goff_b[((ogi * v.Kn + t) * v.dim + a) * v.Pn + ch.p0 + j] = acc[a];
                }
            }
        });
    }
    if (gmask_b != nullptr) {
        at::parallel_for(0, v.mg * v.Kn, 1, [&](int64_t r0, int64_t r1) {
            for (int64_t r = r0; r < r1; ++r) {
                const int64_t mgi = r / v.Kn, t = r % v.Kn;
                for (int64_t j = 0; j < n; ++j) {
                    A acc = A(0);
                    for (int64_t c = mgi * cpm; c < (mgi + 1) * cpm; ++c) {
                        const Sample<A> &sj = tab[(size_t)(((c / cpo) * v.Kn + t) * n + j)];
                        acc += cols[(c * v.Kn + t) * n + j] * sample_value(sj, x_b + c * v.Sn);
                    }
                    gmask_b[(mgi * v.Kn + t) * v.Pn + ch.p0 + j] = acc;
                }
            }
        });
    }
}

// column pixels per chunk: the sampling table and the columns stay bounded
int64_t chunk_pixels(const View &v) {
    const int64_t by_table = (int64_t(1) << 17) / std::max<int64_t>(1, v.og * v.Kn);
    const int64_t by_cols = (int64_t(1) << 24) / std::max<int64_t>(1, v.C * v.Kn);
    return std::max<int64_t>(1, std::min({v.Pn, by_table, by_cols}));
}

at::ScalarType acc_type(at::ScalarType t) { return t == at::kDouble ? at::kDouble : at::kFloat; }

Tensor to_acc(const Tensor &t, at::ScalarType a) { return t.defined() ? t.to(a).contiguous() : t; }

// the mask the kernels use: the tensor, or its activation when it holds logits
// (mask_scale * sigmoid, tvdcn/ops/activations/mask_sigmoid.py:11-21; softmax over the taps of
// each mask group, mask_softmax.py:19-49)
Tensor activated_mask(const View &v, const tvdcn_conv_desc &d, const Tensor &m) {
    if (!m.defined()) return m;
    if (d.flags & TVDCN_FLAG_MASK_SIGMOID) return at::sigmoid(m) * d.mask_scale;
    if (d.flags & TVDCN_FLAG_MASK_SOFTMAX)
        return at::softmax(m.view({v.B, v.mg, v.Kn, v.Pn}), 2).view(m.sizes()).contiguous();
    return m;
}

// gradient of the logits from the gradient of the activated mask ma
Tensor logit_grad(const View &v, const tvdcn_conv_desc &d, const Tensor &gm, const Tensor &ma) {
    if (d.flags & TVDCN_FLAG_MASK_SIGMOID) return gm * ma * (1.0 - ma / d.mask_scale);
    if (d.flags & TVDCN_FLAG_MASK_SOFTMAX) {
        const auto sz = std::vector<int64_t>{v.B, v.mg, v.Kn, v.Pn};
        const Tensor g4 = gm.view(sz), y4 = ma.view(sz);
        return (y4 * (g4 - (g4 * y4).sum(2, true))).view(gm.sizes());
    }
    return gm;
}

template <typename A>
A *ptr(const Tensor &t) {
    return t.defined() ? t.data_ptr<A>() : nullptr;
}

template <typename A>
Tensor forward_impl(const View &v, const Operands &op, at::ScalarType acc) {
    const Tensor x = to_acc(op.input, acc), w = to_acc(op.weight, acc), off = to_acc(op.offset, acc),
                 bias = to_acc(op.bias, acc);
    const Tensor msk = activated_mask(v, op.desc, to_acc(op.mask, acc));
    std::vector<int64_t> out_shape = {v.B, op.desc.out_channels};
    out_shape.insert(out_shape.end(), op.out_size.begin(), op.out_size.end());
    // conv: the output is the GEMM side on the column grid; transposed: the sampled side
    Tensor out = v.transposed ? at::zeros(out_shape, x.options()) : at::empty(out_shape, x.options());
    const Tensor wg = w.view({v.G, v.Mg, v.Cg * v.Kn});
    const int64_t np = chunk_pixels(v);
    std::vector<Sample<A>> tab;
    for (int64_t b = 0; b < v.B; ++b) {
        const A *m_b = v.modulated ? ptr<A>(msk) + b * v.mg * v.Kn * v.Pn : nullptr;
        for (int64_t p0 = 0; p0 < v.Pn; p0 += np) {
            const Chunk ch{b, p0, std::min(np, v.Pn - p0)};
            build_samples<A>(v, ptr<A>(off), b, p0, ch.n, tab);
            if (!v.transposed) {
                Tensor cols = at::empty({v.G, v.Cg * v.Kn, ch.n}, x.options());
                gather<A>(v, tab, ch, ptr<A>(x) + b * v.C * v.Sn, m_b, ptr<A>(cols));
                out[b].view({v.M, v.Pn}).narrow(1, p0, ch.n).copy_(at::bmm(wg, cols).view({v.M, ch.n}));
            } else {
                const Tensor xg = x[b].view({v.G, v.Mg, v.Pn}).narrow(2, p0, ch.n);
                const Tensor cols = at::bmm(wg.transpose(1, 2), xg).contiguous();
                scatter<A>(v, tab, ch, ptr<A>(cols), m_b, ptr<A>(out) + b * v.C * v.Sn);
            }
        }
    }
    if (bias.defined()) {
        std::vector<int64_t> bshape(out.dim(), 1);
        bshape[1] = bias.numel();
        out += bias.view(bshape);
    }
    return out.to(op.input.scalar_type());
}

template <typename A>
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward_impl(const View &v, const Operands &op,
                                                                 const Tensor &grad_, at::ScalarType acc) {
    const Tensor x = to_acc(op.input, acc), w = to_acc(op.weight, acc), off = to_acc(op.offset, acc);
    const Tensor msk = activated_mask(v, op.desc, to_acc(op.mask, acc));
    const Tensor grad = to_acc(grad_, acc);
    // conv: grad_input is scattered (zeros first); transposed: written per chunk by a GEMM
    Tensor gi = at::zeros(x.sizes(), x.options());
    Tensor gw = at::zeros(w.sizes(), w.options());
    Tensor goff = v.deformable ? at::zeros(off.sizes(), off.options()) : Tensor();
    Tensor gmask = v.modulated ? at::zeros(msk.sizes(), msk.options()) : Tensor();
    const Tensor wg = w.view({v.G, v.Mg, v.Cg * v.Kn});
    Tensor gwg = gw.view({v.G, v.Mg, v.Cg * v.Kn});
    const int64_t np = chunk_pixels(v);
    std::vector<Sample<A>> tab;
    for (int64_t b = 0; b < v.B; ++b) {
        const A *m_b = v.modulated ? ptr<A>(msk) + b * v.mg * v.Kn * v.Pn : nullptr;
        A *goff_b = v.deformable ? ptr<A>(goff) + b * v.og * v.Kn * v.dim * v.Pn : nullptr;
        A *gmask_b = v.modulated ? ptr<A>(gmask) + b * v.mg * v.Kn * v.Pn : nullptr;
        for (int64_t p0 = 0; p0 < v.Pn; p0 += np) {
            const Chunk ch{b, p0, std::min(np, v.Pn - p0)};
            build_samples<A>(v, ptr<A>(off), b, p0, ch.n, tab);
            if (!v.transposed) {
                // Z = grad_out on the column grid; X = input on the sampled grid
                const A *x_b = ptr<A>(x) + b * v.C * v.Sn;
                const Tensor zg = grad[b].view({v.G, v.Mg, v.Pn}).narrow(2, p0, ch.n);
                const Tensor gcols = at::bmm(wg.transpose(1, 2), zg).contiguous();
                scatter<A>(v, tab, ch, ptr<A>(gcols), m_b, ptr<A>(gi) + b * v.C * v.Sn);
                coordinate_grads<A>(v, tab, ch, ptr<A>(gcols), x_b, m_b, goff_b, gmask_b);
                Tensor cols = at::empty({v.G, v.Cg * v.Kn, ch.n}, x.options());
                gather<A>(v, tab, ch, x_b, m_b, ptr<A>(cols));
                gwg.baddbmm_(zg, cols.transpose(1, 2));
            } else {
                // Z = grad_out on the sampled grid; X = input (GEMM side) on the column grid
                const A *z_b = ptr<A>(grad) + b * v.C * v.Sn;
                const Tensor xg = x[b].view({v.G, v.Mg, v.Pn}).narrow(2, p0, ch.n);
                Tensor gcols = at::empty({v.G, v.Cg * v.Kn, ch.n}, x.options());
                gather<A>(v, tab, ch, z_b, m_b, ptr<A>(gcols));
                gi[b].view({v.M, v.Pn}).narrow(1, p0, ch.n).copy_(at::bmm(wg, gcols).view({v.M, ch.n}));
                gwg.baddbmm_(xg, gcols.transpose(1, 2));
                const Tensor cols = at::bmm(wg.transpose(1, 2), xg).contiguous();
                coordinate_grads<A>(v, tab, ch, ptr<A>(cols), z_b, m_b, goff_b, gmask_b);
            }
        }
    }
    const auto dt = op.input.scalar_type();
    Tensor gb;
    if (op.bias.defined()) {
        std::vector<int64_t> dims = {0};
        for (int64_t i = 2; i < grad.dim(); ++i) dims.push_back(i);
        gb = grad.sum(dims).to(dt);
    }
    if (gmask.defined()) gmask = logit_grad(v, op.desc, gmask, msk);
    auto back = [&](const Tensor &t) { return t.defined() ? t.to(dt) : t; };
    return {back(gi), back(gw), back(goff), back(gmask), gb};
}

}  // namespace

Tensor forward(const Operands &op) {
    const View v = make_view(op);
    const auto acc = acc_type(op.input.scalar_type());
    if (acc == at::kDouble) return forward_impl<double>(v, op, acc);
    return forward_impl<float>(v, op, acc);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> backward(const Operands &op, const Tensor &grad) {
    const View v = make_view(op);
    const auto acc = acc_type(op.input.scalar_type());
    if (acc == at::kDouble) return backward_impl<double>(v, op, grad, acc);
    return backward_impl<float>(v, op, grad, acc);
}

Tensor mask_softmax(const Tensor &x, int64_t B, int64_t G, int64_t K, int64_t S) {
    return at::softmax(x.contiguous().view({B, G, K, S}), 2).view(x.sizes()).contiguous();
}

Tensor mask_softmax_backward(const Tensor &grad, const Tensor &y, int64_t B, int64_t G, int64_t K, int64_t S) {
    const Tensor g4 = grad.contiguous().view({B, G, K, S}), y4 = y.contiguous().view({B, G, K, S});
    return at::_softmax_backward_data(g4, y4, 2, y.scalar_type()).view(y.sizes()).contiguous();
}

}  // namespace cpu
}  // namespace tvdcn_amd
