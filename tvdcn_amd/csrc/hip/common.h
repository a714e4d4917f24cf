// Shared device-side definitions for the gfx950 deformable-convolution kernels.
//
// Three kernel families implement every op (conv and transposed, rank 1/2/3):
//   F  gather-GEMM   Y[b][m][p]   = sum_{c,t} W[m][c][t] * S[c][t][b][p]
//   D  data-grad     G[c][t][b][p] = sum_m W[m][c][t] * Z[b][m][p], then scatter G*mask
//                    into the sampled tensor's gradient and/or reduce the offset/mask grads
//   Wt weight-grad   dW[m][c][t]  = sum_{b,p} Z[b][m][p] * S[c][t][b][p]
// where S is the bilinear sample (times mask) of the "sampled" tensor X at the
// deformed tap positions. Conv: X = input, Z = grad_out, M = Cout, C = Cin.
// Transposed: X = output side (grad_out in backward), Z = input, M = Cin, C = Cout.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <type_traits>

namespace tvdcn_hip {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// Division by a run-time-invariant positive divisor with one multiply-high, an add
// and a shift (Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994): s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1,
// q = (mulhi(n, m) + n) >> s, exact for 0 <= n < 2^31 (the sum cannot overflow).
struct FastDiv {
    uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
    return FastDiv{d, (uint32_t)m, s};
}

__device__ __forceinline__ int fdiv(const FastDiv &f, int n) {
    const uint32_t t = __umulhi((uint32_t)n, f.m);
    return (int)((t + (uint32_t)n) >> f.s);
}

// Problem geometry, passed by value to every kernel. Spatial shapes are embedded
// in rank 3 (unused leading axes have extent 1, stride 1, padding 0).
struct Geo {
    int B;
    int C, M, G, Cg, Mg;   // sampled-side channels, GEMM-side channels, groups
    int og, mg;            // offset / mask groups (0 = absent)
    int cpo, cpm;          // channels per offset / mask group
    int S[3];              // sampled grid (conv: input; transposed: output)
    int P[3];              // column grid (conv: output; transposed: input)
    int K[3], st[3], pad[3], dil[3];
    int Sn, Pn, Kn;
    int NP;                // B * Pn
    FastDiv dPn, dP2, dP12, dK2, dK12;   // divisors Pn, P[2], P[1]*P[2], K[2], K[1]*K[2]
    // mask_act: 0 = the mask tensor holds the mask values; otherwise it holds logits, activated in the
    // kernels' mask load: MASK_ACT_SIGMOID = mask_scale * sigmoid(logit), MASK_ACT_SOFTMAX = softmax
    // over the Kn taps of the logit's (batch, mask group, column pixel)
    int mask_act = 0;
    double mask_scale = 0.0;
};
constexpr int MASK_ACT_SIGMOID = 1;
constexpr int MASK_ACT_SOFTMAX = 2;

// ---------------------------------------------------------------------------
// scalar conversion
// ---------------------------------------------------------------------------
template <typename A, typename T> __device__ __forceinline__ A to_acc(T v) { return static_cast<A>(v); }
template <> __device__ __forceinline__ float to_acc<float, __half>(__half v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_acc<float, __hip_bfloat16>(__hip_bfloat16 v) {
    return __bfloat162float(v);
}
template <typename T, typename A> __device__ __forceinline__ T from_acc(A v) { return static_cast<T>(v); }
template <> __device__ __forceinline__ __half from_acc<__half, float>(float v) { return __float2half(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_acc<__hip_bfloat16, float>(float v) {
    return __float2bfloat16(v);
}

// four consecutive accumulator-typed values (16 B for float, 32 B for double)
template <typename A> struct Vec4 { A x, y, z, w; };

template <typename A>
__device__ __forceinline__ Vec4<A> load4(const A *p) {
    if constexpr (sizeof(A) == 4) {
        const float4 v = *reinterpret_cast<const float4 *>(p);
        return {v.x, v.y, v.z, v.w};
    } else {
        const double2 a = *reinterpret_cast<const double2 *>(p);
        const double2 b = *reinterpret_cast<const double2 *>(p + 2);
        return {a.x, a.y, b.x, b.y};
    }
}

template <typename A>
__device__ __forceinline__ void store4(A *p, Vec4<A> v) {
    if constexpr (sizeof(A) == 4) {
        *reinterpret_cast<float4 *>(p) = make_float4(v.x, v.y, v.z, v.w);
    } else {
        *reinterpret_cast<double2 *>(p) = make_double2(v.x, v.y);
        *reinterpret_cast<double2 *>(p + 2) = make_double2(v.z, v.w);
    }
}

// four consecutive storage-typed values converted to the accumulator type, with
// one vector load (16 B fp32, 2 x 16 B fp64, 8 B fp16/bf16); p must be aligned
// to 4 elements
template <typename A, typename T>
__device__ __forceinline__ Vec4<A> load4_t(const T *p) {
    if constexpr (sizeof(T) == sizeof(A)) {
        return load4<A>(reinterpret_cast<const A *>(p));
    } else {
        const uint2 u = *reinterpret_cast<const uint2 *>(p);
        const T *h = reinterpret_cast<const T *>(&u);
        return {to_acc<A>(h[0]), to_acc<A>(h[1]), to_acc<A>(h[2]), to_acc<A>(h[3])};
    }
}

// ---------------------------------------------------------------------------
// MFMA 16x16x4 (fp32 and fp64). Operand layout, lane l of 64:
//   A[i][k]: i = l % 16, k = l / 16      B[k][j]: j = l % 16, k = l / 16
//   D[i][j]: 4 values per lane v = 0..3, j = l % 16 and
//            fp32: i = 4 * (l / 16) + v        fp64: i = l / 16 + 4 * v
// (both measured on gfx950 with one-hot operands)
// ---------------------------------------------------------------------------
template <typename A> struct Acc4;
template <> struct Acc4<float> { typedef f32x4 type; };
template <> struct Acc4<double> { typedef f64x4 type; };

// row of the 16x16 output block held by lane `lane` in accumulator slot v
template <typename A>
__device__ __forceinline__ int mfma_row(int lane, int v) {
    if constexpr (sizeof(A) == 8)
        return (lane >> 4) + 4 * v;
    else
        return 4 * (lane >> 4) + v;
}

__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f64x4 mfma16x16x4(double a, double b, f64x4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// atomics: hardware float/double add (global_atomic_add_f32 / _f64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void atomic_add(float *p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(double *p, double v) { unsafeAtomicAdd(p, v); }

// ---------------------------------------------------------------------------
// workgroup -> tile mapping that keeps consecutive tiles on one XCD. The
// hardware deals workgroups round-robin to the 8 XCDs (each with its own L2);
// this inverts that so XCD x processes the contiguous tile range
// [base_x, base_x + count_x), keeping neighbouring pixel tiles (which share
// input rows) in the same L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int xcd_remap(int L, int N) {
    constexpr int NX = 8;
    const int q = N / NX, r = N % NX;
    const int xcd = L % NX, k = L / NX;
    const int base = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
    return base + k;
}

// ---------------------------------------------------------------------------
// Sampling geometry of one (column pixel, tap, offset group).
// Restates the reference's per-rank helpers (tvdcn/csrc/ops/cuda/
// deform_conv2d_common_kernels.cu:25-135 and the 1D/3D twins):
//   * sample value: 0 if the point is outside (-1, size) on any axis,
//     else the sum over the in-range corners of (product of axis weights) * x;
//   * scatter (insert) and coordinate weights: no early-out, each corner
//     range-checked on both sides.
// Corner order is the reference's: low/high on the last axis fastest.
// ---------------------------------------------------------------------------
template <int DIM> struct Corners {
    static constexpr int N = 1 << DIM;
    int idx[N];          // flat spatial index into the sampled grid (0 when invalid)
    bool valid[N];       // corner inside the grid
    float frac[3];       // fractional position on each embedded axis used (lo weight = 1-frac)
    bool inside;         // point inside (-1, size) on every axis (sample early-out rule)
};

// Axis a of the DIM used axes corresponds to embedded axis 3-DIM+a.
template <int DIM, typename A>
struct Point {
    A pos[DIM];
    int base[DIM];
};

template <int DIM>
__device__ __forceinline__ void decompose_tap(const Geo &g, int t, int kk[DIM]) {
    if constexpr (DIM == 1) {
        kk[0] = t;
    } else if constexpr (DIM == 2) {
        kk[0] = fdiv(g.dK2, t);
        kk[1] = t - kk[0] * g.K[2];
    } else {
        kk[0] = fdiv(g.dK12, t);
        const int r = t - kk[0] * g.K[1] * g.K[2];
        kk[1] = fdiv(g.dK2, r);
        kk[2] = r - kk[1] * g.K[2];
    }
}

template <int DIM>
__device__ __forceinline__ void decompose_pix(const Geo &g, int p, int pp[DIM]) {
    if constexpr (DIM == 1) {
        pp[0] = p;
    } else if constexpr (DIM == 2) {
        pp[0] = fdiv(g.dP2, p);
        pp[1] = p - pp[0] * g.P[2];
    } else {
        pp[0] = fdiv(g.dP12, p);
        const int r = p - pp[0] * g.P[1] * g.P[2];
        pp[1] = fdiv(g.dP2, r);
        pp[2] = r - pp[1] * g.P[2];
    }
}

// A sample position in the arithmetic of the input's type, as the reference's kernels form
// `y + offset` in scalar_t (tvdcn/csrc/ops/cuda/deform_conv2d_common_kernels.cu:170-178): an exact
// float sum of the integer base and the offset, rounded once to the type -- float32 by the float
// addition itself, float16 to half precision (c10::Half arithmetic), float64 exact. bfloat16 has no
// reference path (its dispatch excludes the type): its positions stay float32.
template <typename T, typename A>
__device__ __forceinline__ A round_position(A v) {
    if constexpr (std::is_same_v<T, __half>)
        return static_cast<A>(__half2float(__float2half(static_cast<float>(v))));
    else
        return v;
}

// Integer base point h*stride - pad + i*dilation per axis
// (deform_conv2d_common_kernels.cu:171-172) plus the offsets of group ogi
// (offset channel ((ogi*Kn + t)*DIM + axis), deform_conv2d_kernel.cpp:278-286).
template <int DIM, typename A, typename T>
__device__ __forceinline__ Point<DIM, A> sample_point(const Geo &g, const T *__restrict__ offset, int b, int p,
                                                      int t, int ogi) {
    int kk[DIM], pp[DIM];
    decompose_tap<DIM>(g, t, kk);
    decompose_pix<DIM>(g, p, pp);
    Point<DIM, A> pt;
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        const int e = 3 - DIM + a;
        pt.base[a] = pp[a] * g.st[e] - g.pad[e] + kk[a] * g.dil[e];
        pt.pos[a] = static_cast<A>(pt.base[a]);
    }
    if (offset != nullptr) {
        const T *o = offset + ((size_t)(b * g.og + ogi) * g.Kn + t) * DIM * (size_t)g.Pn + p;
#pragma unroll
        for (int a = 0; a < DIM; ++a) pt.pos[a] = round_position<T, A>(pt.pos[a] + to_acc<A>(o[(size_t)a * g.Pn]));
    }
    return pt;
}

// Per-axis decomposition of a (possibly fractional) point.
template <int DIM, typename A>
struct AxisW {
    int lo[DIM];
    A fh[DIM];           // high-corner weight = pos - floor(pos); low = 1 - fh
    bool vlo[DIM], vhi[DIM];
    bool inside;         // sample early-out rule
};

template <int DIM, typename A>
__device__ __forceinline__ AxisW<DIM, A> axis_weights(const Geo &g, const Point<DIM, A> &pt, bool deformable) {
    AxisW<DIM, A> w;
    w.inside = true;
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        const int n = g.S[3 - DIM + a];
        if (deformable) {
            const A f = floor(pt.pos[a]);
            w.lo[a] = static_cast<int>(f);
            w.fh[a] = pt.pos[a] - f;
            w.inside = w.inside && !(pt.pos[a] <= A(-1) || A(n) <= pt.pos[a]);
        } else {
            // integer sampling (offset is None): only the low corner exists
            // (deform_conv2d_common_kernels.cu:13-22 `sample` / `insert`)
            w.lo[a] = pt.base[a];
            w.fh[a] = A(0);
            w.inside = w.inside && (0 <= pt.base[a] && pt.base[a] < n);
        }
        w.vlo[a] = 0 <= w.lo[a] && w.lo[a] < n;
        w.vhi[a] = deformable && 0 <= w.lo[a] + 1 && w.lo[a] + 1 < n;
    }
    return w;
}

// Corner i (bit a of i, counted from the last axis, selects high on axis a).
template <int DIM>
__device__ __forceinline__ int corner_bit(int i, int a) {
    return (i >> (DIM - 1 - a)) & 1;
}

// flat index and validity of corner i
template <int DIM, typename A>
__device__ __forceinline__ void corner_at(const Geo &g, const AxisW<DIM, A> &w, int i, int &idx, bool &valid) {
    int flat = 0;
    valid = true;
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        const int hi = corner_bit<DIM>(i, a);
        const int coord = w.lo[a] + hi;
        valid = valid && (hi ? w.vhi[a] : w.vlo[a]);
        flat = flat * g.S[3 - DIM + a] + coord;
    }
    idx = valid ? flat : 0;
}

// bilinear product weight of corner i: prod over axes of (hi ? fh : 1 - fh), in the
// reference's multiplication order (outer axis first).
template <int DIM, typename A>
__device__ __forceinline__ A corner_weight(const AxisW<DIM, A> &w, int i) {
    A r = A(1);
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        const A f = corner_bit<DIM>(i, a) ? w.fh[a] : A(1) - w.fh[a];
        r = (a == 0) ? f : r * f;
    }
    return r;
}

// coordinate weight of corner i for derivative axis d: axis d's factor is -1/+1
// (deform_conv2d_common_kernels.cu:105-135).
template <int DIM, typename A>
__device__ __forceinline__ A corner_dweight(const AxisW<DIM, A> &w, int i, int d) {
    A r = A(1);
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        const int hi = corner_bit<DIM>(i, a);
        const A f = (a == d) ? (hi ? A(1) : A(-1)) : (hi ? w.fh[a] : A(1) - w.fh[a]);
        r = (a == 0) ? f : r * f;
    }
    return r;
}

// Gather-side corner set for the fast paths: flat indices (0 when invalid) and
// sample weights (0 when invalid or when the sample early-out applies).
template <int DIM, typename A>
struct GatherCorners {
    int idx[1 << DIM];
    A w[1 << DIM];
};

template <int DIM, typename A>
__device__ __forceinline__ GatherCorners<DIM, A> gather_corners(const Geo &g, const AxisW<DIM, A> &aw) {
    GatherCorners<DIM, A> gc;
#pragma unroll
    for (int i = 0; i < (1 << DIM); ++i) {
        bool v;
        corner_at<DIM, A>(g, aw, i, gc.idx[i], v);
        gc.w[i] = (v && aw.inside) ? corner_weight<DIM, A>(aw, i) : A(0);
    }
    return gc;
}

// Mask value of (b, mask group, tap, column pixel): the tensor's value, or its activation
// when the mask holds logits (tvdcn/ops/activations/mask_sigmoid.py:11-21 and
// mask_softmax.py:19-126 applied in the load instead of as separate passes)
// (mask_raw: the stored value, 1 without a mask; mask_activate: the sigmoid of a logit —
// split so that batched loads are all issued before any value is used; the softmax needs
// every tap's logit of the pixel: mask_softmax_norm gives its max and 1 / sum)
template <typename A, typename T>
__device__ __forceinline__ A mask_raw(const Geo &g, const T *__restrict__ mask, int b, int mgi, int t, int p) {
    if (mask == nullptr) return A(1);
    return to_acc<A>(mask[((size_t)(b * g.mg + mgi) * g.Kn + t) * (size_t)g.Pn + p]);
}
template <typename A>
__device__ __forceinline__ A mask_activate(const Geo &g, A v) {
    if (g.mask_act == MASK_ACT_SIGMOID) {   // uniform
        // fp32: hardware exp2 and reciprocal (a few instructions, ~2 ulp), so that the rarely
        // taken branch adds little code to the kernels' hot loops
        if constexpr (std::is_same_v<A, float>)
            return (float)g.mask_scale * __builtin_amdgcn_rcpf(1.f + __expf(-v));
        else
            return (A)g.mask_scale / (A(1) + exp(-v));
    }
    return v;
}
// max over the Kn taps of the logits of (b, mask group, pixel), and 1 / sum_t exp(logit_t - max)
template <typename A, typename T>
__device__ __forceinline__ void mask_softmax_norm(const Geo &g, const T *__restrict__ mask, int b, int mgi, int p,
                                                  A &mx, A &inv_sum) {
    const T *ml = mask + (size_t)(b * g.mg + mgi) * g.Kn * (size_t)g.Pn + p;
    mx = -INFINITY;
    for (int t = 0; t < g.Kn; ++t) {
        const A v = to_acc<A>(ml[(size_t)t * g.Pn]);
        mx = v > mx ? v : mx;
    }
    A sum = A(0);
    for (int t = 0; t < g.Kn; ++t) sum += exp(to_acc<A>(ml[(size_t)t * g.Pn]) - mx);
    inv_sum = A(1) / sum;
}
template <typename A, typename T>
__device__ __forceinline__ A mask_at(const Geo &g, const T *__restrict__ mask, int b, int mgi, int t, int p) {
    if (mask != nullptr && g.mask_act == MASK_ACT_SOFTMAX) {
        A mx, inv;
        mask_softmax_norm<A, T>(g, mask, b, mgi, p, mx, inv);
        return exp(mask_raw<A, T>(g, mask, b, mgi, t, p) - mx) * inv;
    }
    return mask_activate<A>(g, mask_raw<A, T>(g, mask, b, mgi, t, p));
}


}  // namespace tvdcn_hip
