// Family Wt: weight gradient as an implicit GEMM over re-gathered columns.
//
//   dW[m][c][t] += sum_{(b,p) in split} Z[b][m][p] * mask * bilinear(X[b][c], pos(b, og(c), t, p))
//
// Replaces the reference's im2col recompute + grad_weight addmm_
// (tvdcn/csrc/ops/cuda/deform_conv2d_kernel.cpp:600-626; transposed
// deform_conv_transpose2d_kernel.cpp:586-613). The reduction runs over all
// column pixels, split across workgroups (split-K); each workgroup adds its
// partial tile to dW with one hardware float atomic per element.
//
// Tile: (64 * WAVES) GEMM-side rows x 64 channels of one tap; K stepped 16
// pixels at a time. A (= Z, pixels contiguous) is read straight from global,
// 4 consecutive pixels per lane; B (sampled values) is gathered cooperatively
// (16 lanes x 16 B = one pixel's 64 channels, coalesced) into a double-buffered
// LDS tile [16 pixels][64 + 4] and read with 4-byte LDS loads.
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int BKP = 16;        // pixels per step
constexpr int BC = 64;         // channels per tile
constexpr int LDB = BC + 4;

template <int DIM, typename T, typename A, int WAVES, bool VEC4>
__global__ void __launch_bounds__(64 * WAVES)
bwd_weight_kernel(const Geo g, const T *__restrict__ z, const A *__restrict__ xcl, const T *__restrict__ offset,
                  const T *__restrict__ mask, A *__restrict__ gw, const int k_chunk, const int m_tiles,
                  const int c_tiles, const int k_splits, const bool z_vec) {
    constexpr int NT = 64 * WAVES;
    constexpr int SLOTS = (BKP * BC / 4) / NT;   // (pixel, quad) slots per thread
    constexpr int NC = 1 << DIM;
    typedef typename Acc4<A>::type acc4;

    __shared__ A sB[2][BKP * LDB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int mt = L % m_tiles;
    const int ct = (L / m_tiles) % c_tiles;
    const int t = (L / (m_tiles * c_tiles)) % g.Kn;
    const int ks = (L / (m_tiles * c_tiles * g.Kn)) % k_splits;
    const int grp = L / (m_tiles * c_tiles * g.Kn * k_splits);
    const int c0 = ct * BC;
    const int mrow0 = mt * 64 * WAVES + wave * 64;
    const int kbeg = ks * k_chunk;
    const int kend = min(g.NP, kbeg + k_chunk);
    const bool deformable = offset != nullptr;

    // gather slots: pixel (tid / 16) + i * (NT / 16), channel quad tid % 16
    const int q = tid & 15;
    const int cl = c0 + 4 * q;
    const int c = grp * g.Cg + cl;
    const bool cvalid = cl < g.Cg;

    auto gather_step = [&](int k0, int buf) {
        A *dst = sB[buf];
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            const int nl = (tid >> 4) + i * (NT / 16);
            const int n = k0 + nl;
            const bool ok = n < kend;
            const int b = ok ? n / g.Pn : 0;
            const int p = ok ? n - b * g.Pn : 0;
            A vals[4] = {A(0), A(0), A(0), A(0)};
            if constexpr (VEC4) {
                if (ok && cvalid) {
                    const int ogi = g.og ? c / g.cpo : 0;
                    const int mgi = g.mg ? c / g.cpm : 0;
                    const GatherCorners<DIM, A> gc = gather_corners<DIM, A>(
                        g, axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, ogi), deformable));
                    const A *base = xcl + (size_t)b * g.Sn * g.C + c;
                    Vec4<A> raw[NC];
#pragma unroll
                    for (int k = 0; k < NC; ++k) raw[k] = load4<A>(base + (size_t)gc.idx[k] * g.C);
#pragma unroll
                    for (int k = 0; k < NC; ++k) {
                        vals[0] += gc.w[k] * raw[k].x;
                        vals[1] += gc.w[k] * raw[k].y;
                        vals[2] += gc.w[k] * raw[k].z;
                        vals[3] += gc.w[k] * raw[k].w;
                    }
                    const A mk = mask_at<A, T>(g, mask, b, mgi, t, p);
#pragma unroll
                    for (int j = 0; j < 4; ++j) vals[j] *= mk;
                }
            } else {
                if (ok) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (cl + j >= g.Cg) continue;
                        const int cj = c + j;
                        const int ogi = g.og ? cj / g.cpo : 0;
                        const int mgi = g.mg ? cj / g.cpm : 0;
                        const GatherCorners<DIM, A> gc = gather_corners<DIM, A>(
                            g, axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, ogi), deformable));
                        const A *base = xcl + (size_t)b * g.Sn * g.C + cj;
                        A v = A(0);
#pragma unroll
                        for (int k = 0; k < NC; ++k) v += gc.w[k] * base[(size_t)gc.idx[k] * g.C];
                        vals[j] = v * mask_at<A, T>(g, mask, b, mgi, t, p);
                    }
                }
            }
            store4<A>(dst + nl * LDB + 4 * q, {vals[0], vals[1], vals[2], vals[3]});
        }
    };

    // A operand: Z[b][m][n .. n+3] for rows m = mrow0 + mb*16 + lane%16, pixels k0 + 4*(lane/16)
    auto load_a = [&](int k0, Vec4<A> (&a)[4]) {
        const int n = k0 + 4 * (lane >> 4);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int m = mrow0 + mb * 16 + (lane & 15);
            A v[4] = {A(0), A(0), A(0), A(0)};
            if (m < g.Mg) {
                const size_t mrow = (size_t)grp * g.Mg + m;
                if (z_vec && n + 3 < kend) {
                    // 4 pixels in one image (Pn % 4 == 0 and n % 4 == 0)
                    const int b = n / g.Pn;
                    const int p = n - b * g.Pn;
                    const T *src = z + ((size_t)b * g.M + mrow) * g.Pn + p;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = to_acc<A>(src[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int ni = n + i;
                        if (ni < kend) {
                            const int b = ni / g.Pn;
                            const int p = ni - b * g.Pn;
                            v[i] = to_acc<A>(z[((size_t)b * g.M + mrow) * g.Pn + p]);
                        }
                    }
                }
            }
            a[mb] = {v[0], v[1], v[2], v[3]};
        }
    };

    acc4 acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = acc4{A(0), A(0), A(0), A(0)};

    const int nsteps = (kend - kbeg + BKP - 1) / BKP;
    if (nsteps > 0) {
        Vec4<A> a_cur[4], a_nxt[4];
        gather_step(kbeg, 0);
        load_a(kbeg, a_cur);
        __syncthreads();
        for (int s = 0; s < nsteps; ++s) {
            const int buf = s & 1;
            const bool more = s + 1 < nsteps;
            if (more) load_a(kbeg + (s + 1) * BKP, a_nxt);
            // B[k = pixel 4*(lane/16) + kk][j = channel cb*16 + lane%16]
            const A *sb = sB[buf] + 4 * (lane >> 4) * LDB + (lane & 15);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                A bv[4];
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) bv[cb] = sb[kk * LDB + cb * 16];
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    const A av = kk == 0 ? a_cur[mb].x : kk == 1 ? a_cur[mb].y : kk == 2 ? a_cur[mb].z : a_cur[mb].w;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = mfma16x16x4(av, bv[cb], acc[mb][cb]);
                }
            }
            if (more) {
                gather_step(kbeg + (s + 1) * BKP, buf ^ 1);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) a_cur[mb] = a_nxt[mb];
            }
            __syncthreads();
        }
    }

    // dW layout (M, Cg, Kn): element (m, cl, t)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int cc = c0 + cb * 16 + (lane & 15);
        if (cc >= g.Cg) continue;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = mrow0 + mb * 16 + mfma_row<A>(lane, v);
                if (m < g.Mg) atomic_add(gw + (((size_t)grp * g.Mg + m) * g.Cg + cc) * g.Kn + t, acc[mb][cb][v]);
            }
    }
}

template <int DIM, typename T, typename A, int WAVES, bool VEC4>
hipError_t launch_t(const Geo &g, const WeightTiles &tl, const void *z, const void *xcl, const void *offset,
                    const void *mask, void *gw, hipStream_t s) {
    const int m_tiles = (g.Mg + 64 * WAVES - 1) / (64 * WAVES);
    const int c_tiles = (g.Cg + BC - 1) / BC;
    const long long blocks = (long long)g.G * tl.k_splits * g.Kn * c_tiles * m_tiles;
    const bool z_vec = g.Pn % 4 == 0;
    hipLaunchKernelGGL((bwd_weight_kernel<DIM, T, A, WAVES, VEC4>), dim3((unsigned)blocks), dim3(64 * WAVES), 0, s,
                       g, static_cast<const T *>(z), static_cast<const A *>(xcl), static_cast<const T *>(offset),
                       static_cast<const T *>(mask), static_cast<A *>(gw), tl.k_chunk, m_tiles, c_tiles, tl.k_splits,
                       z_vec);
    return hipGetLastError();
}

template <int DIM, typename T, typename A>
hipError_t launch_w(const Geo &g, const WeightTiles &tl, const void *z, const void *xcl, const void *offset,
                    const void *mask, void *gw, hipStream_t s) {
#define TVDCN_WGT_CASE(W)                                                                    \
    if (tl.waves == W)                                                                       \
        return tl.vec4 ? launch_t<DIM, T, A, W, true>(g, tl, z, xcl, offset, mask, gw, s)    \
                       : launch_t<DIM, T, A, W, false>(g, tl, z, xcl, offset, mask, gw, s);
    if constexpr (sizeof(T) == 8) {
        TVDCN_WGT_CASE(1)
    } else {
        TVDCN_WGT_CASE(1)
        TVDCN_WGT_CASE(2)
        TVDCN_WGT_CASE(4)
    }
#undef TVDCN_WGT_CASE
    return hipErrorInvalidValue;
}

template <typename T, typename A>
hipError_t launch_d(int dim, const Geo &g, const WeightTiles &tl, const void *z, const void *xcl, const void *offset,
                    const void *mask, void *gw, hipStream_t s) {
    switch (dim) {
        case 1: return launch_w<1, T, A>(g, tl, z, xcl, offset, mask, gw, s);
        case 2: return launch_w<2, T, A>(g, tl, z, xcl, offset, mask, gw, s);
        case 3: return launch_w<3, T, A>(g, tl, z, xcl, offset, mask, gw, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

WeightTiles plan_weight(const Geo &g, int dtype) {
    WeightTiles t;
    if (dtype == kF64)
        t.waves = 1;
    else
        t.waves = g.Mg > 128 ? 4 : (g.Mg > 64 ? 2 : 1);
    t.vec4 = (g.C % 4 == 0) && (g.Cg % 4 == 0) && (g.og == 0 || g.cpo % 4 == 0) && (g.mg == 0 || g.cpm % 4 == 0);
    const long long m_tiles = (g.Mg + 64 * t.waves - 1) / (64 * t.waves);
    const long long c_tiles = (g.Cg + BC - 1) / BC;
    const long long tiles = (long long)g.G * g.Kn * m_tiles * c_tiles;
    // aim for ~2048 workgroups in total, at least 64 pixels per split
    long long splits = (2048 + tiles - 1) / tiles;
    const long long max_splits = (g.NP + 63) / 64;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    long long chunk = (g.NP + splits - 1) / splits;
    chunk = (chunk + BKP - 1) / BKP * BKP;
    t.k_chunk = (int)chunk;
    t.k_splits = (int)((g.NP + chunk - 1) / chunk);
    return t;
}

hipError_t launch_bwd_weight(int dtype, int dim, const Geo &g, const WeightTiles &t, const void *z, const void *xcl,
                             const void *offset, const void *mask, void *gw, hipStream_t s) {
    switch (dtype) {
        case kF32: return launch_d<float, float>(dim, g, t, z, xcl, offset, mask, gw, s);
        case kF64: return launch_d<double, double>(dim, g, t, z, xcl, offset, mask, gw, s);
        case kF16: return launch_d<__half, float>(dim, g, t, z, xcl, offset, mask, gw, s);
        case kBF16: return launch_d<__hip_bfloat16, float>(dim, g, t, z, xcl, offset, mask, gw, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
