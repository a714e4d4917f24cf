// Family F: fused deformable gather + implicit GEMM on MFMA.
//
//   Y[b][m][p] = sum_{t, c in group} W[m][c][t] * mask[b][mg(c)][t][p] * bilinear(X[b][c], pos(b, og(c), t, p))
//
// Replaces the reference's im2col kernel + addmm_ pair
// (tvdcn/csrc/ops/cuda/deform_conv2d_common_kernels.cu:138-256 and
// deform_conv2d_kernel.cpp:341-369); the columns matrix is never written to
// HBM. Used for the conv forward and for grad_input of the transposed op.
//
// Workgroup tile: 64 column pixels x (64 * WAVES) GEMM-side channels, K stepped
// 16 channels of one tap at a time. Each wave owns 64 rows and accumulates
// 4 x 4 MFMA 16x16x4 blocks (64 accumulator registers per lane).
//   * A (weights): read straight from global into registers, 4 consecutive K
//     per lane (one 16-byte load per 16-row block), prefetched one step ahead.
//   * B (sampled columns): gathered cooperatively from the channels-last copy
//     of X (4 lanes x 16 B cover one pixel's 16 channels: coalesced), combined
//     with the bilinear weights and the mask, and staged in a double-buffered
//     LDS tile [64 pixels][16 + 4] read back with 16-byte LDS loads.
// The corner indices/weights of a (pixel, tap, offset group) are computed once
// and reused for every 16-channel step of that tap.
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int BN = 64;   // column pixels per tile
constexpr int BK = 16;   // reduction channels per step
constexpr int LDB = BK + 4;

template <int DIM, typename T, typename A, int WAVES, bool VEC4>
__global__ void __launch_bounds__(64 * WAVES)
fwd_gather_gemm_kernel(const Geo g, const A *__restrict__ xcl, const A *__restrict__ wf,
                       const T *__restrict__ offset, const T *__restrict__ mask, const T *__restrict__ bias,
                       T *__restrict__ y, const int Mg_pad, const int Cg_pad, const int n_tiles, const int m_tiles) {
    constexpr int NT = 64 * WAVES;
    constexpr int SLOTS = (BN * BK / 4) / NT;   // (pixel, channel-quad) slots per thread
    constexpr int NC = 1 << DIM;
    typedef typename Acc4<A>::type acc4;

    __shared__ A sB[2][BN * LDB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int mt = L % m_tiles;
    const int nt = (L / m_tiles) % n_tiles;
    const int grp = L / (m_tiles * n_tiles);
    const int n0 = nt * BN;
    const int mrow0 = mt * (64 * WAVES) + wave * 64;   // first row (within the group) of this wave

    const bool deformable = offset != nullptr;
    const int csteps = Cg_pad / BK;
    const int nsteps = g.Kn * csteps;

    // ---- gather slot bookkeeping -------------------------------------------
    // slot i of this thread: pixel (tid / 4) + i * (NT / 4), channel quad tid % 4
    const int q = tid & 3;
    int s_b[SLOTS], s_p[SLOTS], s_nl[SLOTS];
    bool s_ok[SLOTS];
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
        s_nl[i] = (tid >> 2) + i * (NT / 4);
        const int n = n0 + s_nl[i];
        s_ok[i] = n < g.NP;
        const int nn = s_ok[i] ? n : 0;
        s_b[i] = fdiv(g.dPn, nn);
        s_p[i] = nn - s_b[i] * g.Pn;
    }
    // fast-path corner cache (one set per slot)
    GatherCorners<DIM, A> s_gc[VEC4 ? SLOTS : 1];
    A s_mask[VEC4 ? SLOTS : 1];
    int cached_t = -1, cached_og = -1, cached_mg = -1;

    // Writes the sampled values of step `step` into LDS buffer `buf`.
    auto gather_step = [&](int step, int buf) {
        const int t = step / csteps;
        const int cl = (step - t * csteps) * BK + 4 * q;   // channel within group
        const int c = grp * g.Cg + cl;
        A *dst = sB[buf];
        if constexpr (VEC4) {
            const bool cvalid = cl < g.Cg;
            const int ogi = (g.og && cvalid) ? c / g.cpo : 0;
            const int mgi = (g.mg && cvalid) ? c / g.cpm : 0;
            if (t != cached_t || ogi != cached_og) {
#pragma unroll
                for (int i = 0; i < SLOTS; ++i) {
                    const Point<DIM, A> pt = sample_point<DIM, A, T>(g, offset, s_b[i], s_p[i], t, ogi);
                    s_gc[i] = gather_corners<DIM, A>(g, axis_weights<DIM, A>(g, pt, deformable));
                }
            }
            if (t != cached_t || mgi != cached_mg) {
#pragma unroll
                for (int i = 0; i < SLOTS; ++i) s_mask[i] = mask_at<A, T>(g, mask, s_b[i], mgi, t, s_p[i]);
            }
            cached_t = t;
            cached_og = ogi;
            cached_mg = mgi;
            Vec4<A> raw[SLOTS][NC];
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                const A *base = xcl + (size_t)s_b[i] * g.Sn * g.C + c;
#pragma unroll
                for (int k = 0; k < NC; ++k) {
                    if (cvalid && s_ok[i])
                        raw[i][k] = load4<A>(base + (size_t)s_gc[i].idx[k] * g.C);
                    else
                        raw[i][k] = {A(0), A(0), A(0), A(0)};
                }
            }
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                Vec4<A> v = {A(0), A(0), A(0), A(0)};
#pragma unroll
                for (int k = 0; k < NC; ++k) {
                    const A w = s_gc[i].w[k];
                    v.x += w * raw[i][k].x;
                    v.y += w * raw[i][k].y;
                    v.z += w * raw[i][k].z;
                    v.w += w * raw[i][k].w;
                }
                const A mk = s_mask[i];
                v.x *= mk; v.y *= mk; v.z *= mk; v.w *= mk;
                store4<A>(dst + s_nl[i] * LDB + 4 * q, v);
            }
        } else {
            // generic path: every channel resolves its own offset/mask group
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                A vals[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    vals[j] = A(0);
                    const int clj = cl + j;
                    if (clj < g.Cg && s_ok[i]) {
                        const int cj = c + j;
                        const int ogi = g.og ? cj / g.cpo : 0;
                        const int mgi = g.mg ? cj / g.cpm : 0;
                        const Point<DIM, A> pt = sample_point<DIM, A, T>(g, offset, s_b[i], s_p[i], t, ogi);
                        const GatherCorners<DIM, A> gc = gather_corners<DIM, A>(g, axis_weights<DIM, A>(g, pt, deformable));
                        const A *base = xcl + (size_t)s_b[i] * g.Sn * g.C + cj;
                        A v = A(0);
#pragma unroll
                        for (int k = 0; k < NC; ++k) v += gc.w[k] * base[(size_t)gc.idx[k] * g.C];
                        vals[j] = v * mask_at<A, T>(g, mask, s_b[i], mgi, t, s_p[i]);
                    }
                }
                store4<A>(dst + s_nl[i] * LDB + 4 * q, {vals[0], vals[1], vals[2], vals[3]});
            }
        }
    };

    // weight fragment rows of this wave: mrow0 + mb * 16 + lane % 16, K quad lane / 16
    const A *wrow = wf + ((size_t)grp * g.Kn * Mg_pad + mrow0 + (lane & 15)) * Cg_pad + 4 * (lane >> 4);
    auto load_a = [&](int step, Vec4<A> (&a)[4]) {
        const int t = step / csteps;
        const int k0 = (step - t * csteps) * BK;
        const A *p = wrow + (size_t)t * Mg_pad * Cg_pad + k0;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) a[mb] = load4<A>(p + (size_t)mb * 16 * Cg_pad);
    };

    acc4 acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = acc4{A(0), A(0), A(0), A(0)};

    Vec4<A> a_cur[4], a_nxt[4];
    gather_step(0, 0);
    load_a(0, a_cur);
    __syncthreads();

    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        const bool more = step + 1 < nsteps;
        if (more) load_a(step + 1, a_nxt);

        const A *sb = sB[buf] + (lane & 15) * LDB + 4 * (lane >> 4);
        Vec4<A> bq[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) bq[nb] = load4<A>(sb + nb * 16 * LDB);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) {
                acc[mb][nb] = mfma16x16x4(a_cur[mb].x, bq[nb].x, acc[mb][nb]);
                acc[mb][nb] = mfma16x16x4(a_cur[mb].y, bq[nb].y, acc[mb][nb]);
                acc[mb][nb] = mfma16x16x4(a_cur[mb].z, bq[nb].z, acc[mb][nb]);
                acc[mb][nb] = mfma16x16x4(a_cur[mb].w, bq[nb].w, acc[mb][nb]);
            }

        if (more) {
            gather_step(step + 1, buf ^ 1);
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) a_cur[mb] = a_nxt[mb];
        }
        __syncthreads();
    }

    // ---- epilogue: + bias, store NC<spatial> ---------------------------------
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        const int n = n0 + nb * 16 + (lane & 15);
        if (n >= g.NP) continue;
        const int b = fdiv(g.dPn, n);
        const int p = n - b * g.Pn;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = mrow0 + mb * 16 + mfma_row<A>(lane, v);
                if (m < g.Mg) {
                    const int mg_glob = grp * g.Mg + m;
                    A r = acc[mb][nb][v];
                    if (bias != nullptr) r += to_acc<A>(bias[mg_glob]);
                    y[((size_t)b * g.M + mg_glob) * g.Pn + p] = from_acc<T, A>(r);
                }
            }
    }
}

template <int DIM, typename T, typename A, int WAVES, bool VEC4>
hipError_t launch_t(const Geo &g, const FwdTiles &tl, const void *xcl, const void *wf, const void *offset,
                    const void *mask, const void *bias, void *y, hipStream_t s) {
    const int n_tiles = (g.NP + BN - 1) / BN;
    const int m_tiles = tl.Mg_pad / (64 * WAVES);
    const long long blocks = (long long)n_tiles * m_tiles * g.G;
    hipLaunchKernelGGL((fwd_gather_gemm_kernel<DIM, T, A, WAVES, VEC4>), dim3((unsigned)blocks), dim3(64 * WAVES), 0, s,
                       g, static_cast<const A *>(xcl), static_cast<const A *>(wf), static_cast<const T *>(offset),
                       static_cast<const T *>(mask), static_cast<const T *>(bias), static_cast<T *>(y), tl.Mg_pad,
                       tl.Cg_pad, n_tiles, m_tiles);
    return hipGetLastError();
}

template <int DIM, typename T, typename A>
hipError_t launch_w(const Geo &g, const FwdTiles &tl, const void *xcl, const void *wf, const void *offset,
                    const void *mask, const void *bias, void *y, hipStream_t s) {
#define TVDCN_FWD_CASE(W)                                                                              \
    if (tl.waves == W)                                                                                 \
        return tl.vec4 ? launch_t<DIM, T, A, W, true>(g, tl, xcl, wf, offset, mask, bias, y, s)        \
                       : launch_t<DIM, T, A, W, false>(g, tl, xcl, wf, offset, mask, bias, y, s);
    if constexpr (sizeof(T) == 8) {
        TVDCN_FWD_CASE(1)
    } else {
        TVDCN_FWD_CASE(1)
        TVDCN_FWD_CASE(2)
        TVDCN_FWD_CASE(4)
    }
#undef TVDCN_FWD_CASE
    return hipErrorInvalidValue;
}

template <typename T, typename A>
hipError_t launch_d(int dim, const Geo &g, const FwdTiles &tl, const void *xcl, const void *wf, const void *offset,
                    const void *mask, const void *bias, void *y, hipStream_t s) {
    switch (dim) {
        case 1: return launch_w<1, T, A>(g, tl, xcl, wf, offset, mask, bias, y, s);
        case 2: return launch_w<2, T, A>(g, tl, xcl, wf, offset, mask, bias, y, s);
        case 3: return launch_w<3, T, A>(g, tl, xcl, wf, offset, mask, bias, y, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

FwdTiles plan_fwd(const Geo &g, int dtype) {
    FwdTiles t;
    if (dtype == kF64)
        t.waves = 1;
    else
        t.waves = g.Mg > 128 ? 4 : (g.Mg > 64 ? 2 : 1);
    const int bm = 64 * t.waves;
    t.Mg_pad = (g.Mg + bm - 1) / bm * bm;
    t.Cg_pad = (g.Cg + BK - 1) / BK * BK;
    t.vec4 = (g.C % 4 == 0) && (g.Cg % 4 == 0) && (g.og == 0 || g.cpo % 4 == 0) && (g.mg == 0 || g.cpm % 4 == 0);
    return t;
}

hipError_t launch_fwd_gather_gemm(int dtype, int dim, const Geo &g, const FwdTiles &t, const void *xcl,
                                  const void *wf, const void *offset, const void *mask, const void *bias, void *y,
                                  hipStream_t s) {
    switch (dtype) {
        case kF32: return launch_d<float, float>(dim, g, t, xcl, wf, offset, mask, bias, y, s);
        case kF64: return launch_d<double, double>(dim, g, t, xcl, wf, offset, mask, bias, y, s);
        case kF16: return launch_d<__half, float>(dim, g, t, xcl, wf, offset, mask, bias, y, s);
        case kBF16: return launch_d<__hip_bfloat16, float>(dim, g, t, xcl, wf, offset, mask, bias, y, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
