// Family D: grad-columns on MFMA with a fused scatter / coordinate-gradient epilogue.
//
//   G[c][t][b][p] = sum_{m in group} W[m][c][t] * Z[b][m][p]          (MFMA, never stored)
//   SCATTER: dX[b][corner][c] += w_corner * G * mask                   (bilinear insert)
//   COORD:   dOffset[b][og][t][a][p] += G * mask * d(sample)/d(pos_a)  (summed over c in og)
//            dMask[b][mg][t][p]      += G * sample                      (summed over c in mg)
//
// Replaces, per batch block, the reference's grad-columns addmm_ + col2im +
// compute_grad_offset + compute_grad_mask (tvdcn/csrc/ops/cuda/
// deform_conv2d_kernel.cpp:518-598; kernels deform_conv2d_common_kernels.cu:258-624).
// Conv backward: Z = grad_out, X = input (SCATTER + COORD). Transposed forward:
// Z = input, dX = output (SCATTER only). Transposed backward: Z = input,
// X = grad_out (COORD only).
//
// Tile: 64 column pixels (rows) x WAVES taps x 64 sampled-side channels; each
// wave owns one tap and accumulates 4 x 4 MFMA 16x16x4 blocks. Output layout
// per lane: 4 pixels x 1 channel per block, so every atomic
// instruction covers 4 pixels x 16 consecutive channels of the channels-last
// gradient (4 x 64 B segments). Offset/mask partial sums are reduced across the
// 16 channel lanes with cross-lane shuffles and across the wave's 4 channel
// blocks in registers before one atomic per (pixel, tap, direction).
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int BP = 64;          // pixels per tile
constexpr int BKM = 16;         // GEMM-side channels per step
constexpr int LDA = BKM + 4;

template <typename A>
__device__ __forceinline__ A sum16(A v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

template <int DIM, typename T, typename A, int WAVES, bool SCATTER, bool COORD>
__global__ void __launch_bounds__(64 * WAVES)
bwd_data_kernel(const Geo g, const T *__restrict__ z, const A *__restrict__ wd, const A *__restrict__ xcl,
                const T *__restrict__ offset, const T *__restrict__ mask, A *__restrict__ gx_cl,
                A *__restrict__ goff, A *__restrict__ gmask, const int Mg_pad, const int Cg_pad, const int n_tiles,
                const int c_tiles, const int t_groups) {
    constexpr int NT = 64 * WAVES;
    constexpr int NC = 1 << DIM;
    typedef typename Acc4<A>::type acc4;

    __shared__ A sA[2][BP * LDA];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int tg = L % t_groups;
    const int ct = (L / t_groups) % c_tiles;
    const int nt = (L / (t_groups * c_tiles)) % n_tiles;
    const int grp = L / (t_groups * c_tiles * n_tiles);
    const int n0 = nt * BP;
    const int c0 = ct * 64;                 // first channel (within group) of this tile
    const int t = tg * WAVES + wave;        // this wave's tap
    const bool tap_ok = t < g.Kn;
    const bool deformable = offset != nullptr;

    // ---- Z^T tile loader: thread -> (pixel tid % 64, m quads (tid / 64) + j * WAVES)
    constexpr int QUADS = 4 / WAVES;        // m quads per thread (4 quads = 16 m per step)
    const int zl_pix = tid & 63;
    const int zn = n0 + zl_pix;
    const bool z_ok = zn < g.NP;
    const int zb = z_ok ? zn / g.Pn : 0;
    const int zp = z_ok ? zn - zb * g.Pn : 0;
    const T *zbase = z + ((size_t)zb * g.M + (size_t)grp * g.Mg) * g.Pn + zp;

    auto load_z = [&](int ms, int buf) {
#pragma unroll
        for (int j = 0; j < QUADS; ++j) {
            const int mq = (tid >> 6) + j * WAVES;
            const int m = ms * BKM + 4 * mq;
            A v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[i] = (z_ok && m + i < g.Mg) ? to_acc<A>(zbase[(size_t)(m + i) * g.Pn]) : A(0);
            store4<A>(sA[buf] + zl_pix * LDA + 4 * mq, {v[0], v[1], v[2], v[3]});
        }
    };

    // ---- W fragment (B operand): B[k = m][j = c], lane reads 4 consecutive m of channel c
    const int tt = tap_ok ? t : 0;
    const A *wcol = wd + (((size_t)grp * g.Kn + tt) * Cg_pad + c0 + (lane & 15)) * Mg_pad + 4 * (lane >> 4);
    auto load_w = [&](int ms, Vec4<A> (&w)[4]) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) w[cb] = load4<A>(wcol + (size_t)cb * 16 * Mg_pad + ms * BKM);
    };

    acc4 acc[4][4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[pb][cb] = acc4{A(0), A(0), A(0), A(0)};

    const int msteps = Mg_pad / BKM;
    Vec4<A> w_cur[4], w_nxt[4];
    load_z(0, 0);
    load_w(0, w_cur);
    __syncthreads();
    for (int ms = 0; ms < msteps; ++ms) {
        const int buf = ms & 1;
        const bool more = ms + 1 < msteps;
        if (more) {
            load_w(ms + 1, w_nxt);
            load_z(ms + 1, buf ^ 1);
        }
        if (tap_ok) {
            const A *sa = sA[buf] + (lane & 15) * LDA + 4 * (lane >> 4);
            Vec4<A> aq[4];
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) aq[pb] = load4<A>(sa + pb * 16 * LDA);
#pragma unroll
            for (int pb = 0; pb < 4; ++pb)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    acc[pb][cb] = mfma16x16x4(aq[pb].x, w_cur[cb].x, acc[pb][cb]);
                    acc[pb][cb] = mfma16x16x4(aq[pb].y, w_cur[cb].y, acc[pb][cb]);
                    acc[pb][cb] = mfma16x16x4(aq[pb].z, w_cur[cb].z, acc[pb][cb]);
                    acc[pb][cb] = mfma16x16x4(aq[pb].w, w_cur[cb].w, acc[pb][cb]);
                }
        }
        if (more) {
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) w_cur[cb] = w_nxt[cb];
        }
        __syncthreads();
    }
    if (!tap_ok) return;

    // ---- epilogue ----------------------------------------------------------
    // Offset/mask groups are wave-uniform when the wave's valid channels all fall
    // in one group; then corner geometry is shared by the 4 channel blocks and
    // partial sums are reduced across lanes before the atomics.
    const int cfirst = grp * g.Cg + c0;
    const int clast = grp * g.Cg + min(c0 + 64, g.Cg) - 1;
    const bool og_uni = g.og == 0 || (cfirst / g.cpo == clast / g.cpo);
    const bool mg_uni = g.mg == 0 || (cfirst / g.cpm == clast / g.cpm);
    const bool uni = og_uni && mg_uni;
    const int ogi0 = g.og ? cfirst / g.cpo : 0;
    const int mgi0 = g.mg ? cfirst / g.cpm : 0;

#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = n0 + pb * 16 + mfma_row<A>(lane, v);
            const bool n_ok = n < g.NP;
            const int b = n_ok ? n / g.Pn : 0;
            const int p = n_ok ? n - b * g.Pn : 0;
            AxisW<DIM, A> aw0;
            A mk0 = A(1);
            if (uni) {
                aw0 = axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, ogi0), deformable);
                mk0 = mask_at<A, T>(g, mask, b, mgi0, t, p);
            }
            A part_off[DIM];
            A part_mask = A(0);
#pragma unroll
            for (int a = 0; a < DIM; ++a) part_off[a] = A(0);

#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const int cl = c0 + cb * 16 + (lane & 15);
                if (!n_ok || cl >= g.Cg) continue;
                const int c = grp * g.Cg + cl;
                AxisW<DIM, A> aw = aw0;
                A mk = mk0;
                int ogi = ogi0, mgi = mgi0;
                if (!uni) {
                    ogi = g.og ? c / g.cpo : 0;
                    mgi = g.mg ? c / g.cpm : 0;
                    aw = axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, ogi), deformable);
                    mk = mask_at<A, T>(g, mask, b, mgi, t, p);
                }
                const A gcol = acc[pb][cb][v];
                const size_t img = (size_t)b * g.Sn;
                if constexpr (SCATTER) {
                    const A val = gcol * mk;
#pragma unroll
                    for (int i = 0; i < NC; ++i) {
                        int idx;
                        bool ok;
                        corner_at<DIM, A>(g, aw, i, idx, ok);
                        if (ok) atomic_add(gx_cl + (img + idx) * g.C + c, corner_weight<DIM, A>(aw, i) * val);
                    }
                }
                if constexpr (COORD) {
                    A xv[NC];
#pragma unroll
                    for (int i = 0; i < NC; ++i) {
                        int idx;
                        bool ok;
                        corner_at<DIM, A>(g, aw, i, idx, ok);
                        xv[i] = ok ? xcl[(img + idx) * g.C + c] : A(0);
                    }
                    A contrib_off[DIM];
                    if (deformable) {
#pragma unroll
                        for (int a = 0; a < DIM; ++a) {
                            A cw = A(0);
#pragma unroll
                            for (int i = 0; i < NC; ++i) cw += corner_dweight<DIM, A>(aw, i, a) * xv[i];
                            contrib_off[a] = gcol * cw * mk;
                        }
                    }
                    A contrib_mask = A(0);
                    if (mask != nullptr && aw.inside) {
                        A sv = A(0);
#pragma unroll
                        for (int i = 0; i < NC; ++i) sv += corner_weight<DIM, A>(aw, i) * xv[i];
                        contrib_mask = gcol * sv;
                    }
                    if (uni) {
                        if (deformable)
#pragma unroll
                            for (int a = 0; a < DIM; ++a) part_off[a] += contrib_off[a];
                        part_mask += contrib_mask;
                    } else {
                        if (deformable)
#pragma unroll
                            for (int a = 0; a < DIM; ++a)
                                atomic_add(goff + ((((size_t)b * g.og + ogi) * g.Kn + t) * DIM + a) * g.Pn + p,
                                           contrib_off[a]);
                        if (mask != nullptr)
                            atomic_add(gmask + (((size_t)b * g.mg + mgi) * g.Kn + t) * g.Pn + p, contrib_mask);
                    }
                }
            }
            if constexpr (COORD) {
                if (uni) {
                    if (deformable) {
#pragma unroll
                        for (int a = 0; a < DIM; ++a) part_off[a] = sum16(part_off[a]);
                    }
                    if (mask != nullptr) part_mask = sum16(part_mask);
                    if ((lane & 15) == 0 && n_ok) {
                        if (deformable)
#pragma unroll
                            for (int a = 0; a < DIM; ++a)
                                atomic_add(goff + ((((size_t)b * g.og + ogi0) * g.Kn + t) * DIM + a) * g.Pn + p,
                                           part_off[a]);
                        if (mask != nullptr)
                            atomic_add(gmask + (((size_t)b * g.mg + mgi0) * g.Kn + t) * g.Pn + p, part_mask);
                    }
                }
            }
        }
}

template <int DIM, typename T, typename A, int WAVES, bool SCATTER, bool COORD>
hipError_t launch_t(const Geo &g, const DataTiles &tl, const void *z, const void *wd, const void *xcl,
                    const void *offset, const void *mask, void *gx_cl, void *goff, void *gmask, hipStream_t s) {
    const int n_tiles = (g.NP + BP - 1) / BP;
    const int c_tiles = tl.Cg_pad / 64;
    const int t_groups = (g.Kn + WAVES - 1) / WAVES;
    const long long blocks = (long long)g.G * n_tiles * c_tiles * t_groups;
    hipLaunchKernelGGL((bwd_data_kernel<DIM, T, A, WAVES, SCATTER, COORD>), dim3((unsigned)blocks),
                       dim3(64 * WAVES), 0, s, g, static_cast<const T *>(z), static_cast<const A *>(wd),
                       static_cast<const A *>(xcl), static_cast<const T *>(offset), static_cast<const T *>(mask),
                       static_cast<A *>(gx_cl), static_cast<A *>(goff), static_cast<A *>(gmask), tl.Mg_pad, tl.Cg_pad,
                       n_tiles, c_tiles, t_groups);
    return hipGetLastError();
}

template <int DIM, typename T, typename A, bool SCATTER, bool COORD>
hipError_t launch_w(const Geo &g, const DataTiles &tl, const void *z, const void *wd, const void *xcl,
                    const void *offset, const void *mask, void *gx_cl, void *goff, void *gmask, hipStream_t s) {
    if (tl.waves == 4)
        return launch_t<DIM, T, A, 4, SCATTER, COORD>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    if (tl.waves == 2)
        return launch_t<DIM, T, A, 2, SCATTER, COORD>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    return launch_t<DIM, T, A, 1, SCATTER, COORD>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
}

template <int DIM, typename T, typename A>
hipError_t launch_f(const Geo &g, const DataTiles &tl, bool scatter, bool coord, const void *z, const void *wd,
                    const void *xcl, const void *offset, const void *mask, void *gx_cl, void *goff, void *gmask,
                    hipStream_t s) {
    if (scatter && coord)
        return launch_w<DIM, T, A, true, true>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    if (scatter) return launch_w<DIM, T, A, true, false>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    if (coord) return launch_w<DIM, T, A, false, true>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    return hipSuccess;
}

template <typename T, typename A>
hipError_t launch_d(int dim, const Geo &g, const DataTiles &tl, bool scatter, bool coord, const void *z,
                    const void *wd, const void *xcl, const void *offset, const void *mask, void *gx_cl, void *goff,
                    void *gmask, hipStream_t s) {
    switch (dim) {
        case 1: return launch_f<1, T, A>(g, tl, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
        case 2: return launch_f<2, T, A>(g, tl, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
        case 3: return launch_f<3, T, A>(g, tl, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

DataTiles plan_data(const Geo &g, int dtype) {
    DataTiles t;
    (void)dtype;
    t.waves = g.Kn >= 4 ? 4 : (g.Kn >= 2 ? 2 : 1);
    t.Mg_pad = (g.Mg + BKM - 1) / BKM * BKM;
    t.Cg_pad = (g.Cg + 63) / 64 * 64;
    return t;
}

hipError_t launch_bwd_data(int dtype, int dim, const Geo &g, const DataTiles &t, bool scatter, bool coord,
                           const void *z, const void *wd, const void *xcl, const void *offset, const void *mask,
                           void *gx_cl, void *goff, void *gmask, hipStream_t s) {
    switch (dtype) {
        case kF32:
            return launch_d<float, float>(dim, g, t, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
        case kF64:
            return launch_d<double, double>(dim, g, t, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask,
                                            s);
        case kF16:
            return launch_d<__half, float>(dim, g, t, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
        case kBF16:
            return launch_d<__hip_bfloat16, float>(dim, g, t, scatter, coord, z, wd, xcl, offset, mask, gx_cl, goff,
                                                   gmask, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
