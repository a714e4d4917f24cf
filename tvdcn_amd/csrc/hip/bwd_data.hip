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

// Sum over each row of 16 lanes, result in every lane of the row. fp32 uses DPP
// (quad xor 1, quad xor 2, half-row mirror, row mirror); fp64 uses shuffles.
__device__ __forceinline__ float row_sum16(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    return v;
}
__device__ __forceinline__ double row_sum16(double v) {
    v += __shfl_xor(v, 1, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 8, 16);
    return v;
}

template <int DIM, typename T, typename A, int WAVES, bool SCATTER, bool COORD>
__global__ void __launch_bounds__(64 * WAVES)
bwd_data_kernel(const Geo g, const T *__restrict__ z, const A *__restrict__ wd, const A *__restrict__ xcl,
                const T *__restrict__ offset, const T *__restrict__ mask, A *__restrict__ gx_cl,
                A *__restrict__ goff, A *__restrict__ gmask, const int Mg_pad, const int Cg_pad, const int n_tiles,
                const int c_tiles, const int t_groups, const bool uni) {
    constexpr int NC = 1 << DIM;
    constexpr int LDC = 64 + 4;        // row stride of the staged [32 pixels][64 channels] half tile
    // geometry record of one pixel: corner base offsets (b*Sn + idx)*C (-1 = outside the
    // grid), insert weights, sample weights (0 under the sample early-out), the
    // fractional position per axis and the mask value
    constexpr int GT = 3 * NC + DIM + 1;
    constexpr int NQ = DIM + 1;        // reduced quantities: DIM offset directions + mask
    constexpr int SA = 2 * BP * LDA;                        // Z^T double buffer (K loop)
    constexpr int SC = WAVES * 32 * LDC;                    // staged output half tiles (epilogue)
    typedef typename Acc4<A>::type acc4;
    typedef typename std::conditional<sizeof(A) == 8, long long, int>::type IBits;

    __shared__ A smem[SA > SC ? SA : SC];
    __shared__ A geo[WAVES][64][GT | 1];
    __shared__ A rowpart[COORD ? WAVES : 1][64][4 * NQ];   // 16-lane row partial sums per pixel

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
    const int zb = z_ok ? fdiv(g.dPn, zn) : 0;
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
            store4<A>(smem + buf * BP * LDA + zl_pix * LDA + 4 * mq, {v[0], v[1], v[2], v[3]});
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
            const A *sa = smem + buf * BP * LDA + (lane & 15) * LDA + 4 * (lane >> 4);
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

    // ---- epilogue -------------------------------------------------------------
    // The accumulator tile is staged through LDS in two halves of 32 pixels; then
    // lane = channel c0 + lane and the wave walks the pixels, so the corner loads and
    // the scatter atomics of one pixel cover 64 consecutive channels (256 contiguous
    // bytes) of the channels-last tensors.
    //
    // Uniform groups (all valid channels of the tile in one offset group and one
    // mask group; checked on the host): the corner geometry of the 64 pixels is
    // built once, lane = pixel, into an LDS table; per pixel the corner offsets are
    // moved to scalar registers (uniform branches, scalar address arithmetic), and
    // the offset/mask partial sums are reduced over each 16-lane row with DPP, the
    // 4 row sums parked in LDS and finished by one lane-per-pixel pass with one
    // atomic per output. Otherwise every lane resolves its own groups and geometry.
    const int cl = c0 + lane;
    const bool c_ok = cl < g.Cg;
    const int c = grp * g.Cg + (c_ok ? cl : 0);
    const int ogu = g.og ? (grp * g.Cg + c0) / g.cpo : 0;
    const int mgu = g.mg ? (grp * g.Cg + c0) / g.cpm : 0;
    if (uni) {
        const int n = n0 + lane;
        const bool n_ok = n < g.NP;
        const int b = n_ok ? fdiv(g.dPn, n) : 0;
        const int p = n_ok ? n - b * g.Pn : 0;
        const AxisW<DIM, A> aw = axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, tt, ogu), deformable);
        A *rec = geo[wave][lane];
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            int idx;
            bool ok;
            corner_at<DIM, A>(g, aw, i, idx, ok);
            ok = ok && n_ok;
            rec[i] = __builtin_bit_cast(A, (IBits)(ok ? (b * g.Sn + idx) * g.C : -1));
            const A cw = corner_weight<DIM, A>(aw, i);
            rec[NC + i] = ok ? cw : A(0);
            rec[2 * NC + i] = (ok && aw.inside) ? cw : A(0);
        }
#pragma unroll
        for (int a = 0; a < DIM; ++a) rec[3 * NC + a] = aw.fh[a];
        rec[3 * NC + DIM] = n_ok ? mask_at<A, T>(g, mask, b, mgu, tt, p) : A(0);
    }

    for (int half = 0; half < 2; ++half) {
        __syncthreads();   // K loop / previous half done with the shared buffer
        A *sC = smem + wave * 32 * LDC;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    sC[(hb * 16 + mfma_row<A>(lane, v)) * LDC + cb * 16 + (lane & 15)] =
                        half == 0 ? acc[hb][cb][v] : acc[2 + hb][cb][v];
        __syncthreads();
        if (!tap_ok) continue;
        const int npix = min(32, g.NP - n0 - half * 32);
        if (uni) {
            for (int pl = 0; pl < npix; ++pl) {
                const int pr = half * 32 + pl;
                const A *rec = geo[wave][pr];
                int cbase[NC];
#pragma unroll
                for (int i = 0; i < NC; ++i)
                    cbase[i] = __builtin_amdgcn_readfirstlane((int)__builtin_bit_cast(IBits, rec[i]));
                AxisW<DIM, A> aw;
#pragma unroll
                for (int a = 0; a < DIM; ++a) aw.fh[a] = rec[3 * NC + a];
                const A mk = rec[3 * NC + DIM];
                const A gcol = sC[pl * LDC + lane];
                if constexpr (COORD) {
                    A xv[NC];
#pragma unroll
                    for (int i = 0; i < NC; ++i) xv[i] = (cbase[i] >= 0 && c_ok) ? xcl[cbase[i] + c] : A(0);
                    A q[NQ];
#pragma unroll
                    for (int a = 0; a < DIM; ++a) {
                        A cw = A(0);
#pragma unroll
                        for (int i = 0; i < NC; ++i)
                            if (cbase[i] >= 0) cw += corner_dweight<DIM, A>(aw, i, a) * xv[i];
                        q[a] = gcol * cw * mk;
                    }
                    A sv = A(0);
#pragma unroll
                    for (int i = 0; i < NC; ++i) sv += rec[2 * NC + i] * xv[i];
                    q[DIM] = gcol * sv;
#pragma unroll
                    for (int a = 0; a < NQ; ++a) {
                        const A r = row_sum16(q[a]);
                        if ((lane & 15) == 0) rowpart[wave][pr][4 * a + (lane >> 4)] = r;
                    }
                }
                if constexpr (SCATTER) {
                    const A val = gcol * mk;
#pragma unroll
                    for (int i = 0; i < NC; ++i)
                        if (cbase[i] >= 0 && c_ok) atomic_add(gx_cl + cbase[i] + c, rec[NC + i] * val);
                }
            }
        } else {
            const int ogi = g.og ? c / g.cpo : 0;
            const int mgi = g.mg ? c / g.cpm : 0;
            for (int pl = 0; pl < npix; ++pl) {
                const int n = n0 + half * 32 + pl;
                const int b = fdiv(g.dPn, n);
                const int p = n - b * g.Pn;
                const AxisW<DIM, A> aw =
                    axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, ogi), deformable);
                const A mk = mask_at<A, T>(g, mask, b, mgi, t, p);
                const A gcol = sC[pl * LDC + lane];
                int cbase[NC];
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    int idx;
                    bool ok;
                    corner_at<DIM, A>(g, aw, i, idx, ok);
                    cbase[i] = (ok && c_ok) ? (b * g.Sn + idx) * g.C : -1;
                }
                if constexpr (COORD) {
                    A xv[NC];
#pragma unroll
                    for (int i = 0; i < NC; ++i) xv[i] = cbase[i] >= 0 ? xcl[cbase[i] + c] : A(0);
                    if (c_ok && deformable) {
#pragma unroll
                        for (int a = 0; a < DIM; ++a) {
                            A cw = A(0);
#pragma unroll
                            for (int i = 0; i < NC; ++i)
                                if (cbase[i] >= 0) cw += corner_dweight<DIM, A>(aw, i, a) * xv[i];
                            atomic_add(goff + ((((size_t)b * g.og + ogi) * g.Kn + t) * DIM + a) * g.Pn + p,
                                       gcol * cw * mk);
                        }
                    }
                    if (c_ok && mask != nullptr) {
                        A sv = A(0);
                        if (aw.inside) {
#pragma unroll
                            for (int i = 0; i < NC; ++i)
                                if (cbase[i] >= 0) sv += corner_weight<DIM, A>(aw, i) * xv[i];
                        }
                        atomic_add(gmask + (((size_t)b * g.mg + mgi) * g.Kn + t) * g.Pn + p, gcol * sv);
                    }
                }
                if constexpr (SCATTER) {
                    const A val = gcol * mk;
#pragma unroll
                    for (int i = 0; i < NC; ++i)
                        if (cbase[i] >= 0) atomic_add(gx_cl + cbase[i] + c, corner_weight<DIM, A>(aw, i) * val);
                }
            }
        }
    }
    if constexpr (COORD) {
        if (uni && tap_ok) {
            // lane = pixel: sum the 4 row partials, one atomic per (pixel, quantity);
            // consecutive lanes hit consecutive pixels of the output row
            const int n = n0 + lane;
            if (n < g.NP) {
                const int b = fdiv(g.dPn, n);
                const int p = n - b * g.Pn;
                const A *rp = rowpart[wave][lane];
                if (deformable)
#pragma unroll
                    for (int a = 0; a < DIM; ++a)
                        atomic_add(goff + ((((size_t)b * g.og + ogu) * g.Kn + t) * DIM + a) * g.Pn + p,
                                   rp[4 * a] + rp[4 * a + 1] + rp[4 * a + 2] + rp[4 * a + 3]);
                if (mask != nullptr)
                    atomic_add(gmask + (((size_t)b * g.mg + mgu) * g.Kn + t) * g.Pn + p,
                               rp[4 * DIM] + rp[4 * DIM + 1] + rp[4 * DIM + 2] + rp[4 * DIM + 3]);
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
                       n_tiles, c_tiles, t_groups, tl.uniform);
    return hipGetLastError();
}

template <int DIM, typename T, typename A, bool SCATTER, bool COORD>
hipError_t launch_w(const Geo &g, const DataTiles &tl, const void *z, const void *wd, const void *xcl,
                    const void *offset, const void *mask, void *gx_cl, void *goff, void *gmask, hipStream_t s) {
    if (tl.waves == 4)
        return launch_t<DIM, T, A, 4, SCATTER, COORD>(g, tl, z, wd, xcl, offset, mask, gx_cl, goff, gmask, s);
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
    t.waves = g.Kn >= 4 ? 4 : 1;
    t.Mg_pad = (g.Mg + BKM - 1) / BKM * BKM;
    t.Cg_pad = (g.Cg + 63) / 64 * 64;
    // every 64-channel tile must lie inside one offset group and one mask group
    t.uniform = true;
    for (int grp = 0; grp < g.G && t.uniform; ++grp)
        for (int c0 = 0; c0 < g.Cg; c0 += 64) {
            const int first = grp * g.Cg + c0, last = grp * g.Cg + (c0 + 64 < g.Cg ? c0 + 64 : g.Cg) - 1;
            if ((g.og && first / g.cpo != last / g.cpo) || (g.mg && first / g.cpm != last / g.cpm)) {
                t.uniform = false;
                break;
            }
        }
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
