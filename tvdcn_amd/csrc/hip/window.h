// Tile / window machinery shared by the windowed kernels (bwd_data_win.hip,
// bwd_weight_win.hip).
//
// A tile is a box of 256 column pixels of one image (WinTiles::box) times one
// 16-channel slice of the sampled side. Its window is the box of the sampled grid
// covering the tile's undeformed footprint (low and high bilinear corners of every
// tap) plus a margin R per axis (WinTiles::R, WE). Per tile the kernels keep in LDS:
//   * the sampling table geo[tap][pixel] (position per axis, mask, and for 1D/2D the
//     window cell of the low corner when all corners fall in the window), built once
//     per pass of taps from the offsets and masks;
//   * the X window [cell][XS]: the tile's 16 channels of the sampled tensor at every
//     window cell (zeros outside the grid), read instead of global memory whenever a
//     bilinear corner falls inside the window.
#pragma once

#include "kernels.h"

namespace tvdcn_hip {
namespace win {

constexpr int BPX = 256;   // column pixels per tile
constexpr int BC = 16;     // sampled-side channels per tile
constexpr int XS = BC + 4; // X window cell stride (floats; 16-byte quads)

typedef f32x4 acc4;

// Per-workgroup tile context.
struct Tile {
    int b;              // image
    int grp;            // conv group
    int c0, cg0;        // first channel of the tile: within the group / global
    int ogu, mgu;       // the tile's offset / mask group (uniform over its channels)
    int p0[3], org[3];  // tile origin on the column grid; window origin on the sampled grid

    // s = spatial tile index over (B, ntile0, ntile1, ntile2), row-major
    __device__ __forceinline__ void init(const Geo &g, const WinTiles &wt, int s, int ct, int grp_) {
        int tc[3];
        tc[2] = s % wt.ntile[2];
        s /= wt.ntile[2];
        tc[1] = s % wt.ntile[1];
        s /= wt.ntile[1];
        tc[0] = s % wt.ntile[0];
        b = s / wt.ntile[0];
        grp = grp_;
        c0 = ct * BC;
        cg0 = grp * g.Cg + c0;
        ogu = g.og ? cg0 / g.cpo : 0;
        mgu = g.mg ? cg0 / g.cpm : 0;
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            p0[e] = tc[e] * wt.box[e];
            org[e] = p0[e] * g.st[e] - g.pad[e] - wt.R[e];
        }
    }

    // pixel i of the tile (0..255) -> column pixel index p, or -1 outside the grid
    __device__ __forceinline__ int pixel(const Geo &g, const WinTiles &wt, int i) const {
        const int iz = i >> wt.lbxy;
        const int iy = (i >> wt.lbx) & (wt.box[1] - 1);
        const int ix = i & (wt.box[2] - 1);
        const int pz = p0[0] + iz, py = p0[1] + iy, px = p0[2] + ix;
        if (pz >= g.P[0] || py >= g.P[1] || px >= g.P[2]) return -1;
        return (pz * g.P[1] + py) * g.P[2] + px;
    }

    // window cell -> flat sampled-grid index, or -1 outside the grid
    __device__ __forceinline__ int cell_index(const Geo &g, const WinTiles &wt, int cell) const {
        const int lx = cell % wt.WE[2];
        const int r = cell / wt.WE[2];
        const int ly = r % wt.WE[1];
        const int lz = r / wt.WE[1];
        const int sz = org[0] + lz, sy = org[1] + ly, sx = org[2] + lx;
        if (sz < 0 || sz >= g.S[0] || sy < 0 || sy >= g.S[1] || sx < 0 || sx >= g.S[2]) return -1;
        return (sz * g.S[1] + sy) * g.S[2] + sx;
    }

    // window cell of a corner at low coordinates lo + bit(k), or -1 when outside
    template <int DIM>
    __device__ __forceinline__ int corner_cell(const WinTiles &wt, const AxisW<DIM, float> &aw, int k) const {
        bool in = wt.cells > 0;
        int lin = 0;
#pragma unroll
        for (int a = 0; a < DIM; ++a) {
            const int e = 3 - DIM + a;
            const int l = aw.lo[a] + corner_bit<DIM>(k, a) - org[e];
            in = in && l >= 0 && l < wt.WE[e];
            lin = lin * wt.WE[e] + l;
        }
        return in ? lin : -1;
    }
};

// geo[tl * BPX + i] for the taps t0 .. t0 + ntaps - 1 of the tile. Record layout:
//   DIM <= 2: (position per axis, mask, fast cell), DIM = 3: (position z, y, x, mask).
// "fast cell" (DIM <= 2) is the window cell of the low corner when every bilinear
// corner cell lies inside the window, else -1: then the corners are cell, cell + 1
// (, cell + WE_x, cell + WE_x + 1) and the plain bilinear formulas apply. Corners
// outside the grid need no test there: the X window holds zeros at those cells
// (which reproduces the zero padding and the sample range rule, whose excluded
// points have every corner outside the grid), and scatter into them is dropped
// when the window is flushed. Pixels outside the grid get position -4 on every axis
// (no corner inside the grid), mask 0 and no fast cell.
template <int DIM> __device__ __forceinline__ float rec_mask(const acc4 &r) { return DIM == 3 ? r[3] : r[DIM]; }
template <int DIM> __device__ __forceinline__ int rec_fast_cell(const acc4 &r) {
    return DIM == 3 ? -1 : __float_as_int(r[3]);
}

// Fast cell of a record (DIM <= 2; none for DIM = 3: the 3D windows that fit in LDS
// have margins of at most one cell, where most waves hold a lane outside the window
// and the extra fast path measured slower than the general path alone).
template <int DIM>
__device__ __forceinline__ int fast_cell(const acc4 &r) {
    if constexpr (DIM < 3) return rec_fast_cell<DIM>(r);
    return -1;
}

// Sampled value of one channel quad (offset xq within the cell) at a record whose fast
// cell is fc (DIM <= 2): every corner cell lies in the window (zeros outside the
// grid), so the plain bilinear formulas apply.
template <int DIM>
__device__ __forceinline__ acc4 window_sample(const WinTiles &wt, const float *xwin, int fc, int xq, const acc4 &r) {
    const float *xc = xwin + fc * XS + xq;
    const float fx = r[DIM - 1] - floorf(r[DIM - 1]);
    auto row = [&](int off) {
        const acc4 x0 = *reinterpret_cast<const acc4 *>(xc + off * XS);
        const acc4 x1 = *reinterpret_cast<const acc4 *>(xc + (off + 1) * XS);
        return (1.f - fx) * x0 + fx * x1;
    };
    if constexpr (DIM == 1) {
        return row(0);
    } else {
        const float fy = r[0] - floorf(r[0]);
        return (1.f - fy) * row(0) + fy * row(wt.WE[2]);
    }
}

template <int DIM, typename T>
__device__ __forceinline__ void fill_geo(const Geo &g, const WinTiles &wt, const Tile &tile, const T *__restrict__ offset,
                                         const T *__restrict__ mask, int t0, int ntaps, acc4 *geo, int tid, int nthreads) {
    const bool deformable = offset != nullptr;
    for (int e = tid; e < ntaps * BPX; e += nthreads) {
        const int tl = e / BPX, i = e % BPX;
        const int p = tile.pixel(g, wt, i);
        acc4 r;
        float mk = 0.f;
        int cell = -1;
#pragma unroll
        for (int a = 0; a < DIM; ++a) r[a] = -4.f;
        if (p >= 0) {
            const Point<DIM, float> pt = sample_point<DIM, float, T>(g, offset, tile.b, p, t0 + tl, tile.ogu);
#pragma unroll
            for (int a = 0; a < DIM; ++a) r[a] = pt.pos[a];
            mk = mask_at<float, T>(g, mask, tile.b, tile.mgu, t0 + tl, p);
            if (DIM < 3 && wt.cells > 0) {
                const AxisW<DIM, float> aw = axis_weights<DIM, float>(g, pt, deformable);
                bool fast = true;
                int lin = 0;
#pragma unroll
                for (int a = 0; a < DIM; ++a) {
                    const int ee = 3 - DIM + a;
                    const int l = aw.lo[a] - tile.org[ee];
                    fast = fast && l >= 0 && l + 1 < wt.WE[ee];
                    lin = lin * wt.WE[ee] + l;
                }
                cell = fast ? lin : -1;
            }
        }
        if constexpr (DIM == 3) {
            r[3] = mk;
        } else {
            if (DIM == 1) r[2] = 0.f;
            r[DIM] = mk;
            r[3] = __int_as_float(cell);
        }
        geo[tl * BPX + i] = r;
    }
}

// Walks window cells first, first + step, ... keeping (lz, ly, lx) incrementally (no
// divisions per cell); f(cell, flat index in the sampled grid or -1 outside it).
template <typename F>
__device__ __forceinline__ void for_cells(const Geo &g, const WinTiles &wt, const Tile &tile, int first, int step, F &&f) {
    int lx = first % wt.WE[2];
    int r = first / wt.WE[2];
    int ly = r % wt.WE[1];
    int lz = r / wt.WE[1];
    const int sx_step = step % wt.WE[2], sy_step = (step / wt.WE[2]) % wt.WE[1], sz_step = step / (wt.WE[2] * wt.WE[1]);
    for (int cell = first; cell < wt.cells; cell += step) {
        const int sz = tile.org[0] + lz, sy = tile.org[1] + ly, sx = tile.org[2] + lx;
        const bool in = sz >= 0 && sz < g.S[0] && sy >= 0 && sy < g.S[1] && sx >= 0 && sx < g.S[2];
        f(cell, in ? (sz * g.S[1] + sy) * g.S[2] + sx : -1);
        lx += sx_step;
        ly += sy_step;
        lz += sz_step;
        if (lx >= wt.WE[2]) {
            lx -= wt.WE[2];
            ++ly;
        }
        if (ly >= wt.WE[1]) {
            ly -= wt.WE[1];
            ++lz;
        }
    }
}

// X window: xwin[cell * XS + 4 * quad .. + 3] = channels c0 + 4 * quad .. of the cell
// (threads take (cell, quad) pairs: nthreads must be a multiple of 4)
__device__ __forceinline__ void fill_xwin(const Geo &g, const WinTiles &wt, const Tile &tile, const float *__restrict__ xb,
                                          float *xwin, int tid, int nthreads) {
    const int qd = tid & 3;
    const bool q_ok = tile.c0 + 4 * qd < g.Cg;
    for_cells(g, wt, tile, tid >> 2, nthreads >> 2, [&](int cell, int si) {
        acc4 v = acc4{0.f, 0.f, 0.f, 0.f};
        if (si >= 0 && q_ok) v = *reinterpret_cast<const acc4 *>(xb + (size_t)si * g.C + 4 * qd);
        *reinterpret_cast<acc4 *>(xwin + cell * XS + 4 * qd) = v;
    });
}

// The sampling geometry of a geo record: the point (integer base for offset-free
// sampling, where the stored position is an exact integer) and its axis weights.
template <int DIM>
__device__ __forceinline__ AxisW<DIM, float> record_weights(const Geo &g, const acc4 &r, bool deformable) {
    Point<DIM, float> pt;
#pragma unroll
    for (int a = 0; a < DIM; ++a) {
        pt.pos[a] = r[a];
        pt.base[a] = (int)r[a];
    }
    return axis_weights<DIM, float>(g, pt, deformable);
}

}  // namespace win
}  // namespace tvdcn_hip
