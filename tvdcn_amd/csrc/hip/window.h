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

// Holds the memory operations issued above it in place: IR-level passes may not move loads
// or stores across it (the empty asm clobbers memory) and neither may the machine scheduler
// (sched_barrier); it waits for nothing. Used after prefetches, which would otherwise be
// sunk next to their first use.
__device__ __forceinline__ void issue_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

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
// when the window is flushed. A record with a fast cell holds the fractional part
// of each position (the high-corner weight) in place of the position; offset-free
// records never get one. Pixels outside
// the grid get position -4 on every axis (no corner inside the grid), mask 0 and no
// fast cell.
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

// mask * sampled value of one channel quad (offset xq within the cell) at a fast
// record (DIM <= 2): every corner cell lies in the window (zeros outside the grid), so
// the plain bilinear formulas apply, with the mask folded into the corner weights.
template <int DIM>
__device__ __forceinline__ acc4 window_sample_masked(const WinTiles &wt, const float *xwin, int fc, int xq,
                                                     const acc4 &r, float mk) {
    const float *xc = xwin + fc * XS + xq;
    const float fx = r[DIM - 1];
    const acc4 x00 = *reinterpret_cast<const acc4 *>(xc);
    const acc4 x01 = *reinterpret_cast<const acc4 *>(xc + XS);
    if constexpr (DIM == 1) {
        const float w1 = mk * fx, w0 = mk - w1;
        return w0 * x00 + w1 * x01;
    } else {
        const acc4 x10 = *reinterpret_cast<const acc4 *>(xc + wt.WE[2] * XS);
        const acc4 x11 = *reinterpret_cast<const acc4 *>(xc + (wt.WE[2] + 1) * XS);
        const float a1 = mk * r[0], a0 = mk - a1;
        const float w01 = a0 * fx, w00 = a0 - w01, w11 = a1 * fx, w10 = a1 - w11;
        return w00 * x00 + w01 * x01 + w10 * x10 + w11 * x11;
    }
}

// Corner geometry of a 3D record (absolute positions) against the tile's window and the
// sampled grid: per axis the low corner, the high-corner weight and whether each of the two
// corner coordinates lies in the window / in the grid. Corner k = (z bit, y bit, x bit) sits at
// window cell cell0 + bz * WE_y * WE_x + by * WE_x + bx and grid index idx0 + bz * S_y * S_x +
// by * S_x + bx. Offset-free sampling (integer positions) has only the low corner.
struct Corners3 {
    float fh[3];
    bool win[3][2], grid[3][2];
    int cell0, idx0;
    bool inside;   // sample range rule: -1 < pos < S on every axis
    __device__ __forceinline__ Corners3(const Geo &g, const WinTiles &wt, const Tile &tile, const acc4 &r,
                                        bool deformable) {
        int lo[3], wl[3];
        inside = true;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float f = floorf(r[a]);
            lo[a] = (int)f;
            fh[a] = deformable ? r[a] - f : 0.f;
            inside = inside && r[a] > -1.f && r[a] < (float)g.S[a];
            wl[a] = lo[a] - tile.org[a];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                win[a][b] = (unsigned)(wl[a] + b) < (unsigned)wt.WE[a];
                grid[a][b] = (unsigned)(lo[a] + b) < (unsigned)g.S[a];
            }
        }
        cell0 = (wl[0] * wt.WE[1] + wl[1]) * wt.WE[2] + wl[2];
        idx0 = (lo[0] * g.S[1] + lo[1]) * g.S[2] + lo[2];
    }
    __device__ __forceinline__ bool in_win(int k) const { return win[0][k >> 2] && win[1][(k >> 1) & 1] && win[2][k & 1]; }
    __device__ __forceinline__ bool in_grid(int k) const {
        return grid[0][k >> 2] && grid[1][(k >> 1) & 1] && grid[2][k & 1];
    }
    __device__ __forceinline__ int cell(const WinTiles &wt, int k) const {
        return cell0 + (k >> 2) * (wt.WE[1] * wt.WE[2]) + ((k >> 1) & 1) * wt.WE[2] + (k & 1);
    }
    __device__ __forceinline__ int idx(const Geo &g, int k) const {
        return idx0 + (k >> 2) * (g.S[1] * g.S[2]) + ((k >> 1) & 1) * g.S[2] + (k & 1);
    }
    // trilinear weight of corner k (product in the reference's axis order)
    __device__ __forceinline__ float weight(int k) const {
        const float wz = (k >> 2) ? fh[0] : 1.f - fh[0];
        const float wy = ((k >> 1) & 1) ? fh[1] : 1.f - fh[1];
        const float wx = (k & 1) ? fh[2] : 1.f - fh[2];
        return wz * wy * wx;
    }
};

// X of one channel quad at corner k: from the window when the corner lies in it (window
// cells outside the grid hold zeros), else from global memory (xgq: the channels-last X of
// the tile's image at the quad's first channel), zero outside the grid. The LDS read is
// unconditional (clamped) and the global read sits in its own branch: the two address
// spaces are never merged into one pointer.
__device__ __forceinline__ acc4 corner_x3(const Geo &g, const WinTiles &wt, const Corners3 &cr, int k, const float *xwin,
                                          int xq, const float *__restrict__ xgq, bool q_ok, bool xglobal = false) {
    const bool iw = !xglobal && cr.in_win(k);
    acc4 x = *reinterpret_cast<const acc4 *>(xwin + (iw ? cr.cell(wt, k) : 0) * XS + xq);
    if (!iw) {
        x = acc4{0.f, 0.f, 0.f, 0.f};
        if (q_ok && cr.in_grid(k)) x = *reinterpret_cast<const acc4 *>(xgq + (size_t)cr.idx(g, k) * g.C);
    }
    return x;
}

// mask * sample of one channel quad at a 3D record: one branch-light path for every lane
// (the 3D windows that fit in LDS have margins of about one cell, so most waves hold some
// lane with a corner outside the window; a separate in-window fast path would run beside
// this one rather than instead of it).
__device__ __forceinline__ acc4 sample3_masked(const Geo &g, const WinTiles &wt, const Tile &tile, const float *xwin,
                                               int xq, const float *__restrict__ xgq, bool q_ok, const acc4 &r,
                                               bool deformable) {
    const Corners3 cr(g, wt, tile, r, deformable);
    acc4 sv = acc4{0.f, 0.f, 0.f, 0.f};
    if (!cr.inside) return sv;
    const float mk = r[3];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k > 0 && !deformable) break;
        sv += (mk * cr.weight(k)) * corner_x3(g, wt, cr, k, xwin, xq, xgq, q_ok);
    }
    return sv;
}

// mask * sample of all 16 channels of the tile's slice at a 3D record: s[j] = channels
// 4j .. 4j + 3 (xgs: the channels-last X of the tile's image at the slice's first channel;
// nq: channel quads of the slice inside the group, 4 when FULLQ). The corner geometry and
// the eight mask-folded weights are formed once for the 16 channels. Window cell wt.cells
// must hold zeros (the zero cell): a corner outside the window reads it, and a corner
// outside the window but inside the grid then overwrites it with the global values.
template <bool FULLQ>
__device__ __forceinline__ void sample3_all(const Geo &g, const WinTiles &wt, const Tile &tile, const float *xwin,
                                            const float *__restrict__ xgs, int nq, const acc4 &r, bool deformable,
                                            acc4 (&s)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = acc4{0.f, 0.f, 0.f, 0.f};
    const Corners3 cr(g, wt, tile, r, deformable);
    if (!cr.inside) return;
    auto corner = [&](int k, float w) {
        const bool iw = cr.in_win(k);
        const float *xc = xwin + (iw ? cr.cell(wt, k) : wt.cells) * XS;
        acc4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = *reinterpret_cast<const acc4 *>(xc + 4 * j);
        if (!iw && cr.in_grid(k)) {
            const float *xp = xgs + (size_t)cr.idx(g, k) * g.C;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (FULLQ || j < nq) x[j] = *reinterpret_cast<const acc4 *>(xp + 4 * j);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += w * x[j];
    };
    const float mk = r[3];
    if (deformable) {
        // mask-folded trilinear weights: (z, y) pairs first, then x
        const float z1 = mk * cr.fh[0], z0 = mk - z1;
        const float zy[4] = {z0 - z0 * cr.fh[1], z0 * cr.fh[1], z1 - z1 * cr.fh[1], z1 * cr.fh[1]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float w1 = zy[j] * cr.fh[2];
            corner(2 * j, zy[j] - w1);
            corner(2 * j + 1, w1);
        }
    } else {
        corner(0, mk);   // offset-free sampling: the low corner only
    }
}

// The corner geometry of Corners3 with the window / grid membership of the eight corners as
// 8-bit lane masks (bit k: corner k) held in a vector register, for the branch-free sampler
// below.
struct Corners3M {
    float fh[3];
    int cell0, idx0;
    unsigned wmask, gmask;
    bool inside;   // sample range rule: -1 < pos < S on every axis
    __device__ __forceinline__ Corners3M(const Geo &g, const WinTiles &wt, const Tile &tile, const acc4 &r,
                                         bool deformable) {
        // corners whose axis-a bit is 0 (the low corner of the axis)
        constexpr unsigned LOW[3] = {0x0Fu, 0x33u, 0x55u};
        int lo[3], wl[3];
        inside = true;
        unsigned wm = 0xFFu, gm = 0xFFu;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float f = floorf(r[a]);
            lo[a] = (int)f;
            fh[a] = deformable ? r[a] - f : 0.f;
            inside = inside && r[a] > -1.f && r[a] < (float)g.S[a];
            wl[a] = lo[a] - tile.org[a];
            const unsigned hi = 0xFFu ^ LOW[a];
            wm &= ((unsigned)wl[a] < (unsigned)wt.WE[a] ? 0xFFu : hi) & ((unsigned)(wl[a] + 1) < (unsigned)wt.WE[a] ? 0xFFu : LOW[a]);
            gm &= ((unsigned)lo[a] < (unsigned)g.S[a] ? 0xFFu : hi) & ((unsigned)(lo[a] + 1) < (unsigned)g.S[a] ? 0xFFu : LOW[a]);
        }
        wmask = wm;
        gmask = gm;
        cell0 = (wl[0] * wt.WE[1] + wl[1]) * wt.WE[2] + wl[2];
        idx0 = (lo[0] * g.S[1] + lo[1]) * g.S[2] + lo[2];
    }
    __device__ __forceinline__ int cell(const WinTiles &wt, int k) const {
        return cell0 + (k >> 2) * (wt.WE[1] * wt.WE[2]) + ((k >> 1) & 1) * wt.WE[2] + (k & 1);
    }
    __device__ __forceinline__ int idx(const Geo &g, int k) const {
        return idx0 + (k >> 2) * (g.S[1] * g.S[2]) + ((k >> 1) & 1) * g.S[2] + (k & 1);
    }

};

// sample3_all with every corner read from the window without a branch -- a corner outside it
// reads window cell wt.cells, which must hold zeros (the zero cell) -- and the corners inside the
// grid but outside the window added from global memory afterwards (a sample outside the range
// rule reads zero cells only, whatever its mask). Fewer registers than sample3_all; measured
// faster for the weight gradient's S tiles, slower for the forward's B fragments.
template <bool FULLQ>
__device__ __forceinline__ void sample3_all_fix(const Geo &g, const WinTiles &wt, const Tile &tile, const float *xwin,
                                                const float *__restrict__ xgs, int nq, const acc4 &r, bool deformable,
                                                acc4 (&s)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = acc4{0.f, 0.f, 0.f, 0.f};
    const Corners3M cr(g, wt, tile, r, deformable);
    const unsigned wm = cr.inside ? cr.wmask : 0u;
    auto corner = [&](int k, float w) {
        const float *xc = xwin + (((wm >> k) & 1u) ? cr.cell(wt, k) : wt.cells) * XS;
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += w * *reinterpret_cast<const acc4 *>(xc + 4 * j);
    };
    // (a sample outside the range rule is zero whatever its mask)
    const float mk = cr.inside ? r[3] : 0.f;
    float wk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (deformable) {
        // mask-folded trilinear weights: (z, y) pairs first, then x
        const float z1 = mk * cr.fh[0], z0 = mk - z1;
        const float zy[4] = {z0 - z0 * cr.fh[1], z0 * cr.fh[1], z1 - z1 * cr.fh[1], z1 * cr.fh[1]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wk[2 * j + 1] = zy[j] * cr.fh[2];
            wk[2 * j] = zy[j] - wk[2 * j + 1];
            corner(2 * j, wk[2 * j]);
            corner(2 * j + 1, wk[2 * j + 1]);
        }
    } else {
        wk[0] = mk;
        corner(0, mk);   // offset-free sampling: the low corner only
    }
    // corners in the grid, outside the window (an offset-free sample has only its low corner), in
    // batches of four: a batch's global loads are all issued before any is used
    const unsigned om = cr.inside ? cr.gmask & ~cr.wmask & (deformable ? 0xFFu : 1u) : 0u;
    constexpr int NB = 4;
#pragma unroll
    for (int h = 0; h < 8 / NB; ++h) {
        if ((om >> (NB * h)) & ((1u << NB) - 1u)) {
            acc4 xo[NB][4];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int k = NB * h + b;
#pragma unroll
                for (int j = 0; j < 4; ++j) xo[b][j] = acc4{0.f, 0.f, 0.f, 0.f};
                if ((om >> k) & 1u) {
                    const float *xp = xgs + (size_t)cr.idx(g, k) * g.C;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (FULLQ || j < nq) xo[b][j] = *reinterpret_cast<const acc4 *>(xp + 4 * j);
                }
            }
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[j] += wk[NB * h + b] * xo[b][j];
        }
    }
}

// 4 x 4 transpose of 16-byte blocks across the four 16-lane rows of the wave: on return,
// row r's block c holds what row c held in block r. Two stages of row swaps (gfx950
// v_permlane32_swap: rows 2, 3 of the first operand <-> rows 0, 1 of the second;
// v_permlane16_swap: odd rows of the first <-> even rows of the second).
__device__ __forceinline__ void transpose_rows4(acc4 (&b)[4]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(b[c][v]), __float_as_uint(b[c + 2][v]),
                                                            false, false);
            b[c][v] = __uint_as_float(p[0]);
            b[c + 2][v] = __uint_as_float(p[1]);
        }
#pragma unroll
    for (int c = 0; c < 4; c += 2)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[c][v]), __float_as_uint(b[c + 1][v]),
                                                            false, false);
            b[c][v] = __uint_as_float(p[0]);
            b[c + 1][v] = __uint_as_float(p[1]);
        }
}

// RPT = records per thread per batch (WIN_TMAX * BPX / 512 = 4.5: one batch at 5); a
// caller short of registers passes fewer. mscale (a power of two) multiplies every record's
// mask, after its activation: a caller whose sampled values are wanted at a scale folds it in
// here, once per record, rather than once per sampled value. NORM_LDS: a softmax mask's normaliser
// is formed from the records when the pass holds every tap (below).
template <int DIM, typename T, int RPT = 5, bool NORM_LDS = false>
__device__ __forceinline__ void fill_geo(const Geo &g, const WinTiles &wt, const Tile &tile, const T *__restrict__ offset,
                                         const T *__restrict__ mask, int t0, int ntaps, acc4 *geo, int tid, int nthreads,
                                         float mscale = 1.f) {
    // records e = tid, tid + nthreads, ...: every global load of a batch is issued
    // before any is consumed (one memory latency per batch, not one per record)
    const bool deformable = offset != nullptr;
    const int n = ntaps * BPX;
    for (int e0 = 0; e0 < n; e0 += RPT * nthreads) {
        int pv[RPT];
        float ov[RPT][DIM], mv[RPT];
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int e = e0 + tid + j * nthreads;
            const int tl = e / BPX, i = e % BPX;
            const int p = e < n ? tile.pixel(g, wt, i) : -1;
            pv[j] = p;
            mv[j] = 0.f;
#pragma unroll
            for (int a = 0; a < DIM; ++a) ov[j][a] = 0.f;
            if (p >= 0) {
                const int t = t0 + tl;
                if (deformable) {
                    const T *o = offset + ((size_t)(tile.b * g.og + tile.ogu) * g.Kn + t) * DIM * (size_t)g.Pn + p;
#pragma unroll
                    for (int a = 0; a < DIM; ++a) ov[j][a] = to_acc<float>(o[(size_t)a * g.Pn]);
                }
                mv[j] = mask_raw<float, T>(g, mask, tile.b, tile.mgu, t, p);
            }
        }
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int e = e0 + tid + j * nthreads;
            if (e >= n) continue;
            const int tl = e / BPX, i = e % BPX;
            const int p = pv[j];
            acc4 r;
            float mk = 0.f;
            int cell = -1;
#pragma unroll
            for (int a = 0; a < DIM; ++a) r[a] = -4.f;
            if (p >= 0) {
                int kk[DIM], pp[DIM];
                decompose_tap<DIM>(g, t0 + tl, kk);
                decompose_pix<DIM>(g, p, pp);
                Point<DIM, float> pt;
#pragma unroll
                for (int a = 0; a < DIM; ++a) {
                    const int ee = 3 - DIM + a;
                    pt.base[a] = pp[a] * g.st[ee] - g.pad[ee] + kk[a] * g.dil[ee];
                    pt.pos[a] = round_position<T, float>((float)pt.base[a] + ov[j][a]);
                    r[a] = pt.pos[a];
                }
                // (an activated mask is scaled after its activation, below)
                mk = mask != nullptr && g.mask_act != 0 ? mv[j] : mv[j] * mscale;
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
                    // offset-free sampling never takes the fast paths: its integer sampling reads
                    // the low corner only (a high corner, even at weight 0, must not be touched,
                    // so that a non-finite value there cannot leak in)
                    fast = fast && deformable;
                    cell = fast ? lin : -1;
                    // fast records keep only the fractional part of each position
                    // (the high-corner weight): the fast paths need nothing else
                    if (fast) {
#pragma unroll
                        for (int a = 0; a < DIM; ++a) r[a] = aw.fh[a];
                    }
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
    // mask logits: the thread activates the masks of its own records in a separate pass, so
    // that the loops above keep their code when masks are plain values. The softmax takes a
    // pixel per thread: the normaliser over all Kn taps (also those outside this pass) is
    // formed once and applied to the pixel's records of the pass. Records of pixels outside
    // the grid keep mask 0.
    if (mask != nullptr && g.mask_act == MASK_ACT_SIGMOID) {
        for (int e = tid; e < n; e += nthreads) {
            if (tile.pixel(g, wt, e % BPX) < 0) continue;
            float *m = reinterpret_cast<float *>(geo + e) + (DIM == 3 ? 3 : DIM);
            *m = mask_activate<float>(g, *m) * mscale;
        }
    } else if (mask != nullptr && g.mask_act == MASK_ACT_SOFTMAX) {
        // a pixel's records of the pass were written by other threads (record e belongs to
        // thread e mod nthreads): every caller runs fill_geo with the whole workgroup, under
        // uniform control flow
        __syncthreads();
        // (NORM_LDS) a pass of every tap holds all of a pixel's logits in its records: the
        // normaliser is formed from them, with the operations of mask_softmax_norm in its order
        // (the same values), instead of from global memory (the logits loaded again, paid per
        // tile: cfg3's weight gradient, 64 tiles per workgroup, -5.5%; the data gradient, one
        // tile per workgroup, measured 2.7% slower with it, and keeps the loads)
        const bool all_taps = NORM_LDS && t0 == 0 && ntaps == g.Kn;
        auto logit = [&](int tl, int i) {
            return reinterpret_cast<const float *>(geo + tl * BPX + i)[DIM == 3 ? 3 : DIM];
        };
        for (int i = tid; i < BPX; i += nthreads) {
            const int p = tile.pixel(g, wt, i);
            if (p < 0) continue;
            float mx, inv;
            if (all_taps) {
                mx = -INFINITY;
                for (int tl = 0; tl < ntaps; ++tl) {
                    const float v = logit(tl, i);
                    mx = v > mx ? v : mx;
                }
                float sum = 0.f;
                for (int tl = 0; tl < ntaps; ++tl) sum += exp(logit(tl, i) - mx);
                inv = 1.f / sum;
            } else {
                mask_softmax_norm<float, T>(g, mask, tile.b, tile.mgu, p, mx, inv);
            }
            for (int tl = 0; tl < ntaps; ++tl) {
                float *m = reinterpret_cast<float *>(geo + tl * BPX + i) + (DIM == 3 ? 3 : DIM);
                *m = expf(*m - mx) * inv * mscale;
            }
        }
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
// (threads take (cell, quad) pairs: nthreads must be a multiple of 4). Loads go out in
// batches of XB per thread before any is stored.
__device__ __forceinline__ void fill_xwin(const Geo &g, const WinTiles &wt, const Tile &tile, const float *__restrict__ xb,
                                          float *xwin, int tid, int nthreads) {
    constexpr int XB = 8;
    const int qd = tid & 3;
    const bool q_ok = tile.c0 + 4 * qd < g.Cg;
    const int step = nthreads >> 2;
    const int first = tid >> 2;
    // cell walker (no divisions per cell): (lz, ly, lx) of `cell`
    int lx = first % wt.WE[2];
    int rr = first / wt.WE[2];
    int ly = rr % wt.WE[1];
    int lz = rr / wt.WE[1];
    const int sx_step = step % wt.WE[2], sy_step = (step / wt.WE[2]) % wt.WE[1], sz_step = step / (wt.WE[2] * wt.WE[1]);
    for (int c0 = first; c0 < wt.cells; c0 += XB * step) {
        acc4 v[XB];
#pragma unroll
        for (int j = 0; j < XB; ++j) {
            const int cell = c0 + j * step;
            const int sz = tile.org[0] + lz, sy = tile.org[1] + ly, sx = tile.org[2] + lx;
            const bool in = cell < wt.cells && q_ok && sz >= 0 && sz < g.S[0] && sy >= 0 && sy < g.S[1] && sx >= 0 &&
                            sx < g.S[2];
            v[j] = acc4{0.f, 0.f, 0.f, 0.f};
            if (in) v[j] = *reinterpret_cast<const acc4 *>(xb + (size_t)((sz * g.S[1] + sy) * g.S[2] + sx) * g.C + 4 * qd);
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
#pragma unroll
        for (int j = 0; j < XB; ++j) {
            const int cell = c0 + j * step;
            if (cell < wt.cells) *reinterpret_cast<acc4 *>(xwin + cell * XS + 4 * qd) = v[j];
        }
    }
}

// Absolute sampling positions of a record: a fast record holds fractional parts, whose
// integer parts follow from its cell (lo = window origin + cell coordinates).
template <int DIM>
__device__ __forceinline__ acc4 record_position(const WinTiles &wt, const Tile &tile, acc4 r) {
    const int fc = rec_fast_cell<DIM>(r);
    if (DIM < 3 && fc >= 0) {
        const int lx = fc % wt.WE[2];
        if constexpr (DIM == 1) {
            r[0] += (float)(tile.org[2] + lx);
        } else {
            r[0] += (float)(tile.org[1] + fc / wt.WE[2]);
            r[1] += (float)(tile.org[2] + lx);
        }
    }
    return r;
}

// The sampling geometry of a record holding absolute positions (see record_position):
// the point (integer base for offset-free sampling, where the stored position is an
// exact integer) and its axis weights.
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


// ---------------------------------------------------------------------------
// 16-bit MFMA operands. v_mfma_f32_16x16x32_f16 / _bf16: lane l supplies K = 8 (l / 16) ..
// + 7 of row (A) / column (B) l % 16 as eight 16-bit values in four dwords (the lower K in
// the low half); the 16x16 result has the layout of the 16x16x4 fp32 MFMA. fp32 operands
// go in as two fp16 pieces each, of the value scaled by a power of two 2^s that puts the
// operand's largest magnitude in [2^14, 2^15): p0 = fp16(v 2^s), p1 = fp16(v 2^s - p0) (nearest,
// ties to even; the residual is exact in fp32), so v 2^s = p0 + p1 + r with |r| <= 2^-23 |v 2^s|
// while p1 stays a normal fp16 (|v| >= 2^-17 of the operand's largest; below that the error is
// at most 2^-25 of a unit, 2^-40 of the largest). Of the four cross products p_i q_j the three
// with i + j <= 1 are summed (exact products, fp32 accumulation); the one left out (|p1 q1| <=
// 2^-22 |v w|) and the residuals' terms (<= 2^-23 |v w| each) stay below 2^-21 |v w|, the
// rounding fp32 itself accumulates over a few multiply-adds; the sum is scaled back by
// 2^-(s_a + s_b). An fp32 value is bad for this (split_bad) when it is not finite or at least
// 0x1.ffp127 in magnitude; fp16 / bf16 operands go in as they are.
// ---------------------------------------------------------------------------
template <typename T> constexpr int npiece_of() { return std::is_same<T, float>::value ? 2 : 1; }

__device__ __forceinline__ bool split_bad(float v) {
    return (__float_as_uint(v) & 0x7FFFFFFFu) >= 0x7F7F8000u;
}

// Largest magnitudes of the fp32 path's operands (float bits, raised with atomicMax: non-negative
// floats order as their bit patterns), in the words after the operand flag (kernels.h: amax_word)
enum { AMAX_W = AMAX_SLOT_W, AMAX_X = AMAX_SLOT_X, AMAX_M = AMAX_SLOT_M, AMAX_Z = AMAX_SLOT_Z };
// the largest of a slot's sub-slots; every lane of the wave calls it (each loads one sub-slot)
__device__ __forceinline__ float operand_amax(const int *flag, int slot) {
    static_assert(AMAX_SPREAD == 64, "one sub-slot per lane");
    const unsigned *w = reinterpret_cast<const unsigned *>(flag);
    float m = __uint_as_float(w[amax_word(slot, threadIdx.x & 63)]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    return m;
}
// e with |v| < 2^e for every value of a magnitude bound a (0 for a zero, non-finite or absent bound)
__device__ __forceinline__ int bound_exp(float a) {
    int e = 0;
    if (a > 0.f && a <= 3.402823466e38f) frexpf(a, &e);   // a < 2^e
    return e;
}
// scale exponent of an operand whose values lie below 2^e: the largest lands in [2^14, 2^15)
__device__ __forceinline__ int piece_scale(int e) { return 15 - e; }
// the sampled operand mask * bilinear(X): below (largest |X|) x (largest |mask|): the mask's bound
// is its tensor's largest value, mask_scale (sigmoid) or 1 (softmax, no mask). Every lane of the
// wave calls it.
__device__ __forceinline__ int sampled_scale(const Geo &g, const int *flag, bool has_mask) {
    if (flag == nullptr) return 0;
    const float mm = operand_amax(flag, AMAX_M);
    const float mbound = !has_mask ? 1.f
                         : g.mask_act == MASK_ACT_SIGMOID ? (float)g.mask_scale
                         : g.mask_act == MASK_ACT_SOFTMAX ? 1.f
                                                          : mm;
    return piece_scale(bound_exp(operand_amax(flag, AMAX_X)) + bound_exp(mbound));
}
// every lane of the wave calls it
__device__ __forceinline__ int operand_scale(const int *flag, int slot) {
    return flag == nullptr ? 0 : piece_scale(bound_exp(operand_amax(flag, slot)));
}

// a - (float)h, h the low (HI = false) or high half of the fp16 pair w: one v_fma_mix_f32
// (-h * 1 + a, its fp16 operand taken as it is, so exactly the subtraction a - (float)h)
// where the compiler forms two conversions back to fp32 and two subtractions per pair
template <bool HI> __device__ __forceinline__ float sub_half(float a, uint32_t w) {
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(a));
    else
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(a));
    return r;
}

// two values as their fp16 pieces at scale 2^s, packed two per dword: hi = RN16(v), lo =
// RN16(v - hi)
__device__ __forceinline__ void split2_pk(float a, float b, int s, uint32_t (&w)[2]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    a = ldexpf(a, s);
    b = ldexpf(b, s);
    w[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, h2));
    const f2 r = {sub_half<false>(a, w[0]), sub_half<true>(b, w[0])};
    w[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, h2));
}

// two values rounded to the 16-bit type T (fp16 or bf16), packed
template <typename T> __device__ __forceinline__ uint32_t pack2_16(float a, float b) {
    if constexpr (std::is_same<T, __half>::value) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 h = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, h);
    } else {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        const b2 h = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, h);
    }
}

// one value as its NP 16-bit pieces at scale 2^s (fp32) or as T (fp16 / bf16; s unused)
template <typename T, int NP>
__device__ __forceinline__ void split_one16(float v, int s, uint16_t (&p)[NP]) {
    static_assert(NP == npiece_of<T>(), "pieces per value of T");
    if constexpr (NP == 2) {
        v = ldexpf(v, s);
        p[0] = __builtin_bit_cast(uint16_t, (_Float16)v);
        p[1] = __builtin_bit_cast(uint16_t, (_Float16)sub_half<false>(v, p[0]));
    } else if constexpr (std::is_same<T, __half>::value) {
        p[0] = __builtin_bit_cast(uint16_t, (_Float16)v);
    } else {
        p[0] = __builtin_bit_cast(uint16_t, (__bf16)v);
    }
}

// eight values of a lane as NP 16-bit operand fragments (pieces at scale 2^s for fp32, T's
// values otherwise)
template <typename T, int NP>
__device__ __forceinline__ void pack8_16(const float (&v)[8], int s, uint4 (&out)[NP]) {
    static_assert(NP == npiece_of<T>(), "pieces per value of T");
    uint32_t w[NP][4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        if constexpr (NP == 2) {
            uint32_t p[2];
            split2_pk(v[e], v[e + 1], s, p);
            w[0][e >> 1] = p[0];
            w[1][e >> 1] = p[1];
        } else {
            w[0][e >> 1] = pack2_16<T>(v[e], v[e + 1]);
        }
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) out[k] = uint4{w[k][0], w[k][1], w[k][2], w[k][3]};
}

// D += A * B on one 16x16x32 MFMA: fp16 operands for T = fp16 and for the pieces of fp32, bf16
// otherwise
template <typename T> __device__ __forceinline__ f32x4 mfma16x16x32(uint4 a, uint4 b, f32x4 c) {
    if constexpr (std::is_same<T, __half>::value || std::is_same<T, float>::value) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
    } else {
        typedef __bf16 b8 __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0,
                                                        0);
    }
}

// acc += the split product of A and B fragments (NP pieces each): the three products with
// i + j <= 1, smallest first, for fp32; the one product otherwise
template <typename T, int NP>
__device__ __forceinline__ f32x4 mfma16x16x32_np(const uint4 (&a)[NP], const uint4 (&b)[NP], f32x4 c) {
    static_assert(NP == npiece_of<T>(), "pieces per value of T");
    if constexpr (NP == 2) {
        c = mfma16x16x32<T>(a[1], b[0], c);
        c = mfma16x16x32<T>(a[0], b[1], c);
    }
    return mfma16x16x32<T>(a[0], b[0], c);
}

}  // namespace win
}  // namespace tvdcn_hip
