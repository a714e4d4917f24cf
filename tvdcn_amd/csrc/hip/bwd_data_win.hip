// Family D, windowed variant: grad-columns on MFMA with the bilinear scatter
// pre-accumulated in an LDS window of the sampled grid.
//
//   G[c][t][p] = sum_{m in group} W[m][c][t] * Z[b][m][p]             (MFMA, never stored)
//   SCATTER: dX[b][s][c] += w_corner(s) * mask * G                       (bilinear insert)
//   COORD:   dOffset[b][og][t][a][p] += mask * G * d(sample)/d(pos_a)    (summed over c in og)
//            dMask[b][mg][t][p]      += G * sample                        (summed over c in mg)
//
// Replaces the reference's grad-columns addmm_ + col2im + compute_grad_offset +
// compute_grad_mask per batch block (tvdcn/csrc/ops/cuda/deform_conv2d_kernel.cpp:518-598,
// kernels deform_conv2d_common_kernels.cu:258-624, and the 1D/3D twins).
//
// Workgroup = one tile: a box of 256 column pixels of one image (16x16 in 2D,
// 256 in 1D, 4x8x8 in 3D) x 16 sampled-side channels x every tap; eight waves
// (two per SIMD, so one wave's loads overlap the other's MFMAs), each owning 32
// pixels; one workgroup per CU (the window takes most of the 160 KB of LDS).
//   * K loop over the GEMM-side channels m, operands straight from global memory
//     into registers (the next step's prefetched while the MFMAs of the current one
//     run): wave w computes Gt[c][px] for its 32 pixels, so each lane holds four
//     consecutive channels of one pixel per (tap, 16-pixel block). It runs on
//     16x16x32 MFMAs, 32 channels per step, from 16-bit operands laid out by
//     data_prep_kernel (Z and weight splits, one launch): fp16 and bf16 tensors as they are, fp32
//     tensors as two fp16 pieces each at a per-tensor power-of-two scale, of whose four cross
//     products the three with i + j <= 1 are summed (the rest are within fp32's own rounding;
//     3 MFMAs at 16 cycles against 8 fp32 16x16x4 MFMAs at 32 cycles per 32 channels), the
//     sums scaled back after the K loop. An fp32 operand that is not finite (or at least
//     0x1.ffp127 in magnitude: a device flag set by the layout kernels) sends the launch down
//     the fp32 loop (16x16x4 MFMAs, 16 channels per step), which keeps the reference's inf/nan
//     propagation.
//   * Epilogue per tap: the geometry of the 256 pixels (one per thread) goes to an
//     LDS table. The offset/mask gradients are formed in the MFMA layout (4
//     channels in-lane, two shuffles across the channel quads, one atomic per
//     pixel and quantity).
//   * The scatter accumulates in the LDS window in 32-bit fixed point with
//     integer LDS atomics (ds_add_u32 measured at ~5 cycles per wave instruction
//     on gfx950, ds_add_f32 at ~190). Channel c uses the scale 2^s_c,
//     s_c = 29 - ceil(log2 B_c), B_c = sum of |G * mask| over every (pixel, tap)
//     accumulated so far: a bilinear corner weight is at most 1 and each (pixel,
//     tap) reaches a cell through at most one corner, so every cell sum stays
//     below 2^29 (no overflow); each term is rounded to the unit 2^-s_c <= 2^-28 B_c.
//     Integer sums are also order independent. When a pass of taps grows B_c,
//     the values already held are shifted down to the new scale (rounded to
//     nearest). The unit is relative to the tile's bound, not to each cell, so
//     terms |G * mask| above 2^6 times the typical term of their (pass, channel)
//     (gradient spikes: the bound would be theirs, and the quiet cells of the tile
//     would be rounded at it) bypass the window: they go to global float atomics,
//     and the bound covers the terms that stay. The typical term is 2 to the mean
//     binary exponent of the 128 per-lane mean terms (a geometric mean, which a
//     minority of spikes barely moves: each lane holds 2 pixels x the pass's taps).
//     In 3D a pass with spikes does not use the window. Neither does a pass with a
//     non-finite bound (inf/nan must propagate as in the reference): it goes to
//     global float atomics, after the window flushes what it holds.
//     Corners outside the window go to global float atomics.
//   * The window (sampled-grid box around the tile's undeformed footprint plus a
//     margin R per axis) accumulates over all passes of the tile and is flushed
//     once: one float atomic per non-zero (cell, channel), 16 consecutive channels
//     per cell.
#include "window.h"

namespace tvdcn_hip {
namespace {

using namespace win;

constexpr int NW = 8;             // waves per workgroup (two per SIMD)
constexpr int NT = 64 * NW;       // threads per workgroup
constexpr int PB = 2;             // 16-pixel blocks per wave (NW * PB * 16 = BPX)
constexpr int BM = 16;            // GEMM-side channels per K step
// Fixed-point window: channel-major [16 c][cst], cst = window cells rounded so that
// cst = 4 (mod 16). A scatter instruction's lanes are 16 pixels x 4 channel quads; the
// pixels of a 16-pixel block hit neighbouring cells, and the four channels c, c + 4, c + 8,
// c + 12 of one instruction sit 4 * cst = 16 (mod 64) words apart, so the lanes spread
// over distinct LDS banks (a cell-major [cell][17] layout put lanes of different pixels
// on the same banks).
__host__ __device__ constexpr int fix_stride(int cells) { return ((cells + 11) & ~15) + 4; }
constexpr int FIX_BITS = 29;      // fixed-point headroom: |cell sum| * 2^s_c < 2^29
// Scatter-only plans (transposed forward; the scatter launch of a split conv backward): the unit
// follows the largest term the window keeps, |term| * 2^s_c < 2^PREC_BITS, and the cells sum
// modulo 2^32. An add whose returned old value lies outside [-WRAP_K, WRAP_K) may have wrapped
// (|add| <= 2^PREC_BITS < 2^31 - WRAP_K); a wrap found there sends the wrapped 2^32 units to
// global memory, so the held value plus what went out stays the exact integer sum.
constexpr int PREC_BITS = 26;
constexpr unsigned WRAP_K = 0x78000000u;   // 2^31 - 2^27
static_assert(NW * PB * 16 == BPX, "one tile of pixels per workgroup");
static_assert(NT == BC * 32, "window rescale: 32 threads per channel");

// LDS words ahead of the windows: geometry table [WIN_TMAX][BPX] x (position, mask),
// per-wave channel bounds, scale exponents and flags, held bounds, rescale shifts (or
// spike thresholds), largest terms, exponent statistics
constexpr int GEO_WORDS = WIN_TMAX * BPX * 4;
constexpr int FIXED_WORDS = GEO_WORDS + NW * BC + 5 * BC + 4;
// a term above 2^SPIKE_BITS x 2^(mean exponent of the per-lane mean terms of its pass) is a spike
constexpr int SPIKE_BITS = 6;

// Offset / mask gradient terms of one (pixel, tap) as the reference's corner sums, from
// gk[k] = G contracted with X at corner k (k = 2 * y bit + x bit in 2D, x bit in 1D):
// q[a] = mk * d(sample)/d(pos_a), q[DIM] = sample
template <int DIM>
__device__ __forceinline__ void coord_direct(const float *gk, float fy, float fx, float mk, float *q) {
    if constexpr (DIM == 2) {
        const float gy = -(1.f - fx) * gk[0] - fx * gk[1] + (1.f - fx) * gk[2] + fx * gk[3];
        const float gx = -(1.f - fy) * gk[0] + (1.f - fy) * gk[1] - fy * gk[2] + fy * gk[3];
        q[0] = mk * gy;
        q[1] = mk * gx;
        q[2] = (1.f - fy) * (1.f - fx) * gk[0] + (1.f - fy) * fx * gk[1] + fy * (1.f - fx) * gk[2] + fy * fx * gk[3];
    } else {
        q[0] = mk * (-gk[0] + gk[1]);
        q[1] = (1.f - fx) * gk[0] + fx * gk[1];
    }
}

// Nearest integer, halves rounded up (v_cvt_rpi_i32_f32 = floor(x + 0.5)): one instruction
// where round-to-nearest-even takes two; |x| < 2^29 here
__device__ __forceinline__ int fixed_round(float x) {
    int r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// 2^32 units of scale 2^s in the direction of the add v when old + v wrapped past +-2^31, else 0
__device__ __forceinline__ float wrap_spill(unsigned old, int v, int s) {
    const unsigned nw = old + (unsigned)v;
    if ((int)((old ^ nw) & ((unsigned)v ^ nw)) >= 0) return 0.f;
    return ldexpf(v > 0 ? 1.f : -1.f, 32 - s);
}

// Sum over the four 16-lane rows of the wave (lanes l, l ^ 16, l ^ 32, l ^ 48), every lane
// receiving the total: two row swaps (gfx950 v_permlane16/32_swap) instead of LDS shuffles
__device__ __forceinline__ float row_sum4(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Z (B, G * Mg, Pn) -> zs [B][G][ms32][NP][Pn][32]: per 32-channel step and piece, every pixel's
// 32 channels (zero past Mg) as 4 lane groups of 8 (the 16x16x32 B-operand layout), so that a
// wave's fragment load of one piece for 16 consecutive pixels reads 1 KB of whole lines.
// Block = 64 pixels of one (image, group, step), transposed through LDS.
// (zvec: Pn % 4 == 0 and z aligned to 4 elements: the tile is read in 4-pixel vectors)
template <typename T, int NP>
__device__ __forceinline__ void z_split_block(long long bid, float *smem, const T *__restrict__ z,
                                              uint16_t *__restrict__ zs, uint16_t *__restrict__ zw, int *flag, int G,
                                              int Mg, int Pn, int ms32, int pblocks, bool zvec, size_t zw_plane) {
    float(*tile)[65] = reinterpret_cast<float(*)[65]>(smem);   // [32][65]
    const int sz = NP == 2 ? operand_scale(flag, AMAX_Z) : 0;   // (every lane: before any returns)
    // (the block index is a grid index: 32-bit division, not the 64-bit sequence)
    const unsigned ub = (unsigned)bid;
    const int pb = (int)(ub % (unsigned)pblocks);
    const unsigned bgs = ub / (unsigned)pblocks;   // (b * G + grp) * ms32 + step
    const int st = (int)(bgs % (unsigned)ms32);
    const unsigned bg = bgs / (unsigned)ms32;
    const int grp = (int)(bg % (unsigned)G);
    const unsigned b = bg / (unsigned)G;
    const int p0 = pb * 64;
    const T *src = z + ((size_t)b * G + grp) * (size_t)Mg * Pn;
    if (zvec) {
        for (int i = threadIdx.x; i < 32 * 16; i += 256) {
            const int ml = i >> 4, pl = 4 * (i & 15);
            const int m = st * 32 + ml, p = p0 + pl;
            Vec4<float> v{0.f, 0.f, 0.f, 0.f};
            if (m < Mg && p < Pn) v = load4_t<float, T>(src + (size_t)m * Pn + p);   // all four inside
            tile[ml][pl] = v.x;
            tile[ml][pl + 1] = v.y;
            tile[ml][pl + 2] = v.z;
            tile[ml][pl + 3] = v.w;
        }
    } else {
        for (int i = threadIdx.x; i < 32 * 64; i += 256) {
            const int ml = i >> 6, pl = i & 63;
            const int m = st * 32 + ml, p = p0 + pl;
            float v = 0.f;
            if (m < Mg && p < Pn) v = to_acc<float>(src[(size_t)m * Pn + p]);
            tile[ml][pl] = v;
        }
    }
    __syncthreads();
    if (zw != nullptr) {
        // the same values for the weight gradient, in 8-pixel column blocks: element (image b, row
        // m of Z's M, pixel p) at ((b * Pn / 8 + p / 8) * M + m) * 8 + p % 8 of each piece's plane
        // (Pn % 8 == 0), so that a wave's A fragment (16 rows x 4 blocks of 8 pixels) reads whole
        // lines. Thread = (row ml, 8-pixel block px / 8): consecutive threads, consecutive rows.
        const int ml = threadIdx.x & 31, px = 8 * (threadIdx.x >> 5);
        const int m = st * 32 + ml, pw = p0 + px;
        if (m < Mg && pw < Pn) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = tile[ml][px + e];
            uint4 out[NP];
            pack8_16<T, NP>(v, sz, out);
            const size_t M = (size_t)G * Mg;
            uint16_t *dst = zw + ((size_t)b * (Pn / 8) + pw / 8) * M * 8 + ((size_t)grp * Mg + m) * 8;
#pragma unroll
            for (int k = 0; k < NP; ++k) *reinterpret_cast<uint4 *>(dst + k * zw_plane) = out[k];
        }
    }
    const int pl = threadIdx.x >> 2, q = threadIdx.x & 3, p = p0 + pl;
    if (p >= Pn) return;
    float v[8];
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[e] = tile[q * 8 + e][pl];
        bad = bad || split_bad(v[e]);
    }
    uint4 out[NP];
    pack8_16<T, NP>(v, sz, out);
    uint16_t *dst = zs + ((size_t)bgs * NP * Pn + p) * 32 + q * 8;
#pragma unroll
    for (int k = 0; k < NP; ++k) *reinterpret_cast<uint4 *>(dst + (size_t)k * Pn * 32) = out[k];
    if (NP == 2 && bad) atomicOr(flag, 1);
}

// Reduction over each row of 16 lanes (the lanes of one channel quad's 16 pixels), the
// result in every lane of the row: DPP quad xor 1, quad xor 2, half-row mirror, row
// mirror (VALU only; a shuffle goes through the LDS crossbar)
template <typename F>
__device__ __forceinline__ unsigned row_reduce16(unsigned v, F op) {
    v = op(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true));
    v = op(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true));
    v = op(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, true));
    return op(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_sum16(float v) {
    return __uint_as_float(row_reduce16(__float_as_uint(v), [](unsigned a, unsigned b) {
        return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
    }));
}
__device__ __forceinline__ float row_max16(float v) {
    return __uint_as_float(row_reduce16(__float_as_uint(v), [](unsigned a, unsigned b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}
__device__ __forceinline__ unsigned row_sum16(unsigned v) {
    return row_reduce16(v, [](unsigned a, unsigned b) { return a + b; });
}

template <int DIM, typename T, bool SCATTER, bool COORD>
__global__ void __launch_bounds__(NT)
bwd_data_win_kernel(const Geo g, const WinTiles wt, const T *z, const float *wchunks, const uint16_t *zs,
                    const uint16_t *wsplit, const int *flag, const float *__restrict__ xcl,
                    const T *__restrict__ offset, const T *__restrict__ mask, float *__restrict__ gx_cl,
                    float *__restrict__ goff, float *__restrict__ gmask, const int gx_nchw) {
    constexpr int NC = 1 << DIM;
    constexpr int TMAX = WIN_TMAX;
    // scatter-only: the unit follows the largest kept term, cells sum modulo 2^32 (PREC_BITS)
    constexpr bool PREC = SCATTER && !COORD;

    extern __shared__ float smem[];
    acc4 *geo = reinterpret_cast<acc4 *>(smem);                // [TMAX][BPX] sampling table (window.h)
    float *bsum = smem + GEO_WORDS;                            // [NW][BC] partial bounds
    int *scl = reinterpret_cast<int *>(bsum + NW * BC);        // [BC] scale exponents, then the non-finite
                                                               // flag [BC] and the spike flag [BC + 1]
    float *btot = bsum + NW * BC + BC + 4;                     // [BC] bound of what the window holds
    int *shift = reinterpret_cast<int *>(btot + BC);           // [BC] rescale of the window for a pass
    // [BC] spike thresholds of a pass with spikes, read before its rescale shifts are written (PREC
    // sets both in one step and keeps no bound: the thresholds take the bound's words)
    float *thr = PREC ? btot : reinterpret_cast<float *>(shift);
    int *bmax = shift + BC;                                    // [BC] largest |G * mask| (float bits, >= 0)
    unsigned *bexp = reinterpret_cast<unsigned *>(bmax + BC);  // [BC] exponent sums + (counts << 20)
    // (xg: the offset / mask gradients read X from global memory; no X window)
    const bool xg = COORD && wt.xglobal != 0;
    float *xwin = smem + FIXED_WORDS;                          // [cells][XS] X window (COORD)
    int *iwin = reinterpret_cast<int *>(xwin + (COORD && !xg ? wt.cells * XS : 0));   // [BC][cst] fixed point
    const int cst = fix_stride(wt.cells);
    // [2][tpp][npiece][512] staged weight blocks of the 16-bit K loop (wt.wstage > 0)
    uint16_t *wst = reinterpret_cast<uint16_t *>(iwin + (SCATTER ? BC * cst : 0));

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;
    const int mq = 4 * q;

    // ---- tile: one spatial box x one 16-channel slice --------------------------------
    int L = xcd_remap(blockIdx.x, gridDim.x);
    const int ct = L % wt.c_tiles;
    L /= wt.c_tiles;
    const int n_sp = g.B * wt.ntile[0] * wt.ntile[1] * wt.ntile[2];
    Tile tile;
    tile.init(g, wt, L % n_sp, ct, L / n_sp);
    const int b = tile.b, grp = tile.grp, c0 = tile.c0, cg0 = tile.cg0, ogu = tile.ogu, mgu = tile.mgu;
    const bool deformable = offset != nullptr;
    // the 16-bit K loop when its operands were laid out, and (fp32) none was flagged
    const int use16_flag = zs != nullptr && (flag == nullptr || *flag == 0);
    const bool cq_ok = c0 + mq < g.Cg;           // Cg % 4 == 0: a channel quad is all in or all out
    const float *xb = xcl + (size_t)b * g.Sn * g.C + cg0;
    // grad_input's strides per channel and per pixel: channels-last (B, S, C) or, gx_nchw, the
    // caller's (B, C, S) float32 tensor itself
    const size_t gcs = gx_nchw ? (size_t)g.Sn : 1, gps = gx_nchw ? 1 : (size_t)g.C;
    float *const gxb = gx_cl + (size_t)b * g.Sn * g.C;

    // ---- per-tile LDS state: X window (read by the offset/mask gradients), zeroed
    //      fixed-point window (scatter)
    if constexpr (COORD) {
        if (!xg) fill_xwin(g, wt, tile, xb, xwin, tid, NT);
    }
    if constexpr (SCATTER) {
        // 16-byte stores: BC * cst is a multiple of 64 words and the window is 16-byte aligned
        for (int i = tid; i < BC * cst / 4; i += NT) reinterpret_cast<uint4 *>(iwin)[i] = uint4{0u, 0u, 0u, 0u};
        if (tid < BC) {
            bmax[tid] = 0;
            bexp[tid] = 0u;
        }
    }

    // ---- K-loop operands, straight to registers ---------------------------------
    // B = Z[m][px]: pixel wave * 32 + pb * 16 + lane % 16, m = 4 * (lane / 16) + kk
    // A = W[c][m]:  channel c0 + lane % 16, same m; the K order is permuted the same
    //               way on both operands, which leaves the sum unchanged
    int zp[PB];
    const T *zb[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
        zp[pb] = tile.pixel(g, wt, wave * (PB * 16) + pb * 16 + (lane & 15));
        zb[pb] = z + ((size_t)b * g.M + (size_t)grp * g.Mg) * g.Pn + (zp[pb] < 0 ? 0 : zp[pb]);
    }
    // Loads are unconditional, from clamped (valid) addresses, so that a prefetch is
    // only waited for where its data is consumed. Pixels outside the grid stage some
    // value of a valid pixel: their G is never read (their geometry has no valid
    // corner, no offset/mask output, and the scale bound skips them). Rows m >= Mg
    // meet zero weights; when Mg % 16 != 0 they are zeroed at use (MPAD) so that a
    // non-finite value there cannot leak into the sum.
    auto load_z = [&](int ms, float (&zr)[PB][4]) {
#pragma unroll
        for (int pb = 0; pb < PB; ++pb)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int m = ms * BM + mq + kk;
                zr[pb][kk] = to_acc<float>(zb[pb][(size_t)min(m, g.Mg - 1) * g.Pn]);
            }
    };
    // weight chunks [G][c_tiles][m_steps][Kn][16 c][16 m]
    const float *wbase =
        wchunks + ((size_t)grp * wt.c_tiles + ct) * wt.m_steps * g.Kn * (BC * BM) + (lane & 15) * BM + mq;
    auto load_w = [&](int ms, int t0, int ntaps, acc4 (&wr)[TMAX]) {
        const float *p = wbase + ((size_t)ms * g.Kn + t0) * (BC * BM);
#pragma unroll
        for (int tp = 0; tp < TMAX; ++tp) {
            // slots past the pass hold zeros; their products are never used
            wr[tp] = acc4{0.f, 0.f, 0.f, 0.f};
            if (tp < ntaps) wr[tp] = *reinterpret_cast<const acc4 *>(p + tp * (BC * BM));
        }
    };

    // ---- the fixed-point window accumulates over every pass of the tile and is flushed
    //      once, at the end (or before a pass whose bound is not finite): one float atomic
    //      per non-zero (cell, channel), 16 consecutive channels per cell (channels-last) or
    //      32 consecutive cells per channel (gx_nchw)
    bool win_data = false;   // the window holds accumulated values (uniform)
    // thread = (channel tid % 16, cells tid / 16, + 32, ...) or, gx_nchw, (channel tid / 32, cells
    // tid % 32, + 32, ...); FB cells' values are read before any is used (one LDS latency per
    // batch). keep: the window is used again (cleared as read, barrier at the end); at the end
    // of the workgroup neither is needed.
    auto flush_window = [&](bool keep) {
        constexpr int FB = 8;
        constexpr int STEP = NT / 16;
        static_assert(STEP == 32 && NT / 32 == BC, "both thread maps step 32 cells per channel");
        const int c = gx_nchw ? tid >> 5 : tid & 15;
        const int se = scl[c];
        const bool c_ok = c0 + c < g.Cg;
        float *gbase = gxb + (size_t)(cg0 + c) * gcs;
        const int first = gx_nchw ? tid & 31 : tid >> 4;
        // cell walker (no divisions per cell), as in for_cells
        int lx = first % wt.WE[2];
        int rr = first / wt.WE[2];
        int ly = rr % wt.WE[1];
        int lz = rr / wt.WE[1];
        const int sx_step = STEP % wt.WE[2], sy_step = (STEP / wt.WE[2]) % wt.WE[1],
                  sz_step = STEP / (wt.WE[2] * wt.WE[1]);
        for (int cell0 = first; cell0 < wt.cells; cell0 += FB * STEP) {
            int iv[FB], si[FB];
#pragma unroll
            for (int j = 0; j < FB; ++j) {
                const int cell = cell0 + j * STEP;
                iv[j] = cell < wt.cells ? iwin[c * cst + cell] : 0;
                const int sz = tile.org[0] + lz, sy = tile.org[1] + ly, sx = tile.org[2] + lx;
                // window cells outside the grid hold only contributions of corners outside it
                const bool in = sz >= 0 && sz < g.S[0] && sy >= 0 && sy < g.S[1] && sx >= 0 && sx < g.S[2];
                si[j] = in && c_ok ? (sz * g.S[1] + sy) * g.S[2] + sx : -1;
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
            for (int j = 0; j < FB; ++j) {
                if (iv[j] == 0) continue;
                if (keep) iwin[c * cst + cell0 + j * STEP] = 0;   // cleared for what follows
                if (si[j] >= 0) atomic_add(gbase + (size_t)si[j] * gps, ldexpf((float)iv[j], -se));
            }
        }
        if (keep) __syncthreads();
    };

    for (int t0 = 0; t0 < g.Kn; t0 += wt.tpp) {
        const int ntaps = min(wt.tpp, g.Kn - t0);

        // ---- sampling table of the pass, one (tap, pixel) per thread ------------------
        fill_geo<DIM, T>(g, wt, tile, offset, mask, t0, ntaps, geo, tid, NT);

        acc4 acc[TMAX][PB];
#pragma unroll
        for (int tp = 0; tp < TMAX; ++tp)
#pragma unroll
            for (int pb = 0; pb < PB; ++pb) acc[tp][pb] = acc4{0.f, 0.f, 0.f, 0.f};

        // ---- K loop: Z ping-pong, W rolling reload ----------------------------------
        auto kloop = [&](auto full_tag, auto mpad_tag) {
            constexpr bool FULL = decltype(full_tag)::value;   // every tap slot in use: no guards
            constexpr bool MPAD = decltype(mpad_tag)::value;   // Mg % 16 != 0: zero rows m >= Mg
            // Z: ping-pong pair; W: one register set, each tap's fragment reloaded for
            // the next step as soon as this step's MFMAs on it are issued (the last step
            // re-reads itself, so the step is one straight-line block)
            float za[PB][4], zbb[PB][4];
            acc4 wr[TMAX];
            auto step = [&](int ms, const float (&zr)[PB][4]) {
                const int msn = min(ms + 1, wt.m_steps - 1);
#pragma unroll
                for (int tp = 0; tp < TMAX; ++tp) {
                    if (FULL || tp < ntaps) {
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                            for (int pb = 0; pb < PB; ++pb) {
                                const float zv = (!MPAD || ms * BM + mq + kk < g.Mg) ? zr[pb][kk] : 0.f;
                                acc[tp][pb] = mfma16x16x4(wr[tp][kk], zv, acc[tp][pb]);
                            }
                    }
                    // (slots past the pass are never loaded nor used)
                    if (FULL || tp < ntaps)
                        wr[tp] = *reinterpret_cast<const acc4 *>(wbase + ((size_t)msn * g.Kn + t0 + tp) * (BC * BM));
                    // issue order: this tap's MFMAs, then its reload (a full step ahead of use)
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            load_z(0, za);
            load_w(0, t0, ntaps, wr);
            for (int ms = 0; ms < wt.m_steps; ms += 2) {
                const bool has1 = ms + 1 < wt.m_steps;
                load_z(min(ms + 1, wt.m_steps - 1), zbb);
                // keep the prefetch ahead of this step's MFMAs: without the fence the loads are
                // sunk next to their first use (a full memory latency exposed every step)
                issue_fence();
                step(ms, za);
                if (has1) {
                    load_z(min(ms + 2, wt.m_steps - 1), za);
                    issue_fence();
                    step(ms + 1, zbb);
                }
            }
        };
        // ---- 16-bit K loop: 16x16x32 MFMAs over 32 channels per step, operands straight
        //      from the split layouts into registers; Z of the next step and the weight
        //      fragments of the next two taps (of the (step, tap) sequence) in flight, in a
        //      ring of three that the unrolled tap loop indexes statically (a load one tap
        //      ahead left the MFMAs waiting on it: 5% of the kernel at cfg2)
        auto kloop16 = [&]() {
            constexpr int NP = npiece_of<T>();
            const int ms32 = wt.ms32;
            const size_t zstep = (size_t)g.Pn * (NP * 32);
            const uint16_t *zl[PB];
#pragma unroll
            for (int pb = 0; pb < PB; ++pb)
                zl[pb] = zs + ((size_t)(b * g.G + grp) * ms32 * NP * g.Pn + (zp[pb] < 0 ? 0 : zp[pb])) * 32 + q * 8;
            const uint16_t *wl = wsplit + ((size_t)(grp * wt.c_tiles + ct) * ms32 * g.Kn + t0) * (NP * 512) + lane * 8;
            auto wfrag = [&](int st, int tl, uint4 (&f)[NP]) {
                const uint16_t *pw = wl + ((size_t)min(st, ms32 - 1) * g.Kn + tl) * (NP * 512);
#pragma unroll
                for (int k = 0; k < NP; ++k) f[k] = *reinterpret_cast<const uint4 *>(pw + k * 512);
            };
            auto zfrag = [&](int st, uint4 (&f)[PB][NP]) {
#pragma unroll
                for (int pb = 0; pb < PB; ++pb)
#pragma unroll
                    for (int k = 0; k < NP; ++k)
                        f[pb][k] = *reinterpret_cast<const uint4 *>(zl[pb] + (size_t)st * zstep + (size_t)k * g.Pn * 32);
            };
            uint4 zc[PB][NP], zn[PB][NP], wr[3][NP];
            zfrag(0, zc);
            // (ps, pt): the next weight fragment of the (step, tap) sequence to load; two in flight
            int ps = 0, pt = 0;
            auto advance = [&]() {
                if (++pt == ntaps) {
                    pt = 0;
                    ++ps;
                }
            };
            wfrag(ps, pt, wr[0]);
            advance();
            wfrag(ps, pt, wr[1]);
            advance();
            for (int st = 0; st < ms32; ++st) {
                zfrag(min(st + 1, ms32 - 1), zn);
                issue_fence();
#pragma unroll
                for (int tp = 0; tp < TMAX; ++tp) {
                    if (tp >= ntaps) break;
                    wfrag(ps, pt, wr[(tp + 2) % 3]);
                    advance();
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb)
                        acc[tp][pb] = mfma16x16x32_np<T, NP>(wr[tp % 3], zc[pb], acc[tp][pb]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (ntaps % 3 != 0) {
                    // keep the ring aligned with tap 0 of the next step
                    uint4 t[3][NP];
#pragma unroll
                    for (int i = 0; i < 3; ++i)
#pragma unroll
                        for (int k = 0; k < NP; ++k) t[i][k] = wr[i][k];
                    const int r = ntaps % 3;
#pragma unroll
                    for (int i = 0; i < 3; ++i)
#pragma unroll
                        for (int k = 0; k < NP; ++k) wr[i][k] = r == 1 ? t[(i + 1) % 3][k] : t[(i + 2) % 3][k];
                }
#pragma unroll
                for (int pb = 0; pb < PB; ++pb)
#pragma unroll
                    for (int k = 0; k < NP; ++k) zc[pb][k] = zn[pb][k];
            }
        };
        // ---- 16-bit K loop with the weight blocks staged in LDS: a step's block (the pass's
        //      taps x NP pieces, 1 KB each, contiguous in the split layout) is the same for all
        //      eight waves; read straight from global memory it went eight times through the
        //      vector memory path. The next step's block is copied global -> LDS (one 1 KB wave
        //      instruction per piece, spread over the waves) while this step's MFMAs run, into
        //      the other half of a double buffer; one barrier per step publishes it.
        auto kloop16s = [&]() {
            constexpr int NP = npiece_of<T>();
            const int ms32 = wt.ms32;
            const size_t zstep = (size_t)g.Pn * (NP * 32);
            const uint16_t *zl[PB];
#pragma unroll
            for (int pb = 0; pb < PB; ++pb)
                zl[pb] = zs + ((size_t)(b * g.G + grp) * ms32 * NP * g.Pn + (zp[pb] < 0 ? 0 : zp[pb])) * 32 + q * 8;
            auto zfrag = [&](int st, uint4 (&f)[PB][NP]) {
#pragma unroll
                for (int pb = 0; pb < PB; ++pb)
#pragma unroll
                    for (int k = 0; k < NP; ++k)
                        f[pb][k] = *reinterpret_cast<const uint4 *>(zl[pb] + (size_t)st * zstep + (size_t)k * g.Pn * 32);
            };
            const uint16_t *wblk = wsplit + ((size_t)(grp * wt.c_tiles + ct) * ms32 * g.Kn + t0) * (NP * 512);
            const int blk = wt.tpp * (NP * 512);   // buffer stride (16-bit values)
            const int npc = ntaps * NP;            // 1 KB pieces per step
            auto stage = [&](int st, int buf) {
                const uint16_t *src = wblk + (size_t)st * g.Kn * (NP * 512);
                uint16_t *dst = wst + buf * blk;
                for (int i = wave; i < npc; i += NW)
                    __builtin_amdgcn_global_load_lds(src + i * 512 + lane * 8, dst + i * 512, 16, 0, 0);
            };
            auto wread = [&](const uint16_t *bb, int tl, uint4 (&f)[NP]) {
                const uint16_t *p = bb + tl * (NP * 512) + lane * 8;
#pragma unroll
                for (int k = 0; k < NP; ++k) f[k] = *reinterpret_cast<const uint4 *>(p + k * 512);
            };
            // the staged block's loads done, then the workgroup barrier that publishes it
            auto publish = [&]() {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            };
            uint4 zc[PB][NP], zn[PB][NP], wa[2][NP];
            stage(0, 0);
            zfrag(0, zc);
            publish();
            for (int st = 0; st < ms32; ++st) {
                if (st + 1 < ms32) stage(st + 1, (st + 1) & 1);
                zfrag(min(st + 1, ms32 - 1), zn);
                issue_fence();
                const uint16_t *bb = wst + (st & 1) * blk;
                wread(bb, 0, wa[0]);
#pragma unroll
                for (int tp = 0; tp < TMAX; ++tp) {
                    if (tp >= ntaps) break;
                    // tap tp + 1's fragments read from LDS before tap tp's MFMAs
                    if (tp + 1 < ntaps) wread(bb, tp + 1, wa[(tp + 1) & 1]);
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb)
                        acc[tp][pb] = mfma16x16x32_np<T, NP>(wa[tp & 1], zc[pb], acc[tp][pb]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // the next block landed, every wave done with this one
                publish();
#pragma unroll
                for (int pb = 0; pb < PB; ++pb)
#pragma unroll
                    for (int k = 0; k < NP; ++k) zc[pb][k] = zn[pb][k];
            }
        };
        // (opaque to the optimiser: the choice is made per pass rather than by two copies of
        // the whole pass loop)
        int use16 = __builtin_amdgcn_readfirstlane(use16_flag);
        asm volatile("" : "+s"(use16));
        if (use16) {
            if (wt.wstage > 0)
                kloop16s();
            else
                kloop16();
            if constexpr (npiece_of<T>() == 2) {
                // the pieces' scales back out: G = acc 2^-(s_W + s_Z)
                const int back = -(operand_scale(flag, AMAX_W) + operand_scale(flag, AMAX_Z));
#pragma unroll
                for (int tp = 0; tp < TMAX; ++tp)
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb)
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[tp][pb][v] = ldexpf(acc[tp][pb][v], back);
            }
        } else {
            const bool mpad = g.Mg % BM != 0;
            if (ntaps == TMAX && !mpad)
                kloop(std::true_type(), std::false_type());
            else if (!mpad)
                kloop(std::false_type(), std::false_type());
            else
                kloop(std::false_type(), std::true_type());
        }
        __syncthreads();   // geometry table (and X window) written

        // ---- fixed-point scale per channel: the bound covers this pass plus everything
        //      the window already holds; when it grows, the held values are shifted down
        //      to the new (smaller or equal) scale. Terms above the spike threshold th of
        //      their channel bypass the window and the bound.
        int sexp[4] = {0, 0, 0, 0};   // scale exponents of this lane's channels c0 + mq + v
        float th[4] = {0.f, 0.f, 0.f, 0.f};   // spike thresholds of this lane's channels
        bool use_window = false, spikes = false;
        if constexpr (SCATTER) {
            // first sweep: per-channel sum of the terms (a nan makes it non-finite), their
            // maximum, and over the lanes the sum of the biased exponents of the nonzero lane
            // means + (their count << 20) (128 lanes of exponent < 2^8: no carry); otherwise
            // the sum of the terms at or below lim[v]
            auto bound_sweep = [&](const float (&lim)[4], bool with_max) {
                float part[4] = {0.f, 0.f, 0.f, 0.f}, pmax[4] = {0.f, 0.f, 0.f, 0.f};
                unsigned ex[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int pb = 0; pb < PB; ++pb) {
                    const int i = wave * (PB * 16) + pb * 16 + (lane & 15);
#pragma unroll
                    for (int tp = 0; tp < TMAX; ++tp) {
                        if (tp < ntaps && zp[pb] >= 0) {
                            const float mk = fabsf(rec_mask<DIM>(geo[tp * BPX + i]));
#pragma unroll
                            for (int v = 0; v < 4; ++v) {
                                const float a = fabsf(acc[tp][pb][v]) * mk;
                                if (with_max) {
                                    part[v] += a;
                                    pmax[v] = fmaxf(pmax[v], a);
                                } else {
                                    part[v] += a <= lim[v] ? a : 0.f;
                                }
                            }
                        }
                    }
                }
                if (with_max) {
                    // terms of the lane (per channel): the pass's taps at each valid pixel
                    int npx = 0;
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb) npx += zp[pb] >= 0;
                    const float inv = npx > 0 ? __frcp_rn((float)(npx * ntaps)) : 0.f;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const unsigned e = __float_as_uint(part[v] * inv) >> 23;
                        ex[v] = e != 0u ? e + (1u << 20) : 0u;
                    }
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    part[v] = row_sum16(part[v]);
                    if (with_max) {
                        pmax[v] = row_max16(pmax[v]);
                        ex[v] = row_sum16(ex[v]);
                    }
                }
                if ((lane & 15) == 0) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        bsum[wave * BC + mq + v] = part[v];
                        if (with_max) {
                            // non-negative floats order as their bit patterns (a nan has an
                            // exponent of all ones: it lands above every finite value)
                            atomicMax(bmax + mq + v, __float_as_int(pmax[v]));
                            atomicAdd(bexp + mq + v, ex[v]);
                        }
                    }
                }
            };
            // scale of the pass from its (kept) bound bc, channel tid of wave 0's first 16 lanes
            auto set_scale = [&](float bc) {
                const float tot = (win_data ? btot[tid] : 0.f) + bc;
                // the pass uses the window only if every bound is finite (ballot over 16 lanes)
                const unsigned long long bad = __ballot(!isfinite(tot));
                int e = 0;
                if (tot > 0.f && isfinite(tot)) frexpf(tot, &e);   // tot < 2^e
                shift[tid] = 0;
                if (bad == 0ull) {
                    if (win_data) shift[tid] = scl[tid] - (FIX_BITS - e);   // >= 0: the bound only grows
                    scl[tid] = FIX_BITS - e;
                    btot[tid] = tot;
                }
                if (tid == 0) scl[BC] = bad != 0ull;
            };
            // PREC: the scale of the pass from the largest term the window keeps (kmax; a pass
            // with spikes keeps the terms up to their threshold), coarsened to what the window
            // holds; bc (the sum of every term) only tells whether the pass is finite. A pass that
            // skips the window (not finite; 3D with spikes: skip) leaves the held scale as it is:
            // the window's flush reads it.
            auto set_scale_prec = [&](float kmax, float bc, bool skip) {
                const unsigned long long bad = __ballot(!isfinite(bc));
                int e = 0;
                if (kmax > 0.f) frexpf(kmax, &e);   // kmax < 2^e
                int sc = PREC_BITS - e;
                shift[tid] = 0;
                if (bad == 0ull && !skip) {
                    if (win_data) {
                        const int held = scl[tid];
                        sc = min(sc, held);
                        shift[tid] = held - sc;
                    }
                    scl[tid] = sc;
                }
                if (tid == 0) scl[BC] = bad != 0ull;
            };
            const float no_lim[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
            bound_sweep(no_lim, true);
            __syncthreads();
            if (tid < BC) {
                float bc = 0.f;
#pragma unroll
                for (int w = 0; w < NW; ++w) bc += bsum[w * BC + tid];
                const unsigned es = bexp[tid];
                const float big = __int_as_float(bmax[tid]);
                bmax[tid] = 0;   // for the next pass (read after this pass's last barrier)
                bexp[tid] = 0u;
                // threshold 2^(mean unbiased exponent of the lane means + SPIKE_BITS), the mean
                // rounded down (exact: integers below 2^24, a correctly rounded quotient of
                // denominator <= 128 is an integer only when the true quotient is)
                const float cnt = (float)(es >> 20), esum = (float)(es & ((1u << 20) - 1u));
                const float lim = cnt > 0.f ? ldexpf(1.f, (int)floorf(esum / cnt) - 127 + SPIKE_BITS) : INFINITY;
                const bool spike = isfinite(bc) && big > lim;
                thr[tid] = spike ? lim : INFINITY;
                const unsigned long long any = __ballot(spike);
                if constexpr (PREC)
                    set_scale_prec(spike ? lim : big, bc, DIM == 3 && any != 0ull);
                else if (any == 0ull)
                    set_scale(bc);   // no spike: the bound is final
                if (tid == 0) scl[BC + 1] = any != 0ull;
            }
            __syncthreads();
            // both flags in one read: non-finite [BC], spikes [BC + 1]
            const int2 flags = *reinterpret_cast<const int2 *>(scl + BC);
            spikes = flags.y != 0;
            bool no_window = flags.x != 0;
            if constexpr (DIM == 3) {
                // 3D: a pass with spikes skips the window (the branch-light 3D path has no
                // per-channel routing)
                no_window = no_window || spikes;
            } else if (spikes && PREC) {
#pragma unroll
                for (int v = 0; v < 4; ++v) th[v] = thr[mq + v];
            } else if (spikes) {
                // bound of the terms that stay in the window
#pragma unroll
                for (int v = 0; v < 4; ++v) th[v] = thr[mq + v];
                bound_sweep(th, false);
                __syncthreads();
                if (tid < BC) {
                    float bc = 0.f;
#pragma unroll
                    for (int w = 0; w < NW; ++w) bc += bsum[w * BC + tid];
                    set_scale(bc);
                }
                __syncthreads();
                no_window = scl[BC] != 0;
            }
            if (no_window) {
                // not finite (or 3D spikes): what the window holds goes out at its scale, the
                // pass goes to global float atomics (inf / nan propagate as in the reference)
                if (win_data) flush_window(true);
                win_data = false;
                spikes = false;
            } else {
                if (win_data) {
                    // rescale to nearest (halves up); a shift of 31 or more leaves at most a unit
                    // (PREC: a held value may be anywhere in the 32-bit range)
                    const int c = tid >> 5, sh = shift[c];
                    if (sh > 0) {
                        for (int cell = tid & 31; cell < cst; cell += 32) {
                            const int v = iwin[c * cst + cell];
                            iwin[c * cst + cell] = sh >= 31 ? 0 : (v >> sh) + ((v >> (sh - 1)) & 1);
                        }
                    }
                    __syncthreads();
                }
                use_window = wt.cells > 0;
                win_data = use_window;
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) sexp[v] = scl[mq + v];
        }

        // ---- epilogue: every wave walks its own pixels tap by tap, no barriers -------
        // 2D offset / mask gradients: the next (tap, pixel block)'s record and corner X (fast
        // records; a clamped cell otherwise) are read from LDS at the end of the current one,
        // so their latency overlaps its reductions and atomics (cfg2 data gradient -2%; 1D,
        // whose epilogue is a tenth of the kernel, measured 0.6% slower with it)
        constexpr bool XPF = DIM == 2 && COORD;
        constexpr int NFX = DIM == 2 ? 4 : 2;
        acc4 rn = acc4{0.f, 0.f, 0.f, 0.f};
        acc4 xn[XPF ? NFX : 1];
        auto x_prefetch = [&](int tl, int pb) {
            if constexpr (XPF) {
                rn = geo[tl * BPX + wave * (PB * 16) + pb * 16 + (lane & 15)];
                const int f = max(rec_fast_cell<DIM>(rn), 0);
#pragma unroll
                for (int k = 0; k < NFX; ++k) {
                    const int cell = f + (k & 1) + (k >> 1) * wt.WE[2];
                    xn[k] = *reinterpret_cast<const acc4 *>(xwin + cell * XS + mq);
                }
            }
        };
        if constexpr (XPF) x_prefetch(0, 0);
        for (int tl = 0; tl < ntaps; ++tl) {
            const int t = t0 + tl;
            acc4 gt[PB];
            switch (tl) {
#define TVDCN_SEL(K)                                                            \
    case K:                                                                     \
        if constexpr (K < TMAX) {                                               \
            _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) gt[pb] = acc[K][pb]; \
        }                                                                       \
        break;
                TVDCN_SEL(0) TVDCN_SEL(1) TVDCN_SEL(2) TVDCN_SEL(3) TVDCN_SEL(4)
                TVDCN_SEL(5) TVDCN_SEL(6) TVDCN_SEL(7) TVDCN_SEL(8)
#undef TVDCN_SEL
                default:
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb) gt[pb] = acc4{0.f, 0.f, 0.f, 0.f};
            }

#pragma unroll
            for (int pb = 0; pb < PB; ++pb) {
                const int i = wave * (PB * 16) + pb * 16 + (lane & 15);
                const acc4 r = XPF ? rn : geo[tl * BPX + i];
                const float mk = rec_mask<DIM>(r);
                const acc4 gv = gt[pb];
                const int fc = rec_fast_cell<DIM>(r);
                // channels whose term is a spike of the pass: global float atomics (nan included)
                bool sp[4] = {false, false, false, false};
                bool lane_spike = false;
                if constexpr (SCATTER) {
                    if (spikes) {
                        const float am = fabsf(mk);
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            sp[v] = !(fabsf(gv[v]) * am <= th[v]);
                            lane_spike = lane_spike || sp[v];
                        }
                    }
                }
                float qv[DIM + 1];
                bool done = false;
                if constexpr (DIM == 3) {
                    if (!SCATTER || use_window) {
                        // 3D: one branch-light path for every lane (window margins of about one
                        // cell: most waves hold a lane with a corner outside the window)
                        done = true;
                        const Corners3 cr(g, wt, tile, r, deformable);
                        if constexpr (COORD) {
                            // G contracted with X per corner, then the trilinear / coordinate weights
                            float gs = 0.f, gz = 0.f, gy = 0.f, gxx = 0.f;
#pragma unroll
                            for (int k = 0; k < 8; ++k) {
                                if (k > 0 && !deformable) break;
                                const acc4 x = corner_x3(g, wt, cr, k, xwin, mq, xb + mq, cq_ok, xg);
                                const float gk = gv[0] * x[0] + gv[1] * x[1] + gv[2] * x[2] + gv[3] * x[3];
                                const int bz = k >> 2, by = (k >> 1) & 1, bx = k & 1;
                                const float wz = bz ? cr.fh[0] : 1.f - cr.fh[0];
                                const float wy = by ? cr.fh[1] : 1.f - cr.fh[1];
                                const float wx = bx ? cr.fh[2] : 1.f - cr.fh[2];
                                gs += wz * wy * wx * gk;
                                gz += (bz ? gk : -gk) * (wy * wx);
                                gy += (by ? gk : -gk) * (wz * wx);
                                gxx += (bx ? gk : -gk) * (wz * wy);
                            }
                            qv[0] = mk * gz;
                            qv[1] = mk * gy;
                            qv[2] = mk * gxx;
                            qv[3] = cr.inside ? gs : 0.f;
                        }
                        if constexpr (SCATTER) {
                            if (cq_ok) {
                                // (PREC: mask * G scaled, the corner weight <= 1 applied after, so no
                                // intermediate leaves the float range)
                                float gsc[4];
#pragma unroll
                                for (int v = 0; v < 4; ++v) gsc[v] = ldexpf(PREC ? mk * gv[v] : gv[v], sexp[v]);
                                float *gdst = gxb + (size_t)(cg0 + mq) * gcs;
                                if constexpr (!PREC) {
#pragma unroll
                                    for (int k = 0; k < 8; ++k) {
                                        if (k > 0 && !deformable) break;
                                        if (!cr.in_grid(k)) continue;
                                        const float sw = mk * cr.weight(k);
                                        if (cr.in_win(k)) {
                                            unsigned int *dst = reinterpret_cast<unsigned int *>(iwin + mq * cst + cr.cell(wt, k));
#pragma unroll
                                            for (int v = 0; v < 4; ++v)
                                                atomicAdd(dst + v * cst, (unsigned int)fixed_round(sw * gsc[v]));
                                        } else {
                                            float *dst = gdst + (size_t)cr.idx(g, k) * gps;
#pragma unroll
                                            for (int v = 0; v < 4; ++v) atomic_add(dst + v * gcs, sw * gv[v]);
                                        }
                                    }
                                } else {
                                    // the returned old values of four corners at a time are checked for a
                                    // possible wrap, the adds recomputed where one is
#pragma unroll
                                    for (int h = 0; h < 2; ++h) {
                                        if (h > 0 && !deformable) break;
                                        unsigned near = 0u;
                                        unsigned old[4][4];
#pragma unroll
                                        for (int j = 0; j < 4; ++j) {
                                            const int k = 4 * h + j;
                                            if (k > 0 && !deformable) break;
                                            if (!cr.in_grid(k)) continue;
                                            if (cr.in_win(k)) {
                                                unsigned int *dst = reinterpret_cast<unsigned int *>(iwin + mq * cst + cr.cell(wt, k));
                                                const float sw = cr.weight(k);
#pragma unroll
                                                for (int v = 0; v < 4; ++v) {
                                                    old[j][v] = atomicAdd(dst + v * cst, (unsigned int)fixed_round(sw * gsc[v]));
                                                    near = max(near, old[j][v] + WRAP_K);
                                                }
                                            } else {
                                                float *dst = gdst + (size_t)cr.idx(g, k) * gps;
                                                const float sw = mk * cr.weight(k);
#pragma unroll
                                                for (int v = 0; v < 4; ++v) atomic_add(dst + v * gcs, sw * gv[v]);
                                            }
                                        }
                                        if (near >= 2u * WRAP_K) {
                                            // some add may have wrapped: its 2^32 units go to global memory
#pragma unroll
                                            for (int j = 0; j < 4; ++j) {
                                                const int k = 4 * h + j;
                                                if (k > 0 && !deformable) break;
                                                if (!cr.in_grid(k) || !cr.in_win(k)) continue;
                                                const float sw = cr.weight(k);
#pragma unroll
                                                for (int v = 0; v < 4; ++v) {
                                                    const float sp = wrap_spill(old[j][v], fixed_round(sw * gsc[v]), sexp[v]);
                                                    if (sp != 0.f) atomic_add(gdst + (size_t)cr.idx(g, k) * gps + v * gcs, sp);
                                                }
                                            }
                                        }
                                    }
                                }
                            }
                        }
                    }
                } else if (fc >= 0 && (!SCATTER || use_window) && !lane_spike) {
                    done = true;
                    // fast path: every corner cell is in the window (zeros / dropped
                    // outside the grid), plain bilinear formulas
                    const float fx = r[DIM - 1];   // fast records hold the fractional parts
                    const float fy = DIM == 2 ? r[0] : 0.f;
                    constexpr int NF = DIM == 2 ? 4 : 2;
                    int cell[NF];
                    cell[0] = fc;
                    cell[1] = fc + 1;
                    if constexpr (DIM == 2) {
                        cell[2] = fc + wt.WE[2];
                        cell[3] = fc + wt.WE[2] + 1;
                    }
                    if constexpr (COORD) {
                        // every quantity is linear in X: contract the lane's 4 channels with G
                        // per corner first (gk), then apply the bilinear / coordinate weights
                        float gk[NF];
#pragma unroll
                        for (int k = 0; k < NF; ++k) {
                            const acc4 x = XPF ? xn[XPF ? k : 0] : *reinterpret_cast<const acc4 *>(xwin + cell[k] * XS + mq);
                            gk[k] = gv[0] * x[0] + gv[1] * x[1] + gv[2] * x[2] + gv[3] * x[3];
                        }
                        if constexpr (DIM == 2) {
                            const float ex0 = gk[1] - gk[0], ex1 = gk[3] - gk[2];   // along x, rows y0 / y1
                            const float ey0 = gk[2] - gk[0], ey1 = gk[3] - gk[1];   // along y, columns x0 / x1
                            const float t0 = gk[0] + fx * ex0, t1 = gk[2] + fx * ex1;
                            qv[0] = mk * (ey0 + fx * (ey1 - ey0));   // d/dy
                            qv[1] = mk * (ex0 + fy * (ex1 - ex0));   // d/dx
                            qv[2] = t0 + fy * (t1 - t0);             // sampled value
                        } else {
                            const float ex = gk[1] - gk[0];
                            qv[0] = mk * ex;
                            qv[1] = gk[0] + fx * ex;
                        }
                        // a non-finite gk makes the factored sample non-finite; the reference's
                        // corner sums then keep the +-inf that the factored differences turn
                        // into inf - inf
                        if (!isfinite(qv[DIM])) coord_direct<DIM>(gk, fy, fx, mk, qv);
                    }
                    if constexpr (SCATTER) {
                        if (cq_ok) {
                            // mask-weighted corner weights; G pre-scaled to fixed point per channel
                            // (PREC: mask * G scaled, plain corner weights <= 1 after)
                            const float mw = PREC ? 1.f : mk;
                            float wm[NF];
                            if constexpr (DIM == 2) {
                                const float a1 = mw * fy, a0 = mw - a1;
                                wm[1] = a0 * fx;
                                wm[0] = a0 - wm[1];
                                wm[3] = a1 * fx;
                                wm[2] = a1 - wm[3];
                            } else {
                                wm[1] = mw * fx;
                                wm[0] = mw - wm[1];
                            }
                            float gs[4];
#pragma unroll
                            for (int v = 0; v < 4; ++v) gs[v] = ldexpf(PREC ? mk * gv[v] : gv[v], sexp[v]);
                            unsigned near = 0u;
                            unsigned old[NF][4];
#pragma unroll
                            for (int k = 0; k < NF; ++k) {
                                unsigned int *dst = reinterpret_cast<unsigned int *>(iwin + mq * cst + cell[k]);
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    const int a = fixed_round(wm[k] * gs[v]);
                                    if constexpr (PREC) {
                                        old[k][v] = atomicAdd(dst + v * cst, (unsigned int)a);
                                        near = max(near, old[k][v] + WRAP_K);
                                    } else {
                                        atomicAdd(dst + v * cst, (unsigned int)a);
                                    }
                                }
                            }
                            if (PREC && near >= 2u * WRAP_K) {
                                // some add may have wrapped: its 2^32 units go to global memory
                                // (window cells outside the grid hold what the flush drops)
                                float *gdst = gxb + (size_t)(cg0 + mq) * gcs;
#pragma unroll
                                for (int k = 0; k < NF; ++k) {
                                    const int gi = tile.cell_index(g, wt, cell[k]);
                                    if (gi < 0) continue;
#pragma unroll
                                    for (int v = 0; v < 4; ++v) {
                                        const float sp = wrap_spill(old[k][v], fixed_round(wm[k] * gs[v]), sexp[v]);
                                        if (sp != 0.f) atomic_add(gdst + (size_t)gi * gps + v * gcs, sp);
                                    }
                                }
                            }
                        }
                    }
                }
                if (!done) {
                    // general path: per-corner validity, window membership and global fallback
                    // (also taken by fast records when the pass scatters to global memory)
                    const AxisW<DIM, float> aw = record_weights<DIM>(g, record_position<DIM>(wt, tile, r), deformable);
                    int gidx[NC], loc[NC];
                    float w[NC];
#pragma unroll
                    for (int k = 0; k < NC; ++k) {
                        int idx;
                        bool v;
                        corner_at<DIM, float>(g, aw, k, idx, v);
                        gidx[k] = v ? idx : -1;
                        w[k] = v ? corner_weight<DIM, float>(aw, k) : 0.f;
                        loc[k] = v ? tile.corner_cell<DIM>(wt, aw, k) : -1;
                    }
                    if constexpr (COORD) {
                        acc4 xv[NC];
#pragma unroll
                        for (int k = 0; k < NC; ++k) {
                            // LDS read unconditional (clamped), global read in its own branch
                            xv[k] = *reinterpret_cast<const acc4 *>(xwin + max(loc[k], 0) * XS + mq);
                            if (loc[k] < 0 || xg) {
                                xv[k] = acc4{0.f, 0.f, 0.f, 0.f};
                                if (gidx[k] >= 0 && cq_ok)
                                    xv[k] = *reinterpret_cast<const acc4 *>(xb + (size_t)gidx[k] * g.C + mq);
                            }
                        }
#pragma unroll
                        for (int a = 0; a < DIM; ++a) {
                            acc4 d = acc4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int k = 0; k < NC; ++k) d += corner_dweight<DIM, float>(aw, k, a) * xv[k];
                            qv[a] = mk * (gv[0] * d[0] + gv[1] * d[1] + gv[2] * d[2] + gv[3] * d[3]);
                        }
                        acc4 sv = acc4{0.f, 0.f, 0.f, 0.f};
                        if (aw.inside) {
#pragma unroll
                            for (int k = 0; k < NC; ++k) sv += w[k] * xv[k];
                        }
                        qv[DIM] = gv[0] * sv[0] + gv[1] * sv[1] + gv[2] * sv[2] + gv[3] * sv[3];
                    }
                    if constexpr (SCATTER) {
                        if (cq_ok) {
                            float *gdst = gxb + (size_t)(cg0 + mq) * gcs;
                            // (PREC: mask * G scaled once, the corner weight <= 1 applied after)
                            float gs[4];
#pragma unroll
                            for (int v = 0; v < 4; ++v) gs[v] = PREC ? ldexpf(mk * gv[v], sexp[v]) : 0.f;
                            unsigned near = 0u;
                            unsigned old[NC][4];
#pragma unroll
                            for (int k = 0; k < NC; ++k) {
                                if (gidx[k] < 0) continue;
                                const float s = mk * w[k];
                                if (use_window && loc[k] >= 0) {
                                    unsigned int *dst = reinterpret_cast<unsigned int *>(iwin + mq * cst + loc[k]);
#pragma unroll
                                    for (int v = 0; v < 4; ++v) {
                                        if (sp[v]) {
                                            atomic_add(gdst + (size_t)gidx[k] * gps + v * gcs, s * gv[v]);
                                        } else if constexpr (PREC) {
                                            old[k][v] = atomicAdd(dst + v * cst, (unsigned int)fixed_round(w[k] * gs[v]));
                                            near = max(near, old[k][v] + WRAP_K);
                                        } else {
                                            atomicAdd(dst + v * cst, (unsigned int)fixed_round(ldexpf(s * gv[v], sexp[v])));
                                        }
                                    }
                                } else {
                                    float *dst = gdst + (size_t)gidx[k] * gps;
#pragma unroll
                                    for (int v = 0; v < 4; ++v) atomic_add(dst + v * gcs, s * gv[v]);
                                }
                            }
                            if (PREC && near >= 2u * WRAP_K) {
                                // some add may have wrapped: its 2^32 units go to global memory
#pragma unroll
                                for (int k = 0; k < NC; ++k) {
                                    if (gidx[k] < 0 || !use_window || loc[k] < 0) continue;
#pragma unroll
                                    for (int v = 0; v < 4; ++v) {
                                        if (sp[v]) continue;   // spike terms went to global memory
                                        const float spl = wrap_spill(old[k][v], fixed_round(w[k] * gs[v]), sexp[v]);
                                        if (spl != 0.f) atomic_add(gdst + (size_t)gidx[k] * gps + v * gcs, spl);
                                    }
                                }
                            }
                        }
                    }
                }

                if constexpr (XPF) {
                    if (pb + 1 < PB)
                        x_prefetch(tl, pb + 1);
                    else if (tl + 1 < ntaps)
                        x_prefetch(tl + 1, 0);
                }
                if constexpr (COORD) {
#pragma unroll
                    for (int a = 0; a <= DIM; ++a) {
                        qv[a] = row_sum4(qv[a]);
                    }
                    const int p = zp[pb];
                    if (q == 0 && p >= 0) {
                        if (deformable) {
#pragma unroll
                            for (int a = 0; a < DIM; ++a)
                                atomic_add(goff + ((((size_t)b * g.og + ogu) * g.Kn + t) * DIM + a) * g.Pn + p, qv[a]);
                        }
                        if (mask != nullptr)
                            atomic_add(gmask + (((size_t)b * g.mg + mgu) * g.Kn + t) * g.Pn + p, qv[DIM]);
                    }
                }
            }
        }
        __syncthreads();   // all waves done with the geometry table and the window

        // ---- after the last pass, the window goes out
        if (SCATTER && win_data && t0 + wt.tpp >= g.Kn) {
            flush_window(false);   // the workgroup's last use of the window
            win_data = false;
        }
    }
}

// weight (M, Cg, Kn) -> chunks [G][c_tiles][m_steps][Kn][16 c][16 m], zero padded.
// Block = (group, channel slice, row step, run of up to WL_TK taps): reads 16 rows of
// 16 channels x the run's taps (contiguous runs of taps per channel), transposes through
// LDS, writes its 256 * taps contiguous output floats.
constexpr int WL_TK = 8;   // (LDS of the merged layout kernel: 17 KB per block)
template <typename T>
__device__ __forceinline__ void weight_win_block(int L, float *smem, const T *__restrict__ w, float *__restrict__ out,
                                                 int G, int Mg, int Cg, int Kn, int c_tiles, int m_steps) {
    float(*tile)[BC][BM + 1] = reinterpret_cast<float(*)[BC][BM + 1]>(smem);   // [tap][c][m]
    const int tchunks = (Kn + WL_TK - 1) / WL_TK;
    const int tc = L % tchunks;
    L /= tchunks;
    const int ms = L % m_steps;
    L /= m_steps;
    const int ct = L % c_tiles;
    const int grp = L / c_tiles;
    const int t0 = tc * WL_TK, nt = min(WL_TK, Kn - t0);
    const int n = BM * BC * nt;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int tt = e % nt, r = e / nt;   // (m, c, tap), taps fastest
        const int ci = r % BC, mi = r / BC;
        const int m = ms * BM + mi, c = ct * BC + ci;
        float v = 0.f;
        if (m < Mg && c < Cg) v = to_acc<float>(w[(((size_t)grp * Mg + m) * Cg + c) * Kn + t0 + tt]);
        tile[tt][ci][mi] = v;
    }
    __syncthreads();
    float *dst = out + ((((size_t)grp * c_tiles + ct) * m_steps + ms) * Kn + t0) * (BC * BM);
    for (int e = threadIdx.x; e < n; e += blockDim.x) dst[e] = tile[e / (BM * BC)][(e / BM) % BC][e % BM];
}

// weight (M, Cg, Kn) -> split chunks [G][c_tiles][ms32][Kn][NP][4 q][16 c][8 e]: per (step, tap)
// and piece, the 16x16x32 A-operand fragment of 16 channels x 32 GEMM-side channels (lane
// q * 16 + c holds rows 8q .. 8q + 7 of channel c; zero past Mg / Cg). Block = (group, channel
// slice, step, run of up to WL_TK taps), transposed through LDS.
template <typename T, int NP>
__device__ __forceinline__ void weight_split_block(int L, float *smem, const T *__restrict__ w,
                                                   uint16_t *__restrict__ out, int *flag, int G, int Mg, int Cg,
                                                   int Kn, int c_tiles, int ms32) {
    float(*tile)[BC][33] = reinterpret_cast<float(*)[BC][33]>(smem);   // [tap][c][m]
    const int tchunks = (Kn + WL_TK - 1) / WL_TK;
    const int tc = L % tchunks;
    L /= tchunks;
    const int st = L % ms32;
    L /= ms32;
    const int ct = L % c_tiles;
    const int grp = L / c_tiles;
    const int t0 = tc * WL_TK, nt = min(WL_TK, Kn - t0);
    const int n = 32 * BC * nt;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int tt = e % nt, r = e / nt;   // (m, c, tap), taps fastest
        const int ci = r % BC, mi = r / BC;
        const int m = st * 32 + mi, c = ct * BC + ci;
        float v = 0.f;
        if (m < Mg && c < Cg) v = to_acc<float>(w[(((size_t)grp * Mg + m) * Cg + c) * Kn + t0 + tt]);
        tile[tt][ci][mi] = v;
    }
    __syncthreads();
    uint16_t *dst = out + ((((size_t)grp * c_tiles + ct) * ms32 + st) * Kn + t0) * (NP * 512);
    const int sw = NP == 2 ? operand_scale(flag, AMAX_W) : 0;
    bool bad = false;
    for (int u = threadIdx.x; u < nt * 64; u += blockDim.x) {
        const int tt = u >> 6, l = u & 63, q = l >> 4, c = l & 15;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] = tile[tt][c][q * 8 + e];
            bad = bad || split_bad(v[e]);
        }
        uint4 o[NP];
        pack8_16<T, NP>(v, sw, o);
#pragma unroll
        for (int k = 0; k < NP; ++k) *reinterpret_cast<uint4 *>(dst + (size_t)tt * (NP * 512) + k * 512 + l * 8) = o[k];
    }
    if (NP == 2 && bad) atomicOr(flag, 1);
}

// The data gradient's operand layouts in one launch: blocks [0, nz) split Z (z_split_block),
// the next nws split the weight (weight_split_block), the last nww lay the weight out for the
// fp32 loop (weight_win_block); each block's branch is uniform, so its barriers are too.
template <typename T, int NP>
__global__ void __launch_bounds__(256)
data_prep_kernel(const T *__restrict__ z, uint16_t *__restrict__ zs, const T *__restrict__ w, uint16_t *__restrict__ wsp,
                 float *__restrict__ wd, int *flag, int G, int Mg, int Cg, int Pn, int Kn, int c_tiles, int ms32,
                 int m_steps, int pblocks, long long nz, int nws, bool zvec, uint16_t *__restrict__ zw,
                 size_t zw_plane) {
    __shared__ float smem[WL_TK * BC * 33];
    long long L = blockIdx.x;
    if (L < nz) {
        z_split_block<T, NP>(L, smem, z, zs, zw, flag, G, Mg, Pn, ms32, pblocks, zvec, zw_plane);
        return;
    }
    L -= nz;
    if (L < nws) {
        weight_split_block<T, NP>((int)L, smem, w, wsp, flag, G, Mg, Cg, Kn, c_tiles, ms32);
        return;
    }
    weight_win_block<T>((int)(L - nws), smem, w, wd, G, Mg, Cg, Kn, c_tiles, m_steps);
}

template <bool SCATTER, bool COORD> size_t lds_bytes(const WinTiles &t) {
    return ((size_t)FIXED_WORDS + (SCATTER ? (size_t)BC * fix_stride(t.cells) : 0) +
            (COORD && !t.xglobal ? (size_t)t.cells * XS : 0)) *
               sizeof(float) +
           (size_t)t.wstage;
}

template <int DIM, typename T, bool SCATTER, bool COORD>
hipError_t launch_k(const Geo &g, const WinTiles &tl, const void *z, const void *wchunks, const void *zs,
                    const void *wsplit, const int *flag, const void *xcl, const void *offset, const void *mask,
                    void *gx_cl, void *goff, void *gmask, hipStream_t s, bool gx_nchw) {
    auto kern = bwd_data_win_kernel<DIM, T, SCATTER, COORD>;
    const size_t lds = lds_bytes<SCATTER, COORD>(tl);
    static std::atomic<unsigned long long> lds_raised{0};   // per device, see raise_lds_limit
    if (const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kern), lds_raised); e != hipSuccess)
        return e;
    const long long blocks = (long long)g.G * g.B * tl.ntile[0] * tl.ntile[1] * tl.ntile[2] * tl.c_tiles;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NT), lds, s, g, tl, static_cast<const T *>(z),
                       static_cast<const float *>(wchunks), static_cast<const uint16_t *>(zs),
                       static_cast<const uint16_t *>(wsplit), flag, static_cast<const float *>(xcl),
                       static_cast<const T *>(offset), static_cast<const T *>(mask), static_cast<float *>(gx_cl),
                       static_cast<float *>(goff), static_cast<float *>(gmask), gx_nchw ? 1 : 0);
    return hipGetLastError();
}

template <int DIM, typename T>
hipError_t launch_f(const Geo &g, const WinTiles &tl, bool scatter, bool coord, const void *z, const void *wc,
                    const void *zs, const void *wsp, const int *flag, const void *xcl, const void *offset,
                    const void *mask, void *gx_cl, void *goff, void *gmask, hipStream_t s, bool nchw) {
    if (scatter && coord)
        return launch_k<DIM, T, true, true>(g, tl, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s, nchw);
    if (scatter)
        return launch_k<DIM, T, true, false>(g, tl, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s, nchw);
    if (coord)
        return launch_k<DIM, T, false, true>(g, tl, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s, nchw);
    return hipSuccess;
}

template <typename T>
hipError_t launch_d(int dim, const Geo &g, const WinTiles &tl, bool scatter, bool coord, const void *z,
                    const void *wc, const void *zs, const void *wsp, const int *flag, const void *xcl,
                    const void *offset, const void *mask, void *gx_cl, void *goff, void *gmask, hipStream_t s,
                    bool nchw) {
    switch (dim) {
        case 1:
            return launch_f<1, T>(g, tl, scatter, coord, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s,
                                  nchw);
        case 2:
            return launch_f<2, T>(g, tl, scatter, coord, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s,
                                  nchw);
        case 3:
            return launch_f<3, T>(g, tl, scatter, coord, z, wc, zs, wsp, flag, xcl, offset, mask, gx_cl, goff, gmask, s,
                                  nchw);
    }
    return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_prep(const Geo &g, const WinTiles &t, const void *z, const void *w, void *zs, void *wsp, void *wd,
                       int *flag, hipStream_t s, void *zw) {
    if (zw != nullptr && (z == nullptr || g.Pn % 8 != 0)) return hipErrorInvalidValue;
    constexpr int NP = npiece_of<T>();
    const int pblocks = (g.Pn + 63) / 64;
    const int tchunks = (g.Kn + WL_TK - 1) / WL_TK;
    const long long zblocks = z != nullptr ? (long long)g.B * g.G * t.ms32 * pblocks : 0;
    const long long wblocks = (long long)g.G * t.c_tiles * t.ms32 * tchunks;
    const long long dblocks = wd != nullptr ? (long long)g.G * t.c_tiles * t.m_steps * tchunks : 0;
    const long long total = zblocks + wblocks + dblocks;
    if (wblocks > INT_MAX || dblocks > INT_MAX || total > INT_MAX) return hipErrorInvalidValue;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL((data_prep_kernel<T, NP>), dim3((unsigned)total), dim3(256), 0, s, static_cast<const T *>(z),
                       static_cast<uint16_t *>(zs), static_cast<const T *>(w), static_cast<uint16_t *>(wsp),
                       static_cast<float *>(wd), flag, g.G, g.Mg, g.Cg, g.Pn, g.Kn, t.c_tiles, t.ms32, t.m_steps,
                       pblocks, zblocks, (int)wblocks,
                       g.Pn % 4 == 0 && reinterpret_cast<uintptr_t>(z) % (4 * sizeof(T)) == 0,
                       static_cast<uint16_t *>(zw), (size_t)g.B * g.M * g.Pn);
    return hipGetLastError();
}

int ilog2(int v) {
    int r = 0;
    while ((1 << r) < v) ++r;
    return r;
}

}  // namespace

WinTiles win_resize(const WinTiles &base, const Geo &g, int dim, size_t fixed_bytes, size_t cell_bytes,
                    long long cell_cap) {
    // window = undeformed footprint of the box (low and high corners) plus a margin R[e] per
    // used axis: first the largest common R (up to 8, 32 in 1D) whose LDS fits beside
    // fixed_bytes and whose cell count stays within cell_cap (0: no cap)
    WinTiles t = base;
    int need[3] = {1, 1, 1};
    for (int e = 3 - dim; e < 3; ++e) need[e] = (t.box[e] - 1) * g.st[e] + (g.K[e] - 1) * g.dil[e] + 2;
    long long max_cells =
        WIN_LDS_TARGET > fixed_bytes ? (long long)((WIN_LDS_TARGET - fixed_bytes) / cell_bytes) : 0;
    if (cell_cap > 0 && max_cells > cell_cap) max_cells = cell_cap;
    int R = 0;
    t.cells = 0;
    if (max_cells > 0) {
        for (R = dim == 1 ? 32 : 8; R > -64; --R) {
            long long cells = 1;
            bool degenerate = false;
            for (int e = 3 - dim; e < 3; ++e) {
                const int ext = need[e] + 2 * R;
                if (ext < 1) degenerate = true;
                cells *= ext;
            }
            if (degenerate) break;
            if (cells <= max_cells) {
                t.cells = (int)cells;
                break;
            }
        }
    }
    // then, while the margins are thin (under 3 cells), one more cell on the axis of the
    // smallest window extent that still fits: a short axis (3D boxes are 4 deep) sends the
    // most samples past its faces
    int Re[3] = {R, R, R};
    if (t.cells > 0) {
        for (;;) {
            int best = -1;
            for (int e = 3 - dim; e < 3; ++e) {
                const int ext = need[e] + 2 * Re[e];
                if (Re[e] >= 3 || (long long)t.cells / ext * (ext + 2) > max_cells) continue;
                if (best < 0 || ext < need[best] + 2 * Re[best]) best = e;
            }
            if (best < 0) break;
            const int ext = need[best] + 2 * Re[best];
            t.cells = t.cells / ext * (ext + 2);
            ++Re[best];
        }
    }
    for (int e = 0; e < 3; ++e) {
        const bool used = e >= 3 - dim;
        t.R[e] = (used && t.cells) ? Re[e] : 0;
        t.WE[e] = (used && t.cells) ? need[e] + 2 * Re[e] : 1;
    }
    return t;
}

WinTiles plan_data_win(const Geo &g, int dtype, int dim, bool scatter, bool coord) {
    WinTiles t{};
    t.ok = false;
    if (dtype == kF64) return t;
    if (g.C % 4 || g.Cg % 4) return t;
    // every 16-channel tile must lie inside one offset group and one mask group
    for (int grp = 0; grp < g.G; ++grp)
        for (int c0 = 0; c0 < g.Cg; c0 += BC) {
            const int first = grp * g.Cg + c0, last = grp * g.Cg + (c0 + BC < g.Cg ? c0 + BC : g.Cg) - 1;
            if ((g.og && first / g.cpo != last / g.cpo) || (g.mg && first / g.cpm != last / g.cpm)) return t;
        }
    // tile box: powers of two per used axis, product 256, no wider than the grid needs
    int box[3] = {1, 1, 1};
    auto p2 = [](int v, int cap) {
        int r = 1;
        while (r < v && r < cap) r <<= 1;
        return r;
    };
    if (dim == 1) {
        box[2] = 256;
    } else if (dim == 2) {
        box[2] = p2(g.P[2], 16);
        box[1] = 256 / box[2];
    } else {
        box[2] = p2(g.P[2], 8);
        box[1] = p2(g.P[1], 8);
        box[0] = 256 / (box[1] * box[2]);
    }
    for (int e = 0; e < 3; ++e) {
        t.box[e] = box[e];
        t.ntile[e] = (g.P[e] + box[e] - 1) / box[e];
    }
    t.lbx = ilog2(box[2]);
    t.lbxy = ilog2(box[1] * box[2]);
    t.c_tiles = (g.Cg + BC - 1) / BC;
    t.m_steps = (g.Mg + BM - 1) / BM;
    // per window cell: the fixed-point accumulators (scatter) and / or the X values
    // (offset/mask gradients), as the launches this plan serves need them
    // (+ BC * 16 words: the fixed-point window's stride rounding)
    const size_t fixed = (FIXED_WORDS + (scatter ? BC * 16 : 0)) * sizeof(float);
    const size_t cell = ((scatter ? BC : 0) + (coord ? XS : 0)) * sizeof(float);
    const WinTiles base = t;
    t = win_resize(base, g, dim, fixed, cell);
    const int npass = (g.Kn + WIN_TMAX - 1) / WIN_TMAX;
    t.tpp = (g.Kn + npass - 1) / npass;
    t.npiece = dtype == kF32 ? 2 : 1;
    // 1D / 2D passes of nine taps: the K loop's weight blocks staged in LDS when the window
    // keeps a margin of min(R, 4) cells beside the buffers (3D: short K loops, and the window
    // needs the room; five-tap 1D passes ran slower staged, with two buffers or with three
    // and each block requested two steps ahead, so shorter passes keep the direct loads)
    t.wstage = 0;
    if (dim < 3 && t.cells > 0 && t.tpp == WIN_TMAX) {
        const int stage = 2 * t.tpp * t.npiece * 1024;
        WinTiles ws = win_resize(base, g, dim, fixed + stage, cell);
        bool keep = ws.cells > 0;
        for (int e = 3 - dim; e < 3; ++e) keep = keep && ws.R[e] >= std::min(t.R[e], 4);
        if (keep) {
            ws.tpp = t.tpp;
            ws.npiece = t.npiece;
            ws.wstage = stage;
            t = ws;
        }
    }
    t.chunk_elems = (size_t)g.G * t.c_tiles * t.m_steps * g.Kn * BC * BM;
    t.ms32 = (g.Mg + 31) / 32;
    t.zs_elems = (size_t)g.B * g.G * t.ms32 * g.Pn * t.npiece * 32;
    t.ws_elems = (size_t)g.G * t.c_tiles * t.ms32 * g.Kn * t.npiece * 512;
    // no window at all (the footprint does not fit): a unit-extent window would still place a
    // corner at its origin cell "inside" it, so these problems take the unwindowed kernels
    t.ok = t.cells > 0;
    return t;
}

hipError_t launch_data_win_prep(int dtype, const Geo &g, const WinTiles &t, const void *z, const void *w, void *zs,
                                void *wsplit, void *wd, int *flag, hipStream_t s, void *zw) {
    switch (dtype) {
        case kF32: return launch_prep<float>(g, t, z, w, zs, wsplit, wd, flag, s, zw);
        case kF16: return launch_prep<__half>(g, t, z, w, zs, wsplit, wd, flag, s, zw);
        case kBF16: return launch_prep<__hip_bfloat16>(g, t, z, w, zs, wsplit, wd, flag, s, zw);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_bwd_data_win(int dtype, int dim, const Geo &g, const WinTiles &t, bool scatter, bool coord,
                               const void *z, const void *wchunks, const void *zs, const void *wsplit,
                               const int *flag, const void *xcl, const void *offset, const void *mask, void *gx_cl,
                               void *goff, void *gmask, hipStream_t s, bool gx_nchw) {
    switch (dtype) {
        case kF32:
            return launch_d<float>(dim, g, t, scatter, coord, z, wchunks, zs, wsplit, flag, xcl, offset, mask, gx_cl,
                                   goff, gmask, s, gx_nchw);
        case kF16:
            return launch_d<__half>(dim, g, t, scatter, coord, z, wchunks, zs, wsplit, flag, xcl, offset, mask, gx_cl,
                                    goff, gmask, s, gx_nchw);
        case kBF16:
            return launch_d<__hip_bfloat16>(dim, g, t, scatter, coord, z, wchunks, zs, wsplit, flag, xcl, offset, mask,
                                            gx_cl, goff, gmask, s, gx_nchw);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
