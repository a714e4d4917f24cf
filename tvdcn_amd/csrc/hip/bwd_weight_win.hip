// Family Wt, windowed variant: weight gradient over tiles whose sampled values are
// formed from an LDS window.
//
//   dW[m][c][t] = sum_{b,p} Z[b][m][p] * mask * bilinear(X[b][c], pos(b, og(c), t, p))
//
// Replaces the reference's im2col recompute + grad_weight addmm_
// (tvdcn/csrc/ops/cuda/deform_conv2d_kernel.cpp:600-626; transposed
// deform_conv_transpose2d_kernel.cpp:586-613; 1D/3D twins).
//
// Workgroup = (group, 16-channel slice, up to 256 GEMM-side rows, a run of (pass,
// spatial tile) units, pass-major, so that the runs are equal whatever the number of
// passes); eight waves, wave w owning 32 rows. The dW block [rows][16 c][taps of the
// pass] stays in accumulators (72 registers per lane) across the run's tiles of a pass.
// Per tile (a box of 256 column pixels of one image, see window.h) the sampling
// table and the X window are filled once; then the tile is walked in 32-pixel
// chunks (one barrier each): the sampled columns S[tap][c][px] of the next chunk are
// formed from the window (LDS reads only, global loads for the rare corners outside it)
// into a double-buffered LDS tile while the MFMAs of the current chunk run, per 16-pixel
// half of the chunk:
//   A = Z[m][px] (4 consecutive pixels per lane, one 16-byte load when contiguous),
//   B = S[px][c] of one tap, D = dW[m][c] of that tap.
// The 16-bit loop (16x16x32 MFMAs, 32-pixel K blocks) keeps a single 16-bit S tile per
// chunk, built from pixel pairs (one 32-bit LDS store per row and piece), and reads its A
// fragments as 16-bit values: 8 pixels of a row per 16-byte load,
// from Z's 16-bit values (fp16 / bf16 as they are, fp32 as fp16 pieces) in 8-pixel column
// blocks (a fragment's 16 rows x 4 blocks are whole lines; written by the data gradient's
// operand-prep launch); the chunks run in pairs with alternating fragment sets.
// At the end of each pass of the run the block is stored to the split's slot of the
// workspace; per tap, the splits whose runs meet its pass are summed in a fixed order
// (deterministic).
#include "window.h"

namespace tvdcn_hip {
namespace {

using namespace win;

constexpr int NW = 8;               // waves per workgroup
constexpr int NT = 64 * NW;
// Row layouts: MB 16-row blocks per wave and TG tap groups. The waves split into TG groups
// of NW / TG; group g takes the taps t = g (mod TG) of every pass for the rows of its waves,
// so that a GEMM side of 64 rows still keeps all eight waves on MFMAs:
//   MB = 2, TG = 1: 256 rows per workgroup;  MB = 1, TG = 2: 64 rows, taps split by parity.
template <int MB, int TG> constexpr int rows_of() { return (NW / TG) * MB * 16; }
// Tap slots and chunk size: TM tap slots per pass held in accumulators, KP pixels per chunk.
// Passes of up to 9 taps take (9, 32); passes of up to 5 taps (1D k <= 5, 2D k = 2) take
// (5, 64): the registers the unused tap slots would hold carry a chunk twice as long, so each
// barrier and operand load serves twice the MFMAs.
template <int TMV, int KPV> struct WShape {
    static constexpr int TM = TMV;
    static constexpr int KP = KPV;          // pixels per chunk (16-pixel MFMA K blocks)
    static constexpr int NCH = BPX / KP;    // chunks per tile
    static constexpr int NH = KP / 16;      // 16-pixel MFMA K blocks per chunk
    static constexpr int SS = KP + 4;       // S tile row stride (rows = (tap, channel))
    static constexpr int GEO_WORDS = TM * BPX * 4;
    static constexpr int SBUF_WORDS = 2 * TM * BC * SS;   // the fp32 loop's S tiles, double-buffered
    static constexpr int SS16 = KP + 8;                   // 16-bit S tile row stride
    // the 16-bit loop's S tile, per piece (a multiple of 4 words: the X window stays 16-byte aligned)
    static constexpr int S16_WORDS = TM * BC * SS16 / 2;
    static_assert(S16_WORDS % 4 == 0 && S16_WORDS * 2 <= SBUF_WORDS, "S16 tile words");
    // S words of an instantiation: the 16-bit loop (np pieces) needs less, and the X window takes the rest
    static constexpr int sbuf_words(bool use16, int np) { return use16 ? np * S16_WORDS : SBUF_WORDS; }
};
constexpr int SMALL_TM = 5;
// the (5, 64) shape serves 256-row tiles (GEMM sides above 128 rows); 64-row tiles split the
// taps between two wave groups and keep (9, 32)
bool small_shape(const Geo &g, int tpp) { return tpp <= SMALL_TM && g.Mg > 128; }
size_t fixed_words(const Geo &g, int tpp, bool use16, int np) {
    return small_shape(g, tpp) ? WShape<SMALL_TM, 64>::GEO_WORDS + WShape<SMALL_TM, 64>::sbuf_words(use16, np)
                               : WShape<WIN_TMAX, 32>::GEO_WORDS + WShape<WIN_TMAX, 32>::sbuf_words(use16, np);
}

// FULL: every pass uses all TM tap slots (no per-tap guards). USE16: the instantiation with the
// 16x16x32 MFMA chunks; it runs when the operand flag is clear and the fp32 one when it
// is set (both are launched; each returns at once when the flag selects the other), so that
// neither loop's registers weigh on the other's.
template <int DIM, typename T, bool FULL, int MB, int TG, int TMV, int KPV, bool USE16>
__global__ void __launch_bounds__(NT)
bwd_weight_win_kernel(const Geo g, const WinTiles wt, const WeightWin ww, const T *__restrict__ z,
                      const float *__restrict__ xcl, const T *__restrict__ offset, const T *__restrict__ mask,
                      float *__restrict__ part, const int *flag, const uint16_t *__restrict__ zw) {
    using SH = WShape<TMV, KPV>;
    constexpr int TM = SH::TM, KP = SH::KP, NCH = SH::NCH, NH = SH::NH, SS = SH::SS;
    constexpr int GEO_WORDS = SH::GEO_WORDS, SBUF_WORDS = SH::sbuf_words(USE16, npiece_of<T>());
    constexpr int NC = 1 << DIM;
    constexpr int BMW = rows_of<MB, TG>();
    extern __shared__ float smem[];
    acc4 *geo = reinterpret_cast<acc4 *>(smem);         // [TM][BPX]
    float *sbuf = smem + GEO_WORDS;                     // [2][TM * BC][SS] (16-bit loop: [NP][TM * BC][SS16])
    float *xwin = smem + GEO_WORDS + SBUF_WORDS;        // [cells][XS]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;

    int L = xcd_remap(blockIdx.x, gridDim.x);
    const int ct = L % wt.c_tiles;
    L /= wt.c_tiles;
    const int mt = L % ww.m_tiles;
    L /= ww.m_tiles;
    const int split = L % ww.n_split;
    const int grp = L / ww.n_split;
    // this split's units u = pass * n_spatial + spatial tile, u in [u_beg, u_end)
    const long long n_sp = ww.n_spatial;
    const long long u_beg = (long long)split * ww.units_per_split;
    const long long u_end = min((long long)((g.Kn + wt.tpp - 1) / wt.tpp) * n_sp, u_beg + ww.units_per_split);
    const bool deformable = offset != nullptr;
    const int tg = wave / (NW / TG);                     // this wave's tap group
    const int mrow = mt * BMW + (wave % (NW / TG)) * (MB * 16);   // first row of this wave
    constexpr bool use16 = USE16;
    if (flag != nullptr && (*flag == 0) != use16) return;   // the other instantiation's launch
    // fp32 as fp16 pieces: the scales of Z and of the sampled columns, and the one back out
    const int s_z = use16 ? operand_scale(flag, AMAX_Z) : 0;
    const int s_s = use16 ? sampled_scale(g, flag, mask != nullptr) : 0;
    const int s_back = npiece_of<T>() == 2 && use16 ? -(s_z + s_s) : 0;

    if constexpr (DIM == 3) {
        if (tid < XS) xwin[wt.cells * XS + tid] = 0.f;   // zero cell of the 3D corner reads
    }

    // S-builder item of this thread: chunk pixel j, channel quad sq, taps st, st + SSTEP, ...
    // (3D: chunk pixel j, taps tid / KP, + NT / KP, ..., all 16 channels)
    const int sj = tid % KP, sq = (tid / KP) & 3, st0 = tid / (KP * 4);
    constexpr int SSTEP = NT / (KP * 4);   // tap stride of the items
    // (16-bit S tile, 1D / 2D: chunk pixel pair pj, channel quad pq, taps pt0, pt0 + PSTEP, ...)
    const int pj = tid % (KP / 2), pq = (tid / (KP / 2)) & 3, pt0 = tid / (KP * 2);
    constexpr int PSTEP = NT / (KP * 2);

    for (int pass = (int)(u_beg / n_sp); (long long)pass * n_sp < u_end; ++pass) {
        const int t0 = pass * wt.tpp;
        const int ntaps = min(wt.tpp, g.Kn - t0);
        const int s_beg = (int)(max(u_beg, pass * n_sp) - pass * n_sp);
        const int s_end = (int)(min(u_end, (pass + 1) * n_sp) - pass * n_sp);

        acc4 acc[MB][TM];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int tp = 0; tp < TM; ++tp) acc[mb][tp] = acc4{0.f, 0.f, 0.f, 0.f};

        for (int s = s_beg; s < s_end; ++s) {
            Tile tile;
            tile.init(g, wt, s, ct, grp);
            const float *xb = xcl + (size_t)tile.b * g.Sn * g.C + tile.cg0;
            __syncthreads();   // previous tile done with the tables
            fill_geo<DIM, T, 5, true>(g, wt, tile, offset, mask, t0, ntaps, geo, tid, NT);
            fill_xwin(g, wt, tile, xb, xwin, tid, NT);
            __syncthreads();

            // mask * sampled value of channels 4 sqv .. + 3 at (tap tl, tile pixel i) (1D / 2D)
            auto sample_quad = [&](int tl, int i, int sqv) -> acc4 {
                const bool cq_ok = tile.c0 + 4 * sqv < g.Cg;
                const acc4 r = geo[tl * BPX + i];
                const int fc = fast_cell<DIM>(r);
                const float mk = rec_mask<DIM>(r);
                acc4 sv;
                if (fc >= 0) {
                    // every corner cell is in the window (zeros outside the grid)
                    sv = window_sample_masked<DIM>(wt, xwin, fc, 4 * sqv, r, mk);
                } else {
                    const AxisW<DIM, float> aw = record_weights<DIM>(g, r, deformable);
                    sv = acc4{0.f, 0.f, 0.f, 0.f};
                    if (aw.inside) {
#pragma unroll
                        for (int kk = 0; kk < NC; ++kk) {
                            int idx;
                            bool v;
                            corner_at<DIM, float>(g, aw, kk, idx, v);
                            if (!v) continue;
                            const int cell = tile.corner_cell<DIM>(wt, aw, kk);
                            // LDS read unconditional (clamped), global read in its own branch:
                            // the two address spaces are never merged into one pointer
                            acc4 x = *reinterpret_cast<const acc4 *>(xwin + max(cell, 0) * XS + 4 * sqv);
                            if (cell < 0) {
                                x = acc4{0.f, 0.f, 0.f, 0.f};
                                if (cq_ok) x = *reinterpret_cast<const acc4 *>(xb + (size_t)idx * g.C + 4 * sqv);
                            }
                            sv += corner_weight<DIM, float>(aw, kk) * x;
                        }
                    }
                    sv *= mk;
                }
                return sv;
            };
            // S[tap][c][px] of chunk k into buffer bf
            auto build_s = [&](int k, int bf) {
                float *dst = sbuf + bf * (TM * BC * SS);
                const int i = k * KP + sj;
                if constexpr (DIM == 3) {
                    // 3D: one item per (chunk pixel, tap) for all 16 channels (the corner geometry
                    // formed once per sample rather than once per channel quad)
                    const int nq = min(4, (g.Cg - tile.c0) >> 2);
                    for (int tl = tid / KP; tl < ntaps; tl += NT / KP) {
                        const acc4 r = geo[tl * BPX + i];
                        acc4 sv[4];
                        if (nq == 4)
                            sample3_all_fix<true>(g, wt, tile, xwin, xb, 4, r, deformable, sv);
                        else
                            sample3_all_fix<false>(g, wt, tile, xwin, xb, nq, r, deformable, sv);
                        float *row = dst + tl * BC * SS + sj;
#pragma unroll
                        for (int j = 0; j < 4; ++j)
#pragma unroll
                            for (int v = 0; v < 4; ++v) row[(4 * j + v) * SS] = sv[j][v];
                    }
                    return;
                }
                for (int tl = st0; tl < ntaps; tl += SSTEP) {
                    const acc4 sv = sample_quad(tl, i, sq);
                    float *row = dst + (tl * BC + 4 * sq) * SS + sj;
#pragma unroll
                    for (int v = 0; v < 4; ++v) row[v * SS] = sv[v];
                }
            };

            // A operand: Z[m][4 consecutive chunk pixels], m = mrow + mb * 16 + lane % 16
            const T *zrow[MB];
            size_t zblk[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = min(mrow + mb * 16 + (lane & 15), g.Mg - 1);
                zblk[mb] = (size_t)tile.b * g.M * g.Pn + ((size_t)tile.grp * g.Mg + m) * 8;
                zrow[mb] = z + ((size_t)tile.b * g.M + (size_t)tile.grp * g.Mg + m) * g.Pn;
            }
            // quad path: a 16-pixel half chunk lies within one row of the box (box_x >= 16) and
            // P_x % 4 == 0, so the lane's 4 pixels are consecutive and all inside or all outside
            // the grid; in a tile wholly inside the grid every quad is inside
            const bool quad = ww.z_vec && wt.box[2] >= 16;
            const bool tile_in = tile.p0[0] + wt.box[0] <= g.P[0] && tile.p0[1] + wt.box[1] <= g.P[1] &&
                                 tile.p0[2] + wt.box[2] <= g.P[2];
            const bool full = quad && tile_in;
            // Z of half h of chunk k (pixels k * KP + 16 h + 4 * (lane / 16) .. + 3); pixels
            // outside the grid stay 0 (never loaded, so that a non-finite value there cannot
            // leak into the sums)
            auto load_a = [&](int k, int h, acc4 (&za)[MB]) {
                const int i0 = k * KP + 16 * h + 4 * q;
                if (quad) {
                    const int iz = i0 >> wt.lbxy, iy = (i0 >> wt.lbx) & (wt.box[1] - 1), ix = i0 & (wt.box[2] - 1);
                    const int pz = tile.p0[0] + iz, py = tile.p0[1] + iy, px = tile.p0[2] + ix;
                    const int p = (pz * g.P[1] + py) * g.P[2] + px;
                    if (full) {
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb) {
                            const Vec4<float> v = load4_t<float, T>(zrow[mb] + p);
                            za[mb] = acc4{v.x, v.y, v.z, v.w};
                        }
                    } else {
                        const bool ok = pz < g.P[0] && py < g.P[1] && px < g.P[2];
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb) {
                            za[mb] = acc4{0.f, 0.f, 0.f, 0.f};
                            if (ok) {
                                const Vec4<float> v = load4_t<float, T>(zrow[mb] + p);
                                za[mb] = acc4{v.x, v.y, v.z, v.w};
                            }
                        }
                    }
                } else {
                    int pu[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) pu[u] = tile.pixel(g, wt, i0 + u);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            za[mb][u] = 0.f;
                            if (pu[u] >= 0) za[mb][u] = to_acc<float>(zrow[mb][pu[u]]);
                        }
                }
            };

            if (use16) {
                // ---- 16-bit chunks: S16 [NP][TM * BC][SS16] (16-bit, single buffer) built from
                //      the window, its values split into pieces once per value (fp32) or rounded
                //      to T (the reference's columns of a half-precision input are half); per
                //      32-pixel K block, A = Z[m][8 consecutive pixels of lane group q] (pieces
                //      formed in registers), B = S16[tap][c][the same pixels]
                constexpr int NP = npiece_of<T>();
                constexpr int SS16 = SH::SS16;
                constexpr int KB = KP / 32;
                static_assert(NP * TM * BC * SS16 * 2 <= SBUF_WORDS * 4, "the S16 tile fits its buffer");
                uint16_t *s16 = reinterpret_cast<uint16_t *>(sbuf);
                auto build_s16 = [&](int k) {
                    const int i = k * KP + sj;
                    if constexpr (DIM == 3) {
                        // 3D: one item per (chunk pixel, tap) for all 16 channels, as in build_s
                        const int nq = min(4, (g.Cg - tile.c0) >> 2);
                        for (int tl = tid / KP; tl < ntaps; tl += NT / KP) {
                            const acc4 r = geo[tl * BPX + i];
                            acc4 sv[4];
                            if (nq == 4)
                                sample3_all_fix<true>(g, wt, tile, xwin, xb, 4, r, deformable, sv);
                            else
                                sample3_all_fix<false>(g, wt, tile, xwin, xb, nq, r, deformable, sv);
#pragma unroll
                            for (int j = 0; j < 4; ++j)
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    uint16_t pc[NP];
                                    split_one16<T, NP>(sv[j][v], s_s, pc);
#pragma unroll
                                    for (int kk = 0; kk < NP; ++kk)
                                        s16[((size_t)kk * TM * BC + tl * BC + 4 * j + v) * SS16 + sj] = pc[kk];
                                }
                        }
                        return;
                    }
                    // 1D / 2D: item = (two consecutive chunk pixels, channel quad, tap), so that each
                    // (row, piece) takes one 32-bit LDS store of the two pixels' values, and the fp32
                    // split runs on the pair (packed conversions)
                    const int i0 = k * KP + 2 * pj;
                    for (int tl = pt0; tl < ntaps; tl += PSTEP) {
                        const acc4 s0 = sample_quad(tl, i0, pq), s1 = sample_quad(tl, i0 + 1, pq);
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            uint32_t w[NP];
                            if constexpr (NP == 2)
                                split2_pk(s0[v], s1[v], s_s, w);
                            else
                                w[0] = pack2_16<T>(s0[v], s1[v]);
#pragma unroll
                            for (int kk = 0; kk < NP; ++kk)
                                *reinterpret_cast<uint32_t *>(s16 + ((size_t)kk * TM * BC + tl * BC + 4 * pq + v) * SS16 +
                                                              2 * pj) = w[kk];
                        }
                    }
                };
                // Z of K block kb of chunk k: pixels k * KP + 32 kb + 8 q .. + 7 (zero outside the grid)
                auto load_a8 = [&](int k, int kb, float (&za)[MB][8]) {
                    const int i0 = k * KP + 32 * kb + 8 * q;
                    if (quad) {
                        // the 8 pixels lie in one row of the box (box_x >= 16, 8-aligned), each
                        // half of 4 wholly inside or outside the grid (P_x % 4 == 0)
                        const int iz = i0 >> wt.lbxy, iy = (i0 >> wt.lbx) & (wt.box[1] - 1), ix = i0 & (wt.box[2] - 1);
                        const int pz = tile.p0[0] + iz, py = tile.p0[1] + iy, px = tile.p0[2] + ix;
                        const int p = (pz * g.P[1] + py) * g.P[2] + px;
                        const bool row_ok = pz < g.P[0] && py < g.P[1];
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const bool ok = full || (row_ok && px + 4 * h < g.P[2]);
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb) {
                                Vec4<float> v{0.f, 0.f, 0.f, 0.f};
                                if (ok) v = load4_t<float, T>(zrow[mb] + p + 4 * h);
                                za[mb][4 * h] = v.x;
                                za[mb][4 * h + 1] = v.y;
                                za[mb][4 * h + 2] = v.z;
                                za[mb][4 * h + 3] = v.w;
                            }
                        }
                    } else {
                        int pu[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) pu[u] = tile.pixel(g, wt, i0 + u);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                            for (int u = 0; u < 8; ++u) za[mb][u] = pu[u] >= 0 ? to_acc<float>(zrow[mb][pu[u]]) : 0.f;
                    }
                };
                // A fragments of K block kb of chunk k: with zw (Z as 16-bit values in its own layout:
                // fp16 / bf16 Z itself, the pieces of an fp32 Z), 8 pixels of a row per 16-byte load;
                // else loaded as fp32 and split here. Pixels outside the grid stay 0.
                const bool zdirect = zw != nullptr && ww.z8;
                const size_t zplane = (size_t)g.B * g.M * g.Pn;
                auto load_frag = [&](int k, int kb, uint4 (&za)[MB][NP]) {
                    if (zdirect) {
                        const int i0 = k * KP + 32 * kb + 8 * q;
                        const int iz = i0 >> wt.lbxy, iy = (i0 >> wt.lbx) & (wt.box[1] - 1), ix = i0 & (wt.box[2] - 1);
                        const int pz = tile.p0[0] + iz, py = tile.p0[1] + iy, px = tile.p0[2] + ix;
                        const int p = (pz * g.P[1] + py) * g.P[2] + px;
                        // (the 8 pixels lie in one row of the box, px % 8 == 0 and P_x % 8 == 0: all
                        // inside the grid or all outside)
                        const bool ok = tile_in || (pz < g.P[0] && py < g.P[1] && px < g.P[2]);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                            for (int kk = 0; kk < NP; ++kk) {
                                za[mb][kk] = uint4{0u, 0u, 0u, 0u};
                                // (Z's 16-bit values in 8-pixel column blocks, data_prep_kernel)
                                if (ok)
                                    za[mb][kk] = *reinterpret_cast<const uint4 *>(
                                        zw + zblk[mb] + (size_t)(p >> 3) * (g.M * 8) + kk * zplane);
                            }
                    } else {
                        float v[MB][8];
                        load_a8(k, kb, v);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb) pack8_16<T, NP>(v[mb], s_z, za[mb]);
                    }
                };
                // chunk k on the A fragments in cur, those of chunk k + 1 loaded into nxt
                auto chunk = [&](int k, const uint4 (&cur)[KB][MB][NP], uint4 (&nxt)[KB][MB][NP]) {
                    __syncthreads();   // every wave done with the previous chunk's S16 tile
                    build_s16(k);
                    if (k + 1 < NCH) {
#pragma unroll
                        for (int kb = 0; kb < KB; ++kb) load_frag(k + 1, kb, nxt[kb]);
                    }
                    __syncthreads();
                    const uint16_t *sb = s16 + (size_t)(lane & 15) * SS16 + 8 * q;
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                        for (int tp = 0; tp < TM; ++tp) {
                            if ((FULL || tp < ntaps) && (TG == 1 || tp % TG == tg)) {
                                uint4 bf[NP];
#pragma unroll
                                for (int kk = 0; kk < NP; ++kk)
                                    bf[kk] = *reinterpret_cast<const uint4 *>(sb + ((size_t)kk * TM * BC + tp * BC) * SS16 + 32 * kb);
#pragma unroll
                                for (int mb = 0; mb < MB; ++mb)
                                    acc[mb][tp] = mfma16x16x32_np<T, NP>(cur[kb][mb], bf, acc[mb][tp]);
                            }
                        }
                    }
                };
                // chunks in pairs, the fragment sets alternating (no copies between chunks)
                static_assert(NCH % 2 == 0, "an even number of chunks per tile");
                uint4 za[KB][MB][NP], zb[KB][MB][NP];
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) load_frag(0, kb, za[kb]);
                for (int k = 0; k < NCH; k += 2) {
                    chunk(k, za, zb);
                    chunk(k + 1, zb, za);
                }
            } else {
                acc4 za[NH][MB], zn[NH][MB];
#pragma unroll
                for (int h = 0; h < NH; ++h) load_a(0, h, za[h]);
                build_s(0, 0);
                __syncthreads();
                for (int k = 0; k < NCH; ++k) {
                    const int bf = k & 1;
                    const bool more = k + 1 < NCH;
                    if (more) {
#pragma unroll
                        for (int h = 0; h < NH; ++h) load_a(k + 1, h, zn[h]);
                    }
                    const float *sb = sbuf + bf * (TM * BC * SS) + (lane & 15) * SS + 4 * q;
#pragma unroll
                    for (int h = 0; h < NH; ++h)
#pragma unroll
                        for (int tp = 0; tp < TM; ++tp) {
                            if ((FULL || tp < ntaps) && (TG == 1 || tp % TG == tg)) {
                                const acc4 bv = *reinterpret_cast<const acc4 *>(sb + tp * BC * SS + 16 * h);
#pragma unroll
                                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                                    for (int mb = 0; mb < MB; ++mb)
                                        acc[mb][tp] = mfma16x16x4(za[h][mb][kk], bv[kk], acc[mb][tp]);
                            }
                        }
                    if (more) {
                        build_s(k + 1, bf ^ 1);
#pragma unroll
                        for (int h = 0; h < NH; ++h)
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb) za[h][mb] = zn[h][mb];
                    }
                    __syncthreads();
                }
            }
        }

        // this split's block: part[split][grp][t][m][c]
#pragma unroll
        for (int tp = 0; tp < TM; ++tp) {
            if (tp >= ntaps || (TG > 1 && tp % TG != tg)) continue;
            float *dst = part + (((size_t)split * g.G + grp) * g.Kn + t0 + tp) * g.Mg * (size_t)g.Cg;
            const int c = ct * BC + (lane & 15);
            if (c >= g.Cg) continue;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int m = mrow + mb * 16 + 4 * q + v;
                    if (m < g.Mg) dst[(size_t)m * g.Cg + c] = s_back != 0 ? ldexpf(acc[mb][tp][v], s_back) : acc[mb][tp][v];
                }
        }
    }
}

template <int DIM, typename T, bool FULL, int MB, int TG, int TMV, int KPV, bool USE16>
hipError_t launch_k1(const Geo &g, const WinTiles &wt, const WeightWin &ww, const void *z, const void *xcl,
                     const void *offset, const void *mask, void *part, const int *flag, const void *zw, hipStream_t s) {
    using SH = WShape<TMV, KPV>;
    auto kern = bwd_weight_win_kernel<DIM, T, FULL, MB, TG, TMV, KPV, USE16>;
    const size_t lds = ((size_t)SH::GEO_WORDS + SH::sbuf_words(USE16, npiece_of<T>()) +
                        (size_t)(wt.cells + (DIM == 3)) * XS) *
                       sizeof(float);
    static std::atomic<unsigned long long> lds_raised{0};   // per device, see raise_lds_limit
    if (const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kern), lds_raised); e != hipSuccess)
        return e;
    const long long blocks = (long long)g.G * ww.n_split * ww.m_tiles * wt.c_tiles;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NT), lds, s, g, wt, ww, static_cast<const T *>(z),
                       static_cast<const float *>(xcl), static_cast<const T *>(offset), static_cast<const T *>(mask),
                       static_cast<float *>(part), flag, USE16 ? static_cast<const uint16_t *>(zw) : nullptr);
    return hipGetLastError();
}

// the fp32 instantiation, and (with an operand flag) the 16-bit one beside it
template <int DIM, typename T, bool FULL, int MB, int TG, int TMV, int KPV>
hipError_t launch_k(const Geo &g, const WinTiles &wt, const WinTiles &wt16, const WeightWin &ww, const void *z,
                    const void *xcl, const void *offset, const void *mask, void *part, const int *flag,
                    const void *zw, hipStream_t s) {
    if (wt.tpp > TMV || wt16.tpp != wt.tpp) return hipErrorInvalidValue;   // a pass must fit the tap slots
    if (flag != nullptr) {
        const hipError_t e = launch_k1<DIM, T, FULL, MB, TG, TMV, KPV, true>(g, wt16, ww, z, xcl, offset, mask, part,
                                                                              flag, zw, s);
        if (e != hipSuccess) return e;
    }
    return launch_k1<DIM, T, FULL, MB, TG, TMV, KPV, false>(g, wt, ww, z, xcl, offset, mask, part, flag, nullptr, s);
}

template <typename T>
hipError_t launch_d(int dim, const Geo &g, const WinTiles &wt, const WinTiles &wt16, const WeightWin &ww, const void *z,
                    const void *xcl, const void *offset, const void *mask, void *part, const int *flag, const void *zw,
                    hipStream_t s) {
    const bool small = small_shape(g, wt.tpp);
    const int tm = small ? SMALL_TM : WIN_TMAX;
    const bool full = wt.tpp == tm && g.Kn % tm == 0;
    auto pick = [&](auto dim_tag) -> hipError_t {
        constexpr int D = decltype(dim_tag)::value;
        if (ww.tg == 2) return full ? launch_k<D, T, true, 1, 2, WIN_TMAX, 32>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s)
                                    : launch_k<D, T, false, 1, 2, WIN_TMAX, 32>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s);
        if (small)
            return full ? launch_k<D, T, true, 2, 1, SMALL_TM, 64>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s)
                        : launch_k<D, T, false, 2, 1, SMALL_TM, 64>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s);
        return full ? launch_k<D, T, true, 2, 1, WIN_TMAX, 32>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s)
                    : launch_k<D, T, false, 2, 1, WIN_TMAX, 32>(g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s);
    };
    switch (dim) {
        case 1: return pick(std::integral_constant<int, 1>());
        case 2: return pick(std::integral_constant<int, 2>());
        case 3: return pick(std::integral_constant<int, 3>());
    }
    return hipErrorInvalidValue;
}

}  // namespace

size_t weight_win_fixed_bytes(const Geo &g, int dim, int tpp, int npiece) {
    return (fixed_words(g, tpp, npiece > 0, npiece) + (dim == 3 ? XS : 0)) * sizeof(float);
}

WeightWin plan_weight_win(const Geo &g, const WinTiles &wt, int dim) {
    WeightWin w{};
    w.ok = false;
    // needs the windowed tiling; GEMM sides up to 128 rows take 64-row tiles with the taps
    // split between two wave groups, larger ones 256-row tiles
    if (!wt.ok || wt.cells == 0 || g.Mg < 16 || weight_win_fixed_bytes(g, dim, wt.tpp, 0) + (size_t)wt.cells * XS * 4 > WIN_LDS_TARGET)
        return w;
    w.tg = g.Mg <= 128 ? 2 : 1;
    const int rows = w.tg == 2 ? rows_of<1, 2>() : rows_of<2, 1>();
    w.m_tiles = (g.Mg + rows - 1) / rows;
    w.n_spatial = g.B * wt.ntile[0] * wt.ntile[1] * wt.ntile[2];
    const long long per_split_groups = (long long)g.G * w.m_tiles * wt.c_tiles;
    // one workgroup per CU, about one wave of workgroups, over units of (pass, spatial tile)
    const long long units = (long long)((g.Kn + wt.tpp - 1) / wt.tpp) * w.n_spatial;
    if (units > INT_MAX) return w;   // the reduction indexes units in 32 bits
    long long splits = (256 + per_split_groups - 1) / per_split_groups;
    if (splits > units) splits = units;
    if (splits < 1) splits = 1;
    // (at least one unit per split: an empty batch has no spatial tiles)
    w.units_per_split = (int)std::max<long long>(1, (units + splits - 1) / splits);
    w.n_split = (int)std::max<long long>(1, (units + w.units_per_split - 1) / w.units_per_split);
    w.z_vec = g.P[2] % 4 == 0 && wt.box[2] >= 4;
    w.z8 = g.P[2] % 8 == 0 && wt.box[2] >= 8;
    w.part_elems = (size_t)w.n_split * g.G * g.Kn * g.Mg * g.Cg;
    w.ok = g.B > 0;
    return w;
}

hipError_t launch_bwd_weight_win(int dtype, int dim, const Geo &g, const WinTiles &wt, const WinTiles &wt16,
                                 const WeightWin &ww, const void *z, const void *xcl, const void *offset,
                                 const void *mask, void *part, void *gw, bool accumulate, const int *flag,
                                 hipStream_t s, const void *zw) {
    // the 16-bit loop's A fragments straight from Z's 16-bit values in column blocks (zw)
    if (!ww.z8) zw = nullptr;
    hipError_t e = hipErrorInvalidValue;
    switch (dtype) {
        case kF32: e = launch_d<float>(dim, g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s); break;
        case kF16: e = launch_d<__half>(dim, g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s); break;
        case kBF16:
            e = launch_d<__hip_bfloat16>(dim, g, wt, wt16, ww, z, xcl, offset, mask, part, flag, zw, s);
            break;
    }
    if (e != hipSuccess) return e;
    return launch_weight_reduce(dtype, g, ww.n_split, part, gw, accumulate, s, ww.units_per_split, ww.n_spatial,
                                wt.tpp);
}

}  // namespace tvdcn_hip
