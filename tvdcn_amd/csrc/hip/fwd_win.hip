// Family F, windowed variant: the forward gather-GEMM with the sampled columns formed
// from an LDS window of the sampled tensor.
//
//   Y[b][m][p] = bias[m] + sum_{t, c in group} W[m][c][t] * mask * bilinear(X[b][c], pos(b, og(c), t, p))
//
// Replaces the reference's im2col kernel + addmm_ pair
// (tvdcn/csrc/ops/cuda/deform_conv2d_common_kernels.cu:138-256 and
// deform_conv2d_kernel.cpp:341-380; 1D/3D twins); the columns are never written
// to HBM. Also computes the transposed op's input gradient.
//
// Workgroup = (spatial tile of 256 column pixels, 128 or 64 GEMM-side rows); eight
// waves, wave w owning 32 pixels x all rows (64 or 32 accumulators per lane; 64-row
// tiles serve small GEMM sides and grids too small to fill the chip). The reduction runs
// over 16-channel slices x taps; per step (slice, tap) every lane forms its own MFMA
// B fragment -- the sampled values of 4 channels of one of its pixels -- straight from
// the X window (LDS) and the sampling table, one step ahead, while the MFMAs of the
// current step run with A = W[m][c] (16-byte fragments of the re-laid-out weight, each
// reloaded for the next step right after its last use). Waves own disjoint pixels, so
// nothing is exchanged between them inside a slice: barriers only where the X window
// of the next slice (prefetched into registers during the last step of the current
// one) replaces the current one, and where the sampling table is rebuilt (when the
// offset / mask group changes). See window.h for the tile / window machinery.
#include "window.h"

namespace tvdcn_hip {
namespace {

using namespace win;

constexpr int NW = 8;               // waves per workgroup
constexpr int NT = 64 * NW;
constexpr int PB = 2;               // 16-pixel blocks per wave
constexpr int TM = WIN_TMAX;
constexpr int PF = 3;               // X window prefetch distance, steps
// MB = 16-row blocks per wave (rows per workgroup 16 * MB); XQ = X window quads
// prefetched per thread (cells * 4 <= XQ * NT): the 64-row variant spends the
// registers its smaller accumulator frees on a larger window
constexpr int xq_of(int mb) { return mb == 8 ? 8 : 12; }
static_assert(NW * PB * 16 == BPX, "one tile of pixels per workgroup");

constexpr int GEO_WORDS = TM * BPX * 4;

// STAGE: the 16-bit loop's weight blocks are staged in LDS (1D / 2D, fw.stage_bytes > 0)
template <int DIM, typename T, int MB, bool STAGE>
__global__ void __launch_bounds__(NT)
fwd_win_kernel(const Geo g, const WinTiles wt, const FwdWin fw, const float *__restrict__ xcl,
               const float *__restrict__ wf, const uint16_t *__restrict__ w16, const int *flag,
               const T *__restrict__ offset, const T *__restrict__ mask, const T *__restrict__ bias,
               T *__restrict__ y, float *__restrict__ y32) {
    constexpr int NC = 1 << DIM;
    constexpr int BMR = MB * 16;
    constexpr int XQ = xq_of(MB);
    extern __shared__ float smem[];
    acc4 *geo = reinterpret_cast<acc4 *>(smem);     // [TM][BPX]
    float *xwin = smem + GEO_WORDS;                 // [cells][XS]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;

    int L = xcd_remap(blockIdx.x, gridDim.x);
    const int mt = L % fw.m_tiles;
    L /= fw.m_tiles;
    const int ks = L % fw.ksplit;   // share of the channel slices (fw.ksplit == 2: fp32 partials in y32)
    L /= fw.ksplit;
    const int n_sp = g.B * wt.ntile[0] * wt.ntile[1] * wt.ntile[2];
    const int sp = L % n_sp;
    const int grp = L / n_sp;
    const bool deformable = offset != nullptr;
    const int slices = (g.Cg + BC - 1) / BC;
    // the 16-bit loop when its weight was laid out and (fp32) no operand was flagged
    const bool use16_flag = w16 != nullptr && (flag == nullptr || *flag == 0);
    // fp32 as fp16 pieces: the sampled columns' scale, and the one back out (the weight's with it)
    const int s_b = npiece_of<T>() == 2 && use16_flag ? sampled_scale(g, flag, mask != nullptr) : 0;
    const int s_back = npiece_of<T>() == 2 && use16_flag ? -(s_b + operand_scale(flag, AMAX_W)) : 0;
    // the sampling table's masks carry 2^s_b, so that the B fragments come out of the sampling at
    // their pieces' scale
    const float mscale_b = ldexpf(1.f, s_b);
    const int cs_lo = ks * fw.slices_per, cs_hi = min(slices, cs_lo + fw.slices_per);

    Tile tile;
    tile.init(g, wt, sp, 0, grp);
    if constexpr (DIM == 3) {
        if (tid < XS) xwin[wt.cells * XS + tid] = 0.f;   // zero cell of the 3D corner reads
    }
    const float *xg = xcl + (size_t)tile.b * g.Sn * g.C + (size_t)grp * g.Cg;   // group's channel 0


    // X window prefetch: quad e = tid + j * NT of the window (cell e / 4, quad e % 4). The
    // cells (and their grid indices) are the same for every slice: resolved once.
    // (3D resolves them at each fill: its registers are taken by the B fragments of a tap group)
    int xsi[XQ];   // flat sampled-grid index of the thread's cells (-1: outside the grid / window)
    auto resolve_cells = [&]() {
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int e = tid + j * NT;
            xsi[j] = e < wt.cells * 4 ? tile.cell_index(g, wt, e >> 2) : -1;
        }
    };
    if constexpr (DIM != 3) resolve_cells();
    acc4 xpre[XQ];
    auto prefetch_x = [&](int cs) {
        const float *xb = xg + cs * BC + 4 * (tid & 3);
        const bool q_ok = cs * BC + 4 * (tid & 3) < g.Cg;   // quad of thread tid + j * NT is tid % 4
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            xpre[j] = acc4{0.f, 0.f, 0.f, 0.f};
            if (xsi[j] >= 0 && q_ok) xpre[j] = *reinterpret_cast<const acc4 *>(xb + (size_t)xsi[j] * g.C);
        }
    };
    auto store_x = [&]() {
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int e = tid + j * NT;
            if (e < wt.cells * 4) *reinterpret_cast<acc4 *>(xwin + (e >> 2) * XS + 4 * (e & 3)) = xpre[j];
        }
    };

    // B fragment of pixel block pb for (slice cs, tap tl of the pass): the sampled values of
    // channels cs * 16 + 4 * (lane / 16) .. + 3 at pixel wave * 32 + pb * 16 + lane % 16
    auto build_b = [&](int cs, int tl, acc4 (&bv)[PB]) {
        const int qd = q;
        const bool q_ok = cs * BC + 4 * qd < g.Cg;
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) {
            const acc4 r = geo[tl * BPX + wave * (PB * 16) + pb * 16 + (lane & 15)];
            const int fc = fast_cell<DIM>(r);
            const float mk = rec_mask<DIM>(r);
            acc4 sv;
            if (fc >= 0) {
                sv = window_sample_masked<DIM>(wt, xwin, fc, 4 * qd, r, mk);
            } else {
                Point<DIM, float> pt;
#pragma unroll
                for (int a = 0; a < DIM; ++a) {
                    pt.pos[a] = r[a];
                    pt.base[a] = (int)r[a];
                }
                const AxisW<DIM, float> aw = axis_weights<DIM, float>(g, pt, deformable);
                sv = acc4{0.f, 0.f, 0.f, 0.f};
                if (aw.inside) {
#pragma unroll
                    for (int kk = 0; kk < NC; ++kk) {
                        int idx;
                        bool v;
                        corner_at<DIM, float>(g, aw, kk, idx, v);
                        if (!v) continue;
                        const int cell = tile.corner_cell<DIM>(wt, aw, kk);
                        // LDS read unconditional (clamped), global read in its own branch: the two
                        // address spaces are never merged into one pointer
                        acc4 x = *reinterpret_cast<const acc4 *>(xwin + max(cell, 0) * XS + 4 * qd);
                        if (cell < 0) {
                            x = acc4{0.f, 0.f, 0.f, 0.f};
                            if (q_ok) x = *reinterpret_cast<const acc4 *>(xg + cs * BC + (size_t)idx * g.C + 4 * qd);
                        }
                        sv += corner_weight<DIM, float>(aw, kk) * x;
                    }
                }
                sv *= mk;
            }
            bv[pb] = sv;
        }
    };

    // A operand: W[m][c] fragments, rows m = mt * BMR + mb * 16 + lane % 16, channels
    // 4 * (lane / 16) .. + 3 of the slice. Layout Wp[grp][slice][t][Mg_pad / 16][16 m][16 c]
    // (fwd_win_weight_kernel): the row blocks of one (slice, tap) are 1 KB apart and each
    // is one contiguous 1 KB wave load; consecutive taps of a slice are adjacent.
    const size_t step_elems = (size_t)fw.Mg_pad * BC;
    const float *wlane = wf + (size_t)grp * slices * g.Kn * step_elems + (size_t)mt * MB * 256 + (lane & 15) * BC + 4 * q;
    auto wptr = [&](int cs, int t) { return wlane + ((size_t)cs * g.Kn + t) * step_elems; };
    auto load_w = [&](const float *p, acc4 (&wr)[MB]) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) wr[mb] = *reinterpret_cast<const acc4 *>(p + mb * 256);
    };

    acc4 acc[MB][PB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) acc[mb][pb] = acc4{0.f, 0.f, 0.f, 0.f};

    // MFMAs of one step with B fragments bv and A fragments wr; each row block's fragment
    // is reloaded from pn (the next step's, or this step's own at the end of a pass) right
    // after its last use (issue order pinned)
    auto mfma_step = [&](const acc4 (&bv)[PB], acc4 (&wr)[MB], const float *pn) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int pb = 0; pb < PB; ++pb) acc[mb][pb] = mfma16x16x4(wr[mb][kk], bv[pb][kk], acc[mb][pb]);
            wr[mb] = *reinterpret_cast<const acc4 *>(pn + mb * 256);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // switch the tables to slice cs: X window from the prefetch registers, sampling
    // table rebuilt when the slice's offset / mask group differs from the last one
    int geo_og = -1, geo_mg = -1;
    auto open_slice = [&](int cs, int t0, int ntaps) {
        if constexpr (DIM == 3) {
            resolve_cells();
            prefetch_x(cs);
        }
        store_x();
        const int c_first = grp * g.Cg + cs * BC;
        const int og_s = g.og ? c_first / g.cpo : 0, mg_s = g.mg ? c_first / g.cpm : 0;
        if (og_s != geo_og || mg_s != geo_mg) {
            tile.ogu = og_s;
            tile.mgu = mg_s;
            // (the sampled values' piece scale folded into the records' masks)
            fill_geo<DIM, T, 3, true>(g, wt, tile, offset, mask, t0, ntaps, geo, tid, NT, mscale_b);
            geo_og = og_s;
            geo_mg = mg_s;
        }
    };

    // ---- 16-bit pass (1D / 2D): steps of (slice, tap pair) on 16x16x32 MFMAs. Lane (row
    //      l % 16, K group q = l / 16) holds at e = 0..7 the value of channel 4q + e % 4 at tap
    //      2j + e / 4 of the pair: its B fragment is the pair's two sampled quads (zero past the
    //      pass), split into pieces for fp32 and rounded to T otherwise (the reference's columns
    //      of a half-precision input are half). W16 holds the A fragments in the same K order.
    //      The weight blocks are staged in LDS (below).
    auto pass16 = [&](int t0, int ntaps) {
        if constexpr (DIM < 3) {
            constexpr int NP = npiece_of<T>();
            const int npair = (ntaps + 1) >> 1;
            const int nsteps = (cs_hi - cs_lo) * npair;
            geo_og = geo_mg = -1;   // a new pass of taps: the table must be rebuilt
            const int nmb = fw.Mg_pad / 16;
            const int pp0 = (t0 / wt.tpp) * fw.hp;
            // (the step's block: wave-uniform; lanes add their offsets when they load)
            const uint16_t *wl = w16 + (size_t)mt * MB * (NP * 512);
            auto wptr16 = [&](int cs, int j) {
                return wl + (((size_t)grp * slices + cs) * fw.pp + pp0 + j) * nmb * (NP * 512);
            };
            auto build_pair = [&](int cs, int j, uint4 (&bp)[PB][NP]) {
                acc4 b0[PB], b1[PB];
                build_b(cs, 2 * j, b0);
                if (2 * j + 1 < ntaps) {
                    build_b(cs, 2 * j + 1, b1);
                } else {
#pragma unroll
                    for (int pb = 0; pb < PB; ++pb) b1[pb] = acc4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int pb = 0; pb < PB; ++pb) {
                    const float v[8] = {b0[pb][0], b0[pb][1], b0[pb][2], b0[pb][3],
                                        b1[pb][0], b1[pb][1], b1[pb][2], b1[pb][3]};
                    pack8_16<T, NP>(v, 0, bp[pb]);   // (already at scale 2^s_b)
                }
            };
            if constexpr (STAGE) {
                // The weight blocks (per step MB row blocks x NP pieces, 1 KB each, contiguous in W16)
                // are staged in LDS, double-buffered, in units of U = 8 / MB steps (64-row tiles take
                // two steps per unit, so that a unit's MFMAs cover the loads of the next): the
                // global-to-LDS loads of unit u + 1 are issued at the top of unit u (one 1 KB wave
                // instruction per piece, spread over the waves), and every wave reads its A fragments
                // from LDS. Loaded straight from global memory each wave fetched the same blocks:
                // eight times the bytes through the vector memory path, which then bounded the MFMAs.
                constexpr int U = 8 / MB;            // steps per staging unit
                constexpr int NI = MB * NP;          // 1 KB pieces per step
                constexpr int WBLK = NI * 512;       // 16-bit values per step
                uint16_t *wst = reinterpret_cast<uint16_t *>(xwin + (size_t)wt.cells * XS);   // [2][U][WBLK]
                // (slice, pair) of the next step to stage, advanced step by step (no divisions)
                int s_cs = cs_lo, s_j = 0;
                auto stage_unit = [&](int u, int buf) {
#pragma unroll
                    for (int su = 0; su < U; ++su) {
                        const int k = u * U + su;
                        if (k >= nsteps) break;
                        const uint16_t *blk = wptr16(s_cs, s_j);
                        if (++s_j == npair) {
                            s_j = 0;
                            ++s_cs;
                        }
                        uint16_t *dst = wst + (buf * U + su) * WBLK;
                        for (int i = wave; i < NI; i += NW)
                            __builtin_amdgcn_global_load_lds(blk + i * 512 + lane * 8, dst + i * 512, 16, 0, 0);
                    }
                };
                auto load_w16 = [&](const uint16_t *blk, int mb, uint4 (&f)[NP]) {
                    const uint16_t *p = blk + mb * (NP * 512) + lane * 8;
#pragma unroll
                    for (int k = 0; k < NP; ++k) f[k] = *reinterpret_cast<const uint4 *>(p + k * 512);
                };
                // MFMAs of one step on its staged block; block mb + 1's fragments are read before
                // block mb's MFMAs
                auto mfma_pair = [&](const uint4 (&bv)[PB][NP], uint4 (&wa)[2][NP], const uint16_t *blk) {
                    load_w16(blk, 0, wa[0]);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        if (mb + 1 < MB) load_w16(blk, mb + 1, wa[(mb + 1) & 1]);
#pragma unroll
                        for (int pb = 0; pb < PB; ++pb)
                            acc[mb][pb] = mfma16x16x32_np<T, NP>(wa[mb & 1], bv[pb], acc[mb][pb]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                };
                // the staged unit's loads done, then the workgroup barrier that publishes it
                auto publish = [&]() {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                };
                // step k: its B fragments are built, then its MFMAs run (the LDS latency of the
                // sampling is covered by the other wave of the SIMD)
                uint4 wa[2][NP], bv[PB][NP];
                prefetch_x(cs_lo);
                __syncthreads();   // previous pass done with the tables and the staging buffers
                stage_unit(0, 0);
                open_slice(cs_lo, t0, ntaps);
                publish();
                // the next slice's X window is requested two pair steps before it is needed
                const int pf_j = max(npair - 2, 0);
                // (slice, pair) of step k, advanced step by step
                int cs = cs_lo, j = 0;
                for (int k = 0; k < nsteps; ++k) {
                    const bool more = k + 1 < nsteps;
                    const int u = k / U, su = k - u * U;
                    const int jn = j + 1 == npair ? 0 : j + 1;
                    if (su == 0 && (u + 1) * U < nsteps) stage_unit(u + 1, (u + 1) & 1);
                    if (j == pf_j && cs + 1 < cs_hi) prefetch_x(cs + 1);
                    build_pair(cs, j, bv);
                    mfma_pair(bv, wa, wst + ((u & 1) * U + su) * WBLK);
                    // the unit's end: every wave done with its buffer (and, at a slice change, with
                    // the window), the next unit's blocks visible
                    const bool unit_end = su == U - 1 || !more;
                    if (unit_end) publish();
                    if (more && jn == 0) {
                        if (!unit_end) __syncthreads();   // every wave done reading the window
                        open_slice(cs + 1, t0, ntaps);
                        __syncthreads();
                    }
                    j = jn;
                    if (jn == 0) ++cs;
                }
            } else {
                // (the weight's staging would cost the window its margin: fragments straight from
                // global memory, each row block's loaded one block ahead)
                auto load_w16g = [&](const uint16_t *p, uint4 (&f)[NP]) {
#pragma unroll
                    for (int k = 0; k < NP; ++k) f[k] = *reinterpret_cast<const uint4 *>(p + lane * 8 + k * 512);
                };
                // MFMAs of one step; block mb + 1's fragments (the next step's block 0 at the end)
                // are loaded before block mb's MFMAs
                auto mfma_pair_g = [&](const uint4 (&bv)[PB][NP], uint4 (&wa)[2][NP], const uint16_t *pcur,
                                       const uint16_t *pnext) {
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        load_w16g(mb + 1 < MB ? pcur + (size_t)(mb + 1) * (NP * 512) : pnext, wa[(mb + 1) & 1]);
#pragma unroll
                        for (int pb = 0; pb < PB; ++pb)
                            acc[mb][pb] = mfma16x16x32_np<T, NP>(wa[mb & 1], bv[pb], acc[mb][pb]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                };
                static_assert(MB % 2 == 0, "row blocks in pairs: the next step's block 0 lands in slot 0");
                uint4 wa[2][NP], bv[PB][NP];
                prefetch_x(cs_lo);
                load_w16g(wptr16(cs_lo, 0), wa[0]);
                __syncthreads();   // previous pass done with the tables
                open_slice(cs_lo, t0, ntaps);
                __syncthreads();
                const int pf_j = max(npair - 2, 0);
                int cs = cs_lo, j = 0;   // step k's (slice, pair), advanced step by step
                for (int k = 0; k < nsteps; ++k) {
                    const bool more = k + 1 < nsteps;
                    const int jn = j + 1 == npair ? 0 : j + 1;
                    const int csn = jn == 0 ? cs + 1 : cs;
                    if (j == pf_j && cs + 1 < cs_hi) prefetch_x(cs + 1);
                    build_pair(cs, j, bv);
                    const uint16_t *pcur = wptr16(cs, j);
                    mfma_pair_g(bv, wa, pcur, more ? wptr16(csn, jn) : pcur);
                    if (more && jn == 0) {
                        __syncthreads();   // every wave done reading the current window
                        open_slice(csn, t0, ntaps);
                        __syncthreads();
                    }
                    cs = csn;
                    j = jn;
                }
            }
        }
    };

    if constexpr (DIM == 3) {
        // 3D: taps in groups of four, lane row q sampling tap 4 * group + q at its pixel for
        // all 16 channels of the slice (the corner geometry formed once per (pixel, tap)
        // rather than once per channel quad); a row transpose then gives every lane its
        // channel quad of the group's four taps, the B fragments of four steps.
        auto build_group = [&](int cs, int tg, int ntaps, acc4 (&bq)[4][PB]) {
            const int tl = tg * 4 + q;
            const int nq = min(4, (g.Cg - cs * BC) >> 2);   // channel quads of the slice in the group
#pragma unroll
            for (int pb = 0; pb < PB; ++pb) {
                acc4 sv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) sv[j] = acc4{0.f, 0.f, 0.f, 0.f};
                if (tl < ntaps) {
                    const acc4 r = geo[tl * BPX + wave * (PB * 16) + pb * 16 + (lane & 15)];
                    if (nq == 4)
                        sample3_all<true>(g, wt, tile, xwin, xg + cs * BC, 4, r, deformable, sv);
                    else
                        sample3_all<false>(g, wt, tile, xwin, xg + cs * BC, nq, r, deformable, sv);
                }
                transpose_rows4(sv);
#pragma unroll
                for (int j = 0; j < 4; ++j) bq[j][pb] = sv[j];
            }
        };
        if (use16_flag) {
            // 16x16x32 steps: a group's four taps are two tap pairs, each pair's B fragment its
            // two sampled quads (the 16-bit loop's K order, W16 below), split into pieces (fp32)
            // or rounded to T; the pair's A fragments come from global memory, each row block's
            // loaded one block ahead
            constexpr int NP = npiece_of<T>();
            const int nmb = fw.Mg_pad / 16;
            const uint16_t *wl = w16 + (size_t)mt * MB * (NP * 512);
            auto load_w16g = [&](const uint16_t *p, uint4 (&f)[NP]) {
#pragma unroll
                for (int k = 0; k < NP; ++k) f[k] = *reinterpret_cast<const uint4 *>(p + lane * 8 + k * 512);
            };
            static_assert(MB % 2 == 0, "row blocks in pairs: the next step's block 0 lands in slot 0");
            for (int t0 = 0; t0 < g.Kn; t0 += wt.tpp) {
                const int ntaps = min(wt.tpp, g.Kn - t0);
                const int ngr = (ntaps + 3) >> 2;
                const int ngroups = (cs_hi - cs_lo) * ngr;
                geo_og = geo_mg = -1;
                const int pp0 = (t0 / wt.tpp) * fw.hp;
                auto wptr16 = [&](int cs, int j) {
                    return wl + (((size_t)grp * slices + cs) * fw.pp + pp0 + j) * nmb * (NP * 512);
                };
                uint4 wa[2][NP];
                load_w16g(wptr16(cs_lo, 0), wa[0]);
                __syncthreads();   // previous pass done with the tables
                open_slice(cs_lo, t0, ntaps);
                __syncthreads();
                int cs = cs_lo, tg = 0;
                for (int k = 0; k < ngroups; ++k) {
                    const bool more = k + 1 < ngroups;
                    const int tgn = tg + 1 == ngr ? 0 : tg + 1;
                    const int csn = tgn == 0 ? cs + 1 : cs;
                    acc4 bq[4][PB];
                    build_group(cs, tg, ntaps, bq);
                    const int npr = (min(4, ntaps - tg * 4) + 1) >> 1;   // tap pairs of the group
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        if (h < npr) {
                            uint4 bv[PB][NP];
#pragma unroll
                            for (int pb = 0; pb < PB; ++pb) {
                                const float v[8] = {bq[2 * h][pb][0],     bq[2 * h][pb][1],     bq[2 * h][pb][2],
                                                    bq[2 * h][pb][3],     bq[2 * h + 1][pb][0], bq[2 * h + 1][pb][1],
                                                    bq[2 * h + 1][pb][2], bq[2 * h + 1][pb][3]};
                                pack8_16<T, NP>(v, 0, bv[pb]);   // (already at scale 2^s_b)
                            }
                            const uint16_t *pcur = wptr16(cs, 2 * tg + h);
                            const uint16_t *pnext =
                                h + 1 < npr ? wptr16(cs, 2 * tg + h + 1) : (more ? wptr16(csn, 2 * tgn) : pcur);
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb) {
                                load_w16g(mb + 1 < MB ? pcur + (size_t)(mb + 1) * (NP * 512) : pnext, wa[(mb + 1) & 1]);
#pragma unroll
                                for (int pb = 0; pb < PB; ++pb)
                                    acc[mb][pb] = mfma16x16x32_np<T, NP>(wa[mb & 1], bv[pb], acc[mb][pb]);
                                __builtin_amdgcn_sched_barrier(0);
                            }
                        }
                    }
                    if (more && tgn == 0) {
                        __syncthreads();   // every wave done reading the current window
                        open_slice(csn, t0, ntaps);
                        __syncthreads();
                    }
                    cs = csn;
                    tg = tgn;
                }
            }
        } else {
            for (int t0 = 0; t0 < g.Kn; t0 += wt.tpp) {
                const int ntaps = min(wt.tpp, g.Kn - t0);
                const int ngr = (ntaps + 3) >> 2;   // tap groups per slice
                const int ngroups = (cs_hi - cs_lo) * ngr;
                geo_og = geo_mg = -1;   // a new pass of taps: the table must be rebuilt

                // group k = (slice cs_lo + k / ngr, taps 4 * (k % ngr) ..): its B fragments are
                // built at its start (the sampling's LDS latency is covered by the other wave of
                // the SIMD), then its steps run; wa holds the weight fragments of the next step.
                // The X window of a slice is loaded at the slice switch (the registers a prefetch
                // would hold across the steps are taken by the group's B fragments).
                acc4 wa[MB];
                load_w(wptr(cs_lo, t0), wa);
                __syncthreads();   // previous pass done with the tables
                open_slice(cs_lo, t0, ntaps);
                __syncthreads();
                int cs = cs_lo, tg = 0;   // group k's (slice, tap group), advanced group by group
                for (int k = 0; k < ngroups; ++k) {
                    const bool more = k + 1 < ngroups;
                    const int tgn = tg + 1 == ngr ? 0 : tg + 1;
                    const int csn = tgn == 0 ? cs + 1 : cs;
                    acc4 bq[4][PB];
                    build_group(cs, tg, ntaps, bq);
                    const int nt = min(4, ntaps - tg * 4);
                    const int tb = t0 + tg * 4;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (j < nt) {
                            // weight fragments of the step after this one (this step's own at the end)
                            const float *pn = j + 1 < nt ? wptr(cs, tb + j + 1)
                                                         : (more ? wptr(csn, t0 + tgn * 4) : wptr(cs, tb + j));
                            mfma_step(bq[j], wa, pn);
                        }
                    }
                    if (more && tgn == 0) {
                        __syncthreads();   // every wave done reading the current window
                        open_slice(csn, t0, ntaps);
                        __syncthreads();
                    }
                    cs = csn;
                    tg = tgn;
                }
            }
        }
    } else if (use16_flag) {
        for (int t0 = 0; t0 < g.Kn; t0 += wt.tpp) pass16(t0, min(wt.tpp, g.Kn - t0));
    } else {
        for (int t0 = 0; t0 < g.Kn; t0 += wt.tpp) {
            const int ntaps = min(wt.tpp, g.Kn - t0);
            const int nsteps = (cs_hi - cs_lo) * ntaps;
            geo_og = geo_mg = -1;   // a new pass of taps: the table must be rebuilt

            // step k = (slice cs_lo + k / ntaps, tap k % ntaps). Invariant at the top of step k:
            // its B fragments are in bcur, its weight fragments in wa.
            acc4 wa[MB], bcur[PB], bnxt[PB];
            prefetch_x(cs_lo);
            load_w(wptr(cs_lo, t0), wa);
            __syncthreads();   // previous pass done with the tables
            open_slice(cs_lo, t0, ntaps);
            __syncthreads();
            build_b(cs_lo, 0, bcur);
            // the next slice's X window is requested PF steps before it is needed (memory
            // latency exceeds one step's MFMAs), or at the slice's first step when shorter
            const int pf_tl = max(ntaps - PF, 0);
            int cs = cs_lo, tl = 0;   // step k's (slice, tap), advanced step by step
            for (int k = 0; k < nsteps; ++k) {
                const bool more = k + 1 < nsteps;
                const int tln = tl + 1 == ntaps ? 0 : tl + 1;
                const int csn = tln == 0 ? cs + 1 : cs;
                const bool new_slice = more && tln == 0;
                if (tl == pf_tl && cs + 1 < cs_hi) prefetch_x(cs + 1);
                if (more && !new_slice) build_b(csn, tln, bnxt);
                mfma_step(bcur, wa, more ? wptr(csn, t0 + tln) : wptr(cs, t0 + tl));
                if (new_slice) {
                    __syncthreads();   // every wave done reading the current window
                    open_slice(csn, t0, ntaps);
                    __syncthreads();
                    build_b(csn, 0, bnxt);
                }
#pragma unroll
                for (int pb = 0; pb < PB; ++pb) bcur[pb] = bnxt[pb];
                cs = csn;
                tl = tln;
            }
        }
    }

    // ---- epilogue: + bias, store NC<spatial>. With two slice shares, each adds its fp32
    //      partial to y32 (zeroed by the caller; bias with the first share): a sum of two
    //      terms onto zero is the same in either order, so the result is deterministic.
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
        const int p = tile.pixel(g, wt, wave * (PB * 16) + pb * 16 + (lane & 15));
        if (p < 0) continue;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = mt * BMR + mb * 16 + 4 * q + v;
                if (m < g.Mg) {
                    const int mg_glob = grp * g.Mg + m;
                    float r = s_back != 0 ? ldexpf(acc[mb][pb][v], s_back) : acc[mb][pb][v];
                    if (bias != nullptr && ks == 0) r += to_acc<float>(bias[mg_glob]);
                    const size_t o = ((size_t)tile.b * g.M + mg_glob) * g.Pn + p;
                    if (fw.ksplit == 1)
                        y[o] = from_acc<T, float>(r);
                    else
                        atomic_add(y32 + o, r);
                }
            }
    }
}

// weight (M, Cg, Kn) -> Wp[G][slices][Kn][Mg_pad / 16][16 m][16 c], zero padded (grid-stride loop
// over the calling grid)
template <typename T>
__device__ __forceinline__ void fwd_weight_f32(const T *__restrict__ w, float *__restrict__ wp, int G, int Mg, int Cg,
                                               int Kn, int slices, int Mg_pad) {
    // 32-bit index arithmetic (the launcher refuses layouts of 2^31 elements or more)
    const unsigned total = (unsigned)G * slices * Kn * Mg_pad * BC;
    for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int ci = (int)(i % BC);
        unsigned r = i / BC;
        const int m = (int)(r % Mg_pad);   // row blocks of 16 are consecutive: m = block * 16 + row
        r /= Mg_pad;
        const int t = (int)(r % Kn);
        r /= Kn;
        const int cs = (int)(r % slices);
        const int grp = (int)(r / slices);
        const int c = cs * BC + ci;
        float v = 0.f;
        if (m < Mg && c < Cg) v = to_acc<float>(w[(((size_t)grp * Mg + m) * Cg + c) * Kn + t]);
        wp[i] = v;
    }
}

template <typename T>
__global__ void fwd_win_weight_kernel(const T *__restrict__ w, float *__restrict__ wp, int G, int Mg, int Cg, int Kn,
                                      int slices, int Mg_pad) {
    fwd_weight_f32<T>(w, wp, G, Mg, Cg, Kn, slices, Mg_pad);
}

// weight (M, Cg, Kn) -> W16[G][slices][pp][Mg_pad / 16][NP][64 lanes][8]: per (slice, tap pair j
// of pass p, 16-row block) the 16x16x32 A fragments: lane l = m % 16 + 16 q holds at e = 0..7
// W[m][slice * 16 + 4 q + e % 4] at tap p * tpp + 2 j + e / 4 (zero past the pass, Mg, Cg); fp32
// as two fp16 pieces at the weight's scale (*flag set for a value bad for the split), fp16 / bf16
// as they are
// (wp: when not null, the fp32 layout of fwd_win_weight_kernel is written by the same launch)
template <typename T, int NP>
__global__ void __launch_bounds__(256)
fwd_w16_kernel(const T *__restrict__ w, uint16_t *__restrict__ out, int *flag, int G, int Mg, int Cg, int Kn, int slices,
               int nmb, int tpp, int hp, int pp, float *__restrict__ wp) {
    if (wp != nullptr) fwd_weight_f32<T>(w, wp, G, Mg, Cg, Kn, slices, nmb * 16);
    const unsigned total = (unsigned)G * slices * pp * nmb * 64;
    const int sw = NP == 2 ? operand_scale(flag, AMAX_W) : 0;
    bool bad = false;
    for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int l = (int)(i & 63);
        unsigned r = i >> 6;
        const int mb = (int)(r % nmb);
        r /= nmb;
        const int pq = (int)(r % pp);
        r /= pp;
        const int cs = (int)(r % slices);
        const int grp = (int)(r / slices);
        const int pass = pq / hp, j = pq - pass * hp;
        const int tf = pass * tpp, ntp = min(tpp, Kn - tf);
        const int m = mb * 16 + (l & 15), q = l >> 4;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int tl = 2 * j + (e >> 2), c = cs * BC + 4 * q + (e & 3);
            v[e] = (tl < ntp && m < Mg && c < Cg) ? to_acc<float>(w[(((size_t)grp * Mg + m) * Cg + c) * Kn + tf + tl]) : 0.f;
            bad = bad || split_bad(v[e]);
        }
        uint4 o[NP];
        pack8_16<T, NP>(v, sw, o);
        uint16_t *dst = out + ((((size_t)grp * slices + cs) * pp + pq) * nmb + mb) * (NP * 512) + l * 8;
#pragma unroll
        for (int k = 0; k < NP; ++k) *reinterpret_cast<uint4 *>(dst + k * 512) = o[k];
    }
    if (NP == 2 && bad) atomicOr(flag, 1);
}

template <int DIM, typename T, int MB, bool STAGE>
hipError_t launch_k(const Geo &g, const WinTiles &wt, const FwdWin &fw, const void *xcl, const void *wf,
                    const void *w16, const int *flag, const void *offset, const void *mask, const void *bias, void *y,
                    void *y32, hipStream_t s) {
    auto kern = fwd_win_kernel<DIM, T, MB, STAGE>;
    const size_t lds = ((size_t)GEO_WORDS + (size_t)(wt.cells + (DIM == 3)) * XS) * sizeof(float) + fw.stage_bytes;
    static std::atomic<unsigned long long> lds_raised{0};   // per device, see raise_lds_limit
    if (const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kern), lds_raised); e != hipSuccess)
        return e;
    const long long blocks = (long long)g.G * g.B * wt.ntile[0] * wt.ntile[1] * wt.ntile[2] * fw.m_tiles * fw.ksplit;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NT), lds, s, g, wt, fw, static_cast<const float *>(xcl),
                       static_cast<const float *>(wf), static_cast<const uint16_t *>(w16), flag,
                       static_cast<const T *>(offset), static_cast<const T *>(mask),
                       static_cast<const T *>(bias), static_cast<T *>(y), static_cast<float *>(y32));
    return hipGetLastError();
}

template <int DIM, typename T>
hipError_t launch_m(const Geo &g, const WinTiles &wt, const FwdWin &fw, const void *xcl, const void *wf,
                    const void *w16, const int *flag, const void *offset, const void *mask, const void *bias, void *y,
                    void *y32, hipStream_t s) {
    // 3D: 64-row tiles only (the trilinear sampler needs the registers), no weight staging
    if constexpr (DIM < 3) {
        if (fw.stage_bytes > 0) {
            if (fw.mb == 8) return launch_k<DIM, T, 8, true>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
            if (fw.mb == 4) return launch_k<DIM, T, 4, true>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
            return hipErrorInvalidValue;
        }
        if (fw.mb == 8) return launch_k<DIM, T, 8, false>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
    }
    if (fw.mb == 4) return launch_k<DIM, T, 4, false>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
    return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_d(int dim, const Geo &g, const WinTiles &wt, const FwdWin &fw, const void *xcl, const void *wf,
                    const void *w16, const int *flag, const void *offset, const void *mask, const void *bias, void *y,
                    void *y32, hipStream_t s) {
    switch (dim) {
        case 1: return launch_m<1, T>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
        case 2: return launch_m<2, T>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
        case 3: return launch_m<3, T>(g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

size_t x_window_cell_bytes() { return XS * sizeof(float); }

FwdWin plan_fwd_win(const Geo &g, const WinTiles &base, int dim, WinTiles &wt) {
    FwdWin f{};
    f.ok = false;
    wt = base;
    if (!base.ok || g.Mg < 16) return f;
    // 128-row tiles unless the GEMM side is small or the grid would leave CUs idle
    // (one workgroup per CU at a time: the window takes most of the LDS)
    const long long spatial = (long long)g.G * g.B * base.ntile[0] * base.ntile[1] * base.ntile[2];
    f.mb = (dim == 3 || g.Mg <= 64 || spatial * ((g.Mg + 127) / 128) < 256) ? 4 : 8;
    const int rows = 16 * f.mb;
    const long long max_cells = (long long)xq_of(f.mb) * NT / 4;
    // (3D: one more cell, the zero cell)
    const int zc = dim == 3 ? 1 : 0;
    wt = win_resize(base, g, dim, (size_t)(GEO_WORDS + zc * XS) * sizeof(float), XS * sizeof(float), max_cells - zc);
    if (wt.cells == 0) return f;   // no window fits: the unwindowed forward
    // 1D / 2D: two staging buffers of the 16-bit loop's weight blocks (8 row blocks x npiece KB
    // each: one step of 128-row tiles or two of 64-row tiles) when the window keeps a margin of
    // min(R, 4) cells beside them (a smaller window sends samples to global memory)
    f.stage_bytes = 0;
    if (dim < 3) {
        const int stage = 2 * 8 * base.npiece * 1024;
        const WinTiles ws =
            win_resize(base, g, dim, (size_t)(GEO_WORDS + zc * XS) * sizeof(float) + stage, XS * sizeof(float),
                       max_cells - zc);
        const int e = 2;   // the last axis: used in every rank
        if (ws.cells > 0 && ws.R[e] >= std::min(wt.R[e], 4)) {
            wt = ws;
            f.stage_bytes = stage;
        }
    }
    const size_t lds = ((size_t)GEO_WORDS + (size_t)(wt.cells + zc) * XS) * sizeof(float) + f.stage_bytes;
    if (lds > WIN_LDS_TARGET || wt.cells > max_cells) return f;
    f.m_tiles = (g.Mg + rows - 1) / rows;
    f.Mg_pad = f.m_tiles * rows;
    f.Cg_pad = (g.Cg + BC - 1) / BC * BC;
    // a grid that cannot give every CU a workgroup splits the channel slices in two (fp32
    // partials added onto a zeroed output: deterministic for two shares)
    const int slices = f.Cg_pad / BC;
    f.ksplit = (spatial * f.m_tiles < 256 && slices >= 2) ? 2 : 1;
    f.slices_per = (slices + f.ksplit - 1) / f.ksplit;
    // 3D samples taps in groups of four: passes of eight taps fill their groups (27 taps:
    // 8, 8, 8, 3 = seven groups, where passes of nine would take nine)
    if (dim == 3 && g.Kn > WIN_TMAX) wt.tpp = 8;
    // 16-bit weight fragments
    f.npiece = base.npiece;
    f.tpp = wt.tpp;
    f.hp = (wt.tpp + 1) / 2;
    f.pp = (g.Kn + wt.tpp - 1) / wt.tpp * f.hp;
    f.w16_elems = (size_t)g.G * slices * f.pp * (f.Mg_pad / 16) * f.npiece * 512;
    // the layout kernels index in 32 bits
    if ((size_t)g.G * slices * g.Kn * f.Mg_pad * BC > (size_t)INT_MAX || f.w16_elems / 8 > (size_t)INT_MAX) return f;
    f.ok = true;
    return f;
}

hipError_t launch_fwd_win_layout(int dtype, const Geo &g, const FwdWin &fw, const void *w, void *wp, hipStream_t s) {
    const int slices = fw.Cg_pad / BC;
    const size_t n = (size_t)g.G * slices * g.Kn * fw.Mg_pad * BC;
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
#define TVDCN_FWL(T)                                                                                             \
    hipLaunchKernelGGL((fwd_win_weight_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const T *>(w), \
                       static_cast<float *>(wp), g.G, g.Mg, g.Cg, g.Kn, slices, fw.Mg_pad);                      \
    return hipGetLastError();
    switch (dtype) {
        case kF32: { TVDCN_FWL(float) }
        case kF16: { TVDCN_FWL(__half) }
        case kBF16: { TVDCN_FWL(__hip_bfloat16) }
    }
#undef TVDCN_FWL
    return hipErrorInvalidValue;
}

hipError_t launch_fwd_win_layout16(int dtype, const Geo &g, const FwdWin &fw, const void *w, void *w16, int *flag,
                                   hipStream_t s, void *wp) {
    if (fw.w16_elems == 0) return wp != nullptr ? launch_fwd_win_layout(dtype, g, fw, w, wp, s) : hipSuccess;
    const int slices = fw.Cg_pad / BC;
    size_t n = fw.w16_elems / (fw.npiece * 8);   // threads: one per lane fragment
    if (wp != nullptr) n = std::max(n, (size_t)g.G * slices * g.Kn * fw.Mg_pad * BC);
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
#define TVDCN_FW16(T, NP)                                                                                              \
    hipLaunchKernelGGL((fwd_w16_kernel<T, NP>), dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const T *>(w),    \
                       static_cast<uint16_t *>(w16), flag, g.G, g.Mg, g.Cg, g.Kn, slices, fw.Mg_pad / 16, fw.tpp,    \
                       fw.hp, fw.pp, static_cast<float *>(wp));                                                        \
    return hipGetLastError();
    switch (dtype) {
        case kF32: { TVDCN_FW16(float, npiece_of<float>()) }
        case kF16: { TVDCN_FW16(__half, npiece_of<__half>()) }
        case kBF16: { TVDCN_FW16(__hip_bfloat16, npiece_of<__hip_bfloat16>()) }
    }
#undef TVDCN_FW16
    return hipErrorInvalidValue;
}

hipError_t launch_fwd_win(int dtype, int dim, const Geo &g, const WinTiles &wt, const FwdWin &fw, const void *xcl,
                          const void *wf, const void *w16, const int *flag, const void *offset, const void *mask,
                          const void *bias, void *y, void *y32, hipStream_t s) {
    if (fw.ksplit != 1 && y32 == nullptr) return hipErrorInvalidValue;
    switch (dtype) {
        case kF32: return launch_d<float>(dim, g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
        case kF16: return launch_d<__half>(dim, g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
        case kBF16:
            return launch_d<__hip_bfloat16>(dim, g, wt, fw, xcl, wf, w16, flag, offset, mask, bias, y, y32, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
