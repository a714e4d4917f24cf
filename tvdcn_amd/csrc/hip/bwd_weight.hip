// Family Wt: weight gradient as an implicit GEMM over re-gathered columns.
//
//   dW[m][c][t] += sum_{(b,p) in split} Z[b][m][p] * mask * bilinear(X[b][c], pos(b, og(c), t, p))
//
// Replaces the reference's im2col recompute + grad_weight addmm_
// (tvdcn/csrc/ops/cuda/deform_conv2d_kernel.cpp:600-626; transposed
// deform_conv_transpose2d_kernel.cpp:586-613). The reduction runs over all
// column pixels, split across workgroups (split-K); each workgroup stores its
// partial tile to a workspace and a second kernel sums the splits in a fixed
// order (deterministic, no atomics: contended float atomics run at about half
// the rate of coalesced stores on this part).
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
                  const T *__restrict__ mask, A *__restrict__ part, const int k_chunk, const int m_tiles,
                  const int c_tiles, const int k_splits, const bool z_vec) {
    constexpr int NT = 64 * WAVES;
    constexpr int SLOTS = (BKP * BC / 4) / NT;   // (pixel, quad) slots per thread
    constexpr int NC = 1 << DIM;
    typedef typename Acc4<A>::type acc4;

    __shared__ A smem[2 * BKP * LDB];

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

    const int ogi = (g.og && cvalid) ? c / g.cpo : 0;
    const int mgi = (g.mg && cvalid) ? c / g.cpm : 0;

    // Generic path (channel quads may straddle offset/mask groups): gather one
    // step synchronously, every channel resolving its own group.
    auto gather_generic = [&](int k0, int buf) {
        A *dst = smem + buf * BKP * LDB;
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            const int nl = (tid >> 4) + i * (NT / 16);
            const int n = k0 + nl;
            const bool ok = n < kend;
            const int b = ok ? fdiv(g.dPn, n) : 0;
            const int p = ok ? n - b * g.Pn : 0;
            A vals[4] = {A(0), A(0), A(0), A(0)};
            if (ok) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (cl + j >= g.Cg) continue;
                    const int cj = c + j;
                    const int oj = g.og ? cj / g.cpo : 0;
                    const int mj = g.mg ? cj / g.cpm : 0;
                    const GatherCorners<DIM, A> gc = gather_corners<DIM, A>(
                        g, axis_weights<DIM, A>(g, sample_point<DIM, A, T>(g, offset, b, p, t, oj), deformable));
                    const A *base = xcl + (size_t)b * g.Sn * g.C + cj;
                    A v = A(0);
#pragma unroll
                    for (int k = 0; k < NC; ++k) v += gc.w[k] * base[(size_t)gc.idx[k] * g.C];
                    vals[j] = v * mask_at<A, T>(g, mask, b, mj, t, p);
                }
            }
            store4<A>(dst + nl * LDB + 4 * q, {vals[0], vals[1], vals[2], vals[3]});
        }
    };

    // Fast path: a three-stage software pipeline per slot. During step s the
    // thread holds the corner geometry of step s+1 (whose corner loads it issues
    // before the MFMAs) and the raw offsets/mask of step s+2.
    struct Slot {
        GatherCorners<DIM, A> gc;   // geometry of the next step to gather
        A mk;                       // its mask value
        bool ok;
        int b;
        A off[DIM];                 // raw offsets two steps ahead
        A mraw;
        bool ok2;
        int b2, p2;
    };
    Slot sl[VEC4 ? SLOTS : 1];
    Vec4<A> raw[VEC4 ? SLOTS : 1][NC];

    auto fetch_geo_inputs = [&](int k0, Slot &st, int i) {   // loads for step at k0 into st.off / st.mraw
        const int nl = (tid >> 4) + i * (NT / 16);
        const int n = k0 + nl;
        st.ok2 = n < kend && cvalid;
        st.b2 = st.ok2 ? fdiv(g.dPn, n) : 0;
        st.p2 = st.ok2 ? n - st.b2 * g.Pn : 0;
        if (deformable) {
            const T *o = offset + ((size_t)(st.b2 * g.og + ogi) * g.Kn + t) * DIM * (size_t)g.Pn + st.p2;
#pragma unroll
            for (int a = 0; a < DIM; ++a) st.off[a] = to_acc<A>(o[(size_t)a * g.Pn]);
        }
        st.mraw = mask_at<A, T>(g, mask, st.b2, mgi, t, st.p2);
    };
    auto make_geo = [&](Slot &st) {   // turn the fetched inputs into corner geometry
        Point<DIM, A> pt = sample_point<DIM, A, T>(g, nullptr, st.b2, st.p2, t, 0);
        if (deformable) {
#pragma unroll
            for (int a = 0; a < DIM; ++a) pt.pos[a] = round_position<T, A>(pt.pos[a] + st.off[a]);
        }
        st.gc = gather_corners<DIM, A>(g, axis_weights<DIM, A>(g, pt, deformable));
        st.mk = st.mraw;
        st.ok = st.ok2;
        st.b = st.b2;
    };
    auto issue_corners = [&]() {
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            const A *base = xcl + (size_t)sl[i].b * g.Sn * g.C + c;
#pragma unroll
            for (int k = 0; k < NC; ++k)
                raw[i][k] = sl[i].ok ? load4<A>(base + (size_t)sl[i].gc.idx[k] * g.C) : Vec4<A>{A(0), A(0), A(0), A(0)};
        }
    };
    auto combine_to_lds = [&](int buf) {
        A *dst = smem + buf * BKP * LDB;
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) {
            Vec4<A> v = {A(0), A(0), A(0), A(0)};
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                const A w = sl[i].gc.w[k];
                v.x += w * raw[i][k].x;
                v.y += w * raw[i][k].y;
                v.z += w * raw[i][k].z;
                v.w += w * raw[i][k].w;
            }
            const A mk = sl[i].mk;
            v.x *= mk; v.y *= mk; v.z *= mk; v.w *= mk;
            const int nl = (tid >> 4) + i * (NT / 16);
            store4<A>(dst + nl * LDB + 4 * q, v);
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
                    const int b = fdiv(g.dPn, n);
                    const int p = n - b * g.Pn;
                    const Vec4<A> q4 = load4_t<A, T>(z + ((size_t)b * g.M + mrow) * g.Pn + p);
                    v[0] = q4.x;
                    v[1] = q4.y;
                    v[2] = q4.z;
                    v[3] = q4.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int ni = n + i;
                        if (ni < kend) {
                            const int b = fdiv(g.dPn, ni);
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
        if constexpr (VEC4) {
            // prologue: step 0 gathered into buffer 0, geometry of step 1 ready
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                fetch_geo_inputs(kbeg, sl[i], i);
                make_geo(sl[i]);
            }
            issue_corners();
            combine_to_lds(0);
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                fetch_geo_inputs(kbeg + BKP, sl[i], i);
                make_geo(sl[i]);
            }
        } else {
            gather_generic(kbeg, 0);
        }
        load_a(kbeg, a_cur);
        __syncthreads();
        for (int s = 0; s < nsteps; ++s) {
            const int buf = s & 1;
            const bool more = s + 1 < nsteps;
            if (more) {
                load_a(kbeg + (s + 1) * BKP, a_nxt);
                if constexpr (VEC4) {
                    issue_corners();   // step s+1
#pragma unroll
                    for (int i = 0; i < SLOTS; ++i) fetch_geo_inputs(kbeg + (s + 2) * BKP, sl[i], i);
                }
            }
            // B[k = pixel 4*(lane/16) + kk][j = channel cb*16 + lane%16]
            const A *sb = smem + buf * BKP * LDB + 4 * (lane >> 4) * LDB + (lane & 15);
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
                if constexpr (VEC4) {
                    combine_to_lds(buf ^ 1);
#pragma unroll
                    for (int i = 0; i < SLOTS; ++i) make_geo(sl[i]);   // step s+2
                } else {
                    gather_generic(kbeg + (s + 1) * BKP, buf ^ 1);
                }
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) a_cur[mb] = a_nxt[mb];
            }
            __syncthreads();
        }
    }

    // partial tile of split ks, layout [ks][grp][t][m][c] (c contiguous: 64-byte
    // stores per 16 lanes); summed over ks by weight_reduce_kernel
    A *dst = part + (((size_t)ks * g.G + grp) * g.Kn + t) * g.Mg * (size_t)g.Cg;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int cc = c0 + cb * 16 + (lane & 15);
        if (cc >= g.Cg) continue;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = mrow0 + mb * 16 + mfma_row<A>(lane, v);
                if (m < g.Mg) dst[(size_t)m * g.Cg + cc] = acc[mb][cb][v];
            }
    }
}

// dW[grp*Mg + m][c][t] = sum over splits of part[ks][grp][t][m][c] (fixed order: deterministic)
// units_per_split > 0: split ks covers units [ks * ups, (ks + 1) * ups) of (pass, spatial tile),
// pass-major; tap t (pass t / tpp) sums the splits that meet units [pass * n_sp, (pass + 1) * n_sp).
// 32-bit index arithmetic: the weight's element count and the unit count fit in int.
template <typename T, typename A>
__global__ void __launch_bounds__(256) weight_reduce_kernel(const A *__restrict__ part, T *__restrict__ gw, int k_splits,
                                                            int G, int Kn, int Mg, int Cg, int ups, int n_sp, int tpp,
                                                            bool accumulate) {
    const int per_split = G * Kn * Mg * Cg;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < per_split; i += gridDim.x * blockDim.x) {
        const int c = i % Cg;
        const int r = i / Cg;
        const int m = r % Mg;
        const int t = (r / Mg) % Kn;
        const int grp = r / (Mg * Kn);
        int ks0 = 0, ks1 = k_splits;
        if (ups > 0) {
            const unsigned pass = (unsigned)(t / tpp);
            ks0 = (int)(pass * (unsigned)n_sp / (unsigned)ups);
            ks1 = min(k_splits, (int)(((pass + 1u) * (unsigned)n_sp - 1u) / (unsigned)ups) + 1);
        }
        A sum = A(0);
        for (int ks = ks0; ks < ks1; ++ks) sum += part[(size_t)ks * per_split + i];
        T *dst = gw + (((size_t)grp * Mg + m) * Cg + c) * Kn + t;
        *dst = from_acc<T, A>(accumulate ? to_acc<A>(*dst) + sum : sum);
    }
}

// The same sum for Cg % 4 == 0 and 16-byte aligned partials: a block holds 4 rows (grp, t, m) of
// 64 threads, each thread 4 consecutive channels per 16-byte load; the row's split range is
// formed once per row (no per-element index divisions)
template <typename T, typename A>
__global__ void __launch_bounds__(256) weight_reduce4_kernel(const A *__restrict__ part, T *__restrict__ gw,
                                                             int k_splits, int G, int Kn, int Mg, int Cg, int ups,
                                                             int n_sp, int tpp, bool accumulate) {
    const int rows = G * Kn * Mg;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int m = r % Mg;
    const int t = (r / Mg) % Kn;
    const int grp = r / (Mg * Kn);
    int ks0 = 0, ks1 = k_splits;
    if (ups > 0) {
        const unsigned pass = (unsigned)(t / tpp);
        ks0 = (int)(pass * (unsigned)n_sp / (unsigned)ups);
        ks1 = min(k_splits, (int)(((pass + 1u) * (unsigned)n_sp - 1u) / (unsigned)ups) + 1);
    }
    const size_t per_split = (size_t)rows * Cg;
    const A *src = part + (size_t)r * Cg;   // layout [ks][grp][t][m][c]: row r = (grp * Kn + t) * Mg + m
    T *dst = gw + ((size_t)grp * Mg + m) * Cg * Kn + t;
    for (int c = 4 * (threadIdx.x & 63); c < Cg; c += 256) {
        Vec4<A> sum{A(0), A(0), A(0), A(0)};
        for (int ks = ks0; ks < ks1; ++ks) {
            const Vec4<A> v = *reinterpret_cast<const Vec4<A> *>(src + ks * per_split + c);
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        const A sv[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            T *o = dst + (size_t)(c + j) * Kn;
            *o = from_acc<T, A>(accumulate ? to_acc<A>(*o) + sv[j] : sv[j]);
        }
    }
}

template <typename T, typename A>
hipError_t launch_reduce(const Geo &g, int k_splits, const void *part, void *gw, bool accumulate, hipStream_t s, int ups,
                         int n_sp, int tpp) {
    if (ups > 0 && (n_sp <= 0 || tpp <= 0)) return hipErrorInvalidValue;
    const size_t n = (size_t)g.G * g.Kn * g.Mg * g.Cg;
    if (n > (size_t)INT_MAX) return hipErrorInvalidValue;
    if (g.Cg % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0) {
        const unsigned blocks = (unsigned)(((size_t)g.G * g.Kn * g.Mg + 3) / 4);
        hipLaunchKernelGGL((weight_reduce4_kernel<T, A>), dim3(blocks), dim3(256), 0, s, static_cast<const A *>(part),
                           static_cast<T *>(gw), k_splits, g.G, g.Kn, g.Mg, g.Cg, ups, n_sp, tpp, accumulate);
        return hipGetLastError();
    }
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL((weight_reduce_kernel<T, A>), dim3(blocks), dim3(256), 0, s, static_cast<const A *>(part),
                       static_cast<T *>(gw), k_splits, g.G, g.Kn, g.Mg, g.Cg, ups, n_sp, tpp, accumulate);
    return hipGetLastError();
}

template <int DIM, typename T, typename A, int WAVES, bool VEC4>
hipError_t launch_t(const Geo &g, const WeightTiles &tl, const void *z, const void *xcl, const void *offset,
                    const void *mask, void *part, hipStream_t s) {
    const int m_tiles = (g.Mg + 64 * WAVES - 1) / (64 * WAVES);
    const int c_tiles = (g.Cg + BC - 1) / BC;
    const long long blocks = (long long)g.G * tl.k_splits * g.Kn * c_tiles * m_tiles;
    const bool z_vec = g.Pn % 4 == 0;
    hipLaunchKernelGGL((bwd_weight_kernel<DIM, T, A, WAVES, VEC4>), dim3((unsigned)blocks), dim3(64 * WAVES), 0, s,
                       g, static_cast<const T *>(z), static_cast<const A *>(xcl), static_cast<const T *>(offset),
                       static_cast<const T *>(mask), static_cast<A *>(part), tl.k_chunk, m_tiles, c_tiles, tl.k_splits,
                       z_vec);
    return hipGetLastError();
}

template <int DIM, typename T, typename A>
hipError_t launch_w(const Geo &g, const WeightTiles &tl, const void *z, const void *xcl, const void *offset,
                    const void *mask, void *part, hipStream_t s) {
#define TVDCN_WGT_CASE(W)                                                                    \
    if (tl.waves == W)                                                                       \
        return tl.vec4 ? launch_t<DIM, T, A, W, true>(g, tl, z, xcl, offset, mask, part, s)  \
                       : launch_t<DIM, T, A, W, false>(g, tl, z, xcl, offset, mask, part, s);
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
                    const void *mask, void *part, void *gw, bool accumulate, hipStream_t s) {
    hipError_t e = hipErrorInvalidValue;
    switch (dim) {
        case 1: e = launch_w<1, T, A>(g, tl, z, xcl, offset, mask, part, s); break;
        case 2: e = launch_w<2, T, A>(g, tl, z, xcl, offset, mask, part, s); break;
        case 3: e = launch_w<3, T, A>(g, tl, z, xcl, offset, mask, part, s); break;
    }
    if (e != hipSuccess) return e;
    return launch_reduce<T, A>(g, tl.k_splits, part, gw, accumulate, s, 0, 0, 0);
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
    // aim for ~1024 workgroups in total, at least 256 pixels per split
    long long splits = (1024 + tiles - 1) / tiles;
    const long long max_splits = (g.NP + 255) / 256;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    long long chunk = g.NP > 0 ? (g.NP + splits - 1) / splits : BKP;
    chunk = (chunk + BKP - 1) / BKP * BKP;
    t.k_chunk = (int)chunk;
    t.k_splits = g.NP > 0 ? (int)((g.NP + chunk - 1) / chunk) : 1;
    t.part_elems = (size_t)t.k_splits * g.G * g.Kn * g.Mg * g.Cg;
    return t;
}

hipError_t launch_weight_reduce(int dtype, const Geo &g, int k_splits, const void *part, void *gw, bool accumulate,
                                hipStream_t s,
                                int ups, int n_sp, int tpp) {
    switch (dtype) {
        case kF32: return launch_reduce<float, float>(g, k_splits, part, gw, accumulate, s, ups, n_sp, tpp);
        case kF64: return launch_reduce<double, double>(g, k_splits, part, gw, accumulate, s, ups, n_sp, tpp);
        case kF16: return launch_reduce<__half, float>(g, k_splits, part, gw, accumulate, s, ups, n_sp, tpp);
        case kBF16: return launch_reduce<__hip_bfloat16, float>(g, k_splits, part, gw, accumulate, s, ups, n_sp, tpp);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_bwd_weight(int dtype, int dim, const Geo &g, const WeightTiles &t, const void *z, const void *xcl,
                             const void *offset, const void *mask, void *part, void *gw, bool accumulate,
                             hipStream_t s) {
    switch (dtype) {
        case kF32: return launch_d<float, float>(dim, g, t, z, xcl, offset, mask, part, gw, accumulate, s);
        case kF64: return launch_d<double, double>(dim, g, t, z, xcl, offset, mask, part, gw, accumulate, s);
        case kF16: return launch_d<__half, float>(dim, g, t, z, xcl, offset, mask, part, gw, accumulate, s);
        case kBF16: return launch_d<__hip_bfloat16, float>(dim, g, t, z, xcl, offset, mask, part, gw, accumulate, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace tvdcn_hip
