// Layout and elementwise helpers around the GEMM families (all HBM-bound).
//   * channels-last conversion of the sampled tensor ([B][C][S] -> [B][S][C]),
//     so that a bilinear corner fetch of consecutive channels is one coalesced
//     load; and the inverse (+ optional bias) for gradients / transposed outputs;
//   * weight re-layouts for the two MFMA operand orders;
//   * zero fill (a kernel, so it is safe inside captured HIP graphs);
//   * grad_bias = sum over batch and space of grad_out
//     (reference: tvdcn/csrc/ops/cuda/deform_conv2d_kernel.cpp:415-417).
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int TT = 64;   // transpose tile

// Raises sub-slot (linear block index % AMAX_SPREAD) of amax slot `slot` after *flag to the block's
// largest m (every thread of a 256-thread block calls it): one atomic per block, on one of
// AMAX_SPREAD lines (atomics on one address serialise)
__device__ __forceinline__ void block_amax(float m, int *flag, int slot) {
    __shared__ float wmax[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        const unsigned blk = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        if (m > 0.f)
            atomicMax(reinterpret_cast<unsigned *>(flag) + amax_word(slot, (int)(blk % AMAX_SPREAD)),
                      __float_as_uint(m));
    }
}

// The extra jobs of a channels-last copy launch, in the z slices past the batch: the mask's range
// check against chk_limit (into *flag) and its largest magnitude, the weight's largest magnitude;
// with amax_x the copy itself records the copied values' largest magnitude (fp32 path pieces)
struct CopyJobs {
    const float *chk;
    size_t chk_n;
    float chk_limit;
    const float *w;
    size_t w_n;
    bool amax_x;
};
__device__ __forceinline__ int copy_extra_slices(const CopyJobs &j) { return (j.chk != nullptr) + (j.w != nullptr); }

// slice k of the extra z slices (blocks of that slice stride over the tensor)
__device__ __forceinline__ void copy_extra_job(const CopyJobs &j, int k, int *flag) {
    const bool is_chk = j.chk != nullptr && k == 0;
    const float *v = is_chk ? j.chk : j.w;
    const size_t n = is_chk ? j.chk_n : j.w_n;
    const size_t nb = (size_t)gridDim.x * gridDim.y;
    bool bad = false;
    float m = 0.f;
    for (size_t i = ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += nb * blockDim.x) {
        const float a = fabsf(v[i]);
        bad = bad || !(a < j.chk_limit);
        m = fmaxf(m, a);
    }
    if (is_chk && bad) atomicOr(flag, 1);
    block_amax(m, flag, is_chk ? AMAX_SLOT_M : AMAX_SLOT_W);
}

// x [B][C][S] (T) -> xcl [B][S][C] (A); 64 x 64 tile through LDS, 256 threads. The z slices past the
// batch run the launch's other jobs (CopyJobs: one launch for the copy and the checks of other
// operands, e.g. the mask).
template <typename T, typename A>
__global__ void __launch_bounds__(256) to_cl_kernel(const T *__restrict__ x, A *__restrict__ xcl, int C, int S,
                                                    int *flag, const CopyJobs jobs) {
    __shared__ A tile[TT][TT + 1];
    const int b = blockIdx.z;
    const int nextra = flag != nullptr ? copy_extra_slices(jobs) : 0;
    if (b >= (int)gridDim.z - nextra) {
        copy_extra_job(jobs, b - ((int)gridDim.z - nextra), flag);
        return;
    }
    const int s0 = blockIdx.x * TT, c0 = blockIdx.y * TT;
    const T *xb = x + (size_t)b * C * S;
    A *ob = xcl + (size_t)b * C * S;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    bool big = false;
    float m = 0.f;
    for (int r = ty; r < TT; r += 4) {
        const int c = c0 + r, s = s0 + tx;
        const A v = (c < C && s < S) ? to_acc<A>(xb[(size_t)c * S + s]) : A(0);
        if constexpr (std::is_same<A, float>::value) {
            big = big || !(fabsf(v) < SAMPLED_LIMIT);
            m = fmaxf(m, fabsf(v));
        }
        tile[r][tx] = v;
    }
    if (flag != nullptr && big) atomicOr(flag, 1);
    if constexpr (std::is_same<A, float>::value) {
        if (flag != nullptr && jobs.amax_x) block_amax(m, flag, AMAX_SLOT_X);
    }
    __syncthreads();
    for (int r = ty; r < TT; r += 4) {
        const int s = s0 + r, c = c0 + tx;
        if (s < S && c < C) ob[(size_t)s * C + c] = tile[tx][r];
    }
}

// float32 x [B][C][S] -> xcl [B][S][C] with 16-byte accesses on both sides (C % 4 == 0 and
// S % 4 == 0: a quad is wholly inside or outside the tensor): 64 x 64 tile through LDS, 256
// threads; a load quad runs along s, a store quad along c. Same jobs as to_cl_kernel.
__global__ void __launch_bounds__(256) to_cl4_kernel(const float *__restrict__ x, float *__restrict__ xcl, int C,
                                                     int S, int *flag, const CopyJobs jobs) {
    __shared__ float tile[TT][TT + 1];   // [c][s]
    const int b = blockIdx.z;
    const int nextra = flag != nullptr ? copy_extra_slices(jobs) : 0;
    if (b >= (int)gridDim.z - nextra) {
        copy_extra_job(jobs, b - ((int)gridDim.z - nextra), flag);
        return;
    }
    const int s0 = blockIdx.x * TT, c0 = blockIdx.y * TT;
    const float *xb = x + (size_t)b * C * S;
    float *ob = xcl + (size_t)b * C * S;
    const int u = threadIdx.x & 15, r0 = threadIdx.x >> 4;
    bool big = false;
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int cl = r0 + 16 * k, c = c0 + cl, s = s0 + 4 * u;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < C && s < S) v = *reinterpret_cast<const float4 *>(xb + (size_t)c * S + s);
        big = big || !(fabsf(v.x) < SAMPLED_LIMIT) || !(fabsf(v.y) < SAMPLED_LIMIT) ||
              !(fabsf(v.z) < SAMPLED_LIMIT) || !(fabsf(v.w) < SAMPLED_LIMIT);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        tile[cl][4 * u] = v.x;
        tile[cl][4 * u + 1] = v.y;
        tile[cl][4 * u + 2] = v.z;
        tile[cl][4 * u + 3] = v.w;
    }
    if (flag != nullptr && big) atomicOr(flag, 1);
    if (flag != nullptr && jobs.amax_x) block_amax(m, flag, AMAX_SLOT_X);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int sl = r0 + 16 * k, s = s0 + sl, c = c0 + 4 * u;
        if (s < S && c < C)
            *reinterpret_cast<float4 *>(ob + (size_t)s * C + c) =
                make_float4(tile[4 * u][sl], tile[4 * u + 1][sl], tile[4 * u + 2][sl], tile[4 * u + 3][sl]);
    }
}

// float32 xcl [B][S][C] -> x [B][C][S] (+ bias[c]) with 16-byte accesses (C % 4 == 0, S % 4 == 0)
__global__ void __launch_bounds__(256) from_cl4_kernel(const float *__restrict__ xcl, float *__restrict__ x,
                                                       const float *__restrict__ bias, int C, int S) {
    __shared__ float tile[TT][TT + 1];   // [s][c]
    const int b = blockIdx.z;
    const int s0 = blockIdx.x * TT, c0 = blockIdx.y * TT;
    const float *ib = xcl + (size_t)b * C * S;
    float *ob = x + (size_t)b * C * S;
    const int u = threadIdx.x & 15, r0 = threadIdx.x >> 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int sl = r0 + 16 * k, s = s0 + sl, c = c0 + 4 * u;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (s < S && c < C) v = *reinterpret_cast<const float4 *>(ib + (size_t)s * C + c);
        tile[sl][4 * u] = v.x;
        tile[sl][4 * u + 1] = v.y;
        tile[sl][4 * u + 2] = v.z;
        tile[sl][4 * u + 3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int cl = r0 + 16 * k, c = c0 + cl, s = s0 + 4 * u;
        if (c < C && s < S) {
            const float bv = bias != nullptr ? bias[c] : 0.f;
            *reinterpret_cast<float4 *>(ob + (size_t)c * S + s) =
                make_float4(tile[4 * u][cl] + bv, tile[4 * u + 1][cl] + bv, tile[4 * u + 2][cl] + bv,
                            tile[4 * u + 3][cl] + bv);
        }
    }
}

// xcl [B][S][C] (A) -> x [B][C][S] (T), plus bias[c]
template <typename T, typename A>
__global__ void __launch_bounds__(256) from_cl_kernel(const A *__restrict__ xcl, T *__restrict__ x,
                                                      const T *__restrict__ bias, int C, int S) {
    __shared__ A tile[TT][TT + 1];
    const int b = blockIdx.z;
    const int s0 = blockIdx.x * TT, c0 = blockIdx.y * TT;
    const A *ib = xcl + (size_t)b * C * S;
    T *ob = x + (size_t)b * C * S;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < TT; r += 4) {
        const int s = s0 + r, c = c0 + tx;
        tile[r][tx] = (s < S && c < C) ? ib[(size_t)s * C + c] : A(0);
    }
    __syncthreads();
    for (int r = ty; r < TT; r += 4) {
        const int c = c0 + r, s = s0 + tx;
        if (c < C && s < S) {
            A v = tile[tx][r];
            if (bias != nullptr) v += to_acc<A>(bias[c]);
            ob[(size_t)c * S + s] = from_acc<T, A>(v);
        }
    }
}

// weight (M, Cg, Kn) -> Wf [G][Kn][Mg_pad][Cg_pad] (zero padded)
template <typename T, typename A>
__global__ void weight_f_kernel(const T *__restrict__ w, A *__restrict__ wf, int G, int Mg, int Cg, int Kn,
                                int Mg_pad, int Cg_pad) {
    const size_t total = (size_t)G * Kn * Mg_pad * Cg_pad;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % Cg_pad);
        const int m = (int)((i / Cg_pad) % Mg_pad);
        const int t = (int)((i / ((size_t)Cg_pad * Mg_pad)) % Kn);
        const int g = (int)(i / ((size_t)Cg_pad * Mg_pad * Kn));
        A v = A(0);
        if (m < Mg && c < Cg) v = to_acc<A>(w[(((size_t)g * Mg + m) * Cg + c) * Kn + t]);
        wf[i] = v;
    }
}

// weight (M, Cg, Kn) -> Wd [G][Kn][Cg_pad][Mg_pad] (zero padded)
template <typename T, typename A>
__global__ void weight_d_kernel(const T *__restrict__ w, A *__restrict__ wd, int G, int Mg, int Cg, int Kn,
                                int Mg_pad, int Cg_pad) {
    const size_t total = (size_t)G * Kn * Mg_pad * Cg_pad;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(i % Mg_pad);
        const int c = (int)((i / Mg_pad) % Cg_pad);
        const int t = (int)((i / ((size_t)Mg_pad * Cg_pad)) % Kn);
        const int g = (int)(i / ((size_t)Mg_pad * Cg_pad * Kn));
        A v = A(0);
        if (m < Mg && c < Cg) v = to_acc<A>(w[(((size_t)g * Mg + m) * Cg + c) * Kn + t]);
        wd[i] = v;
    }
}

template <typename A>
__global__ void fill_zero_kernel(A *__restrict__ p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = A{};
}

// Several buffers zeroed by one launch: the 16-byte-aligned body of each with vector stores
// (one flat index space over the bodies), the unaligned head and tail (under 16 bytes each)
// with 2-byte stores by block 0.
struct FillSet {
    uint4 *body[kFillMax];
    size_t start[kFillMax + 1];      // prefix sums of the body word counts
    uint16_t *edge[2 * kFillMax];    // head and tail of each buffer
    int edge_n[2 * kFillMax];        // 2-byte units, < 8
    int n;
};
__global__ void __launch_bounds__(256) fill_zero_multi_kernel(const FillSet f) {
    const size_t total = f.start[f.n];
    const size_t nt = (size_t)gridDim.x * blockDim.x;
    // four 16-byte stores per thread and round (a grid of a few thousand blocks)
    for (size_t i0 = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i0 < total; i0 += 4 * nt) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t i = i0 + u * nt;
            if (i >= total) break;
            int k = 0;
            while (k + 1 < f.n && i >= f.start[k + 1]) ++k;
            f.body[k][i - f.start[k]] = uint4{0u, 0u, 0u, 0u};
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < 2 * kFillMax * 8) {
        const int e = threadIdx.x >> 3, j = threadIdx.x & 7;
        if (e < 2 * f.n && j < f.edge_n[e]) f.edge[e][j] = 0;
    }
}

template <typename T, typename A>
__global__ void acc_to_storage_kernel(const A *__restrict__ a, T *__restrict__ o, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        o[i] = from_acc<T, A>(a[i]);
}

// two conversions in one launch: elements [0, n0) of the first pair, then [0, n1) of the second
template <typename T, typename A>
__global__ void acc_to_storage2_kernel(const A *__restrict__ a0, T *__restrict__ o0, size_t n0,
                                       const A *__restrict__ a1, T *__restrict__ o1, size_t n1) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n0 + n1; i += (size_t)gridDim.x * blockDim.x) {
        if (i < n0)
            o0[i] = from_acc<T, A>(a0[i]);
        else
            o1[i - n0] = from_acc<T, A>(a1[i - n0]);
    }
}

// Mask gradient of logits: the kernels accumulate d(loss)/d(mask value) per (b, group, tap,
// pixel); with mask value m = scale * sigmoid(logit), d(m)/d(logit) = m * (1 - m / scale)
// depends on that element only, so it scales the accumulated sum once.
template <typename T, typename A>
__global__ void mask_sigmoid_grad_kernel(const T *__restrict__ logits, A *__restrict__ gmask, double scale, size_t n) {
    const A sc = (A)scale;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const A v = to_acc<A>(logits[i]);
        A m;
        if constexpr (std::is_same_v<A, float>)
            m = sc / (1.f + expf(-v));
        else
            m = sc / (A(1) + exp(-v));
        gmask[i] *= m - m * m / sc;
    }
}

template <typename T, typename A>
__global__ void storage_to_acc_kernel(const T *__restrict__ x, A *__restrict__ a, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        a[i] = to_acc<A>(x[i]);
}

// grad_bias[c] = sum_{b, s} gout[b][c][s]; one 1024-thread workgroup per channel,
// four consecutive positions per load when rows are 4-aligned; per-thread partial sums
// in a fixed order, then a fixed reduction tree (deterministic)
template <typename T, typename A>
__global__ void __launch_bounds__(1024) bias_grad_kernel(const T *__restrict__ gout, T *__restrict__ gb, int B, int C,
                                                         int S, bool accumulate, int *flag) {
    __shared__ A red[16];
    __shared__ float mx[16];
    const int c = blockIdx.x;
    const int tid = threadIdx.x;
    const bool vec = sizeof(T) <= 4 && S % 4 == 0;
    A acc = A(0);
    float m = 0.f;
    for (int b = 0; b < B; ++b) {
        const T *row = gout + ((size_t)b * C + c) * S;
        if (vec) {
            for (int s4 = tid; s4 < S / 4; s4 += 1024) {
                const Vec4<A> v = load4_t<A, T>(row + 4 * s4);
                acc += (v.x + v.y) + (v.z + v.w);
                m = fmaxf(m, (float)fmax(fmax(fabs(v.x), fabs(v.y)), fmax(fabs(v.z), fabs(v.w))));
            }
        } else {
            for (int s = tid; s < S; s += 1024) {
                const A v = to_acc<A>(row[s]);
                acc += v;
                m = fmaxf(m, (float)fabs(v));
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        acc += __shfl_xor(acc, o);
        m = fmaxf(m, __shfl_xor(m, o));
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = acc;
        mx[tid >> 6] = m;
    }
    __syncthreads();
    if (tid == 0) {
        A sum = A(0);
        float big = 0.f;
        for (int w = 0; w < 16; ++w) {
            sum += red[w];
            big = fmaxf(big, mx[w]);
        }
        if (gb != nullptr) gb[c] = from_acc<T, A>(accumulate ? to_acc<A>(gb[c]) + sum : sum);
        if (flag != nullptr && big > 0.f)
            atomicMax(reinterpret_cast<unsigned *>(flag) + amax_word(AMAX_SLOT_Z, c % AMAX_SPREAD), __float_as_uint(big));
    }
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

unsigned grid_for(size_t n) {
    size_t b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

template <typename F>
hipError_t by_dtype(int dtype, F &&f) {
    switch (dtype) {
        case kF32: return f(float(), float());
        case kF64: return f(double(), double());
        case kF16: return f(__half(), float());
        case kBF16: return f(__hip_bfloat16(), float());
    }
    return hipErrorInvalidValue;
}

// largest |value| of up to four fp32 tensors: blockIdx.y = item, a grid-stride loop over the item
// (16-byte loads when vec: the pointer 16-byte aligned and n % 4 == 0), one atomicMax of the
// wave's largest per wave (float bits: non-negative floats order as their patterns). fmaxf passes
// over nan.
struct AmaxSet {
    const float *p[4];
    size_t n[4];
    int slot[4];
    bool vec[4];
};
__global__ void __launch_bounds__(256) amax_kernel(const AmaxSet set, int *flag) {
    const int it = blockIdx.y;
    const float *p = set.p[it];
    const size_t n = set.n[it];
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    float m = 0.f;
    if (set.vec[it]) {
        const size_t n4 = n / 4;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
            const float4 v = reinterpret_cast<const float4 *>(p)[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) m = fmaxf(m, fabsf(p[i]));
    }
    block_amax(m, flag, set.slot[it]);
}

}  // namespace

hipError_t launch_amax(const AmaxItem *items, int n, int *flag, hipStream_t s) {
    AmaxSet set{};
    int k = 0;
    size_t most = 0;
    for (int i = 0; i < n; ++i) {
        if (items[i].p == nullptr || items[i].n == 0) continue;
        if (k == 4 || items[i].slot < 0 || items[i].slot >= AMAX_SLOTS) return hipErrorInvalidValue;
        set.p[k] = items[i].p;
        set.n[k] = items[i].n;
        set.slot[k] = items[i].slot;
        set.vec[k] = al16(items[i].p) && items[i].n % 4 == 0;
        most = std::max(most, items[i].n);
        ++k;
    }
    if (k == 0) return hipSuccess;
    // about 16 values per thread on the largest item, at most 1024 blocks per item
    const size_t blocks = std::min<size_t>(std::max<size_t>((most + 4095) / 4096, 1), 1024);
    hipLaunchKernelGGL(amax_kernel, dim3((unsigned)blocks, (unsigned)k), dim3(256), 0, s, set, flag);
    return hipGetLastError();
}

hipError_t launch_to_channels_last(int dtype, const void *x, void *xcl, int B, int C, int Sn, hipStream_t s,
                                   int *flag, const void *chk, size_t chk_n, float chk_limit, const void *amax_w,
                                   size_t amax_w_n) {
    CopyJobs jobs{};
    if (flag != nullptr) {
        if (chk != nullptr && chk_n > 0) {
            jobs.chk = static_cast<const float *>(chk);
            jobs.chk_n = chk_n;
            jobs.chk_limit = chk_limit;
        }
        if (dtype == kF32 && amax_w != nullptr && amax_w_n > 0) {
            jobs.w = static_cast<const float *>(amax_w);
            jobs.w_n = amax_w_n;
            jobs.amax_x = true;
        }
    }
    const int extra = (jobs.chk != nullptr) + (jobs.w != nullptr);
    dim3 grid((Sn + TT - 1) / TT, (C + TT - 1) / TT, B + extra);
    if (dtype == kF32 && C % 4 == 0 && Sn % 4 == 0 && al16(x) && al16(xcl)) {
        hipLaunchKernelGGL(to_cl4_kernel, grid, dim3(256), 0, s, static_cast<const float *>(x), static_cast<float *>(xcl),
                           C, Sn, flag, jobs);
        return hipGetLastError();
    }
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((to_cl_kernel<T, A>), grid, dim3(256), 0, s, static_cast<const T *>(x),
                           static_cast<A *>(xcl), C, Sn, flag, jobs);
        return hipGetLastError();
    });
}

hipError_t launch_fill_zero_multi(const FillItem *items, int n, hipStream_t s) {
    FillSet f{};
    size_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (items[i].p == nullptr || items[i].bytes == 0) continue;
        if (f.n == kFillMax) return hipErrorInvalidValue;
        char *p = static_cast<char *>(items[i].p);
        const size_t bytes = items[i].bytes;
        if (reinterpret_cast<uintptr_t>(p) % 2 != 0 || bytes % 2 != 0) return hipErrorInvalidValue;
        size_t head = (16 - reinterpret_cast<uintptr_t>(p) % 16) % 16;
        if (head > bytes) head = bytes;
        const size_t words = (bytes - head) / 16;
        const size_t tail = bytes - head - words * 16;
        const int k = f.n++;
        f.body[k] = reinterpret_cast<uint4 *>(p + head);
        f.start[k] = total;
        total += words;
        f.edge[2 * k] = reinterpret_cast<uint16_t *>(p);
        f.edge_n[2 * k] = (int)(head / 2);
        f.edge[2 * k + 1] = reinterpret_cast<uint16_t *>(p + head + words * 16);
        f.edge_n[2 * k + 1] = (int)(tail / 2);
    }
    if (f.n == 0) return hipSuccess;
    f.start[f.n] = total;
    const size_t blocks = std::min<size_t>(std::max<size_t>((total + 1023) / 1024, 1), 4096);
    hipLaunchKernelGGL(fill_zero_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, s, f);
    return hipGetLastError();
}

hipError_t launch_from_channels_last(int dtype, const void *xcl, void *x, const void *bias, int B, int C, int Sn,
                                     hipStream_t s) {
    if (dtype == kF32 && C % 4 == 0 && Sn % 4 == 0 && al16(x) && al16(xcl)) {
        dim3 grid((Sn + TT - 1) / TT, (C + TT - 1) / TT, B);
        hipLaunchKernelGGL(from_cl4_kernel, grid, dim3(256), 0, s, static_cast<const float *>(xcl),
                           static_cast<float *>(x), static_cast<const float *>(bias), C, Sn);
        return hipGetLastError();
    }
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        dim3 grid((Sn + TT - 1) / TT, (C + TT - 1) / TT, B);
        hipLaunchKernelGGL((from_cl_kernel<T, A>), grid, dim3(256), 0, s, static_cast<const A *>(xcl),
                           static_cast<T *>(x), static_cast<const T *>(bias), C, Sn);
        return hipGetLastError();
    });
}

hipError_t launch_weight_fwd_layout(int dtype, const Geo &g, const void *w, void *wf, int Mg_pad, int Cg_pad,
                                    hipStream_t s) {
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        const size_t n = (size_t)g.G * g.Kn * Mg_pad * Cg_pad;
        hipLaunchKernelGGL((weight_f_kernel<T, A>), dim3(grid_for(n)), dim3(256), 0, s, static_cast<const T *>(w),
                           static_cast<A *>(wf), g.G, g.Mg, g.Cg, g.Kn, Mg_pad, Cg_pad);
        return hipGetLastError();
    });
}

hipError_t launch_weight_data_layout(int dtype, const Geo &g, const void *w, void *wd, int Mg_pad, int Cg_pad,
                                     hipStream_t s) {
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        const size_t n = (size_t)g.G * g.Kn * Mg_pad * Cg_pad;
        hipLaunchKernelGGL((weight_d_kernel<T, A>), dim3(grid_for(n)), dim3(256), 0, s, static_cast<const T *>(w),
                           static_cast<A *>(wd), g.G, g.Mg, g.Cg, g.Kn, Mg_pad, Cg_pad);
        return hipGetLastError();
    });
}

hipError_t launch_fill_zero(int elem_bytes, void *p, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return hipErrorInvalidValue;
    // 16-byte aligned buffers: the whole 16-byte words with vector stores, the few
    // elements past the last one with the element kernel
    if (reinterpret_cast<uintptr_t>(p) % 16 == 0) {
        const size_t words = n * elem_bytes / 16;
        if (words > 0) {
            hipLaunchKernelGGL((fill_zero_kernel<uint4>), dim3(grid_for(words)), dim3(256), 0, s, static_cast<uint4 *>(p),
                               words);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        const size_t done = words * 16 / elem_bytes;
        if (done == n) return hipSuccess;
        p = static_cast<char *>(p) + done * elem_bytes;
        n -= done;
    }
    if (elem_bytes == 8)
        hipLaunchKernelGGL((fill_zero_kernel<double>), dim3(grid_for(n)), dim3(256), 0, s, static_cast<double *>(p), n);
    else if (elem_bytes == 4)
        hipLaunchKernelGGL((fill_zero_kernel<float>), dim3(grid_for(n)), dim3(256), 0, s, static_cast<float *>(p), n);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL((fill_zero_kernel<uint16_t>), dim3(grid_for(n)), dim3(256), 0, s, static_cast<uint16_t *>(p),
                           n);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_acc_to_storage(int dtype, const void *acc, void *out, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((acc_to_storage_kernel<T, A>), dim3(grid_for(n)), dim3(256), 0, s,
                           static_cast<const A *>(acc), static_cast<T *>(out), n);
        return hipGetLastError();
    });
}

hipError_t launch_acc_to_storage2(int dtype, const void *acc0, void *out0, size_t n0, const void *acc1, void *out1,
                                  size_t n1, hipStream_t s) {
    if (n0 == 0) return launch_acc_to_storage(dtype, acc1, out1, n1, s);
    if (n1 == 0) return launch_acc_to_storage(dtype, acc0, out0, n0, s);
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((acc_to_storage2_kernel<T, A>), dim3(grid_for(n0 + n1)), dim3(256), 0, s,
                           static_cast<const A *>(acc0), static_cast<T *>(out0), n0, static_cast<const A *>(acc1),
                           static_cast<T *>(out1), n1);
        return hipGetLastError();
    });
}

hipError_t launch_mask_sigmoid_grad(int dtype, const void *logits, void *gmask_acc, double scale, size_t n,
                                    hipStream_t s) {
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((mask_sigmoid_grad_kernel<T, A>), dim3(grid_for(n)), dim3(256), 0, s,
                           static_cast<const T *>(logits), static_cast<A *>(gmask_acc), scale, n);
        return hipGetLastError();
    });
}

// *flag |= any of v[0 .. n) is not below `limit` in magnitude (nan included)
__global__ void __launch_bounds__(256) check_range_kernel(const float *__restrict__ v, size_t n, float limit,
                                                          int *flag) {
    bool big = false;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        big = big || !(fabsf(v[i]) < limit);
    if (big) atomicOr(flag, 1);
}

hipError_t launch_check_range(const void *v, size_t n, float limit, int *flag, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(check_range_kernel, dim3(grid_for(n)), dim3(256), 0, s, static_cast<const float *>(v), n, limit,
                       flag);
    return hipGetLastError();
}

hipError_t launch_storage_to_acc(int dtype, const void *x, void *acc, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((storage_to_acc_kernel<T, A>), dim3(grid_for(n)), dim3(256), 0, s,
                           static_cast<const T *>(x), static_cast<A *>(acc), n);
        return hipGetLastError();
    });
}

hipError_t launch_bias_grad(int dtype, const void *gout, void *gbias, int B, int C, int Sn, hipStream_t s,
                            bool accumulate, int *flag) {
    if (dtype != kF32) flag = nullptr;
    if (gbias == nullptr && flag == nullptr) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((bias_grad_kernel<T, A>), dim3(C), dim3(1024), 0, s, static_cast<const T *>(gout),
                           static_cast<T *>(gbias), B, C, Sn, accumulate, flag);
        return hipGetLastError();
    });
}

}  // namespace tvdcn_hip
