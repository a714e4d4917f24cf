// mask_softmax forward / backward over the kernel taps.
//
// The mask (B, mg*K, *S) is viewed as (B*mg, K, S) and normalised over K
// (reference: tvdcn/ops/activations/mask_softmax.py:19-126, torch.softmax on the
// view). K is strided by S in memory, so the reduction axis runs *down* a lane,
// not across lanes: each lane owns CPT (b, g, s) columns 64 apart and keeps their K
// values in registers, while the 64 lanes of a wavefront cover 64 consecutive s, which
// makes every load and store a fully coalesced 256-byte wavefront access. One read +
// one write per element in the forward, two reads + one write in the backward.
// The tensors are small (1-5 MB at the BASELINE configs), so the kernels are latency
// bound: the tap count is a template parameter for the common kernel sizes (all K
// loads of a column unconditional and issued before any is used), the columns of a
// thread are independent, and the index arithmetic is 32-bit (grid = (s blocks, bg);
// the launchers fall back to 64-bit loops past 2^31 elements). K > 32 re-reads the
// column (three passes).
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int KMAX_REG = 32;
constexpr int SB = 256;   // threads per block

// tap count: KC at compile time (0: k runs to the run-time K <= KMAX_REG)
template <int KC> __device__ __forceinline__ bool tap_on(int k, int K) { return KC ? k < KC : k < K; }
template <int KC> constexpr int tap_slots() { return KC ? KC : KMAX_REG; }

// Column c of the block's CPT x 64 columns per wave: s = s0 + c * 64 + lane.
template <typename T, typename A, int KC, int CPT>
__global__ void __launch_bounds__(SB) softmax_fwd_kernel(const T *__restrict__ x, T *__restrict__ y, int BG, int K,
                                                         int S) {
    constexpr int KS = tap_slots<KC>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = (blockIdx.x * (SB / 64) + wave) * (64 * CPT) + lane;
    for (int bg = blockIdx.y; bg < BG; bg += gridDim.y) {
        const T *xb = x + (size_t)bg * K * S;
        T *yb = y + (size_t)bg * K * S;
        A v[CPT][KS];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int sc = min(s0 + c * 64, S - 1);   // clamped: every load in bounds
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) v[c][k] = to_acc<A>(xb[k * S + sc]);
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            A mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) mx = v[c][k] > mx ? v[c][k] : mx;
            A sum = A(0);
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) {
                    v[c][k] = exp(v[c][k] - mx);
                    sum += v[c][k];
                }
            const A inv = A(1) / sum;
            const int sc = s0 + c * 64;
            if (sc < S) {
#pragma unroll
                for (int k = 0; k < KS; ++k)
                    if (tap_on<KC>(k, K)) yb[k * S + sc] = from_acc<T, A>(v[c][k] * inv);
            }
        }
    }
}

// gx = y * (gy - sum_k gy_k * y_k)
template <typename T, typename A, int KC, int CPT>
__global__ void __launch_bounds__(SB) softmax_bwd_kernel(const T *__restrict__ y, const T *__restrict__ gy,
                                                         T *__restrict__ gx, int BG, int K, int S) {
    constexpr int KS = tap_slots<KC>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = (blockIdx.x * (SB / 64) + wave) * (64 * CPT) + lane;
    for (int bg = blockIdx.y; bg < BG; bg += gridDim.y) {
        const size_t o = (size_t)bg * K * S;
        A yv[CPT][KS], gv[CPT][KS];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int sc = min(s0 + c * 64, S - 1);
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) {
                    yv[c][k] = to_acc<A>(y[o + k * S + sc]);
                    gv[c][k] = to_acc<A>(gy[o + k * S + sc]);
                }
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            A dot = A(0);
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) dot += yv[c][k] * gv[c][k];
            const int sc = s0 + c * 64;
            if (sc < S) {
#pragma unroll
                for (int k = 0; k < KS; ++k)
                    if (tap_on<KC>(k, K)) gx[o + k * S + sc] = from_acc<T, A>(yv[c][k] * (gv[c][k] - dot));
            }
        }
    }
}

// K > KMAX_REG, or more than 2^31 elements: one column per thread, 64-bit indices, re-reads
template <typename T, typename A>
__global__ void __launch_bounds__(SB) softmax_fwd_loop_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t BG,
                                                              int K, int64_t S) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= BG * S) return;
    const int64_t bg = i / S, s = i - bg * S;
    const T *xi = x + bg * K * S + s;
    T *yi = y + bg * K * S + s;
    A mx = -INFINITY;
    for (int k = 0; k < K; ++k) {
        const A a = to_acc<A>(xi[k * S]);
        mx = a > mx ? a : mx;
    }
    A sum = A(0);
    for (int k = 0; k < K; ++k) sum += exp(to_acc<A>(xi[k * S]) - mx);
    const A inv = A(1) / sum;
    for (int k = 0; k < K; ++k) yi[k * S] = from_acc<T, A>(exp(to_acc<A>(xi[k * S]) - mx) * inv);
}

template <typename T, typename A>
__global__ void __launch_bounds__(SB) softmax_bwd_loop_kernel(const T *__restrict__ y, const T *__restrict__ gy,
                                                              T *__restrict__ gx, int64_t BG, int K, int64_t S) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= BG * S) return;
    const int64_t bg = i / S, s = i - bg * S;
    const int64_t o = bg * K * S + s;
    A dot = A(0);
    for (int k = 0; k < K; ++k) dot += to_acc<A>(y[o + k * S]) * to_acc<A>(gy[o + k * S]);
    for (int k = 0; k < K; ++k)
        gx[o + k * S] = from_acc<T, A>(to_acc<A>(y[o + k * S]) * (to_acc<A>(gy[o + k * S]) - dot));
}

// Gradient with respect to the logits of a mask the convolution kernels softmax-activated in
// their mask load: g (accumulation type, in place) holds d(loss)/d(y) summed over channels;
// y is recomputed from the logits x as in the forward, then g <- y * (g - sum_k g_k * y_k).
// Register version (K <= KMAX_REG, 32-bit indices): one read of x and g, one write of g.
template <typename T, typename A, int KC, int CPT>
__global__ void __launch_bounds__(SB) softmax_logit_grad_reg_kernel(const T *__restrict__ x, A *__restrict__ g, int BG,
                                                                    int K, int S) {
    constexpr int KS = tap_slots<KC>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = (blockIdx.x * (SB / 64) + wave) * (64 * CPT) + lane;
    for (int bg = blockIdx.y; bg < BG; bg += gridDim.y) {
        const size_t o = (size_t)bg * K * S;
        A xv[CPT][KS], gv[CPT][KS];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int sc = min(s0 + c * 64, S - 1);
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) {
                    xv[c][k] = to_acc<A>(x[o + k * S + sc]);
                    gv[c][k] = g[o + k * S + sc];
                }
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            A mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) mx = xv[c][k] > mx ? xv[c][k] : mx;
            A sum = A(0), dot = A(0);
#pragma unroll
            for (int k = 0; k < KS; ++k)
                if (tap_on<KC>(k, K)) {
                    xv[c][k] = exp(xv[c][k] - mx);
                    sum += xv[c][k];
                    dot += xv[c][k] * gv[c][k];
                }
            const A inv = A(1) / sum;
            dot *= inv;
            const int sc = s0 + c * 64;
            if (sc < S) {
#pragma unroll
                for (int k = 0; k < KS; ++k)
                    if (tap_on<KC>(k, K)) g[o + k * S + sc] = xv[c][k] * inv * (gv[c][k] - dot);
            }
        }
    }
}

template <typename T, typename A>
__global__ void __launch_bounds__(SB) softmax_logit_grad_kernel(const T *__restrict__ x, A *__restrict__ g,
                                                                int64_t BG, int K, int64_t S) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= BG * S) return;
    const int64_t bg = i / S, s = i - bg * S;
    const int64_t o = bg * K * S + s;
    A mx = -INFINITY;
    for (int k = 0; k < K; ++k) {
        const A v = to_acc<A>(x[o + k * S]);
        mx = v > mx ? v : mx;
    }
    A sum = A(0), dot = A(0);
    for (int k = 0; k < K; ++k) {
        const A e = exp(to_acc<A>(x[o + k * S]) - mx);
        sum += e;
        dot += e * g[o + k * S];
    }
    const A inv = A(1) / sum;
    dot *= inv;
    for (int k = 0; k < K; ++k) {
        const A y = exp(to_acc<A>(x[o + k * S]) - mx) * inv;
        g[o + k * S] = y * (g[o + k * S] - dot);
    }
}

// Register kernels: small problems take one column per thread (more threads in flight), large
// ones four (tap counts up to 16: the registers of four columns); common tap counts get their
// own instantiation.
// grid of the register kernels at cpt columns per thread: (s blocks, bg)
dim3 grid_of(int64_t BG, int64_t S, int cpt) {
    const int64_t sblocks = (S + (int64_t)SB * cpt - 1) / ((int64_t)SB * cpt);
    return dim3((unsigned)sblocks, (unsigned)std::min<int64_t>(BG, 65535));
}
// four columns per thread for large problems with a compile-time tap count up to 16
bool four_columns(int KC, int64_t BG, int64_t S) { return KC != 0 && KC <= 16 && BG * S >= (int64_t)256 * 1024; }
bool reg_path(int64_t BG, int K, int64_t S) { return K <= KMAX_REG && BG * K * S < INT32_MAX && S > 0; }

template <typename F>
hipError_t by_taps(int K, F &&f) {
    switch (K) {
        case 3: return f(std::integral_constant<int, 3>());
        case 4: return f(std::integral_constant<int, 4>());
        case 5: return f(std::integral_constant<int, 5>());
        case 9: return f(std::integral_constant<int, 9>());
        case 16: return f(std::integral_constant<int, 16>());
        case 25: return f(std::integral_constant<int, 25>());
        case 27: return f(std::integral_constant<int, 27>());
        default: return f(std::integral_constant<int, 0>());
    }
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

}  // namespace

hipError_t launch_mask_softmax_fwd(int dtype, const void *x, void *y, int64_t BG, int K, int64_t S, hipStream_t s) {
    const int64_t n = BG * S;
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        if (!reg_path(BG, K, S)) {
            hipLaunchKernelGGL((softmax_fwd_loop_kernel<T, A>), dim3((unsigned)((n + SB - 1) / SB)), dim3(SB), 0, s,
                               static_cast<const T *>(x), static_cast<T *>(y), BG, K, S);
            return hipGetLastError();
        }
        return by_taps(K, [&](auto kc) {
            constexpr int KC = decltype(kc)::value;
            if (four_columns(KC, BG, S))
                hipLaunchKernelGGL((softmax_fwd_kernel<T, A, KC, 4>), grid_of(BG, S, 4), dim3(SB), 0, s,
                                   static_cast<const T *>(x), static_cast<T *>(y), (int)BG, K, (int)S);
            else
                hipLaunchKernelGGL((softmax_fwd_kernel<T, A, KC, 1>), grid_of(BG, S, 1), dim3(SB), 0, s,
                                   static_cast<const T *>(x), static_cast<T *>(y), (int)BG, K, (int)S);
            return hipGetLastError();
        });
    });
}

hipError_t launch_mask_softmax_bwd(int dtype, const void *y, const void *gy, void *gx, int64_t BG, int K, int64_t S,
                                   hipStream_t s) {
    const int64_t n = BG * S;
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        if (!reg_path(BG, K, S)) {
            hipLaunchKernelGGL((softmax_bwd_loop_kernel<T, A>), dim3((unsigned)((n + SB - 1) / SB)), dim3(SB), 0, s,
                               static_cast<const T *>(y), static_cast<const T *>(gy), static_cast<T *>(gx), BG, K, S);
            return hipGetLastError();
        }
        return by_taps(K, [&](auto kc) {
            constexpr int KC = decltype(kc)::value;
            if (four_columns(KC, BG, S))
                hipLaunchKernelGGL((softmax_bwd_kernel<T, A, KC, 4>), grid_of(BG, S, 4), dim3(SB), 0, s,
                                   static_cast<const T *>(y), static_cast<const T *>(gy), static_cast<T *>(gx), (int)BG,
                                   K, (int)S);
            else
                hipLaunchKernelGGL((softmax_bwd_kernel<T, A, KC, 1>), grid_of(BG, S, 1), dim3(SB), 0, s,
                                   static_cast<const T *>(y), static_cast<const T *>(gy), static_cast<T *>(gx), (int)BG,
                                   K, (int)S);
            return hipGetLastError();
        });
    });
}

hipError_t launch_mask_softmax_logit_grad(int dtype, const void *logits, void *gmask_acc, int64_t BG, int K, int64_t S,
                                          hipStream_t s) {
    const int64_t n = BG * S;
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        if (!reg_path(BG, K, S)) {
            hipLaunchKernelGGL((softmax_logit_grad_kernel<T, A>), dim3((unsigned)((n + SB - 1) / SB)), dim3(SB), 0, s,
                               static_cast<const T *>(logits), static_cast<A *>(gmask_acc), BG, K, S);
            return hipGetLastError();
        }
        return by_taps(K, [&](auto kc) {
            constexpr int KC = decltype(kc)::value;
            if (four_columns(KC, BG, S))
                hipLaunchKernelGGL((softmax_logit_grad_reg_kernel<T, A, KC, 4>), grid_of(BG, S, 4), dim3(SB), 0, s,
                                   static_cast<const T *>(logits), static_cast<A *>(gmask_acc), (int)BG, K, (int)S);
            else
                hipLaunchKernelGGL((softmax_logit_grad_reg_kernel<T, A, KC, 1>), grid_of(BG, S, 1), dim3(SB), 0, s,
                                   static_cast<const T *>(logits), static_cast<A *>(gmask_acc), (int)BG, K, (int)S);
            return hipGetLastError();
        });
    });
}

}  // namespace tvdcn_hip
