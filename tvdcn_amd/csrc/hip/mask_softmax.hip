// mask_softmax forward / backward over the kernel taps.
//
// The mask (B, mg*K, *S) is viewed as (B*mg, K, S) and normalised over K
// (reference: tvdcn/ops/activations/mask_softmax.py:19-126, torch.softmax on the
// view). K is strided by S in memory, so the reduction axis runs *down* a lane,
// not across lanes: each lane owns one (b, g, s) column and keeps its K values
// in registers, while the 64 lanes of a wavefront cover 64 consecutive s, which
// makes every load and store a fully coalesced 256-byte wavefront access. One
// read + one write per element in the forward (2 passes over HBM-equivalent
// bytes), two reads + one write in the backward. K > 32 falls back to a
// re-reading loop (three passes).
#include "kernels.h"

namespace tvdcn_hip {
namespace {

constexpr int KMAX_REG = 32;

template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_fwd_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t BG,
                                                          int K, int64_t S) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= BG * S) return;
    const int64_t bg = i / S, s = i - bg * S;
    const T *xi = x + bg * K * S + s;
    T *yi = y + bg * K * S + s;
    if (K <= KMAX_REG) {
        A v[KMAX_REG];
        A mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < KMAX_REG; ++k)
            if (k < K) {
                v[k] = to_acc<A>(xi[k * S]);
                mx = v[k] > mx ? v[k] : mx;
            }
        A sum = A(0);
#pragma unroll
        for (int k = 0; k < KMAX_REG; ++k)
            if (k < K) {
                v[k] = exp(v[k] - mx);
                sum += v[k];
            }
        const A inv = A(1) / sum;
#pragma unroll
        for (int k = 0; k < KMAX_REG; ++k)
            if (k < K) yi[k * S] = from_acc<T, A>(v[k] * inv);
    } else {
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
}

// gx = y * (gy - sum_k gy_k * y_k)
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_bwd_kernel(const T *__restrict__ y, const T *__restrict__ gy,
                                                          T *__restrict__ gx, int64_t BG, int K, int64_t S) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= BG * S) return;
    const int64_t bg = i / S, s = i - bg * S;
    const int64_t o = bg * K * S + s;
    if (K <= KMAX_REG) {
        A yv[KMAX_REG], gv[KMAX_REG];
        A dot = A(0);
#pragma unroll
        for (int k = 0; k < KMAX_REG; ++k)
            if (k < K) {
                yv[k] = to_acc<A>(y[o + k * S]);
                gv[k] = to_acc<A>(gy[o + k * S]);
                dot += yv[k] * gv[k];
            }
#pragma unroll
        for (int k = 0; k < KMAX_REG; ++k)
            if (k < K) gx[o + k * S] = from_acc<T, A>(yv[k] * (gv[k] - dot));
    } else {
        A dot = A(0);
        for (int k = 0; k < K; ++k) dot += to_acc<A>(y[o + k * S]) * to_acc<A>(gy[o + k * S]);
        for (int k = 0; k < K; ++k)
            gx[o + k * S] = from_acc<T, A>(to_acc<A>(y[o + k * S]) * (to_acc<A>(gy[o + k * S]) - dot));
    }
}

// Gradient with respect to the logits of a mask the convolution kernels softmax-activated in
// their mask load: g (accumulation type, in place) holds d(loss)/d(y) summed over channels;
// y is recomputed from the logits x as in the forward, then g <- y * (g - sum_k g_k * y_k).
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_logit_grad_kernel(const T *__restrict__ x, A *__restrict__ g,
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
        hipLaunchKernelGGL((softmax_fwd_kernel<T, A>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           static_cast<const T *>(x), static_cast<T *>(y), BG, K, S);
        return hipGetLastError();
    });
}

hipError_t launch_mask_softmax_bwd(int dtype, const void *y, const void *gy, void *gx, int64_t BG, int K, int64_t S,
                                   hipStream_t s) {
    const int64_t n = BG * S;
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((softmax_bwd_kernel<T, A>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           static_cast<const T *>(y), static_cast<const T *>(gy), static_cast<T *>(gx), BG, K, S);
        return hipGetLastError();
    });
}

hipError_t launch_mask_softmax_logit_grad(int dtype, const void *logits, void *gmask_acc, int64_t BG, int K, int64_t S,
                                          hipStream_t s) {
    const int64_t n = BG * S;
    if (n == 0) return hipSuccess;
    return by_dtype(dtype, [&](auto tv, auto av) {
        using T = decltype(tv);
        using A = decltype(av);
        hipLaunchKernelGGL((softmax_logit_grad_kernel<T, A>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           static_cast<const T *>(logits), static_cast<A *>(gmask_acc), BG, K, S);
        return hipGetLastError();
    });
}

}  // namespace tvdcn_hip
