/*
 * tvdcn_hip.h -- C ABI of the MI355X (gfx950) deformable-convolution library
 * (libtvdcn_hip.so). Plain pointers and sizes only: no torch, no C++ types.
 *
 * Every entry point is stateless, re-entrant and stream-ordered: work is
 * enqueued on `stream` (a hipStream_t passed as void*; NULL = legacy default
 * stream), nothing is synchronised, no device memory is allocated or freed,
 * and no pointer is kept after return. Device buffers are dense, contiguous
 * in the reference's layouts (NC<spatial>, row-major), 16-byte aligned, and of
 * the element type named by `dtype`. Scratch memory is supplied by the caller
 * as `workspace` of at least the size returned by the matching *_workspace_size
 * query. Errors return a non-zero tvdcn_status; tvdcn_last_error() then holds a
 * thread-local message.
 *
 * Reference interface being replaced (tvdcn 1.1.0, paths relative to
 * tvdcn/csrc/): the twelve `tvdcn::` operator schemas
 *   deform_conv{1,2,3}d               ops/deform_conv1d.cpp:82-91, ops/deform_conv2d.cpp:117-126,
 *                                     ops/deform_conv3d.cpp (same block)
 *   _deform_conv{1,2,3}d_backward     same TORCH_LIBRARY_FRAGMENT blocks
 *   deform_conv_transpose{1,2,3}d     ops/deform_conv_transpose2d.cpp:125-136 and the 1D/3D twins
 *   _deform_conv_transpose{1,2,3}d_backward   same blocks
 * whose CUDA-key kernels are ops/cuda/deform_conv*_kernel.cpp (forward / backward
 * drivers), and the Python-level mask_softmax{1,2,3}d (ops/activations/mask_softmax.py).
 */
#ifndef TVDCN_HIP_H
#define TVDCN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TVDCN_DTYPE_FLOAT32 = 0,
    TVDCN_DTYPE_FLOAT64 = 1,
    TVDCN_DTYPE_FLOAT16 = 2,
    TVDCN_DTYPE_BFLOAT16 = 3
} tvdcn_dtype;

typedef enum {
    TVDCN_STATUS_SUCCESS = 0,
    TVDCN_STATUS_INVALID_ARGUMENT = 1,   /* shape / parameter check failed (RuntimeError in the reference) */
    TVDCN_STATUS_WORKSPACE_TOO_SMALL = 2,
    TVDCN_STATUS_NOT_SUPPORTED = 3,      /* e.g. one image's tensor above the batch-block limit */
    TVDCN_STATUS_HIP_ERROR = 4           /* a kernel launch failed */
} tvdcn_status;

/*
 * Problem descriptor shared by the conv and transposed-conv entry points.
 * Spatial arrays hold `dim` entries in the reference's axis order ((d,) h, w).
 *   conv       (transposed = 0): input (batch, in_channels, *in_size),
 *              weight (out_channels, in_channels / groups, *kernel),
 *              offset (batch, offset_groups * dim * prod(kernel), *out_size),
 *              mask   (batch, mask_groups * prod(kernel), *out_size),
 *              bias   (out_channels), output (batch, out_channels, *out_size)
 *   transposed (transposed = 1): input (batch, in_channels, *in_size),
 *              weight (in_channels, out_channels / groups, *kernel),
 *              offset / mask on the *input* grid (*in_size),
 *              output (batch, out_channels, *out_size)
 * offset_groups = 0 means offset is None; mask_groups = 0 means mask is None.
 * output_padding is used only when transposed = 1.
 * flags: TVDCN_FLAG_CHANNELS_LAST (conv only) = input, and in the backward grad_input, are in
 * channels-last order (batch, *in_size, in_channels); every other tensor keeps the layout
 * above. No counterpart in the reference, which makes every input NC<spatial>-contiguous
 * (cuda/deform_conv2d_kernel.cpp:114-118); it spares the layout copies for callers whose
 * activations are channels-last.
 * TVDCN_FLAG_MASK_SIGMOID = the mask tensor holds logits: the kernels use
 * mask_scale * sigmoid(logit) as the mask (tvdcn's MaskSigmoid, ops/activations/mask_sigmoid.py:11-21,
 * folded into the mask load), and the backward's grad_mask is the gradient with respect to the
 * logits. Needs a mask and mask_scale > 0. No counterpart in the reference, whose packed modules
 * run the activation as a separate pass.
 * TVDCN_FLAG_MASK_SOFTMAX = the mask tensor holds logits: the kernels use their softmax over the
 * prod(kernel) taps of each (batch, mask group, column pixel) as the mask (tvdcn's
 * mask_softmax{1,2,3}d, ops/activations/mask_softmax.py:19-126, folded into the mask load), and
 * the backward's grad_mask is the gradient with respect to the logits. Needs a mask; excludes
 * TVDCN_FLAG_MASK_SIGMOID. Same counterpart as above.
 */
#define TVDCN_FLAG_CHANNELS_LAST 1
#define TVDCN_FLAG_MASK_SIGMOID 2
#define TVDCN_FLAG_MASK_SOFTMAX 4
typedef struct {
    int32_t dim;
    int32_t transposed;
    int32_t dtype;            /* tvdcn_dtype */
    int32_t flags;            /* TVDCN_FLAG_*; 0 = the layouts above */
    int64_t batch;
    int64_t in_channels;
    int64_t out_channels;
    int64_t groups;
    int64_t offset_groups;
    int64_t mask_groups;
    int64_t in_size[3];
    int64_t kernel[3];
    int64_t stride[3];
    int64_t padding[3];
    int64_t dilation[3];
    int64_t output_padding[3];
    double mask_scale;        /* TVDCN_FLAG_MASK_SIGMOID only */
} tvdcn_conv_desc;

/* Output spatial size (out_size[0..dim)); returns TVDCN_STATUS_SUCCESS or an error
 * when the descriptor fails the reference's shape checks. */
tvdcn_status tvdcn_conv_output_size(const tvdcn_conv_desc *desc, int64_t out_size[3]);

/* Bytes of workspace needed by tvdcn_deform_conv_forward / _backward (0 when the descriptor is
 * invalid). The kernels index in 32 bits: the entry points run the batch in blocks of images whose
 * tensors hold at most tvdcn_set_max_block_elements' limit of elements each (2^31 - 1 by default;
 * the weight gradient is accumulated over the blocks), and the workspace serves one block at a
 * time. The reference blocks its batch as well (n_parallel_imgs, ops/utils/parallel_helpers.h:7-16,
 * ops/cuda/deform_conv2d_kernel.cpp:149). One image above the limit is TVDCN_STATUS_NOT_SUPPORTED. */
size_t tvdcn_deform_conv_forward_workspace_size(const tvdcn_conv_desc *desc);
size_t tvdcn_deform_conv_backward_workspace_size(const tvdcn_conv_desc *desc);

/* Sets the largest element count of any batch-sized tensor in one batch block (1 .. 2^31 - 1;
 * default 2^31 - 1): a lower limit means smaller blocks and a smaller workspace. Process-wide;
 * call it while no entry point runs. Counterpart of the reference's kMaxParallelImgs
 * (ops/utils/parallel_helpers.h:7-16), counted in elements instead of images. */
tvdcn_status tvdcn_set_max_block_elements(int64_t max_elements);

/* Images per batch block of a call described by desc (0 for an empty batch), under the current
 * limit. When the batch is split, the block is rounded down to a multiple of the image count m at
 * which every batch-sized tensor's bytes reach a multiple of 16 (m <= 16), so that each block's
 * pointers are as aligned as the caller's; when fewer than m images fit in a block, later blocks'
 * pointers may be less aligned, which the kernels accept. Counterpart of the reference's
 * n_parallel_imgs = get_greatest_divisor_below_bound(batch, kMaxParallelImgs)
 * (ops/utils/parallel_helpers.h:7-16, ops/cuda/deform_conv2d_kernel.cpp:149), a query here. */
tvdcn_status tvdcn_conv_batch_block(const tvdcn_conv_desc *desc, int64_t *images_per_block);

/*
 * Forward of deform_conv{1,2,3}d / deform_conv_transpose{1,2,3}d.
 * Replaces the CUDA-key forward drivers ops/cuda/deform_conv2d_kernel.cpp:85-385,
 * ops/cuda/deform_conv_transpose2d_kernel.cpp:85-372 and their 1D/3D twins,
 * called through the schemas listed above. offset, mask, bias may be NULL.
 */
tvdcn_status tvdcn_deform_conv_forward(const tvdcn_conv_desc *desc, const void *input, const void *weight,
                                       const void *offset, const void *mask, const void *bias, void *output,
                                       void *workspace, size_t workspace_bytes, void *stream);

/*
 * Allocation-free variant of tvdcn_deform_conv_forward. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, checks and results as
 * tvdcn_deform_conv_forward minus the workspace: the forward's scratch memory (the channels-last
 * copy of the input, the weight re-layout, the split accumulator) is a library-owned device array
 * of TVDCN_SCRATCH_BYTES per GPU, held until the process ends; its address is looked up at the
 * first call on each device. A problem whose forward workspace
 * (tvdcn_deform_conv_forward_workspace_size) exceeds TVDCN_SCRATCH_BYTES returns
 * TVDCN_STATUS_WORKSPACE_TOO_SMALL with a message naming both sizes (a float32 input passed
 * channels-last, TVDCN_FLAG_CHANNELS_LAST, needs no input copy: only the weight re-layout).
 * Every call on a GPU uses that GPU's one array: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialised by the caller. No hipMalloc / hipFree, no
 * allocating library call.
 */
#define TVDCN_SCRATCH_BYTES (64u << 20)
tvdcn_status tvdcn_deform_conv_forward_noalloc(const tvdcn_conv_desc *desc, const void *input, const void *weight,
                                               const void *offset, const void *mask, const void *bias, void *output,
                                               void *stream);

/*
 * Backward (the `_..._backward` schemas). Replaces ops/cuda/deform_conv2d_kernel.cpp:387-642,
 * ops/cuda/deform_conv_transpose2d_kernel.cpp:374-636 and their 1D/3D twins.
 * grad_offset must be NULL iff offset is NULL, grad_mask iff mask is NULL;
 * grad_bias may be NULL (not computed). All outputs are overwritten.
 */
tvdcn_status tvdcn_deform_conv_backward(const tvdcn_conv_desc *desc, const void *grad_out, const void *input,
                                        const void *weight, const void *offset, const void *mask, void *grad_input,
                                        void *grad_weight, void *grad_offset, void *grad_mask, void *grad_bias,
                                        void *workspace, size_t workspace_bytes, void *stream);

/*
 * mask_softmax{1,2,3}d (ops/activations/mask_softmax.py:19-126): x viewed as
 * (batch * groups, kernel_numel, spatial_numel), softmax over the middle axis.
 * Backward: grad_x = y * (grad_y - sum_k grad_y * y).
 */
tvdcn_status tvdcn_mask_softmax_forward(int32_t dtype, int64_t batch, int64_t groups, int64_t kernel_numel,
                                        int64_t spatial_numel, const void *x, void *y, void *stream);
tvdcn_status tvdcn_mask_softmax_backward(int32_t dtype, int64_t batch, int64_t groups, int64_t kernel_numel,
                                         int64_t spatial_numel, const void *y, const void *grad_y, void *grad_x,
                                         void *stream);

/*
 * Copies a float32 NC<spatial> tensor (batch x channels x spatial_numel, contiguous) into
 * channels-last order N<spatial>C, the order the convolution kernels sample. Passed as the
 * input of tvdcn_deform_conv_forward / _backward with TVDCN_FLAG_CHANNELS_LAST, the copy
 * stands in for the layout copy each of those calls makes otherwise, so one copy can serve a
 * forward and its backward. No counterpart in the reference (its kernels gather from
 * NC<spatial> directly, tvdcn/csrc/ops/cuda/deform_conv2d_common_kernels.cu:170-200); for
 * training loops that keep the input of a forward for its backward.
 */
tvdcn_status tvdcn_to_channels_last(int32_t dtype, int64_t batch, int64_t channels, int64_t spatial_numel,
                                    const void *input, void *output, void *stream);
/* The inverse copy, N<spatial>C -> NC<spatial> (float32): brings a gradient that a
 * channels-last backward call wrote back to the order of the caller's tensor. */
tvdcn_status tvdcn_from_channels_last(int32_t dtype, int64_t batch, int64_t channels, int64_t spatial_numel,
                                      const void *input, void *output, void *stream);

/* Thread-local text of the last error (empty string when none). */
const char *tvdcn_last_error(void);

/* Library identity (replaces tvdcn/csrc/tvdcn.cpp:24-48 `_cuda_version` /
 * `_cuda_arch_flags`): HIP runtime version the library was built against
 * (HIP_VERSION, e.g. 70226015) and the offload targets ("gfx950"). */
int64_t tvdcn_hip_version(void);
const char *tvdcn_arch_flags(void);

/*
 * Optional kernel timing (no counterpart in the reference; used by bench.py).
 * When enabled, every kernel launch of the entry points above is bracketed by
 * two HIP events recorded on its launch stream. tvdcn_kernel_timer_read waits
 * for the recorded events and returns the summed elapsed time and launch count
 * of one kernel family since the last enable call. Enabling (or disabling)
 * clears the totals. Off by default; costs two event records per launch when on.
 */
enum {
    TVDCN_KERNEL_LAYOUT = 0,        /* channels-last / weight re-layouts, fills, casts */
    TVDCN_KERNEL_GATHER_GEMM = 1,   /* fused deformable gather + MFMA contraction */
    TVDCN_KERNEL_DATA_GRAD = 2,     /* MFMA grad-columns + scatter / offset-mask grads */
    TVDCN_KERNEL_WEIGHT_GRAD = 3,   /* re-gather + MFMA weight gradient */
    TVDCN_KERNEL_BIAS_GRAD = 4,
    TVDCN_KERNEL_MASK_SOFTMAX = 5,
    TVDCN_KERNEL_FAMILIES = 6
};
void tvdcn_kernel_timer_enable(int32_t enable);
tvdcn_status tvdcn_kernel_timer_read(int32_t family, double *total_ms, int64_t *launches);

#ifdef __cplusplus
}
#endif
#endif /* TVDCN_HIP_H */
