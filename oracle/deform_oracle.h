/*
 * deform_oracle.h -- CPU restatement of tvdcn's deformable-convolution math.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * implementation in tvdcn_amd/. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. Product code never links it.
 *
 * All arithmetic is float64. Spatial problems of rank 1, 2 and 3 are handled by
 * embedding them in rank 3 with unit leading extents; that embedding reproduces
 * the reference's per-rank helpers exactly (a unit extent only ever contributes a
 * factor 1.0 and a skipped out-of-range corner).
 *
 * Layout conventions are the reference's (all NC<spatial>, contiguous):
 *   conv:       input (B, Cin, *S_in), weight (Cout, Cin/G, *K),
 *               offset (B, og*dim*prod(K), *S_out), mask (B, mg*prod(K), *S_out)
 *   transposed: input (B, Cin, *S_in), weight (Cin, Cout/G, *K),
 *               offset (B, og*dim*prod(K), *S_in), mask (B, mg*prod(K), *S_in)
 */
#ifndef TVDCN_DEFORM_ORACLE_H
#define TVDCN_DEFORM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t dim;            /* 1, 2 or 3 */
    int32_t transposed;     /* 0: deform_convNd, 1: deform_conv_transposeNd */
    int64_t batch;
    int64_t in_channels;
    int64_t out_channels;
    int64_t groups;
    int64_t offset_groups;  /* 0 when offset is None */
    int64_t mask_groups;    /* 0 when mask is None */
    /* per spatial axis, in the reference's order ((d,) h, w); only [0, dim) used */
    int64_t in_size[3];
    int64_t kernel[3];
    int64_t stride[3];
    int64_t padding[3];
    int64_t dilation[3];
    int64_t output_padding[3];
} oracle_conv_desc;

/* Output spatial size of the op, per axis; returns prod. */
int64_t oracle_output_size(const oracle_conv_desc *d, int64_t out_size[3]);

/* Forward. offset / mask / bias may be NULL (None). */
void oracle_deform_conv_forward(const oracle_conv_desc *d,
                                const double *input, const double *weight,
                                const double *offset, const double *mask,
                                const double *bias, double *output);

/* Backward. grad_offset / grad_mask / grad_bias may be NULL when the matching
 * forward argument was None. All outputs are overwritten. */
void oracle_deform_conv_backward(const oracle_conv_desc *d,
                                 const double *grad_out, const double *input,
                                 const double *weight, const double *offset,
                                 const double *mask,
                                 double *grad_input, double *grad_weight,
                                 double *grad_offset, double *grad_mask,
                                 double *grad_bias);

/* mask_softmax: x viewed as (B, groups, K, S), softmax over K. */
void oracle_mask_softmax_forward(int64_t B, int64_t groups, int64_t K, int64_t S,
                                 const double *x, double *y);
/* backward of the above: gx = y * (gy - sum_k gy*y) */
void oracle_mask_softmax_backward(int64_t B, int64_t groups, int64_t K, int64_t S,
                                  const double *y, const double *gy, double *gx);

#ifdef __cplusplus
}
#endif
#endif
