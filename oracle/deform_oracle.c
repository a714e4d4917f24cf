/*
 * deform_oracle.c -- float64 CPU restatement of tvdcn 1.1.0's deformable
 * convolution (forward, backward, transposed) and mask_softmax.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for tvdcn_amd's HIP kernels.
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
 * never by product code.
 *
 * Every function names the reference lines it restates (paths relative to the
 * reference's tvdcn/csrc/ops/). The reference keeps one file per spatial rank;
 * here rank 1 and 2 are embedded in rank 3 (unit leading extents, zero offset on
 * the missing axes), which reproduces the per-rank helpers bit for bit: a unit
 * axis contributes exactly the factor 1.0 on its low corner and an always
 * out-of-range high corner.
 */
#include "deform_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* geometry                                                                   */
/* ------------------------------------------------------------------------- */

typedef struct {
    int dim;
    int64_t B;
    int64_t C;       /* channels of the sampled side (conv: Cin, transposed: Cout) */
    int64_t M;       /* channels of the GEMM side (conv: Cout, transposed: Cin)    */
    int64_t G;
    int64_t og, mg;  /* 0 when absent */
    int64_t cpo, cpm;
    int64_t S[3];    /* sampled grid, embedded in rank 3 */
    int64_t P[3];    /* column grid (where offsets/masks live), rank 3 */
    int64_t K[3], st[3], pad[3], dil[3];
    int64_t Sn, Pn, Kn;
} geo_t;

static void embed3(int dim, const int64_t *src, int64_t fill, int64_t dst[3]) {
    for (int i = 0; i < 3; ++i) dst[i] = fill;
    for (int i = 0; i < dim; ++i) dst[3 - dim + i] = src[i];
}

/* Output sizes: conv follows cpu/deform_conv2d_kernel.cpp:167-168,
 * transposed follows cpu/deform_conv_transpose2d_kernel.cpp:172-173 (and the
 * 1D/3D twins). */
int64_t oracle_output_size(const oracle_conv_desc *d, int64_t out_size[3]) {
    int64_t prod = 1;
    for (int i = 0; i < d->dim; ++i) {
        int64_t o;
        if (!d->transposed)
            o = (d->in_size[i] + 2 * d->padding[i] - (d->dilation[i] * (d->kernel[i] - 1) + 1)) / d->stride[i] + 1;
        else
            o = (d->in_size[i] - 1) * d->stride[i] - 2 * d->padding[i] + d->dilation[i] * (d->kernel[i] - 1) + 1 +
                d->output_padding[i];
        out_size[i] = o;
        prod *= o;
    }
    return prod;
}

static void make_geo(const oracle_conv_desc *d, geo_t *g) {
    int64_t out[3];
    oracle_output_size(d, out);
    g->dim = d->dim;
    g->B = d->batch;
    g->G = d->groups;
    g->og = d->offset_groups;
    g->mg = d->mask_groups;
    if (!d->transposed) {
        g->C = d->in_channels;
        g->M = d->out_channels;
        embed3(d->dim, d->in_size, 1, g->S);
        embed3(d->dim, out, 1, g->P);
    } else {
        g->C = d->out_channels;
        g->M = d->in_channels;
        embed3(d->dim, out, 1, g->S);
        embed3(d->dim, d->in_size, 1, g->P);
    }
    /* channels per offset/mask group: cpu/deform_conv2d_common_kernels.cpp:216-217 */
    g->cpo = g->og ? g->C / g->og : 1;
    g->cpm = g->mg ? g->C / g->mg : 1;
    embed3(d->dim, d->kernel, 1, g->K);
    embed3(d->dim, d->stride, 1, g->st);
    embed3(d->dim, d->padding, 0, g->pad);
    embed3(d->dim, d->dilation, 1, g->dil);
    g->Sn = g->S[0] * g->S[1] * g->S[2];
    g->Pn = g->P[0] * g->P[1] * g->P[2];
    g->Kn = g->K[0] * g->K[1] * g->K[2];
}

/* ------------------------------------------------------------------------- */
/* sampling helpers                                                           */
/* ------------------------------------------------------------------------- */

/* integer sample with zero padding: cpu/deform_conv2d_common_kernels.cpp:10-20
 * (1D :10-18, 3D cpu/deform_conv3d_common_kernels.cpp:10-22) */
static double sample_int(const double *img, const int64_t S[3], int64_t z, int64_t y, int64_t x) {
    if (0 <= z && z < S[0] && 0 <= y && y < S[1] && 0 <= x && x < S[2])
        return img[(z * S[1] + y) * S[2] + x];
    return 0.0;
}

/* bilinear/trilinear sample: cpu/deform_conv2d_common_kernels.cpp:22-55
 * (3D cpu/deform_conv3d_common_kernels.cpp:24-79, 1D cpu/deform_conv1d_common_kernels.cpp:20-41).
 * Early-out when the point is outside (-1, size) on any axis; low corners are
 * only checked against 0 and high corners only against size, as there. */
static double sample_interp(const double *img, const int64_t S[3], double z, double y, double x) {
    if (z <= -1 || S[0] <= z || y <= -1 || S[1] <= y || x <= -1 || S[2] <= x)
        return 0.0;
    int64_t zl = (int64_t) floor(z), yl = (int64_t) floor(y), xl = (int64_t) floor(x);
    int64_t zh = zl + 1, yh = yl + 1, xh = xl + 1;
    double dzh = z - zl, dyh = y - yl, dxh = x - xl;
    double dzl = 1 - dzh, dyl = 1 - dyh, dxl = 1 - dxh;
    int vzl = zl >= 0, vzh = zh < S[0], vyl = yl >= 0, vyh = yh < S[1], vxl = xl >= 0, vxh = xh < S[2];
#define AT(zz, yy, xx) img[((zz) * S[1] + (yy)) * S[2] + (xx)]
    double v = 0;
    if (vzl && vyl && vxl) v += dzl * dyl * dxl * AT(zl, yl, xl);
    if (vzl && vyl && vxh) v += dzl * dyl * dxh * AT(zl, yl, xh);
    if (vzl && vyh && vxl) v += dzl * dyh * dxl * AT(zl, yh, xl);
    if (vzl && vyh && vxh) v += dzl * dyh * dxh * AT(zl, yh, xh);
    if (vzh && vyl && vxl) v += dzh * dyl * dxl * AT(zh, yl, xl);
    if (vzh && vyl && vxh) v += dzh * dyl * dxh * AT(zh, yl, xh);
    if (vzh && vyh && vxl) v += dzh * dyh * dxl * AT(zh, yh, xl);
    if (vzh && vyh && vxh) v += dzh * dyh * dxh * AT(zh, yh, xh);
#undef AT
    return v;
}

/* integer insert: cpu/deform_conv2d_common_kernels.cpp:57-69 */
static void insert_int(double *img, const int64_t S[3], int64_t z, int64_t y, int64_t x, double val) {
    if (0 <= z && z < S[0] && 0 <= y && y < S[1] && 0 <= x && x < S[2])
        img[(z * S[1] + y) * S[2] + x] += val;
}

/* bilinear scatter, no early-out, every corner range-checked on both sides:
 * cpu/deform_conv2d_common_kernels.cpp:71-100 (3D :93-145 of the 3D file,
 * 1D :43-60 of the 1D file) */
static void insert_interp(double *img, const int64_t S[3], double z, double y, double x, double val) {
    int64_t zl = (int64_t) floor(z), yl = (int64_t) floor(y), xl = (int64_t) floor(x);
    int64_t zh = zl + 1, yh = yl + 1, xh = xl + 1;
    double dzh = z - zl, dyh = y - yl, dxh = x - xl;
    double dzl = 1 - dzh, dyl = 1 - dyh, dxl = 1 - dxh;
    int vzl = 0 <= zl && zl < S[0], vzh = 0 <= zh && zh < S[0];
    int vyl = 0 <= yl && yl < S[1], vyh = 0 <= yh && yh < S[1];
    int vxl = 0 <= xl && xl < S[2], vxh = 0 <= xh && xh < S[2];
#define AT(zz, yy, xx) img[((zz) * S[1] + (yy)) * S[2] + (xx)]
    if (vzl && vyl && vxl) AT(zl, yl, xl) += dzl * dyl * dxl * val;
    if (vzl && vyl && vxh) AT(zl, yl, xh) += dzl * dyl * dxh * val;
    if (vzl && vyh && vxl) AT(zl, yh, xl) += dzl * dyh * dxl * val;
    if (vzl && vyh && vxh) AT(zl, yh, xh) += dzl * dyh * dxh * val;
    if (vzh && vyl && vxl) AT(zh, yl, xl) += dzh * dyl * dxl * val;
    if (vzh && vyl && vxh) AT(zh, yl, xh) += dzh * dyl * dxh * val;
    if (vzh && vyh && vxl) AT(zh, yh, xl) += dzh * dyh * dxl * val;
    if (vzh && vyh && vxh) AT(zh, yh, xh) += dzh * dyh * dxh * val;
#undef AT
}

/* d(sample)/d(coordinate `axis`) (axis 0=z, 1=y, 2=x in the rank-3 embedding):
 * the weights along `axis` become -1 (low) / +1 (high); no early-out.
 * cpu/deform_conv2d_common_kernels.cpp:102-133 (3D :147-202 of the 3D file;
 * 1D :62-78 of the 1D file, whose weights are always (-1, +1)). */
static double coord_weight(const double *img, const int64_t S[3], double z, double y, double x, int axis) {
    int64_t zl = (int64_t) floor(z), yl = (int64_t) floor(y), xl = (int64_t) floor(x);
    int64_t zh = zl + 1, yh = yl + 1, xh = xl + 1;
    double dzh = axis == 0 ? 1.0 : z - zl;
    double dyh = axis == 1 ? 1.0 : y - yl;
    double dxh = axis == 2 ? 1.0 : x - xl;
    double dzl = axis == 0 ? -1.0 : 1 - dzh;
    double dyl = axis == 1 ? -1.0 : 1 - dyh;
    double dxl = axis == 2 ? -1.0 : 1 - dxh;
    int vzl = 0 <= zl && zl < S[0], vzh = 0 <= zh && zh < S[0];
    int vyl = 0 <= yl && yl < S[1], vyh = 0 <= yh && yh < S[1];
    int vxl = 0 <= xl && xl < S[2], vxh = 0 <= xh && xh < S[2];
#define AT(zz, yy, xx) img[((zz) * S[1] + (yy)) * S[2] + (xx)]
    double v = 0;
    if (vzl && vyl && vxl) v += dzl * dyl * dxl * AT(zl, yl, xl);
    if (vzl && vyl && vxh) v += dzl * dyl * dxh * AT(zl, yl, xh);
    if (vzl && vyh && vxl) v += dzl * dyh * dxl * AT(zl, yh, xl);
    if (vzl && vyh && vxh) v += dzl * dyh * dxh * AT(zl, yh, xh);
    if (vzh && vyl && vxl) v += dzh * dyl * dxl * AT(zh, yl, xl);
    if (vzh && vyl && vxh) v += dzh * dyl * dxh * AT(zh, yl, xh);
    if (vzh && vyh && vxl) v += dzh * dyh * dxl * AT(zh, yh, xl);
    if (vzh && vyh && vxh) v += dzh * dyh * dxh * AT(zh, yh, xh);
#undef AT
    return v;
}

/* ------------------------------------------------------------------------- */
/* per-(b, tap, column pixel) sampling position                               */
/* ------------------------------------------------------------------------- */

/* Decomposes tap index t and column pixel p, and returns the sample point.
 * Offset channel of (group g, tap t, direction o) is (g*Kn + t)*dim + o with o
 * ordered ((z,) y, x): cpu/deform_conv2d_kernel.cpp:278-286 (offset view
 * (B, og, kh, kw, 2, oh, ow)), 3D cpu/deform_conv3d_kernel.cpp view
 * (B, og, kd, kh, kw, 3, ...), 1D view (B, og, kw, 1, ow).
 * Base point h*stride - pad + i*dilation: cpu/deform_conv2d_common_kernels.cpp:169-170. */
typedef struct {
    int64_t base[3];   /* integer base point */
    double pos[3];     /* base + offset */
} point_t;

static void sample_point(const geo_t *g, const double *offset, int64_t b, int64_t og_idx, int64_t t, int64_t p,
                         point_t *pt) {
    int64_t kk[3], pp[3];
    kk[2] = t % g->K[2];
    kk[1] = (t / g->K[2]) % g->K[1];
    kk[0] = t / (g->K[2] * g->K[1]);
    pp[2] = p % g->P[2];
    pp[1] = (p / g->P[2]) % g->P[1];
    pp[0] = p / (g->P[2] * g->P[1]);
    for (int a = 0; a < 3; ++a) {
        pt->base[a] = pp[a] * g->st[a] - g->pad[a] + kk[a] * g->dil[a];
        pt->pos[a] = (double) pt->base[a];
    }
    if (offset) {
        for (int o = 0; o < g->dim; ++o) {
            int64_t ch = (og_idx * g->Kn + t) * g->dim + o;
            double off = offset[(b * g->og * g->Kn * g->dim + ch) * g->Pn + p];
            pt->pos[3 - g->dim + o] += off;
        }
    }
}

static double mask_value(const geo_t *g, const double *mask, int64_t b, int64_t mg_idx, int64_t t, int64_t p) {
    /* mask channel (g*Kn + t): cpu/deform_conv2d_kernel.cpp:291-298 */
    if (!mask) return 1.0;
    return mask[((b * g->mg + mg_idx) * g->Kn + t) * g->Pn + p];
}

/* ------------------------------------------------------------------------- */
/* im2col / col2im / coordinate gradients                                     */
/* columns layout: [C][Kn][B][Pn] (cpu/deform_conv2d_kernel.cpp:331-340)       */
/* ------------------------------------------------------------------------- */

/* cpu/deform_conv2d_common_kernels.cpp:136-190 (im2col_kernel):
 * columns[c][t][b][p] = sample(src[b][c], point) * mask */
static void im2col(const geo_t *g, const double *src, const double *offset, const double *mask, double *cols) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < g->B; ++b)
        for (int64_t c = 0; c < g->C; ++c) {
            const int64_t ogi = c / g->cpo, mgi = c / g->cpm;
            const double *img = src + (b * g->C + c) * g->Sn;
            for (int64_t t = 0; t < g->Kn; ++t)
                for (int64_t p = 0; p < g->Pn; ++p) {
                    point_t pt;
                    sample_point(g, offset, b, ogi, t, p, &pt);
                    double v = offset ? sample_interp(img, g->S, pt.pos[0], pt.pos[1], pt.pos[2])
                                      : sample_int(img, g->S, pt.base[0], pt.base[1], pt.base[2]);
                    cols[((c * g->Kn + t) * g->B + b) * g->Pn + p] = v * mask_value(g, mask, b, mgi, t, p);
                }
        }
}

/* cpu/deform_conv2d_common_kernels.cpp:251-304 (col2im_kernel; serial there,
 * parallel over (b, c) here, which touches disjoint images):
 * dst[b][c] += bilinear scatter of columns * mask */
static void col2im(const geo_t *g, const double *cols, const double *offset, const double *mask, double *dst) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < g->B; ++b)
        for (int64_t c = 0; c < g->C; ++c) {
            const int64_t ogi = c / g->cpo, mgi = c / g->cpm;
            double *img = dst + (b * g->C + c) * g->Sn;
            for (int64_t p = 0; p < g->Pn; ++p)
                for (int64_t t = 0; t < g->Kn; ++t) {
                    point_t pt;
                    sample_point(g, offset, b, ogi, t, p, &pt);
                    double v = cols[((c * g->Kn + t) * g->B + b) * g->Pn + p] * mask_value(g, mask, b, mgi, t, p);
                    if (offset)
                        insert_interp(img, g->S, pt.pos[0], pt.pos[1], pt.pos[2], v);
                    else
                        insert_int(img, g->S, pt.base[0], pt.base[1], pt.base[2], v);
                }
        }
}

/* cpu/deform_conv2d_common_kernels.cpp:365-424 (compute_grad_offset_kernel):
 * grad_offset[b][og][t][o][p] = sum_{c in og} columns * coord_weight(src, point, o) * mask */
static void grad_offset_kernel(const geo_t *g, const double *cols, const double *src, const double *offset,
                               const double *mask, double *grad_offset) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < g->B; ++b)
        for (int64_t ogi = 0; ogi < g->og; ++ogi)
            for (int64_t t = 0; t < g->Kn; ++t)
                for (int o = 0; o < g->dim; ++o)
                    for (int64_t p = 0; p < g->Pn; ++p) {
                        point_t pt;
                        sample_point(g, offset, b, ogi, t, p, &pt);
                        double acc = 0;
                        for (int64_t c = ogi * g->cpo; c < (ogi + 1) * g->cpo; ++c) {
                            const double *img = src + (b * g->C + c) * g->Sn;
                            double w = coord_weight(img, g->S, pt.pos[0], pt.pos[1], pt.pos[2], 3 - g->dim + o);
                            acc += cols[((c * g->Kn + t) * g->B + b) * g->Pn + p] * w *
                                   mask_value(g, mask, b, c / g->cpm, t, p);
                        }
                        grad_offset[(((b * g->og + ogi) * g->Kn + t) * g->dim + o) * g->Pn + p] = acc;
                    }
}

/* cpu/deform_conv2d_common_kernels.cpp:486-542 (compute_grad_mask_kernel):
 * grad_mask[b][mg][t][p] = sum_{c in mg} columns * sample(src, point) */
static void grad_mask_kernel(const geo_t *g, const double *cols, const double *src, const double *offset,
                             double *grad_mask) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < g->B; ++b)
        for (int64_t mgi = 0; mgi < g->mg; ++mgi)
            for (int64_t t = 0; t < g->Kn; ++t)
                for (int64_t p = 0; p < g->Pn; ++p) {
                    double acc = 0;
                    for (int64_t c = mgi * g->cpm; c < (mgi + 1) * g->cpm; ++c) {
                        const double *img = src + (b * g->C + c) * g->Sn;
                        point_t pt;
                        sample_point(g, offset, b, c / g->cpo, t, p, &pt);
                        double v = offset ? sample_interp(img, g->S, pt.pos[0], pt.pos[1], pt.pos[2])
                                          : sample_int(img, g->S, pt.base[0], pt.base[1], pt.base[2]);
                        acc += cols[((c * g->Kn + t) * g->B + b) * g->Pn + p] * v;
                    }
                    grad_mask[((b * g->mg + mgi) * g->Kn + t) * g->Pn + p] = acc;
                }
}

/* ------------------------------------------------------------------------- */
/* the three contractions (the reference's addmm_ call sites)                 */
/* weight viewed as W[m][c_local][t] with shape (M, C/G, Kn) for both conv    */
/* (Cout, Cin/G, K) and transposed (Cin, Cout/G, K)                           */
/* ------------------------------------------------------------------------- */

/* Y[b][m][p] = sum_{c in group(m), t} W[m][c][t] * cols[c][t][b][p]
 * conv forward cpu/deform_conv2d_kernel.cpp:366-368, transposed backward grad_input
 * cpu/deform_conv_transpose2d_kernel.cpp:610-611 */
static void gemm_w_cols(const geo_t *g, const double *W, const double *cols, double *Y) {
    const int64_t Cg = g->C / g->G, Mg = g->M / g->G;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < g->B; ++b)
        for (int64_t m = 0; m < g->M; ++m) {
            const int64_t grp = m / Mg;
            double *y = Y + (b * g->M + m) * g->Pn;
            for (int64_t p = 0; p < g->Pn; ++p) y[p] = 0;
            for (int64_t cl = 0; cl < Cg; ++cl)
                for (int64_t t = 0; t < g->Kn; ++t) {
                    const double w = W[(m * Cg + cl) * g->Kn + t];
                    const double *col = cols + (((grp * Cg + cl) * g->Kn + t) * g->B + b) * g->Pn;
                    for (int64_t p = 0; p < g->Pn; ++p) y[p] += w * col[p];
                }
        }
}

/* cols[c][t][b][p] = sum_{m in group(c)} W[m][c][t] * Z[b][m][p]
 * conv backward grad-columns cpu/deform_conv2d_kernel.cpp:519-522, transposed forward
 * cpu/deform_conv_transpose2d_kernel.cpp:333-337 */
static void gemm_wt_z(const geo_t *g, const double *W, const double *Z, double *cols) {
    const int64_t Cg = g->C / g->G, Mg = g->M / g->G;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t c = 0; c < g->C; ++c)
        for (int64_t t = 0; t < g->Kn; ++t) {
            const int64_t grp = c / Cg, cl = c % Cg;
            for (int64_t b = 0; b < g->B; ++b) {
                double *col = cols + ((c * g->Kn + t) * g->B + b) * g->Pn;
                for (int64_t p = 0; p < g->Pn; ++p) col[p] = 0;
                for (int64_t ml = 0; ml < Mg; ++ml) {
                    const int64_t m = grp * Mg + ml;
                    const double w = W[(m * Cg + cl) * g->Kn + t];
                    const double *z = Z + (b * g->M + m) * g->Pn;
                    for (int64_t p = 0; p < g->Pn; ++p) col[p] += w * z[p];
                }
            }
        }
}

/* dW[m][c][t] = sum_{b,p} Z[b][m][p] * cols[c][t][b][p]
 * conv backward grad_weight cpu/deform_conv2d_kernel.cpp:624-626, transposed backward
 * cpu/deform_conv_transpose2d_kernel.cpp:612 */
static void gemm_z_colsT(const geo_t *g, const double *Z, const double *cols, double *dW) {
    const int64_t Cg = g->C / g->G, Mg = g->M / g->G;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < g->M; ++m)
        for (int64_t cl = 0; cl < Cg; ++cl) {
            const int64_t grp = m / Mg;
            for (int64_t t = 0; t < g->Kn; ++t) {
                double acc = 0;
                for (int64_t b = 0; b < g->B; ++b) {
                    const double *z = Z + (b * g->M + m) * g->Pn;
                    const double *col = cols + (((grp * Cg + cl) * g->Kn + t) * g->B + b) * g->Pn;
                    for (int64_t p = 0; p < g->Pn; ++p) acc += z[p] * col[p];
                }
                dW[(m * Cg + cl) * g->Kn + t] = acc;
            }
        }
}

static void add_bias(int64_t B, int64_t Cn, int64_t Sn, const double *bias, double *y) {
    if (!bias) return;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < Cn; ++c)
            for (int64_t s = 0; s < Sn; ++s) y[(b * Cn + c) * Sn + s] += bias[c];
}

/* ------------------------------------------------------------------------- */
/* public entry points                                                        */
/* ------------------------------------------------------------------------- */

/* conv: cpu/deform_conv2d_kernel.cpp:85-385 (im2col, GEMM, bias);
 * transposed: cpu/deform_conv_transpose2d_kernel.cpp:85-372 (GEMM, col2im into the
 * output, bias). */
void oracle_deform_conv_forward(const oracle_conv_desc *d, const double *input, const double *weight,
                                const double *offset, const double *mask, const double *bias, double *output) {
    geo_t g;
    make_geo(d, &g);
    double *cols = (double *) calloc((size_t) (g.C * g.Kn * g.B * g.Pn), sizeof(double));
    if (!d->transposed) {
        im2col(&g, input, offset, mask, cols);
        gemm_w_cols(&g, weight, cols, output);
        add_bias(g.B, g.M, g.Pn, bias, output);
    } else {
        gemm_wt_z(&g, weight, input, cols);
        memset(output, 0, sizeof(double) * (size_t) (g.B * g.C * g.Sn));
        col2im(&g, cols, offset, mask, output);
        add_bias(g.B, g.C, g.Sn, bias, output);
    }
    free(cols);
}

/* conv: cpu/deform_conv2d_kernel.cpp:387-642; transposed:
 * cpu/deform_conv_transpose2d_kernel.cpp:374-636. grad_bias = sum of grad_out
 * over batch and space (conv :415-417). */
void oracle_deform_conv_backward(const oracle_conv_desc *d, const double *grad_out, const double *input,
                                 const double *weight, const double *offset, const double *mask,
                                 double *grad_input, double *grad_weight, double *grad_offset, double *grad_mask,
                                 double *grad_bias) {
    geo_t g;
    make_geo(d, &g);
    const size_t ncols = (size_t) (g.C * g.Kn * g.B * g.Pn);
    double *cols = (double *) calloc(ncols, sizeof(double));
    /* Z: the tensor on the GEMM side (conv: grad_out, transposed: input);
     * src: the sampled tensor (conv: input, transposed: grad_out). */
    const double *Z = d->transposed ? input : grad_out;
    const double *src = d->transposed ? grad_out : input;
    gemm_wt_z(&g, weight, Z, cols);
    if (offset && grad_offset) grad_offset_kernel(&g, cols, src, offset, mask, grad_offset);
    if (mask && grad_mask) grad_mask_kernel(&g, cols, src, offset, grad_mask);
    if (!d->transposed) {
        memset(grad_input, 0, sizeof(double) * (size_t) (g.B * g.C * g.Sn));
        col2im(&g, cols, offset, mask, grad_input);
        im2col(&g, src, offset, mask, cols);
        gemm_z_colsT(&g, Z, cols, grad_weight);
    } else {
        im2col(&g, src, offset, mask, cols);
        gemm_w_cols(&g, weight, cols, grad_input);
        gemm_z_colsT(&g, Z, cols, grad_weight);
    }
    if (grad_bias) {
        const int64_t Cout = d->out_channels;
        int64_t out_sz[3];
        const int64_t So = oracle_output_size(d, out_sz);
        for (int64_t c = 0; c < Cout; ++c) {
            double acc = 0;
            for (int64_t b = 0; b < g.B; ++b)
                for (int64_t s = 0; s < So; ++s) acc += grad_out[(b * Cout + c) * So + s];
            grad_bias[c] = acc;
        }
    }
    free(cols);
}

/* ops/activations/mask_softmax.py:19-49 (and the 2D/3D twins): view
 * (B, mg, K, *S), torch.softmax over dim 2. Max-subtracted exponentials. */
void oracle_mask_softmax_forward(int64_t B, int64_t groups, int64_t K, int64_t S, const double *x, double *y) {
    for (int64_t bg = 0; bg < B * groups; ++bg)
        for (int64_t s = 0; s < S; ++s) {
            const double *xi = x + bg * K * S + s;
            double *yi = y + bg * K * S + s;
            double mx = -INFINITY;
            for (int64_t k = 0; k < K; ++k) mx = xi[k * S] > mx ? xi[k * S] : mx;
            double sum = 0;
            for (int64_t k = 0; k < K; ++k) sum += exp(xi[k * S] - mx);
            for (int64_t k = 0; k < K; ++k) yi[k * S] = exp(xi[k * S] - mx) / sum;
        }
}

/* softmax backward (autograd of torch.softmax): gx = y * (gy - sum_k gy_k y_k) */
void oracle_mask_softmax_backward(int64_t B, int64_t groups, int64_t K, int64_t S, const double *y,
                                  const double *gy, double *gx) {
    for (int64_t bg = 0; bg < B * groups; ++bg)
        for (int64_t s = 0; s < S; ++s) {
            const int64_t o = bg * K * S + s;
            double dot = 0;
            for (int64_t k = 0; k < K; ++k) dot += gy[o + k * S] * y[o + k * S];
            for (int64_t k = 0; k < K; ++k) gx[o + k * S] = y[o + k * S] * (gy[o + k * S] - dot);
        }
}
