// C ABI of libtvdcn_hip.so (declared in include/tvdcn_hip.h).
//
// Validates a descriptor with the reference's shape rules, lays out the
// caller-provided workspace, and enqueues the kernel sequence of each op on the
// caller's stream. Host-side only: no allocation, no synchronisation.
#include <string>
#include <cstring>
#include <climits>
#include <cmath>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <numeric>
#include <initializer_list>
#include <vector>

#include "../../../include/tvdcn_hip.h"
#include "kernels.h"

using namespace tvdcn_hip;

namespace {

thread_local std::string g_last_error;

tvdcn_status fail(tvdcn_status st, const std::string &msg) {
    g_last_error = msg;
    return st;
}

size_t acc_size(int dtype) { return dtype == TVDCN_DTYPE_FLOAT64 ? 8 : 4; }
size_t elem_size(int dtype) {
    switch (dtype) {
        case TVDCN_DTYPE_FLOAT32: return 4;
        case TVDCN_DTYPE_FLOAT64: return 8;
        default: return 2;
    }
}
bool acc_is_storage(int dtype) { return dtype == TVDCN_DTYPE_FLOAT32 || dtype == TVDCN_DTYPE_FLOAT64; }

size_t align_up(size_t v) { return (v + 255) / 256 * 256; }

// Output size: conv per ops/cuda/deform_conv2d_kernel.cpp:167-168, transposed per
// ops/cuda/deform_conv_transpose2d_kernel.cpp:172-173 (1D/3D files identical in form).
tvdcn_status output_size(const tvdcn_conv_desc *d, int64_t out[3]) {
    if (d == nullptr) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "null descriptor");
    if (d->dim < 1 || d->dim > 3) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "dim must be 1, 2 or 3");
    for (int i = 0; i < d->dim; ++i) {
        if (d->kernel[i] <= 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "kernel size must be positive");
        if (d->stride[i] <= 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "stride must be positive");
        if (d->padding[i] < 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "padding must be non-negative");
        if (d->dilation[i] <= 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "dilation must be positive");
        if (d->transposed)
            out[i] = (d->in_size[i] - 1) * d->stride[i] - 2 * d->padding[i] + d->dilation[i] * (d->kernel[i] - 1) + 1 +
                     d->output_padding[i];
        else
            out[i] = (d->in_size[i] + 2 * d->padding[i] - (d->dilation[i] * (d->kernel[i] - 1) + 1)) / d->stride[i] + 1;
        if (out[i] <= 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "Calculated output size too small");
    }
    return TVDCN_STATUS_SUCCESS;
}

struct Plan {
    Geo g;
    int64_t out_size[3];
    int dim;
    bool transposed;
    int dtype;
    FwdTiles ft;
    DataTiles dt;
    WinTiles wn_s;   // windowed data-gradient plan, scatter + offset/mask gradients (conv backward)
    WinTiles wn_x;   // the same tiling, scatter only (transposed forward): a larger window
    WinTiles wn_c;   // the same tiling, offset/mask gradients only (transposed backward)
    WinTiles wn_xg;  // 3D conv backward: one launch on the scatter window, X read from global memory
    bool data_split; // conv backward: scatter (wn_x) and offset/mask gradients (wn_c) as two
                     // launches, when the shared window of wn_s would be too small
    WeightTiles wt;
    WinTiles wn_w;   // the wn_s tiling with the weight-gradient kernel's window margin (fp32 loop)
    WinTiles wn_w16; // ... and with its 16-bit loop's (a smaller S tile leaves a larger window)
    WinTiles wn_f;   // the wn_s tiling with the forward kernel's window margin
    WeightWin ww;    // windowed weight-gradient plan (over wn_w)
    FwdWin fw;       // windowed forward plan (over wn_f)
    // conv backward: grad_input accumulated in the caller's tensor, no channels-last accumulator
    // (a channels-last input of the accumulation type, or float32 on the windowed data gradient,
    // whose window flush and atomics address the (B, C, *S) tensor directly)
    bool gx_in_place;
    bool gx_nchw;    // ... and that tensor is (B, C, *S)
};

bool fits_int(int64_t v) { return v >= 0 && v <= (int64_t)INT_MAX; }

// Plan of one batch block of `batch` images (the descriptor's other fields as given).
tvdcn_status make_plan(const tvdcn_conv_desc *d, Plan &pl, int64_t batch) {
    tvdcn_status st = output_size(d, pl.out_size);
    if (st) return st;
    if (d->dtype < 0 || d->dtype > 3) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "unknown dtype");
    if (d->batch < 0 || d->in_channels <= 0 || d->out_channels <= 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "batch must be >= 0 and channels positive");
    if (d->groups <= 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "groups must be positive");
    if (d->flags & ~(TVDCN_FLAG_CHANNELS_LAST | TVDCN_FLAG_MASK_SIGMOID | TVDCN_FLAG_MASK_SOFTMAX))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "unknown flags");
    if ((d->flags & TVDCN_FLAG_MASK_SIGMOID) && (d->flags & TVDCN_FLAG_MASK_SOFTMAX))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "TVDCN_FLAG_MASK_SIGMOID and TVDCN_FLAG_MASK_SOFTMAX exclude each other");
    if ((d->flags & TVDCN_FLAG_MASK_SIGMOID) && (d->mask_groups == 0 || !(d->mask_scale > 0.0) ||
                                                 !(d->mask_scale < 1e300)))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "a sigmoid mask needs a mask and a positive finite mask_scale");
    if ((d->flags & TVDCN_FLAG_MASK_SOFTMAX) && d->mask_groups == 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "a softmax mask needs a mask");
    if ((d->flags & TVDCN_FLAG_CHANNELS_LAST) && d->transposed)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "channels-last input is supported for the non-transposed ops");
    if (d->in_channels % d->groups || d->out_channels % d->groups)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "in_channels and out_channels must be divisible by groups");
    if (d->offset_groups < 0 || d->mask_groups < 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "offset_groups / mask_groups must be >= 0");
    // Groups of offsets/masks partition the channels of the sampled side (columns).
    // The reference checks input.size(1) % groups (deform_conv2d_kernel.cpp:205, 233;
    // transposed :216, :247); for the transposed op the columns are the output
    // channels, so they must divide those too (the reference indexes past the
    // offset tensor otherwise).
    const int64_t C = d->transposed ? d->out_channels : d->in_channels;
    const int64_t M = d->transposed ? d->in_channels : d->out_channels;
    if (d->offset_groups && (d->in_channels % d->offset_groups || C % d->offset_groups))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "channels must be divisible by offset_groups");
    if (d->mask_groups && (d->in_channels % d->mask_groups || C % d->mask_groups))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "channels must be divisible by mask_groups");

    pl.dim = d->dim;
    pl.transposed = d->transposed != 0;
    pl.dtype = d->dtype;
    Geo &g = pl.g;
    int64_t S3[3] = {1, 1, 1}, P3[3] = {1, 1, 1}, K3[3] = {1, 1, 1}, st3[3] = {1, 1, 1}, pd3[3] = {0, 0, 0},
            dl3[3] = {1, 1, 1};
    for (int i = 0; i < d->dim; ++i) {
        const int e = 3 - d->dim + i;
        S3[e] = pl.transposed ? pl.out_size[i] : d->in_size[i];
        P3[e] = pl.transposed ? d->in_size[i] : pl.out_size[i];
        K3[e] = d->kernel[i];
        st3[e] = d->stride[i];
        pd3[e] = d->padding[i];
        dl3[e] = d->dilation[i];
    }
    const int64_t Sn = S3[0] * S3[1] * S3[2], Pn = P3[0] * P3[1] * P3[2], Kn = K3[0] * K3[1] * K3[2];
    const int64_t B = batch;
    // int32 indexing inside the kernels: every tensor of the block must stay below 2^31 elements
    const int64_t biggest[] = {B * C * Sn, B * M * Pn, M * (C / d->groups) * Kn,
                               B * (d->offset_groups ? d->offset_groups : 1) * Kn * d->dim * Pn,
                               B * (d->mask_groups ? d->mask_groups : 1) * Kn * Pn};
    for (int64_t v : biggest)
        if (!fits_int(v)) return fail(TVDCN_STATUS_NOT_SUPPORTED, "tensor too large for 32-bit indexing");
    for (int i = 0; i < 3; ++i) {
        g.S[i] = (int)S3[i];
        g.P[i] = (int)P3[i];
        g.K[i] = (int)K3[i];
        g.st[i] = (int)st3[i];
        g.pad[i] = (int)pd3[i];
        g.dil[i] = (int)dl3[i];
    }
    g.B = (int)B;
    g.C = (int)C;
    g.M = (int)M;
    g.G = (int)d->groups;
    g.Cg = (int)(C / d->groups);
    g.Mg = (int)(M / d->groups);
    g.og = (int)d->offset_groups;
    g.mg = (int)d->mask_groups;
    g.cpo = g.og ? g.C / g.og : 1;
    g.cpm = g.mg ? g.C / g.mg : 1;
    g.Sn = (int)Sn;
    g.Pn = (int)Pn;
    g.Kn = (int)Kn;
    g.NP = (int)(B * Pn);
    g.mask_act = (d->flags & TVDCN_FLAG_MASK_SIGMOID) ? MASK_ACT_SIGMOID
                 : (d->flags & TVDCN_FLAG_MASK_SOFTMAX) ? MASK_ACT_SOFTMAX
                                                         : 0;
    g.mask_scale = (d->flags & TVDCN_FLAG_MASK_SIGMOID) ? d->mask_scale : 0.0;
    g.dPn = make_fastdiv((uint32_t)g.Pn);
    g.dP2 = make_fastdiv((uint32_t)g.P[2]);
    g.dP12 = make_fastdiv((uint32_t)(g.P[1] * g.P[2]));
    g.dK2 = make_fastdiv((uint32_t)g.K[2]);
    g.dK12 = make_fastdiv((uint32_t)(g.K[1] * g.K[2]));
    pl.ft = plan_fwd(g, pl.dtype);
    pl.dt = plan_data(g, pl.dtype);
    pl.wn_s = plan_data_win(g, pl.dtype, pl.dim, true, true);
    pl.wn_x = plan_data_win(g, pl.dtype, pl.dim, true, false);
    pl.wn_c = plan_data_win(g, pl.dtype, pl.dim, false, true);
    // the launches use all three sizes of the windowed plan (and the operand layouts prepared for
    // wn_s): one without a window disables them all
    if (!pl.wn_s.ok || !pl.wn_x.ok || !pl.wn_c.ok) pl.wn_s.ok = pl.wn_x.ok = pl.wn_c.ok = false;
    // a margin under 2 cells loses a large share of the corners to global atomics
    // (3D: the window grows with the cube of its extent); two launches recompute the
    // grad-columns contraction but each gets about twice the window
    pl.data_split = pl.wn_s.ok && pl.wn_s.R[2] < 2 && pl.wn_x.R[2] > pl.wn_s.R[2] && pl.wn_c.R[2] > pl.wn_s.R[2];
    pl.wn_xg = pl.wn_x;
    pl.wn_xg.xglobal = 1;
    pl.wt = plan_weight(g, pl.dtype);
    pl.wn_w = win_resize(pl.wn_s, g, pl.dim, weight_win_fixed_bytes(g, pl.dim, pl.wn_s.tpp, 0), x_window_cell_bytes());
    // (only where the fp32 loop's window keeps a margin under 4 cells on some axis: a margin of 4
    // already holds nearly every corner, and a larger window costs its fill -- cfg2 weight gradient
    // +5% at margin 8 against 6, cfg5 fp16 -25% at margin 1 against -2)
    pl.wn_w16 = pl.wn_w;
    bool small_margin = false;
    for (int e = 3 - pl.dim; e < 3; ++e) small_margin = small_margin || pl.wn_w.R[e] < 4;
    if (small_margin)
        pl.wn_w16 = win_resize(pl.wn_s, g, pl.dim,
                               weight_win_fixed_bytes(g, pl.dim, pl.wn_s.tpp, pl.dtype == kF32 ? 2 : 1),
                               x_window_cell_bytes());
    pl.ww = plan_weight_win(g, pl.wn_w, pl.dim);
    pl.fw = plan_fwd_win(g, pl.wn_s, pl.dim, pl.wn_f);
    const bool cl_in = (d->flags & TVDCN_FLAG_CHANNELS_LAST) != 0;
    // (1D only: there a window row is the tile's 256 pixels + margins, whole lines of each channel;
    // 2D / 3D window rows are 10-26 cells, and the flush and out-of-window corners then reach
    // 2-4x the memory transactions per wave instruction of the 16-channel cells of the
    // channels-last order -- cfg2 data gradient +8%, cfg4 +86%)
    pl.gx_nchw = !pl.transposed && !cl_in && pl.dtype == kF32 && pl.wn_s.ok && pl.dim == 1;
    pl.gx_in_place = !pl.transposed && ((cl_in && acc_is_storage(pl.dtype)) || pl.gx_nchw);
    return TVDCN_STATUS_SUCCESS;
}

// ---------------------------------------------------------------------------
// Batch blocks. The kernels index in 32 bits, so the entry points run the batch in blocks of
// images whose batch-sized tensors and workspace buffers stay at or below g_block_limit
// elements (2^31 - 1 unless tvdcn_set_max_block_elements lowers it); the weight gradient is
// accumulated across blocks. The reference blocks its batch too, by n_parallel_imgs
// (cuda/deform_conv2d_kernel.cpp:149, utils/parallel_helpers.h:7-16), for its columns buffer.
// ---------------------------------------------------------------------------
std::atomic<int64_t> g_block_limit{INT_MAX};

int64_t mul_sat(int64_t a, int64_t b) {   // a * b for a, b >= 0, saturating at INT64_MAX
    if (a == 0 || b == 0) return 0;
    return a > INT64_MAX / b ? INT64_MAX : a * b;
}

// per-image element counts of the user tensors: input, output, offset, mask
struct ImageElems {
    int64_t in = 1, out = 1, offset = 0, mask = 0;
    int64_t largest() const { return std::max(std::max(in, out), std::max(offset, mask)); }
};

ImageElems image_elems(const tvdcn_conv_desc *d, const int64_t out_size[3]) {
    ImageElems e;
    int64_t si = 1, so = 1, kn = 1;
    for (int i = 0; i < d->dim; ++i) {
        si = mul_sat(si, d->in_size[i]);
        so = mul_sat(so, out_size[i]);
        kn = mul_sat(kn, d->kernel[i]);
    }
    const int64_t grid = d->transposed ? si : so;   // offsets / masks live on the column grid
    e.in = mul_sat(d->in_channels, si);
    e.out = mul_sat(d->out_channels, so);
    e.offset = mul_sat(mul_sat(d->offset_groups, mul_sat(kn, d->dim)), grid);
    e.mask = mul_sat(mul_sat(d->mask_groups, kn), grid);
    return e;
}

// images per block (>= 1 for a non-empty batch): every buffer of the kernels is as large as
// one of the user tensors or batch-independent, so the user tensors' per-image sizes decide
tvdcn_status batch_block(const tvdcn_conv_desc *d, int64_t &block, ImageElems *elems = nullptr) {
    int64_t out[3] = {1, 1, 1};
    tvdcn_status st = output_size(d, out);
    if (st) return st;
    if (d->batch < 0) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "batch must be >= 0 and channels positive");
    const ImageElems e = image_elems(d, out);
    if (elems) *elems = e;
    const int64_t lim = g_block_limit.load();
    if (e.largest() > lim)
        return fail(TVDCN_STATUS_NOT_SUPPORTED, "one image's tensors exceed " + std::to_string(lim) +
                                                    " elements (the kernels index in 32 bits)");
    block = d->batch == 0 ? 0 : std::max<int64_t>(1, std::min<int64_t>(d->batch, lim / std::max<int64_t>(e.largest(), 1)));
    if (block < d->batch) {
        // a block of m images spans a multiple of 16 bytes of every user tensor, so a block that
        // is a multiple of m keeps every block's pointers as aligned as the caller's (the layout
        // copies then take their 16-byte paths); a block below m leaves them less aligned, which
        // the kernels accept (they need 16-byte alignment only of what stays aligned anyway: a
        // channels-last input with channels % 4 == 0, rows of 4-element quads)
        const int64_t es = (int64_t)elem_size(d->dtype);
        int64_t m = 1;
        for (const int64_t n : {e.in, e.out, e.offset, e.mask}) {
            const int64_t bytes = n * es % 16;
            if (bytes != 0) m = std::max<int64_t>(m, 16 / std::gcd<int64_t>(bytes, 16));
        }
        if (block >= m) block -= block % m;
    }
    return TVDCN_STATUS_SUCCESS;
}

// Workspace sub-buffers (byte offsets into the caller's workspace).
struct Layout {
    size_t xcl = 0, wf = 0, wd = 0, cl_acc = 0, wpart = 0, goff_acc = 0, gmask_acc = 0, yacc = 0;
    size_t zs = 0, wsplit = 0;   // the windowed data gradient's 16-bit MFMA operands
    size_t zw = 0;               // Z's 16-bit values in column blocks, for the weight gradient's 16-bit loop
    size_t w16 = 0;              // the windowed forward's 16-bit weight
    size_t flag = 0;             // operand flag: some fp32 operand too large or not finite for them
    size_t total = 0;
};

Layout layout(const Plan &pl, bool backward) {
    const Geo &g = pl.g;
    const size_t a = acc_size(pl.dtype);
    const size_t cl_bytes = align_up((size_t)g.B * g.Sn * g.C * a);
    // forward weight layout Wf[G][Kn][Mg_pad][Cg_pad], padded for whichever forward kernel runs
    const size_t wf_bytes = pl.fw.ok ? align_up((size_t)g.G * g.Kn * pl.fw.Mg_pad * pl.fw.Cg_pad * sizeof(float))
                                     : align_up((size_t)g.G * g.Kn * pl.ft.Mg_pad * pl.ft.Cg_pad * a);
    // data-gradient weight: windowed-kernel chunks when eligible, else the [G][Kn][Cg][Mg] layout
    const size_t wd_bytes = pl.wn_s.ok ? align_up(pl.wn_s.chunk_elems * sizeof(float))
                                       : align_up((size_t)g.G * g.Kn * pl.dt.Mg_pad * pl.dt.Cg_pad * a);
    Layout L;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += bytes;
        return o;
    };
    const size_t SENTINEL = (size_t)-1;
    L.xcl = L.wf = L.wd = L.cl_acc = L.wpart = L.goff_acc = L.gmask_acc = L.yacc = SENTINEL;
    L.zs = L.wsplit = L.w16 = L.flag = L.zw = SENTINEL;
    L.flag = take(align_up(sizeof(int) * OPERAND_FLAG_WORDS));   // the flag and the operands' largest magnitudes
    // windowed data gradient (conv backward, transposed forward and backward): split operands
    auto take_split = [&]() {
        if (!pl.wn_s.ok) return;
        L.zs = take(align_up(pl.wn_s.zs_elems * 2));
        L.wsplit = take(align_up(pl.wn_s.ws_elems * 2));
    };
    // windowed forward (conv forward, transposed backward's input gradient)
    auto take_w16 = [&]() {
        if (pl.fw.ok && pl.fw.w16_elems) L.w16 = take(align_up(pl.fw.w16_elems * 2));
    };
    // fp32 output of a slice-split windowed forward when the output dtype is not fp32
    const bool split_acc = pl.fw.ok && pl.fw.ksplit > 1 && pl.dtype != kF32;
    const size_t yacc_bytes = align_up((size_t)g.B * g.M * g.Pn * sizeof(float));
    if (!backward) {
        if (!pl.transposed) {
            L.xcl = take(cl_bytes);
            L.wf = take(wf_bytes);
            take_w16();
            if (split_acc) L.yacc = take(yacc_bytes);
        } else {
            L.wd = take(wd_bytes);
            L.cl_acc = take(cl_bytes);
            take_split();
        }
    } else {
        L.xcl = take(cl_bytes);
        L.wd = take(wd_bytes);
        take_split();
        // written beside the data gradient's split of Z (same launch), read by the weight gradient
        if ((pl.dtype == kF32 || pl.dtype == kF16 || pl.dtype == kBF16) && pl.wn_s.ok && pl.ww.ok && pl.ww.z8)
            L.zw = take(align_up((size_t)g.B * g.M * g.Pn * (pl.dtype == kF32 ? 2 : 1) * sizeof(uint16_t)));
        if (pl.transposed) {
            L.wf = take(wf_bytes);
            take_w16();
            if (split_acc) L.yacc = take(yacc_bytes);
        } else if (!pl.gx_in_place)
            L.cl_acc = take(cl_bytes);
        L.wpart = take(align_up(pl.ww.ok ? pl.ww.part_elems * sizeof(float) : pl.wt.part_elems * a));
        if (!acc_is_storage(pl.dtype)) {
            if (g.og) L.goff_acc = take(align_up((size_t)g.B * g.og * g.Kn * pl.dim * g.Pn * a));
            if (g.mg) L.gmask_acc = take(align_up((size_t)g.B * g.mg * g.Kn * g.Pn * a));
        }
    }
    L.total = off;
    return L;
}

void *at(void *ws, size_t off) { return off == (size_t)-1 ? nullptr : static_cast<char *>(ws) + off; }

#define TVDCN_CHECK_HIP(expr)                                                                     \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return fail(TVDCN_STATUS_HIP_ERROR, std::string(#expr " failed: ") + hipGetErrorString(e_)); \
    } while (0)

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// the caller's tensor pointers (null: absent) are 16-byte aligned
tvdcn_status check_aligned(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (p && !aligned16(p)) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
    return TVDCN_STATUS_SUCCESS;
}

// ---------------------------------------------------------------------------
// Optional per-kernel timing: HIP events recorded on the launch stream around
// each kernel family (off by default; see tvdcn_kernel_timer_enable).
// ---------------------------------------------------------------------------
struct KernelTimer {
    std::mutex mu;
    bool enabled = false;
    struct Rec {
        int family;
        hipEvent_t start, stop;
    };
    std::vector<Rec> pending;
    std::vector<hipEvent_t> pool;
    double total_ms[TVDCN_KERNEL_FAMILIES] = {};
    int64_t count[TVDCN_KERNEL_FAMILIES] = {};

    hipEvent_t get_event() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    void drain() {
        for (auto &r : pending) {
            float ms = 0.f;
            if (hipEventSynchronize(r.stop) == hipSuccess && hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
                total_ms[r.family] += ms;
                count[r.family] += 1;
            }
            pool.push_back(r.start);
            pool.push_back(r.stop);
        }
        pending.clear();
    }
};

KernelTimer &timer() {
    static KernelTimer t;
    return t;
}

struct TimedScope {
    int family;
    hipStream_t stream;
    hipEvent_t start = nullptr;
    TimedScope(int fam, hipStream_t s) : family(fam), stream(s) {
        KernelTimer &t = timer();
        std::lock_guard<std::mutex> lk(t.mu);
        if (!t.enabled) return;
        start = t.get_event();
        if (start && hipEventRecord(start, stream) != hipSuccess) start = nullptr;
    }
    ~TimedScope() {
        if (!start) return;
        KernelTimer &t = timer();
        std::lock_guard<std::mutex> lk(t.mu);
        hipEvent_t stop = t.get_event();
        if (stop && hipEventRecord(stop, stream) == hipSuccess)
            t.pending.push_back({family, start, stop});
        else
            t.pool.push_back(start);
    }
};

#define TVDCN_LAUNCH(fam, stream, expr)     \
    do {                                    \
        TimedScope ts_((fam), (stream));    \
        TVDCN_CHECK_HIP(expr);              \
    } while (0)

tvdcn_status layout_copy(bool to_cl, int32_t dtype, int64_t batch, int64_t channels, int64_t spatial_numel,
                         const void *input, void *output, void *stream) {
    const char *what = to_cl ? "to_channels_last" : "from_channels_last";
    if (dtype != TVDCN_DTYPE_FLOAT32) return fail(TVDCN_STATUS_NOT_SUPPORTED, std::string(what) + ": float32 only");
    if (batch < 0 || channels < 0 || spatial_numel < 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, std::string(what) + ": negative size");
    if (!fits_int(batch) || !fits_int(channels) || !fits_int(spatial_numel) ||
        (double)batch * (double)channels * (double)spatial_numel > (double)INT_MAX)
        return fail(TVDCN_STATUS_NOT_SUPPORTED, std::string(what) + ": tensor too large for 32-bit indexing");
    g_last_error.clear();
    if (batch == 0 || channels == 0 || spatial_numel == 0) return TVDCN_STATUS_SUCCESS;
    if (input == nullptr || output == nullptr)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, std::string(what) + ": null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int B = (int)batch, C = (int)channels, Sn = (int)spatial_numel;
    if (to_cl)
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_to_channels_last(kF32, input, output, B, C, Sn, s));
    else
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_from_channels_last(kF32, input, output, nullptr, B, C, Sn, s));
    return TVDCN_STATUS_SUCCESS;
}

tvdcn_status check_forward_pointers(const tvdcn_conv_desc *desc, const void *offset, const void *mask) {
    if ((desc->offset_groups == 0) != (offset == nullptr))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "offset pointer and offset_groups disagree");
    if ((desc->mask_groups == 0) != (mask == nullptr))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "mask pointer and mask_groups disagree");
    return TVDCN_STATUS_SUCCESS;
}

// Forward on a validated plan (batch > 0, pointers checked) with a workspace of at least layout(pl, false).total
// bytes; shared by tvdcn_deform_conv_forward (caller's workspace) and
// tvdcn_deform_conv_forward_noalloc (the per-device scratch array). Every workspace byte the
// kernels read is written first in the same call (the zero-filled accumulator by a fill kernel),
// so the workspace may hold anything on entry.
// The sampled side of the 16-bit forward loop: mask * bilinear(X) in scaled fp16 pieces (fp32) needs
// |X| < SAMPLED_LIMIT and |mask| < MASK_LIMIT (checked on the device into *flag: the product and its
// scale stay in the float range); a sigmoid mask activation bounds the mask by its scale, a softmax
// by 1.
bool sampled16_host_ok(const Plan &pl, const tvdcn_conv_desc *desc) {
    if (pl.dtype != kF32) return true;
    if (desc->flags & TVDCN_FLAG_MASK_SIGMOID) return std::fabs(desc->mask_scale) < (double)MASK_LIMIT;
    return true;
}
// the mask when its values feed the 16-bit loops unbounded (fp32, no activation), else null
const void *mask_to_check(const Plan &pl, const tvdcn_conv_desc *desc, const void *mask) {
    if (pl.dtype != kF32 || mask == nullptr || (desc->flags & (TVDCN_FLAG_MASK_SIGMOID | TVDCN_FLAG_MASK_SOFTMAX)))
        return nullptr;
    return mask;
}
size_t mask_numel(const Geo &g) { return (size_t)g.B * g.mg * g.Kn * g.Pn; }

// float32: the largest magnitudes of the 16-bit MFMA operands (their pieces' scales) -- the weight,
// the sampled tensor X, a mask given as values (an activated mask's bound is known), the GEMM-side
// tensor Z -- into the words after the zeroed operand flag (null pointers: not needed)
hipError_t operand_amax(const Plan &pl, const tvdcn_conv_desc *desc, const void *weight, const void *x,
                        const void *mask, const void *z, int *flag, hipStream_t s) {
    const Geo &g = pl.g;
    if (pl.dtype != kF32) return hipSuccess;
    const bool plain_mask = !(desc->flags & (TVDCN_FLAG_MASK_SIGMOID | TVDCN_FLAG_MASK_SOFTMAX));
    const AmaxItem items[4] = {
        {static_cast<const float *>(weight), (size_t)g.M * g.Cg * g.Kn, AMAX_SLOT_W},
        {static_cast<const float *>(x), (size_t)g.B * g.C * g.Sn, AMAX_SLOT_X},
        {plain_mask ? static_cast<const float *>(mask) : nullptr, mask_numel(g), AMAX_SLOT_M},
        {static_cast<const float *>(z), (size_t)g.B * g.M * g.Pn, AMAX_SLOT_Z}};
    return launch_amax(items, 4, flag, s);
}

hipError_t check_sampled(const Plan &pl, const tvdcn_conv_desc *desc, const void *x_in_place, const void *mask,
                         int *flag, hipStream_t s) {
    const Geo &g = pl.g;
    if (pl.dtype != kF32) return hipSuccess;
    if (x_in_place != nullptr) {
        const hipError_t e = launch_check_range(x_in_place, (size_t)g.B * g.Sn * g.C, SAMPLED_LIMIT, flag, s);
        if (e != hipSuccess) return e;
    }
    if (mask != nullptr && !(desc->flags & (TVDCN_FLAG_MASK_SIGMOID | TVDCN_FLAG_MASK_SOFTMAX)))
        return launch_check_range(mask, (size_t)g.B * g.mg * g.Kn * g.Pn, MASK_LIMIT, flag, s);
    return hipSuccess;
}

tvdcn_status forward_planned(const Plan &pl, const tvdcn_conv_desc *desc, const void *input, const void *weight,
                             const void *offset, const void *mask, const void *bias, void *output, void *workspace,
                             void *stream) {
    const Geo &g = pl.g;
    const Layout L = layout(pl, false);
    if (!input || !weight || !output) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "null tensor pointer");
    // (the caller's pointers are checked at the entry; a later block's may be less aligned)
    if (!aligned16(workspace)) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int dt = pl.dtype;
    g_last_error.clear();
    int *flag = static_cast<int *>(at(workspace, L.flag));
    if (!pl.transposed) {
        void *xcl = at(workspace, L.xcl), *wf = at(workspace, L.wf);
        void *w16 = pl.fw.ok && sampled16_host_ok(pl, desc) ? at(workspace, L.w16) : nullptr;
        // the flag and (split channel slices) the fp32 accumulator zeroed by one launch
        void *y32 = pl.fw.ok && pl.fw.ksplit > 1 ? (dt == kF32 ? output : at(workspace, L.yacc)) : nullptr;
        const FillItem fills[2] = {{flag, 4 * OPERAND_FLAG_WORDS}, {y32, y32 ? (size_t)g.B * g.M * g.Pn * 4 : 0}};
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fill_zero_multi(fills, 2, s));
        const void *x_in_place = nullptr;
        // the 16-bit loop's mask range check and (fp32) its operands' largest magnitudes ride on the
        // input's layout copy when there is one
        const void *mchk = w16 != nullptr ? mask_to_check(pl, desc, mask) : nullptr;
        if (!(desc->flags & TVDCN_FLAG_CHANNELS_LAST)) {
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_to_channels_last(dt, input, xcl, g.B, g.C, g.Sn, s, flag, mchk,
                                                                         mask_numel(g), MASK_LIMIT,
                                                                         w16 != nullptr ? weight : nullptr,
                                                                         (size_t)g.M * g.Cg * g.Kn));
        } else {
            if (acc_is_storage(dt))
                x_in_place = xcl = const_cast<void *>(input);   // already the kernels' layout and type
            else
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_storage_to_acc(dt, input, xcl, (size_t)g.B * g.Sn * g.C, s));
            if (w16 != nullptr)
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, operand_amax(pl, desc, weight, input, mask, nullptr, flag, s));
        }
        if (pl.fw.ok) {
            if (w16 != nullptr) {
                // both weight layouts (16-bit pieces and the fp32 loop's) in one launch
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fwd_win_layout16(dt, g, pl.fw, weight, w16, flag, s, wf));
                if (desc->flags & TVDCN_FLAG_CHANNELS_LAST)
                    TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, check_sampled(pl, desc, x_in_place, mask, flag, s));
            } else {
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fwd_win_layout(dt, g, pl.fw, weight, wf, s));
            }
            TVDCN_LAUNCH(TVDCN_KERNEL_GATHER_GEMM, s,
                         launch_fwd_win(dt, pl.dim, g, pl.wn_f, pl.fw, xcl, wf, w16, flag, offset, mask, bias, output,
                                        y32, s));
            if (pl.fw.ksplit > 1 && dt != kF32)
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_acc_to_storage(dt, y32, output, (size_t)g.B * g.M * g.Pn, s));
        } else {
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_weight_fwd_layout(dt, g, weight, wf, pl.ft.Mg_pad, pl.ft.Cg_pad, s));
            TVDCN_LAUNCH(TVDCN_KERNEL_GATHER_GEMM, s,
                         launch_fwd_gather_gemm(dt, pl.dim, g, pl.ft, xcl, wf, offset, mask, bias, output, s));
        }
    } else {
        void *wd = at(workspace, L.wd), *ycl = at(workspace, L.cl_acc);
        const FillItem fills[2] = {{flag, 4 * OPERAND_FLAG_WORDS}, {ycl, (size_t)g.B * g.Sn * g.C * acc_size(dt)}};
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fill_zero_multi(fills, 2, s));
        if (pl.wn_s.ok) {
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, operand_amax(pl, desc, weight, nullptr, nullptr, input, flag, s));
            void *zs = at(workspace, L.zs), *wsp = at(workspace, L.wsplit);
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_data_win_prep(dt, g, pl.wn_s, input, weight, zs, wsp, wd, flag, s));
            TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, pl.wn_x, true, false, input, wd, zs,
                                                                        wsp, flag, nullptr, offset, mask, ycl, nullptr,
                                                                        nullptr, s));
        } else {
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_weight_data_layout(dt, g, weight, wd, pl.dt.Mg_pad, pl.dt.Cg_pad, s));
            TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data(dt, pl.dim, g, pl.dt, true, false, input, wd, nullptr, offset,
                                                                    mask, ycl, nullptr, nullptr, s));
        }
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_from_channels_last(dt, ycl, output, bias, g.B, g.C, g.Sn, s));
    }
    return TVDCN_STATUS_SUCCESS;
}

// Backward of one batch block on its plan (pointers at the block's first image), except the
// bias gradient; the weight gradient is written (first block) or added (accumulate_weight).
tvdcn_status backward_planned(const Plan &pl, const tvdcn_conv_desc *desc, const void *grad_out, const void *input,
                              const void *weight, const void *offset, const void *mask, void *grad_input,
                              void *grad_weight, void *grad_offset, void *grad_mask, void *grad_bias, void *workspace,
                              void *stream, bool accumulate_weight) {
    const Geo &g = pl.g;
    const Layout L = layout(pl, true);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int dt = pl.dtype;
    const int ab = (int)acc_size(dt);
    const bool direct = acc_is_storage(dt);

    const size_t n_goff = g.og ? (size_t)g.B * g.og * g.Kn * pl.dim * g.Pn : 0;
    const size_t n_gmask = g.mg ? (size_t)g.B * g.mg * g.Kn * g.Pn : 0;
    void *goff = direct ? grad_offset : at(workspace, L.goff_acc);
    void *gmask = direct ? grad_mask : at(workspace, L.gmask_acc);

    // Z: the GEMM-side tensor (conv: grad_out; transposed: input)
    // X: the sampled tensor (conv: input; transposed: grad_out)
    const void *Z = pl.transposed ? input : grad_out;
    const void *X = pl.transposed ? grad_out : input;
    {
        void *xcl = at(workspace, L.xcl), *wd = at(workspace, L.wd);
        int *flag = static_cast<int *>(at(workspace, L.flag));
        const bool cl_in = (desc->flags & TVDCN_FLAG_CHANNELS_LAST) != 0;   // conv only
        // conv: grad_input accumulated in place (channels-last of the accumulation type, or the
        // float32 (B, C, *S) tensor on the windowed data gradient), else a channels-last accumulator
        void *gx_cl = pl.transposed ? nullptr : pl.gx_in_place ? grad_input : at(workspace, L.cl_acc);
        // transposed, input gradient on the split forward plan: its fp32 accumulator
        void *y32 = pl.transposed && pl.fw.ok && pl.fw.ksplit > 1 ? (dt == kF32 ? grad_input : at(workspace, L.yacc))
                                                                   : nullptr;
        // the offset / mask gradient accumulators, the operand flag, grad_input (conv) or the split
        // accumulator (transposed) zeroed by one launch
        const FillItem fills[5] = {{goff, goff ? n_goff * ab : 0},
                                   {gmask, gmask ? n_gmask * ab : 0},
                                   {flag, 4 * OPERAND_FLAG_WORDS},
                                   {gx_cl, gx_cl ? (size_t)g.B * g.Sn * g.C * ab : 0},
                                   {y32, y32 ? (size_t)g.B * g.M * g.Pn * 4 : 0}};
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fill_zero_multi(fills, 5, s));
        const bool coord = offset != nullptr || mask != nullptr;
        // the 16-bit loops of the sampled side (weight gradient; transposed: input gradient)
        const bool sampled16 = sampled16_host_ok(pl, desc) && (pl.ww.ok || (pl.transposed && pl.fw.ok));
        const void *x_in_place = nullptr;
        // (fp32) the 16-bit MFMA operands' largest magnitudes: the weight and X ride on X's layout
        // copy, Z = grad_out on the bias gradient (this block's, accumulated over the blocks),
        // whatever else on a launch of its own
        if (!cl_in) {
            // the mask's range check rides on the layout copy
            const void *mchk = sampled16 ? mask_to_check(pl, desc, mask) : nullptr;
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_to_channels_last(dt, X, xcl, g.B, g.C, g.Sn, s, flag, mchk,
                                                                         mask_numel(g), MASK_LIMIT, weight,
                                                                         (size_t)g.M * g.Cg * g.Kn));
        } else {
            if (direct)
                x_in_place = xcl = const_cast<void *>(X);   // already the kernels' layout and type
            else
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_storage_to_acc(dt, X, xcl, (size_t)g.B * g.Sn * g.C, s));
            if (sampled16) TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, check_sampled(pl, desc, x_in_place, mask, flag, s));
        }
        // grad_out (B, Cout, *out_size): conv Cout = M on the column grid, transposed Cout = C on the
        // sampled grid
        if (!pl.transposed)
            TVDCN_LAUNCH(TVDCN_KERNEL_BIAS_GRAD, s, launch_bias_grad(dt, grad_out, grad_bias, g.B, g.M, g.Pn, s,
                                                                     accumulate_weight, flag));
        else
            TVDCN_LAUNCH(TVDCN_KERNEL_BIAS_GRAD, s, launch_bias_grad(dt, grad_out, grad_bias, g.B, g.C, g.Sn, s,
                                                                     accumulate_weight));
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, operand_amax(pl, desc, cl_in ? weight : nullptr, cl_in ? X : nullptr,
                                                          cl_in ? mask : nullptr, pl.transposed ? Z : nullptr, flag,
                                                          s));
        void *zs = at(workspace, L.zs), *wsp = at(workspace, L.wsplit);
        // (16-bit weight-gradient loop) Z's 16-bit values in column blocks, from the same launch
        void *zw = sampled16 && pl.wn_s.ok ? at(workspace, L.zw) : nullptr;
        if (pl.wn_s.ok)
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                         launch_data_win_prep(dt, g, pl.wn_s, Z, weight, zs, wsp, wd, flag, s, zw));
        else
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_weight_data_layout(dt, g, weight, wd, pl.dt.Mg_pad, pl.dt.Cg_pad, s));
        if (!pl.transposed) {
            if (pl.wn_s.ok && coord && pl.data_split && pl.dim == 3) {
                // 3D: one launch on the scatter window, the offset / mask gradients reading X
                // from global memory (cached), instead of two that each recompute the contraction
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, pl.wn_xg, true, true, Z, wd, zs, wsp,
                                                                            flag, xcl, offset, mask, gx_cl, goff, gmask, s,
                                                                            pl.gx_nchw));
            } else if (pl.wn_s.ok && coord && pl.data_split) {
                // two launches, each with the larger window its LDS share allows
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, pl.wn_x, true, false, Z, wd, zs, wsp,
                                                                            flag, xcl, offset, mask, gx_cl, nullptr, nullptr,
                                                                            s, pl.gx_nchw));
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, pl.wn_c, false, true, Z, wd, zs, wsp,
                                                                            flag, xcl, offset, mask, nullptr, goff, gmask, s));
            } else if (pl.wn_s.ok)
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, coord ? pl.wn_s : pl.wn_x, true, coord,
                                                                            Z, wd, zs, wsp, flag, xcl, offset, mask, gx_cl,
                                                                            goff, gmask, s, pl.gx_nchw));
            else
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data(dt, pl.dim, g, pl.dt, true, coord, Z, wd, xcl, offset, mask,
                                                                        gx_cl, goff, gmask, s));
            if (!pl.gx_in_place && !cl_in)
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                             launch_from_channels_last(dt, gx_cl, grad_input, nullptr, g.B, g.C, g.Sn, s));
            else if (!pl.gx_in_place)
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                             launch_acc_to_storage(dt, gx_cl, grad_input, (size_t)g.B * g.Sn * g.C, s));
        } else {
            void *wf = at(workspace, L.wf);
            if (pl.fw.ok) {
                void *w16 = sampled16 ? at(workspace, L.w16) : nullptr;
                if (w16 != nullptr)
                    TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fwd_win_layout16(dt, g, pl.fw, weight, w16, flag, s, wf));
                else
                    TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_fwd_win_layout(dt, g, pl.fw, weight, wf, s));
                TVDCN_LAUNCH(TVDCN_KERNEL_GATHER_GEMM, s,
                             launch_fwd_win(dt, pl.dim, g, pl.wn_f, pl.fw, xcl, wf, w16, flag, offset, mask, nullptr,
                                            grad_input, y32, s));
                if (pl.fw.ksplit > 1 && dt != kF32)
                    TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                                 launch_acc_to_storage(dt, y32, grad_input, (size_t)g.B * g.M * g.Pn, s));
            } else {
                TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_weight_fwd_layout(dt, g, weight, wf, pl.ft.Mg_pad, pl.ft.Cg_pad, s));
                TVDCN_LAUNCH(TVDCN_KERNEL_GATHER_GEMM, s,
                             launch_fwd_gather_gemm(dt, pl.dim, g, pl.ft, xcl, wf, offset, mask, nullptr, grad_input, s));
            }
            if (coord && pl.wn_c.ok)
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data_win(dt, pl.dim, g, pl.wn_c, false, true, Z, wd, zs, wsp,
                                                                            flag, xcl, offset, mask, nullptr, goff, gmask, s));
            else if (coord)
                TVDCN_LAUNCH(TVDCN_KERNEL_DATA_GRAD, s, launch_bwd_data(dt, pl.dim, g, pl.dt, false, true, Z, wd, xcl, offset, mask,
                                                                        nullptr, goff, gmask, s));
        }
        if (pl.ww.ok)
            TVDCN_LAUNCH(TVDCN_KERNEL_WEIGHT_GRAD, s, launch_bwd_weight_win(dt, pl.dim, g, pl.wn_w, pl.wn_w16, pl.ww, Z, xcl, offset,
                                                                            mask, at(workspace, L.wpart), grad_weight,
                                                                            accumulate_weight, sampled16 ? flag : nullptr, s,
                                                                            zw));
        else
            TVDCN_LAUNCH(TVDCN_KERNEL_WEIGHT_GRAD, s, launch_bwd_weight(dt, pl.dim, g, pl.wt, Z, xcl, offset, mask,
                                                                        at(workspace, L.wpart), grad_weight,
                                                                        accumulate_weight, s));
    }
    // mask logits: the accumulated mask gradient through d(mask value) / d(logit) -- elementwise for
    // the sigmoid, over the taps of each (batch, mask group, pixel) for the softmax
    if (gmask && (desc->flags & TVDCN_FLAG_MASK_SIGMOID))
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s, launch_mask_sigmoid_grad(dt, mask, gmask, desc->mask_scale, n_gmask, s));
    if (gmask && (desc->flags & TVDCN_FLAG_MASK_SOFTMAX))
        TVDCN_LAUNCH(TVDCN_KERNEL_MASK_SOFTMAX, s,
                     launch_mask_softmax_logit_grad(dt, mask, gmask, (int64_t)g.B * g.mg, g.Kn, g.Pn, s));
    if (!direct && (goff || gmask))
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                     launch_acc_to_storage2(dt, goff, grad_offset, goff ? n_goff : 0, gmask, grad_mask,
                                            gmask ? n_gmask : 0, s));
    return TVDCN_STATUS_SUCCESS;
}

// Workspace bytes of a call: the largest of its blocks' layouts (a full block and the remainder).
size_t workspace_bytes_of(const tvdcn_conv_desc *desc, bool backward) {
    int64_t block = 0;
    if (batch_block(desc, block)) return 0;
    Plan pl;
    if (make_plan(desc, pl, block)) return 0;
    size_t n = layout(pl, backward).total;
    const int64_t tail = block > 0 ? desc->batch % block : 0;
    if (tail > 0) {
        Plan pt;
        if (make_plan(desc, pt, tail)) return 0;
        n = std::max(n, layout(pt, backward).total);
    }
    return n;
}

// The forward over the batch blocks (pointers checked, workspace large enough).
tvdcn_status forward_blocks(const tvdcn_conv_desc *desc, int64_t block, const void *input, const void *weight,
                            const void *offset, const void *mask, const void *bias, void *output, void *workspace,
                            void *stream) {
    ImageElems ie;
    int64_t blk = 0;
    tvdcn_status st = batch_block(desc, blk, &ie);
    if (st) return st;
    const size_t es = elem_size(desc->dtype);
    auto adv = [](const void *p, size_t bytes) -> void * {
        return p ? static_cast<char *>(const_cast<void *>(p)) + bytes : nullptr;
    };
    for (int64_t b0 = 0; b0 < desc->batch; b0 += block) {
        const int64_t nb = std::min<int64_t>(block, desc->batch - b0);
        Plan pl;
        st = make_plan(desc, pl, nb);
        if (st) return st;
        st = forward_planned(pl, desc, adv(input, b0 * ie.in * es), weight, adv(offset, b0 * ie.offset * es),
                             adv(mask, b0 * ie.mask * es), bias, adv(output, b0 * ie.out * es), workspace, stream);
        if (st) return st;
    }
    return TVDCN_STATUS_SUCCESS;
}

// ---------------------------------------------------------------------------
// Scratch of tvdcn_deform_conv_forward_noalloc: one array per GPU in the code object's
// device memory, held until the process ends. Its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) at the entry point's first call on
// the device, and only that address is handed to kernels (the array's name is a host-side
// stand-in in host code).
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[TVDCN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

tvdcn_status scratch_of_current_device(void **out) {
    static std::mutex mu;
    static void *ptrs[kMaxDevices] = {};
    int dev = -1;
    TVDCN_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(TVDCN_STATUS_NOT_SUPPORTED, "forward_noalloc: device index above 63");
    std::lock_guard<std::mutex> lk(mu);
    if (ptrs[dev] == nullptr) {
        void *p = nullptr;
        TVDCN_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr) return fail(TVDCN_STATUS_HIP_ERROR, "forward_noalloc: no device address for the scratch array");
        ptrs[dev] = p;
    }
    *out = ptrs[dev];
    return TVDCN_STATUS_SUCCESS;
}

}  // namespace

extern "C" {

tvdcn_status tvdcn_conv_batch_block(const tvdcn_conv_desc *desc, int64_t *images_per_block) {
    int64_t block = 0;
    const tvdcn_status st = batch_block(desc, block);
    if (st == TVDCN_STATUS_SUCCESS && images_per_block) *images_per_block = block;
    return st;
}

tvdcn_status tvdcn_conv_output_size(const tvdcn_conv_desc *desc, int64_t out_size[3]) {
    int64_t tmp[3] = {1, 1, 1};
    tvdcn_status st = output_size(desc, tmp);
    if (st == TVDCN_STATUS_SUCCESS && out_size)
        for (int i = 0; i < 3; ++i) out_size[i] = tmp[i];
    return st;
}

size_t tvdcn_deform_conv_forward_workspace_size(const tvdcn_conv_desc *desc) {
    return workspace_bytes_of(desc, false);
}

size_t tvdcn_deform_conv_backward_workspace_size(const tvdcn_conv_desc *desc) {
    return workspace_bytes_of(desc, true);
}

tvdcn_status tvdcn_set_max_block_elements(int64_t max_elements) {
    if (max_elements < 1 || max_elements > INT_MAX)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "max_elements must be in [1, 2^31 - 1]");
    g_block_limit.store(max_elements);
    return TVDCN_STATUS_SUCCESS;
}

tvdcn_status tvdcn_deform_conv_forward(const tvdcn_conv_desc *desc, const void *input, const void *weight,
                                       const void *offset, const void *mask, const void *bias, void *output,
                                       void *workspace, size_t workspace_bytes, void *stream) {
    int64_t block = 0;
    tvdcn_status st = batch_block(desc, block);
    if (st) return st;
    Plan pl;
    st = make_plan(desc, pl, block);
    if (st) return st;
    if (desc->batch == 0) return TVDCN_STATUS_SUCCESS;   // empty batch: empty output, nothing to do
    st = check_forward_pointers(desc, offset, mask);
    if (st) return st;
    st = check_aligned({input, weight, offset, mask, bias, output});
    if (st) return st;
    if (workspace_bytes < workspace_bytes_of(desc, false))
        return fail(TVDCN_STATUS_WORKSPACE_TOO_SMALL, "workspace too small");
    return forward_blocks(desc, block, input, weight, offset, mask, bias, output, workspace, stream);
}

tvdcn_status tvdcn_deform_conv_forward_noalloc(const tvdcn_conv_desc *desc, const void *input, const void *weight,
                                               const void *offset, const void *mask, const void *bias, void *output,
                                               void *stream) {
    int64_t block = 0;
    tvdcn_status st = batch_block(desc, block);
    if (st) return st;
    Plan pl;
    st = make_plan(desc, pl, block);
    if (st) return st;
    if (desc->batch == 0) return TVDCN_STATUS_SUCCESS;
    st = check_forward_pointers(desc, offset, mask);
    if (st) return st;
    st = check_aligned({input, weight, offset, mask, bias, output});
    if (st) return st;
    const size_t need = workspace_bytes_of(desc, false);
    if (need > (size_t)TVDCN_SCRATCH_BYTES)
        return fail(TVDCN_STATUS_WORKSPACE_TOO_SMALL,
                    "forward_noalloc: this problem needs " + std::to_string(need) +
                        " bytes of scratch; the library's per-GPU scratch holds " +
                        std::to_string((size_t)TVDCN_SCRATCH_BYTES) +
                        " (use tvdcn_deform_conv_forward with a workspace)");
    void *ws = nullptr;
    st = scratch_of_current_device(&ws);
    if (st) return st;
    return forward_blocks(desc, block, input, weight, offset, mask, bias, output, ws, stream);
}

tvdcn_status tvdcn_deform_conv_backward(const tvdcn_conv_desc *desc, const void *grad_out, const void *input,
                                        const void *weight, const void *offset, const void *mask, void *grad_input,
                                        void *grad_weight, void *grad_offset, void *grad_mask, void *grad_bias,
                                        void *workspace, size_t workspace_bytes, void *stream) {
    int64_t block = 0;
    ImageElems ie;
    tvdcn_status st = batch_block(desc, block, &ie);
    if (st) return st;
    Plan pl;
    st = make_plan(desc, pl, block);
    if (st) return st;
    const Geo &g = pl.g;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int dt = pl.dtype;
    if (desc->batch == 0) {
        // empty batch: the reference returns zero weight / bias gradients; the
        // batch-sized tensors are empty (their pointers may be null)
        if (!grad_weight) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "null tensor pointer");
        g_last_error.clear();
        TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                     launch_fill_zero((int)elem_size(dt), grad_weight, (size_t)g.M * g.Cg * g.Kn, s));
        if (grad_bias)
            TVDCN_LAUNCH(TVDCN_KERNEL_LAYOUT, s,
                         launch_fill_zero((int)elem_size(dt), grad_bias, (size_t)desc->out_channels, s));
        return TVDCN_STATUS_SUCCESS;
    }
    if ((desc->offset_groups == 0) != (offset == nullptr) || (offset == nullptr) != (grad_offset == nullptr))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "offset / grad_offset pointers and offset_groups disagree");
    if ((desc->mask_groups == 0) != (mask == nullptr) || (mask == nullptr) != (grad_mask == nullptr))
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "mask / grad_mask pointers and mask_groups disagree");
    if (workspace_bytes < workspace_bytes_of(desc, true))
        return fail(TVDCN_STATUS_WORKSPACE_TOO_SMALL, "workspace too small");
    if (!grad_out || !input || !weight || !grad_input || !grad_weight)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "null tensor pointer");
    if (!aligned16(workspace)) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    st = check_aligned({grad_out, input, weight, offset, mask, grad_input, grad_weight, grad_offset, grad_mask,
                        grad_bias});
    if (st) return st;
    if (!fits_int(desc->batch)) return fail(TVDCN_STATUS_NOT_SUPPORTED, "batch above 2^31 - 1");
    g_last_error.clear();
    // per image: X / grad_input and Z follow the op's input and output tensors
    const size_t es = elem_size(dt);
    const size_t in_b = (size_t)ie.in * es, out_b = (size_t)ie.out * es, off_b = (size_t)ie.offset * es,
                 mask_b = (size_t)ie.mask * es;
    auto adv = [](const void *p, size_t bytes) -> void * {
        return p ? static_cast<char *>(const_cast<void *>(p)) + bytes : nullptr;
    };
    for (int64_t b0 = 0; b0 < desc->batch; b0 += block) {
        const int64_t nb = std::min<int64_t>(block, desc->batch - b0);
        Plan bp;
        st = nb == block ? TVDCN_STATUS_SUCCESS : make_plan(desc, bp, nb);
        if (st) return st;
        st = backward_planned(nb == block ? pl : bp, desc, adv(grad_out, b0 * out_b), adv(input, b0 * in_b), weight,
                              adv(offset, b0 * off_b), adv(mask, b0 * mask_b), adv(grad_input, b0 * in_b),
                              grad_weight, adv(grad_offset, b0 * off_b), adv(grad_mask, b0 * mask_b), grad_bias,
                              workspace, stream, b0 > 0);
        if (st) return st;
    }
    return TVDCN_STATUS_SUCCESS;
}

tvdcn_status tvdcn_to_channels_last(int32_t dtype, int64_t batch, int64_t channels, int64_t spatial_numel,
                                    const void *input, void *output, void *stream) {
    return layout_copy(true, dtype, batch, channels, spatial_numel, input, output, stream);
}

tvdcn_status tvdcn_from_channels_last(int32_t dtype, int64_t batch, int64_t channels, int64_t spatial_numel,
                                      const void *input, void *output, void *stream) {
    return layout_copy(false, dtype, batch, channels, spatial_numel, input, output, stream);
}

tvdcn_status tvdcn_mask_softmax_forward(int32_t dtype, int64_t batch, int64_t groups, int64_t kernel_numel,
                                        int64_t spatial_numel, const void *x, void *y, void *stream) {
    if (dtype < 0 || dtype > 3) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "unknown dtype");
    if (batch < 0 || groups < 0 || kernel_numel <= 0 || spatial_numel < 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "invalid mask_softmax sizes");
    if (!fits_int(kernel_numel)) return fail(TVDCN_STATUS_NOT_SUPPORTED, "kernel_numel too large");
    g_last_error.clear();
    hipStream_t s = static_cast<hipStream_t>(stream);
    TVDCN_LAUNCH(TVDCN_KERNEL_MASK_SOFTMAX, s,
                 launch_mask_softmax_fwd(dtype, x, y, batch * groups, (int)kernel_numel, spatial_numel, s));
    return TVDCN_STATUS_SUCCESS;
}

tvdcn_status tvdcn_mask_softmax_backward(int32_t dtype, int64_t batch, int64_t groups, int64_t kernel_numel,
                                         int64_t spatial_numel, const void *y, const void *grad_y, void *grad_x,
                                         void *stream) {
    if (dtype < 0 || dtype > 3) return fail(TVDCN_STATUS_INVALID_ARGUMENT, "unknown dtype");
    if (batch < 0 || groups < 0 || kernel_numel <= 0 || spatial_numel < 0)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "invalid mask_softmax sizes");
    if (!fits_int(kernel_numel)) return fail(TVDCN_STATUS_NOT_SUPPORTED, "kernel_numel too large");
    g_last_error.clear();
    hipStream_t s = static_cast<hipStream_t>(stream);
    TVDCN_LAUNCH(TVDCN_KERNEL_MASK_SOFTMAX, s, launch_mask_softmax_bwd(dtype, y, grad_y, grad_x, batch * groups,
                                                                      (int)kernel_numel, spatial_numel, s));
    return TVDCN_STATUS_SUCCESS;
}

const char *tvdcn_last_error(void) { return g_last_error.c_str(); }

int64_t tvdcn_hip_version(void) { return (int64_t)HIP_VERSION; }

const char *tvdcn_arch_flags(void) { return "gfx950"; }

void tvdcn_kernel_timer_enable(int32_t enable) {
    KernelTimer &t = timer();
    std::lock_guard<std::mutex> lk(t.mu);
    t.drain();
    t.enabled = enable != 0;
    for (int i = 0; i < TVDCN_KERNEL_FAMILIES; ++i) {
        t.total_ms[i] = 0.0;
        t.count[i] = 0;
    }
}

tvdcn_status tvdcn_kernel_timer_read(int32_t family, double *total_ms, int64_t *launches) {
    if (family < 0 || family >= TVDCN_KERNEL_FAMILIES)
        return fail(TVDCN_STATUS_INVALID_ARGUMENT, "unknown kernel family");
    KernelTimer &t = timer();
    std::lock_guard<std::mutex> lk(t.mu);
    t.drain();
    if (total_ms) *total_ms = t.total_ms[family];
    if (launches) *launches = t.count[family];
    return TVDCN_STATUS_SUCCESS;
}

}  // extern "C"
