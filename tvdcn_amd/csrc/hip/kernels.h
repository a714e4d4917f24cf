// Host-side launchers of the gfx950 kernels (one definition per .hip file).
// All launches are asynchronous on `stream`; none allocates or synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <atomic>
#include "common.h"

namespace tvdcn_hip {

enum DType { kF32 = 0, kF64 = 1, kF16 = 2, kBF16 = 3 };

// Tile parameters shared by host and device code.
struct FwdTiles {
    int waves;       // 1, 2 or 4 waves along the GEMM-side channels (64 rows each)
    bool vec4;       // channel quads share offset/mask group (fast gather)
    int Mg_pad;      // Mg rounded up to 64 * waves
    int Cg_pad;      // Cg rounded up to 16
};
struct DataTiles {
    int waves;       // taps per workgroup (one 64-channel x 64-pixel tile per wave)
    int Mg_pad;      // Mg rounded up to 16
    int Cg_pad;      // Cg rounded up to 64
    bool uniform;    // every 64-channel tile lies in one offset group and one mask group
};
struct WeightTiles {
    int waves;       // 64-row GEMM-side blocks per workgroup
    bool vec4;
    int k_chunk;     // column pixels per workgroup (split-K)
    int k_splits;
    size_t part_elems;   // workspace elements for the split partials
};

// Windowed data-gradient kernel (bwd_data_win.hip): 256-pixel box x 16 channels x
// up to WIN_TMAX taps per pass, bilinear scatter pre-accumulated in LDS.
constexpr int WIN_TMAX = 9;                   // taps held in accumulators per pass
constexpr size_t WIN_LDS_TARGET = 156 * 1024; // bytes of LDS per workgroup (gfx950: 160 KB per CU)

// Raise a kernel's dynamic-LDS limit to WIN_LDS_TARGET on the current device, once per
// device (devices 0..63 tracked as bits of `done`; others set it on every call). Safe to
// call from several host threads: setting the attribute twice is harmless.
inline hipError_t raise_lds_limit(const void *kern, std::atomic<unsigned long long> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const unsigned long long bit = dev >= 0 && dev < 64 ? 1ull << dev : 0ull;
    if (bit != 0ull && (done.load(std::memory_order_acquire) & bit) != 0ull) return hipSuccess;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)WIN_LDS_TARGET);
    if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
    return e;
}
struct WinTiles {
    bool ok;             // eligible: fp32/fp16/bf16, C % 4 == 0, 16-channel tiles group-uniform
    int box[3];          // tile box (embedded axes), product 256, powers of two
    int lbx, lbxy;       // log2(box[2]), log2(box[1] * box[2])
    int ntile[3];        // tiles per axis
    int R[3];            // window margin per axis
    int WE[3];           // window extent per axis (1 on unused axes)
    int cells;           // window cells (0 = no window: scatter goes straight to global)
    int c_tiles, m_steps;
    int tpp;             // taps per pass (<= WIN_TMAX)
    size_t chunk_elems;  // floats of the re-laid-out weight
    // 16-bit MFMA operands of the data gradient (16x16x32 MFMAs over 32 GEMM-side channels per
    // step): fp32 tensors split into two fp16 pieces each (per-tensor power-of-two scale), fp16 /
    // bf16 tensors as they are
    int xglobal;         // 3D only: offset / mask gradients read X from global memory, no X window
    int ms32;            // 32-channel steps of the GEMM side (zero padded)
    int npiece;          // 16-bit pieces per value: 2 (fp32), 1 (fp16 / bf16)
    size_t zs_elems;     // 16-bit elements of the split Z: [B][G][ms32][npiece][Pn][32]
    size_t ws_elems;     // 16-bit elements of the split weight: [G][c_tiles][ms32][Kn][npiece][512]
    int wstage;          // bytes of LDS staging the 16-bit K loop's weight blocks (double-buffered
                         // [2][tpp][npiece][512]); 0: fragments straight from global memory
};

// Windowed weight-gradient kernel (bwd_weight_win.hip): workgroups own (group,
// 16-channel slice, 256 rows) and a run of (pass, spatial tile) units of the WinTiles tiling.
struct WeightWin {
    bool ok;
    int tg;              // tap groups: 1 (256-row tiles) or 2 (64-row tiles, taps split by parity)
    int m_tiles;         // row tiles of the GEMM side
    int n_spatial;       // spatial tiles (B x ntile0 x ntile1 x ntile2)
    // split = a run of units_per_split (pass, spatial tile) units, pass-major: a split may
    // cover the end of one pass and the start of the next, so the work divides evenly
    // whatever the number of passes
    int units_per_split, n_split;
    bool z_vec;          // 4 consecutive tile pixels are contiguous and 16-byte aligned
    bool z8;             // 8 consecutive tile pixels are contiguous in every row (P_x % 8 == 0 and
                         // the box's rows at least 8 wide): the 16-bit loop can read its A fragments
                         // as 16-bit values, 8 per 16-byte load
    size_t part_elems;   // workspace floats for the split partials
};

// Windowed forward kernel (fwd_win.hip): workgroups own (spatial tile, 128 rows) of the
// WinTiles tiling and reduce over 16-channel slices x taps.
struct FwdWin {
    bool ok;
    int mb;              // 16-row blocks per workgroup (8 or 4)
    int m_tiles;         // (16 * mb)-row blocks of the GEMM side
    int ksplit;          // 1, or 2: the channel slices split between two workgroups whose fp32
                         // partials are added onto a zeroed fp32 output (y32)
    int slices_per;      // 16-channel slices per share
    int Mg_pad, Cg_pad;  // padded weight layout Wf[G][Kn][Mg_pad][Cg_pad]
    // 16x16x32 MFMAs over (tap pair, 16 channels) steps (1D / 2D): the weight as
    // W16[G][slices][pp][Mg_pad / 16][npiece][512] 16-bit values, pp = passes x hp tap pairs
    int tpp, hp, pp, npiece;   // taps per pass, tap pairs per pass, pairs, pieces per value
    size_t w16_elems;    // 0: no 16-bit path
    int stage_bytes;     // LDS past the X window: the 16-bit loop's two weight staging buffers
};

FwdTiles plan_fwd(const Geo &g, int dtype);
// windowed forward plan over the base tiling; wt receives the tiling with the forward's
// own window margin
FwdWin plan_fwd_win(const Geo &g, const WinTiles &base, int dim, WinTiles &wt);
WeightWin plan_weight_win(const Geo &g, const WinTiles &wt, int dim);
WinTiles plan_data_win(const Geo &g, int dtype, int dim, bool scatter, bool coord);
// the same tiling with the window margin re-sized for another kernel's LDS budget
// (cell_cap > 0: at most that many window cells)
WinTiles win_resize(const WinTiles &base, const Geo &g, int dim, size_t fixed_bytes, size_t cell_bytes,
                    long long cell_cap = 0);
// LDS of the windowed weight gradient besides its X window (its shape follows the pass length):
// npiece 0 for its fp32 loop, else the 16-bit pieces per value of its 16-bit loop (whose S tile
// is smaller, so that its X window can be larger)
size_t weight_win_fixed_bytes(const Geo &g, int dim, int tpp, int npiece);
size_t x_window_cell_bytes();
DataTiles plan_data(const Geo &g, int dtype);
WeightTiles plan_weight(const Geo &g, int dtype);

// layout / elementwise helpers (prep.hip)
// (flag: when not null, fp32 values not below SAMPLED_LIMIT in magnitude set *flag; chk: when not
// null, an fp32 tensor of chk_n values range-checked against chk_limit into *flag by the same
// launch, as launch_check_range does, its largest magnitude into the mask slot after *flag;
// amax_w: fp32 only, when not null, the largest magnitudes of amax_w's amax_w_n values (the
// weight slot) and of the copied values (the sampled-tensor slot), by the same launch)
hipError_t launch_to_channels_last(int dtype, const void *x, void *xcl, int B, int C, int Sn, hipStream_t s,
                                   int *flag = nullptr, const void *chk = nullptr, size_t chk_n = 0,
                                   float chk_limit = 0.f, const void *amax_w = nullptr, size_t amax_w_n = 0);
// 16-bit MFMA operands of the sampled side (forward, weight gradient): the sampled values are
// mask * bilinear(X), below 2^126 (finite, with a finite piece scale) when |X| < SAMPLED_LIMIT
// and |mask| < MASK_LIMIT; larger or non-finite values send the launch to its fp32 MFMA loop.
constexpr float SAMPLED_LIMIT = 0x1p96f;
constexpr float MASK_LIMIT = 0x1p30f;
// *flag |= some fp32 value of v[0 .. n) is not below limit in magnitude (or is nan)
hipError_t launch_check_range(const void *v, size_t n, float limit, int *flag, hipStream_t s);
hipError_t launch_from_channels_last(int dtype, const void *xcl, void *x, const void *bias, int B, int C, int Sn,
                                     hipStream_t s);
hipError_t launch_weight_fwd_layout(int dtype, const Geo &g, const void *w, void *wf, int Mg_pad, int Cg_pad,
                                    hipStream_t s);
hipError_t launch_weight_data_layout(int dtype, const Geo &g, const void *w, void *wd, int Mg_pad, int Cg_pad,
                                     hipStream_t s);
hipError_t launch_fill_zero(int elem_bytes, void *p, size_t n, hipStream_t s);   // elem_bytes 2, 4 or 8
// Zeroes up to kFillMax buffers in one launch (entries with p == nullptr or bytes == 0 are
// skipped); every buffer 2-byte aligned with an even byte count.
constexpr int kFillMax = 4;
struct FillItem {
    void *p;
    size_t bytes;
};
hipError_t launch_fill_zero_multi(const FillItem *items, int n, hipStream_t s);
// The fp32 path's 16-bit MFMA operands are fp16 pieces at a per-tensor power-of-two scale: the
// workspace's operand flag (one int) is followed by the largest magnitudes of the operands (float
// bits; slots: weight, sampled tensor, mask, GEMM-side tensor), zeroed with it. Each slot is spread
// over AMAX_SPREAD sub-slots, one per 64-byte line (AMAX_STRIDE words apart): producing blocks raise
// sub-slot (block index % AMAX_SPREAD), so that their atomics do not all meet on one address, and a
// consumer takes the largest of the sub-slots.
constexpr int AMAX_SLOT_W = 0, AMAX_SLOT_X = 1, AMAX_SLOT_M = 2, AMAX_SLOT_Z = 3, AMAX_SLOTS = 4;
constexpr int AMAX_SPREAD = 64, AMAX_STRIDE = 16;
constexpr int OPERAND_FLAG_WORDS = AMAX_STRIDE + AMAX_SLOTS * AMAX_SPREAD * AMAX_STRIDE;
// word (after the flag's first) of sub-slot k of slot
__host__ __device__ constexpr int amax_word(int slot, int k) { return AMAX_STRIDE + (slot * AMAX_SPREAD + k) * AMAX_STRIDE; }
struct AmaxItem {
    const float *p;   // nullptr / n == 0: skipped
    size_t n;
    int slot;
};
// raises slot `slot` of the words after *flag to the largest |p[i]| of every item (up to 4, one
// launch; nan values are passed over: the layout kernels' checks flag them)
hipError_t launch_amax(const AmaxItem *items, int n, int *flag, hipStream_t s);
hipError_t launch_acc_to_storage(int dtype, const void *acc, void *out, size_t n, hipStream_t s);
// the same for two tensors in one launch (acc0 -> out0, n0 elements; acc1 -> out1, n1 elements)
hipError_t launch_acc_to_storage2(int dtype, const void *acc0, void *out0, size_t n0, const void *acc1, void *out1,
                                  size_t n1, hipStream_t s);
hipError_t launch_storage_to_acc(int dtype, const void *x, void *acc, size_t n, hipStream_t s);   // elementwise widening
// gmask_acc (accumulation type) *= d(scale * sigmoid(logit)) / d(logit), elementwise
// gmask_acc (accumulation type) <- y * (gmask_acc - sum_k gmask_acc_k * y_k), y = softmax over K of the
// logits viewed as (BG, K, S): the gradient of a softmax-activated mask with respect to its logits
hipError_t launch_mask_softmax_logit_grad(int dtype, const void *logits, void *gmask_acc, int64_t BG, int K, int64_t S,
                                          hipStream_t s);
hipError_t launch_mask_sigmoid_grad(int dtype, const void *logits, void *gmask_acc, double scale, size_t n,
                                    hipStream_t s);
// gbias (when not null) = (accumulate: gbias +) sum over batch and space of gout; flag (fp32, when not
// null): gout's largest magnitude into the GEMM-side slot after *flag, by the same launch
hipError_t launch_bias_grad(int dtype, const void *gout, void *gbias, int B, int C, int Sn, hipStream_t s,
                            bool accumulate = false, int *flag = nullptr);

// the three GEMM families
hipError_t launch_fwd_gather_gemm(int dtype, int dim, const Geo &g, const FwdTiles &t, const void *xcl,
                                  const void *wf, const void *offset, const void *mask, const void *bias, void *y,
                                  hipStream_t s);
// weight -> the windowed forward's fragment-major layout (fwd_win.hip)
hipError_t launch_fwd_win_layout(int dtype, const Geo &g, const FwdWin &fw, const void *w, void *wp, hipStream_t s);
// the weight as W16 (fp32: two fp16 pieces at the weight's scale; *flag set for a value bad for the split)
// (wp: when not null, also the fp32 layout of launch_fwd_win_layout, in the same launch)
hipError_t launch_fwd_win_layout16(int dtype, const Geo &g, const FwdWin &fw, const void *w, void *w16, int *flag,
                                   hipStream_t s, void *wp = nullptr);
// w16 / flag: the 16-bit weight and the operand flag (w16 null, or *flag set: the fp32 loop)
hipError_t launch_fwd_win(int dtype, int dim, const Geo &g, const WinTiles &wt, const FwdWin &fw, const void *xcl,
                          const void *wf, const void *w16, const int *flag, const void *offset, const void *mask,
                          const void *bias, void *y, void *y32, hipStream_t s);
hipError_t launch_bwd_data(int dtype, int dim, const Geo &g, const DataTiles &t, bool scatter, bool coord,
                           const void *z, const void *wd, const void *xcl, const void *offset, const void *mask,
                           void *gx_cl, void *goff, void *gmask, hipStream_t s);
// Z (the GEMM-side tensor, (B, M, Pn)) and the weight as the data gradient's 16-bit MFMA operands
// (zs, wsplit), and the weight's fp32-loop chunks (wd: [G][c_tiles][m_steps][Kn][16 c][16 m]; skipped
// when null), in one launch. For fp32 tensors, *flag (zeroed by the caller first) is set
// when a value is not finite or at least 0x1.ffp127 in magnitude: the data gradient then runs its
// fp32 MFMA loop.
// zw (may be null): Z again as 16-bit values (fp32: two fp16 pieces at its scale, piece k at
// zw + k * B * M * Pn) in 8-pixel column blocks [B][Pn / 8][M][8], for the weight gradient's
// 16-bit loop (needs WeightWin::z8)
hipError_t launch_data_win_prep(int dtype, const Geo &g, const WinTiles &t, const void *z, const void *w, void *zs,
                                void *wsplit, void *wd, int *flag, hipStream_t s, void *zw = nullptr);
// gx_nchw: gx_cl is grad_input as the caller's float32 (B, C, *S) tensor (zeroed), not the
// channels-last accumulator
hipError_t launch_bwd_data_win(int dtype, int dim, const Geo &g, const WinTiles &t, bool scatter, bool coord,
                               const void *z, const void *wchunks, const void *zs, const void *wsplit,
                               const int *flag, const void *xcl, const void *offset, const void *mask, void *gx_cl,
                               void *goff, void *gmask, hipStream_t s, bool gx_nchw = false);
// flag: the operand flag (null: the fp32 MFMA loop; set: the same). zw: Z's 16-bit values
// written by launch_data_win_prep (null: the kernel forms them in registers)
// wt / wt16: the tiling with the fp32 loop's / the 16-bit loop's window (same tiles and passes)
hipError_t launch_bwd_weight_win(int dtype, int dim, const Geo &g, const WinTiles &wt, const WinTiles &wt16,
                                 const WeightWin &ww, const void *z, const void *xcl, const void *offset,
                                 const void *mask, void *part, void *gw, bool accumulate, const int *flag,
                                 hipStream_t s, const void *zw = nullptr);
// gw (storage type, layout (M, Cg, Kn)) = sum over k_splits of part[ks][G][Kn][Mg][Cg]
// dW = sum over splits of the partials; with units_per_split > 0 (windowed kernel) tap t sums only
// the splits whose unit range meets its pass (t / tpp) over n_spatial tiles
// (accumulate: gw += that sum, for batch blocks after the first)
hipError_t launch_weight_reduce(int dtype, const Geo &g, int k_splits, const void *part, void *gw, bool accumulate,
                                hipStream_t s, int units_per_split = 0, int n_spatial = 0, int tpp = 0);
// writes split partials to `part` (WeightTiles::part_elems accumulator elements),
// then reduces them into gw (storage type, layout (M, Cg, Kn))
hipError_t launch_bwd_weight(int dtype, int dim, const Geo &g, const WeightTiles &t, const void *z, const void *xcl,
                             const void *offset, const void *mask, void *part, void *gw, bool accumulate,
                             hipStream_t s);

// mask_softmax (mask_softmax.hip)
hipError_t launch_mask_softmax_fwd(int dtype, const void *x, void *y, int64_t BG, int K, int64_t S, hipStream_t s);
hipError_t launch_mask_softmax_bwd(int dtype, const void *y, const void *gy, void *gx, int64_t BG, int K, int64_t S,
                                   hipStream_t s);

}  // namespace tvdcn_hip
