// launch.h — host-side launchers of the DenseBlock kernels (internal to
// libsoklyn_hip.so; the public surface is include/soklyn_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_math.h"

namespace skl {

// ---- GEMM epilogue parameters ------------------------------------------------
// Forward: Z = X.W (+b); when fuse_act, act + dropout write predrop/out/mask
// (forward.cu:8-28 + 130-161 fused; norm Disabled), otherwise Z is the
// prenorm cache and the row-norm kernel finishes the layer.
struct FwdEpi {
    const void *bias;          // T[N] or null
    void *z_out;               // T [M x ldc]: preact (fused) or prenorm
    void *predrop, *out, *mask;
    uint32_t fuse_act, act, use_dropout, seed;
    float leaky, p;
    uint32_t ldc, pad;
};

// The bias / norm-parameter update: column partial sums -> optimiser step.
struct VecOptArgs {
    uint32_t dtype, rows, n, splits;
    const float *src[3];          // d_prenorm (bias), d_norm_w, d_norm_b (null = skip)
    float *partials;              // [splits][3][n]
    // targets: 0 bias, 1 norm_w, 2 norm_b
    void *param[3];
    float *master[3], *dv[3], *dm[3];
    uint32_t enabled[3];
    OptParams opt[3];
    float lr, clamp, inv_m;
    uint32_t cpb;                 // columns per workgroup (set by the launchers)
};

// dW + optimiser on W (backward.cu:180-186 + 227-233).
struct OptEpi {
    float *master;        // fp32 master (the parameter itself for fp32 blocks)
    void *param;          // T copy (null when param is the master)
    float *dv, *dm;
    OptParams opt;
    float lr, clamp, inv_m, regu_coeff;
    uint32_t regularisation, ldc;
    // the 256x256 kernel's fused form only: after its tiles, workgroup w runs
    // blocks w, w + grid, ... < vec_blocks of the bias / norm-parameter update
    uint32_t vec_blocks;
    VecOptArgs vec;
    // fp16 blocks: an element whose sum over fp16 operands is not finite (a
    // d_prenorm beyond the fp16 range made its fp16 copy infinite) is summed
    // again in fp32 from these, as the reference's fp32 dW does
    // (backward.cu:181-186); null dp32: no such check
    const void *x;           // the dW's input rows [batch x K] at pitch ldx, T
    const float *dp32;       // d_prenorm [batch x N] at pitch lddp
    uint32_t ldx, lddp, batch, pad2;
};

// Plain fp32 store (input gradient) or split-K partial store.
struct StoreEpi {
    float *out;
    uint64_t split_stride;   // elements between split-K partial planes
    uint32_t ldc, pad;
};

// Hidden-layer error fused into the dX GEMM's epilogue (backward.cu:59-102 in
// one kernel, as the reference has it): from the sum s in the accumulators,
// e = mask * act'(s, predrop, preact), grad = e, the element-local norm
// gradient into d_prenorm / d_prenorm_h / dNorm, and the column sums of
// d_prenorm / dNorm_w / dNorm_b of each 256-row tile into
// partials[tile_m][k][ncols] (k = 0, and 1, 2 with a norm).
struct ErrEpi {
    const void *predrop, *preact, *mask;          // T [rows x ldc]
    const void *norm_rstd, *centered, *prenorm;   // T
    const float *nw;                              // master norm weight [ncols]
    float *grad, *d_prenorm, *d_norm_w, *d_norm_b;
    half_t *d_prenorm_h;
    float *partials;
    uint32_t norm, act, ldc, ncols;
    float leaky, inv_n, inv_m, pad;
};

enum class Op { Fwd, InputGrad, DwOpt, DwPartial, HiddenErr };
// The fused hidden error fits the 256x256 kernel's output of M x N (whole tiles,
// 4-aligned rows, 16-byte aligned buffers).
bool hidden_err_fusable(const ErrEpi &e, uint32_t M, uint32_t N);

// One GEMM launch.  dtype selects fp16 (MFMA 32x32x16 f16) or fp32
// (MFMA 32x32x2 f32).  a_kcontig / b_kcontig as in gemm.h.
struct GemmLaunch {
    uint32_t dtype;
    uint32_t M, N, K, lda, ldb;
    bool a_kcontig, b_kcontig;
    const void *A, *B;
    uint32_t splits;      // split-K factor (DwPartial only; 1 otherwise)
    uint32_t tile;        // direct-to-LDS kernel: 128 (4 waves, two workgroups per CU) or 256 (0 = 256);
                          // fp32 register-staged kernel: 128 asks for 128x128 tiles on any grid
    uint32_t mv, nv;      // real output extent when A / B are zero-padded copies (0 = M, N)
    // direct-to-LDS kernel: the launch covers output rows [m_begin, m_begin + m_rows)
    // only (0, 0: all M), m_begin a multiple of 256 and m_rows of the tile edge;
    // not for HiddenErr, whose column sums are indexed by the tile row
    uint32_t m_begin, m_rows;
    Op op;
    FwdEpi fwd;
    OptEpi opt;
    StoreEpi st;
    ErrEpi err;
    const float *b32;     // dW: fp32 d_prenorm (ld N), read by the skinny kernel instead of B
    // When set, the GEMM kernel's own dispatch records these events at its start
    // and end (hipExtLaunchKernelGGL: no marker packets between kernels).
    hipEvent_t time_start, time_stop;
};

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t stream);
// Skinny outputs (N <= 16).  Forward: a streaming kernel, W staged in LDS
// (fits when skinny_fwd_ok).  dW: batch-sliced partial sums of X^T . d_prenorm
// (fp32) into partials [slices x K x 16]; skinny_dw_slices gives the slice count.
bool skinny_fwd_ok(const GemmLaunch &g);
hipError_t launch_skinny_fwd(const GemmLaunch &g, hipStream_t stream);
uint32_t skinny_dw_slices(uint32_t rows, uint32_t K);
hipError_t launch_skinny_dw(const GemmLaunch &g, float *partials, uint32_t slices, hipStream_t stream);
// The 256x256 direct-to-LDS kernel on operands that fit it (gemm_dma_shape_ok):
// M, N whole 256 tiles (zero-padded copies allowed: the epilogue stops at mv, nv),
// K a multiple of 128; DwPartial may split K into g.splits slices.
hipError_t launch_gemm_dma(const GemmLaunch &g, hipStream_t stream);
bool gemm_dma_shape_ok(const GemmLaunch &g);
bool gemm_dma_enabled();
// Output tile edge of the direct-to-LDS kernel forced by SOKLYN_GEMM_TILE (128 or
// 256), or 0: the planner picks per GEMM.
uint32_t gemm_dma_tile_forced();
// Number of split-K slices launch_gemm_dma makes when asked for `splits`.
uint32_t gemm_dma_splits(uint32_t K, uint32_t splits);
// Number of output tiles the launcher would use (for split-K sizing).
uint32_t gemm_tiles(uint32_t dtype, uint32_t M, uint32_t N);
// True when an fp16 GEMM of this output size uses the 256x256 tile (k-contiguous operands only).
bool gemm_large_tile(uint32_t dtype, uint32_t M, uint32_t N);
// True when this launch runs on the 256x256 direct-to-LDS kernel with its operand
// layouts as given (then transposed operand copies buy nothing).
bool gemm_direct_ok(const GemmLaunch &g);
uint32_t gemm_bk(uint32_t dtype);

// ---- element-wise / row / column kernels -------------------------------------
hipError_t launch_fill(void *dst, uint32_t dtype, float v, size_t n, hipStream_t s);
hipError_t launch_cast(const void *src, uint32_t sdt, void *dst, uint32_t ddt, size_t n, hipStream_t s);

struct RowNormArgs {
    uint32_t dtype, m, n, norm, act, use_dropout, seed;
    float leaky, p;
    const void *prenorm, *norm_w, *norm_b;
    void *centered, *preact, *predrop, *out, *mask, *norm_rstd;
    uint64_t keep_min;   // set by launch_norm_act: dropout_keep_min(p)
};
// fwd1 + fwd2 fused (RMS / LN per row; BN per column then act).
hipError_t launch_norm_act(const RowNormArgs &a, hipStream_t s);

hipError_t launch_softmax(uint32_t dtype, void *out, uint32_t rows, uint32_t n, hipStream_t s);

struct ErrArgs {
    uint32_t dtype, rows, n, norm, act, loss;
    float leaky, inv_n, inv_m, loss_scale;
    const void *out, *preact, *target;                 // output error
    const float *s;                                    // error_from_sum
    uint32_t s_ld, pad;                                // row pitch of s (0 = n)
    const void *predrop, *mask;                        // error_from_sum
    const void *norm_rstd, *centered, *prenorm;
    const void *norm_in;                               // set by the launchers: prenorm (RMS) or centered
    const void *sk_a, *sk_w;                           // launch_error_skinny: T [rows x 16], T [n x 16]
    const float *nw;
    float *grad, *d_prenorm, *d_norm_w, *d_norm_b;
    half_t *d_prenorm_h;
};
// Both also write partial column sums of d_prenorm / dNorm_w / dNorm_b into
// partials [splits x 3 x n]; their sum over the splits rows is the column sum
// over all rows.  splits must come from err_col_splits.
hipError_t launch_output_error(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s);
hipError_t launch_error_from_sum(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s);
// Partial-sum rows the error kernels write for [rows x n].
uint32_t err_col_splits(uint32_t rows, uint32_t n, uint32_t resident = 0);
// Workgroups of the flat error kernel for (dtype, src: 0 output error, 1 from
// a sum, 2 skinny sum in-kernel, n, norm != 0) the current GPU holds at once
// (0 if unknown): err_col_splits' resident.
uint32_t err_resident(uint32_t dtype, uint32_t src, uint32_t n, bool norm);
// Hidden error from a next layer of at most 16 outputs without the GEMM: s =
// A . W^T formed inside the error kernel from zero-padded copies A [rows x 16]
// (the next layer's d_prenorm, or its fp16 copy) and W [n x 16] (its weights)
// in the block's type T, which launch_skinny_operands writes (dtype 1: fp16,
// else fp32; cols <= 16).  err_skinny_ok: the buffers (16-byte aligned) and
// n >= 4 fit that kernel.
hipError_t launch_skinny_operands(uint32_t dtype, const void *a, uint32_t a_rows, const void *w, uint32_t w_rows,
                                  uint32_t cols, void *a16, void *w16, hipStream_t s);
bool err_skinny_ok(const ErrArgs &a, const float *partials);
hipError_t launch_error_skinny(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s);

// Column sums of up to three fp32 [rows x n] arrays into partials
// [splits x 3 x n]; then the bias / norm-parameter optimiser.
hipError_t launch_colsum(const VecOptArgs &a, hipStream_t s);
// Columns per workgroup of the parameter update for `splits` partial rows.
uint32_t vec_opt_cpb(uint32_t splits);
// Row splits for launch_colsum so the grid has ~1024 workgroups.
uint32_t colsum_splits(uint32_t rows, uint32_t n);
hipError_t launch_vec_opt(const VecOptArgs &a, hipStream_t s);

// Split-K dW reduction + W optimiser.
struct DwReduceArgs {
    uint32_t dtype, rows, n, splits;
    const float *partials;         // split sp, element (r, c) at sp * plane + r * pld + c
    uint64_t plane;
    uint32_t pld, pad;
    OptEpi e;
    // with_vec: the same launch also runs launch_vec_opt(vec) (the bias / norm-
    // parameter update, independent of W) in its first workgroups
    uint32_t with_vec, vec_blocks;
    VecOptArgs vec;
};
hipError_t launch_dw_reduce_opt(const DwReduceArgs &a, hipStream_t s);

// fp16 transpose: out [cols x rows] (ld_out) = in [rows x cols] (ld_in)^T.
// rows, cols, ld_in, ld_out multiples of 8; both buffers 16-byte aligned.
// Zero-padded fp16 copy: out [rows_p x cols_p] (cols_p % 8 == 0, 16-byte aligned)
// holds in [rows x cols] (leading dim ld) and zeros elsewhere.
hipError_t launch_pad_h(const void *in, uint32_t rows, uint32_t cols, uint32_t ld, void *out, uint32_t rows_p,
                        uint32_t cols_p, hipStream_t s);

}  // namespace skl
