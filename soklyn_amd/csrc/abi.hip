// abi.hip — implementation of include/soklyn_hip.h.
//
// Each entry point validates its arguments the way the reference's
// DenseBlock / GpuContext do (src/mlp.rs, src/io/device.rs) — that is also
// what keeps every kernel launch inside the shapes it assumes — then issues
// the MI355X kernels on the context's stream.
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <cmath>
#include <mutex>
#include <unordered_map>

#include <hip/hip_runtime.h>

#include "../../include/soklyn_hip.h"
#include "launch.h"

using namespace skl;

// Column sums of d_prenorm / dNorm_w / dNorm_b (partials [splits x 3 x n])
// written by an error entry point as a by-product of its pass over the rows.
// skl_dense_backward uses them instead of reading the three buffers again when
// they describe the same block and batch and were made by the call just
// before it on this context (every entry point counts as a call, so anything
// issued through the context in between invalidates them).
struct ColSums {
    const float *dp, *dnw, *dnb;
    uint32_t rows, n, splits, norm;
    uint64_t call;
    uint64_t gen;        // rewrite_gen(dp) when made
    bool valid;
};

// A block's fp16 d_prenorm copied zero-padded to [round_up(rows, 256) x ld],
// ld = round_up(n, 256), by the GEMM that first needed it padded (a dW reads
// d_prenorm_h as its B, the hidden error of the layer below and the input
// gradient as their A; the direct-to-LDS kernel cannot read an odd-width or
// ragged operand in place).  The context keeps it so that the other GEMM on the
// same d_prenorm_h reads it instead of padding it again: when it mirrors the
// same buffer, rows and n and was made by the same call or the one just before
// it (as with ColSums), and no error entry point has rewritten d_prenorm_h since.
// One slot per block, up to kPadSlots (the least recently made one reused).
constexpr int kPadSlots = 8;
struct PadCopy {
    half_t *buf;
    size_t bytes;
    const void *src;   // the d_prenorm_h it mirrors
    uint32_t rows, n, ld;
    uint64_t call;
    uint64_t gen;      // rewrite_gen(src) when made
    bool valid;
};

struct skl_ctx {
    int device;
    uint32_t tile_dim;
    hipStream_t own_stream;
    hipStream_t stream;
    uint32_t sync;
    void *ws;
    size_t ws_bytes;
    uint64_t calls;      // entry-point calls so far
    float *cols;         // ColSums storage
    size_t cols_bytes;
    ColSums cs;
    PadCopy pads[kPadSlots];
    bool keep_pads;      // SOKLYN_PAD_KEEP=0 at skl_ctx_create: GEMMs pad d_prenorm_h into the workspace every time
    hipEvent_t gemm_start, gemm_stop;   // skl_ctx_time_next_gemm
    void *scratch;       // device address of this device's copy of `scratch` (below)
};

// Scratch of the allocation-free entry point (skl_dense_error_from_sum_noalloc):
// the error kernel's column partial sums [splits x 3 x n] fp32 go here instead
// of the context's grown buffer.  One copy per GPU, allocated with the code
// object and held until the process ends.  Host code never uses the array's
// name as an address: skl_ctx_create looks up each device's copy once with
// hipGetSymbolAddress and every launch takes that pointer.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(16) << 20;
static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

int32_t hip_status(hipError_t e) { return e == hipSuccess ? SKL_OK : (int32_t)e; }

#define SKL_TRY(expr)                                                  \
    do {                                                               \
        hipError_t _e = (expr);                                        \
        if (_e != hipSuccess) return hip_status(_e);                   \
    } while (0)

#define SKL_CHECK(cond, code)                                          \
    do {                                                               \
        if (!(cond)) return (code);                                    \
    } while (0)

// Synchronous calls wait for their stream, except on a stream that is being
// captured into a HIP graph (a synchronize there would invalidate the capture).
int32_t finish(skl_ctx *ctx) {
    SKL_TRY(hipGetLastError());
    if (ctx->sync) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        SKL_TRY(hipStreamIsCapturing(ctx->stream, &cs));
        if (cs == hipStreamCaptureStatusNone) SKL_TRY(hipStreamSynchronize(ctx->stream));
    }
    return SKL_OK;
}

int32_t enter(skl_ctx *ctx) {
    if (!ctx) return SKL_ERR_NULL_POINTER;
    ++ctx->calls;
    SKL_TRY(hipSetDevice(ctx->device));
    return SKL_OK;
}

// Grow a context-owned device buffer (work in flight may still use it: sync first).
int32_t ensure_buf(skl_ctx *ctx, void **buf, size_t *have, size_t bytes) {
    if (bytes <= *have) return SKL_OK;
    SKL_TRY(hipStreamSynchronize(ctx->stream));
    if (*buf) SKL_TRY(hipFree(*buf));
    *buf = nullptr;
    *have = 0;
    const size_t want = bytes + (bytes >> 3);
    SKL_TRY(hipMalloc(buf, want));
    *have = want;
    return SKL_OK;
}

int32_t ensure_ws(skl_ctx *ctx, size_t bytes) { return ensure_buf(ctx, &ctx->ws, &ctx->ws_bytes, bytes); }

// Device address of `scratch` on device `dev` (current), looked up once per device.
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES];

int32_t scratch_address(int dev, void **out) {
    *out = nullptr;
    if (dev < 0 || dev >= MAX_DEVICES) return SKL_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (!p) return SKL_ERR_NULL_POINTER;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SKL_OK;
}

// Room for column sums of `splits` row slices over n columns.
int32_t ensure_cols_splits(skl_ctx *ctx, uint32_t splits, uint32_t n) {
    void *p = ctx->cols;
    const int32_t r = ensure_buf(ctx, &p, &ctx->cols_bytes, (size_t)splits * 3 * n * sizeof(float));
    ctx->cols = reinterpret_cast<float *>(p);
    return r;
}

// Room for the column sums of an error call over [rows x n]; returns the
// splits.  src: the flat error kernel that runs (0 output error, 1 from a sum,
// 2 skinny sum in-kernel), whose resident workgroups cap the grid.
int32_t ensure_cols(skl_ctx *ctx, const skl_dense_desc *b, uint32_t rows, uint32_t src, uint32_t *splits) {
    *splits = err_col_splits(rows, b->outputs, err_resident(b->dtype, src, b->outputs, b->norm != 0));
    return ensure_cols_splits(ctx, *splits, b->outputs);
}

// Rewrites of a block's d_prenorm / d_prenorm_h by the error entry points,
// counted per buffer address over the whole process: a kept padded copy or
// column-sum set remembers the count of its source when it was made and is
// stale once an error call on any context has rewritten that buffer since.
std::mutex g_gen_mu;
std::unordered_map<const void *, uint64_t> g_gen;

uint64_t rewrite_gen(const void *p) {
    std::lock_guard<std::mutex> lock(g_gen_mu);
    const auto it = g_gen.find(p);
    return it == g_gen.end() ? 0 : it->second;
}

void pad_forget(skl_ctx *ctx, const void *src);

// An error entry point is about to rewrite b's d_prenorm (and d_prenorm_h).
void note_rewrite(skl_ctx *ctx, const skl_dense_desc *b) {
    {
        std::lock_guard<std::mutex> lock(g_gen_mu);
        ++g_gen[b->d_prenorm];
        if (b->d_prenorm_h) ++g_gen[b->d_prenorm_h];
    }
    if (b->d_prenorm_h) pad_forget(ctx, b->d_prenorm_h);
}

void record_cols(skl_ctx *ctx, const skl_dense_desc *b, uint32_t rows, uint32_t splits) {
    ColSums &c = ctx->cs;
    c.dp = b->d_prenorm;
    c.dnw = b->d_norm_w;
    c.dnb = b->d_norm_b;
    c.rows = rows;
    c.n = b->outputs;
    c.splits = splits;
    c.norm = b->norm;
    c.call = ctx->calls;
    c.gen = rewrite_gen(b->d_prenorm);
    c.valid = true;
}

bool overlaps(const void *a, size_t an, const void *b, size_t bn) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return a && b && x < y + bn && y < x + an;
}

bool cols_match(const skl_ctx *ctx, const skl_dense_desc *b, uint32_t rows) {
    const ColSums &c = ctx->cs;
    return c.valid && c.call + 1 >= ctx->calls && c.dp == b->d_prenorm && c.rows == rows && c.n == b->outputs &&
           c.norm == b->norm && (b->norm == SKL_NORM_DISABLED || (c.dnw == b->d_norm_w && c.dnb == b->d_norm_b)) &&
           c.gen == rewrite_gen(b->d_prenorm);
}

uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1) / m * m; }

// An error entry point rewrote d_prenorm_h: its padded copy is stale.
void pad_forget(skl_ctx *ctx, const void *src) {
    for (PadCopy &c : ctx->pads)
        if (c.src == src) c.valid = false;
}

// The current padded copy of a GEMM operand stored as [rows x cols] at pitch ld, if any.
const PadCopy *pad_copy_of(const skl_ctx *ctx, const void *p, uint32_t rows, uint32_t cols, uint32_t ld) {
    for (const PadCopy &c : ctx->pads)
        if (c.valid && c.src == p && c.rows == rows && c.n == cols && ld == cols && c.call + 1 >= ctx->calls &&
            c.gen == rewrite_gen(p))
            return &c;
    return nullptr;
}

// Pads d_prenorm_h p ([rows x cols] at pitch ld) into its slot (the one already
// mirroring p, else the least recently made) and records it; *out = nullptr
// when the copy would not suit the kernel's 32-bit operand offsets.
int32_t pad_keep(skl_ctx *ctx, const void *p, uint32_t rows, uint32_t cols, uint32_t ld, const PadCopy **out) {
    *out = nullptr;
    const uint32_t rows_p = round_up(rows, 256), ld_p = round_up(cols, 256);
    const size_t need = (size_t)rows_p * ld_p * sizeof(half_t);
    if (need >= (size_t(1) << 32)) return SKL_OK;
    PadCopy *c = &ctx->pads[0];
    for (PadCopy &s : ctx->pads) {
        if (s.src == p) {
            c = &s;
            break;
        }
        if (s.call < c->call) c = &s;
    }
    c->valid = false;
    if (need > c->bytes) {
        SKL_TRY(hipStreamSynchronize(ctx->stream));
        if (c->buf) SKL_TRY(hipFree(c->buf));
        c->buf = nullptr;
        c->bytes = 0;
        void *b = nullptr;
        SKL_TRY(hipMalloc(&b, need));
        c->buf = reinterpret_cast<half_t *>(b);
        c->bytes = need;
    }
    // every element of [rows_p x ld_p]: the source, then zeros
    SKL_TRY(launch_pad_h(p, rows, cols, ld, c->buf, rows_p, ld_p, ctx->stream));
    c->src = p;
    c->rows = rows;
    c->n = cols;
    c->ld = ld_p;
    c->call = ctx->calls;
    c->gen = rewrite_gen(p);
    c->valid = true;
    *out = c;
    return SKL_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- GEMM planning ------------------------------------------------------------------
// Every DenseBlock GEMM runs on the fastest path its shapes allow:
//  * the 256x256 direct-to-LDS kernel (fp16).  Operands it cannot read as
//    stored (M, N not whole 256 tiles, K not a multiple of 128, rows not
//    16-byte aligned) are first copied into the workspace zero-padded to those
//    multiples, and the epilogue stops at the real M x N.  Used when the padded
//    output wastes at most half of its grid and there are at least 192 tiles,
//    counting the split-K slices a dW with fewer tiles than CUs is given (their
//    fp32 partial sums, in the workspace, are reduced by the optimiser kernel).
//  * the register-staged kernels otherwise (fp32; small or skinny fp16), with
//    the same split-K for small dW grids.
struct GemmPlan {
    bool skinny;               // N <= 16: the streaming kernels (forward, dW partials)
    bool dma;
    bool pad_a, pad_b;
    uint32_t tile;             // direct-to-LDS output tile edge (128 or 256); 128: fp32 dW on 128x128 tiles
    uint32_t band;             // > 0: rows [0, band) on 256x256 tiles, the rest on 128x128 (two launches)
    uint32_t Mp, Np, Kp;       // dims the kernel runs on
    uint32_t splits;           // split-K slices of a dW (then DwPartial + reduce)
    size_t a_bytes, b_bytes, part_bytes;
    size_t bytes() const { return a_bytes + b_bytes + part_bytes; }
};

// A stored operand the DMA kernel can read in place: rows x cols (k-contiguous:
// rows = m or n, cols = k; else rows = k, cols = m or n) with whole tiles.
bool dma_operand_ok(const void *p, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t rows_mult,
                    uint32_t cols_mult) {
    return rows % rows_mult == 0 && cols % cols_mult == 0 && ld % 8 == 0 && aligned16(p);
}

// Split-K slices for a dW grid of `tiles` 256x256 tiles over Kp (slices of at
// least 512 k, at most 16): the count with the least estimated time, with one
// workgroup per CU (256 CUs: a grid of w workgroups runs in ceil(w / 256)
// rounds, each as long as one slice, ~3.4 us per 128 k as measured on the C3 dW
// kernel) plus the fp32 partial planes the slices write and the optimiser kernel
// reads back (8 bytes per element and slice at ~5 TB/s).  A count that just
// overflows a round loses to one fewer slice: 72 tiles take 3 slices (216
// workgroups, one round), not 4 (288, two rounds).  *tile: the same choice
// over 128x128 tiles (two workgroups per CU, a round of 512 taking half a
// 256x256 round's time per slice, times 1.25 for that kernel on the dW layout)
// when that is faster: C5's 1024 x 1536 dW (24 tiles) on 128x128 tiles in 5
// slices, 17 us faster than 256x256 in 10; C4's 2048 x 2048 dW stays on
// 256x256 in 4 slices (128x128 in 2: +26 us a layer).
uint32_t dw_dma_splits(uint32_t tiles, uint32_t Kp, uint64_t out_elems, uint32_t *tile) {
    constexpr uint32_t kCus = 256;
    uint32_t best = 1;
    double best_us = 0.0;
    *tile = 256;
    for (uint32_t t : {256u, 128u}) {
        const uint32_t wg = t == 256 ? tiles : 4 * tiles;      // workgroups per slice
        const uint32_t per_round = t == 256 ? kCus : 2 * kCus;
        const double slice_scale = t == 256 ? 1.0 : 0.5 * 1.25;
        for (uint32_t req = 1; req <= 16 && (req == 1 || req <= Kp / 512); ++req) {
            const uint32_t sp = gemm_dma_splits(Kp, req);
            const uint32_t kps = ((Kp / req + 127) / 128) * 128;   // launch_gemm_dma's slice length
            const uint32_t rounds = (wg * sp + per_round - 1) / per_round;
            const double us = rounds * (kps / 128.0) * 3.4 * slice_scale +
                              (sp > 1 ? sp * (double)out_elems * 8.0 / 5.0e6 : 0.0);
            if ((t == 256 && req == 1) || us < best_us) {
                best = sp;
                best_us = us;
                *tile = t;
            }
        }
    }
    return best;
}

// Output tile edge for a direct-to-LDS GEMM of Mp x Np (multiples of 256): the
// one with fewer estimated rounds of work.  A round is 256 workgroups of 256x256
// (one per CU) or 512 of 128x128 (two per CU); measured on the C3 shapes, the
// 128x128 kernel does the same work 1.09-1.15x slower (1.23x with the Adam
// epilogue), so it wins only where the 256x256 grid leaves most of its last
// round empty (C5's 12544 x 1536 hidden error: 294 tiles, 2 rounds for 1.15
// of work; 0.151 -> 0.130 ms).  Split-K grids keep 256.
// *band (forward and dX sums): a third choice, the first rows of the grid on
// 256x256 tiles in at least two whole rounds and the remaining rows on
// 128x128 tiles in a second launch, when that is estimated faster still.
// Measured on C5's 12544 x 3072 forward (588 tiles): 142 us on 256x256, 141
// on 128x128, 132 as 2 rounds + 84 tiles' worth of 128x128 rows; on its
// 12544 x 1536 GEMMs (294 tiles) one 256x256 round plus a 128x128 launch ran
// 3-4 us slower than 128x128 alone (a launch of fewer 128x128 workgroups than
// CUs takes as long as a full round of them), hence two rounds at least.
uint32_t dma_tile(Op op, uint32_t Mp, uint32_t Np, uint32_t splits, uint32_t *band) {
    *band = 0;
    if (const uint32_t f = gemm_dma_tile_forced()) return f;
    if (splits > 1) return 256;
    const uint32_t R = Mp / 256, Cn = Np / 256;   // 256x256 tile rows and columns
    const double f128 = op == Op::DwOpt ? 1.25 : 1.15;
    auto rounds256 = [](double tiles) { return std::ceil(tiles / 256.0); };
    auto rounds128 = [&](double tiles256) { return std::ceil(4.0 * tiles256 / 512.0) * 0.5 * f128; };
    const double r256 = rounds256((double)R * Cn), r128 = rounds128((double)R * Cn);
    const uint32_t tile = r128 < 0.95 * r256 ? 128u : 256u;
    if (op != Op::Fwd && op != Op::InputGrad) return tile;
    double best = tile == 128 ? r128 : r256;
    uint32_t best_rows = 0;
    for (uint32_t k = 2; k < (uint32_t)r256; ++k) {
        uint32_t r1 = 256u * k / Cn;   // tile rows filling k rounds
        if (r1 >= R) r1 = R - 1;
        if (r1 == 0) continue;
        const double t = rounds256((double)r1 * Cn) + rounds128((double)(R - r1) * Cn);
        if (t < 0.95 * best) {
            best = t;
            best_rows = r1;
        }
    }
    if (best_rows == 0) return tile;
    *band = best_rows * 256u;
    return 256u;
}

GemmPlan plan_gemm(const GemmLaunch &g) {
    GemmPlan p{};
    p.tile = 256;
    p.splits = 1;
    p.Mp = g.M;
    p.Np = g.N;
    p.Kp = g.K;
    const bool dw = g.op == Op::DwOpt;
    // skinny outputs: a stream over X beats any MFMA tile that is >90% padding
    if (g.N <= 16 && g.M && g.K && ((g.op == Op::Fwd && skinny_fwd_ok(g)) || (dw && g.b32 && !g.a_kcontig))) {
        p.skinny = true;
        if (dw) {
            p.splits = skinny_dw_slices(g.K, g.M);
            p.part_bytes = (size_t)p.splits * g.M * 16 * sizeof(float);
        }
        return p;
    }
    if (g.dtype == SKL_F16 && gemm_dma_enabled() && g.M && g.N && g.K) {
        const uint32_t Mp = round_up(g.M, 256), Np = round_up(g.N, 256), Kp = round_up(g.K, 128);
        // in units of 256x256 tiles whatever the kernel's tile edge
        const uint32_t tiles = (Mp / 256) * (Np / 256);
        uint32_t dw_tile = 256;
        const uint32_t splits = dw && tiles < 160 ? dw_dma_splits(tiles, Kp, (uint64_t)Mp * Np, &dw_tile) : 1;
        const bool waste_ok = (uint64_t)Mp * Np <= (uint64_t)g.M * g.N * 3 / 2;
        // the kernel's operand offsets are 32-bit
        const uint64_t a_span = g.a_kcontig ? (uint64_t)Mp * (g.lda > Kp ? g.lda : Kp)
                                            : (uint64_t)Kp * (g.lda > Mp ? g.lda : Mp);
        const uint64_t b_span = g.b_kcontig ? (uint64_t)Np * (g.ldb > Kp ? g.ldb : Kp)
                                            : (uint64_t)Kp * (g.ldb > Np ? g.ldb : Np);
        const bool offsets_ok = a_span * 2 < (1ull << 32) && b_span * 2 < (1ull << 32);
        // enough workgroups to fill the GPU: 192 of 256x256, or 384 of 128x128 (two per CU)
        const uint32_t fill = dw_tile == 128 ? 4 * tiles * splits / 2 : tiles * splits;
        if (waste_ok && offsets_ok && fill >= 192) {
            p.dma = true;
            p.Mp = Mp;
            p.Np = Np;
            p.Kp = Kp;
            p.splits = splits;
            p.tile = dma_tile(g.op, Mp, Np, splits, &p.band);
            if (dw && dw_tile == 128 && !gemm_dma_tile_forced()) p.tile = 128;
            // A: k-contiguous [M x K] or m-contiguous [K x M]; B likewise with N
            p.pad_a = g.a_kcontig ? !dma_operand_ok(g.A, g.M, g.K, g.lda, 256, 128)
                                  : !dma_operand_ok(g.A, g.K, g.M, g.lda, 128, 256);
            p.pad_b = g.b_kcontig ? !dma_operand_ok(g.B, g.N, g.K, g.ldb, 256, 128)
                                  : !dma_operand_ok(g.B, g.K, g.N, g.ldb, 128, 256);
            // 256-byte aligned regions
            p.a_bytes = p.pad_a ? ((size_t)Mp * Kp * 2 + 255) & ~(size_t)255 : 0;
            p.b_bytes = p.pad_b ? ((size_t)Np * Kp * 2 + 255) & ~(size_t)255 : 0;
            p.part_bytes = splits > 1 ? (size_t)splits * Mp * Np * sizeof(float) : 0;
            return p;
        }
    }
    // register-staged kernels; split-K for small dW grids
    if (dw) {
        uint32_t tiles = gemm_tiles(g.dtype, g.M, g.N);
        const uint32_t bk = gemm_bk(g.dtype);
        // fp32: 128x128 tiles split over the batch rather than the 64x64 tiles a
        // small grid would otherwise get (C2's 1024 x 1024 dW over 4096 rows: 4
        // slices of 64 tiles, 103 -> 77 us, against 256 whole 64x64 tiles)
        const uint32_t t128 = ((g.M + 127) / 128) * ((g.N + 127) / 128);
        if (g.dtype == SKL_F32 && t128 < 160 && g.K >= 8 * 4 * bk) {
            tiles = t128;
            p.tile = 128;
        }
        if (tiles < 160 && g.K >= 8 * bk) {
            uint32_t splits = (256 + tiles - 1) / tiles;
            const uint32_t max_splits = g.K / (4 * bk);
            if (splits > max_splits) splits = max_splits;
            if (splits > 16) splits = 16;
            if (splits >= 2) {
                p.splits = splits;
                p.part_bytes = (size_t)splits * g.M * g.N * sizeof(float);
            }
        }
    }
    return p;
}

enum class GemmKind { Dma, Staged, SkinnyFwd, SkinnyDw };

// One GEMM launch; when skl_ctx_time_next_gemm armed a pair of events, the GEMM
// kernel's own dispatch records them (no marker packets in the stream).
hipError_t timed_gemm(skl_ctx *ctx, const GemmLaunch &g0, GemmKind kind, float *partials = nullptr,
                      uint32_t slices = 0) {
    GemmLaunch g = g0;
    g.time_start = ctx->gemm_start;
    g.time_stop = ctx->gemm_stop;
    ctx->gemm_start = ctx->gemm_stop = nullptr;
    switch (kind) {
    case GemmKind::Dma: return launch_gemm_dma(g, ctx->stream);
    case GemmKind::Staged: return launch_gemm(g, ctx->stream);
    case GemmKind::SkinnyFwd: return launch_skinny_fwd(g, ctx->stream);
    case GemmKind::SkinnyDw: return launch_skinny_dw(g, partials, slices, ctx->stream);
    }
    return hipSuccess;
}

// Runs g as planned; ws holds plan.bytes() of workspace.  full_out: the output
// buffer has room for the padded grid (p.Mp x p.Np at its ldc), so the kernel
// may write all of it (rows and columns past M, N come out zero).
// vec (a dW only): the bias / norm-parameter update to run inside the split-K
// reduction's launch or the fused direct-to-LDS kernel when there is one;
// *vec_done says whether it ran.  keep: KEEP_A / KEEP_B, the operand is a
// d_prenorm_h whose padded copy goes to the context's PadCopy slots.
enum : uint32_t { KEEP_A = 1, KEEP_B = 2 };
int32_t exec_gemm(skl_ctx *ctx, GemmLaunch g, const GemmPlan &p, char *ws, bool full_out = false,
                  const VecOptArgs *vec = nullptr, bool *vec_done = nullptr, uint32_t keep = 0) {
    if (vec_done) *vec_done = false;
    char *wa = ws, *wb = ws + p.a_bytes, *wpart = ws + p.a_bytes + p.b_bytes;
    const OptEpi oe = g.opt;
    const uint32_t M = g.M, N = g.N;
    if (p.skinny) {
        if (g.op == Op::Fwd) return hip_status(timed_gemm(ctx, g, GemmKind::SkinnyFwd));
        SKL_TRY(timed_gemm(ctx, g, GemmKind::SkinnyDw, reinterpret_cast<float *>(wpart), p.splits));
        DwReduceArgs d{};
        d.dtype = g.dtype;
        d.rows = M;
        d.n = N;
        d.splits = p.splits;
        d.partials = reinterpret_cast<const float *>(wpart);
        d.plane = (uint64_t)M * 16;
        d.pld = 16;
        d.e = oe;
        if (vec) {
            d.with_vec = 1;
            d.vec = *vec;
        }
        SKL_TRY(launch_dw_reduce_opt(d, ctx->stream));
        if (vec_done) *vec_done = vec != nullptr;
        return SKL_OK;
    }
    if (p.dma) {
        // a d_prenorm_h padded by the GEMM before (or padded now into a kept slot),
        // else a padded copy in the workspace
        if (p.pad_a) {
            const uint32_t rows = g.a_kcontig ? g.M : g.K, cols = g.a_kcontig ? g.K : g.M;
            const PadCopy *c = pad_copy_of(ctx, g.A, rows, cols, g.lda);
            if (!c && (keep & KEEP_A) && ctx->keep_pads) {
                const int32_t r = pad_keep(ctx, g.A, rows, cols, g.lda, &c);
                if (r) return r;
            }
            if (c) {
                g.A = c->buf;
                g.lda = c->ld;
            } else {
                if (g.a_kcontig)
                    SKL_TRY(launch_pad_h(g.A, g.M, g.K, g.lda, wa, p.Mp, p.Kp, ctx->stream));
                else
                    SKL_TRY(launch_pad_h(g.A, g.K, g.M, g.lda, wa, p.Kp, p.Mp, ctx->stream));
                g.A = wa;
                g.lda = g.a_kcontig ? p.Kp : p.Mp;
            }
        }
        if (p.pad_b) {
            const uint32_t rows = g.b_kcontig ? g.N : g.K, cols = g.b_kcontig ? g.K : g.N;
            const PadCopy *c = pad_copy_of(ctx, g.B, rows, cols, g.ldb);
            if (!c && (keep & KEEP_B) && ctx->keep_pads) {
                const int32_t r = pad_keep(ctx, g.B, rows, cols, g.ldb, &c);
                if (r) return r;
            }
            if (c) {
                g.B = c->buf;
                g.ldb = c->ld;
            } else {
                if (g.b_kcontig)
                    SKL_TRY(launch_pad_h(g.B, g.N, g.K, g.ldb, wb, p.Np, p.Kp, ctx->stream));
                else
                    SKL_TRY(launch_pad_h(g.B, g.K, g.N, g.ldb, wb, p.Kp, p.Np, ctx->stream));
                g.B = wb;
                g.ldb = g.b_kcontig ? p.Kp : p.Np;
            }
        }
        g.mv = full_out ? p.Mp : M;
        g.nv = full_out ? p.Np : N;
        g.tile = p.tile;
        if (vec && g.op == Op::DwOpt && p.splits == 1) {
            // the bias / norm-parameter update rides in the fused kernel's launch;
            // its 64 NW threads take cpb columns each with the lanes per column of a
            // 256-thread vec_opt_kernel, so every column is summed in the same order
            // as there (and in the split-K reduction's launch)
            g.opt.vec = *vec;
            g.opt.vec.cpb = vec_opt_cpb(vec->splits) * (p.tile == 128 ? 1u : 2u);
            g.opt.vec_blocks = (vec->n + g.opt.vec.cpb - 1) / g.opt.vec.cpb;
            if (vec_done) *vec_done = true;
        }
        g.M = p.Mp;
        g.N = p.Np;
        g.K = p.Kp;
        if (p.splits > 1) {
            // fp32 partial planes on the padded grid; the optimiser kernel adds them up
            g.op = Op::DwPartial;
            g.splits = p.splits;
            g.st.out = reinterpret_cast<float *>(wpart);
            g.st.split_stride = (uint64_t)p.Mp * p.Np;
            g.st.ldc = p.Np;
            g.mv = g.M;
            g.nv = g.N;
        }
        if (p.band && (g.op == Op::Fwd || g.op == Op::InputGrad)) {
            // rows [0, band) on 256x256 tiles, the rest on 128x128; the timing
            // events, when armed, bracket both launches
            GemmLaunch g1 = g, g2 = g;
            g1.tile = 256;
            g1.m_begin = 0;
            g1.m_rows = p.band;
            g1.time_start = ctx->gemm_start;
            g2.tile = 128;
            g2.m_begin = p.band;
            g2.m_rows = p.Mp - p.band;
            g2.time_stop = ctx->gemm_stop;
            ctx->gemm_start = ctx->gemm_stop = nullptr;
            SKL_TRY(launch_gemm_dma(g1, ctx->stream));
            SKL_TRY(launch_gemm_dma(g2, ctx->stream));
        } else {
            SKL_TRY(timed_gemm(ctx, g, GemmKind::Dma));
        }
    } else {
        if (p.splits > 1) {
            g.op = Op::DwPartial;
            g.splits = p.splits;
            g.st.out = reinterpret_cast<float *>(wpart);
            g.st.split_stride = (uint64_t)M * N;
            g.st.ldc = N;
        }
        g.tile = p.tile;
        SKL_TRY(timed_gemm(ctx, g, GemmKind::Staged));
    }
    if (p.splits > 1) {
        DwReduceArgs d{};
        d.dtype = g.dtype;
        d.rows = M;
        d.n = N;
        d.splits = p.splits;
        d.partials = reinterpret_cast<const float *>(wpart);
        d.plane = p.dma ? (uint64_t)p.Mp * p.Np : (uint64_t)M * N;
        d.pld = p.dma ? p.Np : N;
        d.e = oe;
        if (vec) {
            d.with_vec = 1;
            d.vec = *vec;
        }
        SKL_TRY(launch_dw_reduce_opt(d, ctx->stream));
        if (vec_done) *vec_done = vec != nullptr;
    }
    return SKL_OK;
}

// Common configuration checks of a block descriptor.
int32_t check_desc(const skl_ctx *ctx, const skl_dense_desc *b) {
    SKL_CHECK(b, SKL_ERR_NULL_POINTER);
    SKL_CHECK(b->dtype <= SKL_F16, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(b->inputs > 0 && b->outputs > 0, SKL_ERR_INVALID_CONFIGURATION);   // mlp.rs:350-354
    SKL_CHECK(b->max_batch > 0, SKL_ERR_INVALID_CONFIGURATION);                  // mlp.rs:356-360
    SKL_CHECK(b->norm <= SKL_NORM_BATCH, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(b->act <= SKL_ACT_MISH, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(b->regularisation <= SKL_REGU_L2, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(b->w, SKL_ERR_NULL_POINTER);
    return SKL_OK;
}

// check_tile_dim (device.rs:248-258).  The reference runs it in gpu_forward_pass
// (ffn_device.rs:20) and gpu_hidden_layer_backward_pass (ffn_device.rs:369) only,
// after the DenseBlock method's own checks; the same calls here check it at the
// same point, and the output error and output-layer backward do not.
int32_t check_tile(const skl_ctx *ctx, const skl_dense_desc *b) {
    SKL_CHECK(!(b->dtype == SKL_F16 && ctx->tile_dim != 16), SKL_ERR_HARDWARE_CONSTRAINT);
    return SKL_OK;
}

// check_input_dimension (mlp.rs:492-519)
int32_t check_input(const skl_dense_desc *b, const void *in, uint32_t in_rows, uint32_t in_cols, uint32_t batch) {
    SKL_CHECK(in, SKL_ERR_NULL_POINTER);
    SKL_CHECK(in_rows >= batch, SKL_ERR_MISMATCHED_DIMENSIONS);
    SKL_CHECK(in_rows <= b->max_batch, SKL_ERR_ALLOCATION_LIMIT);
    SKL_CHECK(in_cols == b->inputs, SKL_ERR_MISMATCHED_DIMENSIONS);
    return SKL_OK;
}

// Softmax / batch-size checks shared by forward and the backward calls
// (mlp.rs:558-575, 620-639, 710-726).
int32_t check_act_batch(const skl_dense_desc *b, uint32_t batch) {
    SKL_CHECK(b->act != SKL_ACT_SOFTMAX, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(batch > 0, SKL_ERR_INVALID_BATCH_SIZE);
    SKL_CHECK(!(b->norm == SKL_NORM_BATCH && batch == 1), SKL_ERR_INVALID_BATCH_SIZE);
    return SKL_OK;
}

int32_t check_norm_cache(const skl_dense_desc *b) {
    if (b->norm == SKL_NORM_DISABLED) return SKL_OK;
    SKL_CHECK(b->prenorm && b->centered && b->norm_rstd && b->norm_w && b->norm_b, SKL_ERR_NULL_POINTER);
    return SKL_OK;
}

int32_t check_backward_buffers(const skl_dense_desc *b) {
    SKL_CHECK(b->grad && b->d_prenorm, SKL_ERR_NULL_POINTER);
    if (b->dtype == SKL_F16) SKL_CHECK(b->d_prenorm_h, SKL_ERR_NULL_POINTER);
    if (b->norm != SKL_NORM_DISABLED) SKL_CHECK(b->d_norm_w && b->d_norm_b, SKL_ERR_NULL_POINTER);
    return check_norm_cache(b);
}

const float *master_norm_w(const skl_dense_desc *b) {
    return b->dtype == SKL_F16 ? b->master_norm_w : reinterpret_cast<const float *>(b->norm_w);
}

OptParams opt_params(const skl_optimiser &o, uint32_t step) {
    OptParams p;
    p.kind = o.kind;
    p.beta1 = o.beta1;
    p.beta2 = o.beta2;
    p.epsilon = o.epsilon;
    p.nesterov = o.nesterov;
    // backward.cu:141-142 (powf(beta, step)); step 0 divides by zero there too
    p.bc1 = 1.0f - powf(o.beta1, (float)step);
    p.bc2 = 1.0f - powf(o.beta2, (float)step);
    return p;
}

// The reference zero-fills dNorm before every backward kernel
// (ffn_device.rs:148-149, 370-371) and the kernels then write rows [0, rows).
// Only the rows no kernel writes need the fill.  With norm Disabled the
// buffers are never written at all (they keep the zeros of allocation,
// mlp.rs:404-410), so nothing is launched.
int32_t zero_dnorm_tail(skl_ctx *ctx, const skl_dense_desc *b, uint32_t rows_written) {
    if (b->norm == SKL_NORM_DISABLED || rows_written >= b->max_batch) return SKL_OK;
    const size_t off = (size_t)rows_written * b->outputs;
    const size_t n = (size_t)(b->max_batch - rows_written) * b->outputs;
    SKL_TRY(launch_fill(b->d_norm_w + off, SKL_F32, 0.0f, n, ctx->stream));
    SKL_TRY(launch_fill(b->d_norm_b + off, SKL_F32, 0.0f, n, ctx->stream));
    return SKL_OK;
}

}  // namespace

extern "C" {

const char *skl_status_string(int32_t s) {
    switch (s) {
    case SKL_OK: return "ok";
    case SKL_ERR_INVALID_CONFIGURATION: return "invalid configuration";
    case SKL_ERR_TRAINING_MODE_REQUIRED: return "training mode required";
    case SKL_ERR_ALLOCATION_LIMIT: return "allocation limit exceeded (batch, or an allocation-free call's scratch)";
    case SKL_ERR_MISMATCHED_DIMENSIONS: return "mismatched dimensions";
    case SKL_ERR_INVALID_BATCH_SIZE: return "invalid batch size";
    case SKL_ERR_HARDWARE_CONSTRAINT: return "hardware constraint violation (fp16 requires tile_dim 16)";
    case SKL_ERR_TRY_FROM_INT: return "integer conversion overflow";
    case SKL_ERR_NULL_POINTER: return "required pointer is null";
    case SKL_ERR_UNSUPPORTED_CAST: return "unsupported precision cast";
    case SKL_ERR_NO_DEVICE: return "no usable device";
    default: return s > 0 ? hipGetErrorString((hipError_t)s) : "unknown status";
    }
}

int32_t skl_ctx_create(int32_t ordinal, uint32_t tile_dim, skl_ctx **out) {
    if (!out) return SKL_ERR_NULL_POINTER;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || ordinal < 0 || ordinal >= count) return SKL_ERR_NO_DEVICE;
    if (tile_dim == 0) return SKL_ERR_INVALID_CONFIGURATION;
    SKL_TRY(hipSetDevice(ordinal));
    skl_ctx *c = new skl_ctx();
    c->device = ordinal;
    c->tile_dim = tile_dim;
    c->sync = 1;
    c->ws = nullptr;
    c->ws_bytes = 0;
    {
        // SOKLYN_PAD_KEEP=0: no kept padded copies (A/B comparisons)
        const char *e = getenv("SOKLYN_PAD_KEEP");
        c->keep_pads = !(e && atoi(e) == 0);
    }
    {
        const int32_t sr = scratch_address(ordinal, &c->scratch);
        if (sr != SKL_OK) {
            delete c;
            return sr;
        }
    }
    // blocking w.r.t. the legacy null stream, so callers on stream 0 stay ordered
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamDefault);
    if (e != hipSuccess) {
        delete c;
        return hip_status(e);
    }
    c->stream = c->own_stream;
    *out = c;
    return SKL_OK;
}

int32_t skl_ctx_destroy(skl_ctx *ctx) {
    if (!ctx) return SKL_ERR_NULL_POINTER;
    // every release is attempted; the first failure is reported
    hipError_t first = hipSuccess;
    auto note = [&](hipError_t e) {
        if (first == hipSuccess && e != hipSuccess) first = e;
    };
    note(hipSetDevice(ctx->device));
    note(hipStreamSynchronize(ctx->stream));
    if (ctx->ws) note(hipFree(ctx->ws));
    if (ctx->cols) note(hipFree(ctx->cols));
    for (PadCopy &c : ctx->pads)
        if (c.buf) note(hipFree(c.buf));
    note(hipStreamDestroy(ctx->own_stream));
    delete ctx;
    return first == hipSuccess ? SKL_OK : hip_status(first);
}

int32_t skl_ctx_set_sync(skl_ctx *ctx, uint32_t sync_each_call) {
    if (!ctx) return SKL_ERR_NULL_POINTER;
    ctx->sync = sync_each_call ? 1 : 0;
    return SKL_OK;
}

int32_t skl_ctx_time_next_gemm(skl_ctx *ctx, void *start_event, void *stop_event) {
    if (!ctx) return SKL_ERR_NULL_POINTER;
    if (!start_event != !stop_event) return SKL_ERR_NULL_POINTER;
    ctx->gemm_start = reinterpret_cast<hipEvent_t>(start_event);
    ctx->gemm_stop = reinterpret_cast<hipEvent_t>(stop_event);
    return SKL_OK;
}

int32_t skl_ctx_set_stream(skl_ctx *ctx, void *hip_stream) {
    if (!ctx) return SKL_ERR_NULL_POINTER;
    ctx->stream = hip_stream ? reinterpret_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    return SKL_OK;
}

void *skl_ctx_stream(skl_ctx *ctx) { return ctx ? reinterpret_cast<void *>(ctx->stream) : nullptr; }

int32_t skl_synchronize(skl_ctx *ctx) {
    int32_t r = enter(ctx);
    if (r) return r;
    SKL_TRY(hipStreamSynchronize(ctx->stream));
    return SKL_OK;
}

int32_t skl_malloc(skl_ctx *ctx, void **ptr, size_t bytes) {
    int32_t r = enter(ctx);
    if (r) return r;
    if (!ptr) return SKL_ERR_NULL_POINTER;
    *ptr = nullptr;
    SKL_TRY(hipMalloc(ptr, bytes ? bytes : 1));
    return SKL_OK;
}

int32_t skl_free(skl_ctx *ctx, void *ptr) {
    int32_t r = enter(ctx);
    if (r) return r;
    if (!ptr) return SKL_OK;
    SKL_TRY(hipStreamSynchronize(ctx->stream));
    SKL_TRY(hipFree(ptr));
    return SKL_OK;
}

static int32_t copy(skl_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
    int32_t r = enter(ctx);
    if (r) return r;
    if (bytes == 0) return SKL_OK;
    if (!dst || !src) return SKL_ERR_NULL_POINTER;
    SKL_TRY(hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    SKL_TRY(hipStreamSynchronize(ctx->stream));
    return SKL_OK;
}

int32_t skl_memcpy_h2d(skl_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyHostToDevice);
}
int32_t skl_memcpy_d2h(skl_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost);
}
int32_t skl_memcpy_d2d(skl_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice);
}

int32_t skl_fill(skl_ctx *ctx, void *dst, uint32_t dtype, float v, size_t n) {
    int32_t r = enter(ctx);
    if (r) return r;
    if (dtype > SKL_F16) return SKL_ERR_INVALID_CONFIGURATION;
    if (n && !dst) return SKL_ERR_NULL_POINTER;
    SKL_TRY(launch_fill(dst, dtype, v, n, ctx->stream));
    return finish(ctx);
}

int32_t skl_cast(skl_ctx *ctx, const void *src, uint32_t sdt, void *dst, uint32_t ddt, size_t n) {
    int32_t r = enter(ctx);
    if (r) return r;
    // gpu_cast_t (util_device.rs:23-32) knows f32 -> f16 and f16 -> f32 only
    if (sdt > SKL_F16 || ddt > SKL_F16 || sdt == ddt) return SKL_ERR_UNSUPPORTED_CAST;
    if (n && (!src || !dst)) return SKL_ERR_NULL_POINTER;
    SKL_TRY(launch_cast(src, sdt, dst, ddt, n, ctx->stream));
    return finish(ctx);
}

uint32_t skl_scramble_seed(uint32_t step, uint32_t layer_id) {
    uint32_t h = step * 1103515245u + layer_id;
    h = (h ^ (h >> 16)) * 1103515245u;
    return h ^ (h >> 15);
}

int32_t skl_dense_forward(skl_ctx *ctx, const skl_dense_desc *b, const void *in, uint32_t in_rows,
                          uint32_t in_cols, uint32_t batch, uint32_t use_dropout, uint32_t seed) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = check_desc(ctx, b))) return r;
    if ((r = check_input(b, in, in_rows, in_cols, batch))) return r;   // mlp.rs:549
    if ((r = check_act_batch(b, batch))) return r;                    // mlp.rs:551-568
    if ((r = check_tile(ctx, b))) return r;                           // ffn_device.rs:20
    if ((r = check_norm_cache(b))) return r;
    SKL_CHECK(b->out && b->predrop && b->preact, SKL_ERR_NULL_POINTER);
    const bool use_bias = b->norm != SKL_NORM_BATCH;   // ffn_device.rs:30
    SKL_CHECK(!use_bias || b->b, SKL_ERR_NULL_POINTER);
    SKL_CHECK(!use_dropout || b->mask, SKL_ERR_NULL_POINTER);

    GemmLaunch g{};
    g.dtype = b->dtype;
    g.M = batch;
    g.N = b->outputs;
    g.K = b->inputs;
    g.lda = in_cols;
    g.ldb = b->outputs;
    g.a_kcontig = true;
    g.b_kcontig = false;
    g.A = in;
    g.B = b->w;
    g.splits = 1;
    g.op = Op::Fwd;
    g.fwd.bias = use_bias ? b->b : nullptr;
    g.fwd.z_out = b->norm == SKL_NORM_DISABLED ? b->preact : b->prenorm;   // ffn_device.rs:51-55
    g.fwd.predrop = b->predrop;
    g.fwd.out = b->out;
    g.fwd.mask = b->mask;
    g.fwd.fuse_act = b->norm == SKL_NORM_DISABLED;
    g.fwd.act = b->act;
    g.fwd.use_dropout = use_dropout ? 1 : 0;
    g.fwd.seed = seed;
    g.fwd.leaky = b->act == SKL_ACT_LEAKY_RELU ? b->leaky : 0.0f;       // ffn_device.rs:32-35
    g.fwd.p = b->mask_coeff;
    g.fwd.ldc = b->outputs;
    const GemmPlan plan = plan_gemm(g);
    if ((r = ensure_ws(ctx, plan.bytes()))) return r;
    if ((r = exec_gemm(ctx, g, plan, reinterpret_cast<char *>(ctx->ws)))) return r;

    if (b->norm != SKL_NORM_DISABLED) {
        RowNormArgs a{};
        a.dtype = b->dtype;
        a.m = batch;
        a.n = b->outputs;
        a.norm = b->norm;
        a.act = b->act;
        a.use_dropout = use_dropout ? 1 : 0;
        a.seed = seed;
        a.leaky = g.fwd.leaky;
        a.p = b->mask_coeff;
        a.prenorm = b->prenorm;
        a.norm_w = b->norm_w;
        a.norm_b = b->norm_b;
        a.centered = b->centered;
        a.preact = b->preact;
        a.predrop = b->predrop;
        a.out = b->out;
        a.mask = b->mask;
        a.norm_rstd = b->norm_rstd;
        SKL_TRY(launch_norm_act(a, ctx->stream));
    }
    return finish(ctx);
}

int32_t skl_dense_output_error(skl_ctx *ctx, const skl_dense_desc *b, const void *target, uint32_t target_rows,
                               uint32_t target_cols, uint32_t loss, uint32_t act, float leaky) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = check_desc(ctx, b))) return r;
    // compute_loss (mlp.rs:756-821)
    SKL_CHECK(b->is_training, SKL_ERR_TRAINING_MODE_REQUIRED);
    SKL_CHECK(target, SKL_ERR_NULL_POINTER);
    SKL_CHECK(target_cols == b->outputs, SKL_ERR_MISMATCHED_DIMENSIONS);
    SKL_CHECK(target_rows <= b->max_batch, SKL_ERR_ALLOCATION_LIMIT);
    SKL_CHECK(loss <= SKL_LOSS_BCE && act <= SKL_ACT_MISH, SKL_ERR_INVALID_CONFIGURATION);
    if (loss == SKL_LOSS_MSE) SKL_CHECK(act != SKL_ACT_SOFTMAX, SKL_ERR_INVALID_CONFIGURATION);
    if (loss == SKL_LOSS_CE) SKL_CHECK(act == SKL_ACT_SOFTMAX, SKL_ERR_INVALID_CONFIGURATION);
    if (loss == SKL_LOSS_BCE) SKL_CHECK(act == SKL_ACT_SIGMOID, SKL_ERR_INVALID_CONFIGURATION);
    if ((r = check_backward_buffers(b))) return r;
    SKL_CHECK(b->out && b->preact, SKL_ERR_NULL_POINTER);
    if (b->dtype == SKL_F16 && b->norm) SKL_CHECK(b->master_norm_w, SKL_ERR_NULL_POINTER);

    // The reference zero-fills all dNorm rows, then writes rows [0, m).
    if ((r = zero_dnorm_tail(ctx, b, target_rows))) return r;
    // Softmax in place on out over all cache rows (ffn_device.rs:167-186).
    if (act == SKL_ACT_SOFTMAX) SKL_TRY(launch_softmax(b->dtype, b->out, b->max_batch, b->outputs, ctx->stream));

    ErrArgs a{};
    a.dtype = b->dtype;
    a.rows = target_rows;   // kernel m = max_batch (Q: ffn_device.rs:152); rows past target_rows are not readable
    a.n = b->outputs;
    a.norm = b->norm;
    a.act = act;
    a.loss = loss;
    a.leaky = act == SKL_ACT_LEAKY_RELU ? leaky : 0.0f;
    a.inv_n = 1.0f / (float)b->outputs;
    a.inv_m = 1.0f / (float)b->max_batch;
    a.loss_scale = 512.0f;
    a.out = b->out;
    a.preact = b->preact;
    a.target = target;
    a.norm_rstd = b->norm_rstd;
    a.centered = b->centered;
    a.prenorm = b->prenorm;
    a.nw = master_norm_w(b);
    a.grad = b->grad;
    a.d_prenorm = b->d_prenorm;
    a.d_norm_w = b->d_norm_w;
    a.d_norm_b = b->d_norm_b;
    a.d_prenorm_h = b->dtype == SKL_F16 ? reinterpret_cast<half_t *>(b->d_prenorm_h) : nullptr;
    uint32_t splits = 0;
    if ((r = ensure_cols(ctx, b, target_rows, 0, &splits))) return r;
    note_rewrite(ctx, b);
    SKL_TRY(launch_output_error(a, ctx->cols, splits, ctx->stream));
    record_cols(ctx, b, target_rows, splits);
    return finish(ctx);
}

static int32_t hidden_error_impl(skl_ctx *ctx, const skl_dense_desc *cur, const skl_dense_desc *next,
                                 uint32_t batch) {
    int32_t r;
    if ((r = check_desc(ctx, cur))) return r;
    if ((r = check_desc(ctx, next))) return r;
    SKL_CHECK(cur->dtype == next->dtype, SKL_ERR_INVALID_CONFIGURATION);
    SKL_CHECK(cur->is_training, SKL_ERR_TRAINING_MODE_REQUIRED);                 // mlp.rs:682-686
    SKL_CHECK(next->inputs == cur->outputs, SKL_ERR_MISMATCHED_DIMENSIONS);      // mlp.rs:690-697
    SKL_CHECK(batch <= cur->max_batch, SKL_ERR_ALLOCATION_LIMIT);
    SKL_CHECK(next->max_batch >= batch, SKL_ERR_MISMATCHED_DIMENSIONS);          // mlp.rs:699-706
    if ((r = check_act_batch(cur, batch))) return r;
    if ((r = check_tile(ctx, cur))) return r;                                    // ffn_device.rs:369
    if ((r = check_backward_buffers(cur))) return r;
    SKL_CHECK(cur->predrop && cur->preact && cur->mask, SKL_ERR_NULL_POINTER);
    SKL_CHECK(next->d_prenorm, SKL_ERR_NULL_POINTER);
    if (cur->dtype == SKL_F16) {
        SKL_CHECK(next->d_prenorm_h, SKL_ERR_NULL_POINTER);
        if (cur->norm) SKL_CHECK(cur->master_norm_w, SKL_ERR_NULL_POINTER);
    }
    if ((r = zero_dnorm_tail(ctx, cur, batch))) return r;
    ctx->cs.valid = false;

    // act' * mask and the element-local norm gradient (backward.cu:79-100), with the
    // column sums of d_prenorm / dNorm for cur's backward
    ErrArgs a{};
    a.dtype = cur->dtype;
    a.rows = batch;
    a.n = cur->outputs;
    a.norm = cur->norm;
    a.act = cur->act;
    a.leaky = cur->act == SKL_ACT_LEAKY_RELU ? cur->leaky : 0.0f;
    a.inv_n = 1.0f / (float)cur->outputs;
    a.inv_m = 1.0f / (float)batch;
    a.loss_scale = 1.0f;
    a.predrop = cur->predrop;
    a.preact = cur->preact;
    a.mask = cur->mask;
    a.norm_rstd = cur->norm_rstd;
    a.centered = cur->centered;
    a.prenorm = cur->prenorm;
    a.nw = master_norm_w(cur);
    a.grad = cur->grad;
    a.d_prenorm = cur->d_prenorm;
    a.d_norm_w = cur->d_norm_w;
    a.d_norm_b = cur->d_norm_b;
    a.d_prenorm_h = cur->dtype == SKL_F16 ? reinterpret_cast<half_t *>(cur->d_prenorm_h) : nullptr;
    const void *next_dp = cur->dtype == SKL_F16 ? next->d_prenorm_h : next->d_prenorm;
    const uint32_t keep = cur->dtype == SKL_F16 ? KEEP_A : 0;   // next_dp is a d_prenorm_h
    note_rewrite(ctx, cur);

    // A next layer of at most 16 outputs: its GEMM would pad k to 128, so the
    // error kernel forms s = next.d_prenorm . next.W^T itself, per element, from
    // copies of the two operands padded to 16 columns (same operands as the
    // GEMM: f16(d_prenorm) and the working W for fp16 blocks).
    if (next->outputs <= 16) {
        uint32_t splits = 0;
        if ((r = ensure_cols(ctx, cur, batch, 2, &splits))) return r;
        const size_t esz = cur->dtype == SKL_F16 ? 2 : 4;
        const size_t a_bytes = ((size_t)batch * 16 * esz + 255) & ~(size_t)255;
        if ((r = ensure_ws(ctx, a_bytes + (size_t)cur->outputs * 16 * esz))) return r;
        char *a16 = reinterpret_cast<char *>(ctx->ws), *w16 = a16 + a_bytes;
        a.sk_a = a16;
        a.sk_w = w16;
        if (err_skinny_ok(a, ctx->cols)) {
            SKL_TRY(launch_skinny_operands(cur->dtype, next_dp, batch, next->w, cur->outputs, next->outputs, a16, w16,
                                           ctx->stream));
            SKL_TRY(launch_error_skinny(a, ctx->cols, splits, ctx->stream));
            record_cols(ctx, cur, batch, splits);
            return SKL_OK;
        }
        a.sk_a = a.sk_w = nullptr;
    }

    // s = next.d_prenorm . next.W^T into the workspace (backward.cu:72-77; fp16:
    // f16(d_prenorm) and the working W, == f16(master) after every update) ...
    GemmLaunch g{};
    g.dtype = cur->dtype;
    g.M = batch;
    g.N = cur->outputs;
    g.K = next->outputs;
    g.lda = next->outputs;
    g.ldb = next->outputs;
    g.a_kcontig = true;
    g.b_kcontig = true;
    g.A = next_dp;
    g.B = next->w;
    g.splits = 1;
    g.op = Op::InputGrad;
    const GemmPlan plan = plan_gemm(g);
    ErrEpi &e = g.err;
    // an operand act' does not read aliases the mask (loaded anyway: cache hits)
    e.predrop = act_uses_output(cur->act) ? cur->predrop : cur->mask;
    e.preact = act_uses_input(cur->act) ? cur->preact : cur->mask;
    e.mask = cur->mask;
    e.norm_rstd = cur->norm_rstd;
    e.centered = cur->centered;
    e.prenorm = cur->prenorm;
    e.nw = master_norm_w(cur);
    e.grad = cur->grad;
    e.d_prenorm = cur->d_prenorm;
    e.d_norm_w = cur->d_norm_w;
    e.d_norm_b = cur->d_norm_b;
    e.d_prenorm_h = reinterpret_cast<half_t *>(cur->d_prenorm_h);
    e.norm = cur->norm;
    e.act = cur->act;
    e.ldc = cur->outputs;
    e.ncols = cur->outputs;
    e.leaky = cur->act == SKL_ACT_LEAKY_RELU ? cur->leaky : 0.0f;
    e.inv_n = 1.0f / (float)cur->outputs;
    e.inv_m = 1.0f / (float)batch;
    if (plan.dma && hidden_err_fusable(e, batch, cur->outputs)) {
        // One kernel, as the reference has it (backward.cu:59-102): the 256x256
        // GEMM's epilogue computes the error from the sum in its accumulators
        // and leaves the column sums of each 256-row tile for cur's backward.
        const uint32_t tiles_m = plan.Mp / plan.tile;
        if ((r = ensure_cols_splits(ctx, tiles_m, cur->outputs))) return r;
        if ((r = ensure_ws(ctx, plan.bytes()))) return r;
        e.partials = ctx->cols;
        g.op = Op::HiddenErr;
        if ((r = exec_gemm(ctx, g, plan, reinterpret_cast<char *>(ctx->ws), false, nullptr, nullptr, keep))) return r;
        record_cols(ctx, cur, batch, tiles_m);
        return SKL_OK;
    }
    // s on the kernel's whole (padded) grid: the full-tile epilogue, 16-byte rows
    const uint32_t s_ld = plan.Np;
    const size_t s_bytes = ((size_t)plan.Mp * s_ld * sizeof(float) + 255) & ~(size_t)255;
    if ((r = ensure_ws(ctx, s_bytes + plan.bytes()))) return r;
    float *sum = reinterpret_cast<float *>(ctx->ws);
    g.st.out = sum;
    g.st.ldc = s_ld;
    if ((r = exec_gemm(ctx, g, plan, reinterpret_cast<char *>(ctx->ws) + s_bytes, true, nullptr, nullptr, keep)))
        return r;

    // ... then the error kernel on it
    a.s = sum;
    a.s_ld = s_ld;
    uint32_t splits = 0;
    if ((r = ensure_cols(ctx, cur, batch, 1, &splits))) return r;
    SKL_TRY(launch_error_from_sum(a, ctx->cols, splits, ctx->stream));
    record_cols(ctx, cur, batch, splits);
    return SKL_OK;
}

int32_t skl_dense_hidden_error(skl_ctx *ctx, const skl_dense_desc *cur, const skl_dense_desc *next,
                               uint32_t batch) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = hidden_error_impl(ctx, cur, next, batch))) return r;
    return finish(ctx);
}

static int32_t backward_impl(skl_ctx *ctx, const skl_dense_desc *b, const void *in, uint32_t in_rows,
                             uint32_t in_cols, const skl_train_ctx *t, uint32_t step) {
    int32_t r;
    if ((r = check_desc(ctx, b))) return r;
    SKL_CHECK(t, SKL_ERR_NULL_POINTER);
    SKL_CHECK(b->is_training, SKL_ERR_TRAINING_MODE_REQUIRED);                   // mlp.rs:614-618
    const uint32_t batch = t->batch_size;
    if ((r = check_input(b, in, in_rows, in_cols, batch))) return r;
    if ((r = check_act_batch(b, batch))) return r;
    if ((r = check_backward_buffers(b))) return r;
    SKL_CHECK(t->optimiser.kind <= SKL_OPT_ADAM && t->norm_optimiser.kind <= SKL_OPT_ADAM,
              SKL_ERR_INVALID_CONFIGURATION);
    const bool use_bias = b->norm != SKL_NORM_BATCH;   // ffn_device.rs:245
    const bool f16 = b->dtype == SKL_F16;
    SKL_CHECK(b->dv_w && b->dm_w, SKL_ERR_NULL_POINTER);
    if (f16) SKL_CHECK(b->master_w, SKL_ERR_NULL_POINTER);
    if (use_bias) {
        SKL_CHECK(b->b && b->dv_b && b->dm_b, SKL_ERR_NULL_POINTER);
        if (f16) SKL_CHECK(b->master_b, SKL_ERR_NULL_POINTER);
    }
    if (b->norm) {
        SKL_CHECK(b->dv_norm_w && b->dm_norm_w, SKL_ERR_NULL_POINTER);
        if (f16) SKL_CHECK(b->master_norm_w, SKL_ERR_NULL_POINTER);
        if (b->norm > 1) {
            SKL_CHECK(b->dv_norm_b && b->dm_norm_b, SKL_ERR_NULL_POINTER);
            if (f16) SKL_CHECK(b->master_norm_b, SKL_ERR_NULL_POINTER);
        }
    }

    const float inv_m = 1.0f / (float)batch;
    const uint32_t K = b->inputs, N = b->outputs;

    // -- dW = in^T . dP, fused with the optimiser step on W ----------------------------
    OptEpi oe{};
    oe.master = f16 ? b->master_w : reinterpret_cast<float *>(b->w);   // device.rs:262-272
    oe.param = f16 ? b->w : nullptr;
    oe.dv = b->dv_w;
    oe.dm = b->dm_w;
    oe.opt = opt_params(t->optimiser, step);
    oe.lr = t->learn_rate;
    oe.clamp = t->grad_clamp;
    oe.inv_m = inv_m;
    oe.regu_coeff = b->regularisation ? b->regu_coeff : 0.0f;
    oe.regularisation = b->regularisation;
    oe.ldc = N;
    if (f16) {
        // elements whose fp16-operand sum is not finite are summed again from these in fp32
        oe.x = in;
        oe.ldx = in_cols;
        oe.dp32 = b->d_prenorm;
        oe.lddp = N;
        oe.batch = batch;
    }

    // column partial sums for db / dNorm sums: left by the error call just
    // before, or made here in the workspace after the GEMM's region
    const bool cached = cols_match(ctx, b, batch);
    const uint32_t csplits = cached ? ctx->cs.splits : colsum_splits(batch, N);

    GemmLaunch g{};
    g.dtype = b->dtype;
    g.M = K;
    g.N = N;
    g.K = batch;
    g.lda = in_cols;
    g.ldb = N;
    g.a_kcontig = false;
    g.b_kcontig = false;
    g.A = in;
    g.B = f16 ? b->d_prenorm_h : b->d_prenorm;
    g.b32 = b->d_prenorm;
    g.splits = 1;
    g.op = Op::DwOpt;
    g.opt = oe;
    const GemmPlan plan = plan_gemm(g);
    const size_t gemm_bytes = (plan.bytes() + 255) & ~(size_t)255;
    const size_t col_bytes = cached ? 0 : (size_t)csplits * 3 * N * sizeof(float);
    if ((r = ensure_ws(ctx, gemm_bytes + col_bytes))) return r;
    char *ws = reinterpret_cast<char *>(ctx->ws);
    float *ws_col = reinterpret_cast<float *>(ws + gemm_bytes);

    // -- db, sum dNorm_w, sum dNorm_b and their optimiser steps -----------------------
    VecOptArgs v{};
    v.dtype = b->dtype;
    v.rows = batch;
    v.n = N;
    v.splits = csplits;
    v.src[0] = use_bias ? b->d_prenorm : nullptr;
    v.src[1] = b->norm > 0 ? b->d_norm_w : nullptr;
    v.src[2] = b->norm > 1 ? b->d_norm_b : nullptr;
    v.partials = cached ? ctx->cols : ws_col;
    void *params[3] = {b->b, b->norm_w, b->norm_b};
    float *masters[3] = {b->master_b, b->master_norm_w, b->master_norm_b};
    float *dvs[3] = {b->dv_b, b->dv_norm_w, b->dv_norm_b};
    float *dms[3] = {b->dm_b, b->dm_norm_w, b->dm_norm_b};
    for (int k = 0; k < 3; ++k) {
        v.enabled[k] = v.src[k] != nullptr;
        v.param[k] = f16 ? params[k] : nullptr;
        v.master[k] = f16 ? masters[k] : reinterpret_cast<float *>(params[k]);
        v.dv[k] = dvs[k];
        v.dm[k] = dms[k];
        v.opt[k] = opt_params(k == 0 ? t->optimiser : t->norm_optimiser, step);
    }
    v.lr = t->learn_rate;
    v.clamp = t->grad_clamp;
    v.inv_m = inv_m;
    const bool any_vec = v.enabled[0] || v.enabled[1] || v.enabled[2];
    // the column sums read only the error call's outputs, so they go first; the
    // parameter update then rides in the dW's split-K reduction launch when it has one
    if (any_vec && !cached) SKL_TRY(launch_colsum(v, ctx->stream));
    bool vec_done = false;
    if ((r = exec_gemm(ctx, g, plan, ws, false, any_vec ? &v : nullptr, &vec_done, f16 ? KEEP_B : 0))) return r;
    if (any_vec && !vec_done) SKL_TRY(launch_vec_opt(v, ctx->stream));
    return SKL_OK;
}

int32_t skl_dense_backward(skl_ctx *ctx, const skl_dense_desc *b, const void *in, uint32_t in_rows,
                           uint32_t in_cols, const skl_train_ctx *t, uint32_t step) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = backward_impl(ctx, b, in, in_rows, in_cols, t, step))) return r;
    return finish(ctx);
}

int32_t skl_dense_backward_hidden(skl_ctx *ctx, const skl_dense_desc *cur, const skl_dense_desc *next,
                                  const void *in, uint32_t in_rows, uint32_t in_cols, const skl_train_ctx *t,
                                  uint32_t step) {
    int32_t r = enter(ctx);
    if (r) return r;
    SKL_CHECK(t, SKL_ERR_NULL_POINTER);
    if ((r = check_desc(ctx, cur))) return r;
    if ((r = check_desc(ctx, next))) return r;
    // backward_hidden (mlp.rs:682-726), in its order
    SKL_CHECK(cur->is_training, SKL_ERR_TRAINING_MODE_REQUIRED);
    if ((r = check_input(cur, in, in_rows, in_cols, t->batch_size))) return r;
    SKL_CHECK(next->inputs == cur->outputs, SKL_ERR_MISMATCHED_DIMENSIONS);      // mlp.rs:690-697
    SKL_CHECK(next->max_batch >= in_rows, SKL_ERR_MISMATCHED_DIMENSIONS);        // mlp.rs:699-706
    if ((r = check_act_batch(cur, t->batch_size))) return r;                     // mlp.rs:708-726
    if ((r = hidden_error_impl(ctx, cur, next, t->batch_size))) return r;
    if ((r = backward_impl(ctx, cur, in, in_rows, in_cols, t, step))) return r;
    return finish(ctx);
}

// skl_dense_error_from_sum's checks, in order, and its kernel arguments
static int32_t error_from_sum_checks(skl_ctx *ctx, const skl_dense_desc *b, const float *s, uint32_t batch) {
    int32_t r;
    if ((r = check_desc(ctx, b))) return r;
    SKL_CHECK(b->is_training, SKL_ERR_TRAINING_MODE_REQUIRED);
    SKL_CHECK(s, SKL_ERR_NULL_POINTER);
    SKL_CHECK(batch <= b->max_batch, SKL_ERR_ALLOCATION_LIMIT);
    if ((r = check_act_batch(b, batch))) return r;
    if ((r = check_backward_buffers(b))) return r;
    SKL_CHECK(b->predrop && b->preact && b->mask, SKL_ERR_NULL_POINTER);
    if (b->dtype == SKL_F16 && b->norm) SKL_CHECK(b->master_norm_w, SKL_ERR_NULL_POINTER);
    return SKL_OK;
}

static ErrArgs error_from_sum_args(const skl_dense_desc *b, const float *s, uint32_t batch) {
    ErrArgs a{};
    a.dtype = b->dtype;
    a.rows = batch;
    a.n = b->outputs;
    a.norm = b->norm;
    a.act = b->act;
    a.leaky = b->act == SKL_ACT_LEAKY_RELU ? b->leaky : 0.0f;
    a.inv_n = 1.0f / (float)b->outputs;
    a.inv_m = 1.0f / (float)batch;
    a.loss_scale = 1.0f;
    a.s = s;
    a.predrop = b->predrop;
    a.preact = b->preact;
    a.mask = b->mask;
    a.norm_rstd = b->norm_rstd;
    a.centered = b->centered;
    a.prenorm = b->prenorm;
    a.nw = master_norm_w(b);
    a.grad = b->grad;
    a.d_prenorm = b->d_prenorm;
    a.d_norm_w = b->d_norm_w;
    a.d_norm_b = b->d_norm_b;
    a.d_prenorm_h = b->dtype == SKL_F16 ? reinterpret_cast<half_t *>(b->d_prenorm_h) : nullptr;
    return a;
}

int32_t skl_dense_error_from_sum(skl_ctx *ctx, const skl_dense_desc *b, const float *s, uint32_t batch) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = error_from_sum_checks(ctx, b, s, batch))) return r;
    if ((r = zero_dnorm_tail(ctx, b, batch))) return r;
    const ErrArgs a = error_from_sum_args(b, s, batch);
    uint32_t splits = 0;
    if ((r = ensure_cols(ctx, b, batch, 1, &splits))) return r;
    note_rewrite(ctx, b);
    SKL_TRY(launch_error_from_sum(a, ctx->cols, splits, ctx->stream));
    record_cols(ctx, b, batch, splits);
    return finish(ctx);
}

int32_t skl_dense_error_from_sum_noalloc(skl_ctx *ctx, const skl_dense_desc *b, const float *s, uint32_t batch) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = error_from_sum_checks(ctx, b, s, batch))) return r;
    SKL_CHECK(ctx->scratch, SKL_ERR_NULL_POINTER);
    const uint32_t splits = err_col_splits(batch, b->outputs, err_resident(b->dtype, 1, b->outputs, b->norm != 0));
    SKL_CHECK((size_t)splits * 3 * b->outputs * sizeof(float) <= NOALLOC_SCRATCH_BYTES, SKL_ERR_ALLOCATION_LIMIT);
    if ((r = zero_dnorm_tail(ctx, b, batch))) return r;
    const ErrArgs a = error_from_sum_args(b, s, batch);
    // every split writes all of its partial-sum rows: nothing in the scratch needs clearing
    note_rewrite(ctx, b);
    SKL_TRY(launch_error_from_sum(a, reinterpret_cast<float *>(ctx->scratch), splits, ctx->stream));
    // the partials sit in memory every call on this GPU shares: skl_dense_backward
    // must not take them for its column sums, it reads d_prenorm / dNorm again
    ctx->cs.valid = false;
    return finish(ctx);
}

int32_t skl_dense_input_grad(skl_ctx *ctx, const skl_dense_desc *b, uint32_t batch, float *dx) {
    int32_t r = enter(ctx);
    if (r) return r;
    if ((r = check_desc(ctx, b))) return r;
    SKL_CHECK(dx, SKL_ERR_NULL_POINTER);
    SKL_CHECK(batch > 0, SKL_ERR_INVALID_BATCH_SIZE);
    SKL_CHECK(batch <= b->max_batch, SKL_ERR_ALLOCATION_LIMIT);
    const bool f16 = b->dtype == SKL_F16;
    SKL_CHECK(f16 ? b->d_prenorm_h != nullptr : b->d_prenorm != nullptr, SKL_ERR_NULL_POINTER);
    GemmLaunch g{};
    g.dtype = b->dtype;
    g.M = batch;
    g.N = b->inputs;
    g.K = b->outputs;
    g.lda = b->outputs;
    g.ldb = b->outputs;
    g.a_kcontig = true;
    g.b_kcontig = true;
    g.A = f16 ? b->d_prenorm_h : b->d_prenorm;
    g.B = b->w;
    g.splits = 1;
    g.op = Op::InputGrad;
    g.st.out = dx;
    g.st.split_stride = 0;
    g.st.ldc = b->inputs;
    const GemmPlan plan = plan_gemm(g);
    if ((r = ensure_ws(ctx, plan.bytes()))) return r;
    if ((r = exec_gemm(ctx, g, plan, reinterpret_cast<char *>(ctx->ws), false, nullptr, nullptr, f16 ? KEEP_A : 0)))
        return r;
    // dX reads d_prenorm (or its fp16 copy) and W and writes dx only: column sums
    // that the error call just before left stay valid for the backward after
    // this call (a single block's dX before its optimiser step), unless dx
    // overlaps a buffer they were summed from
    ColSums &c = ctx->cs;
    if (c.valid && c.call + 1 >= ctx->calls) {
        const size_t dx_bytes = (size_t)batch * b->inputs * sizeof(float);
        const size_t buf_bytes = (size_t)c.rows * c.n * sizeof(float);
        const bool hit = overlaps(dx, dx_bytes, c.dp, buf_bytes) ||
                         (c.norm != SKL_NORM_DISABLED &&
                          (overlaps(dx, dx_bytes, c.dnw, buf_bytes) || overlaps(dx, dx_bytes, c.dnb, buf_bytes)));
        if (hit)
            c.valid = false;
        else
            c.call = ctx->calls;
    }
    return finish(ctx);
}

}  // extern "C"
