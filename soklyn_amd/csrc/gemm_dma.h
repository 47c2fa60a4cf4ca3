// gemm_dma.h — fp16 GEMM on whole 256x256 tiles (M % 256 == N % 256 == 0,
// K % 128 == 0), gfx950.  Each operand is either k-contiguous in HBM or
// m/n-contiguous (the forward's W, both operands of dW), so no layout needs a
// transposed copy.
//
//  * MFMA shape MI = 32 (v_mfma_f32_32x32x16_f16, 32-row fragments) or 16
//    (v_mfma_f32_16x16x32_f16, 16-row fragments, 32 k per MFMA).  A
//    register-only loop of independent MFMAs on all 256 CUs sustains 2032
//    TFLOP/s at 2.09 GHz with 16x16x32 and 1704 TFLOP/s at 1.68 GHz with
//    32x32x16: the 16x16 form draws less power per flop.  With MI = 16 the A
//    fragments are single-buffered (fragment i of the next k-step is read in
//    place after its row's MFMAs), which keeps 8 waves inside the register
//    budget when A is k-contiguous.
//  * NW = 4 or 8 waves.  NW = 4 on a 256 x 256 tile: one wave per SIMD, wave
//    tile 128 x 128 = 8 x 8 v_mfma_f32_16x16x32_f16 blocks, 256 accumulators per
//    lane held in AGPRs by an asm MFMA (DmaMma<16>::run_agpr), both fragment sets
//    double-buffered, 16 fragment reads and 16 DMA instructions spread evenly over
//    the 64 MFMAs of a k-step.  NW = 8: two waves per SIMD, wave tile 128 x 64
//    (128 accumulators), 1.5x the LDS fragment bytes per flop, but while one wave
//    of a SIMD waits on its LDS reads the other issues MFMAs.  The GEMMs run at the
//    board's power limit (the clock settles near 1.8-2.0 GHz), where fewer bytes
//    per flop buy clock: on the C3 shapes the 4-wave main loop is ~4% faster per k
//    than the 8-wave one for every layout, but with half the threads the
//    store-heavy epilogues (forward caches, fused hidden error) run slower, so the
//    launcher takes 4 waves for the fp32-store and optimiser epilogues and 8 for
//    the others.
//  * BK = 64 halves; 2 stages of 64 KB (A tile + B tile, 32 KB each, laid out
//    per operand layout as described at OpK / OpN).  Stages are filled by
//    buffer_load_dwordx4 ... lds (no staging registers, no ds_write): one wave
//    instruction fills 1 KB of LDS, each lane fetching the global chunk that
//    the swizzle puts in its slot; a wave issues 32 / NW per operand per tile.
//    The buffer form (32-bit lane offset + scalar offset against a resource)
//    ran 1-3% faster than global_load_lds_dwordx4 (64-bit lane addresses) on
//    the C3 shapes.
//  * Fragments are software-pipelined: the four k-steps of a tile alternate
//    between two fragment register sets, and the reads of k-step ks + 1 are
//    issued between the MFMAs of k-step ks, one fragment (two at 8 waves)
//    behind each MFMA from the first on, so no burst of reads fills the LDS
//    queues and the rest of the k-step covers their latency (scheduling
//    barriers hold that order; 1-2% faster than the whole next set read ahead
//    of the MFMAs).
//  * Per tile: after k-step 2's MFMAs, wait for this wave's DMA of the next
//    tile (vmcnt 0: it is the only one outstanding) and for k-step 3's
//    fragments, s_barrier without a fence (LDS DMA completion is what vmcnt
//    tracks); then k-step 3's MFMAs, each followed by one DMA instruction of
//    tile kt+2 (into the stage every wave has just finished reading) and the
//    reads of the next tile's k-step 0.
//  * The k loop body has no branches (a branchy body made the register
//    allocator spill): K is a multiple of 2 k-tiles, the last two
//    refills fetch the final k-tile again (in bounds, never read), and the last
//    cross-barrier fragment read lands in registers nobody reads.
//  * Fragment reads are inline ds_read_b128 / ds_read_b64_tr_b16 (left to
//    itself the compiler sinks each read next to its first MFMA behind an
//    lgkmcnt(0), serialising LDS latency with the MFMA pipe).  The compiler
//    does not count them, so the kernel waits for them itself: when a set is
//    about to be consumed its reads are the only ones pending, so the wait is
//    lgkmcnt(0) (a scalar load in flight only makes it stricter), and after
//    it an empty asm statement per fragment register claims to rewrite it, so
//    no MFMA can be scheduled above the wait.
// Operand offsets are 32-bit (rows * ld * 2 bytes < 4 GiB).
#pragma once

#include <type_traits>

#include "gemm.h"
#include "vec_opt.h"

namespace skl {

template <int NW_, int MI_ = 32, int BM_ = 256, int BN_ = 256> struct DmaCfg {
    static_assert(NW_ == 4 || NW_ == 8, "4 or 8 waves");
    static_assert(MI_ == 16 || MI_ == 32, "16x16x32 or 32x32x16 MFMA");
    static_assert((BM_ == 256 && BN_ == 256) || (BM_ == 128 && BN_ == 128 && NW_ == 4), "tile shapes");
    static constexpr int NW = NW_, MI = MI_;
    static constexpr int BM = BM_, BN = BN_, BK = 64, WM = 2, WN = NW / 2, NT = 64 * NW;
    static constexpr int TWM = BM / WM, TWN = BN / WN, MT = TWM / MI, NTL = TWN / MI;
    static constexpr int KSTEP = 512 / MI;         // k per MFMA
    static constexpr int KS = BK / KSTEP;          // k-steps per tile
    static constexpr int OPA = BM * BK * 2;        // bytes per operand tile (32 KB at 256 rows)
    static constexpr int OPB = BN * BK * 2;
    static constexpr int STAGEB = OPA + OPB;       // 64 KB per stage at 256 x 256
    // waves per SIMD: one 256x256 workgroup per CU, or two 128x128 ones
    static constexpr int WPE = BM == 256 ? NW / 4 : 2;
};

// One MFMA block; the B fragment (n rows) is the instruction's first operand and
// the A fragment (m rows) its second, so a lane's accumulators are consecutive
// n of one m.  32: lane l, register r holds (n = 8 (r / 4) + 4 (l / 32) + r % 4,
// m = l % 32); 16: (n = 4 (l / 16) + r, m = l % 16).
template <int MI> struct DmaMma;
template <> struct DmaMma<32> {
    typedef floatx16 Acc;
    __device__ __forceinline__ static void run(Acc &acc, const u32x4 &bop, const u32x4 &aop) {
        Mfma<half_t>::run(acc, bop, aop);
    }
};
template <> struct DmaMma<16> {
    typedef floatx4 Acc;
    __device__ __forceinline__ static void run(Acc &acc, const u32x4 &bop, const u32x4 &aop) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8, bop), __builtin_bit_cast(halfx8, aop),
                                                     acc, 0, 0, 0);
    }
    // The same MFMA with the accumulator bound to AGPRs by the asm constraint.  With
    // 256 accumulators per lane (one wave per SIMD) the register allocator, left to
    // itself, moves them between AGPRs and VGPRs around the k loop and spills.  The
    // compiler's hazard checks do not see into the asm: the kernel adds the wait
    // states itself (after zeroing the accumulators, before the epilogue reads them);
    // inside the loop no VALU writes a VGPR or AGPR these MFMAs read.
    __device__ __forceinline__ static void run_agpr(Acc &acc, const u32x4 &bop, const u32x4 &aop) {
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(bop), "v"(aop));
    }
};

typedef __attribute__((address_space(3))) char lds_char;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Direct-to-LDS source of one lane: a raw buffer resource over the operand
// (gfx9 dword 3 = 0x00020000) and the lane's byte offset.  load() moves the
// lane's 16 bytes at voff + add to dst + 16 lane (buffer_load_dwordx4 ... lds;
// the immediate offset, which would move the LDS address too, stays 0).
struct DmaSrc {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff;
    __device__ __forceinline__ void init(const half_t *p, uint32_t bytes, uint32_t off) {
        rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(p), (short)0, (int)bytes, 0x00020000);
        voff = off;
    }
    __device__ __forceinline__ void load(uint32_t add, lds_char *dst) const {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, reinterpret_cast<__attribute__((address_space(3))) void *>(dst),
                                                 16, (int)voff, (int)add, 0, 0);
    }
};

// s_waitcnt with only one counter constrained (gfx9 encoding: vmcnt[3:0] +
// vmcnt[5:4] at bits 15:14, expcnt bits 6:4, lgkmcnt bits 11:8).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
template <int N> __device__ __forceinline__ void wait_lgkmcnt() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

template <int OFF> __device__ __forceinline__ void ds_read16(u32x4 &dst, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF) : "memory");
}
template <int OFF> __device__ __forceinline__ void ds_read8_tr(u32x2 &dst, uint32_t addr) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF) : "memory");
}
// Claims to rewrite v: orders every later use of v after the preceding asm.
__device__ __forceinline__ void pin(u32x4 &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(u32x2 &v) { asm volatile("" : "+v"(v)); }

// ---- operand staging ------------------------------------------------------------
// One operand tile of a stage: 256 rows (m or n) x 64 k, 32 KB, filled by
// direct-to-LDS loads (one wave instruction = 1 KB of LDS, lane l writing
// bytes 16 l .. 16 l + 15; instruction t of wave w fills KB NW t + w), read
// as NF 32-row MFMA fragments of the wave's rows per k-step.  The fragment of
// a lane holds 8 consecutive k of row l % 32 (k = 8 (l / 32) .. + 7 within
// the 16-k step).
//
// OpK: k-contiguous in HBM (row r at p + r ld).  LDS row = 128 bytes = 8
// chunks of 8 halves, chunk c of row r stored at slot c ^ ((r >> 1) & 7): any
// 16 consecutive rows of one chunk column hit 16 distinct 16-byte bank groups.
// A fragment is one ds_read_b128.
template <int NW, int NF, int MI = 32, int ROWS = 256> struct OpK {
    static constexpr int IPO = ROWS / 8 / NW;   // DMA instructions per tile and wave
    static constexpr uint32_t CPK = 512 / MI / 8;   // 16-byte chunks of a row per k-step
    struct Frag { u32x4 v[NF]; };
    DmaSrc dma;                       // DMA source of this lane, t = 0, k-tile 0
    uint32_t step;                    // bytes between DMA instructions (8 NW rows)
    uint32_t lds;                     // LDS byte address of this lane's fragment row, stage 0
    uint32_t g;                       // swizzle term of the fragment row

    __device__ __forceinline__ void init(const half_t *p, uint32_t ld, uint32_t rows, uint32_t mn0, uint32_t wbase,
                                         uint32_t wave, uint32_t lane, uint32_t lds_op) {
        // instruction t fills rows 8 (NW t + wave) .. + 7; lane -> row + lane / 8, slot lane % 8;
        // (row >> 1) & 7 does not depend on t (8 NW t >> 1 is a multiple of 8)
        const uint32_t row0 = 8u * wave + (lane >> 3);
        const uint32_t kc = (lane & 7u) ^ ((row0 >> 1) & 7u);
        dma.init(p, rows * ld * 2u, (mn0 + row0) * ld * 2u + kc * 16u);
        step = 8u * NW * ld * 2u;
        // wbase is a multiple of 32: the fragment row's swizzle is that of lane % MI
        const uint32_t frow = lane % MI;
        g = (lane / MI) ^ ((frow >> 1) & 7u);
        lds = lds_op + (wbase + frow) * 128u;
    }
    __device__ __forceinline__ void issue(int kt, int t, lds_char *dst) const {
        dma.load((uint32_t)kt * 128u + t * step, dst + t * (NW * 1024u));
    }
    // fragment i: logical chunk CPK ks + lane / MI of row MI i + lane % MI (the
    // two terms have disjoint bits, so the swizzle XOR applies to them apart)
    __device__ __forceinline__ void read_frag(Frag &f, uint32_t stage_off, int ks, int i) const {
        const uint32_t a = lds + stage_off + ((CPK * ks) ^ g) * 16u;
        switch (i) {
        case 0: ds_read16<0>(f.v[0], a); break;
        case 1: ds_read16<1 * MI * 128>(f.v[1], a); break;
        case 2: if constexpr (NF > 2) ds_read16<2 * MI * 128>(f.v[2], a); break;
        case 3: if constexpr (NF > 3) ds_read16<3 * MI * 128>(f.v[3], a); break;
        case 4: if constexpr (NF > 4) ds_read16<4 * MI * 128>(f.v[4], a); break;
        case 5: if constexpr (NF > 5) ds_read16<5 * MI * 128>(f.v[5], a); break;
        case 6: if constexpr (NF > 6) ds_read16<6 * MI * 128>(f.v[6], a); break;
        default: if constexpr (NF > 7) ds_read16<7 * MI * 128>(f.v[7], a); break;
        }
    }
    __device__ __forceinline__ static u32x4 op(const Frag &f, int i) { return f.v[i]; }
    static constexpr int RPF = 1;   // LDS reads per fragment
    __device__ __forceinline__ static void pin_one(Frag &f, int i) { pin(f.v[i]); }
    __device__ __forceinline__ static void pin_all(Frag &f) {
#pragma unroll
        for (int i = 0; i < NF; ++i) pin(f.v[i]);
    }
};

// OpN: m- (or n-) contiguous in HBM (k-row k at p + k ld).  LDS holds the
// tile k-major: 64 rows of 512 bytes (256 halves), chunk c of k-row r stored
// at slot c ^ (4 (r & 3)).  A fragment is two ds_read_b64_tr_b16: in each
// group of 16 lanes, lane s supplies the 8 bytes at k-row 4 h + s / 4 (+ 8 for
// lanes 32..63), halves 4 (s % 4) .. + 3 of the group's 16 rows, and receives
// 4 consecutive k of its own row; h = 0, 1 give k 0..3 and 4..7.  The 32 lanes
// of a half-wave read 4 k-rows x 64 bytes, which the swizzle spreads over the
// 4 distinct 64-byte bank windows.  Fragment i of the wave sits 32 rows
// further on: chunk + 4 i, i.e. the lane's address XOR 64 i (the wave's first
// row is a multiple of 32 NF, so the chunk bits that i flips start clear).
template <int NW, int NF, int MI = 32, int COLS = 256> struct OpN {
    static constexpr uint32_t P = 2u * COLS;             // bytes per LDS k-row
    static constexpr uint32_t LPR = P / 16u;             // DMA lanes per k-row
    static constexpr uint32_t RPI = 64u / LPR;           // k-rows per DMA instruction
    static constexpr int IPO = 64 / RPI / NW;
    static constexpr uint32_t KSB = P * (512 / MI);      // bytes per k-step (KSTEP k-rows)
    struct Frag { u32x2 v[NF][2]; };
    DmaSrc dma[2];                    // even / odd instructions (their swizzle differs for MI = 16, NW = 4)
    uint32_t step;                    // 2 NW k-rows per DMA instruction of a wave
    uint32_t kstep;                   // bytes per k-tile (64 k-rows)
    uint32_t lds_op, rel;             // operand tile base; this lane's offset of fragment 0 (k-step 0, h = 0)

    // MI = 16 adds 2 ((r >> 3) & 1): the two 16-lane groups of a half-wave read
    // k-rows r and r + 8, which this moves to different banks
    __device__ __forceinline__ static uint32_t swz(uint32_t r) {
        return (4u * (r & 3u)) ^ (MI == 16 ? 2u * ((r >> 3) & 1u) : 0u);
    }

    __device__ __forceinline__ void init(const half_t *p, uint32_t ld, uint32_t rows, uint32_t mn0, uint32_t wbase,
                                         uint32_t wave, uint32_t lane, uint32_t lds_op_) {
        // instruction t (q = wave + NW t) fills k-rows RPI q .. RPI q + RPI - 1; lane -> k-row
        // RPI q + lane / LPR, slot lane % LPR; r & 3 does not depend on t (NW is even), (r >> 3) & 1
        // at most on t's parity
#pragma unroll
        for (uint32_t t = 0; t < 2; ++t) {
            const uint32_t r = RPI * (wave + NW * t) + lane / LPR;
            const uint32_t cl = (lane % LPR) ^ swz(r);
            dma[t].init(p, rows * ld * 2u, (RPI * wave + lane / LPR) * ld * 2u + mn0 * 2u + cl * 16u);
        }
        step = RPI * NW * ld * 2u;
        kstep = 64u * ld * 2u;
        const uint32_t grp = lane >> 4, s = lane & 15u;
        uint32_t row, col;
        if constexpr (MI == 32) {
            row = 8u * (grp >> 1) + (s >> 2);
            col = wbase + 16u * (grp & 1u) + 4u * (s & 3u);   // wbase % (32 NF) == 0
        } else {
            row = 8u * grp + (s >> 2);
            col = wbase + 4u * (s & 3u);                      // wbase % (16 NF) == 0
        }
        rel = row * P + (((col >> 3) ^ swz(row)) * 16u) + (col & 7u) * 2u;
        lds_op = lds_op_;
    }
    __device__ __forceinline__ void issue(int kt, int t, lds_char *dst) const {
        dma[t & 1].load((uint32_t)kt * kstep + t * step, dst + t * (NW * 1024u));
    }
    // fragment i sits MI rows further on: the lane's offset XOR 2 MI i; k-rows
    // KSTEP ks + 4 h (+ 8 g) at offsets KSB ks + 2048 h keep the swizzle
    __device__ __forceinline__ void read_frag(Frag &f, uint32_t stage_off, int ks, int i) const {
        const uint32_t a = lds_op + (rel ^ (2u * MI * i)) + stage_off + KSB * ks;
        ds_read8_tr<0>(f.v[i][0], a);
        ds_read8_tr<4 * P>(f.v[i][1], a);
    }
    __device__ __forceinline__ static u32x4 op(const Frag &f, int i) {
        return u32x4{f.v[i][0].x, f.v[i][0].y, f.v[i][1].x, f.v[i][1].y};
    }
    static constexpr int RPF = 2;   // LDS reads per fragment
    __device__ __forceinline__ static void pin_one(Frag &f, int i) {
        pin(f.v[i][0]);
        pin(f.v[i][1]);
    }
    __device__ __forceinline__ static void pin_all(Frag &f) {
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            pin(f.v[i][0]);
            pin(f.v[i][1]);
        }
    }
};

// Epilogues with running column sums (EpiErrK) declare kColSums, an Acc type,
// finish(..., Acc &) and flush<NW>(), and run on whole tiles only; the others
// have none.
struct NoAcc {};
template <class E, class = void> struct EpiSums {
    static constexpr bool value = false;
    typedef NoAcc Acc;
};
template <class E> struct EpiSums<E, std::void_t<decltype(E::kColSums)>> {
    static constexpr bool value = E::kColSums;
    typedef typename E::Acc Acc;
};

// Epilogues with kVec = 8 also take 8 consecutive columns per thread (column8,
// finish8) on whole tiles.
template <class E, class = void> struct EpiVec8 { static constexpr bool value = false; };
template <class E> struct EpiVec8<E, std::void_t<decltype(E::kVec)>> { static constexpr bool value = E::kVec == 8; };

// Epilogues with kDirect finish each accumulator block from its registers
// (direct(params, idx, m, n, 4 columns, its loads)) when the tile runs one wave per
// SIMD on whole tiles, instead of going through LDS; the per-element loads of
// kDirectBatch blocks are issued before any of them is used.  Only stores take it:
// loads in this shape (16 rows x 64 bytes per instruction, rows a power-of-two
// pitch apart) ran the fused optimiser's epilogue ~10x slower (C3 dW + Adam
// 272 -> 3090 us), the rows falling into few vector-L1 sets.
template <class E, class = void> struct EpiDirect {
    static constexpr bool value = false;
    static constexpr int batch = 1;
};
template <class E> struct EpiDirect<E, std::void_t<decltype(E::kDirect)>> {
    static constexpr bool value = E::kDirect;
    static constexpr int batch = E::kDirectBatch;
};

// MFMAs per DMA instruction in a tile's last k-step, where the refill of the
// stage just read is issued (16x16x32 schedule): 1 = all of them behind the
// first MFMAs.  Measured on C3 / C4 (steady clocks): every second MFMA runs the
// forward 0.2357 -> 0.2317 ms and the fused hidden error 0.2689 -> 0.2672 ms,
// while the fp32-store dX is fastest front-loaded (0.2178 ms; 0.2188 at 2,
// 0.2224 at 4), so an epilogue may set its own kDmaSpacing.
template <class E, class = void> struct EpiDmaSpacing { static constexpr int value = 2; };
template <class E> struct EpiDmaSpacing<E, std::void_t<decltype(E::kDmaSpacing)>> {
    static constexpr int value = E::kDmaSpacing;
};

// 32x32x16 schedule: the next k-step's fragment reads issued behind each MFMA
// (2 at 8 waves).  The split-K dW partial (fp32 store) runs faster with 1 (C4
// step 2.578 -> 2.568 ms), dW + Adam slower (0.2825 -> 0.288 ms).
template <class E, int NW, class = void> struct EpiReadsPerMfma { static constexpr int value = NW == 8 ? 2 : 1; };
template <class E, int NW> struct EpiReadsPerMfma<E, NW, std::void_t<decltype(E::kReadsPerMfma)>> {
    static constexpr int value = E::kReadsPerMfma;
};

template <bool KC, int NW, int NF, int MI, int R> struct DmaOpSel { typedef OpK<NW, NF, MI, R> type; };
template <int NW, int NF, int MI, int R> struct DmaOpSel<false, NW, NF, MI, R> { typedef OpN<NW, NF, MI, R> type; };

// Grid: (tiles, splits); each workgroup takes one (tile, split) pair (split-K grids
// remap the pairs onto the XCDs, below).  Split y reduces k in [y k_per_split,
// (y + 1) k_per_split) (k_per_split a multiple of 128; the last split may be
// shorter, also a multiple of 128).  EDGE: the operands are zero-padded copies whose M, N
// extend past the real output [mv x nv]; the epilogue then goes element by
// element through Epi::apply with those bounds (any leading dimension).
template <class Epi, bool A_KC, bool B_KC, int NW, bool EDGE, int MI = 32, int BT = 256>
__global__ void __launch_bounds__(64 * NW)
    __attribute__((amdgpu_waves_per_eu(DmaCfg<NW, MI, BT, BT>::WPE, DmaCfg<NW, MI, BT, BT>::WPE)))
    gemm_dma_kernel(GemmShape sh, const half_t *__restrict__ A, const half_t *__restrict__ B,
                    typename Epi::Params ep) {
    typedef DmaCfg<NW, MI, BT, BT> C;
    typedef typename DmaOpSel<A_KC, NW, C::MT, MI, C::BM>::type OA;
    typedef typename DmaOpSel<B_KC, NW, C::NTL, MI, C::BN>::type OB;
    typedef DmaMma<MI> MM;
    static_assert(C::KS % 2 == 0, "k-steps alternate between two fragment sets");
    constexpr int EPITCH = C::BN + 4;
    constexpr int RPP = 64;                                  // rows of a wave row per epilogue pass
    constexpr int MTP = RPP / MI;                            // accumulator blocks per pass
    constexpr int PROWS = C::WM * RPP;
    constexpr int EPI_BYTES = PROWS * EPITCH * 4;
    constexpr int MAIN_BYTES = 2 * C::STAGEB;
    __shared__ __attribute__((aligned(16))) char smem[MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES];
    lds_char *lsm = (lds_char *)(smem);   // address-space cast: flat -> LDS

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    // wave-uniform in an SGPR: every DMA's LDS destination (M0) is then scalar
    // arithmetic; derived from the thread index it was a VGPR, read back with a
    // v_readfirstlane before each DMA instruction, a VALU -> SGPR -> M0 chain that
    // held the in-order wave off its next MFMA (one-wave-per-SIMD k-step with the
    // refill: 1493 -> 1213 cycles per k-tile; C3 dX 205.5 -> 201.2 us)
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / C::WN, wn = wave % C::WN;

    uint32_t tm, tn;
    uint32_t split = blockIdx.y;
    if (gridDim.y > 1 && ((gridDim.x * gridDim.y) & 7u) == 0) {
        // split-K: workgroup L = x + tiles * y runs on XCD L % 8.  Each XCD takes a
        // contiguous run of the split-major work list, mostly one k-slice of a 4-row
        // tile group, instead of the same tiles of every k-slice (C4's 64-tile dW over
        // 4 slices: an XCD's 32 tiles read 12 operand panels instead of 24; its
        // partial GEMM 111.6 -> 108.8 us, C4 step -1%)
        const uint32_t T = gridDim.x, TS = gridDim.x * gridDim.y, L = blockIdx.x + T * blockIdx.y;
        const uint32_t v = (L & 7u) * (TS >> 3) + (L >> 3);
        split = v / T;
        tile_coords_grouped(v - split * T, sh.tiles_m, sh.tiles_n, tm, tn);
    } else {
        tile_coords(blockIdx.x, sh.tiles_m, sh.tiles_n, tm, tn);
    }
    const uint32_t m0 = sh.m_base + tm * C::BM, n0 = tn * C::BN;
    const uint32_t kbeg = split * sh.k_per_split;
    const int kb = (int)(kbeg / C::BK);                                  // first k-tile of this split
    const int nk = (int)((min(sh.K, kbeg + sh.k_per_split) - kbeg) / C::BK);

    const uint32_t lds0 = (uint32_t)(uintptr_t)lsm;   // LDS byte address of smem
    OA oa;
    OB ob;
    oa.init(A, sh.lda, A_KC ? sh.M : sh.K, m0, wm * C::TWM, wave, lane, lds0);
    ob.init(B, sh.ldb, B_KC ? sh.N : sh.K, n0, wn * C::TWN, wave, lane, lds0 + C::OPA);

    auto issue = [&](int kt, int stage) {
        lds_char *st = lsm + stage * C::STAGEB + wave * 1024u;
#pragma unroll
        for (int t = 0; t < OA::IPO; ++t) oa.issue(kt, t, st);
#pragma unroll
        for (int t = 0; t < OB::IPO; ++t) ob.issue(kt, t, st + C::OPA);
    };

    typename MM::Acc acc[C::MT][C::NTL];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NTL; ++j)
#pragma unroll
            for (int r = 0; r < (int)(sizeof(typename MM::Acc) / 4); ++r) acc[i][j][r] = 0.0f;
    // one wave per SIMD on a 256 x 256 tile: 16x16x32 MFMAs on AGPR accumulators
    // (DmaMma<16>::run_agpr), both fragment sets double-buffered, reads and DMA spread
    // evenly over each k-step
    constexpr bool AGPR_ASM = MI == 16 && NW == 4 && BT == 256;
    if constexpr (AGPR_ASM) {
        // two wait states between each accumulator's zeroing and its first MFMA
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) asm volatile("s_nop 1" : "+a"(acc[i][j]));
    }

    typename OA::Frag fa[2];
    typename OB::Frag fb[2];
    constexpr int NFR = C::MT + C::NTL;            // fragments per set
    constexpr int NMM = C::MT * C::NTL;            // MFMAs per k-step
    constexpr int NDMA = OA::IPO + OB::IPO;        // DMA instructions per tile and wave
    constexpr int FPM = EpiReadsPerMfma<Epi, NW>::value;   // fragment reads behind each MFMA
    static_assert(NFR <= NMM * FPM && NDMA <= NMM, "every read and DMA has an MFMA to follow");
    auto read_frag = [&](int set, int stage, int ks, int f) {
        if (f < C::MT)
            oa.read_frag(fa[set], stage * C::STAGEB, ks, f);
        else
            ob.read_frag(fb[set], stage * C::STAGEB, ks, f - C::MT);
    };
    auto read = [&](int set, int stage, int ks) {
#pragma unroll
        for (int f = 0; f < NFR; ++f) read_frag(set, stage, ks, f);
    };
    auto mfma = [&](int set, int q) {
        const int i = q / C::NTL, j = q % C::NTL;
        if constexpr (AGPR_ASM)
            DmaMma<16>::run_agpr(acc[i][j], OB::op(fb[set], j), OA::op(fa[set], i));
        else
            MM::run(acc[i][j], OB::op(fb[set], j), OA::op(fa[set], i));
    };
    // one wave per SIMD: fragment f of the next k-step behind MFMA f * RSP, the k-step's
    // DMA instruction d behind MFMA d * DSP + 1 (a burst of reads behind the first MFMAs
    // stalled the lone wave: main loop 3-4% slower on the C3 shapes)
    constexpr int RSP = NMM / NFR > 0 ? NMM / NFR : 1, DSP = NMM / NDMA > 0 ? NMM / NDMA : 1;
    auto dma = [&](int kt, int stage, int q) {
        lds_char *st = lsm + stage * C::STAGEB + wave * 1024u;
        if (q < OA::IPO)
            oa.issue(kt, q, st);
        else
            ob.issue(kt, q - OA::IPO, st + C::OPA);
    };
    // The fragment set `cur` is complete (its reads were the only LDS reads
    // pending), and no MFMA on it may be scheduled above this point.
    auto land = [&](int cur) {
        wait_lgkmcnt<0>();
        OA::pin_all(fa[cur]);
        OB::pin_all(fb[cur]);
        __builtin_amdgcn_sched_barrier(0);
    };
    // One k-step: MFMA q of set `cur`, then FPM fragment reads of the next
    // k-step into the other set (all of them within the first NFR / FPM MFMAs,
    // so the rest of the k-step covers their latency), with scheduling barriers
    // keeping that order.
    auto kstep = [&](int cur, int stage, int ks_next) {
        land(cur);
#pragma unroll
        for (int q = 0; q < NMM; ++q) {
            mfma(cur, q);
            if constexpr (AGPR_ASM) {
                if (q % RSP == 0 && q / RSP < NFR) read_frag(cur ^ 1, stage, ks_next, q / RSP);
            } else {
#pragma unroll
                for (int u = 0; u < FPM; ++u)
                    if (q * FPM + u < NFR) read_frag(cur ^ 1, stage, ks_next, q * FPM + u);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int klast = kb + nk - 1;
    if constexpr (MI == 16 && !AGPR_ASM) {
        // 16x16x32: A fragments single-buffered, B double-buffered.  A fragment i
        // of the next k-step is read in place right after row i's MFMAs (its last
        // use), the next k-step's B fragments behind row 0's MFMAs.  LDS reads
        // complete in order; before row i the reads issued after A fragment i may
        // still be pending: the other A fragments of its k-step plus, from row 1
        // on, this k-step's B reads (capped at the counter's 15: stricter).
        typename OA::Frag &fa1 = fa[0];
        constexpr int SPC = EpiDmaSpacing<Epi>::value;
        static_assert(NDMA * SPC <= C::MT * C::NTL, "every DMA instruction follows an MFMA of the last k-step");
        constexpr int W0 = (C::MT - 1) * OA::RPF < 15 ? (C::MT - 1) * OA::RPF : 15;
        constexpr int W1 = (C::MT - 1) * OA::RPF + C::NTL * OB::RPF < 15
                               ? (C::MT - 1) * OA::RPF + C::NTL * OB::RPF : 15;
        auto mfma1 = [&](int set, int i, int j) { MM::run(acc[i][j], OB::op(fb[set], j), OA::op(fa1, i)); };
        auto row_wait = [&](int cur, int i) {
            if (i == 0) {
                wait_lgkmcnt<W0>();
                OB::pin_all(fb[cur]);
            } else {
                wait_lgkmcnt<W1>();
            }
            OA::pin_one(fa1, i);
            __builtin_amdgcn_sched_barrier(0);
        };
        auto kstep1 = [&](int cur, int stage, int ks_next) {
#pragma unroll
            for (int i = 0; i < C::MT; ++i) {
                row_wait(cur, i);
#pragma unroll
                for (int j = 0; j < C::NTL; ++j) {
                    mfma1(cur, i, j);
                    if (i == 0) ob.read_frag(fb[cur ^ 1], stage * C::STAGEB, ks_next, j);
                    __builtin_amdgcn_sched_barrier(0);
                }
                oa.read_frag(fa1, stage * C::STAGEB, ks_next, i);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // prologue: tile 0 resident, tile 1 in flight; B fragments before A
        // fragments, as in every later k-step
        issue(kb, 0);
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        issue(kb + (nk > 1 ? 1 : 0), 1);
#pragma unroll
        for (int j = 0; j < C::NTL; ++j) ob.read_frag(fb[0], 0, 0, j);
#pragma unroll
        for (int i = 0; i < C::MT; ++i) oa.read_frag(fa1, 0, 0, i);
        for (int kt0 = 0; kt0 < nk; kt0 += 2) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int kt = kt0 + s;
#pragma unroll
                for (int ks = 0; ks + 1 < C::KS; ++ks) kstep1(ks & 1, s, ks + 1);
                // the last k-step crosses the barrier: every read of stage s done
                wait_vmcnt<0>();
                wait_lgkmcnt<0>();
                OB::pin_all(fb[1]);
                OA::pin_all(fa1);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                const int kn = min(kb + kt + 2, klast);
#pragma unroll
                for (int i = 0; i < C::MT; ++i) {
#pragma unroll
                    for (int j = 0; j < C::NTL; ++j) {
                        mfma1(1, i, j);
                        const int q = i * C::NTL + j;
                        if (q % SPC == 0 && q / SPC < NDMA) dma(kn, s, q / SPC);
                        if (i == 0) ob.read_frag(fb[0], (s ^ 1) * C::STAGEB, 0, j);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    oa.read_frag(fa1, (s ^ 1) * C::STAGEB, 0, i);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    } else {
    // prologue: tile 0 resident, tile 1 in flight, first fragments read
    issue(kb, 0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    issue(kb + (nk > 1 ? 1 : 0), 1);
    read(0, 0, 0);

    for (int kt0 = 0; kt0 < nk; kt0 += 2) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kt = kt0 + s;
#pragma unroll
            for (int ks = 0; ks + 1 < C::KS; ++ks) kstep(ks & 1, s, ks + 1);
            // the last k-step (3) crosses the barrier: after it, MFMA q of set 1 is followed
            // by DMA instruction q of tile kt+2 (into the stage every wave has
            // just finished reading) and the reads of the next tile's k-step 0
            wait_vmcnt<0>();                    // this wave's DMA of tile kt+1 landed
            land(1);                            // set 1 (k-step 3) is in registers
            __builtin_amdgcn_s_barrier();       // everyone's DMA landed; stage s fully read
            __builtin_amdgcn_sched_barrier(0);
            const int kn = min(kb + kt + 2, klast);
#pragma unroll
            for (int q = 0; q < NMM; ++q) {
                mfma(1, q);
                if constexpr (AGPR_ASM) {
                    if (q % DSP == 1 % DSP && q / DSP < NDMA) dma(kn, s, q / DSP);
                    if (q % RSP == 0 && q / RSP < NFR) read_frag(0, s ^ 1, 0, q / RSP);
                } else {
                    if (q < NDMA) dma(kn, s, q);
#pragma unroll
                    for (int u = 0; u < FPM; ++u)
                        if (q * FPM + u < NFR) read_frag(0, s ^ 1, 0, q * FPM + u);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    }
    wait_vmcnt<0>();     // no DMA may land in the epilogue's staging area
    wait_lgkmcnt<0>();
    if constexpr (AGPR_ASM) {
        // wait states before the epilogue's reads of the last MFMAs' accumulators (the
        // empty statements that claim to rewrite each accumulator keep those reads below)
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) asm volatile("" : "+a"(acc[i][j]));
    }
    if constexpr (AGPR_ASM && EpiDirect<Epi>::value && !EDGE) {
        // a lane's accumulator block holds 4 consecutive columns of one row: stored
        // straight from the AGPRs, each instruction 16 rows x 64 bytes (the L2 joins
        // the two halves of each line), no LDS round trip (C3 dX 210.4 -> 204.2 us in
        // the step)
        // (the kernel ends here: an epilogue with work after its tiles, the fused
        // optimiser's bias update, must not take this path)
        static_assert(!std::is_same<typename Epi::Params, OptEpi>::value, "direct epilogue with a trailing update");
        const typename Epi::Params eps = Epi::at_split(ep, split);
        constexpr int DB = EpiDirect<Epi>::batch;   // blocks whose per-element loads go first
        static_assert(C::NTL % DB == 0, "direct epilogue batch");
#pragma unroll
        for (int i = 0; i < C::MT; ++i) {
            const uint32_t m = m0 + wm * C::TWM + i * MI + (lane & 15u);
#pragma unroll
            for (int jb = 0; jb < C::NTL; jb += DB) {
                typename Epi::Pre pre[DB];
#pragma unroll
                for (int u = 0; u < DB; ++u) {
                    const uint32_t n = n0 + wn * C::TWN + (jb + u) * MI + (lane >> 4) * 4u;
                    Epi::load(eps, (uint64_t)m * Epi::ldc(eps) + n, m, pre[u]);
                }
#pragma unroll
                for (int u = 0; u < DB; ++u) {
                    const uint32_t n = n0 + wn * C::TWN + (jb + u) * MI + (lane >> 4) * 4u;
                    Epi::direct(eps, (uint64_t)m * Epi::ldc(eps) + n, m, n, acc[i][jb + u], pre[u]);
                }
            }
        }
        return;
    }
    __syncthreads();

    // Epilogue through LDS: passes of 128 rows (rows of accumulator block
    // i = pass * MTP + ii of both wave rows; two passes at 256 x 256, one at
    // 128 x 128).  A thread owns the fixed 4-column group c of the tile (a wave
    // covers RPS whole rows per step: one of 256 columns or two of 128, so LDS
    // reads and global accesses are contiguous) and walks its rows; the
    // per-element loads of EPI_BATCH rows are issued
    // before any of them is consumed, so the loop keeps that many in flight
    // instead of paying one memory latency per row (4 rows for large per-row
    // operand sets at 8 waves, whose 256-register budget they would overflow).
    constexpr int EPI_BATCH = (NW == 8 && sizeof(typename Epi::Pre) > 32) ? 4 : 8;
    constexpr bool SUMS = EpiSums<Epi>::value;
    static_assert(!(SUMS && EDGE), "column-sum epilogues run on whole tiles only");
    typename EpiSums<Epi>::Acc csum{};
    constexpr int CPL = C::BN / 4;                 // 4-column groups per row
    constexpr int RPS = 64 / CPL;                  // rows per wave step
    constexpr int ROWS_PER_THREAD = PROWS / (NW * RPS);
    static_assert(ROWS_PER_THREAD % EPI_BATCH == 0, "epilogue batch");
    float *E = reinterpret_cast<float *>(smem);
    const uint32_t c = (lane % CPL) * 4u, sub = lane / CPL;
    GemmShape shv = sh;   // EDGE: bounds of the real output
    shv.M = sh.mv;
    shv.N = sh.nv;
    const typename Epi::Params eps = Epi::at_split(ep, split);
    const typename Epi::Col col = EDGE ? typename Epi::Col{} : Epi::column(eps, n0 + c);
    // EDGE: lane l's columns n0 + l + 64 q, their per-column operands loaded once
    constexpr int EQ = C::BN / 64;
    typename Epi::Col1 col1[EQ];
    if constexpr (EDGE) {
#pragma unroll
        for (int q = 0; q < EQ; ++q) {
            const uint32_t n = n0 + lane + 64u * q;
            col1[q] = n < shv.N ? Epi::column1(ep, n) : typename Epi::Col1{};
        }
    }
#pragma unroll
    for (int pass = 0; pass < C::TWM / RPP; ++pass) {
#pragma unroll
        for (int ii = 0; ii < MTP; ++ii) {
            const int i = pass * MTP + ii;
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) {
                if constexpr (MI == 32) {
                    const uint32_t r = wm * RPP + ii * 32 + (lane & 31u);
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        const uint32_t cc = wn * C::TWN + j * 32 + gq * 8 + (lane >> 5) * 4;
                        floatx4 v = {acc[i][j][4 * gq + 0], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                     acc[i][j][4 * gq + 3]};
                        *reinterpret_cast<floatx4 *>(E + r * EPITCH + cc) = v;
                    }
                } else {
                    const uint32_t r = wm * RPP + ii * 16 + (lane & 15u);
                    const uint32_t cc = wn * C::TWN + j * 16 + (lane >> 4) * 4;
                    *reinterpret_cast<floatx4 *>(E + r * EPITCH + cc) = acc[i][j];
                }
            }
        }
        lds_barrier();
        if constexpr (EDGE) {
            // element by element, lane l taking columns l, l + 64, ... of the
            // row: each store instruction covers 64 consecutive columns
            // whatever the output's alignment; the per-column operands (bias)
            // were loaded above, so a row is stores only (plus dW's per-element
            // optimiser state)
#pragma unroll 2
            for (int b = 0; b < PROWS / NW; ++b) {
                const uint32_t r = wave + (uint32_t)NW * b;
                const uint32_t wmi = r / RPP, rr = r % RPP;
                const uint32_t m = m0 + wmi * C::TWM + pass * RPP + rr;
                if (m >= shv.M) continue;
#pragma unroll
                for (int q = 0; q < EQ; ++q) {
                    const uint32_t n = n0 + lane + 64u * q;
                    if (n >= shv.N) break;
                    Epi::apply1(ep, m, n, E[r * EPITCH + lane + 64u * q], col1[q], split);
                }
            }
            if (pass + 1 < C::TWM / RPP) lds_barrier();
            continue;
        }
        if constexpr (EpiVec8<Epi>::value && !SUMS) {
            // 8 columns per thread (16-byte fp16 stores), R8 rows per wave step:
            // 8-byte stores of 4 columns ran the C3 forward 6% slower, and this
            // loop unrolled by 2 ran it 2% slower
            constexpr uint32_t L8 = C::BN / 8, R8 = 64 / L8;
            const uint32_t c8 = (lane % L8) * 8u, s8 = lane / L8;
            const typename Epi::Col8 col8 = Epi::column8(eps, n0 + c8);
#pragma unroll 1
            for (int b = 0; b < PROWS / (NW * (int)R8); ++b) {
                const uint32_t r = (wave + (uint32_t)NW * b) * R8 + s8;
                const uint32_t wmi = r / RPP, rr = r % RPP;
                const uint32_t m = m0 + wmi * C::TWM + pass * RPP + rr;
                const floatx4 v0 = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c8);
                const floatx4 v1 = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c8 + 4);
                Epi::finish8(eps, (uint64_t)m * Epi::ldc(eps) + n0 + c8, m, n0 + c8, v0, v1, col8);
            }
            if (pass + 1 < C::TWM / RPP) lds_barrier();
            continue;
        }
#pragma unroll 1
        for (int b = 0; b < ROWS_PER_THREAD; b += EPI_BATCH) {
            typename Epi::Pre pre[EPI_BATCH];
            uint32_t mrow[EPI_BATCH];
#pragma unroll
            for (int u = 0; u < EPI_BATCH; ++u) {
                // E row r holds tile row wmi * TWM + pass * RPP + rr
                const uint32_t r = (wave + (uint32_t)NW * (b + u)) * RPS + sub;
                const uint32_t wmi = r / RPP, rr = r % RPP;
                mrow[u] = m0 + wmi * C::TWM + pass * RPP + rr;
                Epi::load(eps, (uint64_t)mrow[u] * Epi::ldc(eps) + n0 + c, mrow[u], pre[u]);
            }
#pragma unroll
            for (int u = 0; u < EPI_BATCH; ++u) {
                const uint32_t r = (wave + (uint32_t)NW * (b + u)) * RPS + sub;
                const floatx4 v = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c);
                if constexpr (SUMS)
                    Epi::finish(eps, (uint64_t)mrow[u] * Epi::ldc(eps) + n0 + c, mrow[u], n0 + c, v, col, pre[u],
                                csum);
                else
                    Epi::finish(eps, (uint64_t)mrow[u] * Epi::ldc(eps) + n0 + c, mrow[u], n0 + c, v, col, pre[u]);
            }
        }
        if (pass + 1 < C::TWM / RPP) lds_barrier();   // E is rewritten by the next pass
    }
    if constexpr (SUMS) {
        static_assert(NW * RPS * 3 * C::BN * 4 <= EPI_BYTES, "column-sum staging fits the epilogue's LDS");
        lds_barrier();   // every wave is done reading E
        Epi::template flush<NW, C::BN>(eps, csum, E, tid, tm, n0);
    }
    // The fused dW + optimiser form also runs the bias / norm-parameter update
    // (independent of W): workgroup w takes its blocks w, w + grid, ... after
    // its tile, which saves that update a launch of its own (its own LDS).
    if constexpr (std::is_same<typename Epi::Params, OptEpi>::value) {
        const uint32_t nwg = gridDim.x * gridDim.y;
        for (uint32_t blk = blockIdx.x + gridDim.x * blockIdx.y; blk < ep.vec_blocks; blk += nwg)
            vec_opt_block<typename Epi::elem, 64 * NW>(ep.vec, blk);
    }
}

}  // namespace skl
