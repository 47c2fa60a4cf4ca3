// gemm_dma.h — fp16 GEMM for the all-k-contiguous layout on whole 256x256
// tiles (M % 256 == N % 256 == 0, K % 128 == 0), gfx950.
//
//  * 4 waves (1 per SIMD), wave tile 128 x 128 = 4 x 4 v_mfma_f32_32x32x16_f16
//    blocks; the 256 accumulators live in AGPRs, fragments in VGPRs.  Per
//    k-step a wave reads 8 x 1 KB fragments from LDS for 16 MFMAs, a third
//    less LDS read traffic per flop than a 128 x 64 wave tile.
//  * BK = 64 halves: an LDS row is 128 bytes = 8 chunks of 16 bytes; 2 stages
//    of 64 KB (A 256 rows + B 256 rows).  Stages are filled by
//    global_load_lds_dwordx4 (no staging registers, no ds_write): one wave
//    instruction fills 8 rows x 8 chunks = 1 KB, lane l fetching the global
//    chunk that belongs in slot l under phys = chunk ^ ((row >> 1) & 7); with
//    128-byte rows that makes every 16 consecutive rows of a fragment read hit
//    16 distinct 16-byte bank groups.
//  * Fragments are software-pipelined across the per-tile barrier: the four
//    k-steps of a tile alternate between two fragment register sets, and the
//    MFMAs of a tile's last k-step are issued after the barrier, behind the
//    reads of the next tile's first k-step.
//  * Per tile: wait for this wave's DMA of the next tile (vmcnt 0: it is the
//    only one outstanding), s_barrier without a fence (LDS DMA completion is
//    what vmcnt tracks), then DMA tile kt+2 into the stage every wave has just
//    finished reading.
//  * The k loop body has no branches (a branchy body made the register
//    allocator spill): K is a multiple of 2 k-tiles, the last two
//    refills fetch the final k-tile again (in bounds, never read), and the last
//    cross-barrier fragment read lands in registers nobody reads.
//  * Fragment reads are inline ds_read_b128 (left to itself the compiler sinks
//    each read next to its first MFMA behind an lgkmcnt(0), serialising LDS
//    latency with the MFMA pipe).  The compiler does not count them, so the
//    kernel waits for them itself: before a fragment set is consumed at most
//    the other set's 8 reads may be pending (LDS returns in order; a scalar
//    load in flight only makes the wait stricter), and the wait is an asm
//    statement that rewrites the set's registers, so no MFMA can be scheduled
//    above it.
// Operand offsets are 32-bit (rows * ld * 2 bytes < 4 GiB).
#pragma once

#include "gemm.h"

namespace skl {

struct Dma256 {
    static constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 2, NT = 256, NWAVES = 4;
    static constexpr int TWM = BM / WM, TWN = BN / WN, MT = TWM / 32, NTL = TWN / 32;
    static constexpr int ROWB = BK * 2;            // 128 bytes per LDS row
    static constexpr int OPB = 256 * ROWB;         // 32 KB per operand tile
    static constexpr int STAGEB = 2 * OPB;         // 64 KB per stage
    static constexpr int IPO = OPB / 1024 / NWAVES;   // 8 DMA instructions per operand per wave
    static constexpr int FRAG_READS = MT + NTL;       // ds_read_b128 per k-step per wave
};

typedef __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ void dma16(const char *src, lds_char *dst) {
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src),
                                     reinterpret_cast<__attribute__((address_space(3))) void *>(dst), 16, 0, 0);
}

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
// lgkmcnt(N) that also claims to rewrite the eight fragments it guards, so
// every MFMA reading them is ordered after the wait by data dependence (a
// bare s_waitcnt builtin orders memory operations, not the pure MFMAs).
template <int N> __device__ __forceinline__ void wait_lgkm_frags(u32x4 (&a)[4], u32x4 (&b)[4]) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3])
                 : "i"(N));
}

template <class Epi>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
    gemm_dma_kernel(GemmShape sh, const half_t *__restrict__ A, const half_t *__restrict__ B,
                    typename Epi::Params ep) {
    typedef Dma256 C;
    constexpr int EPITCH = C::BN + 4;
    constexpr int MTP = 2;                                   // accumulator rows per epilogue pass
    constexpr int PROWS = C::WM * MTP * 32;
    constexpr int EPI_BYTES = PROWS * EPITCH * 4;
    constexpr int MAIN_BYTES = 2 * C::STAGEB;
    __shared__ __attribute__((aligned(16))) char smem[MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES];
    lds_char *lsm = (lds_char *)(smem);   // address-space cast: flat -> LDS

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = wave / C::WN, wn = wave % C::WN;
    const uint32_t frow = lane & 31u;
    const uint32_t fhalf = lane >> 5;

    uint32_t tm, tn;
    tile_coords(blockIdx.x, sh.tiles_m, sh.tiles_n, tm, tn);
    const uint32_t m0 = tm * C::BM, n0 = tn * C::BN;
    const int nk = (int)(sh.K / C::BK);

    // DMA instruction t of this wave (per operand) fills LDS rows
    // 32 t + 8 wave .. +7; lane l takes row 32 t + 8 wave + l / 8 and slot
    // l % 8.  The swizzle term (row >> 1) & 7 does not depend on t.
    const uint32_t row0 = 8u * wave + (lane >> 3);
    const uint32_t kc = (lane & 7u) ^ ((row0 >> 1) & 7u);
    const char *Ab = reinterpret_cast<const char *>(A) + ((size_t)(m0 + row0) * sh.lda * 2u + kc * 16u);
    const char *Bb = reinterpret_cast<const char *>(B) + ((size_t)(n0 + row0) * sh.ldb * 2u + kc * 16u);
    const uint32_t astep = 32u * sh.lda * 2u, bstep = 32u * sh.ldb * 2u;

    auto issue = [&](int kt, int stage) {
        const uint32_t kb = (uint32_t)kt * C::BK * 2u;
        lds_char *st = lsm + stage * C::STAGEB + wave * 1024u;
#pragma unroll
        for (int t = 0; t < C::IPO; ++t) dma16(Ab + kb + t * astep, st + t * 4096u);
#pragma unroll
        for (int t = 0; t < C::IPO; ++t) dma16(Bb + kb + t * bstep, st + C::OPB + t * 4096u);
    };

    floatx16 acc[C::MT][C::NTL];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NTL; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Fragment byte offsets in a stage: row part + swizzled chunk for k-step ks:
    // phys = (2 ks + fhalf) ^ ((row >> 1) & 7) = 2 ks ^ g with g = fhalf ^ ((frow >> 1) & 7)
    // (tile and wave row bases are multiples of 32, so they do not change the swizzle).
    const uint32_t g = fhalf ^ ((frow >> 1) & 7u);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lsm;   // LDS byte address of smem
    const uint32_t a_row = lds0 + (wm * C::TWM + frow) * C::ROWB;
    const uint32_t b_row = lds0 + C::OPB + (wn * C::TWN + frow) * C::ROWB;

    u32x4 fa[2][C::MT], fb[2][C::NTL];
    auto read = [&](int set, int stage, int ks) {
        const uint32_t c = stage * C::STAGEB + ((2u * ks) ^ g) * 16u;
        ds_read16<0 * 32 * C::ROWB>(fa[set][0], a_row + c);
        ds_read16<1 * 32 * C::ROWB>(fa[set][1], a_row + c);
        ds_read16<2 * 32 * C::ROWB>(fa[set][2], a_row + c);
        ds_read16<3 * 32 * C::ROWB>(fa[set][3], a_row + c);
        ds_read16<0 * 32 * C::ROWB>(fb[set][0], b_row + c);
        ds_read16<1 * 32 * C::ROWB>(fb[set][1], b_row + c);
        ds_read16<2 * 32 * C::ROWB>(fb[set][2], b_row + c);
        ds_read16<3 * 32 * C::ROWB>(fb[set][3], b_row + c);
    };
    static_assert(C::MT == 4 && C::NTL == 4, "read() is written out for a 4 x 4 wave tile");
    auto mma = [&](int set) {
        // This set landed; the other set's 8 reads may still be in flight.
        wait_lgkm_frags<C::FRAG_READS>(fa[set], fb[set]);
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) Mfma<half_t>::run(acc[i][j], fb[set][j], fa[set][i]);
    };

    // prologue: tile 0 resident, tile 1 in flight, first fragments read
    issue(0, 0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    issue(nk > 1 ? 1 : 0, 1);
    read(0, 0, 0);

    const int klast = nk - 1;
    for (int kt0 = 0; kt0 < nk; kt0 += 2) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kt = kt0 + s;
            read(1, s, 1);
            mma(0);
            read(0, s, 2);
            mma(1);
            read(1, s, 3);
            mma(0);
            // k-step 3: cross the barrier before issuing its MFMAs
            wait_lgkmcnt<0>();                  // set 1 (k-step 3) is in registers
            wait_vmcnt<0>();                    // this wave's DMA of tile kt+1 landed
            __builtin_amdgcn_s_barrier();       // everyone's landed; stage s fully read
            issue(min(kt + 2, klast), s);
            read(0, s ^ 1, 0);
            mma(1);
        }
    }
    wait_vmcnt<0>();     // no DMA may land in the epilogue's staging area
    wait_lgkmcnt<0>();
    __syncthreads();

    // Epilogue through LDS: two passes of 128 rows (rows of accumulator block
    // i = pass * MTP + ii of both wave rows).  A thread owns the fixed 4-column
    // group c of the tile (a wave covers one whole 256-column row per step, so
    // LDS reads and global accesses are contiguous) and walks rows
    // wave, wave + 4, ...; the per-element loads of EPI_BATCH rows are issued
    // before any of them is consumed, so the loop keeps that many in flight
    // instead of paying one memory latency per row.
    constexpr int EPI_BATCH = 8;
    constexpr int ROWS_PER_THREAD = PROWS / C::NWAVES;   // 32 per pass
    static_assert(ROWS_PER_THREAD % EPI_BATCH == 0, "epilogue batch");
    static_assert(C::BN / 4 == 64, "one wave per 256-column row");
    float *E = reinterpret_cast<float *>(smem);
    const uint32_t c = lane * 4u;
    const typename Epi::Col col = Epi::column(ep, n0 + c);
#pragma unroll
    for (int pass = 0; pass < C::MT / MTP; ++pass) {
#pragma unroll
        for (int ii = 0; ii < MTP; ++ii) {
            const int i = pass * MTP + ii;
            const uint32_t r = (wm * MTP + ii) * 32 + frow;
#pragma unroll
            for (int j = 0; j < C::NTL; ++j)
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const uint32_t cc = wn * C::TWN + j * 32 + gq * 8 + fhalf * 4;
                    floatx4 v = {acc[i][j][4 * gq + 0], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                 acc[i][j][4 * gq + 3]};
                    *reinterpret_cast<floatx4 *>(E + r * EPITCH + cc) = v;
                }
        }
        __syncthreads();
#pragma unroll 1
        for (int b = 0; b < ROWS_PER_THREAD; b += EPI_BATCH) {
            typename Epi::Pre pre[EPI_BATCH];
            uint32_t mrow[EPI_BATCH];
#pragma unroll
            for (int u = 0; u < EPI_BATCH; ++u) {
                // E row r holds tile row wmi * TWM + pass * MTP * 32 + rr
                const uint32_t r = wave + (uint32_t)C::NWAVES * (b + u);
                const uint32_t wmi = r / (MTP * 32), rr = r % (MTP * 32);
                mrow[u] = m0 + wmi * C::TWM + pass * MTP * 32 + rr;
                Epi::load(ep, (uint64_t)mrow[u] * Epi::ldc(ep) + n0 + c, mrow[u], pre[u]);
            }
#pragma unroll
            for (int u = 0; u < EPI_BATCH; ++u) {
                const uint32_t r = wave + (uint32_t)C::NWAVES * (b + u);
                const floatx4 v = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c);
                Epi::finish(ep, (uint64_t)mrow[u] * Epi::ldc(ep) + n0 + c, mrow[u], n0 + c, v, col, pre[u]);
            }
        }
        __syncthreads();
    }
}

}  // namespace skl
