// gemm_dma.h — fp16 GEMM for the all-k-contiguous layout on whole 256x256
// tiles (M % 256 == N % 256 == 0, K % 64 == 0), gfx950.
//
//  * 8 waves (2 per SIMD), wave tile 128 x 64 of v_mfma_f32_32x32x16_f16.
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
//    reads of the next tile's first k-step, so the MFMA pipe has work while
//    the new LDS reads are in flight.
//  * Per tile: wait for this wave's DMA of the next tile (vmcnt 0: it is the
//    only one outstanding), s_barrier without a fence (LDS DMA completion is
//    what vmcnt tracks), then DMA tile kt+2 into the stage every wave has just
//    finished reading.
// Operand offsets are 32-bit (rows * ld * 2 bytes < 4 GiB).
#pragma once

#include "gemm.h"

namespace skl {

struct Dma64 {
    static constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 4, NT = 512, NWAVES = 8;
    static constexpr int TWM = BM / WM, TWN = BN / WN, MT = TWM / 32, NTL = TWN / 32;
    static constexpr int ROWB = BK * 2;            // 128 bytes per LDS row
    static constexpr int OPB = 256 * ROWB;         // 32 KB per operand tile
    static constexpr int STAGEB = 2 * OPB;         // 64 KB per stage
    static constexpr int NINSTR = 2 * OPB / 1024;  // 64 DMA instructions per stage
    static constexpr int IPW = NINSTR / NWAVES;    // 8 per wave
};

typedef __attribute__((address_space(3))) char lds_char;
typedef const __attribute__((address_space(3))) u32x4 lds_u32x4;

__device__ __forceinline__ void dma16(const char *src, lds_char *dst) {
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src),
                                     reinterpret_cast<__attribute__((address_space(3))) void *>(dst), 16, 0, 0);
}

// vmcnt(n) with expcnt / lgkmcnt left alone (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// lgkmcnt(0) with vmcnt / expcnt left alone.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

template <class Epi>
__global__ void __launch_bounds__(512)
    gemm_dma_kernel(GemmShape sh, const half_t *__restrict__ A, const half_t *__restrict__ B, typename Epi::Params ep) {
    typedef Dma64 C;
    constexpr int EPITCH = C::BN + 4;
    constexpr int EPI_BYTES = C::WM * 2 * 32 * EPITCH * 4;
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

    // DMA instructions of a stage: q = 0..31 fill A rows 8q..8q+7, q = 32..63
    // fill B rows 8(q-32)..; instruction q belongs to wave q % 8.
    const uint32_t lrow = lane >> 3;
    uint32_t goff[C::IPW];
#pragma unroll
    for (int t = 0; t < C::IPW; ++t) {
        const uint32_t q = wave + (uint32_t)C::NWAVES * t;
        const bool is_b = q >= 32;
        const uint32_t row = (q & 31u) * 8u + lrow;
        const uint32_t kc = (lane & 7u) ^ ((row >> 1) & 7u);
        goff[t] = ((is_b ? n0 : m0) + row) * (is_b ? sh.ldb : sh.lda) * 2u + kc * 16u;
    }
    const char *Ab = reinterpret_cast<const char *>(A);
    const char *Bb = reinterpret_cast<const char *>(B);

    auto issue = [&](int kt, int stage) {
        const uint32_t kb = (uint32_t)kt * C::BK * 2u;
        lds_char *st = lsm + stage * C::STAGEB;
#pragma unroll
        for (int t = 0; t < C::IPW; ++t) {
            const uint32_t q = wave + (uint32_t)C::NWAVES * t;
            const bool is_b = q >= 32;
            dma16((is_b ? Bb : Ab) + kb + goff[t], st + (is_b ? C::OPB : 0) + (q & 31u) * 1024u);
        }
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
    const uint32_t a_row = (wm * C::TWM + frow) * C::ROWB;
    const uint32_t b_row = C::OPB + (wn * C::TWN + frow) * C::ROWB;

    u32x4 fa[2][C::MT], fb[2][C::NTL];
    auto read = [&](int set, int stage, int ks) {
        const lds_char *st = lsm + stage * C::STAGEB;
        const uint32_t c = ((2u * ks) ^ g) * 16u;
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
            fa[set][i] = *reinterpret_cast<lds_u32x4 *>(st + a_row + c + i * 32 * C::ROWB);
#pragma unroll
        for (int j = 0; j < C::NTL; ++j)
            fb[set][j] = *reinterpret_cast<lds_u32x4 *>(st + b_row + c + j * 32 * C::ROWB);
    };
    auto mma = [&](int set) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int j = 0; j < C::NTL; ++j) Mfma<half_t>::run(acc[i][j], fb[set][j], fa[set][i]);
    };

    // prologue: tile 0 resident, tile 1 in flight, first fragments read
    issue(0, 0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (nk > 1) issue(1, 1);
    read(0, 0, 0);

    for (int kt0 = 0; kt0 < nk; kt0 += 2) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kt = kt0 + s;
            if (kt >= nk) break;
            read(1, s, 1);
            mma(0);
            read(0, s, 2);
            mma(1);
            read(1, s, 3);
            mma(0);
            // k-step 3: cross the barrier before issuing its MFMAs
            wait_lgkm0();                      // set 1 (k-step 3) is in registers
            if (kt + 1 < nk) {
                wait_vmcnt<0>();               // this wave's DMA of tile kt+1 landed
                __builtin_amdgcn_s_barrier();  // everyone's landed; stage s fully read
                if (kt + 2 < nk) issue(kt + 2, s);
                read(0, s ^ 1, 0);
            }
            mma(1);
        }
    }
    __syncthreads();

    // Epilogue through LDS (two passes of 128 rows), as in gemm_kernel.
    constexpr int MTP = 2;
    constexpr int PROWS = C::WM * MTP * 32;
    float *E = reinterpret_cast<float *>(smem);
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
                    const uint32_t c = wn * C::TWN + j * 32 + gq * 8 + fhalf * 4;
                    floatx4 v = {acc[i][j][4 * gq + 0], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                 acc[i][j][4 * gq + 3]};
                    *reinterpret_cast<floatx4 *>(E + r * EPITCH + c) = v;
                }
        }
        __syncthreads();
#pragma unroll 1
        for (uint32_t q = tid; q < (uint32_t)(PROWS * C::BN / 4); q += C::NT) {
            const uint32_t r = q / (C::BN / 4);
            const uint32_t c = (q % (C::BN / 4)) * 4;
            const uint32_t wmi = r / (MTP * 32);
            const uint32_t rr = r % (MTP * 32);
            const uint32_t m = m0 + wmi * C::TWM + pass * MTP * 32 + rr;
            const floatx4 v = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c);
            Epi::apply(ep, sh, m, n0 + c, v, 0);
        }
        __syncthreads();
    }
}

}  // namespace skl
