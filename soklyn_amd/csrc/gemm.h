// gemm.h — MFMA GEMM core for gfx950 (CDNA4, wave64).
//
//   C[M x N] = sum_k A(m, k) * B(k, n)       fp32 accumulation
//   A(m, k) = A_KCONTIG ? A[m * lda + k] : A[k * lda + m]
//   B(k, n) = B_KCONTIG ? B[n * ldb + k] : B[k * ldb + n]
//
// The three DenseBlock contractions map onto it as
//   forward  Z  = X . W        A = X  (k-contig),  B = W   (n-contig, or W^T k-contig)
//   dX       s  = dP . W^T     A = dP (k-contig),  B = W   (k-contig)
//   dW       dW = X^T . dP     A = X  (m-contig),  B = dP  (n-contig, or both transposed: k-contig)
//
// Design:
//  * Block tile BM x BN x BK, WM x WN waves, each wave owns a (BM/WM) x (BN/WN)
//    sub-tile built from 32x32 MFMA tiles (v_mfma_f32_32x32x16_f16 for fp16,
//    v_mfma_f32_32x32x2_f32 for fp32).
//  * LDS holds both operands k-contiguous in 16-byte chunks (8 halves / 4
//    floats per chunk, 8 chunks per row), double buffered.  When both
//    operands are k-contiguous in HBM, rows are padded to 9 chunks: 8
//    consecutive rows start 9 chunks apart (conflict-free 16-byte reads) and
//    every fragment / staging address is a per-lane base plus a compile-time
//    offset.  Otherwise the 8 chunks of a row are XOR-swizzled by
//    (row ^ row >> 3) & 7, which also keeps the transposed staging writes
//    conflict-free.
//  * Operands that are not k-contiguous in HBM are transposed in registers
//    while staging (8x8 halves with v_perm_b32, 4x4 floats by renaming).
//  * Interior tiles with a whole number of K-tiles run a loop with no bounds
//    checks at all; edge tiles run the guarded loop.
//  * The MFMA is issued with the operands swapped (B fragment as the "A"
//    input), so each lane ends up owning 4 consecutive output columns of one
//    row; the accumulator tile then goes through LDS to a compact epilogue
//    loop in which consecutive lanes own consecutive 4-column groups.
//  * Workgroup -> tile mapping is XCD-aware: consecutive tiles of an
//    8 x TN group land on one XCD so they share that XCD's L2.
//  * Optional split-K over blockIdx.z (partials go to a workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_math.h"

namespace skl {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GemmShape {
    uint32_t M, N, K;        // output rows, output cols, reduction length
    uint32_t lda, ldb;       // leading dimensions (elements)
    uint32_t k_per_split;    // reduction length per split (multiple of BK)
    uint32_t tiles_m, tiles_n;
    uint32_t mv, nv;         // 256x256 kernel on zero-padded operands: the real output extent
    uint32_t m_base;         // direct-to-LDS kernel: first output row of the launch's tiles
};

// Workgroup barrier that orders LDS only: wait for this wave's LDS accesses,
// then s_barrier.  __syncthreads() also waits for every outstanding global
// access (its release fence), which would stall on the next tile's loads in the
// k loop and on the epilogue's global stores; neither needs ordering here.  The
// empty asm statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS chunk index of (row, kc) in a k-contiguous tile.
template <bool PADDED> struct LdsLayout;
template <> struct LdsLayout<true> {
    static constexpr int PITCH = 9;   // chunks per row (8 data + 1 pad)
    __device__ __forceinline__ static uint32_t idx(uint32_t row, uint32_t kc) { return row * 9u + kc; }
};
template <> struct LdsLayout<false> {
    static constexpr int PITCH = 8;
    __device__ __forceinline__ static uint32_t idx(uint32_t row, uint32_t kc) {
        return row * 8u + (kc ^ ((row ^ (row >> 3)) & 7u));
    }
};

template <typename T> struct Mfma;

template <> struct Mfma<half_t> {
    static constexpr int VEC = 8;       // elements per 16-byte chunk
    static constexpr int KSTEP = 16;    // k covered by one chunk per lane-half
    __device__ __forceinline__ static void run(floatx16 &acc, const u32x4 &bop, const u32x4 &aop) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, bop),
                                                     __builtin_bit_cast(halfx8, aop), acc, 0, 0, 0);
    }
};

template <> struct Mfma<float> {
    static constexpr int VEC = 4;
    static constexpr int KSTEP = 8;     // 4 MFMAs of k=2, lane-half h holds k = 4h + s
    // The four k-slices are spelled out with constant lanes: an unrolled
    // `bop[s]` loop here was compiled to four MFMAs on lane 0 only.
    __device__ __forceinline__ static void run(floatx16 &acc, const u32x4 &bop, const u32x4 &aop) {
        const floatx4 b = __builtin_bit_cast(floatx4, bop);
        const floatx4 a = __builtin_bit_cast(floatx4, aop);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b.x, a.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b.y, a.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b.z, a.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b.w, a.w, acc, 0, 0, 0);
    }
};

// 8x8 transpose of halves: in[i] holds row i (8 halves); out[j] gets column j.
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            out[j][p] = __builtin_amdgcn_perm(in[2 * p + 1][j >> 1], in[2 * p][j >> 1], sel);
    }
}

// 4x4 transpose of floats (register renaming only).
__device__ __forceinline__ void transpose4x4(const u32x4 (&in)[4], u32x4 (&out)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int p = 0; p < 4; ++p) out[j][p] = in[p][j];
}

// Global -> register staging of one operand tile (ROWS x BK, k-contiguous in LDS).
//  KCONTIG: global element (row, k) at p[row * ld + k]
//  else   : global element (row, k) at p[k * ld + row]
// VECOK: ld, the contiguous extent and the base are multiples of VEC
// elements, so whole 16-byte chunks are either fully in range or fully out.
// GUARD = false: the caller guarantees the whole tile is in range.
template <typename T, int ROWS, int BK, int NT, bool KCONTIG, bool VECOK, bool PADDED>
struct Stager {
    typedef LdsLayout<PADDED> L;
    static constexpr int VEC = Mfma<T>::VEC;
    static constexpr int KC = BK / VEC;                 // chunks per LDS row (8)
    static_assert(KC == 8, "LDS rows must hold 8 chunks");
    // k-contiguous: one 16-byte chunk per slot.
    static constexpr int NCHUNK = ROWS * KC;
    static_assert(NCHUNK % NT == 0, "tile chunks must divide over threads");
    static constexpr int PER = NCHUNK / NT;
    // otherwise: VEC x VEC blocks (VEC k-rows of VEC contiguous elements).
    static constexpr int NBLK = (ROWS / VEC) * KC;
    static_assert(NBLK % NT == 0 || NT % NBLK == 0, "blocks must divide over threads");
    static constexpr int BPER = NBLK >= NT ? NBLK / NT : 1;
    static constexpr int BACTIVE = NBLK >= NT ? NT : NBLK;   // threads holding a block
    static constexpr int NREG = KCONTIG ? PER : BPER * VEC;

    u32x4 r[NREG];

    __device__ __forceinline__ static u32x4 load_chunk(const T *p, uint64_t off) {
        return *reinterpret_cast<const u32x4 *>(p + off);
    }

    // Element-wise gather for shapes that are not 16-byte friendly.
    __device__ __forceinline__ static u32x4 gather(const T *p, uint32_t ld, uint32_t row, uint32_t k,
                                                   uint32_t rows, uint32_t kmax) {
        T v[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const uint32_t rr = KCONTIG ? row : row + e;
            const uint32_t kk = KCONTIG ? k + e : k;
            v[e] = (rr < rows && kk < kmax)
                       ? (KCONTIG ? p[(uint64_t)rr * ld + kk] : p[(uint64_t)kk * ld + rr])
                       : (T)0;
        }
        return __builtin_bit_cast(u32x4, v);
    }

    template <bool GUARD>
    __device__ __forceinline__ void load(const T *p, uint32_t ld, uint32_t row0, uint32_t k0, uint32_t rows,
                                         uint32_t kmax, uint32_t tid) {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const uint32_t c = tid + i * NT;
                const uint32_t row = row0 + c / KC;
                const uint32_t k = k0 + (c % KC) * VEC;
                if constexpr (!VECOK) {
                    r[i] = gather(p, ld, row, k, rows, kmax);
                } else if constexpr (GUARD) {
                    r[i] = (row < rows && k < kmax) ? load_chunk(p, (uint64_t)row * ld + k) : u32x4{0, 0, 0, 0};
                } else {
                    r[i] = load_chunk(p, (uint64_t)row * ld + k);
                }
            }
        } else {
            if (NBLK < NT && tid >= (uint32_t)BACTIVE) return;
#pragma unroll
            for (int b = 0; b < BPER; ++b) {
                const uint32_t blk = tid + b * NT;
                const uint32_t rb = blk % (ROWS / VEC);
                const uint32_t kb = blk / (ROWS / VEC);
                const uint32_t row = row0 + rb * VEC;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const uint32_t k = k0 + kb * VEC + e;
                    if constexpr (!VECOK) {
                        r[b * VEC + e] = gather(p, ld, row, k, rows, kmax);
                    } else if constexpr (GUARD) {
                        r[b * VEC + e] = (row < rows && k < kmax) ? load_chunk(p, (uint64_t)k * ld + row)
                                                                   : u32x4{0, 0, 0, 0};
                    } else {
                        r[b * VEC + e] = load_chunk(p, (uint64_t)k * ld + row);
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(u32x4 *lds, uint32_t tid) const {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const uint32_t c = tid + i * NT;
                lds[L::idx(c / KC, c % KC)] = r[i];
            }
        } else {
            if (NBLK < NT && tid >= (uint32_t)BACTIVE) return;
#pragma unroll
            for (int b = 0; b < BPER; ++b) {
                const uint32_t blk = tid + b * NT;
                const uint32_t rb = blk % (ROWS / VEC);
                const uint32_t kb = blk / (ROWS / VEC);
                u32x4 in[VEC], t[VEC];
#pragma unroll
                for (int e = 0; e < VEC; ++e) in[e] = r[b * VEC + e];
                if constexpr (VEC == 8) {
                    transpose8x8(in, t);
                } else {
                    transpose4x4(in, t);
                }
#pragma unroll
                for (int e = 0; e < VEC; ++e) lds[L::idx(rb * VEC + e, kb)] = t[e];
            }
        }
    }
};

// Maps a linear workgroup id to an output tile (tm, tn): XCD-contiguous
// chunks, then groups of GROUP_M tile rows.  Workgroup w runs on XCD w % 8, so
// XCD x works through tiles [x total / 8, (x + 1) total / 8) of the grouped
// order; with GROUP_M = 4 an XCD's 32 concurrent 256x256 tiles of the C3
// shapes are 4 tile rows x 8 tile columns, and its second round reuses the
// same 4 A row panels from its L2 (2-4% faster than GROUP_M = 8 on the C3
// forward and dX; 16 is slower).
__device__ __forceinline__ void tile_coords_grouped(uint32_t t, uint32_t tiles_m, uint32_t tiles_n, uint32_t &tm,
                                                    uint32_t &tn) {
    constexpr uint32_t GROUP_M = 4;
    const uint32_t per_group = GROUP_M * tiles_n;
    const uint32_t group = t / per_group;
    const uint32_t first_m = group * GROUP_M;
    const uint32_t gsize = min(tiles_m - first_m, GROUP_M);
    const uint32_t in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}
__device__ __forceinline__ void tile_coords(uint32_t wg, uint32_t tiles_m, uint32_t tiles_n, uint32_t &tm,
                                            uint32_t &tn) {
    const uint32_t total = tiles_m * tiles_n;
    uint32_t t = wg;
    if ((total & 7u) == 0) t = (wg & 7u) * (total >> 3) + (wg >> 3);
    tile_coords_grouped(t, tiles_m, tiles_n, tm, tn);
}

// The K loop: double-buffered LDS, register prefetch one K-tile ahead,
// unrolled by two so each half works on a compile-time buffer.
template <typename T, int BM, int BN, int BK, int WM, int WN, bool A_KCONTIG, bool B_KCONTIG, bool VECOK,
          bool PADDED>
struct MainLoop {
    static constexpr int NT = WM * WN * 64;
    static constexpr int VEC = Mfma<T>::VEC;
    static constexpr int KSTEP = Mfma<T>::KSTEP;
    static constexpr int TWM = BM / WM, TWN = BN / WN;
    static constexpr int MT = TWM / 32, NTL = TWN / 32;
    static constexpr int PITCH = LdsLayout<PADDED>::PITCH;
    static constexpr int A_CHUNKS = BM * PITCH, B_CHUNKS = BN * PITCH;
    static constexpr int STAGE = A_CHUNKS + B_CHUNKS;
    typedef Stager<T, BM, BK, NT, A_KCONTIG, VECOK, PADDED> SA;
    typedef Stager<T, BN, BK, NT, B_KCONTIG, VECOK, PADDED> SB;

    template <int BUF>
    __device__ __forceinline__ static void compute(const u32x4 *smem, floatx16 (&acc)[MT][NTL], uint32_t wm,
                                                   uint32_t wn, uint32_t frow, uint32_t fhalf) {
        const u32x4 *as = smem + BUF * STAGE;
        const u32x4 *bs = as + A_CHUNKS;
#pragma unroll
        for (int ks = 0; ks < BK / KSTEP; ++ks) {
            const uint32_t kc = (uint32_t)ks * 2u + fhalf;
            u32x4 af[MT], bf[NTL];
            if constexpr (PADDED) {
                const u32x4 *ab = as + (wm * TWM + frow) * PITCH + fhalf;
                const u32x4 *bb = bs + (wn * TWN + frow) * PITCH + fhalf;
#pragma unroll
                for (int i = 0; i < MT; ++i) af[i] = ab[i * 32 * PITCH + ks * 2];
#pragma unroll
                for (int j = 0; j < NTL; ++j) bf[j] = bb[j * 32 * PITCH + ks * 2];
            } else {
#pragma unroll
                for (int i = 0; i < MT; ++i) af[i] = as[LdsLayout<false>::idx(wm * TWM + i * 32 + frow, kc)];
#pragma unroll
                for (int j = 0; j < NTL; ++j) bf[j] = bs[LdsLayout<false>::idx(wn * TWN + j * 32 + frow, kc)];
            }
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NTL; ++j) Mfma<T>::run(acc[i][j], bf[j], af[i]);
        }
    }

    template <bool GUARD, int BUF>
    __device__ __forceinline__ static void step(u32x4 *smem, floatx16 (&acc)[MT][NTL], SA &sa, SB &sb,
                                                const GemmShape &sh, const T *A, const T *B, uint32_t m0,
                                                uint32_t n0, uint32_t kbeg, uint32_t kend, int kt, int nk,
                                                uint32_t tid, uint32_t wm, uint32_t wn, uint32_t frow,
                                                uint32_t fhalf) {
        const bool more = kt + 1 < nk;
        if (more) {
            const uint32_t k0 = kbeg + (uint32_t)(kt + 1) * BK;
            sa.template load<GUARD>(A, sh.lda, m0, k0, sh.M, kend, tid);
            sb.template load<GUARD>(B, sh.ldb, n0, k0, sh.N, kend, tid);
        }
        compute<BUF>(smem, acc, wm, wn, frow, fhalf);
        if (more) {
            u32x4 *nxt = smem + (BUF ^ 1) * STAGE;
            sa.store(nxt, tid);
            sb.store(nxt + A_CHUNKS, tid);
        }
        lds_barrier();
    }

    template <bool GUARD>
    __device__ __forceinline__ static void run(u32x4 *smem, floatx16 (&acc)[MT][NTL], const GemmShape &sh,
                                               const T *A, const T *B, uint32_t m0, uint32_t n0, uint32_t kbeg,
                                               uint32_t kend, int nk, uint32_t tid, uint32_t wm, uint32_t wn,
                                               uint32_t frow, uint32_t fhalf) {
        SA sa;
        SB sb;
        sa.template load<GUARD>(A, sh.lda, m0, kbeg, sh.M, kend, tid);
        sb.template load<GUARD>(B, sh.ldb, n0, kbeg, sh.N, kend, tid);
        sa.store(smem, tid);
        sb.store(smem + A_CHUNKS, tid);
        lds_barrier();
        for (int kt = 0; kt < nk; kt += 2) {
            step<GUARD, 0>(smem, acc, sa, sb, sh, A, B, m0, n0, kbeg, kend, kt, nk, tid, wm, wn, frow, fhalf);
            if (kt + 1 < nk)
                step<GUARD, 1>(smem, acc, sa, sb, sh, A, B, m0, n0, kbeg, kend, kt + 1, nk, tid, wm, wn, frow,
                               fhalf);
        }
    }
};

// The GEMM kernel.  Epi provides:
//   struct Params;
//   static void apply(const Params&, const GemmShape&, uint32_t m, uint32_t n, floatx4 v, uint32_t split)
// called once per (row m, 4 consecutive columns n..n+3) the lane owns; it must
// bounds-check m < M and n + j < N itself.
template <typename T, int BM, int BN, int BK, int WM, int WN, bool A_KCONTIG, bool B_KCONTIG, bool VECOK,
          class Epi>
__global__ void __launch_bounds__(WM *WN * 64)
    gemm_kernel(GemmShape sh, const T *__restrict__ A, const T *__restrict__ B, typename Epi::Params ep) {
    constexpr bool PADDED = A_KCONTIG && B_KCONTIG;
    typedef MainLoop<T, BM, BN, BK, WM, WN, A_KCONTIG, B_KCONTIG, VECOK, PADDED> ML;
    constexpr int NT = ML::NT;
    constexpr int TWM = ML::TWM, TWN = ML::TWN;
    constexpr int MT = ML::MT, NTL = ML::NTL;
    constexpr int MAIN_CHUNKS = 2 * ML::STAGE;
    constexpr int EPITCH = BN + 4;                      // floats per staged epilogue row (bank skew)
    constexpr int EPI_CHUNKS = (WM * ((MT >= 2) ? 2 : 1) * 32 * EPITCH) / 4;
    __shared__ u32x4 smem[MAIN_CHUNKS > EPI_CHUNKS ? MAIN_CHUNKS : EPI_CHUNKS];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t frow = lane & 31u;   // row within a 32-row MFMA tile
    const uint32_t fhalf = lane >> 5;   // k lane-half

    uint32_t tm, tn;
    tile_coords(blockIdx.x, sh.tiles_m, sh.tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kbeg = blockIdx.z * sh.k_per_split;
    const uint32_t kend = min(sh.K, kbeg + sh.k_per_split);
    const int nk = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;

    floatx16 acc[MT][NTL];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTL; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (nk > 0) {
        const bool interior = m0 + BM <= sh.M && n0 + BN <= sh.N && (kend - kbeg) % BK == 0;
        if (VECOK && interior)
            ML::template run<false>(smem, acc, sh, A, B, m0, n0, kbeg, kend, nk, tid, wm, wn, frow, fhalf);
        else
            ML::template run<true>(smem, acc, sh, A, B, m0, n0, kbeg, kend, nk, tid, wm, wn, frow, fhalf);
    }

    // Epilogue.  The accumulator tile goes through LDS (in passes when it is
    // larger than the LDS arena) so that the per-element epilogue runs as one
    // compact loop in which consecutive lanes own consecutive 4-column groups
    // of a row: coalesced HBM traffic and no per-register code duplication.
    // Lane layout after the swapped MFMA: C[m][n..n+3] with
    // m = wave row + 32 i + (lane & 31), n = wave col + 32 j + 8 g + 4 (lane >> 5).
    constexpr int ARENA = (int)(sizeof(smem) / 4);      // floats
    constexpr int MTP = (WM * MT * 32 * EPITCH <= ARENA) ? MT : (MT >= 2 ? 2 : 1);
    static_assert(MT % MTP == 0, "epilogue passes");
    constexpr int PROWS = WM * MTP * 32;                // staged rows per pass
    float *E = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int pass = 0; pass < MT / MTP; ++pass) {
#pragma unroll
        for (int ii = 0; ii < MTP; ++ii) {
            const int i = pass * MTP + ii;
            const uint32_t r = (wm * MTP + ii) * 32 + frow;
#pragma unroll
            for (int j = 0; j < NTL; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t c = wn * TWN + j * 32 + g * 8 + fhalf * 4;
                    floatx4 v = {acc[i][j][4 * g + 0], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                 acc[i][j][4 * g + 3]};
                    *reinterpret_cast<floatx4 *>(E + r * EPITCH + c) = v;
                }
        }
        lds_barrier();
#pragma unroll 1
        for (uint32_t q = tid; q < (uint32_t)(PROWS * BN / 4); q += NT) {
            const uint32_t r = q / (BN / 4);
            const uint32_t c = (q % (BN / 4)) * 4;
            const uint32_t wmi = r / (MTP * 32);
            const uint32_t rr = r % (MTP * 32);
            const uint32_t m = m0 + wmi * TWM + pass * MTP * 32 + rr;
            const floatx4 v = *reinterpret_cast<const floatx4 *>(E + r * EPITCH + c);
            Epi::apply(ep, sh, m, n0 + c, v, blockIdx.z);
        }
        if (pass + 1 < MT / MTP) lds_barrier();   // E is rewritten by the next pass
    }
}

}  // namespace skl
