// gemm.hip — GEMM epilogues and launchers for the three DenseBlock
// contractions (forward, dX, dW) on gfx950.
#include <stdlib.h>

#include "gemm.h"
#include "gemm_dma.h"
#include "launch.h"

namespace skl {

template <typename T> __device__ __forceinline__ T ld_t(const void *p, uint64_t i) {
    return reinterpret_cast<const T *>(p)[i];
}
template <typename T> __device__ __forceinline__ void st_t(void *p, uint64_t i, T v) {
    reinterpret_cast<T *>(p)[i] = v;
}

// ---- forward: bias (+ act + dropout) ------------------------------------------
//
// Every epilogue has a whole-vector form in three parts, so a caller can batch
// the global loads of many 4-column groups before computing any of them:
//   column(e, n)        per-column operands of columns n..n+3 (loaded once)
//   load(e, idx, m, p)  per-element operands of row m, columns n..n+3
//   finish(e, idx, m, n, v, col, p)  compute from the fp32 accumulators v, store
// apply() handles one 4-column group, including ragged edges.
template <typename T> struct EpiFwdK {
    typedef FwdEpi Params;
    __device__ __forceinline__ static uint32_t ldc(const FwdEpi &e) { return e.ldc; }
    __device__ __forceinline__ static FwdEpi at_split(const FwdEpi &e, uint32_t) { return e; }
    struct Col { f32x4 bias; };
    struct Pre {};
    __device__ __forceinline__ static Col column(const FwdEpi &e, uint32_t n) {
        Col c;
        c.bias = e.bias ? load4<T>(e.bias, n) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        return c;
    }
    __device__ __forceinline__ static void load(const FwdEpi &, uint64_t, uint32_t, Pre &) {}
    __device__ __forceinline__ static void finish(const FwdEpi &e, uint64_t idx, uint32_t m, uint32_t n, floatx4 v,
                                                  const Col &col, const Pre &) {
        // 4 consecutive columns: one 8-byte (fp16) / 16-byte (fp32) access per tensor
        f32x4 z = v;
        if (e.bias) z = z + col.bias;
        store4<T>(e.z_out, idx, z);
        if (!e.fuse_act) return;
        const f32x4 zt = round4<T>(z);
        f32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = activation(e.act, zt[j], e.leaky);
        store4<T>(e.predrop, idx, a);
        if (e.use_dropout) {
            const float scale = 1.0f / (1.0f - e.p);
            f32x4 mk, o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool keep = dropout_u(n + j, m, e.seed + m * 7u) >= e.p;
                mk[j] = keep ? scale : 0.0f;
                o[j] = keep ? a[j] * scale : 0.0f;
            }
            store4<T>(e.mask, idx, mk);
            store4<T>(e.out, idx, o);
        } else {
            store4<T>(e.out, idx, a);
        }
    }
    __device__ __forceinline__ static void apply(const FwdEpi &e, const GemmShape &sh, uint32_t m, uint32_t n,
                                                 floatx4 v, uint32_t) {
        if (m >= sh.M) return;
        if (n + 3 < sh.N && (e.ldc & 3u) == 0) {
            finish(e, (uint64_t)m * e.ldc + n, m, n, v, column(e, n), Pre{});
            return;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = n + j;
            if (c >= sh.N) break;
            float z = v[j];
            if (e.bias) z = z + to_f32(ld_t<T>(e.bias, c));   // f32 acc + f32(b), one rounding
            const T zt = from_f32<T>(z);
            const uint64_t idx = (uint64_t)m * e.ldc + c;
            st_t<T>(e.z_out, idx, zt);
            if (e.fuse_act) {
                const float a = activation(e.act, to_f32(zt), e.leaky);
                st_t<T>(e.predrop, idx, from_f32<T>(a));
                if (e.use_dropout) {
                    if (dropout_u(c, m, e.seed + m * 7u) >= e.p) {
                        const float scale = 1.0f / (1.0f - e.p);
                        st_t<T>(e.mask, idx, from_f32<T>(scale));
                        st_t<T>(e.out, idx, from_f32<T>(a * scale));
                    } else {
                        st_t<T>(e.mask, idx, (T)0);
                        st_t<T>(e.out, idx, (T)0);
                    }
                } else {
                    st_t<T>(e.out, idx, from_f32<T>(a));
                }
            }
        }
    }
};

// ---- plain fp32 store (input gradient; split-K partials) -----------------------
struct EpiStoreK {
    typedef StoreEpi Params;
    __device__ __forceinline__ static uint32_t ldc(const StoreEpi &e) { return e.ldc; }
    // the partial plane of split-K slice `split`
    __device__ __forceinline__ static StoreEpi at_split(const StoreEpi &e, uint32_t split) {
        StoreEpi r = e;
        r.out += (uint64_t)split * e.split_stride;
        return r;
    }
    struct Col {};
    struct Pre {};
    __device__ __forceinline__ static Col column(const StoreEpi &, uint32_t) { return Col{}; }
    __device__ __forceinline__ static void load(const StoreEpi &, uint64_t, uint32_t, Pre &) {}
    __device__ __forceinline__ static void finish(const StoreEpi &e, uint64_t idx, uint32_t, uint32_t, floatx4 v,
                                                  const Col &, const Pre &) {
        *reinterpret_cast<floatx4 *>(e.out + idx) = v;
    }
    __device__ __forceinline__ static void apply(const StoreEpi &e, const GemmShape &sh, uint32_t m, uint32_t n,
                                                 floatx4 v, uint32_t split) {
        if (m >= sh.M) return;
        float *o = e.out + (uint64_t)split * e.split_stride + (uint64_t)m * e.ldc;
        if (n + 3 < sh.N && (e.ldc & 3u) == 0) {
            *reinterpret_cast<floatx4 *>(o + n) = v;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (n + j < sh.N) o[n + j] = v[j];
        }
    }
};

// ---- dW + optimiser on W (fused) -----------------------------------------------
template <typename T> struct EpiOptK {
    typedef OptEpi Params;
    __device__ __forceinline__ static uint32_t ldc(const OptEpi &e) { return e.ldc; }
    __device__ __forceinline__ static OptEpi at_split(const OptEpi &e, uint32_t) { return e; }
    struct Col {};
    struct Pre { floatx4 p, dv, dm; };
    __device__ __forceinline__ static Col column(const OptEpi &, uint32_t) { return Col{}; }
    __device__ __forceinline__ static void load(const OptEpi &e, uint64_t idx, uint32_t, Pre &q) {
        q.p = *reinterpret_cast<const floatx4 *>(e.master + idx);
        q.dv = *reinterpret_cast<const floatx4 *>(e.dv + idx);
        q.dm = *reinterpret_cast<const floatx4 *>(e.dm + idx);
    }
    __device__ __forceinline__ static void finish(const OptEpi &e, uint64_t idx, uint32_t, uint32_t, floatx4 v,
                                                  const Col &, const Pre &q) {
        floatx4 p = q.p, dv = q.dv, dm = q.dm;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float pj = p[j], vj = dv[j], mj = dm[j];
            optimiser_step(pj, vj, mj, v[j] * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt, e.regularisation,
                           e.regu_coeff, true);
            p[j] = pj; dv[j] = vj; dm[j] = mj;
        }
        *reinterpret_cast<floatx4 *>(e.master + idx) = p;
        *reinterpret_cast<floatx4 *>(e.dv + idx) = dv;
        *reinterpret_cast<floatx4 *>(e.dm + idx) = dm;
        if (e.param) {
            T t[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) t[j] = from_f32<T>(p[j]);
            if constexpr (sizeof(T) == 2) {
                *reinterpret_cast<uint64_t *>(reinterpret_cast<T *>(e.param) + idx) = __builtin_bit_cast(uint64_t, t);
            } else {
                *reinterpret_cast<floatx4 *>(reinterpret_cast<T *>(e.param) + idx) = __builtin_bit_cast(floatx4, t);
            }
        }
    }
    __device__ __forceinline__ static void apply(const OptEpi &e, const GemmShape &sh, uint32_t m, uint32_t n,
                                                 floatx4 v, uint32_t) {
        if (m >= sh.M) return;
        const uint64_t base = (uint64_t)m * e.ldc;
        if (n + 3 < sh.N && (e.ldc & 3u) == 0) {
            Pre q;
            load(e, base + n, m, q);
            finish(e, base + n, m, n, v, Col{}, q);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t c = n + j;
                if (c >= sh.N) break;
                const uint64_t idx = base + c;
                float pj = e.master[idx], vj = e.dv[idx], mj = e.dm[idx];
                optimiser_step(pj, vj, mj, v[j] * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt, e.regularisation,
                               e.regu_coeff, true);
                e.master[idx] = pj;
                e.dv[idx] = vj;
                e.dm[idx] = mj;
                if (e.param) st_t<T>(e.param, idx, from_f32<T>(pj));
            }
        }
    }
};

// ---- tile configurations ----------------------------------------------------------
template <typename T, int BM, int BN, int BK, int WM, int WN> struct Cfg {
    typedef T type;
    static constexpr int bm = BM, bn = BN, bk = BK, wm = WM, wn = WN, nt = WM * WN * 64;
};
typedef Cfg<half_t, 256, 256, 64, 2, 4> CfgH256w8;   // 8 waves, 128x64 per wave, 2 waves / SIMD
typedef Cfg<half_t, 128, 128, 64, 2, 2> CfgH128;
typedef Cfg<float, 128, 128, 32, 2, 2> CfgF128;
typedef Cfg<float, 64, 64, 32, 2, 2> CfgF64;

template <class C, bool AK, bool BK_, bool VOK, class Epi>
static hipError_t run(const GemmLaunch &g, const typename Epi::Params &p, hipStream_t s) {
    typedef typename C::type T;
    GemmShape sh;
    sh.M = g.M;
    sh.N = g.N;
    sh.K = g.K;
    sh.lda = g.lda;
    sh.ldb = g.ldb;
    sh.tiles_m = (g.M + C::bm - 1) / C::bm;
    sh.tiles_n = (g.N + C::bn - 1) / C::bn;
    const uint32_t splits = g.splits ? g.splits : 1;
    const uint32_t kps_raw = (g.K + splits - 1) / splits;
    sh.k_per_split = ((kps_raw + C::bk - 1) / C::bk) * C::bk;
    dim3 grid(sh.tiles_m * sh.tiles_n, 1, splits);
    hipLaunchKernelGGL((gemm_kernel<T, C::bm, C::bn, C::bk, C::wm, C::wn, AK, BK_, VOK, Epi>), grid,
                       dim3(C::nt), 0, s, sh, reinterpret_cast<const T *>(g.A),
                       reinterpret_cast<const T *>(g.B), p);
    return hipGetLastError();
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Decide whether both operands can be staged in 16-byte chunks.
static bool vec_ok(const GemmLaunch &g, int vec) {
    // contiguous extent of A: K if k-contig else M; of B: K if k-contig else N
    const uint32_t a_ext = g.a_kcontig ? g.K : g.M;
    const uint32_t b_ext = g.b_kcontig ? g.K : g.N;
    return (g.lda % vec) == 0 && (g.ldb % vec) == 0 && (a_ext % vec) == 0 && (b_ext % vec) == 0 &&
           aligned16(g.A) && aligned16(g.B);
}

template <class C, bool AK, bool BK_, class Epi>
static hipError_t dispatch_vec(const GemmLaunch &g, const typename Epi::Params &p, hipStream_t s) {
    constexpr int VEC = Mfma<typename C::type>::VEC;
    if (g.a_kcontig != AK || g.b_kcontig != BK_) return hipErrorInvalidValue;
    return vec_ok(g, VEC) ? run<C, AK, BK_, true, Epi>(g, p, s) : run<C, AK, BK_, false, Epi>(g, p, s);
}

// Only the (layout, epilogue) pairs the DenseBlock path uses are instantiated:
//   forward  : A k-contig, B n-contig
//   dX       : A k-contig, B k-contig
//   dW       : A m-contig, B n-contig
template <class C> static hipError_t dispatch_op(const GemmLaunch &g, hipStream_t s) {
    typedef typename C::type T;
    switch (g.op) {
    // forward on W or on a transposed copy of W
    case Op::Fwd:
        return g.b_kcontig ? dispatch_vec<C, true, true, EpiFwdK<T>>(g, g.fwd, s)
                           : dispatch_vec<C, true, false, EpiFwdK<T>>(g, g.fwd, s);
    case Op::InputGrad: return dispatch_vec<C, true, true, EpiStoreK>(g, g.st, s);
    // dW also runs on transposed copies of X and dP (both k-contiguous)
    case Op::DwPartial:
        return g.a_kcontig ? dispatch_vec<C, true, true, EpiStoreK>(g, g.st, s)
                           : dispatch_vec<C, false, false, EpiStoreK>(g, g.st, s);
    case Op::DwOpt:
        return g.a_kcontig ? dispatch_vec<C, true, true, EpiOptK<T>>(g, g.opt, s)
                           : dispatch_vec<C, false, false, EpiOptK<T>>(g, g.opt, s);
    }
    return hipErrorInvalidValue;
}

// The 256x256 tile only runs the all-k-contiguous layout (large fp16
// problems are given transposed operands by the caller).
template <class C> static hipError_t dispatch_kk(const GemmLaunch &g, hipStream_t s) {
    typedef typename C::type T;
    switch (g.op) {
    case Op::Fwd: return dispatch_vec<C, true, true, EpiFwdK<T>>(g, g.fwd, s);
    case Op::InputGrad:
    case Op::DwPartial: return dispatch_vec<C, true, true, EpiStoreK>(g, g.st, s);
    case Op::DwOpt: return dispatch_vec<C, true, true, EpiOptK<T>>(g, g.opt, s);
    }
    return hipErrorInvalidValue;
}

bool gemm_large_tile(uint32_t dtype, uint32_t M, uint32_t N) {
    return dtype == 1 && ((M + 255) / 256) * ((N + 255) / 256) >= 192;
}

// Output tiles of the general (non-256) configuration; drives split-K.
uint32_t gemm_tiles(uint32_t dtype, uint32_t M, uint32_t N) {
    if (dtype == 1) return ((M + 127) / 128) * ((N + 127) / 128);
    const uint32_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (t128 >= 192) return t128;
    return ((M + 63) / 64) * ((N + 63) / 64);
}

uint32_t gemm_bk(uint32_t dtype) { return dtype == 1 ? 64 : 32; }

// The direct-to-LDS 256x256 kernel (gemm_dma.h).  SOKLYN_GEMM_DMA=0 selects
// the register-staged kernels instead (A/B comparisons).
bool gemm_dma_enabled() {
    static bool on = [] {
        const char *e = getenv("SOKLYN_GEMM_DMA");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

// Operand layouts the direct-to-LDS kernel is instantiated for: every op with
// both operands k-contiguous, the forward on W as stored (n-contiguous), and dW
// on X and dP as stored (m- and n-contiguous).
static bool dma_layout_ok(const GemmLaunch &g) {
    if (g.a_kcontig && g.b_kcontig) return true;
    if (g.op == Op::Fwd) return g.a_kcontig && !g.b_kcontig;
    if (g.op == Op::DwOpt || g.op == Op::DwPartial) return !g.a_kcontig && !g.b_kcontig;
    return false;
}

static uint32_t epi_ldc(const GemmLaunch &g) {
    switch (g.op) {
    case Op::Fwd: return g.fwd.ldc;
    case Op::InputGrad:
    case Op::DwPartial: return g.st.ldc;
    case Op::DwOpt: return g.opt.ldc;
    }
    return 0;
}

// The operands as given fit the 256x256 kernel: fp16, whole tiles, K a multiple
// of 128 (two k-tiles), 16-byte rows, 32-bit byte offsets within each operand.
bool gemm_dma_shape_ok(const GemmLaunch &g) {
    if (!gemm_dma_enabled() || g.dtype != 1 || !dma_layout_ok(g)) return false;
    if ((g.M % 256) || (g.N % 256) || (g.K % 128) || g.K == 0) return false;
    if (!vec_ok(g, 8)) return false;
    const uint64_t a_rows = g.a_kcontig ? g.M : g.K, b_rows = g.b_kcontig ? g.N : g.K;
    return a_rows * g.lda * 2 < (1ull << 32) && b_rows * g.ldb * 2 < (1ull << 32);
}

// Whole output tiles with a 4-aligned leading dimension: the batched epilogue.
static bool dma_full_epilogue(const GemmLaunch &g) {
    const uint32_t mv = g.mv ? g.mv : g.M, nv = g.nv ? g.nv : g.N;
    return mv == g.M && nv == g.N && epi_ldc(g) % 4 == 0;
}

bool gemm_direct_ok(const GemmLaunch &g) {
    return gemm_large_tile(g.dtype, g.M, g.N) && gemm_dma_shape_ok(g) && dma_full_epilogue(g) &&
           (g.splits == 0 || g.splits == 1);
}

// Waves per workgroup: 8 when an operand is read through the transposing LDS
// path (its 8-byte reads leave one wave per SIMD waiting on LDS latency), 4
// when both operands are k-contiguous (see gemm_dma.h).
template <class Epi, bool AK, bool BK_>
static hipError_t run_dma(const GemmLaunch &g, const typename Epi::Params &p, uint32_t splits, uint32_t kps,
                          hipStream_t s) {
    constexpr int NW = (AK && BK_) ? 4 : 8;
    GemmShape sh{};
    sh.M = g.M;
    sh.N = g.N;
    sh.K = g.K;
    sh.lda = g.lda;
    sh.ldb = g.ldb;
    sh.k_per_split = kps;
    sh.tiles_m = g.M / 256;
    sh.tiles_n = g.N / 256;
    sh.mv = g.mv ? g.mv : g.M;
    sh.nv = g.nv ? g.nv : g.N;
    const dim3 grid(sh.tiles_m * sh.tiles_n, splits);
    const half_t *A = reinterpret_cast<const half_t *>(g.A);
    const half_t *B = reinterpret_cast<const half_t *>(g.B);
    if (dma_full_epilogue(g))
        hipLaunchKernelGGL((gemm_dma_kernel<Epi, AK, BK_, NW, false>), grid, dim3(DmaCfg<NW>::NT), 0, s, sh, A, B,
                           p);
    else
        hipLaunchKernelGGL((gemm_dma_kernel<Epi, AK, BK_, NW, true>), grid, dim3(DmaCfg<NW>::NT), 0, s, sh, A, B,
                           p);
    return hipGetLastError();
}

hipError_t launch_gemm_dma(const GemmLaunch &g, hipStream_t s) {
    if (!gemm_dma_shape_ok(g)) return hipErrorInvalidValue;
    // split-K: slices of k_per_split (a multiple of 128), the last one possibly shorter
    const uint32_t splits_req = g.splits ? g.splits : 1;
    const uint32_t kps = ((g.K / splits_req + 127) / 128) * 128;
    const uint32_t splits = (g.K + kps - 1) / kps;
    if (splits > 1 && g.op != Op::DwPartial) return hipErrorInvalidValue;
    const bool kk = g.a_kcontig && g.b_kcontig;
    switch (g.op) {
    case Op::Fwd:
        return kk ? run_dma<EpiFwdK<half_t>, true, true>(g, g.fwd, splits, kps, s)
                  : run_dma<EpiFwdK<half_t>, true, false>(g, g.fwd, splits, kps, s);
    case Op::InputGrad: return run_dma<EpiStoreK, true, true>(g, g.st, splits, kps, s);
    case Op::DwPartial:
        return kk ? run_dma<EpiStoreK, true, true>(g, g.st, splits, kps, s)
                  : run_dma<EpiStoreK, false, false>(g, g.st, splits, kps, s);
    case Op::DwOpt:
        return kk ? run_dma<EpiOptK<half_t>, true, true>(g, g.opt, splits, kps, s)
                  : run_dma<EpiOptK<half_t>, false, false>(g, g.opt, splits, kps, s);
    }
    return hipErrorInvalidValue;
}

// Split-K slices launch_gemm_dma makes of K for `splits` requested.
uint32_t gemm_dma_splits(uint32_t K, uint32_t splits) {
    const uint32_t kps = ((K / (splits ? splits : 1) + 127) / 128) * 128;
    return (K + kps - 1) / kps;
}

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t s) {
    if (g.M == 0 || g.N == 0) return hipSuccess;
    if (gemm_direct_ok(g)) return launch_gemm_dma(g, s);
    if (g.dtype == 1) {
        if (gemm_large_tile(g.dtype, g.M, g.N) && g.a_kcontig && g.b_kcontig) return dispatch_kk<CfgH256w8>(g, s);
        return dispatch_op<CfgH128>(g, s);
    }
    const uint32_t t128 = ((g.M + 127) / 128) * ((g.N + 127) / 128);
    return t128 >= 192 ? dispatch_op<CfgF128>(g, s) : dispatch_op<CfgF64>(g, s);
}

}  // namespace skl
