// gemm.hip — GEMM epilogues and launchers for the three DenseBlock
// contractions (forward, dX, dW) on gfx950.
#include <stdlib.h>

#include <hip/hip_ext.h>

#include "gemm.h"
#include "gemm_dma.h"
#include "launch.h"

namespace skl {

// Launches a GEMM kernel; with g.time_start / g.time_stop set, the dispatch
// itself carries the timing events.
template <typename K, typename... Args>
static void launch_timed(const GemmLaunch &g, K kernel, dim3 grid, dim3 block, hipStream_t s, Args... args) {
    if (g.time_start || g.time_stop)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, s, g.time_start, g.time_stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}


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
        store4_nt<T>(e.z_out, idx, z);
        if (!e.fuse_act) return;
        const f32x4 zt = round4<T>(z);
        f32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = activation<T>(e.act, zt[j], e.leaky);
        store4_nt<T>(e.predrop, idx, a);
        if (e.use_dropout) {
            const float scale = 1.0f / (1.0f - e.p);
            f32x4 mk, o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool keep = dropout_u(n + j, m, e.seed + m * 7u) >= e.p;
                mk[j] = keep ? scale : 0.0f;
                o[j] = keep ? a[j] * scale : 0.0f;
            }
            store4_nt<T>(e.mask, idx, mk);
            store4_nt<T>(e.out, idx, o);
        } else {
            store4_nt<T>(e.out, idx, a);
        }
    }
    // 8 consecutive columns (fp16 outputs: 16-byte stores)
    static constexpr int kVec = sizeof(T) == 2 ? 8 : 4;
    struct Col8 { f32x4 lo, hi; };
    __device__ __forceinline__ static Col8 column8(const FwdEpi &e, uint32_t n) {
        Col8 c;
        c.lo = e.bias ? load4<T>(e.bias, n) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        c.hi = e.bias ? load4<T>(e.bias, n + 4) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        return c;
    }
    __device__ __forceinline__ static void st8(void *p, uint64_t idx, f32x4 lo, f32x4 hi) {
        const half_t h[8] = {(half_t)lo[0], (half_t)lo[1], (half_t)lo[2], (half_t)lo[3],
                             (half_t)hi[0], (half_t)hi[1], (half_t)hi[2], (half_t)hi[3]};
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(h),
                                    reinterpret_cast<u32x4 *>(reinterpret_cast<half_t *>(p) + idx));
    }
    __device__ __forceinline__ static void finish8(const FwdEpi &e, uint64_t idx, uint32_t m, uint32_t n, floatx4 v0,
                                                   floatx4 v1, const Col8 &col) {
        f32x4 z0 = v0, z1 = v1;
        if (e.bias) {
            z0 = z0 + col.lo;
            z1 = z1 + col.hi;
        }
        st8(e.z_out, idx, z0, z1);
        if (!e.fuse_act) return;
        const f32x4 t0 = round4<T>(z0), t1 = round4<T>(z1);
        f32x4 a0, a1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a0[j] = activation<T>(e.act, t0[j], e.leaky);
            a1[j] = activation<T>(e.act, t1[j], e.leaky);
        }
        st8(e.predrop, idx, a0, a1);
        if (e.use_dropout) {
            const float scale = 1.0f / (1.0f - e.p);
            f32x4 m0, m1, o0, o1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool k0 = dropout_u(n + j, m, e.seed + m * 7u) >= e.p;
                const bool k1 = dropout_u(n + 4 + j, m, e.seed + m * 7u) >= e.p;
                m0[j] = k0 ? scale : 0.0f;
                o0[j] = k0 ? a0[j] * scale : 0.0f;
                m1[j] = k1 ? scale : 0.0f;
                o1[j] = k1 ? a1[j] * scale : 0.0f;
            }
            st8(e.mask, idx, m0, m1);
            st8(e.out, idx, o0, o1);
        } else {
            st8(e.out, idx, a0, a1);
        }
    }
    // one element (ragged tiles): per-column operands loaded once per column
    struct Col1 { float bias; };
    __device__ __forceinline__ static Col1 column1(const FwdEpi &e, uint32_t n) {
        return Col1{e.bias ? to_f32(ld_t<T>(e.bias, n)) : 0.0f};
    }
    __device__ __forceinline__ static void apply1(const FwdEpi &e, uint32_t m, uint32_t n, float v, const Col1 &col,
                                                  uint32_t) {
        float z = v;
        if (e.bias) z = z + col.bias;   // f32 acc + f32(b), one rounding
        const T zt = from_f32<T>(z);
        const uint64_t idx = (uint64_t)m * e.ldc + n;
        st_t<T>(e.z_out, idx, zt);
        if (!e.fuse_act) return;
        const float a = activation<T>(e.act, to_f32(zt), e.leaky);
        st_t<T>(e.predrop, idx, from_f32<T>(a));
        if (e.use_dropout) {
            if (dropout_u(n, m, e.seed + m * 7u) >= e.p) {
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
                const float a = activation<T>(e.act, to_f32(zt), e.leaky);
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
    static constexpr int kDmaSpacing = 1;   // front-loaded refill (measured fastest for dX)
    static constexpr int kReadsPerMfma = 1; // 32x32 schedule (the split-K dW partial)
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
        __builtin_nontemporal_store(v, reinterpret_cast<floatx4 *>(e.out + idx));
    }
    // one-wave-per-SIMD tiles: from the accumulator registers (half-line row segments,
    // so a plain store the L2 can join)
    static constexpr bool kDirect = true;
    static constexpr int kDirectBatch = 8;
    __device__ __forceinline__ static void direct(const StoreEpi &e, uint64_t idx, uint32_t, uint32_t, floatx4 v,
                                                  const Pre &) {
        *reinterpret_cast<floatx4 *>(e.out + idx) = v;
    }
    struct Col1 {};
    __device__ __forceinline__ static Col1 column1(const StoreEpi &, uint32_t) { return Col1{}; }
    __device__ __forceinline__ static void apply1(const StoreEpi &e, uint32_t m, uint32_t n, float v, const Col1 &,
                                                  uint32_t split) {
        e.out[(uint64_t)split * e.split_stride + (uint64_t)m * e.ldc + n] = v;
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
    typedef T elem;
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
    __device__ __forceinline__ static void finish(const OptEpi &e, uint64_t idx, uint32_t m, uint32_t n, floatx4 v,
                                                  const Col &, const Pre &q) {
        floatx4 p = q.p, dv = q.dv, dm = q.dm;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float pj = p[j], vj = dv[j], mj = dm[j];
            const float g = dw_checked<T>(e, m, n + j, v[j]);
            optimiser_step<sizeof(T) == 2>(pj, vj, mj, g * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt,
                                           e.regularisation, e.regu_coeff, true);
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
    struct Col1 {};
    __device__ __forceinline__ static Col1 column1(const OptEpi &, uint32_t) { return Col1{}; }
    __device__ __forceinline__ static void apply1(const OptEpi &e, uint32_t m, uint32_t n, float v, const Col1 &,
                                                  uint32_t) {
        const uint64_t idx = (uint64_t)m * e.ldc + n;
        float pj = e.master[idx], vj = e.dv[idx], mj = e.dm[idx];
        const float g = dw_checked<T>(e, m, n, v);
        optimiser_step<sizeof(T) == 2>(pj, vj, mj, g * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt,
                                       e.regularisation, e.regu_coeff, true);
        e.master[idx] = pj;
        e.dv[idx] = vj;
        e.dm[idx] = mj;
        if (e.param) st_t<T>(e.param, idx, from_f32<T>(pj));
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
                const float g = dw_checked<T>(e, m, c, v[j]);
                optimiser_step<sizeof(T) == 2>(pj, vj, mj, g * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt,
                                               e.regularisation, e.regu_coeff, true);
                e.master[idx] = pj;
                e.dv[idx] = vj;
                e.dm[idx] = mj;
                if (e.param) st_t<T>(e.param, idx, from_f32<T>(pj));
            }
        }
    }
};

// ---- hidden-layer error from the dX sum (fused) -----------------------------------
// compute_hidden_layer_error_kernel's epilogue (backward.cu:79-100) on the sum in
// the accumulators: e = mask * act'(s, predrop, preact); grad = e; the element-
// local norm gradient (util.cu:175-215, loss scale 1) into d_prenorm, its fp16
// copy and dNorm; and per-thread running column sums of d_prenorm / dNorm_w /
// dNorm_b, which flush() reduces over the 8 waves in a fixed order into the
// tile's row of partials (the inputs of the bias / norm-parameter update).
template <typename T> struct EpiErrK {
    typedef ErrEpi Params;
    static constexpr bool kColSums = true;
    __device__ __forceinline__ static uint32_t ldc(const ErrEpi &e) { return e.ldc; }
    __device__ __forceinline__ static ErrEpi at_split(const ErrEpi &e, uint32_t) { return e; }
    // per-column operands of 4 columns: the norm weight, and BatchNorm's per-column rstd
    struct Col { f32x4 nw, rstd; };
    // per-element operands of one row's 4 columns, as loaded (T)
    struct Pre { f16x4 pd, pa, mk, pn; float rstd; };
    // running sums of the thread's 4 columns
    struct Acc { f32x4 dp, nw, nb; };
    __device__ __forceinline__ static Col column(const ErrEpi &e, uint32_t n) {
        Col c;
        c.nw = e.norm ? load4<float>(e.nw, n) : f32x4{0, 0, 0, 0};
        c.rstd = e.norm == 3 ? load4<T>(e.norm_rstd, n) : f32x4{0, 0, 0, 0};
        return c;
    }
    // nontemporal: the forward caches are read once here (C4's fused hidden error
    // 0.268 -> 0.262 ms against plain loads)
    __device__ __forceinline__ static f16x4 ld4h(const void *p, uint64_t idx) {
        return __builtin_nontemporal_load(reinterpret_cast<const f16x4 *>(reinterpret_cast<const half_t *>(p) + idx));
    }
    __device__ __forceinline__ static void load(const ErrEpi &e, uint64_t idx, uint32_t m, Pre &q) {
        static_assert(sizeof(T) == 2, "the 256x256 kernel is fp16");
        q.pd = ld4h(e.predrop, idx);
        q.pa = ld4h(e.preact, idx);
        q.mk = ld4h(e.mask, idx);
        q.pn = e.norm ? ld4h(e.norm == 1 ? e.prenorm : e.centered, idx) : f16x4{0, 0, 0, 0};
        q.rstd = (e.norm == 1 || e.norm == 2) ? to_f32(reinterpret_cast<const T *>(e.norm_rstd)[m]) : 0.0f;
    }
    __device__ __forceinline__ static void finish(const ErrEpi &e, uint64_t idx, uint32_t, uint32_t, floatx4 v,
                                                  const Col &col, const Pre &q, Acc &acc) {
        f32x4 g, dp, dnw = {0, 0, 0, 0}, dnb = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g[j] = (float)q.mk[j] * activation_derivative<T>(e.act, v[j], (float)q.pd[j], (float)q.pa[j], e.leaky);
            dp[j] = g[j];
            if (e.norm) {
                const float p = (float)q.pn[j];
                const NormGrad ng = norm_grad(e.norm, g[j], p, p, e.norm == 3 ? col.rstd[j] : q.rstd, col.nw[j],
                                              e.inv_n, e.inv_m);
                dp[j] = ng.d_prenorm;
                dnw[j] = ng.dnw;
                dnb[j] = ng.dnb;
            }
        }
        __builtin_nontemporal_store(g, reinterpret_cast<f32x4 *>(e.grad + idx));
        *reinterpret_cast<f32x4 *>(e.d_prenorm + idx) = dp;
        *reinterpret_cast<f16x4 *>(e.d_prenorm_h + idx) = f16x4{(half_t)dp[0], (half_t)dp[1], (half_t)dp[2],
                                                                (half_t)dp[3]};
        if (e.norm) {
            __builtin_nontemporal_store(dnw, reinterpret_cast<f32x4 *>(e.d_norm_w + idx));
            __builtin_nontemporal_store(dnb, reinterpret_cast<f32x4 *>(e.d_norm_b + idx));
        }
        acc.dp += dp;
        acc.nw += dnw;
        acc.nb += dnb;
    }
    struct Col1 {};   // no element-by-element form: whole tiles only
    // The tile's column sums: each of the NW waves leaves its 3 x 256 running sums
    // in LDS (column 4 lane + j of the tile), then the block adds the waves in
    // order 0..NW-1 and writes the columns < ncols of partials[tm][k].  lds:
    // NW x 3 x 256 floats; the caller has made sure no wave still reads it.
    template <int NW, int BN>
    __device__ __forceinline__ static void flush(const ErrEpi &e, const Acc &acc, float *lds, uint32_t tid,
                                                 uint32_t tm, uint32_t n0) {
        // thread (wave, lane) holds the sums of columns 4 (lane % CPL) .. + 3 over
        // its rows; slot wave RPS + lane / CPL of the NW RPS partials per column
        constexpr uint32_t CPL = BN / 4, RPS = 64 / CPL, SLOTS = NW * RPS;
        const uint32_t lane = tid & 63u, wave = tid >> 6;
        const uint32_t slot = wave * RPS + lane / CPL;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = 4u * (lane % CPL) + j;
            lds[(slot * 3 + 0) * BN + c] = acc.dp[j];
            lds[(slot * 3 + 1) * BN + c] = acc.nw[j];
            lds[(slot * 3 + 2) * BN + c] = acc.nb[j];
        }
        __syncthreads();
        for (uint32_t t = tid; t < 3 * BN; t += 64 * NW) {
            const uint32_t k = t / BN, c = t % BN;
            if ((k > 0 && !e.norm) || n0 + c >= e.ncols) continue;
            float s = 0.0f;
#pragma unroll
            for (uint32_t w = 0; w < SLOTS; ++w) s += lds[(w * 3 + k) * BN + c];
            e.partials[((uint64_t)tm * 3 + k) * e.ncols + n0 + c] = s;
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
// fp32: 8 waves of 64x32 on a 128x128 tile (two per SIMD hide each other's LDS and
// barrier waits; C2 on 256 tiles, one workgroup per CU: dX 75.6 -> 72.0 us, step +2.3%
// against 4 waves of 64x64)
typedef Cfg<float, 128, 128, 32, 2, 4> CfgF128;
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
    launch_timed(g, gemm_kernel<T, C::bm, C::bn, C::bk, C::wm, C::wn, AK, BK_, VOK, Epi>, grid, dim3(C::nt), s, sh,
                 reinterpret_cast<const T *>(g.A), reinterpret_cast<const T *>(g.B), p);
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
    case Op::HiddenErr: break;   // the 256x256 kernel only
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
    case Op::HiddenErr: break;   // the 256x256 kernel only
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

uint32_t gemm_dma_tile_forced() {
    static uint32_t t = [] {
        const char *e = getenv("SOKLYN_GEMM_TILE");
        const int v = e ? atoi(e) : 0;
        return v == 128 || v == 256 ? (uint32_t)v : 0u;
    }();
    return t;
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
    case Op::HiddenErr: return g.err.ldc;
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

// The fused error epilogue's 4-column accesses need every per-element buffer
// 16-byte aligned (fp32) / 8-byte aligned (fp16 at a multiple of 4 elements).
static bool err_epi_aligned(const ErrEpi &e) {
    const void *p[] = {e.predrop, e.preact, e.mask, e.grad, e.d_prenorm, e.d_prenorm_h,
                       e.norm ? e.d_norm_w : nullptr, e.norm ? e.d_norm_b : nullptr,
                       e.norm == 1 ? e.prenorm : nullptr, e.norm >= 2 ? e.centered : nullptr,
                       e.norm ? e.nw : nullptr, e.norm == 3 ? e.norm_rstd : nullptr};
    for (const void *q : p)
        if (q && !aligned16(q)) return false;
    return true;
}

// The hidden error of an M x N output can be fused into the 256x256 kernel:
// whole tiles (no padded output), 4-aligned rows, aligned buffers.  Ragged
// outputs keep the GEMM + error kernel pair: an element-by-element form of the
// fused epilogue was measured 1.3x slower than that pair on config 5's shapes.
bool hidden_err_fusable(const ErrEpi &e, uint32_t M, uint32_t N) {
    return M % 256 == 0 && N % 256 == 0 && e.ldc % 4 == 0 && err_epi_aligned(e);
}

// Whole output tiles with a 4-aligned leading dimension: the batched epilogue.
static bool dma_full_epilogue(const GemmLaunch &g) {
    const uint32_t mv = g.mv ? g.mv : g.M, nv = g.nv ? g.nv : g.N;
    if (g.op == Op::HiddenErr && !err_epi_aligned(g.err)) return false;
    return mv == g.M && nv == g.N && epi_ldc(g) % 4 == 0;
}

bool gemm_direct_ok(const GemmLaunch &g) {
    return gemm_large_tile(g.dtype, g.M, g.N) && gemm_dma_shape_ok(g) && dma_full_epilogue(g) &&
           (g.splits == 0 || g.splits == 1);
}

// 256x256: 4 waves (one per SIMD, 16x16x32 MFMAs on AGPR accumulators) for the
// epilogues DmaOneWave selects on whole tiles; otherwise 8 waves (two per SIMD: one
// issues MFMAs while the other waits on LDS; see gemm_dma.h) with
// v_mfma_f32_16x16x32_f16 when A is k-contiguous (C3 shapes: dX 2% faster back to
// back, 5% with a cold last-level cache; forward 2-3%) and 32x32x16 when both
// operands are transposed, whose 16x16 fragments at 8 waves overflow the register
// budget even with A single-buffered.  128x128: 4 waves of 64x64, two workgroups per
// CU, 16x16x32 for every layout.
template <class Epi, bool AK, bool BK_, int NW, int MI, int BT>
static hipError_t run_dma_t(const GemmLaunch &g, const typename Epi::Params &p, uint32_t splits, uint32_t kps,
                            hipStream_t s) {
    GemmShape sh{};
    sh.M = g.M;
    sh.N = g.N;
    sh.K = g.K;
    sh.lda = g.lda;
    sh.ldb = g.ldb;
    sh.k_per_split = kps;
    sh.tiles_m = (g.m_rows ? g.m_rows : g.M) / BT;
    sh.tiles_n = g.N / BT;
    sh.m_base = g.m_begin;
    sh.mv = g.mv ? g.mv : g.M;
    sh.nv = g.nv ? g.nv : g.N;
    const dim3 grid(sh.tiles_m * sh.tiles_n, splits);
    const half_t *A = reinterpret_cast<const half_t *>(g.A);
    const half_t *B = reinterpret_cast<const half_t *>(g.B);
    if (dma_full_epilogue(g))
        launch_timed(g, gemm_dma_kernel<Epi, AK, BK_, NW, false, MI, BT>, grid, dim3(64 * NW), s, sh, A, B, p);
    else if constexpr (EpiSums<Epi>::value || (NW == 4 && BT == 256))
        return hipErrorInvalidValue;   // whole tiles only (hidden_err_fusable; the one-wave-per-SIMD tile)
    else
        launch_timed(g, gemm_dma_kernel<Epi, AK, BK_, NW, true, MI, BT>, grid, dim3(64 * NW), s, sh, A, B, p);
    return hipGetLastError();
}

// Epilogues that run the 256x256 tile with one wave per SIMD (4 waves, 16x16x32 MFMAs
// on AGPR accumulators, a third fewer LDS fragment bytes per flop than 8 waves): the
// fp32 store (dX, split-K dW partials) and the fused optimiser.  Measured on the C3
// shapes against 8 waves on one box: main loop 4% faster per k for dX and dW; dX
// 213.1 -> 207.7 us, dW + Adam 281.3 -> 267.8 us.  The forward and the fused hidden
// error keep 8 waves: their store-heavy epilogues run slower with half the threads
// (forward 225.0 -> 241.3 us).
template <class Epi> struct DmaOneWave { static constexpr bool value = false; };
template <> struct DmaOneWave<EpiStoreK> { static constexpr bool value = true; };
template <> struct DmaOneWave<EpiOptK<half_t>> { static constexpr bool value = true; };

template <class Epi, bool AK, bool BK_>
static hipError_t run_dma(const GemmLaunch &g, const typename Epi::Params &p, uint32_t splits, uint32_t kps,
                          hipStream_t s) {
    if (g.tile == 128) return run_dma_t<Epi, AK, BK_, 4, 16, 128>(g, p, splits, kps, s);
    if constexpr (DmaOneWave<Epi>::value)
        if (dma_full_epilogue(g)) return run_dma_t<Epi, AK, BK_, 4, 16, 256>(g, p, splits, kps, s);
    return run_dma_t<Epi, AK, BK_, 8, AK ? 16 : 32, 256>(g, p, splits, kps, s);
}

hipError_t launch_gemm_dma(const GemmLaunch &g, hipStream_t s) {
    if (!gemm_dma_shape_ok(g)) return hipErrorInvalidValue;
    // split-K: slices of k_per_split (a multiple of 128), the last one possibly shorter
    const uint32_t splits_req = g.splits ? g.splits : 1;
    const uint32_t kps = ((g.K / splits_req + 127) / 128) * 128;
    const uint32_t splits = (g.K + kps - 1) / kps;
    if (splits > 1 && g.op != Op::DwPartial) return hipErrorInvalidValue;
    if (g.m_rows || g.m_begin) {
        // a band of output rows: whole tiles inside M, not the column-sum epilogue
        const uint32_t t = g.tile == 128 ? 128u : 256u;
        if (g.op == Op::HiddenErr || g.m_begin % 256 || g.m_rows % t || g.m_rows == 0 ||
            (uint64_t)g.m_begin + g.m_rows > g.M)
            return hipErrorInvalidValue;
    }
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
    case Op::HiddenErr:
        return kk ? run_dma<EpiErrK<half_t>, true, true>(g, g.err, splits, kps, s) : hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

// Split-K slices launch_gemm_dma makes of K for `splits` requested.
uint32_t gemm_dma_splits(uint32_t K, uint32_t splits) {
    const uint32_t kps = ((K / (splits ? splits : 1) + 127) / 128) * 128;
    return (K + kps - 1) / kps;
}

// ---- skinny outputs (N <= 16) ---------------------------------------------------------
// The output layers of the MLP configurations have 10 and 13 columns: a 256x256
// (or 128x128) MFMA tile would be >90% padding, and the work is a stream over X.
constexpr uint32_t SKINNY_N = 16;
constexpr uint32_t SKINNY_LDS = 96 * 1024;

// Sum of v[0..15] over the wave by recursive halving: each xor-shuffle step sends
// half of the values a lane still holds and keeps the other half, so lane l ends
// with column (l >> 2) & 15 summed over its 4 lanes after 8+4+2+1 shuffles, then 2
// more finish it (17 in all, fixed order).  Returns the column sum lane l holds.
__device__ __forceinline__ float wave_sum16(float (&v)[SKINNY_N], uint32_t lane) {
#pragma unroll
    for (int h = 8, m = 32; h >= 1; h >>= 1, m >>= 1) {
        const bool up = (lane & (uint32_t)m) != 0;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float send = up ? v[i] : v[i + h];
            const float keep = up ? v[i + h] : v[i];
            v[i] = keep + __shfl_xor(send, m, 64);
        }
    }
    float t = v[0];
    t += __shfl_xor(t, 2, 64);
    t += __shfl_xor(t, 1, 64);
    return t;
}

// Forward, one wave per row: lane l takes the 8-element k chunks l, l + 64, ... of
// the row (one 16-byte load per chunk on 16-byte aligned rows, 8 element loads
// otherwise: a wave still covers 512 consecutive elements), and for each of the 16
// columns one 16-byte LDS read of W^T (staged n-major, rows of Kp = K rounded up to
// 8, zero past K and past N) feeds 8 FMAs into the lane's partial column sums.  The
// sums are reduced over the wave, and the lane holding column n < N runs the forward
// epilogue for it (bias, act, dropout, the three cache stores).  One workgroup per CU
// stages W once for all of its rows.
template <typename T, bool VECX>
__global__ void __launch_bounds__(1024) skinny_fwd_kernel(GemmShape sh, const T *__restrict__ A,
                                                          const T *__restrict__ B, FwdEpi ep) {
    constexpr int CH = 8;   // k per chunk
    __shared__ __attribute__((aligned(16))) T ws[SKINNY_LDS / sizeof(T)];
    const uint32_t K = sh.K, N = sh.N, Kp = (K + CH - 1) / CH * CH;
    for (uint32_t i = threadIdx.x; i < SKINNY_N * Kp; i += blockDim.x) {
        const uint32_t n = i / Kp, k = i - n * Kp;
        ws[i] = (n < N && k < K) ? B[(uint64_t)k * sh.ldb + n] : (T)0;
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    for (uint32_t m = blockIdx.x * waves + wave; m < sh.M; m += gridDim.x * waves) {
        float acc[SKINNY_N];
#pragma unroll
        for (int n = 0; n < (int)SKINNY_N; ++n) acc[n] = 0.0f;
        const T *x = A + (uint64_t)m * sh.lda;
#pragma unroll 2
        for (uint32_t k0 = lane * CH; k0 < K; k0 += 64 * CH) {
            T xv[CH];
            if (VECX && k0 + CH <= K) {
                static_assert(sizeof(xv) % 16 == 0, "chunk of whole 16-byte words");
#pragma unroll
                for (int q = 0; q < (int)(sizeof(xv) / 16); ++q)
                    reinterpret_cast<u32x4 *>(xv)[q] = reinterpret_cast<const u32x4 *>(x + k0)[q];
            } else {
#pragma unroll
                for (int e = 0; e < CH; ++e) xv[e] = k0 + e < K ? x[k0 + e] : (T)0;
            }
#pragma unroll
            for (int n = 0; n < (int)SKINNY_N; ++n) {
                T w8[CH];
#pragma unroll
                for (int q = 0; q < (int)(sizeof(w8) / 16); ++q)
                    reinterpret_cast<u32x4 *>(w8)[q] = reinterpret_cast<const u32x4 *>(ws + n * Kp + k0)[q];
#pragma unroll
                for (int e = 0; e < CH; ++e) acc[n] = fmaf(to_f32(xv[e]), to_f32(w8[e]), acc[n]);
            }
        }
        const float z = wave_sum16(acc, lane);
        const uint32_t n = (lane >> 2) & 15u;
        if ((lane & 3u) == 0 && n < N) {
            GemmShape one = sh;   // column n alone
            one.N = n + 1;
            EpiFwdK<T>::apply(ep, one, m, n, floatx4{z, 0.0f, 0.0f, 0.0f}, 0);
        }
    }
}

// The same on MFMA (fp16): a quad of 4 waves takes a block of 16 rows (one 16 x 16
// output block, columns past N zero), wave w of the quad the k-chunks w, w + 4, ...
// of 32 k, each a v_mfma_f32_16x16x32_f16 with lane l feeding X[row l % 16][k + 8
// (l / 16) .. + 7] and W^T[column l % 16][same k] (LDS rows of P halves, P = 8
// mod 128: the 16 rows of a read sit in distinct banks).  Rows that are not 16-byte
// aligned are cut out of the two aligned 16-byte chunks covering them (funnel
// shifts; the second chunk only when it holds a row element), k past K reads as
// zero.  The quad's 4 partial blocks are added in wave order in LDS, and the
// forward epilogue runs per element (lane l: rows 4 (l / 16) .. + 3 of column
// l % 16, whose bias is loaded once).  One workgroup of 16 waves per CU stages W^T
// once; every quad runs the same number of row-block rounds (barriers).
constexpr uint32_t SKINNY_MFMA_P_MAX = 4104;   // LDS row pitch bound (K <= 4096): 16 rows + the sums fit 160 KB
__device__ __forceinline__ halfx8 skinny_x8(const half_t *__restrict__ A, uint64_t rb, uint32_t k, uint32_t K,
                                           uint64_t in_elems, bool vecx) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const uint64_t e = rb + k;
    u32x4v v = {0, 0, 0, 0};
    if (vecx) {
        v = *reinterpret_cast<const u32x4v *>(A + e);
    } else {
        const uint64_t a0 = e & ~7ull;
        const uint32_t sh = (uint32_t)(e - a0);   // halves past the aligned chunk
        const u32x4v lo = *reinterpret_cast<const u32x4v *>(A + a0);
        const u32x4v hi = (sh && a0 + 8 < in_elems) ? *reinterpret_cast<const u32x4v *>(A + a0 + 8) : u32x4v{0, 0, 0, 0};
        const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const uint32_t wd = sh >> 1, bits = (sh & 1u) * 16u;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t x0 = wd == 0 ? w[d] : wd == 1 ? w[d + 1] : wd == 2 ? w[d + 2] : w[d + 3];
            const uint32_t x1 = wd == 0 ? w[d + 1] : wd == 1 ? w[d + 2] : wd == 2 ? w[d + 3] : w[d + 4];
            v[d] = __builtin_amdgcn_alignbit(x1, x0, bits);   // (x1:x0) >> bits
        }
    }
    halfx8 h = __builtin_bit_cast(halfx8, v);
    if (k + 8 > K) {
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            if (k + i >= K) h[i] = (_Float16)0.0f;
    }
    return h;
}

template <bool VECX>
__global__ void __launch_bounds__(1024) skinny_fwd_mfma_kernel(GemmShape sh, const half_t *__restrict__ A,
                                                               const half_t *__restrict__ B, FwdEpi ep, uint32_t P) {
    __shared__ __attribute__((aligned(16))) half_t ws[SKINNY_N * SKINNY_MFMA_P_MAX];
    __shared__ __attribute__((aligned(16))) float red[16][256];
    const uint32_t K = sh.K, N = sh.N, M = sh.M;
    const uint32_t Kc = (K + 31) / 32 * 32;
    // W^T staging: 8 element loads in flight per thread (W is read as stored,
    // row k of N halves)
    for (uint32_t i0 = threadIdx.x; i0 < SKINNY_N * Kc; i0 += 8 * blockDim.x) {
        half_t v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t i = i0 + u * blockDim.x, k = i / SKINNY_N, n = i % SKINNY_N;
            v[u] = (i < SKINNY_N * Kc && n < N && k < K) ? B[(uint64_t)k * sh.ldb + n] : (half_t)0;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t i = i0 + u * blockDim.x, k = i / SKINNY_N, n = i % SKINNY_N;
            if (i < SKINNY_N * Kc) ws[n * P + k] = v[u];
        }
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, quad = wave >> 2, wq = wave & 3u;
    const uint32_t r16 = lane & 15u, kg = lane >> 4;
    const uint32_t nblk = (M + 15) / 16, nck = Kc / 32;
    const typename EpiFwdK<half_t>::Col1 c1 =
        r16 < N ? EpiFwdK<half_t>::column1(ep, r16) : typename EpiFwdK<half_t>::Col1{};
    const uint64_t in_elems = (uint64_t)(M - 1) * sh.lda + K;   // readable elements of X
    const half_t *wrow = ws + r16 * P + kg * 8;
    for (uint32_t base = blockIdx.x * 4; base < nblk; base += gridDim.x * 4) {
        const uint32_t blk = base + quad;
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (blk < nblk) {   // uniform in the wave: the MFMAs below run with every lane
            const uint32_t m = blk * 16 + r16;
            const bool mrow = m < M;   // rows past M feed zero fragments
            const uint64_t rb = (uint64_t)(mrow ? m : 0u) * sh.lda;
            // 4 of the wave's k-chunks per round: their loads first, then the MFMAs
            for (uint32_t ck0 = wq; ck0 < nck; ck0 += 16) {
                halfx8 xa[4], wb[4];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    const uint32_t ck = ck0 + 4 * u;   // same in every lane
                    if (ck < nck) {
                        const uint32_t k = ck * 32 + kg * 8;
                        xa[u] = (mrow && k < K) ? skinny_x8(A, rb, k, K, in_elems, VECX && k + 8 <= K) : halfx8{};
                        wb[u] = *reinterpret_cast<const halfx8 *>(wrow + ck * 32);
                    } else {
                        xa[u] = halfx8{};
                        wb[u] = halfx8{};
                    }
                }
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], wb[u], acc, 0, 0, 0);
            }
        }
        *reinterpret_cast<floatx4 *>(&red[wave][lane * 4]) = acc;
        __syncthreads();
        if (blk < nblk && wq == 0) {
            const floatx4 p0 = *reinterpret_cast<const floatx4 *>(&red[quad * 4 + 0][lane * 4]);
            const floatx4 p1 = *reinterpret_cast<const floatx4 *>(&red[quad * 4 + 1][lane * 4]);
            const floatx4 p2 = *reinterpret_cast<const floatx4 *>(&red[quad * 4 + 2][lane * 4]);
            const floatx4 p3 = *reinterpret_cast<const floatx4 *>(&red[quad * 4 + 3][lane * 4]);
            const floatx4 sum = ((p0 + p1) + p2) + p3;
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                const uint32_t mo = blk * 16 + 4 * kg + i;
                if (mo < M && r16 < N) EpiFwdK<half_t>::apply1(ep, mo, r16, sum[i], c1, 0);
            }
        }
        __syncthreads();   // red is rewritten by the next round
    }
}

static uint32_t skinny_mfma_pitch(uint32_t K) { return (K + 127) / 128 * 128 + 8; }

bool skinny_fwd_ok(const GemmLaunch &g) {
    const size_t esz = g.dtype == 1 ? 2 : 4;
    const size_t kp = (g.K + 7) / 8 * 8;
    return g.op == Op::Fwd && g.N <= SKINNY_N && g.a_kcontig && !g.b_kcontig && g.K > 0 &&
           (size_t)SKINNY_N * kp * esz <= SKINNY_LDS;
}

template <typename T> static void launch_skinny_fwd_t(const GemmShape &sh, const GemmLaunch &g, hipStream_t s) {
    const bool vecx = sh.lda % 8 == 0 && (reinterpret_cast<uintptr_t>(g.A) & 15u) == 0;
    if constexpr (sizeof(T) == 2) {
        const uint32_t P = skinny_mfma_pitch(sh.K);
        // the MFMA kernel reads 16-byte chunks of X: a 16-byte aligned base
        if (P <= SKINNY_MFMA_P_MAX && (reinterpret_cast<uintptr_t>(g.A) & 15u) == 0 && sh.M > 0) {
            uint32_t grid = (sh.M + 63) / 64;   // 4 blocks of 16 rows per workgroup and round
            if (grid > 256) grid = 256;
            const half_t *A = reinterpret_cast<const half_t *>(g.A), *B = reinterpret_cast<const half_t *>(g.B);
            if (vecx)
                launch_timed(g, skinny_fwd_mfma_kernel<true>, dim3(grid), dim3(1024), s, sh, A, B, g.fwd, P);
            else
                launch_timed(g, skinny_fwd_mfma_kernel<false>, dim3(grid), dim3(1024), s, sh, A, B, g.fwd, P);
            return;
        }
    }
    uint32_t grid = (sh.M + 15) / 16;   // 16 waves per workgroup, a row per wave at a time
    if (grid > 256) grid = 256;
    const T *A = reinterpret_cast<const T *>(g.A), *B = reinterpret_cast<const T *>(g.B);
    if (vecx)
        launch_timed(g, skinny_fwd_kernel<T, true>, dim3(grid), dim3(1024), s, sh, A, B, g.fwd);
    else
        launch_timed(g, skinny_fwd_kernel<T, false>, dim3(grid), dim3(1024), s, sh, A, B, g.fwd);
}

hipError_t launch_skinny_fwd(const GemmLaunch &g, hipStream_t s) {
    if (!skinny_fwd_ok(g)) return hipErrorInvalidValue;
    GemmShape sh{};
    sh.M = g.M;
    sh.N = g.N;
    sh.K = g.K;
    sh.lda = g.lda;
    sh.ldb = g.ldb;
    if (g.dtype == 1)
        launch_skinny_fwd_t<half_t>(sh, g, s);
    else
        launch_skinny_fwd_t<float>(sh, g, s);
    return hipGetLastError();
}

// dW partial sums, thread per W row: thread k of workgroup (x, y) walks the batch rows
// of slice y in order, acc[n] += X[b][k] * dP[b][n], with 64 rows of dP (fp32) at a
// time in LDS (16-byte broadcast reads) and the X loads of 16 rows issued before
// their FMAs; partials[y][k][0..15].
template <typename T> __global__ void __launch_bounds__(256) skinny_dw_kernel(GemmShape sh, const T *__restrict__ X,
                                                                             const float *__restrict__ dp,
                                                                             float *__restrict__ partials,
                                                                             uint32_t per) {
    __shared__ __attribute__((aligned(16))) float dps[64][SKINNY_N];
    const uint32_t K = sh.M, N = sh.N;          // output [K x N]; reduction over sh.K batch rows
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(sh.K, r0 + per);
    float acc[SKINNY_N];
#pragma unroll
    for (int n = 0; n < (int)SKINNY_N; ++n) acc[n] = 0.0f;
    for (uint32_t rb = r0; rb < r1; rb += 64) {
        const uint32_t nrows = min(64u, r1 - rb);
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < 64 * SKINNY_N; i += 256) {
            const uint32_t r = i / SKINNY_N, n = i % SKINNY_N;
            dps[r][n] = (r < nrows && n < N) ? dp[(uint64_t)(rb + r) * sh.ldb + n] : 0.0f;
        }
        __syncthreads();
        if (k < K) {
            for (uint32_t r0b = 0; r0b < nrows; r0b += 16) {
                float xv[16];
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u)
                    xv[u] = r0b + u < nrows ? to_f32(X[(uint64_t)(rb + r0b + u) * sh.lda + k]) : 0.0f;
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u) {
                    if (r0b + u >= nrows) break;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const floatx4 d = *reinterpret_cast<const floatx4 *>(&dps[r0b + u][4 * q]);
                        acc[4 * q + 0] = fmaf(xv[u], d[0], acc[4 * q + 0]);
                        acc[4 * q + 1] = fmaf(xv[u], d[1], acc[4 * q + 1]);
                        acc[4 * q + 2] = fmaf(xv[u], d[2], acc[4 * q + 2]);
                        acc[4 * q + 3] = fmaf(xv[u], d[3], acc[4 * q + 3]);
                    }
                }
            }
        }
    }
    if (k >= K) return;
    float *p = partials + ((uint64_t)blockIdx.y * K + k) * SKINNY_N;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        *reinterpret_cast<floatx4 *>(p + 4 * q) = floatx4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
}

// The same on MFMA (fp16; dP as its fp16 copy, the dW GEMMs' operand): thread t
// of workgroup (x, y) loads column k = 256 x + t of X for 32 batch rows at a time
// (coalesced 2-byte loads, all 32 issued before use) and writes them to LDS
// transposed (xt[t][0..31], one 64-byte run); the 32 x 16 block of dP goes to
// pt[n][0..31].  Wave w then runs v_mfma_f32_16x16x32_f16 on its 4 tiles of 16 W
// rows: src0 lane l = xt[16 q + l % 16][8 (l / 16) ..] (X^T), src1 lane l =
// pt[l % 16][8 (l / 16) ..] (dP); lane l ends with rows 4 (l / 16) .. + 3 of column
// l % 16 of the tile.  LDS rows of 40 halves (80 bytes) keep the 16-byte reads of
// 16 lanes in distinct banks.  partials[y][k][0..15] as in skinny_dw_kernel.
__global__ void __launch_bounds__(256) skinny_dw_mfma_kernel(GemmShape sh, const half_t *__restrict__ X,
                                                             const half_t *__restrict__ dp16,
                                                             float *__restrict__ partials, uint32_t per) {
    __shared__ __attribute__((aligned(16))) half_t xt[256][40];
    __shared__ __attribute__((aligned(16))) half_t pt[SKINNY_N][40];
    const uint32_t K = sh.M, N = sh.N;          // output [K x N]; reduction over sh.K batch rows
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t k0 = blockIdx.x * 256, k = k0 + tid;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(sh.K, r0 + per);
    floatx4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t rb = r0; rb < r1; rb += 32) {
        const uint32_t nrows = min(32u, r1 - rb);
        half_t xv[32];
#pragma unroll
        for (uint32_t u = 0; u < 32; ++u)
            xv[u] = (u < nrows && k < K) ? X[(uint64_t)(rb + u) * sh.lda + k] : (half_t)0;
        half_t pv[2];
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
            const uint32_t i = tid + 256 * h, u = i >> 4, n = i & 15u;   // 32 rows x 16 columns
            pv[h] = (u < nrows && n < N) ? dp16[(uint64_t)(rb + u) * sh.ldb + n] : (half_t)0;
        }
        __syncthreads();   // the previous block's fragments are read
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<halfx8 *>(&xt[tid][8 * q]) = *reinterpret_cast<const halfx8 *>(&xv[8 * q]);
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
            const uint32_t i = tid + 256 * h;
            pt[i & 15u][i >> 4] = pv[h];
        }
        __syncthreads();
        const halfx8 b = *reinterpret_cast<const halfx8 *>(&pt[lane & 15u][8 * (lane >> 4)]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const halfx8 a = *reinterpret_cast<const halfx8 *>(&xt[wave * 64 + 16 * q + (lane & 15u)][8 * (lane >> 4)]);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[q], 0, 0, 0);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) {
            const uint32_t ko = k0 + wave * 64 + 16 * q + 4 * (lane >> 4) + r;
            if (ko < K) partials[((uint64_t)blockIdx.y * K + ko) * SKINNY_N + (lane & 15u)] = acc[q][r];
        }
    }
}

uint32_t skinny_dw_slices(uint32_t rows, uint32_t K) {
    const uint32_t col_blocks = (K + 255) / 256;
    uint32_t sl = (1024 + col_blocks - 1) / col_blocks;
    const uint32_t cap = (rows + 63) / 64;
    if (sl > cap) sl = cap;
    return sl < 1 ? 1 : sl;
}

hipError_t launch_skinny_dw(const GemmLaunch &g, float *partials, uint32_t slices, hipStream_t s) {
    if (g.N > SKINNY_N || g.a_kcontig || !g.b32 || (reinterpret_cast<uintptr_t>(partials) & 15u))
        return hipErrorInvalidValue;
    GemmShape sh{};
    sh.M = g.M;          // W rows (inputs)
    sh.N = g.N;          // W cols (outputs)
    sh.K = g.K;          // batch rows
    sh.lda = g.lda;      // X row pitch
    sh.ldb = g.N;        // d_prenorm row pitch
    const uint32_t per = (g.K + slices - 1) / slices;
    const dim3 grid((g.M + 255) / 256, slices);
    if (g.dtype == 1 && g.B) {
        // fp16: MFMA on the fp16 copy of d_prenorm (row pitch N)
        launch_timed(g, skinny_dw_mfma_kernel, grid, dim3(256), s, sh, reinterpret_cast<const half_t *>(g.A),
                     reinterpret_cast<const half_t *>(g.B), partials, per);
    } else if (g.dtype == 1)
        launch_timed(g, skinny_dw_kernel<half_t>, grid, dim3(256), s, sh, reinterpret_cast<const half_t *>(g.A),
                     g.b32, partials, per);
    else
        launch_timed(g, skinny_dw_kernel<float>, grid, dim3(256), s, sh, reinterpret_cast<const float *>(g.A),
                     g.b32, partials, per);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t s) {
    if (g.M == 0 || g.N == 0) return hipSuccess;
    if (gemm_direct_ok(g)) return launch_gemm_dma(g, s);
    if (g.dtype == 1) {
        if (gemm_large_tile(g.dtype, g.M, g.N) && g.a_kcontig && g.b_kcontig) return dispatch_kk<CfgH256w8>(g, s);
        return dispatch_op<CfgH128>(g, s);
    }
    const uint32_t t128 = ((g.M + 127) / 128) * ((g.N + 127) / 128);
    return t128 >= 192 || g.tile == 128 ? dispatch_op<CfgF128>(g, s) : dispatch_op<CfgF64>(g, s);
}

}  // namespace skl
