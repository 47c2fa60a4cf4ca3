// elementwise.hip — bandwidth-bound kernels of the DenseBlock hot path
// (gfx950, wave64): fill / cast, norm + activation + dropout, softmax, output
// error, hidden error from a given sum, column reductions + vector optimiser,
// split-K dW reduction + optimiser.
#include "launch.h"

#include <type_traits>
#include <utility>

namespace skl {

template <typename T> __device__ __forceinline__ T ldv(const void *p, uint64_t i) {
    return reinterpret_cast<const T *>(p)[i];
}
template <typename T> __device__ __forceinline__ void stv(void *p, uint64_t i, T v) {
    reinterpret_cast<T *>(p)[i] = v;
}

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---- fill / cast (math.cuh:69-73, util.cuh:9-19) -------------------------------------
template <typename T> __global__ void fill_kernel(T *dst, T v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = v;
}

template <typename S, typename D> __global__ void cast_kernel(const S *src, D *dst, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = (D)src[i];
}

static dim3 grid_for(uint64_t n, uint32_t block) {
    uint64_t g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    if (g == 0) g = 1;
    return dim3((uint32_t)g);
}

hipError_t launch_fill(void *dst, uint32_t dtype, float v, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (dtype == 1)
        hipLaunchKernelGGL(fill_kernel<half_t>, grid_for(n, 256), dim3(256), 0, s, (half_t *)dst, (half_t)v,
                           (uint64_t)n);
    else
        hipLaunchKernelGGL(fill_kernel<float>, grid_for(n, 256), dim3(256), 0, s, (float *)dst, v, (uint64_t)n);
    return hipGetLastError();
}

hipError_t launch_cast(const void *src, uint32_t sdt, void *dst, uint32_t ddt, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (sdt == 0 && ddt == 1)
        hipLaunchKernelGGL((cast_kernel<float, half_t>), grid_for(n, 256), dim3(256), 0, s, (const float *)src,
                           (half_t *)dst, (uint64_t)n);
    else if (sdt == 1 && ddt == 0)
        hipLaunchKernelGGL((cast_kernel<half_t, float>), grid_for(n, 256), dim3(256), 0, s, (const half_t *)src,
                           (float *)dst, (uint64_t)n);
    else
        return hipErrorInvalidValue;   // the C ABI admits f32 <-> f16 only
    return hipGetLastError();
}

// ---- block reduction (256 threads = 4 waves), fixed order ---------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const uint32_t w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max256(float v, float *red) {
    v = wave_max(v);
    const uint32_t w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// act + dropout of one element (forward.cu:139-160), input = rounded preact.
template <typename T>
__device__ __forceinline__ void act_dropout(const RowNormArgs &a, uint64_t idx, uint32_t row, uint32_t col, T pre) {
    const float v = activation(a.act, to_f32(pre), a.leaky);
    stv<T>(a.predrop, idx, from_f32<T>(v));
    if (a.use_dropout) {
        if (dropout_u(col, row, a.seed + row * 7u) >= a.p) {
            const float scale = 1.0f / (1.0f - a.p);
            stv<T>(a.mask, idx, from_f32<T>(scale));
            stv<T>(a.out, idx, from_f32<T>(v * scale));
        } else {
            stv<T>(a.mask, idx, (T)0);
            stv<T>(a.out, idx, (T)0);
        }
    } else {
        stv<T>(a.out, idx, from_f32<T>(v));
    }
}

// RMSNorm / LayerNorm over one row per workgroup (forward.cu:44-126), then act + dropout.
template <typename T> __global__ void __launch_bounds__(256) norm_rows_kernel(RowNormArgs a) {
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint32_t n = a.n;
    const uint64_t base = (uint64_t)row * n;
    if (a.norm == 1) {
        float sq = 0.0f;
        for (uint32_t c = threadIdx.x; c < n; c += 256) {
            const float v = to_f32(ldv<T>(a.prenorm, base + c));
            sq = fmaf(v, v, sq);
        }
        sq = block_sum256(sq, red);
        const float var = sq / (float)n + 1e-6f;
        const float rstd32 = 1.0f / sqrtf(var);
        const T rstd = from_f32<T>(rstd32);
        if (threadIdx.x == 0) stv<T>(a.norm_rstd, row, rstd);
        for (uint32_t c = threadIdx.x; c < n; c += 256) {
            const T z = ldv<T>(a.prenorm, base + c);
            stv<T>(a.centered, base + c, z);
            // T arithmetic: (prenorm * rstd) * norm_w, each product rounded to T
            const T pre = from_f32<T>(to_f32(from_f32<T>(to_f32(z) * to_f32(rstd))) * to_f32(ldv<T>(a.norm_w, c)));
            stv<T>(a.preact, base + c, pre);
            act_dropout<T>(a, base + c, row, c, pre);
        }
    } else {
        float s = 0.0f;
        for (uint32_t c = threadIdx.x; c < n; c += 256) s += to_f32(ldv<T>(a.prenorm, base + c));
        s = block_sum256(s, red);
        const float mean = s / (float)n;
        float ss = 0.0f;
        for (uint32_t c = threadIdx.x; c < n; c += 256) {
            const float v = to_f32(ldv<T>(a.prenorm, base + c)) - mean;
            ss = fmaf(v, v, ss);
        }
        ss = block_sum256(ss, red);
        const float var = ss / (float)n + 1e-6f;
        const float rstd32 = 1.0f / sqrtf(var);
        if (threadIdx.x == 0) stv<T>(a.norm_rstd, row, from_f32<T>(rstd32));
        for (uint32_t c = threadIdx.x; c < n; c += 256) {
            const float v = to_f32(ldv<T>(a.prenorm, base + c)) - mean;
            stv<T>(a.centered, base + c, from_f32<T>(v));
            const T pre = from_f32<T>(
                fmaf(v * rstd32, to_f32(ldv<T>(a.norm_w, c)), to_f32(ldv<T>(a.norm_b, c))));
            stv<T>(a.preact, base + c, pre);
            act_dropout<T>(a, base + c, row, c, pre);
        }
    }
}

// The same with the row held in registers: each element of prenorm is read
// once, and every cache write is a 16-byte store when rows are 16-byte aligned
// (VEC: a thread owns chunks of VW consecutive elements, chunk t + 256 i) or
// a coalesced element store otherwise (a thread owns elements t + 256 i).
// PER = chunks (VEC) or elements per thread; rows up to 256 x PER (x VW).
template <typename T, bool VEC, int PER> __global__ void __launch_bounds__(256) norm_rows_reg_kernel(RowNormArgs a) {
    constexpr int VW = VEC ? 16 / (int)sizeof(T) : 1;
    constexpr int E = PER * VW;   // elements per thread
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint32_t n = a.n;
    const uint64_t base = (uint64_t)row * n;
    const T *pz = reinterpret_cast<const T *>(a.prenorm) + base;
    float z[E];
    bool in[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c0 = (threadIdx.x + 256u * i) * VW;
        in[i] = c0 < n;
        if constexpr (VEC) {
            T v[VW];
            if (in[i]) {
                *reinterpret_cast<u32x4_t *>(v) = *reinterpret_cast<const u32x4_t *>(pz + c0);
            } else {
#pragma unroll
                for (int e = 0; e < VW; ++e) v[e] = (T)0;
            }
#pragma unroll
            for (int e = 0; e < VW; ++e) z[i * VW + e] = to_f32(v[e]);
        } else {
            z[i] = in[i] ? to_f32(pz[c0]) : 0.0f;
        }
    }
    float mean = 0.0f, rstd32;
    T rstd_t;
    if (a.norm == 1) {
        float sq = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) sq = fmaf(z[e], z[e], sq);
        sq = block_sum256(sq, red);
        rstd32 = 1.0f / sqrtf(sq / (float)n + 1e-6f);
        rstd_t = from_f32<T>(rstd32);
    } else {
        float sm = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) sm += z[e];
        mean = block_sum256(sm, red) / (float)n;
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            // padding elements (z = 0) are not part of the row
            const uint32_t c = VEC ? (threadIdx.x + 256u * (e / VW)) * VW + e % VW : threadIdx.x + 256u * e;
            const float v = c < n ? z[e] - mean : 0.0f;
            ss = fmaf(v, v, ss);
        }
        ss = block_sum256(ss, red);
        rstd32 = 1.0f / sqrtf(ss / (float)n + 1e-6f);
        rstd_t = from_f32<T>(rstd32);
    }
    if (threadIdx.x == 0) stv<T>(a.norm_rstd, row, rstd_t);
    const float scale = a.use_dropout ? 1.0f / (1.0f - a.p) : 1.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        if (!in[i]) continue;
        const uint32_t c0 = (threadIdx.x + 256u * i) * VW;
        T cen[VW], pre[VW], pd[VW], mk[VW], ot[VW], g[VW], bb[VW];
        if constexpr (VEC) {
            *reinterpret_cast<u32x4_t *>(g) = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const T *>(a.norm_w) + c0);
            if (a.norm == 2)
                *reinterpret_cast<u32x4_t *>(bb) =
                    *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const T *>(a.norm_b) + c0);
        } else {
            g[0] = ldv<T>(a.norm_w, c0);
            if (a.norm == 2) bb[0] = ldv<T>(a.norm_b, c0);
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            const float zv = z[i * VW + e];
            T p;
            if (a.norm == 1) {
                // T arithmetic: (prenorm * rstd) * norm_w, each product rounded to T (forward.cu:61-72)
                cen[e] = from_f32<T>(zv);
                p = from_f32<T>(to_f32(from_f32<T>(zv * to_f32(rstd_t))) * to_f32(g[e]));
            } else {
                const float v = zv - mean;
                cen[e] = from_f32<T>(v);
                p = from_f32<T>(fmaf(v * rstd32, to_f32(g[e]), to_f32(bb[e])));
            }
            pre[e] = p;
            const float act = activation(a.act, to_f32(p), a.leaky);
            pd[e] = from_f32<T>(act);
            if (a.use_dropout) {
                const bool keep = dropout_u(c0 + e, row, a.seed + row * 7u) >= a.p;
                mk[e] = keep ? from_f32<T>(scale) : (T)0;
                ot[e] = keep ? from_f32<T>(act * scale) : (T)0;
            } else {
                ot[e] = pd[e];
            }
        }
        const uint64_t idx = base + c0;
        if constexpr (VEC) {
            *reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(a.centered) + idx) = *reinterpret_cast<u32x4_t *>(cen);
            *reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(a.preact) + idx) = *reinterpret_cast<u32x4_t *>(pre);
            *reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(a.predrop) + idx) = *reinterpret_cast<u32x4_t *>(pd);
            *reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(a.out) + idx) = *reinterpret_cast<u32x4_t *>(ot);
            if (a.use_dropout)
                *reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(a.mask) + idx) = *reinterpret_cast<u32x4_t *>(mk);
        } else {
            stv<T>(a.centered, idx, cen[0]);
            stv<T>(a.preact, idx, pre[0]);
            stv<T>(a.predrop, idx, pd[0]);
            stv<T>(a.out, idx, ot[0]);
            if (a.use_dropout) stv<T>(a.mask, idx, mk[0]);
        }
    }
}

// Rows that do not start on a 4-element boundary of their buffers (widths not a
// multiple of 4): thread t owns the 4-element groups t, t + 256, ... of the buffer
// that overlap the row, aligned in the buffer, so each tensor moves one 8-byte
// (fp16) / 16-byte (fp32) access per group instead of four element accesses.  A
// group that straddles the row's first or last element contributes only the row's
// own elements to the statistics and is stored element by element, only those
// elements (the neighbouring row's are another workgroup's).  A group holding a
// valid element lies inside the buffer's aligned chunk of that element, so its
// loads stay inside the allocation.  Needs every row tensor 4-element aligned.
// PER = groups per thread: rows up to 1024 PER - 3 elements.  Per element the
// arithmetic is that of norm_rows_reg_kernel.
template <typename T, int PER> __global__ void __launch_bounds__(256) norm_rows_grp_kernel(RowNormArgs a) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    typedef typename std::conditional<sizeof(T) == 2, u32x2_t, u32x4_t>::type G;   // 4 elements
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint32_t n = a.n;
    const uint64_t base = (uint64_t)row * n;
    const uint32_t off = (uint32_t)(base & 3u);        // row start within its group
    const uint64_t g0 = base >> 2;                     // group holding the row's first element
    const uint32_t ng = (off + n + 3u) >> 2;           // groups overlapping the row
    float z[PER][4];
    bool has[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t j = threadIdx.x + 256u * i;
        has[i] = j < ng;
        T v[4] = {(T)0, (T)0, (T)0, (T)0};
        if (has[i]) *reinterpret_cast<G *>(v) = reinterpret_cast<const G *>(a.prenorm)[g0 + j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = (int)(4u * j) + e - (int)off;    // column of element e
            z[i][e] = (has[i] && c >= 0 && c < (int)n) ? to_f32(v[e]) : 0.0f;
        }
    }
    float mean = 0.0f, rstd32;
    T rstd_t;
    if (a.norm == 1) {
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) sq = fmaf(z[i][e], z[i][e], sq);
        sq = block_sum256(sq, red);
        rstd32 = 1.0f / sqrtf(sq / (float)n + 1e-6f);
        rstd_t = from_f32<T>(rstd32);
    } else {
        float sm = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) sm += z[i][e];
        mean = block_sum256(sm, red) / (float)n;
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = (int)(4u * (threadIdx.x + 256u * i)) + e - (int)off;
                const float v = (has[i] && c >= 0 && c < (int)n) ? z[i][e] - mean : 0.0f;
                ss = fmaf(v, v, ss);
            }
        ss = block_sum256(ss, red);
        rstd32 = 1.0f / sqrtf(ss / (float)n + 1e-6f);
        rstd_t = from_f32<T>(rstd32);
    }
    if (threadIdx.x == 0) stv<T>(a.norm_rstd, row, rstd_t);
    const float scale = a.use_dropout ? 1.0f / (1.0f - a.p) : 1.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        if (!has[i]) continue;
        const uint32_t j = threadIdx.x + 256u * i;
        const int c0 = (int)(4u * j) - (int)off;         // column of element 0 (may be < 0)
        const bool whole = c0 >= 0 && c0 + 3 < (int)n;
        T cen[4], pre[4], pd[4], mk[4], ot[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + e;
            const bool ok = c >= 0 && c < (int)n;
            const uint32_t cc = ok ? (uint32_t)c : 0u;
            const float gw = ok ? to_f32(ldv<T>(a.norm_w, cc)) : 0.0f;
            const float zv = z[i][e];
            T p;
            if (a.norm == 1) {
                cen[e] = from_f32<T>(zv);
                p = from_f32<T>(to_f32(from_f32<T>(zv * to_f32(rstd_t))) * gw);
            } else {
                const float gb = ok ? to_f32(ldv<T>(a.norm_b, cc)) : 0.0f;
                const float v = zv - mean;
                cen[e] = from_f32<T>(v);
                p = from_f32<T>(fmaf(v * rstd32, gw, gb));
            }
            pre[e] = p;
            const float act = activation(a.act, to_f32(p), a.leaky);
            pd[e] = from_f32<T>(act);
            if (a.use_dropout) {
                const bool keep = dropout_u(cc, row, a.seed + row * 7u) >= a.p;
                mk[e] = keep ? from_f32<T>(scale) : (T)0;
                ot[e] = keep ? from_f32<T>(act * scale) : (T)0;
            } else {
                ot[e] = pd[e];
            }
        }
        const uint64_t gi = g0 + j;
        if (whole) {
            reinterpret_cast<G *>(a.centered)[gi] = *reinterpret_cast<G *>(cen);
            reinterpret_cast<G *>(a.preact)[gi] = *reinterpret_cast<G *>(pre);
            reinterpret_cast<G *>(a.predrop)[gi] = *reinterpret_cast<G *>(pd);
            reinterpret_cast<G *>(a.out)[gi] = *reinterpret_cast<G *>(ot);
            if (a.use_dropout) reinterpret_cast<G *>(a.mask)[gi] = *reinterpret_cast<G *>(mk);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = c0 + e;
                if (c < 0 || c >= (int)n) continue;
                const uint64_t idx = base + (uint32_t)c;
                stv<T>(a.centered, idx, cen[e]);
                stv<T>(a.preact, idx, pre[e]);
                stv<T>(a.predrop, idx, pd[e]);
                stv<T>(a.out, idx, ot[e]);
                if (a.use_dropout) stv<T>(a.mask, idx, mk[e]);
            }
        }
    }
}

// BatchNorm: one thread per column over the batch rows (forward.cu:74-126 with
// norm == 3), then act + dropout.  Consecutive threads read consecutive columns.
template <typename T> __global__ void __launch_bounds__(256) norm_cols_kernel(RowNormArgs a) {
    const uint32_t col = blockIdx.x * 256 + threadIdx.x;
    if (col >= a.n) return;
    const uint32_t n = a.n, m = a.m;
    float s = 0.0f;
    for (uint32_t r = 0; r < m; ++r) s += to_f32(ldv<T>(a.prenorm, (uint64_t)r * n + col));
    const float mean = s / (float)m;
    float ss = 0.0f;
    for (uint32_t r = 0; r < m; ++r) {
        const float v = to_f32(ldv<T>(a.prenorm, (uint64_t)r * n + col)) - mean;
        ss = fmaf(v, v, ss);
    }
    const float var = ss / (float)m + 1e-6f;
    const float rstd32 = 1.0f / sqrtf(var);
    stv<T>(a.norm_rstd, col, from_f32<T>(rstd32));
    const float g = to_f32(ldv<T>(a.norm_w, col)), b = to_f32(ldv<T>(a.norm_b, col));
    for (uint32_t r = 0; r < m; ++r) {
        const uint64_t idx = (uint64_t)r * n + col;
        const float v = to_f32(ldv<T>(a.prenorm, idx)) - mean;
        stv<T>(a.centered, idx, from_f32<T>(v));
        const T pre = from_f32<T>(fmaf(v * rstd32, g, b));
        stv<T>(a.preact, idx, pre);
        act_dropout<T>(a, idx, r, col, pre);
    }
}

static bool a16p(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows up to 256 x 16 elements run with the row in registers (16-byte chunks when
// rows are 16-byte aligned, aligned 4-element groups when only the buffers are);
// longer rows take the looping kernel.
template <typename T> static void launch_norm_rows(const RowNormArgs &a, hipStream_t s) {
    constexpr uint32_t VW = 16 / sizeof(T);
    const bool vec = a.n % VW == 0 && a16p(a.prenorm) && a16p(a.norm_w) && (a.norm != 2 || a16p(a.norm_b)) &&
                     a16p(a.centered) && a16p(a.preact) && a16p(a.predrop) && a16p(a.out) &&
                     (!a.use_dropout || a16p(a.mask));
    // 4-element groups aligned in every row tensor (rows that are not)
    constexpr uintptr_t GB = 4 * sizeof(T) - 1;
    auto ga = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & GB) == 0; };
    const bool grp = ga(a.prenorm) && ga(a.centered) && ga(a.preact) && ga(a.predrop) && ga(a.out) &&
                     (!a.use_dropout || ga(a.mask));
    const dim3 g(a.m), b(256);
    if (!vec && grp && a.n <= 4 * 1024 - 3) {
        if (a.n <= 1024 - 3)
            hipLaunchKernelGGL((norm_rows_grp_kernel<T, 1>), g, b, 0, s, a);
        else if (a.n <= 2 * 1024 - 3)
            hipLaunchKernelGGL((norm_rows_grp_kernel<T, 2>), g, b, 0, s, a);
        else if (a.n <= 3 * 1024 - 3)
            hipLaunchKernelGGL((norm_rows_grp_kernel<T, 3>), g, b, 0, s, a);
        else
            hipLaunchKernelGGL((norm_rows_grp_kernel<T, 4>), g, b, 0, s, a);
        return;
    }
    if (vec && a.n <= 256 * VW)
        hipLaunchKernelGGL((norm_rows_reg_kernel<T, true, 1>), g, b, 0, s, a);
    else if (vec && a.n <= 2 * 256 * VW)
        hipLaunchKernelGGL((norm_rows_reg_kernel<T, true, 2>), g, b, 0, s, a);
    else if (a.n <= 256 * 4)
        hipLaunchKernelGGL((norm_rows_reg_kernel<T, false, 4>), g, b, 0, s, a);
    else if (a.n <= 256 * 8)
        hipLaunchKernelGGL((norm_rows_reg_kernel<T, false, 8>), g, b, 0, s, a);
    else if (a.n <= 256 * 16)
        hipLaunchKernelGGL((norm_rows_reg_kernel<T, false, 16>), g, b, 0, s, a);
    else
        hipLaunchKernelGGL(norm_rows_kernel<T>, g, b, 0, s, a);
}

hipError_t launch_norm_act(const RowNormArgs &a, hipStream_t s) {
    if (a.m == 0 || a.n == 0) return hipSuccess;
    if (a.norm == 3) {
        if (a.dtype == 1)
            hipLaunchKernelGGL(norm_cols_kernel<half_t>, dim3(cdiv(a.n, 256)), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(norm_cols_kernel<float>, dim3(cdiv(a.n, 256)), dim3(256), 0, s, a);
    } else if (a.dtype == 1) {
        launch_norm_rows<half_t>(a, s);
    } else {
        launch_norm_rows<float>(a, s);
    }
    return hipGetLastError();
}

// ---- softmax (util.cu:95-173), one row per workgroup, in place ----------------------
template <typename T> __global__ void __launch_bounds__(256) softmax_kernel(T *out, uint32_t n) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (uint32_t c = threadIdx.x; c < n; c += 256) mx = fmaxf(mx, to_f32(out[base + c]));
    mx = block_max256(mx, red);
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < n; c += 256) s += expf(to_f32(out[base + c]) - mx);
    s = block_sum256(s, red);
    for (uint32_t c = threadIdx.x; c < n; c += 256) out[base + c] = from_f32<T>(expf(to_f32(out[base + c]) - mx) / s);
}

hipError_t launch_softmax(uint32_t dtype, void *out, uint32_t rows, uint32_t n, hipStream_t s) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (dtype == 1)
        hipLaunchKernelGGL(softmax_kernel<half_t>, dim3(rows), dim3(256), 0, s, (half_t *)out, n);
    else
        hipLaunchKernelGGL(softmax_kernel<float>, dim3(rows), dim3(256), 0, s, (float *)out, n);
    return hipGetLastError();
}

// ---- error kernels ------------------------------------------------------------------
// A thread owns 4 consecutive elements of one row (cnt <= 4 of them exist).
// VEC (n % 4 == 0, 16-byte aligned buffers): GrpV, 16-byte fp32 / 8-byte fp16
// accesses; otherwise GrpUA below.
template <typename T> struct GrpV {
    __device__ __forceinline__ static f32x4 ld(const void *p, uint64_t i, uint32_t) { return load4<T>(p, i); }
    __device__ __forceinline__ static f32x4 ldf(const float *p, uint64_t i, uint32_t, bool nt = false) {
        return nt ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p + i))
                  : *reinterpret_cast<const f32x4 *>(p + i);
    }
    __device__ __forceinline__ static void stf(float *p, uint64_t i, f32x4 v, uint32_t, bool nt = false) {
        if (nt)
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p + i));
        else
            *reinterpret_cast<f32x4 *>(p + i) = v;
    }
    __device__ __forceinline__ static void sth(half_t *p, uint64_t i, f32x4 v, uint32_t) {
        store4<half_t>(p, i, v);
    }
};

// Rows at any alignment (n % 4 != 0, or buffers not 16-byte aligned): the group
// of elements i .. i + cnt - 1 of an array p is read as the aligned 4-element
// chunk holding element i plus, when the group runs into the next chunk, that
// chunk too.  Each chunk read holds an element of the group, so no read leaves
// the 16-byte blocks the group's own elements lie in.  Stores split the group at
// the chunk boundary into aligned 1-, 2- and 4-element pieces.  For a row-
// strided group (first column a multiple of 4) the offset o of element i in its
// chunk is the same in every lane of the row, so the switches on o branch
// uniformly; only the lane that holds a row's last, partial group (cnt < 4)
// takes the element-by-element path.
template <typename T> struct GrpUA {
    __device__ __forceinline__ static uint32_t lead(const void *p) {
        return (uint32_t)((reinterpret_cast<uintptr_t>(p) / sizeof(T)) & 3u);
    }
    // Elements o .. o + 3 of the 8-element concatenation (a, b), o in 1..3.
    // Written as selects: a switch returning the four vectors gave wrong
    // elements for o = 3 inside the error kernel's unrolled row loop (hipcc,
    // ROCm 7.2), while the same switch in a stand-alone loop did not.
    __device__ __forceinline__ static f32x4 pick(f32x4 a, f32x4 b, uint32_t o) {
        const bool o1 = o == 1, o2 = o == 2;
        return f32x4{o1 ? a[1] : o2 ? a[2] : a[3], o1 ? a[2] : o2 ? a[3] : b[0], o1 ? a[3] : o2 ? b[0] : b[1],
                     o1 ? b[0] : o2 ? b[1] : b[2]};
    }
    template <typename E> __device__ __forceinline__ static f32x4 load(const void *p, uint64_t i, uint32_t cnt) {
        const uint32_t b = GrpUA<E>::lead(p);
        const E *q = reinterpret_cast<const E *>(p) - b;   // 4-element aligned
        const uint64_t k = i + b, ch = k & ~3ull;
        const uint32_t o = (uint32_t)(k & 3u);
        const f32x4 lo = load4<E>(q, ch);
        if (o == 0) return lo;
        const f32x4 hi = cnt > 4u - o ? load4<E>(q, ch + 4) : f32x4{0, 0, 0, 0};
        return pick(lo, hi, o);
    }
    __device__ __forceinline__ static f32x4 ld(const void *p, uint64_t i, uint32_t cnt) { return load<T>(p, i, cnt); }
    __device__ __forceinline__ static f32x4 ldf(const float *p, uint64_t i, uint32_t cnt, bool = false) {
        return load<float>(p, i, cnt);
    }
    __device__ __forceinline__ static void stf(float *p, uint64_t i, f32x4 v, uint32_t cnt, bool = false) {
        if (cnt < 4) {
            for (uint32_t j = 0; j < cnt; ++j) p[i + j] = v[j];
            return;
        }
        const uint32_t b = GrpUA<float>::lead(p);
        float *q = p - b;
        const uint64_t k = i + b, ch = k & ~3ull;
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        switch ((uint32_t)(k & 3u)) {
        case 0: *reinterpret_cast<f32x4 *>(q + ch) = v; break;
        case 1:
            q[ch + 1] = v[0];
            *reinterpret_cast<f32x2 *>(q + ch + 2) = f32x2{v[1], v[2]};
            q[ch + 4] = v[3];
            break;
        case 2:
            *reinterpret_cast<f32x2 *>(q + ch + 2) = f32x2{v[0], v[1]};
            *reinterpret_cast<f32x2 *>(q + ch + 4) = f32x2{v[2], v[3]};
            break;
        default:
            q[ch + 3] = v[0];
            *reinterpret_cast<f32x2 *>(q + ch + 4) = f32x2{v[1], v[2]};
            q[ch + 6] = v[3];
            break;
        }
    }
    __device__ __forceinline__ static void sth(half_t *p, uint64_t i, f32x4 v, uint32_t cnt) {
        if (cnt < 4) {
            for (uint32_t j = 0; j < cnt; ++j) p[i + j] = (half_t)v[j];
            return;
        }
        const uint32_t b = GrpUA<half_t>::lead(p);
        half_t *q = p - b;
        const uint64_t k = i + b, ch = k & ~3ull;
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        const half_t h0 = (half_t)v[0], h1 = (half_t)v[1], h2 = (half_t)v[2], h3 = (half_t)v[3];
        switch ((uint32_t)(k & 3u)) {
        case 0: *reinterpret_cast<f16x4 *>(q + ch) = f16x4{h0, h1, h2, h3}; break;
        case 1:
            q[ch + 1] = h0;
            *reinterpret_cast<f16x2 *>(q + ch + 2) = f16x2{h1, h2};
            q[ch + 4] = h3;
            break;
        case 2:
            *reinterpret_cast<f16x2 *>(q + ch + 2) = f16x2{h0, h1};
            *reinterpret_cast<f16x2 *>(q + ch + 4) = f16x2{h2, h3};
            break;
        default:
            q[ch + 3] = h0;
            *reinterpret_cast<f16x2 *>(q + ch + 4) = f16x2{h1, h2};
            q[ch + 6] = h3;
            break;
        }
    }
};
// GrpUA with the offset O of element i in its chunk known at compile time and
// 4-element-aligned base pointers: no branches on the offset, and the picks
// are register moves.
template <typename T, int O> struct GrpUS {
    template <typename E> __device__ __forceinline__ static f32x4 load(const void *p, uint64_t i, uint32_t cnt) {
        const f32x4 lo = load4<E>(p, i - O);
        if constexpr (O == 0) {
            return lo;
        } else {
            const f32x4 hi = cnt > 4u - O ? load4<E>(p, i - O + 4) : f32x4{0, 0, 0, 0};
            if constexpr (O == 1) return f32x4{lo[1], lo[2], lo[3], hi[0]};
            if constexpr (O == 2) return f32x4{lo[2], lo[3], hi[0], hi[1]};
            return f32x4{lo[3], hi[0], hi[1], hi[2]};
        }
    }
    __device__ __forceinline__ static f32x4 ld(const void *p, uint64_t i, uint32_t cnt) { return load<T>(p, i, cnt); }
    __device__ __forceinline__ static f32x4 ldf(const float *p, uint64_t i, uint32_t cnt, bool = false) {
        return load<float>(p, i, cnt);
    }
    template <typename E, typename V2> __device__ __forceinline__ static void put(E *q, f32x4 v) {
        // q = the group's first element; pieces at the chunk boundary
        if constexpr (O == 0) {
            if constexpr (sizeof(E) == 4)
                *reinterpret_cast<f32x4 *>(q) = v;
            else
                *reinterpret_cast<f16x4 *>(q) = f16x4{(E)v[0], (E)v[1], (E)v[2], (E)v[3]};
        } else if constexpr (O == 2) {
            *reinterpret_cast<V2 *>(q) = V2{(E)v[0], (E)v[1]};
            *reinterpret_cast<V2 *>(q + 2) = V2{(E)v[2], (E)v[3]};
        } else {
            q[0] = (E)v[0];
            *reinterpret_cast<V2 *>(q + 1) = V2{(E)v[1], (E)v[2]};
            q[3] = (E)v[3];
        }
    }
    __device__ __forceinline__ static void stf(float *p, uint64_t i, f32x4 v, uint32_t cnt, bool = false) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        if (cnt < 4) {
            for (uint32_t j = 0; j < cnt; ++j) p[i + j] = v[j];
            return;
        }
        put<float, f32x2>(p + i, v);
    }
    __device__ __forceinline__ static void sth(half_t *p, uint64_t i, f32x4 v, uint32_t cnt) {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        if (cnt < 4) {
            for (uint32_t j = 0; j < cnt; ++j) p[i + j] = (half_t)v[j];
            return;
        }
        put<half_t, f16x2>(p + i, v);
    }
};

// Accessor modes of the error kernels: 1 = GrpV (n % 4 == 0, aligned buffers);
// 4 + n % 4 = GrpUS (aligned buffers, n % 4 != 0, row splits a multiple of 4
// rows, so row rb + u with rb % 4 == 0 starts at offset (u n) % 4 of its
// chunk); 0 = GrpUA (anything else).  RowAcc: the row-strided [rows x n]
// arrays of row slot u; ColAcc: per-column vectors and the supplied sum s.
template <typename T, int MODE, int U> struct RowAcc {
    typedef typename std::conditional<
        MODE == 1, GrpV<T>,
        typename std::conditional<MODE == 0, GrpUA<T>, GrpUS<T, (U * (MODE - 4)) & 3>>::type>::type type;
};
template <typename T, int MODE> struct ColAcc {
    typedef typename std::conditional<MODE == 0, GrpUA<T>, GrpV<T>>::type type;
};

// The three values of one 4-column group that feed the column sums of backward.cu:187-194.
struct ErrSums4 {
    f32x4 dp, dnw, dnb;
};

// grad = e; the element-local norm gradient (util.cu:175-215) into d_prenorm and
// dNorm; d_prenorm scaled by the loss scale; its fp16 copy for the GEMMs.
template <typename T, class G, class GC>
__device__ __forceinline__ ErrSums4 write_err4(const ErrArgs &a, uint64_t idx, uint32_t row, uint32_t col,
                                               uint32_t cnt, f32x4 e) {
    G::stf(a.grad, idx, e, cnt, true);
    ErrSums4 o;
    o.dp = e;
    o.dnw = o.dnb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (a.norm) {
        const f32x4 pv = a.norm == 1 ? G::ld(a.prenorm, idx, cnt) : f32x4{0, 0, 0, 0};
        const f32x4 cv = a.norm >= 2 ? G::ld(a.centered, idx, cnt) : f32x4{0, 0, 0, 0};
        const f32x4 nw = GC::ldf(a.nw, col, cnt);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float rstd = to_f32(ldv<T>(a.norm_rstd, a.norm == 3 ? col + (j < (int)cnt ? j : 0) : row));
            const NormGrad g = norm_grad(a.norm, e[j], pv[j], cv[j], rstd, nw[j], a.inv_n, a.inv_m);
            o.dp[j] = g.d_prenorm;
            o.dnw[j] = g.dnw;
            o.dnb[j] = g.dnb;
        }
        G::stf(a.d_norm_w, idx, o.dnw, cnt);
        G::stf(a.d_norm_b, idx, o.dnb, cnt);
    }
    o.dp = o.dp * a.loss_scale;
    G::stf(a.d_prenorm, idx, o.dp, cnt, true);
    if (a.d_prenorm_h) G::sth(a.d_prenorm_h, idx, o.dp, cnt);
    if (cnt < 4) {
        // columns past n add nothing to the sums
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
            if (j >= cnt) o.dp[j] = o.dnw[j] = o.dnb[j] = 0.0f;
    }
    return o;
}

// Loss delta of one 4-column group (backward.cu:24-45).
template <typename T, class G>
__device__ __forceinline__ f32x4 output_err4(const ErrArgs &a, uint64_t idx, uint32_t cnt) {
    const f32x4 out = G::ld(a.out, idx, cnt), tg = G::ld(a.target, idx, cnt), pre = G::ld(a.preact, idx, cnt);
    f32x4 e;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float o = activation(a.act, out[j], a.leaky);
        float ej = 0.0f;
        if (a.loss == 0) {
            ej = activation_derivative(a.act, o - tg[j], o, pre[j], a.leaky);
        } else if ((a.loss == 1 && a.act == 5) || (a.loss == 2 && a.act == 1)) {
            ej = o - tg[j];
        }
        e[j] = ej;
    }
    return e;
}

// Error + column sums in one pass (backward.cu:12-56 for the output layer,
// 79-100 for a supplied sum s).  Workgroup (x, y) owns the columns
// [1024 x, 1024 (x + 1)) of the rows [y per, (y + 1) per): a thread owns one
// 4-column group, loads ERR_UR rows of its operands before computing any
// (ERR_UR x 40 bytes in flight), writes grad / d_prenorm (/ dNorm) and adds
// d_prenorm, dNorm_w and dNorm_b into running column sums, rows in ascending
// order.  The sums go to partials[y][k][n] (k = 0 d_prenorm, 1 dNorm_w,
// 2 dNorm_b; 1 and 2 only with a norm), the inputs of the bias / norm-
// parameter update, so the backward does not read the three [rows x n]
// buffers again.  4 rows per thread and ~1024 workgroups: of the shapes
// measured on the C3 step (rows x column groups per thread in {4x1, 2x2, 1x4,
// 2x4}, 512 to 2048 workgroups) the fastest, both alone and between the GEMMs.
constexpr int ERR_UR = 4;
struct ErrAcc {   // running column sums of one 4-column group
    f32x4 dp, nw, nb;
};
template <typename T, bool FROM_SUM, int MODE, int U>
__device__ __forceinline__ void err_load(const ErrArgs &a, uint32_t rb, uint32_t r1, uint32_t c, uint32_t cnt,
                                         uint32_t s_ld, f32x4 (&x)[4][ERR_UR]) {
    typedef typename RowAcc<T, MODE, U>::type G;
    typedef typename ColAcc<float, MODE>::type GS;
    if (rb + U >= r1) return;
    const uint64_t idx = (uint64_t)(rb + U) * a.n + c;
    x[0][U] = GS::ldf(a.s, (uint64_t)(rb + U) * s_ld + c, cnt, true);
    x[1][U] = G::ld(a.predrop, idx, cnt);
    x[2][U] = G::ld(a.preact, idx, cnt);
    x[3][U] = G::ld(a.mask, idx, cnt);
}
template <typename T, bool FROM_SUM, int MODE, int U>
__device__ __forceinline__ void err_row(const ErrArgs &a, uint32_t rb, uint32_t r1, uint32_t c, uint32_t cnt,
                                        const f32x4 (&x)[4][ERR_UR], ErrAcc &acc) {
    typedef typename RowAcc<T, MODE, U>::type G;
    typedef typename ColAcc<float, MODE>::type GC;
    const uint32_t row = rb + U;
    if (row >= r1) return;
    const uint64_t idx = (uint64_t)row * a.n + c;
    f32x4 e;
    if constexpr (FROM_SUM) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            e[j] = x[3][U][j] * activation_derivative(a.act, x[0][U][j], x[1][U][j], x[2][U][j], a.leaky);
    } else {
        e = output_err4<T, G>(a, idx, cnt);
    }
    const ErrSums4 o = write_err4<T, G, GC>(a, idx, row, c, cnt, e);
    acc.dp += o.dp;
    acc.nw += o.dnw;
    acc.nb += o.dnb;
}
template <typename T, bool FROM_SUM, int MODE, int... U>
__device__ __forceinline__ void err_rows(const ErrArgs &a, uint32_t rb, uint32_t r1, uint32_t c, uint32_t cnt,
                                         uint32_t s_ld, ErrAcc &acc, std::integer_sequence<int, U...>) {
    f32x4 x[4][ERR_UR];
    if constexpr (FROM_SUM) (err_load<T, FROM_SUM, MODE, U>(a, rb, r1, c, cnt, s_ld, x), ...);
    (err_row<T, FROM_SUM, MODE, U>(a, rb, r1, c, cnt, x, acc), ...);
}
template <typename T, bool FROM_SUM, int MODE>
__global__ void __launch_bounds__(256) error_cols_kernel(ErrArgs a, float *__restrict__ partials, uint32_t per) {
    const uint32_t c = blockIdx.x * 1024 + threadIdx.x * 4;
    if (c >= a.n) return;
    const uint32_t cnt = min(4u, a.n - c);
    const uint32_t s_ld = a.s_ld ? a.s_ld : a.n;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(a.rows, r0 + per);
    ErrAcc acc{{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    for (uint32_t rb = r0; rb < r1; rb += ERR_UR)
        err_rows<T, FROM_SUM, MODE>(a, rb, r1, c, cnt, s_ld, acc, std::make_integer_sequence<int, ERR_UR>{});
    typedef typename std::conditional<MODE == 1, GrpV<float>, GrpUA<float>>::type GP;
    float *p = partials + (uint64_t)blockIdx.y * 3 * a.n + c;
    GP::stf(p, 0, acc.dp, cnt);
    if (a.norm) {
        GP::stf(p + a.n, 0, acc.nw, cnt);
        GP::stf(p + 2 * a.n, 0, acc.nb, cnt);
    }
}

static bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Every buffer the kernel touches 16-byte aligned, and s's rows a multiple of 4
// elements apart (partials only matter for GrpV: GrpUS writes them via GrpUA).
static bool err_aligned(const ErrArgs &a, bool from_sum, const float *partials) {
    if (from_sum && (a.s_ld & 3u) != 0) return false;
    const void *ptrs[] = {a.grad, a.d_prenorm, a.d_prenorm_h, a.preact, a.norm ? a.nw : nullptr,
                          a.norm ? a.d_norm_w : nullptr, a.norm ? a.d_norm_b : nullptr,
                          a.norm == 1 ? a.prenorm : nullptr, a.norm >= 2 ? a.centered : nullptr,
                          from_sum ? a.s : a.out, from_sum ? a.predrop : a.target, from_sum ? a.mask : nullptr,
                          (a.n & 3u) == 0 ? partials : nullptr};
    for (const void *p : ptrs)
        if (p && !a16(p)) return false;
    return true;
}

// Row splits of the error kernels: ~1024 workgroups of >= 16 rows for n >= 1024;
// narrower outputs leave most of a workgroup's 256 column-group lanes idle, so
// they get ~256K active lanes in all, in slices of >= 4 rows (at most 4096).
uint32_t err_col_splits(uint32_t rows, uint32_t n) {
    uint32_t sp, cap;
    if (n >= 1024) {
        sp = cdiv(1024, cdiv(n, 1024));
        cap = cdiv(rows, 16);
    } else {
        sp = cdiv(262144u, cdiv(n, 4));
        cap = cdiv(rows, 4);
    }
    if (sp > cap) sp = cap;
    if (sp > 4096) sp = 4096;
    return sp < 1 ? 1 : sp;
}

template <bool FROM_SUM, typename T, int MODE>
static void launch_error_mode(const ErrArgs &a, float *partials, uint32_t splits, uint32_t per, hipStream_t s) {
    hipLaunchKernelGGL((error_cols_kernel<T, FROM_SUM, MODE>), dim3(cdiv(a.n, 1024), splits), dim3(256), 0, s, a,
                       partials, per);
}

template <bool FROM_SUM, typename T>
static void launch_error_t(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s) {
    const uint32_t per = cdiv(a.rows, splits);
    if (!err_aligned(a, FROM_SUM, partials)) {
        launch_error_mode<FROM_SUM, T, 0>(a, partials, splits, per, s);
        return;
    }
    // GrpUS needs every row slice to start on a multiple of 4 rows; the last
    // slices may then be empty (their partial sums are zeros)
    const uint32_t per4 = (per + 3u) & ~3u;
    switch (a.n & 3u) {
    case 0: launch_error_mode<FROM_SUM, T, 1>(a, partials, splits, per, s); break;
    case 1: launch_error_mode<FROM_SUM, T, 5>(a, partials, splits, per4, s); break;
    case 2: launch_error_mode<FROM_SUM, T, 6>(a, partials, splits, per4, s); break;
    default: launch_error_mode<FROM_SUM, T, 7>(a, partials, splits, per4, s); break;
    }
}

hipError_t launch_output_error(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s) {
    if ((uint64_t)a.rows * a.n == 0) return hipSuccess;
    if (a.dtype == 1)
        launch_error_t<false, half_t>(a, partials, splits, s);
    else
        launch_error_t<false, float>(a, partials, splits, s);
    return hipGetLastError();
}

hipError_t launch_error_from_sum(const ErrArgs &a0, float *partials, uint32_t splits, hipStream_t s) {
    if ((uint64_t)a0.rows * a0.n == 0) return hipSuccess;
    // activation_derivative reads the output (predrop) for sigmoid, ReLU, leaky
    // ReLU, tanh and SiLU, the input (preact) for SiLU and Mish.  An operand it
    // does not read aliases the mask (same element type and index, loaded
    // anyway), so its loads hit in cache instead of streaming another [rows x n]
    // tensor from HBM, and the kernel keeps its batched loads free of branches.
    ErrArgs a = a0;
    if (!act_uses_output(a.act)) a.predrop = a.mask;
    if (!act_uses_input(a.act)) a.preact = a.mask;
    if (a.dtype == 1)
        launch_error_t<true, half_t>(a, partials, splits, s);
    else
        launch_error_t<true, float>(a, partials, splits, s);
    return hipGetLastError();
}

// ---- column sums (backward.cu:187-194) + vector optimiser (backward.cu:198-225) -------
__global__ void __launch_bounds__(256) colsum_kernel(VecOptArgs a) {
    const uint32_t col = blockIdx.x * 256 + threadIdx.x;
    if (col >= a.n) return;
    const uint32_t per = (a.rows + a.splits - 1) / a.splits;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(a.rows, r0 + per);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (!a.src[k]) continue;
        float s = 0.0f;
        for (uint32_t r = r0; r < r1; ++r) s += a.src[k][(uint64_t)r * a.n + col];
        a.partials[((uint64_t)blockIdx.y * 3 + k) * a.n + col] = s;
    }
}

// a.cpb columns per workgroup (a power of 2), 256 / cpb lanes per column: lane j
// sums the partials of splits j, j + lanes, ... in order (8 loads in flight), then
// the lanes of a column are added in a fixed tree (halving strides).  cpb comes
// from vec_opt_cpb: at most 16 splits per lane.
template <typename T> __device__ __forceinline__ void vec_opt_block(const VecOptArgs &a, uint32_t block) {
    __shared__ float red[3][256];
    const uint32_t cpb = a.cpb, lanes = 256u / cpb;
    const uint32_t cl = threadIdx.x & (cpb - 1u), j = threadIdx.x / cpb;
    const uint32_t col = block * cpb + cl;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        float s = 0.0f;
        if (a.enabled[k] && col < a.n) {
            const float *p = a.partials + (uint64_t)k * a.n + col;
            const uint64_t st = (uint64_t)3 * a.n;   // between splits
            uint32_t sp = j;
            for (; sp + 7u * lanes < a.splits; sp += 8u * lanes) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = p[(uint64_t)(sp + u * lanes) * st];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += v[u];
            }
            for (; sp < a.splits; sp += lanes) s += p[(uint64_t)sp * st];
        }
        red[k][threadIdx.x] = s;   // = red[k][j cpb + cl]
    }
    __syncthreads();
    for (uint32_t h = lanes / 2u; h >= 1u; h /= 2u) {
        if (j < h) {
#pragma unroll
            for (int k = 0; k < 3; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + h * cpb];
        }
        __syncthreads();
    }
    if (j != 0 || col >= a.n) return;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (!a.enabled[k]) continue;
        const float s = red[k][cl];
        float p = a.master[k][col], v = a.dv[k][col], mm = a.dm[k][col];
        optimiser_step(p, v, mm, s * kLossScaleInv, a.inv_m, a.lr, a.clamp, a.opt[k], 0, 0.0f, false);
        a.master[k][col] = p;
        a.dv[k][col] = v;
        a.dm[k][col] = mm;
        if (a.param[k]) stv<T>(a.param[k], col, from_f32<T>(p));
    }
}
template <typename T> __global__ void __launch_bounds__(256) vec_opt_kernel(VecOptArgs a) { vec_opt_block<T>(a, blockIdx.x); }

// Vector column sums: a thread owns 4 consecutive columns (one 16-byte load per
// row); the row range of its split is walked 8 rows at a time for loads in flight.
__global__ void __launch_bounds__(256) colsum_vec_kernel(VecOptArgs a) {
    const uint32_t c = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= a.n) return;
    const uint32_t per = (a.rows + a.splits - 1) / a.splits;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(a.rows, r0 + per);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (!a.src[k]) continue;
        const float *src = a.src[k] + c;
        f32x4 acc = {0, 0, 0, 0};
        uint32_t r = r0;
        for (; r + 8 <= r1; r += 8) {
            f32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const f32x4 *>(src + (uint64_t)(r + i) * a.n);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc += v[i];
        }
        for (; r < r1; ++r) acc += *reinterpret_cast<const f32x4 *>(src + (uint64_t)r * a.n);
        *reinterpret_cast<f32x4 *>(a.partials + ((uint64_t)blockIdx.y * 3 + k) * a.n + c) = acc;
    }
}

hipError_t launch_colsum(const VecOptArgs &a, hipStream_t s) {
    if (a.n == 0) return hipSuccess;
    bool vec = (a.n & 3u) == 0 && a16(a.partials);
    for (int k = 0; k < 3; ++k)
        if (a.src[k] && !a16(a.src[k])) vec = false;
    if (vec)
        hipLaunchKernelGGL(colsum_vec_kernel, dim3(cdiv(a.n, 1024), a.splits), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(colsum_kernel, dim3(cdiv(a.n, 256), a.splits), dim3(256), 0, s, a);
    return hipGetLastError();
}

uint32_t colsum_splits(uint32_t rows, uint32_t n) {
    const uint32_t col_blocks = (n & 3u) == 0 ? cdiv(n, 1024) : cdiv(n, 256);
    uint32_t sp = cdiv(1024, col_blocks);
    const uint32_t cap = rows / 16 > 0 ? rows / 16 : 1;
    if (sp > cap) sp = cap;
    if (sp > 256) sp = 256;
    return sp < 1 ? 1 : sp;
}

// Columns per workgroup of the parameter update: lanes per column doubled from 16
// (up to 256) until a lane has at most 16 of the `splits` partial rows to add.
uint32_t vec_opt_cpb(uint32_t splits) {
    uint32_t lanes = 16;
    while (lanes < 256 && lanes * 16 < splits) lanes *= 2;
    return 256 / lanes;
}

hipError_t launch_vec_opt(const VecOptArgs &a0, hipStream_t s) {
    if (a0.n == 0) return hipSuccess;
    VecOptArgs a = a0;
    a.cpb = vec_opt_cpb(a.splits);
    if (a.dtype == 1)
        hipLaunchKernelGGL(vec_opt_kernel<half_t>, dim3(cdiv(a.n, a.cpb)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(vec_opt_kernel<float>, dim3(cdiv(a.n, a.cpb)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---- split-K dW reduction + W optimiser ----------------------------------------------
// Thread (x, y) owns VW consecutive columns c of the rows y, y + gridDim.y, ...: it
// adds the partial planes in split order (8 loads in flight; the same sequence of
// additions as one load at a time), then applies the optimiser to each element.
// VW = 4 (16-byte accesses) when n, the plane pitches and every buffer allow it.
// Grid: 1-D, blocks [0, a.vec_blocks) run the bias / norm-parameter update of
// a.vec (vec_opt_block; independent of W), the next blocks the reduction: block
// gx * y + x, or for narrow outputs (gx = 0) one thread per element of the gy.
template <typename T, int VW> __global__ void __launch_bounds__(256) dw_reduce_opt_kernel(DwReduceArgs a, uint32_t gx,
                                                                                         uint32_t gy) {
    if (blockIdx.x < a.vec_blocks) {
        vec_opt_block<T>(a.vec, blockIdx.x);
        return;
    }
    const uint32_t bid = blockIdx.x - a.vec_blocks;
    uint32_t c, r0, rstep;
    if (gx == 0) {
        // narrow outputs (one element per thread, gy = elements): flat index
        const uint32_t el = bid * 256u + threadIdx.x;
        if (el >= gy) return;
        r0 = el / a.n;
        c = el - r0 * a.n;
        rstep = a.rows;   // one row
    } else {
        const uint32_t bx = bid % gx;
        r0 = bid / gx;
        c = (bx * 256u + threadIdx.x) * VW;
        rstep = gy;
    }
    if (c >= a.n) return;
    const OptEpi &e = a.e;
    typedef typename std::conditional<VW == 4, f32x4, float>::type V;
    for (uint32_t r = r0; r < a.rows; r += rstep) {
        const float *pp = a.partials + (uint64_t)r * a.pld + c;
        V sum = V{};
        uint32_t sp = 0;
        for (; sp + 8 <= a.splits; sp += 8) {
            V v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const V *>(pp + (uint64_t)(sp + i) * a.plane);
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += v[i];
        }
        for (; sp < a.splits; ++sp) sum += *reinterpret_cast<const V *>(pp + (uint64_t)sp * a.plane);
        const uint64_t idx = (uint64_t)r * a.n + c;
        V p = *reinterpret_cast<const V *>(e.master + idx), dv = *reinterpret_cast<const V *>(e.dv + idx),
          dm = *reinterpret_cast<const V *>(e.dm + idx);
        if constexpr (VW == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float pj = p[j], vj = dv[j], mj = dm[j];
                optimiser_step(pj, vj, mj, sum[j] * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt, e.regularisation,
                               e.regu_coeff, true);
                p[j] = pj;
                dv[j] = vj;
                dm[j] = mj;
            }
            if (e.param) store4<T>(e.param, idx, p);
        } else {
            optimiser_step(p, dv, dm, sum * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt, e.regularisation,
                           e.regu_coeff, true);
            if (e.param) stv<T>(e.param, idx, from_f32<T>(p));
        }
        *reinterpret_cast<V *>(e.master + idx) = p;
        *reinterpret_cast<V *>(e.dv + idx) = dv;
        *reinterpret_cast<V *>(e.dm + idx) = dm;
    }
}

static bool aligned_to(const void *p, uintptr_t b) { return (reinterpret_cast<uintptr_t>(p) & (b - 1)) == 0; }

template <typename T> static void launch_dw_reduce_t(const DwReduceArgs &a, hipStream_t s) {
    const bool vec = a.n % 4 == 0 && a.pld % 4 == 0 && a.plane % 4 == 0 && aligned_to(a.partials, 16) &&
                     aligned_to(a.e.master, 16) && aligned_to(a.e.dv, 16) && aligned_to(a.e.dm, 16) &&
                     (!a.e.param || aligned_to(a.e.param, 4 * sizeof(T)));
    const uint32_t vw = vec ? 4u : 1u;
    if (!vec && a.n < 128 && (uint64_t)a.rows * a.n < (1ull << 31)) {
        // narrow: one thread per element (gx = 0 selects the flat index)
        const uint32_t elems = a.rows * a.n;
        hipLaunchKernelGGL((dw_reduce_opt_kernel<T, 1>), dim3(a.vec_blocks + cdiv(elems, 256)), dim3(256), 0, s, a,
                           0u, elems);
        return;
    }
    const uint32_t gx = cdiv(a.n, 256u * vw);
    const uint32_t gy = a.rows < cdiv(4096, gx) ? a.rows : cdiv(4096, gx);   // ~4096 workgroups
    const dim3 grid(a.vec_blocks + gx * gy);
    if (vec)
        hipLaunchKernelGGL((dw_reduce_opt_kernel<T, 4>), grid, dim3(256), 0, s, a, gx, gy);
    else
        hipLaunchKernelGGL((dw_reduce_opt_kernel<T, 1>), grid, dim3(256), 0, s, a, gx, gy);
}

hipError_t launch_dw_reduce_opt(const DwReduceArgs &a0, hipStream_t s) {
    DwReduceArgs a = a0;
    a.vec.cpb = vec_opt_cpb(a.vec.splits);
    a.vec_blocks = a.with_vec && a.vec.n ? cdiv(a.vec.n, a.vec.cpb) : 0;
    if ((uint64_t)a.rows * a.n == 0) return a.vec_blocks ? launch_vec_opt(a.vec, s) : hipSuccess;
    if (a.dtype == 1)
        launch_dw_reduce_t<half_t>(a, s);
    else
        launch_dw_reduce_t<float>(a, s);
    return hipGetLastError();
}

// ---- zero-padded fp16 copy (operand staging for the 256x256 GEMM) -----------------------
// out[r][c] = (r < rows && c < cols) ? in[r ld + c] : 0 for r < rows_p, c < cols_p
// (cols_p a multiple of 8).  One wave per padded row (grid-stride over rows), lane
// l writing the 16-byte chunks l, l + 64, ... of it; 32-bit index arithmetic only.
// Every chunk of a row starts (r ld) mod 8 elements past a 16-byte boundary of the
// source, so with a 16-byte aligned base (chunks) a chunk is cut out of the two
// aligned 16-byte source chunks covering it (funnel shifts by that row-wide
// amount), as long as both lie inside the source's readable elements; element
// loads otherwise (the row's last partial chunk, the buffer's tail).
__global__ void __launch_bounds__(256) pad_h_kernel(const half_t *__restrict__ in, uint32_t rows, uint32_t cols,
                                                    uint32_t ld, half_t *__restrict__ out, uint32_t rows_p,
                                                    uint32_t cols_p, uint32_t chunks) {
    const uint32_t gpr = cols_p / 8;
    const uint64_t in_elems = rows ? (uint64_t)(rows - 1) * ld + cols : 0;   // readable source elements
    const uint32_t lane = threadIdx.x & 63u;
    for (uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6); r < rows_p; r += gridDim.x * 4u) {
        u32x4_t *orow = reinterpret_cast<u32x4_t *>(out + (uint64_t)r * cols_p);
        if (r >= rows) {
            for (uint32_t g = lane; g < gpr; g += 64u) orow[g] = u32x4_t{0, 0, 0, 0};
            continue;
        }
        const uint64_t rb = (uint64_t)r * ld;                   // first source element of the row
        const uint32_t sh = (uint32_t)(rb & 7u) * 2u;           // its byte offset within an aligned chunk
        const half_t *abase = in + (rb - (rb & 7u));            // aligned chunk holding it
        const uint32_t wd = sh >> 2, bits = (sh & 3u) * 8u;     // whole dwords, then 0 or 16 bits
        for (uint32_t g = lane; g < gpr; g += 64u) {
            const uint32_t c = g * 8u;
            u32x4_t v = {0, 0, 0, 0};
            if (c < cols) {
                if (chunks && c + 8u <= cols && rb - (rb & 7u) + c + (sh ? 16u : 8u) <= in_elems) {
                    const u32x4_t lo = *reinterpret_cast<const u32x4_t *>(abase + c);
                    const u32x4_t hi = sh ? *reinterpret_cast<const u32x4_t *>(abase + c + 8u) : lo;
                    const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t x0 = wd == 0 ? w[d] : wd == 1 ? w[d + 1] : wd == 2 ? w[d + 2] : w[d + 3];
                        const uint32_t x1 = wd == 0 ? w[d + 1] : wd == 1 ? w[d + 2] : wd == 2 ? w[d + 3] : w[d + 4];
                        v[d] = __builtin_amdgcn_alignbit(x1, x0, bits);   // (x1:x0) >> bits
                    }
                } else {
                    half_t h[8];
                    const half_t *src = in + rb + c;
#pragma unroll
                    for (uint32_t e = 0; e < 8; ++e) h[e] = c + e < cols ? src[e] : (half_t)0;
                    v = __builtin_bit_cast(u32x4_t, h);
                }
            }
            orow[g] = v;
        }
    }
}

hipError_t launch_pad_h(const void *in, uint32_t rows, uint32_t cols, uint32_t ld, void *out, uint32_t rows_p,
                        uint32_t cols_p, hipStream_t s) {
    if (cols_p % 8 || rows_p < rows || cols_p < cols || !a16(out)) return hipErrorInvalidValue;
    if (rows_p == 0 || cols_p == 0) return hipSuccess;
    const uint32_t blocks = (rows_p + 3) / 4 < 8192 ? (rows_p + 3) / 4 : 8192;   // 4 rows per block
    hipLaunchKernelGGL(pad_h_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const half_t *>(in), rows,
                       cols, ld, reinterpret_cast<half_t *>(out), rows_p, cols_p, a16(in) ? 1u : 0u);
    return hipGetLastError();
}

}  // namespace skl
