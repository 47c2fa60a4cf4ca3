// elementwise.hip — bandwidth-bound kernels of the DenseBlock hot path
// (gfx950, wave64): fill / cast, norm + activation + dropout, softmax, output
// error, hidden error from a given sum, column reductions + vector optimiser,
// split-K dW reduction + optimiser.
#include "launch.h"
#include "vec_opt.h"

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

// f32 -> f16 (round to nearest even) four elements per thread: 16-byte loads,
// 8-byte stores (n4 = n / 4 groups; the caller casts the tail).
__global__ void cast_f32_f16_x4_kernel(const f32x4 *src, uint64_t *dst, uint64_t n4) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * blockDim.x) {
        const f32x4 v = __builtin_nontemporal_load(src + i);
        half_t h[4] = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
        dst[i] = __builtin_bit_cast(uint64_t, h);
    }
}

hipError_t launch_cast(const void *src, uint32_t sdt, void *dst, uint32_t ddt, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (sdt == 0 && ddt == 1 && n >= 4 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 &&
        (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
        const uint64_t n4 = n / 4;
        hipLaunchKernelGGL(cast_f32_f16_x4_kernel, dim3((uint32_t)std::min<uint64_t>((n4 + 255) / 256, 8192)),
                           dim3(256), 0, s, (const f32x4 *)src, (uint64_t *)dst, n4);
        if (n % 4)
            hipLaunchKernelGGL((cast_kernel<float, half_t>), dim3(1), dim3(64), 0, s, (const float *)src + 4 * n4,
                               (half_t *)dst + 4 * n4, (uint64_t)(n % 4));
        return hipGetLastError();
    }
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
    const float v = activation<T>(a.act, to_f32(pre), a.leaky);
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

// 16-byte store of the chunk holding element idx of a T array, with the nontemporal hint.
template <typename T> __device__ __forceinline__ void nt_store(void *p, uint64_t idx, u32x4_t v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(reinterpret_cast<T *>(p) + idx));
}

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));
// Two fp16 values <-> their 32-bit word.  The word is a by-value parameter:
// __builtin_bit_cast applied directly to a vector element (w[q]) reads element 0
// whatever q is (seen with this compiler), so it never takes one.
__device__ __forceinline__ h2_t h2_of(uint32_t w) { return __builtin_bit_cast(h2_t, w); }
__device__ __forceinline__ uint32_t word_of(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// One 8-element chunk of an fp16 row (norm_rows_reg_kernel, 16-byte aligned rows)
// from the raw prenorm bits zr and their fp32 values z: RMSNorm's fp16
// products on packed pairs (v_pk_mul_f16), conversions back to fp16 two at a
// time (v_cvt_pk_f16_f32), the centered cache of RMSNorm stored from the raw
// bits, and the dropout keep test as an integer compare on hash bits whose
// column product advances by a constant.  Per element the same values as the
// general path below.
__device__ __forceinline__ void norm_chunk_h(const RowNormArgs &a, uint64_t idx, uint32_t row, uint32_t c0,
                                             u32x4_t zr, const float *z, float mean, float rstd32, half_t rstd_t,
                                             float scale) {
    const u32x4_t gr = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const half_t *>(a.norm_w) + c0);
    u32x4_t pre, cen;
    if (a.norm == 1) {
        // (prenorm * rstd) * norm_w in fp16 (forward.cu:61-72): the product of two fp16
        // values is exact in fp32, so rounding it to fp16 is one fp16 multiply
        const h2_t r2 = {rstd_t, rstd_t};
#pragma unroll
        for (int q = 0; q < 4; ++q) pre[q] = word_of((h2_of(zr[q]) * r2) * h2_of(gr[q]));
        cen = zr;   // RMSNorm's centered cache is prenorm itself
    } else {
        const u32x4_t br = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const half_t *>(a.norm_b) + c0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f2_t v = {z[2 * q] - mean, z[2 * q + 1] - mean};
            const f2_t g = __builtin_convertvector(h2_of(gr[q]), f2_t);
            const f2_t b = __builtin_convertvector(h2_of(br[q]), f2_t);
            cen[q] = word_of(__builtin_convertvector(v, h2_t));
            const f2_t pf = {fmaf(v.x * rstd32, g.x, b.x), fmaf(v.y * rstd32, g.y, b.y)};
            pre[q] = word_of(__builtin_convertvector(pf, h2_t));
        }
    }
    f2_t act[4];
    u32x4_t pd;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f2_t pf = __builtin_convertvector(h2_of(pre[q]), f2_t);
        act[q] = f2_t{activation<half_t>(a.act, pf.x, a.leaky), activation<half_t>(a.act, pf.y, a.leaky)};
        pd[q] = word_of(__builtin_convertvector(act[q], h2_t));
    }
    // nontemporal: five write streams, read again only by later kernels
    nt_store<half_t>(a.centered, idx, cen);
    nt_store<half_t>(a.preact, idx, pre);
    nt_store<half_t>(a.predrop, idx, pd);
    if (!a.use_dropout) {
        nt_store<half_t>(a.out, idx, pd);
        return;
    }
    const uint32_t rk = dropout_rowkey(row, a.seed + row * 7u);
    const uint32_t cm0 = c0 * kDropColMul;
    const half_t sc = (half_t)scale;
    u32x4_t mk, ot;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const h2_t os = __builtin_convertvector(act[q] * scale, h2_t);
        h2_t m2, o2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool keep = (uint64_t)dropout_bits(cm0 + (uint32_t)(2 * q + h) * kDropColMul, rk) >= a.keep_min;
            m2[h] = keep ? sc : (half_t)0;
            o2[h] = keep ? os[h] : (half_t)0;
        }
        mk[q] = word_of(m2);
        ot[q] = word_of(o2);
    }
    nt_store<half_t>(a.mask, idx, mk);
    nt_store<half_t>(a.out, idx, ot);
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
    u32x4_t zr[PER];   // raw chunks (the fp16 chunk path stores RMSNorm's centered cache from them)
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
            zr[i] = *reinterpret_cast<const u32x4_t *>(v);
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
        if constexpr (VEC && sizeof(T) == 2) {
            norm_chunk_h(a, base + c0, row, c0, zr[i], &z[i * VW], mean, rstd32, rstd_t, scale);
            continue;
        }
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
            const float act = activation<T>(a.act, to_f32(p), a.leaky);
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
            // nontemporal: five write streams, read again only by later kernels
            nt_store<T>(a.centered, idx, *reinterpret_cast<u32x4_t *>(cen));
            nt_store<T>(a.preact, idx, *reinterpret_cast<u32x4_t *>(pre));
            nt_store<T>(a.predrop, idx, *reinterpret_cast<u32x4_t *>(pd));
            nt_store<T>(a.out, idx, *reinterpret_cast<u32x4_t *>(ot));
            if (a.use_dropout) nt_store<T>(a.mask, idx, *reinterpret_cast<u32x4_t *>(mk));
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
            const float act = activation<T>(a.act, to_f32(p), a.leaky);
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
            // nontemporal: five write streams, read again only by later kernels
            __builtin_nontemporal_store(*reinterpret_cast<G *>(cen), reinterpret_cast<G *>(a.centered) + gi);
            __builtin_nontemporal_store(*reinterpret_cast<G *>(pre), reinterpret_cast<G *>(a.preact) + gi);
            __builtin_nontemporal_store(*reinterpret_cast<G *>(pd), reinterpret_cast<G *>(a.predrop) + gi);
            __builtin_nontemporal_store(*reinterpret_cast<G *>(ot), reinterpret_cast<G *>(a.out) + gi);
            if (a.use_dropout) __builtin_nontemporal_store(*reinterpret_cast<G *>(mk), reinterpret_cast<G *>(a.mask) + gi);
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

hipError_t launch_norm_act(const RowNormArgs &a0, hipStream_t s) {
    if (a0.m == 0 || a0.n == 0) return hipSuccess;
    RowNormArgs a = a0;
    a.keep_min = dropout_keep_min(a.p);
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

// Rows of at most 64 elements (an output layer's classes): one wave per row,
// lane c holding column c, max and sum over the wave with butterfly shuffles.
// A workgroup per 10-element row (C4) kept 246 of its 256 threads idle and ran
// 15 us for 16384 rows.
template <typename T> __global__ void __launch_bounds__(256) softmax_wave_kernel(T *out, uint32_t rows, uint32_t n) {
    const uint32_t row = blockIdx.x * 4u + threadIdx.x / 64u, c = threadIdx.x & 63u;
    if (row >= rows) return;   // uniform over the wave
    const uint64_t base = (uint64_t)row * n;
    const float x = c < n ? to_f32(out[base + c]) : -INFINITY;
    float mx = x;
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) mx = fmaxf(mx, __shfl_xor(mx, off));
    const float e = c < n ? expf(x - mx) : 0.0f;
    float sum = e;
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) sum += __shfl_xor(sum, off);
    if (c < n) out[base + c] = from_f32<T>(e / sum);
}

hipError_t launch_softmax(uint32_t dtype, void *out, uint32_t rows, uint32_t n, hipStream_t s) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (n <= 64) {
        const dim3 g(cdiv(rows, 4u));
        if (dtype == 1)
            hipLaunchKernelGGL(softmax_wave_kernel<half_t>, g, dim3(256), 0, s, (half_t *)out, rows, n);
        else
            hipLaunchKernelGGL(softmax_wave_kernel<float>, g, dim3(256), 0, s, (float *)out, rows, n);
        return hipGetLastError();
    }
    if (dtype == 1)
        hipLaunchKernelGGL(softmax_kernel<half_t>, dim3(rows), dim3(256), 0, s, (half_t *)out, n);
    else
        hipLaunchKernelGGL(softmax_kernel<float>, dim3(rows), dim3(256), 0, s, (float *)out, n);
    return hipGetLastError();
}

// ---- error kernels ------------------------------------------------------------------
// Loss delta of one element (backward.cu:24-45).
template <typename T> __device__ __forceinline__ float output_err1(const ErrArgs &a, float out, float tg, float pre) {
    const float o = activation<T>(a.act, out, a.leaky);
    if (a.loss == 0) return activation_derivative<T>(a.act, o - tg, o, pre, a.leaky);
    if ((a.loss == 1 && a.act == 5) || (a.loss == 2 && a.act == 1)) return o - tg;
    return 0.0f;
}

// The element-local norm gradient (util.cu:175-215) of one element with error e;
// pc is its prenorm (RMS) or centered (LN, BN) value.  d_prenorm carries the
// loss scale.
struct ErrOut {
    float dp, dnw, dnb;
};
__device__ __forceinline__ ErrOut err_norm1(const ErrArgs &a, float e, float pc, float rstd, float nw) {
    ErrOut o{e, 0.0f, 0.0f};
    if (a.norm) {
        const NormGrad g =
            norm_grad(a.norm, e, a.norm == 1 ? pc : 0.0f, a.norm >= 2 ? pc : 0.0f, rstd, nw, a.inv_n, a.inv_m);
        o = ErrOut{g.d_prenorm, g.dnw, g.dnb};
    }
    o.dp = o.dp * a.loss_scale;
    return o;
}

struct ErrAcc {   // running column sums of a thread's 4 elements
    f32x4 dp, nw, nb;
};

// Error + column sums in one pass (backward.cu:12-56 for the output layer,
// 79-100 for the hidden error from the sum s), on 16-byte aligned buffers: the
// [rows x n] arrays as one flat array.  A band of B = 4 / gcd(n, 4) rows holds
// B n / 4 whole 4-element chunks; thread j owns chunk j of every band of its
// row slice, so each load and store of a row-strided array is one 16-byte
// (fp32) or 8-byte (fp16) access whatever n is.  Element q of the chunk lies
// in row r_q = (4 j + q) / n of the band and column c_q = (4 j + q) % n, the
// same in every band: the per-column operands are loaded once, and the thread
// keeps the column sums of its four elements (rows in ascending order), which
// go to partial row y B + r_q of partials [S B x 3 x n] (k = 0 d_prenorm,
// 1 dNorm_w, 2 dNorm_b; 1 and 2 only with a norm).  The backward adds all
// partial rows for the bias / norm-parameter update, so it does not read the
// three [rows x n] buffers again.  Workgroup (x, y) owns chunks
// [256 x, 256 (x + 1)) of the bands [y per, (y + 1) per); UB bands of every
// operand are loaded before any is computed.
//
// SRC: 0 the output layer's loss delta, 1 the hidden error from s in memory,
// 2 the hidden error with s = A . W^T formed per element (backward.cu:72-77
// for a next layer of at most 16 outputs: A [rows x 16] and W [n x 16] are
// zero-padded T copies of the next layer's d_prenorm (fp16 blocks: its fp16
// copy) and weights, so an element's sum is an fp32 sum over k in ascending
// order (skinny_dot), and s never goes through HBM).  With SRC 2 the thread
// keeps its four columns of W in registers (as T: half the registers of fp32
// for fp16 blocks); the n >= 4 it needs puts a chunk's elements in at most two
// rows, and both rows' sums are formed before the element picks its own.
constexpr int ERR_UB = 4;
// 4 consecutive T elements with the nontemporal hint (read once).
template <typename T> __device__ __forceinline__ f32x4 load4_nt(const void *p, uint64_t i) {
    if constexpr (sizeof(T) == 2) {
        const f16x4 h =
            __builtin_nontemporal_load(reinterpret_cast<const f16x4 *>(reinterpret_cast<const half_t *>(p) + i));
        return f32x4{(float)h.x, (float)h.y, (float)h.z, (float)h.w};
    } else {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(p) + i));
    }
}
struct FlatPos {
    uint32_t r[4], c[4];
};
template <typename T> struct ErrCol {   // per-column operands of the 4 elements
    f32x4 nw, rstd;
    T w[4][16];   // SRC 2: W's 16 values of each element's column
};

template <typename T, int B> struct SkRows {   // SRC 2: A's rows of a chunk's first and last element
    T lo[16], hi[B > 1 ? 16 : 1];
};

// 16 consecutive T of a 16-byte aligned row.
template <typename T> __device__ __forceinline__ void load16(T (&dst)[16], const void *p, uint64_t row) {
    const u32x4_t *src = reinterpret_cast<const u32x4_t *>(reinterpret_cast<const T *>(p) + row * 16);
    constexpr int W = 16 * sizeof(T) / 16;
#pragma unroll
    for (int i = 0; i < W; ++i) reinterpret_cast<u32x4_t *>(dst)[i] = src[i];
}

// s of one element from its row of A and column of W (16 values each): fp32
// FMAs over k in ascending order; fp16 operands as 8 v_dot2_f32_f16 on packed
// pairs (each pair's two exact products added in fp32), so W stays packed.
__device__ __forceinline__ float skinny_dot(const float (&av)[16], const float (&wv)[16]) {
    float sv = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) sv = __builtin_fmaf(av[k], wv[k], sv);
    return sv;
}
__device__ __forceinline__ float skinny_dot(const half_t (&av)[16], const half_t (&wv)[16]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    float sv = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k += 2) sv = __builtin_amdgcn_fdot2(h2{av[k], av[k + 1]}, h2{wv[k], wv[k + 1]}, sv, false);
    return sv;
}

template <typename T, int SRC, int B, bool NORM, int UB>
__device__ __forceinline__ void err_flat_bands(const ErrArgs &a, uint32_t b, uint32_t j, uint32_t s_ld,
                                               const FlatPos &fp, const ErrCol<T> &col, ErrAcc &acc) {
    const uint32_t n = a.n;
    // fp16 blocks without a norm (the single-block error from a sum, C3) read the
    // per-element operands with the nontemporal hint: the C3 error call 0.139 ->
    // 0.118 ms, the step +1.4%; with a norm (C4, C5) it changed nothing or cost
    // up to 0.5%, and C2's fp32 call (its 50 MB stay in the last-level cache)
    // 0.0176 -> 0.019 ms.  Stores stay plain (nontemporal ones cost 10-15% here).
    constexpr bool NTL = !NORM && sizeof(T) == 2;
    f32x4 x[3][UB], mk[UB], pc[UB], rs[UB];
    SkRows<T, B> ar[SRC == 2 ? UB : 1];
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const uint32_t row0 = (b + u) * B;
        const uint64_t base = (uint64_t)row0 * n + 4ull * j;
        if constexpr (SRC == 1) {
            if constexpr (B == 1 && NTL) {
                // the four addresses are consecutive and 16-byte aligned (the launcher
                // checks s_ld % 4 == 0)
                x[0][u] = load4_nt<float>(a.s, (uint64_t)row0 * s_ld + fp.c[0]);
            } else {
                // (one 16-byte load when B == 1: the four addresses are consecutive)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    x[0][u][q] = a.s[(uint64_t)(row0 + fp.r[q]) * s_ld + fp.c[q]];
            }
        } else if constexpr (SRC == 2) {
            load16<T>(ar[u].lo, a.sk_a, row0 + fp.r[0]);
            if constexpr (B > 1) load16<T>(ar[u].hi, a.sk_a, row0 + fp.r[3]);
        }
        if constexpr (SRC != 0) {
            x[1][u] = NTL ? load4_nt<T>(a.predrop, base) : load4<T>(a.predrop, base);
            x[2][u] = NTL ? load4_nt<T>(a.preact, base) : load4<T>(a.preact, base);
            mk[u] = NTL ? load4_nt<T>(a.mask, base) : load4<T>(a.mask, base);
        } else {
            x[0][u] = load4<T>(a.out, base);
            x[1][u] = load4<T>(a.target, base);
            x[2][u] = load4<T>(a.preact, base);
        }
        if constexpr (NORM) {
            pc[u] = load4<T>(a.norm_in, base);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                rs[u][q] = (B == 1 && q > 0) ? rs[u][0] : to_f32(ldv<T>(a.norm_rstd, row0 + fp.r[q]));
        }
    }
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const uint64_t base = (uint64_t)(b + u) * B * n + 4ull * j;
        if constexpr (SRC == 2) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float slo = skinny_dot(ar[u].lo, col.w[q]);
                if constexpr (B > 1)
                    x[0][u][q] = fp.r[q] == fp.r[0] ? slo : skinny_dot(ar[u].hi, col.w[q]);
                else
                    x[0][u][q] = slo;
            }
        }
        f32x4 e;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (SRC != 0)
                e[q] = mk[u][q] * activation_derivative<T>(a.act, x[0][u][q], x[1][u][q], x[2][u][q], a.leaky);
            else
                e[q] = output_err1<T>(a, x[0][u][q], x[1][u][q], x[2][u][q]);
        }
        store4<float>(a.grad, base, e);
        f32x4 dp = e * a.loss_scale;
        if constexpr (NORM) {
            f32x4 dnw, dnb;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // BatchNorm's rstd is per column; the row value loaded for it is not used
                const ErrOut o = err_norm1(a, e[q], pc[u][q], a.norm == 3 ? col.rstd[q] : rs[u][q], col.nw[q]);
                dp[q] = o.dp;
                dnw[q] = o.dnw;
                dnb[q] = o.dnb;
            }
            store4<float>(a.d_norm_w, base, dnw);
            store4<float>(a.d_norm_b, base, dnb);
            acc.nw += dnw;
            acc.nb += dnb;
        }
        store4<float>(a.d_prenorm, base, dp);
        if (a.d_prenorm_h) store4<half_t>(a.d_prenorm_h, base, dp);
        acc.dp += dp;
    }
}

// The last band when rows % B != 0: element by element, rows past the end skipped.
template <typename T, int SRC, int B>
__device__ __forceinline__ void err_flat_tail(const ErrArgs &a, uint32_t b, uint32_t s_ld, const FlatPos &fp,
                                              const ErrCol<T> &col, ErrAcc &acc) {
    const uint32_t n = a.n;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t row = b * B + fp.r[q];
        if (row >= a.rows) continue;
        const uint64_t i = (uint64_t)row * n + fp.c[q];
        float e;
        if constexpr (SRC != 0) {
            float sv;
            if constexpr (SRC == 1) {
                sv = a.s[(uint64_t)row * s_ld + fp.c[q]];
            } else {
                T av[16];
                load16<T>(av, a.sk_a, row);
                sv = skinny_dot(av, col.w[q]);
            }
            e = to_f32(ldv<T>(a.mask, i)) *
                activation_derivative<T>(a.act, sv, to_f32(ldv<T>(a.predrop, i)), to_f32(ldv<T>(a.preact, i)), a.leaky);
        } else {
            e = output_err1<T>(a, to_f32(ldv<T>(a.out, i)), to_f32(ldv<T>(a.target, i)), to_f32(ldv<T>(a.preact, i)));
        }
        const float pcv = a.norm ? to_f32(ldv<T>(a.norm_in, i)) : 0.0f;
        const float rstd = (a.norm == 1 || a.norm == 2) ? to_f32(ldv<T>(a.norm_rstd, row)) : col.rstd[q];
        const ErrOut o = err_norm1(a, e, pcv, rstd, col.nw[q]);
        a.grad[i] = e;
        if (a.norm) {
            a.d_norm_w[i] = o.dnw;
            a.d_norm_b[i] = o.dnb;
        }
        a.d_prenorm[i] = o.dp;
        if (a.d_prenorm_h) a.d_prenorm_h[i] = (half_t)o.dp;
        acc.dp[q] += o.dp;
        acc.nw[q] += o.dnw;
        acc.nb[q] += o.dnb;
    }
}

template <typename T, int SRC, int B, bool NORM>
__global__ void __launch_bounds__(256) error_flat_kernel(ErrArgs a, float *__restrict__ partials, uint32_t per) {
    constexpr int UB = SRC == 2 ? 2 : ERR_UB;
    const uint32_t n = a.n;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if ((uint64_t)j * 4 >= (uint64_t)B * n) return;
    FlatPos fp;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = 4 * j + q;
        fp.r[q] = B == 1 ? 0u : e / n;
        fp.c[q] = e - fp.r[q] * n;
    }
    ErrCol<T> col{};
    if constexpr (NORM) {
#pragma unroll
        for (int q = 0; q < 4; ++q) col.nw[q] = a.nw[fp.c[q]];
        if (a.norm == 3) {   // BatchNorm: rstd per column
#pragma unroll
            for (int q = 0; q < 4; ++q) col.rstd[q] = to_f32(ldv<T>(a.norm_rstd, fp.c[q]));
        }
    }
    if constexpr (SRC == 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) load16<T>(col.w[q], a.sk_w, fp.c[q]);
    }
    const uint32_t s_ld = a.s_ld ? a.s_ld : n;
    const uint32_t full = a.rows / B, bands = (a.rows + B - 1) / B;
    const uint32_t b0 = blockIdx.y * per, b1 = min(bands, b0 + per), bf = min(b1, full);
    ErrAcc acc{{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    uint32_t b = b0;
    for (; b + UB <= bf; b += UB) err_flat_bands<T, SRC, B, NORM, UB>(a, b, j, s_ld, fp, col, acc);
    for (; b < bf; ++b) err_flat_bands<T, SRC, B, NORM, 1>(a, b, j, s_ld, fp, col, acc);
    if (b < b1) err_flat_tail<T, SRC, B>(a, b, s_ld, fp, col, acc);
    float *p = partials + (uint64_t)blockIdx.y * B * 3 * n;
    if constexpr (B == 1) {
        store4<float>(p, 4ull * j, acc.dp);
        if constexpr (NORM) {
            store4<float>(p + n, 4ull * j, acc.nw);
            store4<float>(p + 2 * (uint64_t)n, 4ull * j, acc.nb);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float *pr = p + (uint64_t)fp.r[q] * 3 * n + fp.c[q];
            pr[0] = acc.dp[q];
            if constexpr (NORM) {
                pr[n] = acc.nw[q];
                pr[2 * (uint64_t)n] = acc.nb[q];
            }
        }
    }
}

// Buffers at any alignment (a row-strided array or a per-column vector not
// 16-byte aligned): a thread owns 4 consecutive columns of one row (cnt <= 4 of
// them exist), read as the aligned 4-element chunk holding the group's first
// element plus, when the group runs into the next chunk, that chunk too.  Each
// chunk read holds an element of the group, so no read leaves the 16-byte
// blocks the group's own elements lie in.  Stores split the group at the chunk
// boundary into aligned 1-, 2- and 4-element pieces.  Only the lane that holds
// a row's last, partial group (cnt < 4) takes the element-by-element path.
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
    __device__ __forceinline__ static f32x4 ldf(const float *p, uint64_t i, uint32_t cnt) {
        return load<float>(p, i, cnt);
    }
    __device__ __forceinline__ static void stf(float *p, uint64_t i, f32x4 v, uint32_t cnt) {
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

// The error kernel on GrpUA accesses: workgroup (x, y) owns the columns
// [1024 x, 1024 (x + 1)) of the rows [y per, (y + 1) per), a thread one
// 4-column group, ERR_UR rows loaded before any is computed (from a sum) or
// row by row (output layer); column sums to partials[y][k][n].
constexpr int ERR_UR = 4;
template <typename T, bool FROM_SUM>
__device__ __forceinline__ void err_row_ua(const ErrArgs &a, uint32_t row, uint32_t c, uint32_t cnt, f32x4 s,
                                           f32x4 pd, f32x4 pa, f32x4 mk, ErrAcc &acc) {
    typedef GrpUA<T> G;
    const uint64_t idx = (uint64_t)row * a.n + c;
    f32x4 e;
    if constexpr (FROM_SUM) {
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = mk[j] * activation_derivative<T>(a.act, s[j], pd[j], pa[j], a.leaky);
    } else {
        const f32x4 out = G::ld(a.out, idx, cnt), tg = G::ld(a.target, idx, cnt), pre = G::ld(a.preact, idx, cnt);
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = output_err1<T>(a, out[j], tg[j], pre[j]);
    }
    G::stf(a.grad, idx, e, cnt);
    f32x4 dp, dnw, dnb;
    const f32x4 pc = a.norm ? G::ld(a.norm_in, idx, cnt) : f32x4{0, 0, 0, 0};
    const f32x4 nw = a.norm ? GrpUA<float>::ldf(a.nw, c, cnt) : f32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float rstd =
            a.norm ? to_f32(ldv<T>(a.norm_rstd, a.norm == 3 ? c + (j < (int)cnt ? j : 0) : row)) : 0.0f;
        const ErrOut o = err_norm1(a, e[j], pc[j], rstd, nw[j]);
        const bool live = j < (int)cnt;   // columns past n add nothing to the sums
        dp[j] = live ? o.dp : 0.0f;
        dnw[j] = live ? o.dnw : 0.0f;
        dnb[j] = live ? o.dnb : 0.0f;
    }
    if (a.norm) {
        G::stf(a.d_norm_w, idx, dnw, cnt);
        G::stf(a.d_norm_b, idx, dnb, cnt);
    }
    G::stf(a.d_prenorm, idx, dp, cnt);
    if (a.d_prenorm_h) G::sth(a.d_prenorm_h, idx, dp, cnt);
    acc.dp += dp;
    acc.nw += dnw;
    acc.nb += dnb;
}

template <typename T, bool FROM_SUM>
__global__ void __launch_bounds__(256) error_cols_kernel(ErrArgs a, float *__restrict__ partials, uint32_t per) {
    typedef GrpUA<T> G;
    const uint32_t c = blockIdx.x * 1024 + threadIdx.x * 4;
    if (c >= a.n) return;
    const uint32_t cnt = min(4u, a.n - c);
    const uint32_t s_ld = a.s_ld ? a.s_ld : a.n;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(a.rows, r0 + per);
    ErrAcc acc{{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    for (uint32_t rb = r0; rb < r1; rb += ERR_UR) {
        f32x4 s[ERR_UR] = {}, pd[ERR_UR] = {}, pa[ERR_UR] = {}, mk[ERR_UR] = {};
#pragma unroll
        for (int u = 0; u < ERR_UR; ++u) {
            if (!FROM_SUM || rb + u >= r1) continue;
            const uint64_t idx = (uint64_t)(rb + u) * a.n + c;
            s[u] = GrpUA<float>::ldf(a.s, (uint64_t)(rb + u) * s_ld + c, cnt);
            pd[u] = G::ld(a.predrop, idx, cnt);
            pa[u] = G::ld(a.preact, idx, cnt);
            mk[u] = G::ld(a.mask, idx, cnt);
        }
#pragma unroll
        for (int u = 0; u < ERR_UR; ++u)
            if (rb + u < r1) err_row_ua<T, FROM_SUM>(a, rb + u, c, cnt, s[u], pd[u], pa[u], mk[u], acc);
    }
    float *p = partials + (uint64_t)blockIdx.y * 3 * a.n + c;
    GrpUA<float>::stf(p, 0, acc.dp, cnt);
    if (a.norm) {
        GrpUA<float>::stf(p + a.n, 0, acc.nw, cnt);
        GrpUA<float>::stf(p + 2 * a.n, 0, acc.nb, cnt);
    }
}

static bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Every buffer the flat kernel touches 16-byte aligned (s at any row pitch: a
// pitch other than n is read element by element); partials only when n % 4 == 0
// (its 4-element stores).
static bool err_aligned(const ErrArgs &a, bool from_sum, const float *partials) {
    const void *ptrs[] = {a.grad, a.d_prenorm, a.d_prenorm_h, a.preact, a.norm ? a.nw : nullptr,
                          a.norm ? a.d_norm_w : nullptr, a.norm ? a.d_norm_b : nullptr,
                          a.norm == 1 ? a.prenorm : nullptr, a.norm >= 2 ? a.centered : nullptr,
                          from_sum ? a.s : a.out, from_sum ? a.predrop : a.target, from_sum ? a.mask : nullptr,
                          (a.n & 3u) == 0 ? partials : nullptr};
    for (const void *p : ptrs)
        if (p && !a16(p)) return false;
    return true;
}

// Rows per band of the flat error kernel: 4 / gcd(n, 4).
static uint32_t err_band(uint32_t n) { return (n & 3u) == 0 ? 1u : (n & 1u) ? 4u : 2u; }

// Partial-sum rows of the error kernels: S row slices x err_band(n).  ~1024
// workgroups of >= 16 rows when a band has >= 256 chunks; narrower outputs
// leave most of a workgroup's lanes idle, so they get ~256K active lanes in
// all, in slices of >= 4 rows (at most 4096 slices).  resident (when not 0):
// the kernel's workgroups the GPU holds at once; a grid that would exceed it
// gets fewer, longer slices that fill it exactly, rather than a second round
// of a few workgroups (C5's error kernels: 1026 workgroups of which 1024 fit,
// and 1032 of which 768 fit).
uint32_t err_col_splits(uint32_t rows, uint32_t n, uint32_t resident) {
    const uint32_t band = err_band(n);
    const uint64_t chunks = (uint64_t)band * n / 4;   // lanes per band
    const uint32_t gx = (uint32_t)cdiv(chunks ? chunks : 1, 256);   // workgroups per row slice
    uint32_t sp, cap;
    if (chunks >= 256) {
        sp = cdiv(1024, gx);
        cap = cdiv(rows, 16);
    } else {
        sp = cdiv(262144u, chunks ? chunks : 1);
        cap = cdiv(rows, 4);
    }
    if (sp > cap) sp = cap;
    if (sp > cdiv(rows, band)) sp = cdiv(rows, band);
    if (sp > 4096) sp = 4096;
    if (resident && (uint64_t)sp * gx > resident && resident / gx >= 1) sp = resident / gx;
    return (sp < 1 ? 1 : sp) * band;
}

// Workgroups of error_flat_kernel<T, SRC, B, NORM> per CU (its register use
// sets it), from the runtime's occupancy calculator, once per variant.
template <typename T, int SRC, int B, bool NORM> static uint32_t err_flat_per_cu() {
    static const uint32_t v = [] {
        int nb = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void *>(&error_flat_kernel<T, SRC, B, NORM>), 256, 0);
        return e == hipSuccess && nb > 0 ? (uint32_t)nb : 0u;
    }();
    return v;
}
template <typename T, int SRC, int B> static uint32_t err_flat_per_cu_n(bool norm) {
    return norm ? err_flat_per_cu<T, SRC, B, true>() : err_flat_per_cu<T, SRC, B, false>();
}
template <typename T, int SRC> static uint32_t err_flat_per_cu_b(uint32_t band, bool norm) {
    return band == 1 ? err_flat_per_cu_n<T, SRC, 1>(norm)
                     : band == 2 ? err_flat_per_cu_n<T, SRC, 2>(norm) : err_flat_per_cu_n<T, SRC, 4>(norm);
}
template <typename T> static uint32_t err_flat_per_cu_s(uint32_t src, uint32_t band, bool norm) {
    return src == 0 ? err_flat_per_cu_b<T, 0>(band, norm)
                    : src == 1 ? err_flat_per_cu_b<T, 1>(band, norm) : err_flat_per_cu_b<T, 2>(band, norm);
}

uint32_t err_resident(uint32_t dtype, uint32_t src, uint32_t n, bool norm) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 0;
    const uint32_t band = err_band(n);
    const uint32_t per_cu = dtype == 1 ? err_flat_per_cu_s<half_t>(src, band, norm)
                                       : err_flat_per_cu_s<float>(src, band, norm);
    return per_cu * (uint32_t)cus;
}

template <int SRC, typename T, int B>
static void launch_error_flat(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s) {
    const uint32_t S = splits / B;
    const uint32_t per = cdiv(cdiv(a.rows, B), S);
    const dim3 grid(cdiv((uint64_t)B * a.n, 1024), S);
    if (a.norm)
        hipLaunchKernelGGL((error_flat_kernel<T, SRC, B, true>), grid, dim3(256), 0, s, a, partials, per);
    else
        hipLaunchKernelGGL((error_flat_kernel<T, SRC, B, false>), grid, dim3(256), 0, s, a, partials, per);
}

// splits: the partial-sum rows, from err_col_splits.
template <bool FROM_SUM, typename T>
static hipError_t launch_error_t(const ErrArgs &a0, float *partials, uint32_t splits, hipStream_t s) {
    ErrArgs a = a0;
    a.norm_in = a.norm == 1 ? a.prenorm : a.centered;
    // the flat kernel reads a row of s as 16-byte chunks when n % 4 == 0: the
    // pitch must keep them aligned
    const bool s_ok = !FROM_SUM || (a.n & 3u) != 0 || ((a.s_ld ? a.s_ld : a.n) & 3u) == 0;
    if (!s_ok || !err_aligned(a, FROM_SUM, partials)) {
        hipLaunchKernelGGL((error_cols_kernel<T, FROM_SUM>), dim3(cdiv(a.n, 1024), splits), dim3(256), 0, s, a,
                           partials, cdiv(a.rows, splits));
        return hipGetLastError();
    }
    const uint32_t band = err_band(a.n);
    if (splits < band || splits % band) return hipErrorInvalidValue;
    constexpr int SRC = FROM_SUM ? 1 : 0;
    switch (band) {
    case 1: launch_error_flat<SRC, T, 1>(a, partials, splits, s); break;
    case 2: launch_error_flat<SRC, T, 2>(a, partials, splits, s); break;
    default: launch_error_flat<SRC, T, 4>(a, partials, splits, s); break;
    }
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_error_skinny_t(const ErrArgs &a0, float *partials, uint32_t splits, hipStream_t s) {
    ErrArgs a = a0;
    a.norm_in = a.norm == 1 ? a.prenorm : a.centered;
    const uint32_t band = err_band(a.n);
    if (!err_skinny_ok(a, partials) || splits < band || splits % band) return hipErrorInvalidValue;
    switch (band) {
    case 1: launch_error_flat<2, T, 1>(a, partials, splits, s); break;
    case 2: launch_error_flat<2, T, 2>(a, partials, splits, s); break;
    default: launch_error_flat<2, T, 4>(a, partials, splits, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_output_error(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s) {
    if ((uint64_t)a.rows * a.n == 0) return hipSuccess;
    return a.dtype == 1 ? launch_error_t<false, half_t>(a, partials, splits, s)
                        : launch_error_t<false, float>(a, partials, splits, s);
}

bool err_skinny_ok(const ErrArgs &a, const float *partials) {
    return a.n >= 4 && a.sk_a && a.sk_w && a16(a.sk_a) && a16(a.sk_w) && err_aligned(a, true, partials);
}

// Columns of a skinny operand's fp32 copy.
constexpr uint32_t SK_COLS = 16;

// dst[r][k] = k < cols ? src[r cols + k] : 0 for k < 16: the next layer's
// d_prenorm (rows = batch) or weights (rows = n) as the hidden error's skinny
// operands, rows of A then rows of W in one launch.
template <typename T>
__global__ void __launch_bounds__(256) skinny_operands_kernel(const T *a, uint32_t a_rows, const T *w, uint32_t w_rows,
                                                              uint32_t cols, T *a16, T *w16) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t k = (uint32_t)(i % SK_COLS);
    const uint64_t r = i / SK_COLS;
    if (r < a_rows) {
        a16[i] = k < cols ? a[r * cols + k] : (T)0;
    } else if (r < (uint64_t)a_rows + w_rows) {
        const uint64_t rw = r - a_rows;
        w16[rw * SK_COLS + k] = k < cols ? w[rw * cols + k] : (T)0;
    }
}

hipError_t launch_skinny_operands(uint32_t dtype, const void *a, uint32_t a_rows, const void *w, uint32_t w_rows,
                                  uint32_t cols, void *a16, void *w16, hipStream_t s) {
    if (cols == 0 || cols > SK_COLS) return hipErrorInvalidValue;
    const uint64_t threads = ((uint64_t)a_rows + w_rows) * SK_COLS;
    if (threads == 0) return hipSuccess;
    const dim3 grid(cdiv(threads, 256));
    if (dtype == 1)
        hipLaunchKernelGGL((skinny_operands_kernel<half_t>), grid, dim3(256), 0, s, reinterpret_cast<const half_t *>(a),
                           a_rows, reinterpret_cast<const half_t *>(w), w_rows, cols, reinterpret_cast<half_t *>(a16),
                           reinterpret_cast<half_t *>(w16));
    else
        hipLaunchKernelGGL((skinny_operands_kernel<float>), grid, dim3(256), 0, s, reinterpret_cast<const float *>(a),
                           a_rows, reinterpret_cast<const float *>(w), w_rows, cols, reinterpret_cast<float *>(a16),
                           reinterpret_cast<float *>(w16));
    return hipGetLastError();
}

hipError_t launch_error_skinny(const ErrArgs &a0, float *partials, uint32_t splits, hipStream_t s) {
    if ((uint64_t)a0.rows * a0.n == 0) return hipSuccess;
    ErrArgs a = a0;
    if (!act_uses_output(a.act)) a.predrop = a.mask;
    if (!act_uses_input(a.act)) a.preact = a.mask;
    return a.dtype == 1 ? launch_error_skinny_t<half_t>(a, partials, splits, s)
                        : launch_error_skinny_t<float>(a, partials, splits, s);
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
    return a.dtype == 1 ? launch_error_t<true, half_t>(a, partials, splits, s)
                        : launch_error_t<true, float>(a, partials, splits, s);
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
// loads the element's optimiser state, adds the partial planes in split order
// (batches of 8 loads in flight, the last batch of 1-7 loaded in one go from
// clamped plane indices and added under a select; the same sequence of additions
// as one load at a time), then applies the optimiser to each element (against a
// load-add-wait per plane: C4 unchanged, C5's step 0.6% faster).
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
        const uint64_t idx = (uint64_t)r * a.n + c;
        V p = *reinterpret_cast<const V *>(e.master + idx), dv = *reinterpret_cast<const V *>(e.dv + idx),
          dm = *reinterpret_cast<const V *>(e.dm + idx);
        V sum = V{};
        uint32_t sp = 0;
        for (; sp + 8 <= a.splits; sp += 8) {
            V v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const V *>(pp + (uint64_t)(sp + i) * a.plane);
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += v[i];
        }
        if (sp < a.splits) {
            const uint32_t last = a.splits - 1;
            V v[7];
#pragma unroll
            for (int i = 0; i < 7; ++i) {
                const uint32_t q = sp + i < last ? sp + i : last;
                v[i] = *reinterpret_cast<const V *>(pp + (uint64_t)q * a.plane);
            }
#pragma unroll
            for (int i = 0; i < 7; ++i) sum = sp + i < a.splits ? sum + v[i] : sum;
        }
        if constexpr (VW == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float pj = p[j], vj = dv[j], mj = dm[j];
                const float gj = dw_checked<T>(e, r, c + j, sum[j]);
                optimiser_step<sizeof(T) == 2>(pj, vj, mj, gj * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt,
                                               e.regularisation, e.regu_coeff, true);
                p[j] = pj;
                dv[j] = vj;
                dm[j] = mj;
            }
            if (e.param) store4<T>(e.param, idx, p);
        } else {
            const float g = dw_checked<T>(e, r, c, sum);
            optimiser_step<sizeof(T) == 2>(p, dv, dm, g * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt,
                                           e.regularisation, e.regu_coeff, true);
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
// (cols_p a multiple of 8).  A wave owns a segment of PAD_U x 64 16-byte chunks
// of one padded row (grid-stride over rows x segments); lane l writes chunks
// l, l + 64, ... of the segment and issues all of its loads before any store.
// Every chunk of a source row starts O = (row's first element) mod 8 elements
// past a 16-byte boundary, so a chunk is cut out of the two aligned 16-byte
// source chunks covering it; O is one value per row, so pad_row<O> (picked by a
// wave-uniform switch) does the cut with fixed register selects and 16-bit
// funnel shifts.  A chunk whose aligned pair would leave the source's readable
// elements (a row's last partial chunk, the buffer's ends) is read element by
// element.
constexpr uint32_t PAD_U = 4;
template <int O>
__device__ __forceinline__ void pad_row(const half_t *__restrict__ in, uint64_t rb, int64_t ab, uint32_t cols,
                                        uint64_t in_elems, u32x4_t *orow, uint32_t g0, uint32_t gpr, uint32_t lane) {
    // ab: index of the aligned chunk holding element rb, relative to in (may be < 0)
    u32x4_t lo[PAD_U], hi[PAD_U];
    bool fast[PAD_U];
#pragma unroll
    for (uint32_t u = 0; u < PAD_U; ++u) {
        const uint32_t g = g0 + u * 64u + lane;
        const int64_t first = ab + 8ll * g;   // first element of the aligned pair, relative to in
        fast[u] = g < gpr && 8u * g + 8u <= cols && first >= 0 && (uint64_t)first + (O ? 16u : 8u) <= in_elems;
        if (fast[u]) {
            lo[u] = *reinterpret_cast<const u32x4_t *>(in + first);
            if constexpr (O != 0) hi[u] = *reinterpret_cast<const u32x4_t *>(in + first + 8);
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < PAD_U; ++u) {
        const uint32_t g = g0 + u * 64u + lane;
        if (g >= gpr) continue;
        u32x4_t v = {0, 0, 0, 0};
        const uint32_t c = 8u * g;
        if (fast[u]) {
            if constexpr (O == 0) {
                v = lo[u];
            } else {
                const uint32_t w[8] = {lo[u].x, lo[u].y, lo[u].z, lo[u].w, hi[u].x, hi[u].y, hi[u].z, hi[u].w};
                constexpr int WD = O / 2;            // whole dwords to skip
                constexpr uint32_t BITS = (O & 1) * 16u;
#pragma unroll
                for (int d = 0; d < 4; ++d) v[d] = __builtin_amdgcn_alignbit(w[d + WD + 1], w[d + WD], BITS);
            }
        } else if (c < cols) {
            half_t h[8];
            const half_t *src = in + rb + c;
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) h[e] = c + e < cols ? src[e] : (half_t)0;
            v = __builtin_bit_cast(u32x4_t, h);
        }
        orow[g] = v;
    }
}

__global__ void __launch_bounds__(256) pad_h_kernel(const half_t *__restrict__ in, uint32_t rows, uint32_t cols,
                                                    uint32_t ld, half_t *__restrict__ out, uint32_t rows_p,
                                                    uint32_t cols_p) {
    const uint32_t gpr = cols_p / 8;
    const uint32_t segs = (gpr + PAD_U * 64u - 1) / (PAD_U * 64u);
    const uint64_t in_elems = rows ? (uint64_t)(rows - 1) * ld + cols : 0;   // readable source elements
    const uint32_t lead = (uint32_t)((reinterpret_cast<uintptr_t>(in) / sizeof(half_t)) & 7u);
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t items = (uint64_t)rows_p * segs;
    for (uint64_t it = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6); it < items; it += (uint64_t)gridDim.x * 4u) {
        const uint32_t r = (uint32_t)(it / segs), g0 = (uint32_t)(it % segs) * PAD_U * 64u;
        u32x4_t *orow = reinterpret_cast<u32x4_t *>(out + (uint64_t)r * cols_p);
        if (r >= rows) {
#pragma unroll
            for (uint32_t u = 0; u < PAD_U; ++u) {
                const uint32_t g = g0 + u * 64u + lane;
                if (g < gpr) orow[g] = u32x4_t{0, 0, 0, 0};
            }
            continue;
        }
        const uint64_t rb = (uint64_t)r * ld;              // first source element of the row
        const uint32_t o = (uint32_t)((lead + rb) & 7u);   // its offset within an aligned chunk
        const int64_t ab = (int64_t)rb - o;
        switch (o) {
        case 0: pad_row<0>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 1: pad_row<1>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 2: pad_row<2>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 3: pad_row<3>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 4: pad_row<4>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 5: pad_row<5>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        case 6: pad_row<6>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        default: pad_row<7>(in, rb, ab, cols, in_elems, orow, g0, gpr, lane); break;
        }
    }
}

hipError_t launch_pad_h(const void *in, uint32_t rows, uint32_t cols, uint32_t ld, void *out, uint32_t rows_p,
                        uint32_t cols_p, hipStream_t s) {
    if (cols_p % 8 || rows_p < rows || cols_p < cols || !a16(out) || (reinterpret_cast<uintptr_t>(in) & 1u))
        return hipErrorInvalidValue;
    if (rows_p == 0 || cols_p == 0) return hipSuccess;
    const uint64_t segs = cdiv(cols_p / 8, PAD_U * 64u);
    const uint64_t waves = (uint64_t)rows_p * segs;
    const uint32_t blocks = cdiv(waves, 4) < 8192 ? cdiv(waves, 4) : 8192;   // 4 waves per block
    hipLaunchKernelGGL(pad_h_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const half_t *>(in), rows,
                       cols, ld, reinterpret_cast<half_t *>(out), rows_p, cols_p);
    return hipGetLastError();
}

}  // namespace skl
