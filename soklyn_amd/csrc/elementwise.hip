// elementwise.hip — bandwidth-bound kernels of the DenseBlock hot path
// (gfx950, wave64): fill / cast, norm + activation + dropout, softmax, output
// error, hidden error from a given sum, column reductions + vector optimiser,
// split-K dW reduction + optimiser.
#include "launch.h"

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
    else if (sdt == 0 && ddt == 0)
        hipLaunchKernelGGL((cast_kernel<float, float>), grid_for(n, 256), dim3(256), 0, s, (const float *)src,
                           (float *)dst, (uint64_t)n);
    else
        hipLaunchKernelGGL((cast_kernel<half_t, half_t>), grid_for(n, 256), dim3(256), 0, s, (const half_t *)src,
                           (half_t *)dst, (uint64_t)n);
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

hipError_t launch_norm_act(const RowNormArgs &a, hipStream_t s) {
    if (a.m == 0 || a.n == 0) return hipSuccess;
    if (a.norm == 3) {
        if (a.dtype == 1)
            hipLaunchKernelGGL(norm_cols_kernel<half_t>, dim3(cdiv(a.n, 256)), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(norm_cols_kernel<float>, dim3(cdiv(a.n, 256)), dim3(256), 0, s, a);
    } else {
        if (a.dtype == 1)
            hipLaunchKernelGGL(norm_rows_kernel<half_t>, dim3(a.m), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(norm_rows_kernel<float>, dim3(a.m), dim3(256), 0, s, a);
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
template <typename T>
__device__ __forceinline__ void write_err(const ErrArgs &a, uint64_t idx, uint32_t row, uint32_t col, float e) {
    a.grad[idx] = e;
    float dp = e;
    if (a.norm) {
        const float rstd = to_f32(ldv<T>(a.norm_rstd, a.norm == 3 ? col : row));
        const float pv = a.norm == 1 ? to_f32(ldv<T>(a.prenorm, idx)) : 0.0f;
        const float cv = a.norm >= 2 ? to_f32(ldv<T>(a.centered, idx)) : 0.0f;
        const NormGrad g = norm_grad(a.norm, e, pv, cv, rstd, a.nw[col], a.inv_n, a.inv_m);
        dp = g.d_prenorm;
        a.d_norm_w[idx] = g.dnw;
        a.d_norm_b[idx] = g.dnb;
    }
    dp = dp * a.loss_scale;
    a.d_prenorm[idx] = dp;
    if (a.d_prenorm_h) a.d_prenorm_h[idx] = (half_t)dp;
}

// backward.cu:12-56
template <typename T> __global__ void output_error_kernel(ErrArgs a) {
    const uint64_t total = (uint64_t)a.rows * a.n;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t row = (uint32_t)(idx / a.n), col = (uint32_t)(idx % a.n);
        const float o = activation(a.act, to_f32(ldv<T>(a.out, idx)), a.leaky);
        const float t = to_f32(ldv<T>(a.target, idx));
        float e = 0.0f;
        if (a.loss == 0) {
            e = activation_derivative(a.act, o - t, o, to_f32(ldv<T>(a.preact, idx)), a.leaky);
        } else if ((a.loss == 1 && a.act == 5) || (a.loss == 2 && a.act == 1)) {
            e = o - t;
        }
        write_err<T>(a, idx, row, col, e);
    }
}

// backward.cu:79-100 with s supplied
template <typename T> __global__ void error_from_sum_kernel(ErrArgs a) {
    const uint64_t total = (uint64_t)a.rows * a.n;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t row = (uint32_t)(idx / a.n), col = (uint32_t)(idx % a.n);
        const float d = activation_derivative(a.act, a.s[idx], to_f32(ldv<T>(a.predrop, idx)),
                                              to_f32(ldv<T>(a.preact, idx)), a.leaky);
        write_err<T>(a, idx, row, col, to_f32(ldv<T>(a.mask, idx)) * d);
    }
}

// Vector forms: each thread owns 4 consecutive elements of one row (n % 4 == 0,
// 16-byte aligned buffers): 16-byte fp32 / 8-byte fp16 accesses, 32-bit indexing.
// The three values of one 4-column group that feed the column sums of backward.cu:187-194.
struct ErrSums4 {
    f32x4 dp, dnw, dnb;
};

template <typename T>
__device__ __forceinline__ ErrSums4 write_err4(const ErrArgs &a, uint64_t idx, uint32_t row, uint32_t col, f32x4 e) {
    __builtin_nontemporal_store(e, reinterpret_cast<f32x4 *>(a.grad + idx));
    ErrSums4 o;
    o.dp = e;
    o.dnw = o.dnb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (a.norm) {
        const f32x4 pv = a.norm == 1 ? load4<T>(a.prenorm, idx) : f32x4{0, 0, 0, 0};
        const f32x4 cv = a.norm >= 2 ? load4<T>(a.centered, idx) : f32x4{0, 0, 0, 0};
        const f32x4 nw = *reinterpret_cast<const f32x4 *>(a.nw + col);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float rstd = to_f32(ldv<T>(a.norm_rstd, a.norm == 3 ? col + j : row));
            const NormGrad g = norm_grad(a.norm, e[j], pv[j], cv[j], rstd, nw[j], a.inv_n, a.inv_m);
            o.dp[j] = g.d_prenorm;
            o.dnw[j] = g.dnw;
            o.dnb[j] = g.dnb;
        }
        *reinterpret_cast<f32x4 *>(a.d_norm_w + idx) = o.dnw;
        *reinterpret_cast<f32x4 *>(a.d_norm_b + idx) = o.dnb;
    }
    o.dp = o.dp * a.loss_scale;
    __builtin_nontemporal_store(o.dp, reinterpret_cast<f32x4 *>(a.d_prenorm + idx));
    if (a.d_prenorm_h) store4<half_t>(a.d_prenorm_h, idx, o.dp);
    return o;
}

// Loss delta of one 4-column group (backward.cu:24-45).
template <typename T> __device__ __forceinline__ f32x4 output_err4(const ErrArgs &a, uint64_t idx) {
    const f32x4 out = load4<T>(a.out, idx), tg = load4<T>(a.target, idx), pre = load4<T>(a.preact, idx);
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

// Error + column sums in one pass.  Workgroup (x, y) owns the columns
// [1024 UC x, 1024 UC (x + 1)) of the rows [y per, (y + 1) per): a thread owns
// UC 4-column groups 1024 apart, loads UR rows of all of them before computing
// any (UR x UC x 40 bytes in flight), writes grad / d_prenorm (/ dNorm) and
// adds d_prenorm, dNorm_w and dNorm_b into running column sums, rows in
// ascending order.  The sums go to partials[y][k][n] (k = 0 d_prenorm,
// 1 dNorm_w, 2 dNorm_b; 1 and 2 only with a norm), the inputs of the bias /
// norm-parameter update, so the backward does not read the three [rows x n]
// buffers again.
template <typename T, bool FROM_SUM, int UR, int UC>
__global__ void __launch_bounds__(256) error_cols_kernel(ErrArgs a, float *__restrict__ partials, uint32_t per) {
    const uint32_t cbase = blockIdx.x * (1024 * UC) + threadIdx.x * 4;
    if (cbase >= a.n) return;
    const uint32_t r0 = blockIdx.y * per;
    const uint32_t r1 = min(a.rows, r0 + per);
    f32x4 sdp[UC], snw[UC], snb[UC];
#pragma unroll
    for (int v = 0; v < UC; ++v) sdp[v] = snw[v] = snb[v] = f32x4{0, 0, 0, 0};
    for (uint32_t rb = r0; rb < r1; rb += UR) {
        f32x4 x0[UR][UC], x1[UR][UC], x2[UR][UC], x3[UR][UC];
        if constexpr (FROM_SUM) {
#pragma unroll
            for (int u = 0; u < UR; ++u) {
                if (rb + u >= r1) break;
#pragma unroll
                for (int v = 0; v < UC; ++v) {
                    const uint32_t c = cbase + 1024 * v;
                    if (c >= a.n) break;
                    const uint32_t idx = (rb + u) * a.n + c;
                    x0[u][v] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.s + idx));
                    x1[u][v] = load4<T>(a.predrop, idx);
                    x2[u][v] = load4<T>(a.preact, idx);
                    x3[u][v] = load4<T>(a.mask, idx);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UR; ++u) {
            const uint32_t row = rb + u;
            if (row >= r1) break;
#pragma unroll
            for (int v = 0; v < UC; ++v) {
                const uint32_t c = cbase + 1024 * v;
                if (c >= a.n) break;
                const uint32_t idx = row * a.n + c;
                f32x4 e;
                if constexpr (FROM_SUM) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        e[j] = x3[u][v][j] * activation_derivative(a.act, x0[u][v][j], x1[u][v][j], x2[u][v][j], a.leaky);
                } else {
                    e = output_err4<T>(a, idx);
                }
                const ErrSums4 o = write_err4<T>(a, idx, row, c, e);
                sdp[v] += o.dp;
                snw[v] += o.dnw;
                snb[v] += o.dnb;
            }
        }
    }
#pragma unroll
    for (int v = 0; v < UC; ++v) {
        const uint32_t c = cbase + 1024 * v;
        if (c >= a.n) break;
        float *p = partials + (uint64_t)blockIdx.y * 3 * a.n + c;
        *reinterpret_cast<f32x4 *>(p) = sdp[v];
        if (a.norm) {
            *reinterpret_cast<f32x4 *>(p + a.n) = snw[v];
            *reinterpret_cast<f32x4 *>(p + 2 * a.n) = snb[v];
        }
    }
}

static bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static bool err_vec_ok(const ErrArgs &a, bool from_sum) {
    if ((a.n & 3u) != 0 || (uint64_t)a.rows * a.n >= (1ull << 32)) return false;
    const void *ptrs[] = {a.grad, a.d_prenorm, a.d_prenorm_h, a.preact, a.norm ? a.nw : nullptr,
                          a.norm ? a.d_norm_w : nullptr, a.norm ? a.d_norm_b : nullptr,
                          a.norm == 1 ? a.prenorm : nullptr, a.norm >= 2 ? a.centered : nullptr,
                          from_sum ? a.s : a.out, from_sum ? a.predrop : a.target, from_sum ? a.mask : nullptr};
    for (const void *p : ptrs)
        if (p && !a16(p)) return false;
    return true;
}

// 4 rows x 1 column group per thread and ~1024 workgroups: of the shapes
// measured on the C3 step (UR x UC in {4x1, 2x2, 1x4, 2x4}, 512 to 2048
// workgroups) the fastest, both alone and between the GEMMs of the step.
constexpr int ERR_UR = 4, ERR_UC = 1;

// Row splits of the fused error + column-sum kernels: ~1024 workgroups.
uint32_t err_col_splits(uint32_t rows, uint32_t n) {
    const uint32_t col_blocks = cdiv(n, 1024 * ERR_UC);
    uint32_t sp = cdiv(1024, col_blocks);
    const uint32_t cap = cdiv(rows, 16);
    if (sp > cap) sp = cap;
    if (sp > 1024) sp = 1024;
    return sp < 1 ? 1 : sp;
}

template <bool FROM_SUM>
static hipError_t launch_error(const ErrArgs &a, float *partials, uint32_t splits, hipStream_t s) {
    const uint64_t total = (uint64_t)a.rows * a.n;
    if (total == 0) return hipSuccess;
    if (partials) {
        const uint32_t per = cdiv(a.rows, splits);
        const dim3 g(cdiv(a.n, 1024 * ERR_UC), splits);
        if (a.dtype == 1)
            hipLaunchKernelGGL((error_cols_kernel<half_t, FROM_SUM, ERR_UR, ERR_UC>), g, dim3(256), 0, s, a,
                               partials, per);
        else
            hipLaunchKernelGGL((error_cols_kernel<float, FROM_SUM, ERR_UR, ERR_UC>), g, dim3(256), 0, s, a,
                               partials, per);
    } else if (FROM_SUM) {
        if (a.dtype == 1)
            hipLaunchKernelGGL(error_from_sum_kernel<half_t>, grid_for(total, 256), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(error_from_sum_kernel<float>, grid_for(total, 256), dim3(256), 0, s, a);
    } else {
        if (a.dtype == 1)
            hipLaunchKernelGGL(output_error_kernel<half_t>, grid_for(total, 256), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(output_error_kernel<float>, grid_for(total, 256), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_output_error(const ErrArgs &a, float *partials, uint32_t splits, bool *sums, hipStream_t s) {
    *sums = partials && err_vec_ok(a, false);
    return launch_error<false>(a, *sums ? partials : nullptr, splits, s);
}

hipError_t launch_error_from_sum(const ErrArgs &a, float *partials, uint32_t splits, bool *sums, hipStream_t s) {
    *sums = partials && err_vec_ok(a, true);
    return launch_error<true>(a, *sums ? partials : nullptr, splits, s);
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

// 16 columns per workgroup, 16 lanes per column: lane j sums the partials of
// splits j, j+16, ... in order (four loads in flight per batch), then the 16
// are added in a fixed pairwise order.
template <typename T> __global__ void __launch_bounds__(256) vec_opt_kernel(VecOptArgs a) {
    __shared__ float red[3][16][17];
    const uint32_t cl = threadIdx.x & 15u, j = threadIdx.x >> 4;
    const uint32_t col = blockIdx.x * 16 + cl;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        float s = 0.0f;
        if (a.enabled[k] && col < a.n) {
            const float *p = a.partials + (uint64_t)k * a.n + col;
            const uint64_t st = (uint64_t)3 * a.n;   // between splits
            uint32_t sp = j;
            for (; sp + 48 < a.splits; sp += 64) {
                const float v0 = p[sp * st], v1 = p[(sp + 16) * st], v2 = p[(sp + 32) * st], v3 = p[(sp + 48) * st];
                s += v0;
                s += v1;
                s += v2;
                s += v3;
            }
            for (; sp < a.splits; sp += 16) s += p[sp * st];
        }
        red[k][j][cl] = s;
    }
    __syncthreads();
    if (j != 0 || col >= a.n) return;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (!a.enabled[k]) continue;
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = red[k][2 * i][cl] + red[k][2 * i + 1][cl];
        const float s = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
        float p = a.master[k][col], v = a.dv[k][col], mm = a.dm[k][col];
        optimiser_step(p, v, mm, s * kLossScaleInv, a.inv_m, a.lr, a.clamp, a.opt[k], 0, 0.0f, false);
        a.master[k][col] = p;
        a.dv[k][col] = v;
        a.dm[k][col] = mm;
        if (a.param[k]) stv<T>(a.param[k], col, from_f32<T>(p));
    }
}

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

hipError_t launch_vec_opt(const VecOptArgs &a, hipStream_t s) {
    if (a.n == 0) return hipSuccess;
    if (a.dtype == 1)
        hipLaunchKernelGGL(vec_opt_kernel<half_t>, dim3(cdiv(a.n, 16)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(vec_opt_kernel<float>, dim3(cdiv(a.n, 16)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---- split-K dW reduction + W optimiser ----------------------------------------------
template <typename T> __global__ void dw_reduce_opt_kernel(DwReduceArgs a) {
    const uint64_t total = (uint64_t)a.rows * a.n;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (uint32_t sp = 0; sp < a.splits; ++sp) s += a.partials[(uint64_t)sp * total + idx];
        const OptEpi &e = a.e;
        float p = e.master[idx], v = e.dv[idx], mm = e.dm[idx];
        optimiser_step(p, v, mm, s * kLossScaleInv, e.inv_m, e.lr, e.clamp, e.opt, e.regularisation, e.regu_coeff,
                       true);
        e.master[idx] = p;
        e.dv[idx] = v;
        e.dm[idx] = mm;
        if (e.param) stv<T>(e.param, idx, from_f32<T>(p));
    }
}

hipError_t launch_dw_reduce_opt(const DwReduceArgs &a, hipStream_t s) {
    const uint64_t total = (uint64_t)a.rows * a.n;
    if (total == 0) return hipSuccess;
    if (a.dtype == 1)
        hipLaunchKernelGGL(dw_reduce_opt_kernel<half_t>, grid_for(total, 256), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(dw_reduce_opt_kernel<float>, grid_for(total, 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---- fp16 transpose (64 x 64 LDS tiles) ---------------------------------------------------
// out[c][r] = in[r][c]; in is [rows x cols] (leading dim ld_in), out is [cols x rows]
// (leading dim ld_out).  Loads are 16-byte row chunks; stores are 16-byte column
// chunks gathered from LDS.  rows, cols, ld_in, ld_out are multiples of 8.
__global__ void __launch_bounds__(256) transpose_h_kernel(const half_t *__restrict__ in, half_t *__restrict__ out,
                                                          uint32_t rows, uint32_t cols, uint32_t ld_in,
                                                          uint32_t ld_out) {
    __shared__ half_t tile[64][64 + 8];
    const uint32_t r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t q = t + i * 256;              // 512 chunks of 8 halves
        const uint32_t r = q >> 3, c = (q & 7u) * 8;
        u32x4_t v = {0, 0, 0, 0};
        if (r0 + r < rows && c0 + c < cols)
            v = *reinterpret_cast<const u32x4_t *>(in + (uint64_t)(r0 + r) * ld_in + c0 + c);
        *reinterpret_cast<u32x4_t *>(&tile[r][c]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t q = t + i * 256;
        const uint32_t oc = q >> 3, orr = (q & 7u) * 8;   // out row = in col, out col = in row
        if (c0 + oc >= cols || r0 + orr >= rows) continue;
        half_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = tile[orr + e][oc];
        *reinterpret_cast<u32x4_t *>(out + (uint64_t)(c0 + oc) * ld_out + r0 + orr) = __builtin_bit_cast(u32x4_t, h);
    }
}

hipError_t launch_transpose_h(const void *in, void *out, uint32_t rows, uint32_t cols, uint32_t ld_in,
                              uint32_t ld_out, hipStream_t s) {
    if (rows == 0 || cols == 0) return hipSuccess;
    hipLaunchKernelGGL(transpose_h_kernel, dim3(cdiv(cols, 64), cdiv(rows, 64)), dim3(256), 0, s,
                       reinterpret_cast<const half_t *>(in), reinterpret_cast<half_t *>(out), rows, cols, ld_in,
                       ld_out);
    return hipGetLastError();
}

}  // namespace skl
