// vec_opt.h — the bias / norm-parameter update of a DenseBlock (backward.cu:
// 105-154 on the column sums of d_prenorm, dNorm_w, dNorm_b): one workgroup of
// NT threads per a.cpb columns.  Run by vec_opt_kernel, inside the split-K dW
// reduction's launch, and after the fused dW + optimiser GEMM's epilogue.
#pragma once

#include "launch.h"

namespace skl {

// The gradient sum of W element (k, n): the sum over fp16 operands, or, where
// that is not finite on an fp16 block, the fp32 sum (OptEpi::dp32).
template <typename T> __device__ __forceinline__ float dw_checked(const OptEpi &e, uint32_t k, uint32_t n, float v) {
    if constexpr (sizeof(T) == 2) {
        if (__builtin_expect(!__builtin_isfinite(v), 0) && e.dp32)
            return dw_element_f32<T>(reinterpret_cast<const T *>(e.x), e.ldx, e.dp32, e.lddp, e.batch, k, n);
    }
    return v;
}

// a.cpb columns per workgroup (a power of 2), NT / cpb lanes per column: lane j
// sums the partials of splits j, j + lanes, ... in order (8 loads in flight), then
// the lanes of a column are added in a fixed tree (halving strides).  cpb comes
// from vec_opt_cpb: at most 16 splits per lane.
template <typename T, int NT = 256> __device__ __forceinline__ void vec_opt_block(const VecOptArgs &a, uint32_t block) {
    __shared__ float red[3][NT];
    const uint32_t cpb = a.cpb, lanes = (uint32_t)NT / cpb;
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
            if (sp < a.splits) {   // the last 1-7 rows of this lane in one batch of loads
                float v[7];
#pragma unroll
                for (int u = 0; u < 7; ++u) {
                    const uint32_t q = sp + u * lanes;
                    v[u] = p[(uint64_t)(q < a.splits ? q : a.splits - 1u) * st];
                }
#pragma unroll
                for (int u = 0; u < 7; ++u) s = sp + u * lanes < a.splits ? s + v[u] : s;
            }
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
        optimiser_step<sizeof(T) == 2>(p, v, mm, s * kLossScaleInv, a.inv_m, a.lr, a.clamp, a.opt[k], 0, 0.0f, false);
        a.master[k][col] = p;
        a.dv[k][col] = v;
        a.dm[k][col] = mm;
        if (a.param[k]) reinterpret_cast<T *>(a.param[k])[col] = from_f32<T>(p);
    }
}

}  // namespace skl
