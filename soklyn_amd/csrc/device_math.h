// device_math.h — element-level device functions of the DenseBlock hot path
// (gfx950).  Each restates the reference function cited beside it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace skl {

typedef _Float16 half_t;

// Element type of T tensors.
template <typename T> struct TypeTag;
template <> struct TypeTag<float> { static constexpr uint32_t code = 0; };
template <> struct TypeTag<half_t> { static constexpr uint32_t code = 1; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(half_t v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }  // RNE

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// 4 consecutive T elements <-> 4 floats (8-byte loads for fp16, 16-byte for fp32).
// The element index i must be a multiple of 4 and the base 16-byte aligned.
template <typename T> __device__ __forceinline__ f32x4 load4(const void *p, uint64_t i) {
    if constexpr (sizeof(T) == 2) {
        const f16x4 h = *reinterpret_cast<const f16x4 *>(reinterpret_cast<const half_t *>(p) + i);
        return f32x4{(float)h.x, (float)h.y, (float)h.z, (float)h.w};
    } else {
        return *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(p) + i);
    }
}
// store4 with the nontemporal hint: outputs written once and read by a later
// kernel, kept from displacing the GEMM's operand panels in L2.
template <typename T> __device__ __forceinline__ void store4_nt(void *p, uint64_t i, f32x4 v) {
    if constexpr (sizeof(T) == 2) {
        __builtin_nontemporal_store(f16x4{(half_t)v.x, (half_t)v.y, (half_t)v.z, (half_t)v.w},
                                    reinterpret_cast<f16x4 *>(reinterpret_cast<half_t *>(p) + i));
    } else {
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p) + i));
    }
}
template <typename T> __device__ __forceinline__ void store4(void *p, uint64_t i, f32x4 v) {
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<f16x4 *>(reinterpret_cast<half_t *>(p) + i) =
            f16x4{(half_t)v.x, (half_t)v.y, (half_t)v.z, (half_t)v.w};
    } else {
        *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p) + i) = v;
    }
}
// Round 4 floats through T (the value a T store followed by a load would give).
template <typename T> __device__ __forceinline__ f32x4 round4(f32x4 v) {
    if constexpr (sizeof(T) == 2) {
        return f32x4{(float)(half_t)v.x, (float)(half_t)v.y, (float)(half_t)v.z, (float)(half_t)v.w};
    } else {
        return v;
    }
}

constexpr float kLossScale = 512.0f;            // backward.cu:8
constexpr float kLossScaleInv = 1.0f / 512.0f;  // backward.cu:9

// 1 / (1 + e^-x) from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32):
// a few ulp, well inside every tolerance of this path; saturates to 0 / 1.
__device__ __forceinline__ float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// Mish for fp16 blocks (util.cu:28-39) and its derivative (util.cu:75-87) from
// one hardware exp and reciprocal per element: with u = e^x and n = u (u + 2),
// tanh(softplus(x)) = n / (n + 2) and 1 - tanh^2 = 4 (n + 1) / (n + 2)^2.  Above
// x = 20 the reference takes softplus = x, so tanh is 1 (the derivative 1) until
// e^x overflows, where its result is NaN; both kept here.  Elsewhere the two
// forms differ by a few fp32 ulp, except as x -> -inf, where the reference's
// e^sp - e^-sp cancels (relative error ~1e-7 / e^x): far below what an fp16
// result resolves.  fp32 blocks keep the reference's form.
constexpr float kExpOverflow = 88.72283935546875f;   // least float whose e^x rounds to +inf
__device__ __forceinline__ float mish_fast(float x) {
    const float u = __expf(x);
    const float n = u * (u + 2.0f);
    const float t = n * __builtin_amdgcn_rcpf(n + 2.0f);
    if (x > 20.0f) return x >= kExpOverflow ? __builtin_nanf("") : x;
    return x * t;
}
__device__ __forceinline__ float mish_slope_fast(float x) {
    const float u = __expf(x);
    const float n = u * (u + 2.0f);
    const float r = __builtin_amdgcn_rcpf(n + 2.0f);
    const float t = n * r;
    const float sech2 = (4.0f * (n + 1.0f)) * r * r;
    const float sig = u * __builtin_amdgcn_rcpf(1.0f + u);
    if (x > 20.0f) return x >= kExpOverflow ? __builtin_nanf("") : 1.0f;
    return t + x * sig * sech2;
}

// util.cu:8-47; T is the block's element type (selects the Mish form above).
template <typename T> __device__ __forceinline__ float activation(uint32_t act, float x, float leaky) {
    switch (act) {
    case 1: return sigmoid_fast(x);
    case 2: return fmaxf(0.0f, x);
    case 3: return x > 0.0f ? x : leaky * x;
    case 4: return tanhf(x);
    case 6: return x * sigmoid_fast(x);
    case 7: {
        if constexpr (sizeof(T) == 2) return mish_fast(x);
        const float e_x = expf(x);
        const float sp = x > 20.0f ? x : logf(1.0f + e_x);   // softplus with the reference cutoff
        const float e_sp = expf(sp);
        const float e_sp_inv = 1.0f / e_sp;
        return x * ((e_sp - e_sp_inv) / (e_sp + e_sp_inv));
    }
    default: return x;
    }
}

// util.cu:49-93 (ReLU / LeakyReLU test the post-activation value out_v)
template <typename T>
__device__ __forceinline__ float activation_derivative(uint32_t act, float err, float out_v, float in_x,
                                                       float leaky) {
    switch (act) {
    case 1: return err * (out_v * (1.0f - out_v));
    case 2: return err * (out_v > 0.0f ? 1.0f : 0.0f);
    case 3: return err * (out_v > 0.0f ? 1.0f : leaky);
    case 4: return err * (1.0f - out_v * out_v);
    case 6: {
        const float sig = sigmoid_fast(in_x);
        return err * (sig + out_v * (1.0f - sig));
    }
    case 7: {
        if constexpr (sizeof(T) == 2) return err * mish_slope_fast(in_x);
        const float e_x = expf(in_x);
        const float sp = in_x > 20.0f ? in_x : logf(1.0f + e_x);
        const float e_sp = expf(sp);
        const float e_sp_inv = 1.0f / e_sp;
        const float t = (e_sp - e_sp_inv) / (e_sp + e_sp_inv);
        const float sig = e_x / (1.0f + e_x);
        return err * (t + in_x * sig * (1.0f - t * t));
    }
    default: return err;
    }
}

// Which operands activation_derivative reads: the activation's output (out_v)
// or its input (in_x).
__host__ __device__ __forceinline__ bool act_uses_output(uint32_t act) { return (act >= 1 && act <= 4) || act == 6; }
__host__ __device__ __forceinline__ bool act_uses_input(uint32_t act) { return act == 6 || act == 7; }

// math.cuh:45-53.  The 64-bit product col * 6364136223846793005 keeps only its
// low 32 bits in the 32-bit state, i.e. col * 0x4C957F2D mod 2^32.  The state
// is (row * 1103515245) ^ (col * 0x4C957F2D) ^ seed: dropout_bits takes the
// column product and the row key (row * 1103515245) ^ seed separately, so a
// thread walking consecutive columns adds the constant instead of multiplying.
constexpr uint32_t kDropColMul = 0x4C957F2Du;
__host__ __device__ __forceinline__ uint32_t dropout_rowkey(uint32_t row, uint32_t seed) {
    return (row * 1103515245u) ^ seed;
}
__host__ __device__ __forceinline__ uint32_t dropout_bits(uint32_t colmul, uint32_t rowkey) {
    uint32_t s = rowkey ^ colmul;
    s = s ^ (s >> 17);
    s = s * 1103515245u + 12345u;
    return s ^ (s >> 15);
}
__device__ __forceinline__ float dropout_u(uint32_t col, uint32_t row, uint32_t seed) {
    return (float)dropout_bits(col * kDropColMul, dropout_rowkey(row, seed)) / 4294967296.0f;
}
// The keep test dropout_u(...) >= p as an integer compare, bits >= keep_min:
// (float)s is monotone in s, so {s : (float)s / 2^32 >= p} is [keep_min, 2^32)
// (keep_min = 2^32: never, e.g. p NaN).  Host-side, by bisection with the same
// round-to-nearest-even u32 -> f32 conversion the device's v_cvt_f32_u32 does.
inline uint64_t dropout_keep_min(float p) {
    uint64_t lo = 0, hi = 1ull << 32;   // answer in [lo, hi]
    while (lo < hi) {
        const uint64_t mid = lo + (hi - lo) / 2;
        if ((float)(uint32_t)mid / 4294967296.0f >= p)
            hi = mid;
        else
            lo = mid + 1;
    }
    return lo;
}

// util.cu:175-215 — element-local norm gradient.
struct NormGrad {
    float d_prenorm, dnw, dnb;
};
__device__ __forceinline__ NormGrad norm_grad(uint32_t norm, float e, float prenorm_v, float centered_v,
                                              float rstd, float nw, float inv_n, float inv_m) {
    NormGrad g{e, 0.0f, 0.0f};
    if (norm == 1) {
        g.dnw = e * prenorm_v * rstd;
        g.d_prenorm = nw * rstd * (e - rstd * rstd * prenorm_v * prenorm_v * inv_n);
    } else if (norm == 2) {
        g.dnb = e;
        g.dnw = e * centered_v * rstd;
        g.d_prenorm = nw * rstd * (e - e * inv_n - rstd * rstd * centered_v * centered_v * e * inv_n);
    } else if (norm == 3) {
        g.dnb = e;
        g.dnw = e * centered_v * rstd;
        g.d_prenorm = nw * rstd * (e - e * inv_m - rstd * rstd * centered_v * centered_v * e * inv_m);
    }
    return g;
}

// dW of element (k, n) summed over the batch rows in fp32 from the fp32
// d_prenorm, in the reference's order (backward.cu:181-186: sequential rows,
// x converted to f32, one fused multiply-add per row).
template <typename T>
__device__ __attribute__((noinline)) float dw_element_f32(const T *x, uint32_t ldx, const float *dp, uint32_t lddp,
                                                           uint32_t batch, uint32_t k, uint32_t n) {
    float s = 0.0f;
    for (uint32_t b = 0; b < batch; ++b) s = fmaf((float)x[(uint64_t)b * ldx + k], dp[(uint64_t)b * lddp + n], s);
    return s;
}

// Optimiser hyper-parameters as the update kernels consume them
// (backward.cu:105-154; bias corrections precomputed per call).
struct OptParams {
    uint32_t kind;      // 0 SGD, 1 Adam
    float beta1, beta2, epsilon;
    uint32_t nesterov;
    float bc1, bc2;     // 1 - beta1^step, 1 - beta2^step (Adam)
};

// backward.cu:105-154, one element.  p, v, m are the fp32 master and moments
// (in/out); grad_acc is the raw accumulated gradient, already / LOSS_SCALE.
// FAST (fp16 blocks): Adam's bias corrections and step with the hardware
// reciprocal and square root (v_rcp_f32, v_sqrt_f32, ~1 ulp each), which moves
// the update by a few fp32 ulp and took C3's dW + Adam 0.288 -> 0.283 ms; fp32
// blocks keep the reference's IEEE quotients and sqrtf (it is built without
// fast math) so their masters follow it to the last bit the formula allows.
template <bool FAST>
__device__ __forceinline__ void optimiser_step(float &p, float &v, float &mm, float grad_acc, float inv_m,
                                               float lr, float clamp, const OptParams &o,
                                               uint32_t regularisation, float regu_coeff, bool apply_regul) {
    // no fused multiply-adds: every kernel that applies the step (the fused dW
    // epilogue, the split-K reduction, the parameter update) rounds it alike
#pragma clang fp contract(off)
    const float val = grad_acc * inv_m;
    if (apply_regul) {
        const float sign = p > 0.0f ? 1.0f : (p < 0.0f ? -1.0f : 0.0f);  // math.cuh:60-66 on master
        if (regularisation == 1) p -= regu_coeff * sign;
        if (regularisation == 2) p -= 2.0f * regu_coeff * p;
    }
    if (o.kind == 0) {
        const float dl = o.beta1 * v + val;
        v = dl;
        float u = lr * (o.nesterov ? val + o.beta1 * dl : dl);
        u = fminf(fmaxf(u, -clamp), clamp);
        p -= u;
    } else if (o.kind == 1) {
        const float dml = o.beta1 * mm + (1.0f - o.beta1) * val;
        const float dvl = o.beta2 * v + (1.0f - o.beta2) * val * val;
        mm = dml;
        v = dvl;
        float u;
        if constexpr (FAST) {
            const float mc = dml * __builtin_amdgcn_rcpf(o.bc1);
            const float vc = dvl * __builtin_amdgcn_rcpf(o.bc2);
            u = lr * (mc * __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(vc) + o.epsilon));
        } else {
            const float mc = dml / o.bc1;
            const float vc = dvl / o.bc2;
            u = lr * (mc / (sqrtf(vc) + o.epsilon));
        }
        u = fminf(fmaxf(u, -clamp), clamp);
        p -= u;
    }
}

}  // namespace skl
