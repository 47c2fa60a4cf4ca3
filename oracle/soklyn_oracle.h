/*
 * soklyn_oracle.h — CPU restatement of the Soklyn DenseBlock hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path
 * is compared against (tests/, __graft_entry__.smoke(), bench.py's
 * cpu_baseline leg).  Nothing in the soklyn_amd product path links, loads or
 * calls it.
 *
 * Every function restates the reference algorithm at the cited file:line of
 * Felix1G/soklyn (paths relative to the reference repository root).  Tensors
 * are host float arrays, row-major.  A block in "half" mode stores every
 * T-typed tensor (weights, biases, norm params, forward caches, mask, rstd)
 * as float values that are exactly representable in IEEE binary16: the
 * oracle rounds with orc_round_f16 at every point where the reference stores
 * a T value, and keeps fp32 masters / moments / gradients in fp32, exactly as
 * the reference does for T = half.
 *
 * Pinning (see tests/test_oracle.py): f16 rounding against numpy float16;
 * GEMMs against numpy float64 matmul and brute force on tiny shapes;
 * activations / derivatives against float64 closed forms (and finite
 * differences for the smooth ones); softmax against its closed form and the
 * sum-to-one invariant; norm forward against float64 closed forms; the
 * optimisers against their closed forms at step 1; dropout hash and seed
 * scrambling against hand-computed known answers and the keep-rate
 * invariant.  The element-local norm backward (util.cu:175-215) is pinned
 * only by restatement plus its closed form on hand-picked values, because it
 * deliberately differs from the autograd gradient.
 */
#ifndef SOKLYN_ORACLE_H
#define SOKLYN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- precision helpers (util/type.rs:61-113; half 2.7.1 f16::from_f32 is RNE) ---- */
uint16_t orc_f32_to_f16_bits(float f);
float    orc_f16_bits_to_f32(uint16_t h);
float    orc_round_f16(float f);
void     orc_round_f16_array(float *x, size_t n);

/* ---- integer helpers ---- */
uint32_t orc_scramble_seed(uint32_t step, uint32_t layer_id);            /* util/core.rs:90-94 */
float    orc_dropout_u(uint32_t col, uint32_t row, uint32_t seed);       /* kernel/math.cuh:45-53 */

/* ---- element functions ---- */
float orc_activation(uint32_t act, float x, float leaky);                            /* util.cu:8-47 */
float orc_activation_derivative(uint32_t act, float err, float out_v, float in_x,
                                float leaky);                                        /* util.cu:49-93 */

typedef struct orc_block {
    int32_t  half;          /* 0: T = f32, 1: T = f16 (values rounded at T stores)      */
    uint32_t inputs;        /* K = weight rows                                           */
    uint32_t outputs;       /* N = weight cols                                           */
    uint32_t max_batch;     /* M_max (cache rows)                                        */
    uint32_t norm;          /* 0 Disabled, 1 RMS, 2 LN, 3 BN  (function.rs:65-72)         */
    uint32_t act;           /* 0 Id,1 Sig,2 ReLU,3 Leaky,4 Tanh,5 Softmax,6 SiLU,7 Mish   */
    float    leaky;
    float    mask_coeff;    /* dropout probability p                                     */
    uint32_t regularisation;/* 0 none, 1 L1, 2 L2                                        */
    float    regu_coeff;
    /* parameters (T) */
    float *w, *b, *norm_w, *norm_b;
    /* fp32 masters (half blocks only; NULL for f32 blocks) */
    float *master_w, *master_b, *master_norm_w, *master_norm_b;
    /* optimiser moments (fp32) */
    float *dv_w, *dv_b, *dm_w, *dm_b, *dv_norm_w, *dv_norm_b, *dm_norm_w, *dm_norm_b;
    /* forward caches (T), [max_batch x outputs]; rstd has max(max_batch, outputs) */
    float *out, *predrop, *preact, *centered, *prenorm, *norm_rstd, *mask;
    /* backward buffers (fp32), [max_batch x outputs] */
    float *grad, *d_prenorm, *d_norm_w, *d_norm_b;
} orc_block;

typedef struct orc_optimiser {
    uint32_t kind;       /* 0 SGD, 1 Adam (function.rs:104-116) */
    float beta1, beta2, epsilon;
    uint32_t nesterov;
} orc_optimiser;

typedef struct orc_train {
    orc_optimiser optimiser, norm_optimiser;
    uint32_t batch_size;
    float learn_rate, grad_clamp;
} orc_train;

/* forward.cu:8-161 + forward_wmma.cu:66-72 (fwd0 -> fwd1 -> fwd2) */
int orc_forward(orc_block *blk, const float *in, uint32_t m, uint32_t use_dropout, uint32_t seed);
/* util.cu:95-173, launched on rows = max_batch (ffn_device.rs:167-190) */
void orc_softmax(orc_block *blk);
/* ffn_device.rs:141-231 + backward.cu:12-56 (includes the dNorm zero fill and softmax) */
int orc_output_error(orc_block *blk, const float *target, uint32_t target_rows,
                     uint32_t loss, uint32_t act, float leaky);
/* ffn_device.rs:360-436 + backward.cu:59-102 (fp32 K-loop bound ec; Q15 rounding in half mode) */
int orc_hidden_error(orc_block *cur, const orc_block *next, uint32_t m);
/* backward.cu:79-100: the hidden-error epilogue applied to a caller-supplied upstream sum s */
int orc_error_from_sum(orc_block *cur, const float *s, uint32_t m);
/* backward.cu:72-77 alone: dx[m x K] = d_prenorm[m x N] . W_master^T (the sum a layer below would see) */
int orc_input_grad(const orc_block *blk, uint32_t m, float *dx);
/* backward.cu:105-234 + ffn_device.rs:233-358 */
int orc_backward(orc_block *blk, const float *in, const orc_train *tc, uint32_t step);
/* backward.cu:105-154, one element */
void orc_optimiser_update(float *param, float *master, float *dv, float *dm, size_t idx,
                          float grad_acc, float inv_m, float lr, float clamp,
                          const orc_optimiser *opt, uint32_t step,
                          uint32_t regularisation, float regu_coeff, int apply_regul, int half);

/* Plain fp32 GEMMs used by the CPU baseline leg; per-element k-ascending fma order. */
void orc_gemm_nn(const float *a, const float *b, float *c, uint32_t m, uint32_t k, uint32_t n);
int  orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
