/*
 * soklyn_hip.h — C ABI of the MI355X-native DenseBlock hot path.
 *
 * Drop-in boundary for Felix1G/soklyn's device layer: every entry point here
 * replaces one crate-internal GpuContext method of the reference (the
 * `pub(crate)` functions in src/io/device/ffn_device.rs and
 * src/io/device/util_device.rs) or the context constructor in
 * src/io/device.rs.  A Rust caller builds one `skl_dense_desc` per DenseBlock
 * from the device pointers its tensors own and calls these functions in the
 * order src/ffn.rs and src/mlp.rs already do.
 *
 * Conventions (mirroring the reference):
 *  - Row-major tensors.  W is [inputs x outputs] (src/mlp.rs:364), bias and
 *    norm parameters are [1 x outputs], caches are [max_batch x outputs].
 *  - T-typed tensors (weights, biases, norm params, caches, mask, rstd) are
 *    fp32 or fp16 per `dtype`; masters, moments and gradients are always fp32
 *    (src/cuda/nn_math.cu:123-127,150-156,195-205).
 *  - Mode codes are the reference's ordinals (src/util/function.rs:33-39,
 *    65-72, 104-116, 153-164; LossFunc as u32 at ffn_device.rs:157).
 *  - The caller owns every buffer; no entry point allocates a tensor.  The
 *    context keeps internal buffers (split-K partials, column partial sums,
 *    zero-padded copies of odd-width d_prenorm_h) that it grows on demand.
 *  - Return value: 0 = OK, < 0 = validation error (one code per reference
 *    Error variant, src/util/log.rs:15-99), > 0 = hipError_t.
 *  - Calls are synchronous (the reference synchronises after every launch,
 *    ffn_device.rs:75,110,136,189,228,355,436) unless skl_ctx_set_sync(ctx, 0)
 *    is called; then work is only ordered on the context's stream.  A call on a
 *    stream that is being captured into a HIP graph skips that synchronisation
 *    (it would end the capture); capturing also needs a caller-owned stream
 *    (skl_ctx_set_stream) and a call that grows none of the context's buffers
 *    (skl_dense_error_from_sum_noalloc, or buffers an earlier call of the same
 *    shapes already grew).
 *  - The context keeps padded copies of d_prenorm_h and column sums of
 *    d_prenorm between calls.  An error entry point on any context that
 *    rewrites those buffers makes them stale; a caller that rewrites d_prenorm,
 *    d_prenorm_h or dNorm with its own kernels between two calls must make one
 *    more entry-point call on the context in between (any call does).
 */
#ifndef SOKLYN_HIP_H
#define SOKLYN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------- */
#define SKL_OK                          0
#define SKL_ERR_INVALID_CONFIGURATION  (-1)   /* Error::InvalidConfiguration      */
#define SKL_ERR_TRAINING_MODE_REQUIRED (-2)   /* Error::TrainingModeRequired      */
#define SKL_ERR_ALLOCATION_LIMIT       (-3)   /* Error::AllocationLimitExceeded   */
#define SKL_ERR_MISMATCHED_DIMENSIONS  (-4)   /* Error::MismatchedDimensions      */
#define SKL_ERR_INVALID_BATCH_SIZE     (-5)   /* Error::InvalidBatchSize          */
#define SKL_ERR_HARDWARE_CONSTRAINT    (-6)   /* Error::HardwareConstraintViolation */
#define SKL_ERR_TRY_FROM_INT           (-7)   /* Error::TryFromIntError           */
#define SKL_ERR_NULL_POINTER           (-8)   /* a required device pointer is NULL */
#define SKL_ERR_UNSUPPORTED_CAST       (-9)   /* Error::UnsupportedTypeCast       */
#define SKL_ERR_NO_DEVICE             (-10)   /* no gfx950 device / bad ordinal   */

/* ---- mode codes (reference ordinals) --------------------------------------- */
enum { SKL_F32 = 0, SKL_F16 = 1 };                                   /* Precision */
enum { SKL_NORM_DISABLED = 0, SKL_NORM_RMS = 1, SKL_NORM_LAYER = 2, SKL_NORM_BATCH = 3 };
enum { SKL_ACT_IDENTITY = 0, SKL_ACT_SIGMOID = 1, SKL_ACT_RELU = 2, SKL_ACT_LEAKY_RELU = 3,
       SKL_ACT_TANH = 4, SKL_ACT_SOFTMAX = 5, SKL_ACT_SILU = 6, SKL_ACT_MISH = 7 };
enum { SKL_OPT_SGD = 0, SKL_OPT_ADAM = 1 };
enum { SKL_REGU_NONE = 0, SKL_REGU_L1 = 1, SKL_REGU_L2 = 2 };
enum { SKL_LOSS_MSE = 0, SKL_LOSS_CE = 1, SKL_LOSS_BCE = 2 };

typedef struct skl_ctx skl_ctx;

/*
 * One DenseBlock's device state (src/mlp.rs:265-288: ParamState x2,
 * ForwardCache, grads, mask).  Pointers the block's configuration does not
 * use may be NULL: masters for fp32 blocks; moments, grads and d_prenorm_h
 * when not training; prenorm/centered/norm_rstd when norm is Disabled;
 * d_norm_w/d_norm_b when norm is Disabled.
 */
typedef struct skl_dense_desc {
    uint32_t dtype;            /* SKL_F32 / SKL_F16: type T of the T tensors            */
    uint32_t inputs;           /* K = weight rows                                       */
    uint32_t outputs;          /* N = weight cols                                       */
    uint32_t max_batch;        /* M_max = cache rows                                    */
    uint32_t norm;             /* Normalisation ordinal                                 */
    uint32_t act;              /* Activation ordinal                                    */
    float    leaky;            /* LeakyReLU coeff                                       */
    float    mask_coeff;       /* dropout probability                                   */
    uint32_t regularisation;   /* Regularisation ordinal                                */
    float    regu_coeff;
    uint32_t is_training;
    uint32_t reserved0;
    /* parameters, T */
    void *w, *b, *norm_w, *norm_b;
    /* fp32 masters (fp16 blocks) */
    float *master_w, *master_b, *master_norm_w, *master_norm_b;
    /* fp32 optimiser moments */
    float *dv_w, *dv_b, *dm_w, *dm_b, *dv_norm_w, *dv_norm_b, *dm_norm_w, *dm_norm_b;
    /* forward caches, T; norm_rstd has max(max_batch, outputs) entries */
    void *out, *predrop, *preact, *centered, *prenorm, *norm_rstd, *mask;
    /* fp32 backward buffers [max_batch x outputs] */
    float *grad, *d_prenorm, *d_norm_w, *d_norm_b;
    /* fp16 blocks only: fp16 copy of d_prenorm [max_batch x outputs], the MFMA
     * operand of this block's dW GEMM and of the layer below's dX GEMM.  It
     * holds f16(d_prenorm), the rounding the reference applies when it feeds
     * d_prenorm to its fp16 dX kernel (backward_wmma.cu:44). */
    void *d_prenorm_h;
} skl_dense_desc;

typedef struct skl_optimiser {      /* Optimiser (function.rs:77-101), extracted as at ffn_device.rs:257-267 */
    uint32_t kind;                  /* SKL_OPT_SGD / SKL_OPT_ADAM                         */
    float    beta1;                 /* SGD v_coeff | Adam m_coeff                         */
    float    beta2;                 /* Adam v_coeff                                       */
    float    epsilon;               /* Adam epsilon                                       */
    uint32_t nesterov;              /* SGD nesterov                                       */
} skl_optimiser;

typedef struct skl_train_ctx {      /* TrainContext (context.rs:39-45)                    */
    skl_optimiser optimiser;        /* linear weights and bias                            */
    skl_optimiser norm_optimiser;   /* norm weight and bias                               */
    uint32_t batch_size;
    float    learn_rate;
    float    grad_clamp;            /* FLT_MAX disables clamping                          */
} skl_train_ctx;

/* ---- context (src/io/device.rs) -------------------------------------------- */
/* GpuContext::with_device_index (device.rs:180-183); GpuContext::new is ordinal 0
 * (device.rs:164-167).  tile_dim is validated like check_tile_dim (device.rs:248-258)
 * when fp16 work is launched; the MFMA kernels choose their own tiling. */
int32_t skl_ctx_create(int32_t ordinal, uint32_t tile_dim, skl_ctx **out);
int32_t skl_ctx_destroy(skl_ctx *ctx);
/* Synchronous (default 1, the reference's behaviour) or stream-ordered calls. */
int32_t skl_ctx_set_sync(skl_ctx *ctx, uint32_t sync_each_call);
/* Run on a caller-owned hipStream_t instead of the context's own (NULL = own). */
int32_t skl_ctx_set_stream(skl_ctx *ctx, void *hip_stream);
void   *skl_ctx_stream(skl_ctx *ctx);
int32_t skl_synchronize(skl_ctx *ctx);
/* Human-readable name of a status code. */
const char *skl_status_string(int32_t status);
/* Measurement aid, no counterpart in the reference: the GEMM kernel of the
 * next DenseBlock call that launches one records start_event and stop_event
 * (hipEvent_t, created by the caller) at its own start and end, through its
 * dispatch (no marker packets enter the stream); the GEMM alone, not the
 * operand staging, element-wise or reduction kernels around it.  The hook then
 * clears itself.  NULL, NULL clears it.  Not an entry-point call in the sense
 * of skl_dense_backward's column-sum reuse. */
int32_t skl_ctx_time_next_gemm(skl_ctx *ctx, void *start_event, void *stop_event);

/* ---- memory (replaces cudarc CudaSlice alloc/copy used by core.rs:557-692) -- */
int32_t skl_malloc(skl_ctx *ctx, void **ptr, size_t bytes);
int32_t skl_free(skl_ctx *ctx, void *ptr);
int32_t skl_memcpy_h2d(skl_ctx *ctx, void *dst, const void *src, size_t bytes);
int32_t skl_memcpy_d2h(skl_ctx *ctx, void *dst, const void *src, size_t bytes);
int32_t skl_memcpy_d2d(skl_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ---- utility kernels (util_device.rs) --------------------------------------- */
/* gpu_broadcast (util_device.rs:49-78): dst[0..n) = v in dtype */
int32_t skl_fill(skl_ctx *ctx, void *dst, uint32_t dtype, float v, size_t n);
/* gpu_cast_t (util_device.rs:7-47): f32 -> f16 (round to nearest even) or f16 -> f32;
 * any other pairing, same-type included, is SKL_ERR_UNSUPPORTED_CAST (util_device.rs:23-32) */
int32_t skl_cast(skl_ctx *ctx, const void *src, uint32_t src_dtype, void *dst, uint32_t dst_dtype,
                 size_t n);
/* scramble_seed (util/core.rs:90-94), host side, for the dropout seed */
uint32_t skl_scramble_seed(uint32_t step, uint32_t layer_id);

/* ---- DenseBlock hot path (ffn_device.rs) ------------------------------------ */
/* gpu_forward_pass (ffn_device.rs:12-139): Z = in.W (+b) -> norm -> act -> dropout.
 * in is [in_rows x in_cols] T with in_cols == inputs; the first `batch` rows are used. */
int32_t skl_dense_forward(skl_ctx *ctx, const skl_dense_desc *blk, const void *in,
                          uint32_t in_rows, uint32_t in_cols, uint32_t batch,
                          uint32_t use_dropout, uint32_t seed);

/* gpu_compute_output_layer_error (ffn_device.rs:141-231): zero dNorm, softmax
 * in place on out when act == Softmax, then the loss delta and the norm
 * gradient times LOSS_SCALE = 512 into grad / d_prenorm / dNorm. */
int32_t skl_dense_output_error(skl_ctx *ctx, const skl_dense_desc *blk, const void *target,
                               uint32_t target_rows, uint32_t target_cols,
                               uint32_t loss, uint32_t act, float leaky);

/* compute_hidden_layer_error_* (ffn_device.rs:369-436): s = next.d_prenorm .
 * next.W_master^T, then act'(s) * mask and the element-local norm gradient
 * into cur's grad / d_prenorm / dNorm.  Uses cur->act / cur->leaky. */
int32_t skl_dense_hidden_error(skl_ctx *ctx, const skl_dense_desc *cur, const skl_dense_desc *next,
                               uint32_t batch);

/* gpu_backward_pass (ffn_device.rs:233-358): dW = in^T . d_prenorm, db and
 * norm-parameter sums, scaled by 1/512 and 1/batch, then the optimiser step on
 * W (with regularisation), b (norm != BatchNorm), norm_w (norm > 0) and
 * norm_b (norm > 1); writes masters, moments and the T copies. */
int32_t skl_dense_backward(skl_ctx *ctx, const skl_dense_desc *blk, const void *in,
                           uint32_t in_rows, uint32_t in_cols, const skl_train_ctx *train,
                           uint32_t step);

/* gpu_hidden_layer_backward_pass (ffn_device.rs:360-439): hidden error of cur
 * from next, then gpu_backward_pass(cur). */
int32_t skl_dense_backward_hidden(skl_ctx *ctx, const skl_dense_desc *cur,
                                  const skl_dense_desc *next, const void *in, uint32_t in_rows,
                                  uint32_t in_cols, const skl_train_ctx *train, uint32_t step);

/* The epilogue of compute_hidden_layer_error (backward.cu:79-100) applied to a
 * caller-supplied upstream sum s [batch x outputs] fp32 (e.g. the gradient
 * arriving from a layer that is not a DenseBlock); zeroes dNorm first like
 * ffn_device.rs:370-371.  s already carries the loss scale. */
int32_t skl_dense_error_from_sum(skl_ctx *ctx, const skl_dense_desc *blk, const float *s,
                                 uint32_t batch);

/* skl_dense_error_from_sum that allocates nothing.  No counterpart in the
 * reference: for callers that cannot call hipMalloc (code under HIP graph
 * capture, on a caller-owned stream; tight serving loops; harnesses that forbid
 * allocation).  Same checks
 * and same outputs as skl_dense_error_from_sum, bit for bit; the error kernel's
 * column partial sums go to a 16 MiB device array the library holds per GPU
 * (looked up in skl_ctx_create) instead of the context's grown buffer.
 * Limit: partial rows x 3 x outputs x 4 bytes <= 16 MiB, which holds at any
 * batch for outputs below 466 K (outputs % 4 == 0), 233 K (outputs % 4 == 2)
 * or 116 K (odd outputs); otherwise SKL_ERR_ALLOCATION_LIMIT, nothing
 * written.  Every call on
 * one GPU shares that array: calls that overlap on one GPU (two streams or two
 * contexts) race.  It leaves no column sums behind, so a following
 * skl_dense_backward reads d_prenorm / dNorm again (same results). */
int32_t skl_dense_error_from_sum_noalloc(skl_ctx *ctx, const skl_dense_desc *blk, const float *s,
                                         uint32_t batch);

/* The GEMM of compute_hidden_layer_error (backward.cu:72-77) with no consumer
 * epilogue: dx[batch x inputs] fp32 = d_prenorm . W_master^T — the gradient sum
 * the layer below this block would receive (fp16 blocks: f16 operands, fp32
 * accumulation as backward_wmma.cu:39-63). */
int32_t skl_dense_input_grad(skl_ctx *ctx, const skl_dense_desc *blk, uint32_t batch, float *dx);

#ifdef __cplusplus
}
#endif
#endif /* SOKLYN_HIP_H */
