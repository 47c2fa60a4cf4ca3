/*
 * soklyn_oracle.c — CPU restatement of the Soklyn DenseBlock hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path (tests/, smoke(),
 * bench.py cpu_baseline).  The product (soklyn_amd) never links or calls it.
 *
 * Reference file:line citations are relative to the Felix1G/soklyn root.
 * Accumulations run in the reference's order (k / batch ascending, fused
 * multiply-add as nvcc contracts `sum += a * b`), parallelised only across
 * independent output elements, so results do not depend on thread count.
 * Everything else is compiled with -ffp-contract=off so each C expression
 * rounds where its source expression does.
 *
 * Parity notes:
 *  - CUDA expf/logf/tanhf/powf/rsqrtf are replaced by C libm (expf, logf,
 *    tanhf, powf) and 1/sqrtf; the two differ by a few ulp, which every
 *    tolerance absorbs.
 *  - Reductions that the reference does as block tree sums (norm statistics,
 *    softmax) are sequential here; same values up to fp32 rounding.
 *  - The fp16 hidden-error WMMA kernel's K-loop bound (backward_wmma.cu:39,
 *    runs ceil(n/16) tiles instead of ceil(ec/16)) is NOT reproduced: the
 *    oracle follows the fp32 kernel's `k < ec` (backward.cu:75) for both
 *    precisions, as fp16 is judged against the fp32 semantics.
 */
#include "soklyn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LOSS_SCALE 512.0f                 /* backward.cu:8 */
#define LOSS_SCALE_INV (1.0f / 512.0f)    /* backward.cu:9 */

/* ------------------------------------------------------------------------ */
/* binary16 conversion, round-to-nearest-even (half::f16::from_f32,
 * cuda_fp16 __float2half_rn) — util/type.rs:98-104                          */
/* ------------------------------------------------------------------------ */
static uint32_t rne_shift(uint32_t v, int shift)
{
    if (shift <= 0) return v;
    if (shift >= 32) return 0;
    uint32_t q = v >> shift;
    uint32_t rem = v & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) q++;
    return q;
}

uint16_t orc_f32_to_f16_bits(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (exp == 0) return (uint16_t)sign; /* fp32 zero/subnormal -> signed zero */
        /* value = (mant|2^23) * 2^(exp-150); half subnormal unit is 2^-24 */
        uint32_t q = rne_shift(mant | 0x800000u, 14 - e);
        return (uint16_t)(sign | q);
    }
    uint32_t bits = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (bits & 1u))) bits++;
    return (uint16_t)(sign | bits);
}

float orc_f16_bits_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        float v = ldexpf((float)mant, -24);
        return sign ? -v : v;
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

float orc_round_f16(float f) { return orc_f16_bits_to_f32(orc_f32_to_f16_bits(f)); }

void orc_round_f16_array(float *x, size_t n)
{
    for (size_t i = 0; i < n; i++) x[i] = orc_round_f16(x[i]);
}

static inline float T(int half, float v) { return half ? orc_round_f16(v) : v; }

/* ------------------------------------------------------------------------ */
/* integer helpers                                                            */
/* ------------------------------------------------------------------------ */
/* util/core.rs:90-94 */
uint32_t orc_scramble_seed(uint32_t step, uint32_t layer_id)
{
    uint32_t h = step * 1103515245u + layer_id;
    h = (h ^ (h >> 16)) * 1103515245u;
    return h ^ (h >> 15);
}

/* kernel/math.cuh:45-53.  `col * 6364136223846793005U` is a 64-bit product
 * whose low 32 bits survive the assignment to the 32-bit state. */
float orc_dropout_u(uint32_t col, uint32_t row, uint32_t seed)
{
    uint32_t state = (row * 1103515245u) ^ (uint32_t)((uint64_t)col * 6364136223846793005ull) ^ seed;
    state = state ^ (state >> 17);
    state = state * 1103515245u + 12345u;
    state = state ^ (state >> 15);
    return (float)state / (float)0xFFFFFFFFu;
}

/* ------------------------------------------------------------------------ */
/* activations                                                                */
/* ------------------------------------------------------------------------ */
/* util.cu:8-47 */
float orc_activation(uint32_t act, float x, float leaky)
{
    switch (act) {
    case 1: return 1.0f / (1.0f + expf(-x));
    case 2: return fmaxf(0.0f, x);
    case 3: return x > 0.0f ? x : leaky * x;
    case 4: return tanhf(x);
    case 6: return x / (1.0f + expf(-x));
    case 7: {
        float e_x = expf(x);
        float sp = x > 20.0f ? x : logf(1.0f + e_x);
        float e_sp = expf(sp);
        float e_sp_inv = 1.0f / e_sp;
        float t = (e_sp - e_sp_inv) / (e_sp + e_sp_inv);
        return x * t;
    }
    default: return x;
    }
}

/* util.cu:49-93.  ReLU / LeakyReLU test the post-activation value. */
float orc_activation_derivative(uint32_t act, float err, float out_v, float in_x, float leaky)
{
    switch (act) {
    case 1: return err * (out_v * (1.0f - out_v));
    case 2: return err * (out_v > 0.0f ? 1.0f : 0.0f);
    case 3: return err * (out_v > 0.0f ? 1.0f : leaky);
    case 4: return err * (1.0f - out_v * out_v);
    case 6: {
        float sig = 1.0f / (1.0f + expf(-in_x));
        return err * (sig + out_v * (1.0f - sig));
    }
    case 7: {
        float e_x = expf(in_x);
        float sp = in_x > 20.0f ? in_x : logf(1.0f + e_x);
        float e_sp = expf(sp);
        float e_sp_inv = 1.0f / e_sp;
        float t = (e_sp - e_sp_inv) / (e_sp + e_sp_inv);
        float sig = e_x / (1.0f + e_x);
        float sech2 = 1.0f - t * t;
        return err * (t + in_x * sig * sech2);
    }
    default: return err;
    }
}

/* ------------------------------------------------------------------------ */
/* GEMM helpers (fp32, per-element k-ascending fma)                           */
/* ------------------------------------------------------------------------ */
/* c[m x n] = a[m x k] . b[k x n]; the order math.cu:21-47 accumulates in. */
void orc_gemm_nn(const float *a, const float *b, float *c, uint32_t m, uint32_t k, uint32_t n)
{
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++) {
        float *crow = c + (size_t)r * n;
        for (uint32_t j = 0; j < n; j++) crow[j] = 0.0f;
        for (uint32_t kk = 0; kk < k; kk++) {
            const float av = a[(size_t)r * k + kk];
            const float *brow = b + (size_t)kk * n;
            for (uint32_t j = 0; j < n; j++) crow[j] = fmaf(av, brow[j], crow[j]);
        }
    }
}

int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static float *transpose_alloc(const float *src, uint32_t rows, uint32_t cols, int round_half)
{
    float *t = (float *)malloc((size_t)rows * cols * sizeof(float));
    if (!t) return NULL;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; r++)
        for (uint32_t c = 0; c < cols; c++) {
            float v = src[(size_t)r * cols + c];
            t[(size_t)c * rows + r] = round_half ? orc_round_f16(v) : v;
        }
    return t;
}

/* ------------------------------------------------------------------------ */
/* forward                                                                    */
/* ------------------------------------------------------------------------ */
int orc_forward(orc_block *B, const float *in, uint32_t m, uint32_t use_dropout, uint32_t seed)
{
    const uint32_t K = B->inputs, N = B->outputs;
    const int H = B->half;
    if (m == 0 || m > B->max_batch) return -1;
    float *Z = B->norm == 0 ? B->preact : B->prenorm;   /* ffn_device.rs:51-55 */
    const int use_bias = B->norm != 3;                  /* ffn_device.rs:30 */

    /* fwd0: forward.cu:8-28 (f32) / forward_wmma.cu:66-72 (f16: f32 acc + f32(b), one rounding) */
    orc_gemm_nn(in, B->w, Z, m, K, N);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++)
        for (uint32_t c = 0; c < N; c++) {
            float v = Z[(size_t)r * N + c];
            if (use_bias) v = v + B->b[c];
            Z[(size_t)r * N + c] = T(H, v);
        }

    /* fwd1: forward.cu:31-127 */
    if (B->norm == 1) {
#pragma omp parallel for schedule(static)
        for (long r = 0; r < (long)m; r++) {
            const float *z = Z + (size_t)r * N;
            float sq = 0.0f;
            for (uint32_t c = 0; c < N; c++) sq = fmaf(z[c], z[c], sq);
            const float var = sq / (float)N + 1e-6f;
            const float rstd32 = 1.0f / sqrtf(var);
            const float rstd = T(H, rstd32);
            B->norm_rstd[r] = rstd;
            for (uint32_t c = 0; c < N; c++) {
                size_t idx = (size_t)r * N + c;
                B->centered[idx] = z[c];
                /* T arithmetic: (prenorm * rstd) * norm_w, each product rounded in T */
                B->preact[idx] = T(H, T(H, z[c] * rstd) * B->norm_w[c]);
            }
        }
    } else if (B->norm == 2 || B->norm == 3) {
        const int ln = B->norm == 2;
        const uint32_t groups = ln ? m : N;   /* one block per row (LN) or column (BN) */
        const uint32_t n = ln ? N : m;
#pragma omp parallel for schedule(static)
        for (long g = 0; g < (long)groups; g++) {
#define NIDX(i) (ln ? (size_t)g * N + (i) : (size_t)(i) * N + (size_t)g)
            float s = 0.0f;
            for (uint32_t i = 0; i < n; i++) s += Z[NIDX(i)];
            const float mean = s / (float)n;
            float ss = 0.0f;
            for (uint32_t i = 0; i < n; i++) {
                float v = Z[NIDX(i)] - mean;
                ss = fmaf(v, v, ss);
            }
            const float var = ss / (float)n + 1e-6f;
            const float rstd32 = 1.0f / sqrtf(var);
            B->norm_rstd[g] = T(H, rstd32);
            for (uint32_t i = 0; i < n; i++) {
                size_t idx = NIDX(i);
                uint32_t col = ln ? i : (uint32_t)g;
                float v = Z[idx] - mean;
                B->centered[idx] = T(H, v);
                B->preact[idx] = T(H, fmaf(v * rstd32, B->norm_w[col], B->norm_b[col]));
            }
#undef NIDX
        }
    }

    /* fwd2: forward.cu:130-161 */
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++)
        for (uint32_t c = 0; c < N; c++) {
            size_t idx = (size_t)r * N + c;
            float a = orc_activation(B->act, B->preact[idx], B->leaky);
            B->predrop[idx] = T(H, a);
            if (use_dropout) {
                if (orc_dropout_u(c, (uint32_t)r, seed + (uint32_t)r * 7u) >= B->mask_coeff) {
                    const float scale = 1.0f / (1.0f - B->mask_coeff);
                    B->mask[idx] = T(H, scale);
                    B->out[idx] = T(H, a * scale);
                } else {
                    B->mask[idx] = 0.0f;
                    B->out[idx] = 0.0f;
                }
            } else {
                B->out[idx] = T(H, a);
            }
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* softmax: util.cu:95-173, over rows = max_batch (ffn_device.rs:167-186)     */
/* ------------------------------------------------------------------------ */
void orc_softmax(orc_block *B)
{
    const uint32_t N = B->outputs;
    for (uint32_t r = 0; r < B->max_batch; r++) {
        float *o = B->out + (size_t)r * N;
        float mx = -INFINITY;
        for (uint32_t c = 0; c < N; c++) mx = fmaxf(mx, o[c]);
        float s = 0.0f;
        for (uint32_t c = 0; c < N; c++) s += expf(o[c] - mx);
        for (uint32_t c = 0; c < N; c++) o[c] = T(B->half, expf(o[c] - mx) / s);
    }
}

/* util.cu:175-215 — element-local norm gradient (no row sums; RMS second term
 * has no err factor).  Restated as written. */
static void write_norm_grad(orc_block *B, size_t idx, float rstd, float e, float nw,
                            float loss_scale, float inv_n, float inv_m)
{
    float dnw = 0.0f, dnb = 0.0f, dp = e;
    if (B->norm == 1) {
        const float p = B->prenorm[idx];
        dnw = e * p * rstd;
        dp = nw * rstd * (e - rstd * rstd * p * p * inv_n);
    } else if (B->norm == 2) {
        const float cv = B->centered[idx];
        dnb = e;
        dnw = e * cv * rstd;
        dp = nw * rstd * (e - e * inv_n - rstd * rstd * cv * cv * e * inv_n);
    } else if (B->norm == 3) {
        const float cv = B->centered[idx];
        dnb = e;
        dnw = e * cv * rstd;
        dp = nw * rstd * (e - e * inv_m - rstd * rstd * cv * cv * e * inv_m);
    }
    B->d_prenorm[idx] = dp * loss_scale;
    B->d_norm_w[idx] = dnw;
    B->d_norm_b[idx] = dnb;
}

static const float *master_or(const float *master, const float *fallback)
{
    return master ? master : fallback;   /* device.rs:262-272 */
}

/* ------------------------------------------------------------------------ */
/* output-layer error: ffn_device.rs:141-231, backward.cu:12-56               */
/* ------------------------------------------------------------------------ */
int orc_output_error(orc_block *B, const float *target, uint32_t target_rows,
                     uint32_t loss, uint32_t act, float leaky)
{
    const uint32_t N = B->outputs;
    const size_t all = (size_t)B->max_batch * N;
    memset(B->d_norm_w, 0, all * sizeof(float));   /* ffn_device.rs:148-149 */
    memset(B->d_norm_b, 0, all * sizeof(float));
    if (act == 5) orc_softmax(B);
    /* kernel m = out.rows() = max_batch (ffn_device.rs:152); rows past the
     * target's would read outside it in the reference, so they are skipped. */
    const uint32_t rows = target_rows < B->max_batch ? target_rows : B->max_batch;
    const float inv_m = 1.0f / (float)B->max_batch;
    const float inv_n = 1.0f / (float)N;
    const float *nw = master_or(B->master_norm_w, B->norm_w);
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t c = 0; c < N; c++) {
            size_t idx = (size_t)r * N + c;
            float o = orc_activation(act, B->out[idx], leaky);
            float t = target[idx];
            float e = 0.0f;
            if (loss == 0) {
                e = o - t;
                e = orc_activation_derivative(act, e, o, B->preact[idx], leaky);
            } else if ((loss == 1 && act == 5) || (loss == 2 && act == 1)) {
                e = o - t;
            }
            B->grad[idx] = e;
            const float rstd = B->norm_rstd[B->norm == 3 ? c : r];
            write_norm_grad(B, idx, rstd, e, nw[c], LOSS_SCALE, inv_n, inv_m);
        }
    return 0;
}

/* hidden-error epilogue: backward.cu:79-100 */
static void hidden_epilogue(orc_block *cur, const float *s, uint32_t m)
{
    const uint32_t n = cur->outputs;
    const float inv_m = 1.0f / (float)m, inv_n = 1.0f / (float)n;
    const float *nw = master_or(cur->master_norm_w, cur->norm_w);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++)
        for (uint32_t c = 0; c < n; c++) {
            size_t idx = (size_t)r * n + c;
            float d = orc_activation_derivative(cur->act, s[idx], cur->predrop[idx],
                                                cur->preact[idx], cur->leaky);
            float e = cur->mask[idx] * d;
            cur->grad[idx] = e;
            const float rstd = cur->norm_rstd[cur->norm == 3 ? c : (uint32_t)r];
            write_norm_grad(cur, idx, rstd, e, nw[c], 1.0f, inv_n, inv_m);
        }
}

/* s[m x rows_w] = dp[m x cols_w] . Wm[rows_w x cols_w]^T, k ascending
 * (backward.cu:72-77); half mode rounds both operands to f16 first
 * (backward_wmma.cu:44,51). */
static float *dp_times_wT(const float *dp, const float *wm, uint32_t m, uint32_t rows_w,
                          uint32_t cols_w, int half)
{
    float *wt = transpose_alloc(wm, rows_w, cols_w, half);   /* [cols_w x rows_w] */
    float *s = (float *)malloc((size_t)m * rows_w * sizeof(float));
    if (!wt || !s) { free(wt); free(s); return NULL; }
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++) {
        float *srow = s + (size_t)r * rows_w;
        for (uint32_t j = 0; j < rows_w; j++) srow[j] = 0.0f;
        for (uint32_t k = 0; k < cols_w; k++) {
            float a = dp[(size_t)r * cols_w + k];
            if (half) a = orc_round_f16(a);
            const float *wrow = wt + (size_t)k * rows_w;
            for (uint32_t j = 0; j < rows_w; j++) srow[j] = fmaf(a, wrow[j], srow[j]);
        }
    }
    free(wt);
    return s;
}

/* ffn_device.rs:360-436 */
int orc_hidden_error(orc_block *cur, const orc_block *next, uint32_t m)
{
    const uint32_t n = cur->outputs, ec = next->outputs;
    if (next->inputs != n || m == 0 || m > cur->max_batch) return -1;
    const size_t all = (size_t)cur->max_batch * n;
    memset(cur->d_norm_w, 0, all * sizeof(float));   /* ffn_device.rs:370-371 */
    memset(cur->d_norm_b, 0, all * sizeof(float));
    const float *wm = master_or(next->master_w, next->w);
    float *s = dp_times_wT(next->d_prenorm, wm, m, n, ec, cur->half);
    if (!s) return -2;
    hidden_epilogue(cur, s, m);
    free(s);
    return 0;
}

int orc_error_from_sum(orc_block *cur, const float *s, uint32_t m)
{
    if (m == 0 || m > cur->max_batch) return -1;
    const size_t all = (size_t)cur->max_batch * cur->outputs;
    memset(cur->d_norm_w, 0, all * sizeof(float));
    memset(cur->d_norm_b, 0, all * sizeof(float));
    hidden_epilogue(cur, s, m);
    return 0;
}

int orc_input_grad(const orc_block *B, uint32_t m, float *dx)
{
    const float *wm = master_or(B->master_w, B->w);
    float *s = dp_times_wT(B->d_prenorm, wm, m, B->inputs, B->outputs, B->half);
    if (!s) return -2;
    memcpy(dx, s, (size_t)m * B->inputs * sizeof(float));
    free(s);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* optimiser: backward.cu:105-154                                             */
/* ------------------------------------------------------------------------ */
void orc_optimiser_update(float *param, float *master, float *dv, float *dm, size_t idx,
                          float grad_acc, float inv_m, float lr, float clamp,
                          const orc_optimiser *opt, uint32_t step,
                          uint32_t regularisation, float regu_coeff, int apply_regul, int half)
{
    float p = master[idx];
    float v = dv[idx];
    float mm = dm[idx];
    const float val = grad_acc * inv_m;
    if (apply_regul) {
        const float x = master[idx];
        const float sign = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);   /* math.cuh:60-66 */
        if (regularisation == 1) p -= regu_coeff * sign;
        if (regularisation == 2) p -= 2.0f * regu_coeff * p;
    }
    if (opt->kind == 0) {
        const float dl = opt->beta1 * v + val;
        v = dl;
        float u = lr * (opt->nesterov ? val + opt->beta1 * dl : dl);
        u = fminf(fmaxf(u, -clamp), clamp);
        p -= u;
    } else if (opt->kind == 1) {
        const float b1 = opt->beta1, b2 = opt->beta2;
        const float dml = b1 * mm + (1.0f - b1) * val;
        const float dvl = b2 * v + (1.0f - b2) * val * val;
        mm = dml;
        v = dvl;
        const float mc = dml / (1.0f - powf(b1, (float)step));
        const float vc = dvl / (1.0f - powf(b2, (float)step));
        const float denom = sqrtf(vc) + opt->epsilon;
        float u = lr * (mc / denom);
        u = fminf(fmaxf(u, -clamp), clamp);
        p -= u;
    }
    master[idx] = p;
    param[idx] = T(half, p);
    dv[idx] = v;
    dm[idx] = mm;
}

/* ------------------------------------------------------------------------ */
/* dW / db / norm-param reduction + update: backward.cu:157-234               */
/* ------------------------------------------------------------------------ */
int orc_backward(orc_block *B, const float *in, const orc_train *tc, uint32_t step)
{
    const uint32_t K = B->inputs, N = B->outputs, m = tc->batch_size;
    const int H = B->half;
    if (m == 0 || m > B->max_batch) return -1;
    const int use_bias = B->norm != 3;               /* ffn_device.rs:245 */
    const float inv_m = 1.0f / (float)m;
    const float *dp = B->d_prenorm;

    float *dw = (float *)malloc((size_t)K * N * sizeof(float));
    float *db = (float *)calloc(N, sizeof(float));
    float *gnw = (float *)calloc(N, sizeof(float));
    float *gnb = (float *)calloc(N, sizeof(float));
    if (!dw || !db || !gnw || !gnb) { free(dw); free(db); free(gnw); free(gnb); return -2; }

    /* dW[r][c] = sum_b f32(x[b][r]) * dP[b][c], b ascending (backward.cu:181-186) */
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)K; r++) {
        float *acc = dw + (size_t)r * N;
        for (uint32_t c = 0; c < N; c++) acc[c] = 0.0f;
        for (uint32_t bi = 0; bi < m; bi++) {
            const float x = in[(size_t)bi * K + r];
            const float *prow = dp + (size_t)bi * N;
            for (uint32_t c = 0; c < N; c++) acc[c] = fmaf(x, prow[c], acc[c]);
        }
    }
    /* row-0 reductions (backward.cu:187-194) */
    for (uint32_t bi = 0; bi < m; bi++)
        for (uint32_t c = 0; c < N; c++) {
            size_t idx = (size_t)bi * N + c;
            db[c] += dp[idx];
            if (B->norm > 0) {
                gnw[c] += B->d_norm_w[idx];
                if (B->norm > 1) gnb[c] += B->d_norm_b[idx];
            }
        }

    for (uint32_t c = 0; c < N; c++) {
        if (use_bias)
            orc_optimiser_update(B->b, (float *)master_or(B->master_b, B->b), B->dv_b, B->dm_b, c,
                                 db[c] * LOSS_SCALE_INV, inv_m, tc->learn_rate, tc->grad_clamp,
                                 &tc->optimiser, step, B->regularisation, B->regu_coeff, 0, H);
        if (B->norm > 0) {
            orc_optimiser_update(B->norm_w, (float *)master_or(B->master_norm_w, B->norm_w),
                                 B->dv_norm_w, B->dm_norm_w, c, gnw[c] * LOSS_SCALE_INV, inv_m,
                                 tc->learn_rate, tc->grad_clamp, &tc->norm_optimiser, step,
                                 B->regularisation, B->regu_coeff, 0, H);
            if (B->norm > 1)
                orc_optimiser_update(B->norm_b, (float *)master_or(B->master_norm_b, B->norm_b),
                                     B->dv_norm_b, B->dm_norm_b, c, gnb[c] * LOSS_SCALE_INV, inv_m,
                                     tc->learn_rate, tc->grad_clamp, &tc->norm_optimiser, step,
                                     B->regularisation, B->regu_coeff, 0, H);
        }
    }
    float *mw = (float *)master_or(B->master_w, B->w);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)K; r++)
        for (uint32_t c = 0; c < N; c++) {
            size_t idx = (size_t)r * N + c;
            orc_optimiser_update(B->w, mw, B->dv_w, B->dm_w, idx, dw[idx] * LOSS_SCALE_INV, inv_m,
                                 tc->learn_rate, tc->grad_clamp, &tc->optimiser, step,
                                 B->regularisation, B->regu_coeff, 1, H);
        }
    free(dw); free(db); free(gnw); free(gnb);
    return 0;
}
