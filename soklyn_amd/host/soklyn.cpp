// soklyn.cpp — C++ host API of the DenseBlock path (see soklyn.hpp).
//
// Every device operation goes through the C ABI of libsoklyn_hip.so; this
// file adds the reference's host-side objects around it: tensors with the
// global id counter, the parameter / cache layout and its allocation order,
// the initialisers, and the layer loop of FeedForwardNetwork.
#include "soklyn.hpp"

#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>

namespace soklyn {

// ---- errors -------------------------------------------------------------------------------
ErrorKind error_kind(int32_t status) {
    switch (status) {
    case SKL_ERR_INVALID_CONFIGURATION: return ErrorKind::InvalidConfiguration;
    case SKL_ERR_TRAINING_MODE_REQUIRED: return ErrorKind::TrainingModeRequired;
    case SKL_ERR_ALLOCATION_LIMIT: return ErrorKind::AllocationLimitExceeded;
    case SKL_ERR_MISMATCHED_DIMENSIONS: return ErrorKind::MismatchedDimensions;
    case SKL_ERR_INVALID_BATCH_SIZE: return ErrorKind::InvalidBatchSize;
    case SKL_ERR_HARDWARE_CONSTRAINT: return ErrorKind::HardwareConstraintViolation;
    case SKL_ERR_TRY_FROM_INT: return ErrorKind::TryFromIntError;
    case SKL_ERR_NULL_POINTER: return ErrorKind::NullPointer;
    case SKL_ERR_UNSUPPORTED_CAST: return ErrorKind::UnsupportedTypeCast;
    case SKL_ERR_NO_DEVICE: return ErrorKind::NoDevice;
    default: break;
    }
    if (status <= HOST_STATUS_BASE && status > HOST_STATUS_BASE - 11)
        return static_cast<ErrorKind>(static_cast<int>(ErrorKind::SerdeJSON) + (HOST_STATUS_BASE - status));
    return ErrorKind::DriverError;
}

int32_t host_status(ErrorKind kind) {
    return HOST_STATUS_BASE - (static_cast<int32_t>(kind) - static_cast<int32_t>(ErrorKind::SerdeJSON));
}

void check(int32_t status, const char *what) {
    if (status == SKL_OK) return;
    throw Error(error_kind(status), status, std::string(what) + ": " + skl_status_string(status));
}

[[noreturn]] static void fail(int32_t status, const std::string &what) {
    throw Error(error_kind(status), status, what);
}

// usize -> u32 as the reference's u32::try_from(..)?
static uint32_t to_u32(size_t v, const char *what) {
    if (v > std::numeric_limits<uint32_t>::max()) fail(SKL_ERR_TRY_FROM_INT, std::string(what) + " does not fit in u32");
    return static_cast<uint32_t>(v);
}

// ---- f16 (IEEE binary16, round to nearest even) ---------------------------------------------
f16 f16::from_f32(float v) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    f16 h;
    if (ax >= 0x7f800000u) {   // inf / NaN (NaN keeps a quiet payload bit)
        h.bits = sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u);
        return h;
    }
    if (ax >= 0x477ff000u) {   // >= 65520: rounds to infinity
        h.bits = sign | 0x7c00u;
        return h;
    }
    const uint32_t e = ax >> 23;
    if (e < 113) {             // |v| < 2^-14: binary16 subnormal (or zero) = round(|v| / 2^-24)
        const uint32_t shift = 126 - e;    // |v| / 2^-24 = m * 2^-(126 - e), m with the implicit bit
        if (e == 0 || shift > 24) {
            h.bits = sign;
            return h;
        }
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t q = m >> shift;
        const uint32_t r = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (r > half || (r == half && (q & 1u))) ++q;
        h.bits = sign | static_cast<uint16_t>(q);
        return h;
    }
    uint32_t q = ((e - 112) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t r = ax & 0x1fffu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) ++q;   // a carry moves into the exponent
    h.bits = sign | static_cast<uint16_t>(q);
    return h;
}

float f16::to_f32() const {
    const uint32_t sign = static_cast<uint32_t>(bits & 0x8000u) << 16;
    const uint32_t e = (bits >> 10) & 0x1fu, m = bits & 0x3ffu;
    uint32_t x;
    if (e == 0x1f) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else {   // subnormal: m * 2^-24, exact in f32
        const float f = static_cast<float>(m) * (1.0f / 16777216.0f);
        std::memcpy(&x, &f, 4);
        x |= sign;
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// ---- modes ----------------------------------------------------------------------------------
skl_optimiser Optimiser::to_c() const {
    // Optimiser extraction as at ffn_device.rs:257-267
    skl_optimiser o{};
    o.kind = static_cast<uint32_t>(kind);
    if (kind == Kind::SGD) {
        o.beta1 = v_coeff;
        o.nesterov = nesterov ? 1u : 0u;
    } else {
        o.beta1 = m_coeff;
        o.beta2 = v_coeff;
        o.epsilon = epsilon;
    }
    return o;
}

uint32_t scramble_seed(uint32_t step, uint32_t layer_id) { return skl_scramble_seed(step, layer_id); }

// ---- GpuContext -----------------------------------------------------------------------------
GpuContext::GpuContext(int32_t ordinal, uint32_t tile_dim) {
    check(skl_ctx_create(ordinal, tile_dim, &ctx_), "GpuContext::with_device_index");
}
GpuContext::~GpuContext() {
    if (ctx_) skl_ctx_destroy(ctx_);
}
GpuContext &GpuContext::operator=(GpuContext &&o) noexcept {
    if (this != &o) {
        if (ctx_) skl_ctx_destroy(ctx_);
        ctx_ = o.ctx_;
        o.ctx_ = nullptr;
    }
    return *this;
}
void GpuContext::synchronize() const { check(skl_synchronize(ctx_), "GpuContext::synchronize"); }

DeviceBuffer::DeviceBuffer(const GpuContext &ctx, size_t bytes) : ctx_(ctx.raw()) {
    check(skl_malloc(ctx_, &p_, bytes), "device allocation");
}
DeviceBuffer::~DeviceBuffer() {
    if (p_) skl_free(ctx_, p_);
}
DeviceBuffer &DeviceBuffer::operator=(DeviceBuffer &&o) noexcept {
    if (this != &o) {
        if (p_) skl_free(ctx_, p_);
        ctx_ = o.ctx_;
        p_ = o.p_;
        o.p_ = nullptr;
    }
    return *this;
}

// ---- tensors --------------------------------------------------------------------------------
static std::atomic<size_t> TENSOR_ID_COUNTER{0};   // core.rs:84
size_t generate_unique_tensor_id() { return TENSOR_ID_COUNTER.fetch_add(1, std::memory_order_relaxed); }
size_t peek_tensor_id_counter() { return TENSOR_ID_COUNTER.load(std::memory_order_relaxed); }

template <class T> static constexpr uint32_t dtype_of() { return static_cast<uint32_t>(PrecisionType<T>::precision); }

template <class T, size_t R> size_t Tensor<T, R>::len() const {
    size_t n = 1;
    for (size_t d : shape_) n *= d;
    return n;
}

template <class T, size_t R> void Tensor<T, R>::steal(Tensor &o) noexcept {
    ctx_ = o.ctx_;
    data_ = o.data_;
    shape_ = o.shape_;
    id_ = o.id_;
    o.data_ = nullptr;
}

template <class T, size_t R> void Tensor<T, R>::release() noexcept {
    if (data_) skl_free(ctx_, data_);
    data_ = nullptr;
}

template <class T, size_t R> Tensor<T, R>::~Tensor() { release(); }

template <class T, size_t R> Tensor<T, R> &Tensor<T, R>::operator=(Tensor &&o) noexcept {
    if (this != &o) {
        release();
        steal(o);
    }
    return *this;
}

// core.rs:557-579
template <class T, size_t R>
Tensor<T, R> Tensor<T, R>::from_cpu_vector(const GpuContext &ctx, const std::vector<T> &cpu_data, const Shape &shape) {
    size_t size = 1;
    for (size_t d : shape) size *= d;
    if (size != cpu_data.size())
        fail(SKL_ERR_MISMATCHED_DIMENSIONS, "length of CPU data does not match the total elements of the tensor: expected " +
                                                std::to_string(size) + ", found " + std::to_string(cpu_data.size()));
    Tensor t;
    t.ctx_ = ctx.raw();
    t.shape_ = shape;
    void *p = nullptr;
    check(skl_malloc(t.ctx_, &p, size * sizeof(T)), "Tensor::from_cpu_vector");
    t.data_ = static_cast<T *>(p);
    check(skl_memcpy_h2d(t.ctx_, t.data_, cpu_data.data(), size * sizeof(T)), "Tensor::from_cpu_vector");
    check(skl_synchronize(t.ctx_), "Tensor::from_cpu_vector");
    t.id_ = generate_unique_tensor_id();
    return t;
}

// core.rs:634-645
template <class T, size_t R> Tensor<T, R> Tensor<T, R>::zeros(const GpuContext &ctx, const Shape &shape) {
    Tensor t;
    t.ctx_ = ctx.raw();
    t.shape_ = shape;
    const size_t n = t.len();
    void *p = nullptr;
    check(skl_malloc(t.ctx_, &p, n * sizeof(T)), "Tensor::zeros");
    t.data_ = static_cast<T *>(p);
    check(skl_fill(t.ctx_, t.data_, dtype_of<T>(), 0.0f, n), "Tensor::zeros");
    check(skl_synchronize(t.ctx_), "Tensor::zeros");
    t.id_ = generate_unique_tensor_id();
    return t;
}

// core.rs:611-615
template <class T, size_t R> Tensor<T, R> Tensor<T, R>::fill(const GpuContext &ctx, const Shape &shape, T value) {
    Tensor t = zeros(ctx, shape);
    t.broadcast(ctx, value);
    return t;
}

// core.rs:675-677 (gpu_broadcast)
template <class T, size_t R> void Tensor<T, R>::broadcast(const GpuContext &ctx, T value) {
    check(skl_fill(ctx.raw(), data_, dtype_of<T>(), PrecisionType<T>::to_f32(value), len()), "Tensor::broadcast");
}

// core.rs:686-692
template <class T, size_t R> Tensor<T, R> Tensor<T, R>::clone(const GpuContext &ctx) const {
    Tensor t;
    t.ctx_ = ctx.raw();
    t.shape_ = shape_;
    void *p = nullptr;
    check(skl_malloc(t.ctx_, &p, len() * sizeof(T)), "Tensor::clone");
    t.data_ = static_cast<T *>(p);
    check(skl_memcpy_d2d(t.ctx_, t.data_, data_, len() * sizeof(T)), "Tensor::clone");
    t.id_ = generate_unique_tensor_id();
    return t;
}

// type.rs:164-176: a zeros tensor of the new type (new id), gpu_cast_t, free the source
template <class T, size_t R> template <class U> Tensor<U, R> Tensor<T, R>::cast(const GpuContext &ctx) && {
    Tensor<U, R> t = Tensor<U, R>::zeros(ctx, shape_);
    check(skl_cast(ctx.raw(), data_, dtype_of<T>(), t.data_, dtype_of<U>(), len()), "Tensor::cast");
    std::move(*this).free_and_sync(ctx);
    return t;
}

template <class T, size_t R> std::vector<T> Tensor<T, R>::download(const GpuContext &ctx) const {
    std::vector<T> v(len());
    check(skl_memcpy_d2h(ctx.raw(), v.data(), data_, len() * sizeof(T)), "Tensor::download");
    return v;
}

template <class T, size_t R> void Tensor<T, R>::free_and_sync(const GpuContext &ctx) && {
    release();
    check(skl_synchronize(ctx.raw()), "Tensor::free_and_sync");
}

// ---- initialisers ---------------------------------------------------------------------------
static inline uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

// The ChaCha block function (D. J. Bernstein; RFC 7539 section 2.3) with a
// 64-bit block counter in words 12-13 and a zero stream id in words 14-15.
void ChaCha8Rng::block(const uint32_t k[8], uint64_t counter, int rounds, uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, k[0], k[1], k[2], k[3],
                      k[4],        k[5],        k[6],        k[7],        static_cast<uint32_t>(counter),
                      static_cast<uint32_t>(counter >> 32), 0u, 0u};
    uint32_t x[16];
    std::memcpy(x, s, sizeof(s));
    auto qr = [&x](int a, int b, int c, int d) {
        x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 16);
        x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 12);
        x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 8);
        x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 7);
    };
    for (int r = 0; r < rounds; r += 2) {
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);   // columns
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);   // diagonals
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

ChaCha8Rng ChaCha8Rng::from_seed(const std::array<uint8_t, 32> &key) {
    ChaCha8Rng r;
    for (int i = 0; i < 8; ++i)
        r.key_[i] = static_cast<uint32_t>(key[4 * i]) | (static_cast<uint32_t>(key[4 * i + 1]) << 8) |
                    (static_cast<uint32_t>(key[4 * i + 2]) << 16) | (static_cast<uint32_t>(key[4 * i + 3]) << 24);
    return r;
}

uint32_t pcg32_xsh_rr(uint64_t state) {
    const uint32_t xorshifted = static_cast<uint32_t>(((state >> 18) ^ state) >> 27);
    const uint32_t rot = static_cast<uint32_t>(state >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

// rand_core 0.9.5 SeedableRng::seed_from_u64: each 4 seed bytes are one PCG32
// output, the state advanced before each output (LCG multiplier
// PCG32_MULTIPLIER, increment 11634580027462260723), little endian.
ChaCha8Rng ChaCha8Rng::seed_from_u64(uint64_t state) {
    const uint64_t INC = 11634580027462260723ull;
    std::array<uint8_t, 32> key{};
    for (int i = 0; i < 8; ++i) {
        state = state * PCG32_MULTIPLIER + INC;
        const uint32_t x = pcg32_xsh_rr(state);
        for (int b = 0; b < 4; ++b) key[4 * i + b] = static_cast<uint8_t>(x >> (8 * b));
    }
    return from_seed(key);
}

uint32_t ChaCha8Rng::next_u32() {
    if (pos_ == 16) {
        block(key_, counter_++, 8, buf_);
        pos_ = 0;
    }
    return buf_[pos_++];
}

// function.rs:219-233: Box-Muller, u1 in (0, 1], u2 in [0, 1], f32 arithmetic
// in the reference's evaluation order (the file is built without FP contraction).
static std::vector<float> normal_dist(size_t total, ChaCha8Rng &rng, float factor, float stdev) {
    const float two32 = 4294967296.0f;   // u32::MAX as f32 (+ 1.0 rounds back to it)
    const float two_pi = 2.0f * 3.14159265358979323846f;
    std::vector<float> v(total);
    for (size_t i = 0; i < total; ++i) {
        const float u1 = (static_cast<float>(rng.next_u32()) + 1.0f) / two32;
        const float u2 = static_cast<float>(rng.next_u32()) / two32;
        const float z = std::sqrt(-2.0f * std::log(u1)) * std::cos(two_pi * u2);
        v[i] = factor * z * stdev;
    }
    return v;
}

// function.rs:235-247
static std::vector<float> uniform_dist(size_t total, ChaCha8Rng &rng, float factor, float limit) {
    std::vector<float> v(total);
    for (size_t i = 0; i < total; ++i) {
        const float raw = static_cast<float>(rng.next_u32()) / 4294967296.0f;
        v[i] = factor * (-limit + raw * (2.0f * limit));
    }
    return v;
}

std::vector<float> InitXavierUniformFunc::init_f32(size_t fan_in, size_t fan_out, size_t len) {
    return uniform_dist(len, rng_, factor_, std::sqrt(6.0f / static_cast<float>(fan_in + fan_out)));
}
std::vector<float> InitXavierNormalFunc::init_f32(size_t fan_in, size_t fan_out, size_t len) {
    return normal_dist(len, rng_, factor_, std::sqrt(2.0f / static_cast<float>(fan_in + fan_out)));
}
std::vector<float> InitHeUniformFunc::init_f32(size_t fan_in, size_t, size_t len) {
    return uniform_dist(len, rng_, factor_, std::sqrt(6.0f / static_cast<float>(fan_in)));
}
std::vector<float> InitHeNormalFunc::init_f32(size_t fan_in, size_t, size_t len) {
    return normal_dist(len, rng_, factor_, std::sqrt(2.0f / static_cast<float>(fan_in)));
}

// ---- ParamState / ForwardCache ---------------------------------------------------------------
// mlp.rs:46-76; fields are created in declaration order, which fixes the tensor ids
template <class T>
ParamState<T> ParamState<T>::new_linear(const GpuContext &ctx, const std::vector<T> &w_vec,
                                        const std::array<size_t, 2> &w_shape, const std::array<size_t, 2> &b_shape,
                                        bool is_training) {
    ParamState p;
    p.w = Tensor2D<T>::from_cpu_vector(ctx, w_vec, w_shape);
    p.b = Tensor2D<T>::zeros(ctx, b_shape);
    if (PrecisionType<T>::precision == Precision::FP16) {   // maybe_master_tensor (mlp.rs:27-43)
        std::vector<float> f(w_vec.size());
        for (size_t i = 0; i < w_vec.size(); ++i) f[i] = PrecisionType<T>::to_f32(w_vec[i]);
        p.master_w = Tensor2D<float>::from_cpu_vector(ctx, f, w_shape);
        p.master_b = Tensor2D<float>::zeros(ctx, b_shape);
    }
    if (is_training) {
        p.dv_w = Tensor2D<float>::zeros(ctx, w_shape);
        p.dv_b = Tensor2D<float>::zeros(ctx, b_shape);
        p.dm_w = Tensor2D<float>::zeros(ctx, w_shape);
        p.dm_b = Tensor2D<float>::zeros(ctx, b_shape);
    }
    return p;
}

// mlp.rs:78-110
template <class T>
ParamState<T> ParamState<T>::new_norm(const GpuContext &ctx, const std::array<size_t, 2> &shape, bool is_training) {
    ParamState p;
    p.w = Tensor2D<T>::fill(ctx, shape, PrecisionType<T>::from_f32(1.0f));
    p.b = Tensor2D<T>::zeros(ctx, shape);
    if (PrecisionType<T>::precision == Precision::FP16) {
        p.master_w = Tensor2D<float>::fill(ctx, shape, 1.0f);
        p.master_b = Tensor2D<float>::zeros(ctx, shape);
    }
    if (is_training) {
        p.dv_w = Tensor2D<float>::zeros(ctx, shape);
        p.dv_b = Tensor2D<float>::zeros(ctx, shape);
        p.dm_w = Tensor2D<float>::zeros(ctx, shape);
        p.dm_b = Tensor2D<float>::zeros(ctx, shape);
    }
    return p;
}

// mlp.rs:112-182
template <class T> void ParamState<T>::validate() const {
    auto same = [](const Tensor2D<T> &p, const std::optional<Tensor2D<float>> &s, const char *what) {
        if (!s) return;
        if (p.rows() != s->rows())
            fail(SKL_ERR_MISMATCHED_DIMENSIONS, std::string("optimizer state ") + what + " rows: expected " +
                                                    std::to_string(p.rows()) + ", found " + std::to_string(s->rows()));
        if (p.cols() != s->cols())
            fail(SKL_ERR_MISMATCHED_DIMENSIONS, std::string("optimizer state ") + what + " columns: expected " +
                                                    std::to_string(p.cols()) + ", found " + std::to_string(s->cols()));
    };
    same(w, dv_w, "weight vs dv_w");
    same(w, dm_w, "weight vs dm_w");
    same(b, dv_b, "bias vs dv_b");
    same(b, dm_b, "bias vs dm_b");
}

// mlp.rs:231-241
template <class T>
ForwardCache<T> ForwardCache<T>::create(const GpuContext &ctx, size_t max_batch_size, size_t outputs) {
    ForwardCache c;
    c.out = Tensor2D<T>::zeros(ctx, {max_batch_size, outputs});
    c.predrop_out = Tensor2D<T>::zeros(ctx, {max_batch_size, outputs});
    c.preact_out = Tensor2D<T>::zeros(ctx, {max_batch_size, outputs});
    c.centered_out = Tensor2D<T>::zeros(ctx, {max_batch_size, outputs});
    c.prenorm_out = Tensor2D<T>::zeros(ctx, {max_batch_size, outputs});
    c.norm_rstd = Tensor1D<T>::zeros(ctx, {max_batch_size > outputs ? max_batch_size : outputs});
    return c;
}

// mlp.rs:243-252
template <class T> template <class U> ForwardCache<U> ForwardCache<T>::cast(const GpuContext &ctx) && {
    ForwardCache<U> c;
    c.out = std::move(out).template cast<U>(ctx);
    c.predrop_out = std::move(predrop_out).template cast<U>(ctx);
    c.preact_out = std::move(preact_out).template cast<U>(ctx);
    c.centered_out = std::move(centered_out).template cast<U>(ctx);
    c.prenorm_out = std::move(prenorm_out).template cast<U>(ctx);
    c.norm_rstd = std::move(norm_rstd).template cast<U>(ctx);
    return c;
}

// ---- DenseBlock -----------------------------------------------------------------------------
template <class T>
const Tensor2D<float> &DenseBlock<T>::need(const std::optional<Tensor2D<float>> &t, const char *name) {
    if (!t) fail(SKL_ERR_TRAINING_MODE_REQUIRED, std::string(name) + " exists only in training mode");
    return *t;
}

template <class T> void DenseBlock<T>::alloc_dprenorm_h(const GpuContext &ctx) {
    if (PrecisionType<T>::precision == Precision::FP16 && is_training_)
        d_prenorm_h_ = DeviceBuffer(ctx, max_batch_size_ * linear_state_.w.cols() * sizeof(uint16_t));
    else
        d_prenorm_h_ = DeviceBuffer();
}

template <class T>
DenseBlock<T> DenseBlock<T>::create(const GpuContext &ctx, bool is_training, size_t inputs, size_t outputs,
                                    size_t max_batch_size, InitFunc &init) {
    return new_with_config(ctx, is_training, inputs, outputs, max_batch_size, init, LayerInitConfig{});
}

// mlp.rs:341-375
template <class T>
DenseBlock<T> DenseBlock<T>::new_with_config(const GpuContext &ctx, bool is_training, size_t inputs, size_t outputs,
                                             size_t max_batch_size, InitFunc &init, const LayerInitConfig &cfg) {
    if (inputs == 0 || outputs == 0) fail(SKL_ERR_INVALID_CONFIGURATION, "Input or output size cannot be 0.");
    if (max_batch_size == 0) fail(SKL_ERR_INVALID_CONFIGURATION, "Batch size cannot be 0.");
    const std::vector<T> w_vec = init.template init<T>(inputs, outputs, inputs * outputs);
    const std::array<size_t, 2> weight_shape{inputs, outputs}, bias_shape{1, outputs};
    // the linear state is built before the norm state (argument order at mlp.rs:367-374)
    ParamState<T> linear = ParamState<T>::new_linear(ctx, w_vec, weight_shape, bias_shape, is_training);
    ParamState<T> norm = ParamState<T>::new_norm(ctx, bias_shape, is_training);
    return from_tensors(ctx, is_training, std::move(linear), std::move(norm), max_batch_size, cfg);
}

// mlp.rs:377-421
template <class T>
DenseBlock<T> DenseBlock<T>::from_tensors(const GpuContext &ctx, bool is_training, ParamState<T> linear_state,
                                          ParamState<T> norm_state, size_t max_batch_size,
                                          const LayerInitConfig &cfg) {
    linear_state.validate();
    norm_state.validate();
    const size_t wc = linear_state.w.cols();
    const std::array<size_t, 2> batch_shape{max_batch_size, wc};
    DenseBlock blk;
    blk.linear_state_ = std::move(linear_state);
    blk.norm_state_ = std::move(norm_state);
    blk.cache_ = ForwardCache<T>::create(ctx, max_batch_size, wc);
    if (is_training) {
        blk.grad_ = Tensor2D<float>::zeros(ctx, batch_shape);
        blk.d_prenorm_out_ = Tensor2D<float>::zeros(ctx, batch_shape);
        blk.d_norm_w_ = Tensor2D<float>::zeros(ctx, batch_shape);
        blk.d_norm_b_ = Tensor2D<float>::zeros(ctx, batch_shape);
    }
    blk.mask_ = Tensor2D<T>::fill(ctx, batch_shape, PrecisionType<T>::from_f32(1.0f));
    blk.max_batch_size_ = max_batch_size;
    blk.normalisation_ = cfg.normalisation;
    blk.activation_ = cfg.activation;
    blk.regularisation_ = cfg.regularisation;
    blk.mask_coeff_ = cfg.mask_coeff;
    blk.is_training_ = is_training;
    blk.alloc_dprenorm_h(ctx);
    return blk;
}

template <class T> skl_dense_desc DenseBlock<T>::desc() const {
    auto opt = [](const std::optional<Tensor2D<float>> &t) -> float * { return t ? t->get_data() : nullptr; };
    skl_dense_desc d{};
    d.dtype = dtype_of<T>();
    d.inputs = to_u32(linear_state_.w.rows(), "weight rows");
    d.outputs = to_u32(linear_state_.w.cols(), "weight cols");
    d.max_batch = to_u32(max_batch_size_, "max batch size");
    d.norm = static_cast<uint32_t>(normalisation_);
    d.act = static_cast<uint32_t>(activation_.kind);
    d.leaky = activation_.kind == Activation::Kind::LeakyReLU ? activation_.coeff : 0.0f;   // ffn_device.rs:32-35
    d.mask_coeff = mask_coeff_;
    d.regularisation = static_cast<uint32_t>(regularisation_.kind);
    d.regu_coeff = regularisation_.regu_coeff;
    d.is_training = is_training_ ? 1u : 0u;
    d.w = linear_state_.w.get_data();
    d.b = linear_state_.b.get_data();
    d.norm_w = norm_state_.w.get_data();
    d.norm_b = norm_state_.b.get_data();
    d.master_w = opt(linear_state_.master_w);
    d.master_b = opt(linear_state_.master_b);
    d.master_norm_w = opt(norm_state_.master_w);
    d.master_norm_b = opt(norm_state_.master_b);
    d.dv_w = opt(linear_state_.dv_w);
    d.dv_b = opt(linear_state_.dv_b);
    d.dm_w = opt(linear_state_.dm_w);
    d.dm_b = opt(linear_state_.dm_b);
    d.dv_norm_w = opt(norm_state_.dv_w);
    d.dv_norm_b = opt(norm_state_.dv_b);
    d.dm_norm_w = opt(norm_state_.dm_w);
    d.dm_norm_b = opt(norm_state_.dm_b);
    d.out = cache_.out.get_data();
    d.predrop = cache_.predrop_out.get_data();
    d.preact = cache_.preact_out.get_data();
    d.centered = cache_.centered_out.get_data();
    d.prenorm = cache_.prenorm_out.get_data();
    d.norm_rstd = cache_.norm_rstd.get_data();
    d.mask = mask_.get_data();
    d.grad = opt(grad_);
    d.d_prenorm = opt(d_prenorm_out_);
    d.d_norm_w = opt(d_norm_w_);
    d.d_norm_b = opt(d_norm_b_);
    d.d_prenorm_h = d_prenorm_h_.get();
    return d;
}

template <class T> skl_train_ctx DenseBlock<T>::train_c(const TrainContext &t) const {
    skl_train_ctx c{};
    c.optimiser = t.optimiser->to_c();
    c.norm_optimiser = t.norm_optimiser->to_c();
    c.batch_size = to_u32(t.batch_size, "batch size");
    c.learn_rate = t.learn_rate;
    c.grad_clamp = t.grad_clamp;
    return c;
}

// mlp.rs:548-580 / ffn_device.rs:12-139 (the validation of mlp.rs runs inside the C ABI)
template <class T>
const Tensor2D<T> &DenseBlock<T>::forward(const GpuContext &ctx, const Tensor2D<T> &input, size_t batch_size,
                                          bool use_dropout, size_t step) const {
    const skl_dense_desc d = desc();
    const uint32_t seed = scramble_seed(to_u32(step, "step"), to_u32(linear_state_.w.get_id(), "weight id"));
    check(skl_dense_forward(ctx.raw(), &d, input.get_data(), to_u32(input.rows(), "input rows"),
                            to_u32(input.cols(), "input cols"), to_u32(batch_size, "batch size"),
                            use_dropout ? 1u : 0u, seed),
          "DenseBlock::forward");
    return cache_.out;
}

// mlp.rs:756-821
template <class T>
void DenseBlock<T>::compute_loss(const GpuContext &ctx, const Tensor2D<T> &target, const LossConfig &lc) const {
    const skl_dense_desc d = desc();
    check(skl_dense_output_error(ctx.raw(), &d, target.get_data(), to_u32(target.rows(), "target rows"),
                                 to_u32(target.cols(), "target cols"), static_cast<uint32_t>(lc.loss_func),
                                 static_cast<uint32_t>(lc.activation.kind),
                                 lc.activation.kind == Activation::Kind::LeakyReLU ? lc.activation.coeff : 0.0f),
          "DenseBlock::compute_loss");
}

// mlp.rs:607-658
template <class T>
void DenseBlock<T>::backward_output(const GpuContext &ctx, const Tensor2D<T> &input, const TrainContext &train_ctx,
                                    size_t step) const {
    const skl_dense_desc d = desc();
    const skl_train_ctx t = train_c(train_ctx);
    check(skl_dense_backward(ctx.raw(), &d, input.get_data(), to_u32(input.rows(), "input rows"),
                             to_u32(input.cols(), "input cols"), &t, to_u32(step, "step")),
          "DenseBlock::backward_output");
}

// mlp.rs:674-736
template <class T>
void DenseBlock<T>::backward_hidden(const GpuContext &ctx, const DenseBlock &next_layer, const Tensor2D<T> &input,
                                    const TrainContext &train_ctx, size_t step) const {
    const skl_dense_desc d = desc(), n = next_layer.desc();
    const skl_train_ctx t = train_c(train_ctx);
    check(skl_dense_backward_hidden(ctx.raw(), &d, &n, input.get_data(), to_u32(input.rows(), "input rows"),
                                    to_u32(input.cols(), "input cols"), &t, to_u32(step, "step")),
          "DenseBlock::backward_hidden");
}

// mlp.rs:475-477
template <class T> void DenseBlock<T>::reset_mask(const GpuContext &ctx) {
    mask_.broadcast(ctx, PrecisionType<T>::from_f32(1.0f));
}

// ParamState<f32>::cast_f16 (mlp.rs:204-219) and ParamState<f16>::cast_f32 (mlp.rs:186-202)
static ParamState<f16> param_cast_f16(const GpuContext &ctx, ParamState<float> &&s) {
    Tensor2D<float> w = s.w.clone(ctx);
    Tensor2D<float> b = s.b.clone(ctx);
    ParamState<f16> p;
    p.w = std::move(w).cast<f16>(ctx);
    p.b = std::move(b).cast<f16>(ctx);
    p.master_w = s.w.clone(ctx);
    p.master_b = s.b.clone(ctx);
    p.dv_w = std::move(s.dv_w);
    p.dv_b = std::move(s.dv_b);
    p.dm_w = std::move(s.dm_w);
    p.dm_b = std::move(s.dm_b);
    return p;
}
static ParamState<float> param_cast_f32(const GpuContext &ctx, ParamState<f16> &&s) {
    ParamState<float> p;
    p.w = s.master_w.value().clone(ctx);
    p.b = s.master_b.value().clone(ctx);
    p.dv_w = std::move(s.dv_w);
    p.dv_b = std::move(s.dv_b);
    p.dm_w = std::move(s.dm_w);
    p.dm_b = std::move(s.dm_b);
    return p;
}

// mlp.rs:835-856
template <class T> DenseBlock<f16> DenseBlock<T>::convert_f16(const GpuContext &ctx) && {
    if constexpr (PrecisionType<T>::precision != Precision::FP32) {
        fail(SKL_ERR_UNSUPPORTED_CAST, "convert_f16 is defined for f32 blocks");
    } else {
        DenseBlock<f16> o;
        o.linear_state_ = param_cast_f16(ctx, std::move(linear_state_));
        o.norm_state_ = param_cast_f16(ctx, std::move(norm_state_));
        o.cache_ = std::move(cache_).template cast<f16>(ctx);
        o.grad_ = std::move(grad_);
        o.d_prenorm_out_ = std::move(d_prenorm_out_);
        o.d_norm_w_ = std::move(d_norm_w_);
        o.d_norm_b_ = std::move(d_norm_b_);
        o.mask_ = std::move(mask_).template cast<f16>(ctx);
        o.normalisation_ = normalisation_;
        o.activation_ = activation_;
        o.regularisation_ = regularisation_;
        o.max_batch_size_ = max_batch_size_;
        o.mask_coeff_ = mask_coeff_;
        o.is_training_ = is_training_;
        o.alloc_dprenorm_h(ctx);
        return o;
    }
}

// mlp.rs:868-888
template <class T> DenseBlock<float> DenseBlock<T>::convert_f32(const GpuContext &ctx) && {
    if constexpr (PrecisionType<T>::precision != Precision::FP16) {
        fail(SKL_ERR_UNSUPPORTED_CAST, "convert_f32 is defined for f16 blocks");
    } else {
        DenseBlock<float> o;
        o.linear_state_ = param_cast_f32(ctx, std::move(linear_state_));
        o.norm_state_ = param_cast_f32(ctx, std::move(norm_state_));
        o.cache_ = std::move(cache_).template cast<float>(ctx);
        o.grad_ = std::move(grad_);
        o.d_prenorm_out_ = std::move(d_prenorm_out_);
        o.d_norm_w_ = std::move(d_norm_w_);
        o.d_norm_b_ = std::move(d_norm_b_);
        o.mask_ = std::move(mask_).template cast<float>(ctx);
        o.normalisation_ = normalisation_;
        o.activation_ = activation_;
        o.regularisation_ = regularisation_;
        o.max_batch_size_ = max_batch_size_;
        o.mask_coeff_ = mask_coeff_;
        o.is_training_ = is_training_;
        o.alloc_dprenorm_h(ctx);
        return o;
    }
}

// ---- FeedForwardNetwork (ffn.rs:40-166) ------------------------------------------------------
template <class T>
std::vector<const Tensor2D<T> *> FeedForwardNetwork<T>::forward(const GpuContext &ctx, const Tensor2D<T> &input,
                                                                size_t batch_size, bool use_dropout,
                                                                size_t step) const {
    std::vector<const Tensor2D<T> *> outputs;
    outputs.reserve(layers_.size());
    const Tensor2D<T> *cur = &input;
    for (const DenseBlock<T> &layer : layers_) {
        cur = &layer.forward(ctx, *cur, batch_size, use_dropout, step);
        outputs.push_back(cur);
    }
    return outputs;
}

template <class T>
Tensor2D<T> FeedForwardNetwork<T>::forward_raw(const GpuContext &ctx, const std::vector<T> &raw_pixels,
                                               size_t batch_size, bool use_dropout, size_t step) const {
    Tensor2D<T> input = Tensor2D<T>::from_cpu_vector(ctx, raw_pixels, {batch_size, inputs_});
    const std::vector<const Tensor2D<T> *> outs = forward(ctx, input, batch_size, use_dropout, step);
    if (outs.empty())
        fail(SKL_ERR_INVALID_CONFIGURATION, "Cannot execute raw forward pass on an empty network matrix architecture");
    return outs.back()->clone(ctx);
}

template <class T>
void FeedForwardNetwork<T>::backward(const GpuContext &ctx, const std::vector<const Tensor2D<T> *> &outputs,
                                     const Tensor2D<T> &target, const Tensor2D<T> &input, const LossConfig &loss_config,
                                     const MultiLayerTrainContext &train_ctx, size_t step) const {
    const size_t num_layers = layers_.size();
    if (outputs.size() != num_layers || train_ctx.optimisers.size() != num_layers)
        fail(SKL_ERR_INVALID_CONFIGURATION, "Backward pass expects exactly " + std::to_string(num_layers) +
                                                " activation vectors and optimizers. Found " +
                                                std::to_string(outputs.size()) + " outputs, " +
                                                std::to_string(train_ctx.optimisers.size()) + " optimisers.");
    const size_t last = num_layers - 1;
    const Tensor2D<T> &head_input = last > 0 ? *outputs[last - 1] : input;
    layers_[last].compute_loss(ctx, target, loss_config);
    layers_[last].backward_output(ctx, head_input, train_ctx.get_train_context(last), step);
    for (size_t i = last; i-- > 0;) {
        const Tensor2D<T> &layer_input = i > 0 ? *outputs[i - 1] : input;
        layers_[i].backward_hidden(ctx, layers_[i + 1], layer_input, train_ctx.get_train_context(i), step);
    }
}

// ---- instantiations ---------------------------------------------------------------------------
template class Tensor<float, 1>;
template class Tensor<float, 2>;
template class Tensor<f16, 1>;
template class Tensor<f16, 2>;
template Tensor<f16, 1> Tensor<float, 1>::cast<f16>(const GpuContext &) &&;
template Tensor<f16, 2> Tensor<float, 2>::cast<f16>(const GpuContext &) &&;
template Tensor<float, 1> Tensor<f16, 1>::cast<float>(const GpuContext &) &&;
template Tensor<float, 2> Tensor<f16, 2>::cast<float>(const GpuContext &) &&;
template struct ParamState<float>;
template struct ParamState<f16>;
template struct ForwardCache<float>;
template struct ForwardCache<f16>;
template class DenseBlock<float>;
template class DenseBlock<f16>;
template class FeedForwardNetwork<float>;
template class FeedForwardNetwork<f16>;

}  // namespace soklyn
