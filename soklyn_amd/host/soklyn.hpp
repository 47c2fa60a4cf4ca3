// soklyn.hpp — C++ host API of the DenseBlock path, over the C ABI of
// libsoklyn_hip.so (include/soklyn_hip.h).
//
// Mirrors the reference's public Rust surface for this path, with the same
// names, argument meaning and error behaviour:
//   Tensor / Tensor2D / Tensor1D + the global tensor-id counter  src/util/core.rs:84-94, 414-693
//   GpuContext                                                   src/io/device.rs:61-183
//   Precision / Normalisation / Activation / Regularisation /
//   Optimiser / LossFunc, the Init*Func family                   src/util/function.rs, src/util/type.rs
//   LayerInitConfig / TrainContext / MultiLayerTrainContext /
//   LossConfig                                                   src/util/context.rs:11-85
//   ParamState / ForwardCache / DenseBlock                       src/mlp.rs:14-888
//   FeedForwardNetwork                                           src/ffn.rs:10-166
// Rust `Result<_, Error>` becomes a thrown soklyn::Error whose kind is the
// reference's Error variant (the C ABI's negative status codes).  Every device
// buffer is owned by a Tensor (move-only); the GpuContext must outlive the
// tensors allocated on it, as the Rust tensors hold the context alive.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "soklyn_hip.h"

namespace soklyn {

// ---- errors (src/util/log.rs:15-99) ---------------------------------------------
enum class ErrorKind {
    InvalidConfiguration,
    TrainingModeRequired,
    AllocationLimitExceeded,
    MismatchedDimensions,
    InvalidBatchSize,
    HardwareConstraintViolation,
    TryFromIntError,
    NullPointer,
    UnsupportedTypeCast,
    NoDevice,
    DriverError,
    // host-side variants of the checkpoint format (src/util/log.rs; status codes below -100)
    SerdeJSON,
    IOError,
    PersistError,
    SerializationCasting,
    UnrecognizedTensorKey,
    InvalidTensorName,
    PrecisionMatch,
    NoLayersFound,
    MissingLayer,
    MissingWeights,
    MissingBiases,
};
// Status codes of the host-only error kinds (no C ABI counterpart).
constexpr int32_t HOST_STATUS_BASE = -100;
int32_t host_status(ErrorKind kind);

class Error : public std::runtime_error {
  public:
    Error(ErrorKind kind, int32_t status, const std::string &what)
        : std::runtime_error(what), kind_(kind), status_(status) {}
    ErrorKind kind() const { return kind_; }
    int32_t status() const { return status_; }   // the C ABI status code

  private:
    ErrorKind kind_;
    int32_t status_;
};

ErrorKind error_kind(int32_t status);
// Throws Error for a non-zero C ABI status; `what` names the failing call.
void check(int32_t status, const char *what);

// ---- precision (src/util/type.rs:29-113) ----------------------------------------
enum class Precision : uint32_t { FP32 = SKL_F32, FP16 = SKL_F16 };

// IEEE binary16 storage with round-to-nearest-even conversion from f32 (the
// `half` crate's from_f32, which the reference uses for host data).
struct f16 {
    uint16_t bits = 0;
    static f16 from_f32(float v);
    float to_f32() const;
    bool operator==(const f16 &o) const { return bits == o.bits; }
};

template <class T> struct PrecisionType;
template <> struct PrecisionType<float> {
    static constexpr Precision precision = Precision::FP32;
    static float from_f32(float v) { return v; }
    static float to_f32(float v) { return v; }
};
template <> struct PrecisionType<f16> {
    static constexpr Precision precision = Precision::FP16;
    static f16 from_f32(float v) { return f16::from_f32(v); }
    static float to_f32(f16 v) { return v.to_f32(); }
};

// ---- modes (src/util/function.rs:10-176; ordinals as passed to the kernels) --------
enum class Normalisation : uint32_t { Disabled = 0, RMSNorm = 1, LayerNorm = 2, BatchNorm = 3 };

struct Activation {
    enum class Kind : uint32_t { Identity = 0, Sigmoid, ReLU, LeakyReLU, Tanh, Softmax, SiLU, Mish };
    Kind kind = Kind::Identity;
    float coeff = 0.0f;   // LeakyReLU { coeff }
    static Activation identity() { return {Kind::Identity, 0.0f}; }
    static Activation sigmoid() { return {Kind::Sigmoid, 0.0f}; }
    static Activation relu() { return {Kind::ReLU, 0.0f}; }
    static Activation leaky_relu(float coeff) { return {Kind::LeakyReLU, coeff}; }
    static Activation tanh() { return {Kind::Tanh, 0.0f}; }
    static Activation softmax() { return {Kind::Softmax, 0.0f}; }
    static Activation silu() { return {Kind::SiLU, 0.0f}; }
    static Activation mish() { return {Kind::Mish, 0.0f}; }
    bool operator==(const Activation &o) const { return kind == o.kind && coeff == o.coeff; }
};

struct Regularisation {
    enum class Kind : uint32_t { None = 0, L1Regular = 1, L2Regular = 2 };
    Kind kind = Kind::None;
    float regu_coeff = 0.0f;
    static Regularisation none() { return {}; }
    static Regularisation l1(float c) { return {Kind::L1Regular, c}; }
    static Regularisation l2(float c) { return {Kind::L2Regular, c}; }
};

struct Optimiser {
    enum class Kind : uint32_t { SGD = 0, Adam = 1 };
    Kind kind = Kind::SGD;
    float v_coeff = 0.0f;    // SGD momentum | Adam second-moment decay
    float m_coeff = 0.0f;    // Adam first-moment decay
    float epsilon = 0.0f;    // Adam
    bool nesterov = false;   // SGD
    static Optimiser sgd(float v_coeff, bool nesterov) { return {Kind::SGD, v_coeff, 0.0f, 0.0f, nesterov}; }
    static Optimiser adam(float m_coeff, float v_coeff, float epsilon) {
        return {Kind::Adam, v_coeff, m_coeff, epsilon, false};
    }
    skl_optimiser to_c() const;
};

enum class LossFunc : uint32_t { MeanSquareLoss = 0, CrossEntropyLoss = 1, BinaryCrossEntropy = 2 };

// ---- configs (src/util/context.rs:11-85) -------------------------------------------
struct LayerInitConfig {
    Normalisation normalisation = Normalisation::Disabled;
    Activation activation = Activation::identity();
    Regularisation regularisation = Regularisation::none();
    float mask_coeff = 0.0f;
};

struct TrainContext {
    const Optimiser *optimiser;
    const Optimiser *norm_optimiser;
    size_t batch_size;
    float learn_rate;
    float grad_clamp;   // FLT_MAX turns clamping off
};

struct MultiLayerTrainContext {
    std::vector<Optimiser> optimisers;
    std::vector<Optimiser> norm_optimisers;
    size_t batch_size;
    float learn_rate;
    float grad_clamp;
    TrainContext get_train_context(size_t idx) const {
        return {&optimisers.at(idx), &norm_optimisers.at(idx), batch_size, learn_rate, grad_clamp};
    }
};

struct LossConfig {
    LossFunc loss_func;
    Activation activation;
};

// scramble_seed (src/util/core.rs:90-94): the dropout seed of a forward pass is
// scramble_seed(step, id of the layer's weight tensor).
uint32_t scramble_seed(uint32_t step, uint32_t layer_id);

// ---- GpuContext (src/io/device.rs:61-183) --------------------------------------------
class GpuContext {
  public:
    GpuContext() : GpuContext(0) {}                            // GpuContext::new
    explicit GpuContext(int32_t ordinal, uint32_t tile_dim = 16);   // with_device_index
    static GpuContext with_device_index(int32_t ordinal) { return GpuContext(ordinal); }
    ~GpuContext();
    GpuContext(const GpuContext &) = delete;
    GpuContext &operator=(const GpuContext &) = delete;
    GpuContext(GpuContext &&o) noexcept : ctx_(o.ctx_) { o.ctx_ = nullptr; }
    GpuContext &operator=(GpuContext &&o) noexcept;
    skl_ctx *raw() const { return ctx_; }
    void synchronize() const;

  private:
    skl_ctx *ctx_ = nullptr;
};

// ---- tensors (src/util/core.rs:414-693) ------------------------------------------------
// TENSOR_ID_COUNTER: every allocation (from_cpu_vector, zeros, fill, clone,
// cast) takes the next id, in program order.
size_t generate_unique_tensor_id();
size_t peek_tensor_id_counter();

template <class T, size_t R> class Tensor {
  public:
    typedef std::array<size_t, R> Shape;

    static Tensor from_cpu_vector(const GpuContext &ctx, const std::vector<T> &cpu_data, const Shape &shape);
    static Tensor zeros(const GpuContext &ctx, const Shape &shape);
    static Tensor fill(const GpuContext &ctx, const Shape &shape, T value);

    void broadcast(const GpuContext &ctx, T value);
    Tensor clone(const GpuContext &ctx) const;
    // Casts into a new tensor (new id); this tensor's buffer is released.
    template <class U> Tensor<U, R> cast(const GpuContext &ctx) &&;
    std::vector<T> download(const GpuContext &ctx) const;
    void free_and_sync(const GpuContext &ctx) &&;

    size_t get_id() const { return id_; }
    const Shape &get_shape() const { return shape_; }
    T *get_data() const { return data_; }
    size_t len() const;
    size_t rows() const { return shape_[0]; }
    size_t cols() const { return R > 1 ? shape_[R - 1] : 1; }

    Tensor() = default;
    ~Tensor();
    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;
    Tensor(Tensor &&o) noexcept { steal(o); }
    Tensor &operator=(Tensor &&o) noexcept;

  private:
    template <class, size_t> friend class Tensor;
    void steal(Tensor &o) noexcept;
    void release() noexcept;
    skl_ctx *ctx_ = nullptr;
    T *data_ = nullptr;
    Shape shape_{};
    size_t id_ = 0;
};
template <class T> using Tensor2D = Tensor<T, 2>;
template <class T> using Tensor1D = Tensor<T, 1>;

// ---- initialisers (src/util/function.rs:190-319) ----------------------------------------
// ChaCha8Rng (rand_chacha 0.9.0) seeded with rand_core 0.9.5's seed_from_u64
// (PCG32 expansion of the u64 seed into the 32-byte key), next_u32 walking the
// keystream words in order.
// PCG32's XSH-RR output function of a 64-bit LCG state (M. O'Neill, pcg-random.org).
uint32_t pcg32_xsh_rr(uint64_t state);
constexpr uint64_t PCG32_MULTIPLIER = 6364136223846793005ull;

class ChaCha8Rng {
  public:
    static ChaCha8Rng seed_from_u64(uint64_t seed);
    static ChaCha8Rng from_seed(const std::array<uint8_t, 32> &key);
    uint32_t next_u32();
    // One ChaCha block with `rounds` rounds (8 for ChaCha8; 20 is the RFC 7539
    // cipher), key words k, 64-bit block counter, zero stream id.
    static void block(const uint32_t k[8], uint64_t counter, int rounds, uint32_t out[16]);

  private:
    uint32_t key_[8] = {};
    uint64_t counter_ = 0;
    uint32_t buf_[16] = {};
    int pos_ = 16;
};

class InitFunc {
  public:
    virtual ~InitFunc() = default;
    // `len` values for a [fan_in x fan_out] weight, generated in f32 and
    // converted to T per value (T::from_f32 at function.rs:229).
    template <class T> std::vector<T> init(size_t fan_in, size_t fan_out, size_t len) {
        std::vector<float> v = init_f32(fan_in, fan_out, len);
        std::vector<T> out(v.size());
        for (size_t i = 0; i < v.size(); ++i) out[i] = PrecisionType<T>::from_f32(v[i]);
        return out;
    }
    virtual std::vector<float> init_f32(size_t fan_in, size_t fan_out, size_t len) = 0;
};

class InitXavierUniformFunc : public InitFunc {
  public:
    InitXavierUniformFunc(uint64_t seed, float factor) : rng_(ChaCha8Rng::seed_from_u64(seed)), factor_(factor) {}
    std::vector<float> init_f32(size_t fan_in, size_t fan_out, size_t len) override;
  private:
    ChaCha8Rng rng_;
    float factor_;
};
class InitXavierNormalFunc : public InitFunc {
  public:
    InitXavierNormalFunc(uint64_t seed, float factor) : rng_(ChaCha8Rng::seed_from_u64(seed)), factor_(factor) {}
    std::vector<float> init_f32(size_t fan_in, size_t fan_out, size_t len) override;
  private:
    ChaCha8Rng rng_;
    float factor_;
};
class InitHeUniformFunc : public InitFunc {
  public:
    InitHeUniformFunc(uint64_t seed, float factor) : rng_(ChaCha8Rng::seed_from_u64(seed)), factor_(factor) {}
    std::vector<float> init_f32(size_t fan_in, size_t fan_out, size_t len) override;
  private:
    ChaCha8Rng rng_;
    float factor_;
};
class InitHeNormalFunc : public InitFunc {
  public:
    InitHeNormalFunc(uint64_t seed, float factor) : rng_(ChaCha8Rng::seed_from_u64(seed)), factor_(factor) {}
    std::vector<float> init_f32(size_t fan_in, size_t fan_out, size_t len) override;
  private:
    ChaCha8Rng rng_;
    float factor_;
};
class InitZeroFunc : public InitFunc {
  public:
    InitZeroFunc(uint64_t = 0, float = 0.0f) {}
    std::vector<float> init_f32(size_t, size_t, size_t len) override { return std::vector<float>(len, 0.0f); }
};

// A device allocation that is not a Tensor (takes no tensor id).  Move-only.
class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    DeviceBuffer(const GpuContext &ctx, size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&o) noexcept : ctx_(o.ctx_), p_(o.p_) { o.p_ = nullptr; }
    DeviceBuffer &operator=(DeviceBuffer &&o) noexcept;
    void *get() const { return p_; }

  private:
    skl_ctx *ctx_ = nullptr;
    void *p_ = nullptr;
};

// ---- DenseBlock state (src/mlp.rs:14-262) -------------------------------------------------
template <class T> struct ParamState {
    Tensor2D<T> w, b;
    std::optional<Tensor2D<float>> master_w, master_b;        // fp16 blocks only
    std::optional<Tensor2D<float>> dv_w, dv_b, dm_w, dm_b;    // training only

    static ParamState new_linear(const GpuContext &ctx, const std::vector<T> &w_vec,
                                 const std::array<size_t, 2> &w_shape, const std::array<size_t, 2> &b_shape,
                                 bool is_training);
    static ParamState new_norm(const GpuContext &ctx, const std::array<size_t, 2> &shape, bool is_training);
    void validate() const;
};

template <class T> struct ForwardCache {
    Tensor2D<T> out, predrop_out, preact_out, centered_out, prenorm_out;
    Tensor1D<T> norm_rstd;   // max(max_batch_size, outputs) entries
    static ForwardCache create(const GpuContext &ctx, size_t max_batch_size, size_t outputs);
    template <class U> ForwardCache<U> cast(const GpuContext &ctx) &&;
};

// ---- DenseBlock (src/mlp.rs:265-888) -------------------------------------------------------
template <class T> class DenseBlock {
  public:
    static DenseBlock create(const GpuContext &ctx, bool is_training, size_t inputs, size_t outputs,
                             size_t max_batch_size, InitFunc &init);   // DenseBlock::new
    static DenseBlock new_with_config(const GpuContext &ctx, bool is_training, size_t inputs, size_t outputs,
                                      size_t max_batch_size, InitFunc &init, const LayerInitConfig &init_config);
    static DenseBlock from_tensors(const GpuContext &ctx, bool is_training, ParamState<T> linear_state,
                                   ParamState<T> norm_state, size_t max_batch_size,
                                   const LayerInitConfig &init_config);

    // forward (mlp.rs:548-580): returns this layer's output cache (valid until the next call)
    const Tensor2D<T> &forward(const GpuContext &ctx, const Tensor2D<T> &input, size_t batch_size,
                               bool use_dropout, size_t step) const;
    void compute_loss(const GpuContext &ctx, const Tensor2D<T> &target, const LossConfig &loss_config) const;
    void backward_output(const GpuContext &ctx, const Tensor2D<T> &input, const TrainContext &train_ctx,
                         size_t step) const;
    void backward_hidden(const GpuContext &ctx, const DenseBlock &next_layer, const Tensor2D<T> &input,
                         const TrainContext &train_ctx, size_t step) const;
    void reset_mask(const GpuContext &ctx);

    // getters (mlp.rs:429-470)
    const Tensor2D<T> &get_weights() const { return linear_state_.w; }
    const Tensor2D<T> &get_biases() const { return linear_state_.b; }
    const std::optional<Tensor2D<float>> &get_master_weights() const { return linear_state_.master_w; }
    const std::optional<Tensor2D<float>> &get_master_biases() const { return linear_state_.master_b; }
    const Tensor2D<float> &get_dv_weights() const { return need(linear_state_.dv_w, "dv_w"); }
    const Tensor2D<float> &get_dv_biases() const { return need(linear_state_.dv_b, "dv_b"); }
    const Tensor2D<float> &get_dm_weights() const { return need(linear_state_.dm_w, "dm_w"); }
    const Tensor2D<float> &get_dm_biases() const { return need(linear_state_.dm_b, "dm_b"); }
    const Tensor2D<T> &get_norm_weights() const { return norm_state_.w; }
    const Tensor2D<T> &get_norm_biases() const { return norm_state_.b; }
    const std::optional<Tensor2D<float>> &get_master_norm_weights() const { return norm_state_.master_w; }
    const std::optional<Tensor2D<float>> &get_master_norm_biases() const { return norm_state_.master_b; }
    const Tensor2D<float> &get_norm_weights_grad() const { return need(d_norm_w_, "d_norm_w"); }
    const Tensor2D<float> &get_norm_biases_grad() const { return need(d_norm_b_, "d_norm_b"); }
    const Tensor2D<float> &get_dv_norm_weights() const { return need(norm_state_.dv_w, "dv_norm_w"); }
    const Tensor2D<float> &get_dv_norm_biases() const { return need(norm_state_.dv_b, "dv_norm_b"); }
    const Tensor2D<float> &get_dm_norm_weights() const { return need(norm_state_.dm_w, "dm_norm_w"); }
    const Tensor2D<float> &get_dm_norm_biases() const { return need(norm_state_.dm_b, "dm_norm_b"); }
    const Tensor2D<T> &get_outputs() const { return cache_.out; }
    const Tensor2D<T> &get_predrop_outputs() const { return cache_.predrop_out; }
    const Tensor2D<T> &get_preact_outputs() const { return cache_.preact_out; }
    const Tensor2D<T> &get_centered_outputs() const { return cache_.centered_out; }
    const Tensor2D<T> &get_prenorm_outputs() const { return cache_.prenorm_out; }
    const Tensor1D<T> &get_norm_rstd() const { return cache_.norm_rstd; }
    const Tensor2D<float> &get_grads() const { return need(grad_, "grad"); }
    const Tensor2D<float> &get_delta_prenorm_out() const { return need(d_prenorm_out_, "d_prenorm_out"); }
    const Tensor2D<T> &get_masks() const { return mask_; }
    size_t get_max_batch_size() const { return max_batch_size_; }
    float get_mask_coeff() const { return mask_coeff_; }
    void set_mask_coeff(float v) { mask_coeff_ = v; }
    Normalisation get_normalisation() const { return normalisation_; }
    void set_normalisation(Normalisation v) { normalisation_ = v; }
    Activation get_activation() const { return activation_; }
    void set_activation(Activation v) { activation_ = v; }
    Regularisation get_regularisation() const { return regularisation_; }
    void set_regularisation(Regularisation v) { regularisation_ = v; }
    bool is_training_mode() const { return is_training_; }

    // The C descriptor of this block (every device pointer of the state above).
    skl_dense_desc desc() const;

    // Precision conversion (mlp.rs:835-888).  Consumes the block.
    DenseBlock<f16> convert_f16(const GpuContext &ctx) &&;
    DenseBlock<float> convert_f32(const GpuContext &ctx) &&;

    DenseBlock(DenseBlock &&) noexcept = default;
    DenseBlock &operator=(DenseBlock &&) noexcept = default;

  private:
    template <class> friend class DenseBlock;
    DenseBlock() = default;
    static const Tensor2D<float> &need(const std::optional<Tensor2D<float>> &t, const char *name);
    void alloc_dprenorm_h(const GpuContext &ctx);
    skl_train_ctx train_c(const TrainContext &t) const;

    ParamState<T> linear_state_;
    ParamState<T> norm_state_;
    ForwardCache<T> cache_;
    std::optional<Tensor2D<float>> grad_, d_prenorm_out_, d_norm_w_, d_norm_b_;
    Tensor2D<T> mask_;
    size_t max_batch_size_ = 0;
    Normalisation normalisation_ = Normalisation::Disabled;
    Activation activation_;
    Regularisation regularisation_;
    float mask_coeff_ = 0.0f;
    bool is_training_ = false;
    // fp16 training blocks: f16(d_prenorm), the MFMA operand of dW / dX.  An
    // internal buffer, not a Tensor: it takes no tensor id, so the ids (and
    // with them the dropout seeds) follow the reference's allocation sequence.
    DeviceBuffer d_prenorm_h_;
};

// ---- FeedForwardNetwork (src/ffn.rs:10-166) -------------------------------------------------
template <class T> class FeedForwardNetwork {
  public:
    FeedForwardNetwork(std::vector<DenseBlock<T>> layers, size_t inputs)
        : layers_(std::move(layers)), inputs_(inputs) {}
    // Every layer's output, in order (views into the layer caches).
    std::vector<const Tensor2D<T> *> forward(const GpuContext &ctx, const Tensor2D<T> &input, size_t batch_size,
                                             bool use_dropout, size_t step) const;
    // A copy of the last layer's output for host input data.
    Tensor2D<T> forward_raw(const GpuContext &ctx, const std::vector<T> &raw_pixels, size_t batch_size,
                            bool use_dropout, size_t step) const;
    // compute_loss + backward_output on the last layer, then backward_hidden
    // downwards: each layer's weights are updated before the layer below
    // propagates through them (ffn.rs:113-166).
    void backward(const GpuContext &ctx, const std::vector<const Tensor2D<T> *> &outputs,
                  const Tensor2D<T> &target, const Tensor2D<T> &input, const LossConfig &loss_config,
                  const MultiLayerTrainContext &train_ctx, size_t step) const;
    const std::vector<DenseBlock<T>> &get_layers() const { return layers_; }
    std::vector<DenseBlock<T>> &get_layers() { return layers_; }
    size_t len() const { return layers_.size(); }

  private:
    std::vector<DenseBlock<T>> layers_;
    size_t inputs_;
};

}  // namespace soklyn
