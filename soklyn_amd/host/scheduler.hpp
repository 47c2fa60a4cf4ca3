// scheduler.hpp — learning-rate schedulers of the host API (src/util/scheduler.rs:1-231).
//
// Host-only, f32 arithmetic in the reference's evaluation order (the host build
// uses -ffp-contract=off, so no expression is fused), step counters in size_t.
// A caller passes get_learning_rate() (or step()'s result) as
// TrainContext::learn_rate of the next training step.
#pragma once

#include <cfloat>
#include <cmath>
#include <cstddef>
#include <stdexcept>

namespace soklyn {

// CosineDecayLR (scheduler.rs:3-79): linear warm-up from min_lr to max_lr over
// warmup_steps, then min + 0.5 (max - min) (1 + cos(pi progress)) over the
// remaining total_step - warmup_steps steps.  Past total_step the cosine keeps
// going (no clamp), as in the reference.
class CosineDecayLR {
  public:
    CosineDecayLR(float min_lr, float max_lr, size_t total_step, size_t warmup_steps)
        : min_lr_(min_lr), max_lr_(max_lr), cur_lr_(min_lr), cur_step_(0), total_step_(total_step),
          warmup_steps_(warmup_steps) {
        update_lr();
    }
    void reset() {
        cur_step_ = 0;
        update_lr();
    }
    float get_learning_rate() const { return cur_lr_; }
    float step() {
        cur_step_ += 1;
        update_lr();
        return cur_lr_;
    }
    size_t current_step() const { return cur_step_; }

  private:
    // scheduler.rs:38-57
    void update_lr() {
        if (cur_step_ < warmup_steps_) {
            const float progress = static_cast<float>(cur_step_) / static_cast<float>(warmup_steps_);
            cur_lr_ = min_lr_ + progress * (max_lr_ - min_lr_);
        } else {
            // usize subtraction: total_step < warmup_steps underflows in the reference
            if (total_step_ < warmup_steps_)
                throw std::overflow_error("CosineDecayLR: total_step is smaller than warmup_steps");
            const size_t decay_step = cur_step_ - warmup_steps_;
            const size_t decay_total = total_step_ - warmup_steps_;
            if (decay_total == 0) {
                cur_lr_ = min_lr_;
                return;
            }
            const float progress = static_cast<float>(decay_step) / static_cast<float>(decay_total);
            const float pi = 3.14159265358979323846f;   // std::f32::consts::PI
            cur_lr_ = min_lr_ + 0.5f * (max_lr_ - min_lr_) * (1.0f + std::cos(progress * pi));
        }
    }
    float min_lr_, max_lr_, cur_lr_;
    size_t cur_step_, total_step_, warmup_steps_;
};

// ExponentialLR (scheduler.rs:81-120): cur *= factor per step.
class ExponentialLR {
  public:
    ExponentialLR(float lr_initial, float lr_factor) : ori_lr_(lr_initial), cur_lr_(lr_initial), lr_factor_(lr_factor) {}
    void reset() { cur_lr_ = ori_lr_; }
    float get_learning_rate() const { return cur_lr_; }
    float step() {
        cur_lr_ *= lr_factor_;
        return cur_lr_;
    }

  private:
    float ori_lr_, cur_lr_, lr_factor_;
};

// SchedulerMode (scheduler.rs:136-143)
enum class SchedulerMode { Minimize, Maximize };

// ReduceLROnPlateauScheduler (scheduler.rs:122-231): after `patience`
// consecutive steps without a strict improvement of the test value, the rate is
// multiplied by lr_factor (floored at min_lr) and the count restarts.  NaN test
// values are ignored.  The rate is 0 until reset(learning_rate) sets it, as in
// the reference.
class ReduceLROnPlateauScheduler {
  public:
    ReduceLROnPlateauScheduler(size_t patience, SchedulerMode mode, float lr_factor, float min_lr)
        : best_val_(initial_best(mode)), mode_(mode), min_lr_(min_lr), cur_lr_(0.0f), lr_factor_(lr_factor),
          timer_(0), patience_(patience) {
        if (patience == 0) throw std::invalid_argument("Patience must be non-zero.");   // scheduler.rs:159
    }
    void reset(float learning_rate) {
        cur_lr_ = learning_rate;
        timer_ = 0;
        best_val_ = initial_best(mode_);
    }
    float get_learning_rate() const { return cur_lr_; }
    float step(float test_val) {
        if (std::isnan(test_val)) return cur_lr_;
        const bool improved = mode_ == SchedulerMode::Maximize ? test_val > best_val_ : test_val < best_val_;
        if (improved) {
            best_val_ = test_val;
            timer_ = 0;
        } else {
            timer_ += 1;
            if (timer_ == patience_) {
                timer_ = 0;
                cur_lr_ *= lr_factor_;
                cur_lr_ = std::fmax(cur_lr_, min_lr_);   // f32::max: a NaN operand yields the other
            }
        }
        return cur_lr_;
    }

  private:
    // f32::MIN is the most negative finite value, f32::MAX the largest
    static float initial_best(SchedulerMode m) { return m == SchedulerMode::Maximize ? -FLT_MAX : FLT_MAX; }
    float best_val_;
    SchedulerMode mode_;
    float min_lr_, cur_lr_, lr_factor_;
    size_t timer_, patience_;
};

}  // namespace soklyn
