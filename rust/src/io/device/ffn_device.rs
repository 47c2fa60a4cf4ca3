//! The DenseBlock device methods of `GpuContext` on the MI355X build
//! (replaces src/io/device/ffn_device.rs:12-439).  Each keeps the reference's
//! signature and `Result<(), Error>`; the checks, launches and synchronisation
//! are the C ABI's (include/soklyn_hip.h).
use std::os::raw::c_void;

use super::hip_ffi::*;
use super::{check, GpuContext};
use crate::core::Tensor2D;
use crate::log::Error;
use crate::{Activation, DenseBlock, LossFunc, Optimiser, PrecisionType, Regularisation, TrainContext};

fn ptr<T>(t: &Tensor2D<T>) -> *mut c_void {
    t.get_data().as_ptr()
}

fn ptr_f32(t: &Tensor2D<f32>) -> *mut f32 {
    t.get_data().as_ptr() as *mut f32
}

fn opt_f32(t: Option<&Tensor2D<f32>>) -> *mut f32 {
    t.map_or(std::ptr::null_mut(), ptr_f32)
}

/// The C descriptor of a block: the device pointers of its tensors and its
/// configuration.  Tensors that exist only while training (moments, grads,
/// dNorm, the fp16 copy of d_prenorm) are null on an inference block, masters
/// on an fp32 block.
pub(crate) fn desc<T: PrecisionType>(block: &DenseBlock<T>, activation: &Activation) -> Result<SklDenseDesc, Error> {
    let w = block.get_weights();
    let training = block.is_training_mode();
    let regularisation = block.get_regularisation();
    // ffn_device.rs:274-279
    let regu_coeff = match regularisation {
        Regularisation::None => 0.0,
        Regularisation::L1Regular { regu_coeff } | Regularisation::L2Regular { regu_coeff } => *regu_coeff,
    };
    let train = |f: &dyn Fn() -> *mut f32| if training { f() } else { std::ptr::null_mut() };
    Ok(SklDenseDesc {
        dtype: if T::precision() == crate::Precision::FP16 { SKL_F16 } else { SKL_F32 },
        inputs: u32::try_from(w.rows())?,
        outputs: u32::try_from(w.cols())?,
        max_batch: u32::try_from(block.get_max_batch_size())?,
        norm: u32::try_from(block.get_normalisation().ordinal())?,
        act: u32::try_from(activation.ordinal())?,
        leaky: match activation {
            Activation::LeakyReLU { coeff } => *coeff,
            _ => 0.0,
        },
        mask_coeff: block.get_mask_coeff(),
        regularisation: u32::try_from(regularisation.ordinal())?,
        regu_coeff,
        is_training: u32::from(training),
        reserved0: 0,
        w: ptr(w),
        b: ptr(block.get_biases()),
        norm_w: ptr(block.get_norm_weights()),
        norm_b: ptr(block.get_norm_biases()),
        master_w: opt_f32(block.get_master_weights()),
        master_b: opt_f32(block.get_master_biases()),
        master_norm_w: opt_f32(block.get_master_norm_weights()),
        master_norm_b: opt_f32(block.get_master_norm_biases()),
        dv_w: train(&|| ptr_f32(block.get_dv_weights())),
        dv_b: train(&|| ptr_f32(block.get_dv_biases())),
        dm_w: train(&|| ptr_f32(block.get_dm_weights())),
        dm_b: train(&|| ptr_f32(block.get_dm_biases())),
        dv_norm_w: train(&|| ptr_f32(block.get_dv_norm_weights())),
        dv_norm_b: train(&|| ptr_f32(block.get_dv_norm_biases())),
        dm_norm_w: train(&|| ptr_f32(block.get_dm_norm_weights())),
        dm_norm_b: train(&|| ptr_f32(block.get_dm_norm_biases())),
        out: ptr(block.get_outputs()),
        predrop: ptr(block.get_predrop_outputs()),
        preact: ptr(block.get_preact_outputs()),
        centered: ptr(block.get_centered_outputs()),
        prenorm: ptr(block.get_prenorm_outputs()),
        norm_rstd: block.get_norm_rstd().get_data().as_ptr(),
        mask: ptr(block.get_masks()),
        grad: train(&|| ptr_f32(block.get_grads())),
        d_prenorm: train(&|| ptr_f32(block.get_delta_prenorm_out())),
        d_norm_w: train(&|| ptr_f32(block.get_norm_weights_grad())),
        d_norm_b: train(&|| ptr_f32(block.get_norm_biases_grad())),
        // fp16 training blocks only; a raw buffer, not a Tensor (it takes no tensor id)
        d_prenorm_h: block.get_delta_prenorm_half().map_or(std::ptr::null_mut(), |b| b.as_ptr()),
    })
}

fn optimiser(o: &Optimiser) -> Result<SklOptimiser, Error> {
    // ffn_device.rs:257-267
    Ok(match o {
        Optimiser::SGD { v_coeff, nesterov } => SklOptimiser {
            kind: u32::try_from(o.ordinal())?,
            beta1: *v_coeff,
            beta2: 0.0,
            epsilon: 0.0,
            nesterov: u32::from(*nesterov),
        },
        Optimiser::Adam { m_coeff, v_coeff, epsilon } => SklOptimiser {
            kind: u32::try_from(o.ordinal())?,
            beta1: *m_coeff,
            beta2: *v_coeff,
            epsilon: *epsilon,
            nesterov: 0,
        },
    })
}

fn train(t: &TrainContext) -> Result<SklTrainCtx, Error> {
    Ok(SklTrainCtx {
        optimiser: optimiser(t.optimiser)?,
        norm_optimiser: optimiser(t.norm_optimiser)?,
        batch_size: u32::try_from(t.batch_size)?,
        learn_rate: t.learn_rate,
        grad_clamp: t.grad_clamp,
    })
}

impl GpuContext {
    /// ffn_device.rs:12-139: Z = in.W (+b) -> norm -> act -> dropout, with the
    /// dropout seed scramble_seed(step, W.id) (ffn_device.rs:26-29).
    pub(crate) fn gpu_forward_pass<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        input: &Tensor2D<T>,
        batch_size: usize,
        use_dropout: bool,
        step: usize,
    ) -> Result<(), Error> {
        let seed = unsafe {
            skl_scramble_seed(u32::try_from(step)?, u32::try_from(cur_layer.get_weights().get_id())?)
        };
        let d = desc(cur_layer, cur_layer.get_activation())?;
        check(unsafe {
            skl_dense_forward(self.raw(), &d, ptr(input), u32::try_from(input.rows())?, u32::try_from(input.cols())?,
                              u32::try_from(batch_size)?, u32::from(use_dropout), seed)
        })
    }

    /// ffn_device.rs:141-231: zero dNorm, softmax in place on `out` when the loss
    /// activation is Softmax, then the loss delta and norm gradient x LOSS_SCALE.
    pub(crate) fn gpu_compute_output_layer_error<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        target: &Tensor2D<T>,
        err_mode: LossFunc,
        activation: Activation,
    ) -> Result<(), Error> {
        let d = desc(cur_layer, cur_layer.get_activation())?;
        let leaky = match activation {
            Activation::LeakyReLU { coeff } => coeff,
            _ => 0.0,
        };
        check(unsafe {
            skl_dense_output_error(self.raw(), &d, ptr(target), u32::try_from(target.rows())?,
                                   u32::try_from(target.cols())?, err_mode as u32,
                                   u32::try_from(activation.ordinal())?, leaky)
        })
    }

    /// ffn_device.rs:233-358: dW, db and the norm-parameter sums, then the
    /// optimiser step on W, b and the norm parameters.
    pub(crate) fn gpu_backward_pass<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        input: &Tensor2D<T>,
        train_ctx: &TrainContext,
        step: usize,
    ) -> Result<(), Error> {
        let d = desc(cur_layer, cur_layer.get_activation())?;
        let t = train(train_ctx)?;
        check(unsafe {
            skl_dense_backward(self.raw(), &d, ptr(input), u32::try_from(input.rows())?,
                               u32::try_from(input.cols())?, &t, u32::try_from(step)?)
        })
    }

    /// ffn_device.rs:360-439: the hidden error of cur from next (with cur's
    /// activation `activation`), then gpu_backward_pass(cur).
    pub(crate) fn gpu_hidden_layer_backward_pass<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        next_layer: &DenseBlock<T>,
        input: &Tensor2D<T>,
        activation: Activation,
        train_ctx: &TrainContext,
        step: usize,
    ) -> Result<(), Error> {
        let cur = desc(cur_layer, &activation)?;
        let next = desc(next_layer, next_layer.get_activation())?;
        let t = train(train_ctx)?;
        check(unsafe {
            skl_dense_backward_hidden(self.raw(), &cur, &next, ptr(input), u32::try_from(input.rows())?,
                                      u32::try_from(input.cols())?, &t, u32::try_from(step)?)
        })
    }
}

// Not on the reference's DenseBlock path but exported by the C ABI: the input
// gradient of the first layer and the error from an external upstream sum, for
// callers that chain a DenseBlock after a non-DenseBlock layer.
impl GpuContext {
    pub(crate) fn gpu_input_grad<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        batch_size: usize,
        dx: &Tensor2D<f32>,
    ) -> Result<(), Error> {
        let d = desc(cur_layer, cur_layer.get_activation())?;
        check(unsafe { skl_dense_input_grad(self.raw(), &d, u32::try_from(batch_size)?, ptr_f32(dx)) })
    }

    pub(crate) fn gpu_error_from_sum<T: PrecisionType>(
        &self,
        cur_layer: &DenseBlock<T>,
        upstream: &Tensor2D<f32>,
        batch_size: usize,
    ) -> Result<(), Error> {
        let d = desc(cur_layer, cur_layer.get_activation())?;
        check(unsafe {
            skl_dense_error_from_sum(self.raw(), &d, ptr_f32(upstream) as *const f32, u32::try_from(batch_size)?)
        })
    }
}
