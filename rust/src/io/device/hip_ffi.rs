//! Declarations of the C ABI in include/soklyn_hip.h, for the crate's device
//! layer.  Every struct is `#[repr(C)]` with the header's field order and
//! types, and every function has the header's parameter types; the CPU test
//! tests/test_rust_ffi_layout.py parses this file and checks both against the
//! header (names, parameter and return types, and each field's offset and size
//! against the C compiler's offsetof / sizeof).
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_void};

// ---- status codes (include/soklyn_hip.h; one per crate::log::Error variant) ----
pub const SKL_OK: i32 = 0;
pub const SKL_ERR_INVALID_CONFIGURATION: i32 = -1;
pub const SKL_ERR_TRAINING_MODE_REQUIRED: i32 = -2;
pub const SKL_ERR_ALLOCATION_LIMIT: i32 = -3;
pub const SKL_ERR_MISMATCHED_DIMENSIONS: i32 = -4;
pub const SKL_ERR_INVALID_BATCH_SIZE: i32 = -5;
pub const SKL_ERR_HARDWARE_CONSTRAINT: i32 = -6;
pub const SKL_ERR_TRY_FROM_INT: i32 = -7;
pub const SKL_ERR_NULL_POINTER: i32 = -8;
pub const SKL_ERR_UNSUPPORTED_CAST: i32 = -9;
pub const SKL_ERR_NO_DEVICE: i32 = -10;

// ---- mode codes (the reference's ordinals, src/util/function.rs) ----
pub const SKL_F32: u32 = 0;
pub const SKL_F16: u32 = 1;

/// The context (opaque; created by skl_ctx_create, one per GpuContext).
#[repr(C)]
pub struct SklCtx {
    _opaque: [u8; 0],
}

/// One DenseBlock's device state: the device pointers of its tensors and its
/// configuration.  Pointers a block does not have are null.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct SklDenseDesc {
    pub dtype: u32,
    pub inputs: u32,
    pub outputs: u32,
    pub max_batch: u32,
    pub norm: u32,
    pub act: u32,
    pub leaky: f32,
    pub mask_coeff: f32,
    pub regularisation: u32,
    pub regu_coeff: f32,
    pub is_training: u32,
    pub reserved0: u32,
    pub w: *mut c_void,
    pub b: *mut c_void,
    pub norm_w: *mut c_void,
    pub norm_b: *mut c_void,
    pub master_w: *mut f32,
    pub master_b: *mut f32,
    pub master_norm_w: *mut f32,
    pub master_norm_b: *mut f32,
    pub dv_w: *mut f32,
    pub dv_b: *mut f32,
    pub dm_w: *mut f32,
    pub dm_b: *mut f32,
    pub dv_norm_w: *mut f32,
    pub dv_norm_b: *mut f32,
    pub dm_norm_w: *mut f32,
    pub dm_norm_b: *mut f32,
    pub out: *mut c_void,
    pub predrop: *mut c_void,
    pub preact: *mut c_void,
    pub centered: *mut c_void,
    pub prenorm: *mut c_void,
    pub norm_rstd: *mut c_void,
    pub mask: *mut c_void,
    pub grad: *mut f32,
    pub d_prenorm: *mut f32,
    pub d_norm_w: *mut f32,
    pub d_norm_b: *mut f32,
    pub d_prenorm_h: *mut c_void,
}

/// Optimiser as gpu_backward_pass extracts it (ffn_device.rs:257-267).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct SklOptimiser {
    pub kind: u32,
    pub beta1: f32,
    pub beta2: f32,
    pub epsilon: f32,
    pub nesterov: u32,
}

/// TrainContext (context.rs:39-45).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct SklTrainCtx {
    pub optimiser: SklOptimiser,
    pub norm_optimiser: SklOptimiser,
    pub batch_size: u32,
    pub learn_rate: f32,
    pub grad_clamp: f32,
}

#[link(name = "soklyn_hip")]
extern "C" {
    pub fn skl_ctx_create(ordinal: i32, tile_dim: u32, out: *mut *mut SklCtx) -> i32;
    pub fn skl_ctx_destroy(ctx: *mut SklCtx) -> i32;
    pub fn skl_ctx_set_sync(ctx: *mut SklCtx, sync_each_call: u32) -> i32;
    pub fn skl_ctx_set_stream(ctx: *mut SklCtx, hip_stream: *mut c_void) -> i32;
    pub fn skl_ctx_stream(ctx: *mut SklCtx) -> *mut c_void;
    pub fn skl_synchronize(ctx: *mut SklCtx) -> i32;
    pub fn skl_status_string(status: i32) -> *const c_char;
    pub fn skl_ctx_time_next_gemm(ctx: *mut SklCtx, start_event: *mut c_void, stop_event: *mut c_void) -> i32;

    pub fn skl_malloc(ctx: *mut SklCtx, ptr: *mut *mut c_void, bytes: usize) -> i32;
    pub fn skl_free(ctx: *mut SklCtx, ptr: *mut c_void) -> i32;
    pub fn skl_memcpy_h2d(ctx: *mut SklCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;
    pub fn skl_memcpy_d2h(ctx: *mut SklCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;
    pub fn skl_memcpy_d2d(ctx: *mut SklCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;

    pub fn skl_fill(ctx: *mut SklCtx, dst: *mut c_void, dtype: u32, v: f32, n: usize) -> i32;
    pub fn skl_cast(ctx: *mut SklCtx, src: *const c_void, src_dtype: u32, dst: *mut c_void, dst_dtype: u32,
                    n: usize) -> i32;
    pub fn skl_scramble_seed(step: u32, layer_id: u32) -> u32;

    pub fn skl_dense_forward(ctx: *mut SklCtx, blk: *const SklDenseDesc, input: *const c_void, in_rows: u32,
                             in_cols: u32, batch: u32, use_dropout: u32, seed: u32) -> i32;
    pub fn skl_dense_output_error(ctx: *mut SklCtx, blk: *const SklDenseDesc, target: *const c_void,
                                  target_rows: u32, target_cols: u32, loss: u32, act: u32, leaky: f32) -> i32;
    pub fn skl_dense_hidden_error(ctx: *mut SklCtx, cur: *const SklDenseDesc, next: *const SklDenseDesc,
                                  batch: u32) -> i32;
    pub fn skl_dense_backward(ctx: *mut SklCtx, blk: *const SklDenseDesc, input: *const c_void, in_rows: u32,
                              in_cols: u32, train: *const SklTrainCtx, step: u32) -> i32;
    pub fn skl_dense_backward_hidden(ctx: *mut SklCtx, cur: *const SklDenseDesc, next: *const SklDenseDesc,
                                     input: *const c_void, in_rows: u32, in_cols: u32, train: *const SklTrainCtx,
                                     step: u32) -> i32;
    pub fn skl_dense_error_from_sum(ctx: *mut SklCtx, blk: *const SklDenseDesc, s: *const f32, batch: u32) -> i32;
    pub fn skl_dense_error_from_sum_noalloc(ctx: *mut SklCtx, blk: *const SklDenseDesc, s: *const f32,
                                            batch: u32) -> i32;
    pub fn skl_dense_input_grad(ctx: *mut SklCtx, blk: *const SklDenseDesc, batch: u32, dx: *mut f32) -> i32;
}
