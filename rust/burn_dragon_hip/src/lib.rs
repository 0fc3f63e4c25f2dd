//! burn_dragon_hip: the MI355X (gfx950) HIP path of burn_dragon's recurrent
//! attention, behind the custom-op surface of `burn_dragon_kernel`
//! (crates/burn_dragon_kernel/src/lib.rs:40-56), so that `burn_dragon_core`'s
//! call sites (sequence_dispatch.rs:10,111,119,154,160) switch by import.
//!
//! The compute is libbdh_hip (include/bdh_hip.h, bound in [`ffi`]).  Device
//! pointers and the stream come from the backend through [`HipHandles`],
//! which a maintainer implements for burn-cubecl's HIP runtime (the
//! resource's base pointer plus offset, and the client's stream).  Every op
//! keeps the reference's `Option` convention: `None` means "use the Burn-op
//! reference" (any non-OK status of the C ABI).
//!
//! This crate is source only in this repository: the build image has no Rust
//! toolchain.  tests/test_rust_ffi.py checks [`ffi`] against the C header.

pub mod ffi;

use burn::tensor::backend::Backend;
use burn::tensor::{DType, Tensor};
use std::ffi::CString;
use std::os::raw::c_void;

/// Device memory and stream of a Burn backend running on a HIP device.
pub trait HipHandles: Backend {
    /// Device address of the tensor's first element (row-major contiguous).
    fn device_ptr<const D: usize>(tensor: &Tensor<Self, D>) -> *mut c_void;
    /// The hipStream_t the backend launches on for `device`.
    fn hip_stream(device: &Self::Device) -> *mut c_void;
    /// True when the backend is the HIP runtime on a gfx950 device.
    fn is_hip(device: &Self::Device) -> bool;
}

/// recurrent.rs:65-69.
#[derive(Debug, Clone)]
pub struct RecurrentAttentionOutput<B: Backend> {
    pub context: Tensor<B, 4>,
    pub rho: Tensor<B, 4>,
}

/// recurrent.rs:95-149: six integers, nothing uploaded to the device.
#[derive(Debug, Clone, Copy)]
pub struct CompiledRecurrentAttentionPlan {
    pub c_plan: ffi::bdh_recurrent_plan,
}

impl CompiledRecurrentAttentionPlan {
    pub fn new(batch: usize, heads: usize, value_heads: usize, time: usize, latent: usize,
               embd: usize) -> Option<Self> {
        let mut p = ffi::bdh_recurrent_plan::default();
        let st = unsafe {
            ffi::bdh_recurrent_plan_new(batch as i64, heads as i64, value_heads as i64,
                                        time as i64, latent as i64, embd as i64, &mut p)
        };
        (st == ffi::BDH_OK).then_some(Self { c_plan: p })
    }

    pub fn matches<B: Backend>(&self, query: &Tensor<B, 4>, value: &Tensor<B, 4>) -> bool {
        let [b, h, t, n] = query.dims();
        let [bv, hv, tv, d] = value.dims();
        let p = &self.c_plan;
        [b, h, t, n] == [p.batch as usize, p.heads as usize, p.time as usize, p.latent as usize]
            && [bv, hv, tv, d]
                == [p.batch as usize, p.value_heads as usize, p.time as usize, p.embd as usize]
    }
}

/// recurrent.rs:151-173, exported as supports_recurrent_backend.
pub fn supports_backend<B: HipHandles>(device: &B::Device) -> bool {
    B::is_hip(device) && unsafe { ffi::bdh_supports_backend() } == 1
}

fn dtype_code(dtype: DType) -> Option<i32> {
    match dtype {
        DType::F32 => Some(ffi::BDH_F32),
        DType::BF16 => Some(ffi::BDH_BF16),
        _ => None,
    }
}

fn ptr_or_null<B: HipHandles, const D: usize>(t: Option<&Tensor<B, D>>) -> *mut c_void {
    t.map_or(std::ptr::null_mut(), |x| B::device_ptr(x))
}

/// recurrent.rs:221-359.  `query` is the rotated query; the caller's rho is
/// only read (the reference's private copy, recurrent.rs:259): the state is
/// written to a fresh tensor.
pub fn try_fused_recurrent_attention_wgpu_with_plan<B: HipHandles>(
    query: &Tensor<B, 4>, value: &Tensor<B, 4>, rho: Option<&Tensor<B, 4>>,
    decay: Option<&Tensor<B, 1>>, plan: &CompiledRecurrentAttentionPlan,
) -> Option<RecurrentAttentionOutput<B>> {
    let device = query.device();
    if !supports_backend::<B>(&device) || !plan.matches(query, value) {
        return None;
    }
    let dtype = dtype_code(query.dtype())?;
    if value.dtype() != query.dtype() {
        return None;
    }
    let [b, h, t, n] = query.dims();
    let d = value.dims()[3];
    let rho_in = rho.filter(|r| r.dims() == [b, h, n, d]); // recurrent.rs:243-246
    let decay = decay.filter(|x| x.dims() == [h]); // recurrent.rs:247-250
    let context = Tensor::<B, 4>::empty([b, h, t, d], &device);
    let rho_out = Tensor::<B, 4>::empty([b, h, n, d], &device);
    let st = unsafe {
        ffi::bdh_recurrent_attention_fwd(
            &plan.c_plan, dtype, B::device_ptr(query), B::device_ptr(value),
            ptr_or_null(rho_in) as *const f32, ptr_or_null(decay) as *const f32,
            B::device_ptr(&context) as *mut f32, B::device_ptr(&rho_out) as *mut f32, 0,
            B::hip_stream(&device))
    };
    (st == ffi::BDH_OK).then(|| RecurrentAttentionOutput { context, rho: rho_out })
}

/// recurrent.rs:175-219 (plan built per call).
pub fn try_fused_recurrent_attention_wgpu<B: HipHandles>(
    query: &Tensor<B, 4>, value: &Tensor<B, 4>, rho: Option<&Tensor<B, 4>>,
    decay: Option<&Tensor<B, 1>>,
) -> Option<RecurrentAttentionOutput<B>> {
    let [b, h, t, n] = query.dims();
    let [_, hv, _, d] = value.dims();
    let plan = CompiledRecurrentAttentionPlan::new(b, h, hv, t, n, d)?;
    try_fused_recurrent_attention_wgpu_with_plan(query, value, rho, decay, &plan)
}

/// The opt-in RoPE-fused call replacing rotate_positions[_fixed] + the op in
/// DragonModel::recurrent_attention_with_plan (sequence_dispatch.rs:97-111).
pub fn try_fused_recurrent_attention_rope<B: HipHandles>(
    x: &Tensor<B, 4>, value: &Tensor<B, 4>, rho: Option<&Tensor<B, 4>>,
    decay: Option<&Tensor<B, 1>>, position: usize, fixed: bool, theta: f32,
    plan: &CompiledRecurrentAttentionPlan,
) -> Option<RecurrentAttentionOutput<B>> {
    let device = x.device();
    if !supports_backend::<B>(&device) || !plan.matches(x, value) {
        return None;
    }
    let dtype = dtype_code(x.dtype())?;
    let [b, h, t, n] = x.dims();
    let d = value.dims()[3];
    let rho_in = rho.filter(|r| r.dims() == [b, h, n, d]);
    let decay = decay.filter(|z| z.dims() == [h]);
    let rope = ffi::bdh_rope {
        mode: if fixed { ffi::BDH_ROPE_FIXED } else { ffi::BDH_ROPE_SEQUENTIAL },
        _pad: 0,
        pos0: position as i64,
        theta,
    };
    let context = Tensor::<B, 4>::empty([b, h, t, d], &device);
    let rho_out = Tensor::<B, 4>::empty([b, h, n, d], &device);
    let st = unsafe {
        ffi::bdh_recurrent_attention_rope_fwd(
            &plan.c_plan, dtype, B::device_ptr(x), B::device_ptr(value),
            ptr_or_null(rho_in) as *const f32, ptr_or_null(decay) as *const f32, &rope,
            B::device_ptr(&context) as *mut f32, B::device_ptr(&rho_out) as *mut f32, 0,
            B::hip_stream(&device))
    };
    (st == ffi::BDH_OK).then(|| RecurrentAttentionOutput { context, rho: rho_out })
}

/// dense_causal_attention.rs:162-261: ctx = tril(-1)(Q Q^T * decay^(r-c)) V.
pub fn try_fused_dense_causal_attention_wgpu<B: HipHandles>(
    query: &Tensor<B, 4>, value: &Tensor<B, 4>, decay: &Tensor<B, 1>,
) -> Option<Tensor<B, 4>> {
    let device = query.device();
    let [b, h, t, n] = query.dims();
    let [_, hv, _, d] = value.dims();
    if !supports_backend::<B>(&device) || t > 1024 || decay.dims() != [h] {
        return None; // dense_causal_attention.rs:179-214
    }
    let plan = CompiledRecurrentAttentionPlan::new(b, h, hv, t, n, d)?;
    let dtype = dtype_code(query.dtype())?;
    let context = Tensor::<B, 4>::empty([b, h, t, d], &device);
    let st = unsafe {
        ffi::bdh_dense_causal_attention_fwd(
            &plan.c_plan, dtype, B::device_ptr(query), B::device_ptr(value),
            B::device_ptr(decay) as *const f32, B::device_ptr(&context) as *mut f32,
            B::hip_stream(&device))
    };
    (st == ffi::BDH_OK).then_some(context)
}

/// dense_causal_attention/backward_runtime.rs:5-14.
#[derive(Debug, Clone)]
pub struct DenseCausalAttentionVjp<B: Backend> {
    pub grad_query: Tensor<B, 4>,
    pub grad_value: Tensor<B, 4>,
    pub grad_decay: Tensor<B, 1>,
    pub grad_initial_rho: Option<Tensor<B, 4>>,
}

/// dense_causal_attention/backward_runtime.rs:36-148 (f32).
pub fn dense_causal_attention_vjp_with_initial_rho<B: HipHandles>(
    grad_output: Tensor<B, 4>, query: Tensor<B, 4>, value: Tensor<B, 4>, decay: Tensor<B, 1>,
    initial_rho: Option<Tensor<B, 4>>,
) -> Option<DenseCausalAttentionVjp<B>> {
    let device = query.device();
    let [b, h, t, n] = query.dims();
    let [_, hv, _, d] = value.dims();
    if !supports_backend::<B>(&device) || query.dtype() != DType::F32 {
        return None;
    }
    let plan = CompiledRecurrentAttentionPlan::new(b, h, hv, t, n, d)?;
    let grad_query = Tensor::<B, 4>::empty([b, h, t, n], &device);
    let grad_value = Tensor::<B, 4>::empty([b, hv, t, d], &device);
    let grad_decay = Tensor::<B, 1>::empty([h], &device);
    let grad_rho = initial_rho.as_ref().map(|_| Tensor::<B, 4>::empty([b, h, n, d], &device));
    let st = unsafe {
        ffi::bdh_dense_causal_attention_vjp(
            &plan.c_plan, B::device_ptr(&query) as *const f32, B::device_ptr(&value) as *const f32,
            B::device_ptr(&decay) as *const f32, ptr_or_null(initial_rho.as_ref()) as *const f32,
            B::device_ptr(&grad_output) as *const f32, B::device_ptr(&grad_query) as *mut f32,
            B::device_ptr(&grad_value) as *mut f32, B::device_ptr(&grad_decay) as *mut f32,
            ptr_or_null(grad_rho.as_ref()) as *mut f32, B::hip_stream(&device))
    };
    (st == ffi::BDH_OK).then(|| DenseCausalAttentionVjp {
        grad_query,
        grad_value,
        grad_decay,
        grad_initial_rho: grad_rho,
    })
}

/// dense_causal_attention/backward_runtime.rs:16-27.
pub fn dense_causal_attention_vjp<B: HipHandles>(
    grad_output: Tensor<B, 4>, query: Tensor<B, 4>, value: Tensor<B, 4>, decay: Tensor<B, 1>,
) -> Option<DenseCausalAttentionVjp<B>> {
    dense_causal_attention_vjp_with_initial_rho(grad_output, query, value, decay, None)
}

/// profiling.rs:3-16 field names.
pub use ffi::bdh_profile_snapshot as KernelProfileSnapshot;

/// recurrent.rs:57-59.
pub fn recurrent_profile_reset() {
    unsafe { ffi::bdh_profile_reset() }
}

/// recurrent.rs:61-63.
pub fn recurrent_profile_snapshot() -> KernelProfileSnapshot {
    let mut s = KernelProfileSnapshot::default();
    unsafe { ffi::bdh_profile_get(&mut s) };
    s
}

/// Saves a model's streaming state (position and each layer's rho) through
/// bdh_state_record_save: the StreamingRuntimeStateRecord of
/// runtime_checkpoint.rs:16-112 for the state this path carries.
pub fn save_streaming_state<B: HipHandles>(path: &str, position: usize,
                                           rho: &[Option<Tensor<B, 4>>],
                                           device: &B::Device) -> Result<(), String> {
    let descs: Vec<ffi::bdh_layer_state_desc> = rho
        .iter()
        .map(|r| {
            let [b, h, n, d] = r.as_ref().map_or([0; 4], |t| t.dims());
            ffi::bdh_layer_state_desc {
                batch: b as i64, heads: h as i64, latent: n as i64, embd: d as i64,
                persist_sequence_state: 1, retain_terminal_sequence_state: 1,
            }
        })
        .collect();
    let ptrs: Vec<*const f32> =
        rho.iter().map(|r| ptr_or_null(r.as_ref()) as *const f32).collect();
    let c_path = CString::new(path).map_err(|e| e.to_string())?;
    let st = unsafe {
        ffi::bdh_state_record_save(c_path.as_ptr(), position as i64, descs.len() as i32,
                                   descs.as_ptr(), ptrs.as_ptr(), B::hip_stream(device))
    };
    if st == ffi::BDH_OK { Ok(()) } else { Err(last_error()) }
}

/// Frees the scratch the library keeps for a backend stream, after that
/// stream's queued work (bdh_scratch_release).  Call it before the stream is
/// destroyed and after every graph captured on it is dropped: the library
/// keeps GB-scale scratch per stream until then.  No counterpart in the
/// reference (Burn's allocator owns its buffers).
pub fn release_stream_scratch<B: HipHandles>(device: &B::Device) -> Result<(), String> {
    let st = unsafe { ffi::bdh_scratch_release(B::hip_stream(device)) };
    if st == ffi::BDH_OK { Ok(()) } else { Err(last_error()) }
}

/// The thread-local message of the last failed call.
pub fn last_error() -> String {
    unsafe {
        let p = ffi::bdh_last_error();
        if p.is_null() {
            String::new()
        } else {
            std::ffi::CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}
