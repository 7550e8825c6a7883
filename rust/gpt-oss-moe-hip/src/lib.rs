//! MI355X (gfx950) backend of gpt-oss-rs's MXFP4 mixture-of-experts path.
//!
//! A thin binding of libgossmx (the C ABI in `include/gossmx.h`, built by
//! `build.rs` with hipcc) for the two call sites of the reference's CPU runner:
//!
//! - the kernel boundary, `Kernels::mxfp4_matmul(backend, problem, scratch)`
//!   inside `CpuModel::project_mxfp4_batch`
//!   (`crates/gpt-oss-model-runner/src/cpu_runner.rs:3392-3416`,
//!   `crates/gpt-oss-cpu-kernels/src/matmul.rs:398-414`):
//!   [`HipMoeBackend::project_residual_q8`] / [`HipMoeBackend::project_q8`];
//! - the block, `CpuModel::moe_batch` (`cpu_runner.rs:2794-3013`):
//!   [`HipMoeBackend::moe_batch`] returning one [`MoeStep`] per input row, the
//!   fields of `CpuMoeStep` (`cpu_runner.rs:569-575`).
//!
//! Both produce the reference's scalar CPU bits (router logits, expert
//! indices and order, routing weights, outputs).
//!
//! Faults follow the Xe branch (`cpu_runner.rs:3247-3391`) and the Xe engine's
//! process-wide breaker (`crates/gpt-oss-xe/src/lib.rs:605-724`): a GPU
//! projection that fails at run time opens the library's circuit breaker and
//! is recomputed once on the reference's own CPU kernels; while the breaker
//! is open every projection goes to the CPU without touching the device,
//! until [`reset_circuit`] is called.
//!
//! Backend spelling: with the `backend-variant` feature the crate expects
//! `Mxfp4MatmulBackend::Hip` ("hip") in gpt-oss-cpu-kernels, whose
//! `scratch_requirement` is `Mxfp4ScratchRequirement::NONE` (the device keeps
//! its own operand buffers, see [`scratch_requirement`]).

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::fmt;
use std::ptr;

use gpt_oss_core::error::LLMError;
use gpt_oss_cpu_kernels::{
    KernelError, Kernels, Mxfp4MatmulBackend, Mxfp4MatmulProblem, Mxfp4MatrixView, Mxfp4ScratchRequirement,
    Mxfp4WeightLayout, Q8Block, Q8MatrixView, ResidualQ8Block, ResidualQ8MatrixView,
};
use half::bf16;

/// Raw declarations of `include/gossmx.h` (the subset this crate uses).
pub mod ffi {
    use std::ffi::{c_char, c_int, c_void};

    #[repr(C)]
    pub struct GossmxCtx {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct GossmxWeights {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct GossmxLayer {
        _private: [u8; 0],
    }

    pub const ACT_Q8: c_int = 1;
    pub const ACT_RESIDUAL_Q8: c_int = 2;
    pub const MEM_HOST: c_int = 0;
    pub const MEM_DEVICE: c_int = 1;
    pub const LAYOUT_CANONICAL_V1: c_int = 1;
    pub const LAYOUT_X8_SPLIT_V2: c_int = 2;
    pub const PROJECTION_RESIDUAL_Q8: c_int = 0;
    pub const PROJECTION_Q8: c_int = 1;
    pub const PROJECTION_EXACT_BF16: c_int = 2;

    /// `Q8Block` with a fixed C layout: f32 scale, then 32 codes (36 bytes).
    #[repr(C)]
    #[derive(Clone, Copy)]
    pub struct Q8Record {
        pub scale: f32,
        pub values: [i8; 32],
    }

    /// `ResidualQ8Block` with a fixed C layout (72 bytes).
    #[repr(C)]
    #[derive(Clone, Copy)]
    pub struct ResidualQ8Record {
        pub primary: Q8Record,
        pub residual: Q8Record,
    }

    #[repr(C)]
    pub struct GossmxMatmulProblem {
        pub weights: *const GossmxWeights,
        pub expert: usize,
        pub activation_kind: c_int,
        pub activations: *const c_void,
        pub activations_len: usize,
        pub m: usize,
        pub blocks_per_row: usize,
        pub row_stride: usize,
        pub bias: *const f32,
        pub bias_len: usize,
        pub output: *mut f32,
        pub output_len: usize,
        pub output_stride: usize,
        pub memory: c_int,
    }

    #[repr(C)]
    pub struct GossmxMoeConfig {
        pub experts: usize,
        pub hidden: usize,
        pub intermediate: usize,
        pub top_k: usize,
        pub alpha: f32,
        pub limit: f32,
        pub projection: c_int,
    }

    #[repr(C)]
    pub struct GossmxMoeIo {
        pub x: *const u16,
        pub m: usize,
        pub injected_logits: *const f32,
        pub router_logits: *mut f32,
        pub selected: *mut u32,
        pub routing_weights: *mut f32,
        pub output: *mut f32,
        pub route_order: *mut u32,
        pub trace_down: *mut f32,
        pub memory: c_int,
        pub trace_gate_up: *mut f32,
        pub trace_swiglu: *mut f32,
        /// The combine's sum before its bf16 round trip (nullable).
        pub output_unrounded: *mut f32,
    }

    /// `gossmx_stats`: projections by result, transfer bytes by direction,
    /// resident bytes and the cap (the Xe engine's metrics).
    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default)]
    pub struct GossmxStats {
        pub projections_ok: u64,
        pub projections_failed: u64,
        pub projections_refused: u64,
        pub projections_rejected: u64,
        pub weights_bias_uploaded_bytes: u64,
        pub activation_bytes: u64,
        pub output_bytes: u64,
        pub resident_bytes: u64,
        pub resident_high_water_bytes: u64,
        pub resident_cap_bytes: u64,
        pub capacity_refusals: u64,
        pub repack_cache_hits: u64,
        pub repack_cache_misses: u64,
        pub circuit_open: i32,
        pub reserved: i32,
    }

    extern "C" {
        pub fn gossmx_last_error() -> *const c_char;
        pub fn gossmx_device_count(count: *mut c_int) -> c_int;
        pub fn gossmx_ctx_create(device: c_int, stream: *mut c_void, out: *mut *mut GossmxCtx) -> c_int;
        pub fn gossmx_ctx_destroy(ctx: *mut GossmxCtx);
        pub fn gossmx_synchronize(ctx: *mut GossmxCtx) -> c_int;
        pub fn gossmx_weights_upload(
            ctx: *mut GossmxCtx,
            data: *const u8,
            len: usize,
            experts: usize,
            rows: usize,
            blocks: usize,
            layout: c_int,
            out: *mut *mut GossmxWeights,
        ) -> c_int;
        pub fn gossmx_weights_open_or_create(
            ctx: *mut GossmxCtx,
            cache_root: *const c_char,
            model_revision: *const c_char,
            source_hashes: *const *const c_char,
            n_hashes: usize,
            shards: *const *const c_char,
            n_shards: usize,
            blocks_name: *const c_char,
            scales_name: *const c_char,
            out: *mut *mut GossmxWeights,
        ) -> c_int;
        pub fn gossmx_weights_shape(w: *const GossmxWeights, experts: *mut usize, rows: *mut usize, blocks: *mut usize)
            -> c_int;
        pub fn gossmx_weights_destroy(w: *mut GossmxWeights);
        pub fn gossmx_mxfp4_matmul(ctx: *mut GossmxCtx, problem: *const GossmxMatmulProblem) -> c_int;
        pub fn gossmx_mxfp4_scratch_requirement(
            problem: *const GossmxMatmulProblem,
            size: *mut usize,
            alignment: *mut usize,
        ) -> c_int;
        pub fn gossmx_layer_create(
            ctx: *mut GossmxCtx,
            config: *const GossmxMoeConfig,
            router_weight_bf16: *const u16,
            router_bias: *const f32,
            gate_up: *const GossmxWeights,
            gate_up_bias: *const f32,
            down: *const GossmxWeights,
            down_bias: *const f32,
            out: *mut *mut GossmxLayer,
        ) -> c_int;
        pub fn gossmx_layer_destroy(layer: *mut GossmxLayer);
        pub fn gossmx_moe_forward(ctx: *mut GossmxCtx, layer: *const GossmxLayer, io: *const GossmxMoeIo) -> c_int;
        pub fn gossmx_moe_forward_residual(
            ctx: *mut GossmxCtx,
            layer: *const GossmxLayer,
            io: *const GossmxMoeIo,
            norm_weight: *const f32,
            epsilon: f32,
            next_residual: *mut u16,
        ) -> c_int;
        pub fn gossmx_circuit_is_open() -> c_int;
        pub fn gossmx_circuit_reset();
        pub fn gossmx_inject_fault(ctx: *mut GossmxCtx, armed: c_int) -> c_int;
        pub fn gossmx_stats_read(out: *mut GossmxStats) -> c_int;
        pub fn gossmx_stats_reset();
        pub fn gossmx_set_resident_cap(bytes: u64) -> c_int;
    }
}

/// The status codes of `gossmx_status`, one variant per code.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Status {
    InvalidArgument,
    Unsupported,
    InvalidDimensions,
    NonFiniteInput,
    UnavailableBackend,
    Device,
    OutOfMemory,
    NonFiniteLogits,
    InjectedFault,
    BadFile,
    CircuitOpen,
    Unknown(c_int),
}

impl Status {
    pub const fn from_code(code: c_int) -> Self {
        match code {
            1 => Self::InvalidArgument,
            2 => Self::Unsupported,
            3 => Self::InvalidDimensions,
            4 => Self::NonFiniteInput,
            5 => Self::UnavailableBackend,
            6 => Self::Device,
            7 => Self::OutOfMemory,
            8 => Self::NonFiniteLogits,
            9 => Self::InjectedFault,
            10 => Self::BadFile,
            11 => Self::CircuitOpen,
            other => Self::Unknown(other),
        }
    }
}

/// A failed libgossmx call: its status and `gossmx_last_error()` message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct HipError {
    pub status: Status,
    pub message: String,
}

/// The backend spelling this crate reports in `UnavailableMatmulBackend`.
#[cfg(feature = "backend-variant")]
pub const HIP_BACKEND: Mxfp4MatmulBackend = Mxfp4MatmulBackend::Hip;
#[cfg(not(feature = "backend-variant"))]
pub const HIP_BACKEND: Mxfp4MatmulBackend = Mxfp4MatmulBackend::Auto;

impl HipError {
    fn last(code: c_int) -> Self {
        // SAFETY: gossmx_last_error returns a NUL-terminated thread-local string.
        let message = unsafe { CStr::from_ptr(ffi::gossmx_last_error()) }.to_string_lossy().into_owned();
        Self { status: Status::from_code(code), message }
    }

    /// The `KernelError` a CPU kernel would have returned for the same
    /// problem, for the statuses that have one.
    pub fn kernel_error(&self) -> Option<KernelError> {
        match self.status {
            Status::InvalidDimensions => Some(KernelError::InvalidDimensions(self.message.clone())),
            Status::NonFiniteInput => Some(KernelError::NonFiniteInput),
            Status::UnavailableBackend => {
                Some(KernelError::UnavailableMatmulBackend { backend: HIP_BACKEND, reason: "no gfx950 HIP device" })
            }
            _ => None,
        }
    }

    /// Run-time GPU failures: the library has opened its circuit breaker
    /// (or found it open); the call is recomputed on the CPU.
    pub fn is_device_fault(&self) -> bool {
        matches!(self.status, Status::Device | Status::OutOfMemory | Status::CircuitOpen)
    }
}

impl fmt::Display for HipError {
    fn fmt(&self, formatter: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(formatter, "gossmx {:?}: {}", self.status, self.message)
    }
}

impl std::error::Error for HipError {}

/// One `LLMError` per status: the kernel errors exactly as the runner's
/// `kernel_error` reports them (`cpu_runner.rs:4015-4017`), the router's
/// non-finite logits with its own message (`cpu_runner.rs:2829-2834`), device
/// and memory failures as `GpuError` / `MemoryError`.
impl From<HipError> for LLMError {
    fn from(error: HipError) -> Self {
        if let Some(kernel) = error.kernel_error() {
            return LLMError::ModelError(kernel.to_string());
        }
        match error.status {
            Status::NonFiniteLogits => LLMError::ModelError("CPU router produced non-finite logits".into()),
            Status::Device => LLMError::GpuError(error.message),
            Status::OutOfMemory => LLMError::MemoryError(error.message),
            Status::CircuitOpen => LLMError::GpuError("GPU circuit breaker is open".into()),
            Status::BadFile => LLMError::ModelError(error.message),
            Status::InvalidArgument => LLMError::ModelError(format!("invalid GPU MoE argument: {}", error.message)),
            Status::Unsupported => LLMError::ModelError(format!("GPU MoE shape unsupported: {}", error.message)),
            Status::InjectedFault => LLMError::ModelError(format!("injected GPU MoE fault: {}", error.message)),
            Status::Unknown(code) => LLMError::GpuError(format!("gossmx status {code}: {}", error.message)),
            Status::InvalidDimensions | Status::NonFiniteInput | Status::UnavailableBackend => {
                unreachable!("kernel errors are mapped above")
            }
        }
    }
}

fn check(code: c_int) -> Result<(), HipError> {
    if code == 0 {
        Ok(())
    } else {
        Err(HipError::last(code))
    }
}

/// Whether the process-wide breaker is open (`XeProjectionEngine::circuit_is_open`).
pub fn circuit_is_open() -> bool {
    // SAFETY: no arguments; reads an atomic.
    unsafe { ffi::gossmx_circuit_is_open() != 0 }
}

/// Closes the breaker again (after the operator has dealt with the fault).
pub fn reset_circuit() {
    // SAFETY: no arguments; writes an atomic.
    unsafe { ffi::gossmx_circuit_reset() }
}

/// The process-wide counters, for the caller's metrics exporter
/// (`gpt_oss_xe_projection_total`, `_transfer_bytes_total`,
/// `_expert_cache_resident_bytes`, crates/gpt-oss-xe/src/lib.rs:44-49).
pub fn stats() -> Result<ffi::GossmxStats, HipError> {
    let mut out = ffi::GossmxStats::default();
    // SAFETY: out is a valid, writable gossmx_stats.
    check(unsafe { ffi::gossmx_stats_read(&mut out) })?;
    Ok(out)
}

/// Caps the device bytes of resident weights and layers
/// (`AttachConfig::max_resident_bytes`); 0 removes the cap.
pub fn set_resident_cap(bytes: u64) -> Result<(), HipError> {
    // SAFETY: no pointers; writes an atomic.
    check(unsafe { ffi::gossmx_set_resident_cap(bytes) })
}

/// Number of visible gfx950 devices.
pub fn device_count() -> usize {
    let mut count: c_int = 0;
    // SAFETY: count is a valid out pointer.
    if unsafe { ffi::gossmx_device_count(&mut count) } != 0 {
        return 0;
    }
    count.max(0) as usize
}

/// `Mxfp4MatmulBackend::scratch_requirement` of the GPU backend: always
/// `Mxfp4ScratchRequirement::NONE`.
pub const fn scratch_requirement() -> Mxfp4ScratchRequirement {
    Mxfp4ScratchRequirement::NONE
}

/// One device and one in-order HIP stream; used by one thread at a time
/// (like `CpuExecutionContext`, `cpu_runner.rs:868-876`).
pub struct Context {
    raw: *mut ffi::GossmxCtx,
}

// SAFETY: a context may move between threads; it is never used by two at once (&mut or a lock).
unsafe impl Send for Context {}

impl Context {
    pub fn new(device: i32) -> Result<Self, HipError> {
        let mut raw = ptr::null_mut();
        // SAFETY: raw is a valid out pointer; a null stream lets the library create one.
        check(unsafe { ffi::gossmx_ctx_create(device, ptr::null_mut(), &mut raw) })?;
        Ok(Self { raw })
    }

    pub fn synchronize(&self) -> Result<(), HipError> {
        // SAFETY: self.raw is a live context.
        check(unsafe { ffi::gossmx_synchronize(self.raw) })
    }

    /// Test hook: fail the next projection call as a model error (mode 1)
    /// or as a device fault that opens the breaker (mode 2).
    pub fn inject_fault(&self, mode: i32) -> Result<(), HipError> {
        // SAFETY: self.raw is a live context.
        check(unsafe { ffi::gossmx_inject_fault(self.raw, mode) })
    }

    pub fn as_raw(&self) -> *mut ffi::GossmxCtx {
        self.raw
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // SAFETY: self.raw came from gossmx_ctx_create and is destroyed once.
        unsafe { ffi::gossmx_ctx_destroy(self.raw) }
    }
}

/// A resident MXFP4 tensor `[experts][rows][blocks]` in the GPU layout
/// (owned by the library; independent of the context after creation).
pub struct ResidentMxfp4 {
    raw: *mut ffi::GossmxWeights,
    pub experts: usize,
    pub rows: usize,
    pub blocks: usize,
}

// SAFETY: the handle is immutable device memory.
unsafe impl Send for ResidentMxfp4 {}
unsafe impl Sync for ResidentMxfp4 {}

impl ResidentMxfp4 {
    /// Uploads a repacked tensor (every expert, as `RepackedMxfp4` maps it:
    /// canonical v1 or x8 v2 records) and repacks it on the device.
    pub fn upload(
        ctx: &Context,
        data: &[u8],
        experts: usize,
        rows: usize,
        blocks: usize,
        layout: Mxfp4WeightLayout,
    ) -> Result<Self, HipError> {
        let layout = match layout {
            Mxfp4WeightLayout::CanonicalAdjacentV1 => ffi::LAYOUT_CANONICAL_V1,
            Mxfp4WeightLayout::InterleavedSplitX8V2 => ffi::LAYOUT_X8_SPLIT_V2,
        };
        let mut raw = ptr::null_mut();
        // SAFETY: data is valid for data.len() bytes; raw is a valid out pointer.
        check(unsafe {
            ffi::gossmx_weights_upload(ctx.raw, data.as_ptr(), data.len(), experts, rows, blocks, layout, &mut raw)
        })?;
        Ok(Self { raw, experts, rows, blocks })
    }

    /// `CpuRepackCache::open_or_create` (`cpu_repack.rs:149-216`) with the
    /// resident layout 3: a published cache file is mapped onto the device,
    /// otherwise the SafeTensors shards are read and the file is published.
    #[allow(clippy::too_many_arguments)]
    pub fn open_or_create(
        ctx: &Context,
        cache_root: &str,
        model_revision: &str,
        source_hashes: &[String],
        shards: &[String],
        blocks_name: &str,
        scales_name: &str,
    ) -> Result<Self, HipError> {
        let cstr = |s: &str| CString::new(s).map_err(|_| HipError { status: Status::InvalidArgument, message: "NUL in string".into() });
        let root = cstr(cache_root)?;
        let revision = cstr(model_revision)?;
        let hashes = source_hashes.iter().map(|s| cstr(s)).collect::<Result<Vec<_>, _>>()?;
        let shard_names = shards.iter().map(|s| cstr(s)).collect::<Result<Vec<_>, _>>()?;
        let hash_ptrs = hashes.iter().map(|s| s.as_ptr()).collect::<Vec<*const c_char>>();
        let shard_ptrs = shard_names.iter().map(|s| s.as_ptr()).collect::<Vec<*const c_char>>();
        let blocks_c = cstr(blocks_name)?;
        let scales_c = cstr(scales_name)?;
        let mut raw = ptr::null_mut();
        // SAFETY: every pointer is a live NUL-terminated string or array of them.
        check(unsafe {
            ffi::gossmx_weights_open_or_create(
                ctx.raw,
                root.as_ptr(),
                revision.as_ptr(),
                hash_ptrs.as_ptr(),
                hash_ptrs.len(),
                shard_ptrs.as_ptr(),
                shard_ptrs.len(),
                blocks_c.as_ptr(),
                scales_c.as_ptr(),
                &mut raw,
            )
        })?;
        let (mut experts, mut rows, mut blocks) = (0, 0, 0);
        // SAFETY: raw is a live weights handle.
        check(unsafe { ffi::gossmx_weights_shape(raw, &mut experts, &mut rows, &mut blocks) })?;
        Ok(Self { raw, experts, rows, blocks })
    }
}

impl Drop for ResidentMxfp4 {
    fn drop(&mut self) {
        // SAFETY: created by the library, destroyed once; waits for the device.
        unsafe { ffi::gossmx_weights_destroy(self.raw) }
    }
}

/// `CpuExpertProjection` (`cpu_runner.rs:49-90`).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum ExpertProjection {
    Q8,
    ResidualQ8,
    ExactBf16,
}

/// One GPT-OSS MoE layer resident on the device: router weights and bias,
/// the two expert tensors (borrowed) and their biases.
pub struct MoeLayer<'w> {
    raw: *mut ffi::GossmxLayer,
    pub experts: usize,
    pub hidden: usize,
    pub intermediate: usize,
    pub top_k: usize,
    _weights: std::marker::PhantomData<&'w ResidentMxfp4>,
}

impl<'w> MoeLayer<'w> {
    #[allow(clippy::too_many_arguments)]
    pub fn new(
        ctx: &Context,
        experts: usize,
        hidden: usize,
        intermediate: usize,
        top_k: usize,
        alpha: f32,
        limit: f32,
        projection: ExpertProjection,
        router_weight: &[bf16],
        router_bias: &[f32],
        gate_up: &'w ResidentMxfp4,
        gate_up_bias: &[f32],
        down: &'w ResidentMxfp4,
        down_bias: &[f32],
    ) -> Result<Self, HipError> {
        if router_weight.len() != experts * hidden
            || router_bias.len() != experts
            || gate_up_bias.len() != experts * 2 * intermediate
            || down_bias.len() != experts * hidden
        {
            return Err(HipError { status: Status::InvalidDimensions, message: "MoE layer tensor sizes".into() });
        }
        let config = ffi::GossmxMoeConfig {
            experts,
            hidden,
            intermediate,
            top_k,
            alpha,
            limit,
            projection: match projection {
                ExpertProjection::ResidualQ8 => ffi::PROJECTION_RESIDUAL_Q8,
                ExpertProjection::Q8 => ffi::PROJECTION_Q8,
                ExpertProjection::ExactBf16 => ffi::PROJECTION_EXACT_BF16,
            },
        };
        let mut raw = ptr::null_mut();
        // SAFETY: the slices have the sizes checked above; bf16 is a u16 bit pattern.
        check(unsafe {
            ffi::gossmx_layer_create(
                ctx.raw,
                &config,
                router_weight.as_ptr().cast::<u16>(),
                router_bias.as_ptr(),
                gate_up.raw,
                gate_up_bias.as_ptr(),
                down.raw,
                down_bias.as_ptr(),
                &mut raw,
            )
        })?;
        Ok(Self { raw, experts, hidden, intermediate, top_k, _weights: std::marker::PhantomData })
    }
}

impl Drop for MoeLayer<'_> {
    fn drop(&mut self) {
        // SAFETY: created by the library, destroyed once.
        unsafe { ffi::gossmx_layer_destroy(self.raw) }
    }
}

/// The per-row result of the block, `CpuMoeStep`'s fields (`cpu_runner.rs:569-575`).
#[derive(Debug, Clone, PartialEq)]
pub struct MoeStep {
    pub router_logits: Vec<f32>,
    pub selected_experts: Vec<usize>,
    pub routing_weights: Vec<f32>,
    pub output: Vec<f32>,
    /// Per rank when captured: (gate_up bf16 values, SwiGLU values, down
    /// projection bf16 values) as `CpuExpertTrace` holds them.
    pub traces: Vec<(Vec<f32>, Vec<f32>, Vec<f32>)>,
}

/// Where a projection ran.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Projection {
    Gpu,
    /// The GPU failed at run time or the breaker was open; the reference's
    /// CPU kernel computed the output.
    CpuFallback,
}

/// The GPU backend of one worker: a context (one stream) plus the CPU
/// kernels and scratch of the one-shot fallback.
pub struct HipMoeBackend {
    ctx: Context,
    kernels: Kernels,
    cpu_backend: Mxfp4MatmulBackend,
    cpu_scratch: Vec<u8>,
}

impl HipMoeBackend {
    pub fn new(device: i32, kernels: Kernels, cpu_backend: Mxfp4MatmulBackend) -> Result<Self, HipError> {
        Ok(Self { ctx: Context::new(device)?, kernels, cpu_backend, cpu_scratch: Vec::new() })
    }

    pub fn context(&self) -> &Context {
        &self.ctx
    }

    fn cpu_scratch(&mut self, requirement: Mxfp4ScratchRequirement) -> &mut [u8] {
        // CpuExecutionContext::matrix_scratch (cpu_runner.rs:908-929).
        if requirement.size == 0 {
            return &mut [];
        }
        let allocation = requirement.size + requirement.alignment - 1;
        if self.cpu_scratch.len() < allocation {
            self.cpu_scratch.resize(allocation, 0);
        }
        let offset = (requirement.alignment - self.cpu_scratch.as_ptr() as usize % requirement.alignment)
            % requirement.alignment;
        &mut self.cpu_scratch[offset..offset + requirement.size]
    }

    fn gpu_matmul(
        &self,
        weights: &ResidentMxfp4,
        expert: usize,
        kind: c_int,
        activations: *const c_void,
        activations_len: usize,
        m: usize,
        bias: Option<&[f32]>,
        output: &mut [f32],
        output_stride: usize,
    ) -> Result<(), HipError> {
        let problem = ffi::GossmxMatmulProblem {
            weights: weights.raw,
            expert,
            activation_kind: kind,
            activations,
            activations_len,
            m,
            blocks_per_row: weights.blocks,
            row_stride: weights.blocks,
            bias: bias.map_or(ptr::null(), <[f32]>::as_ptr),
            bias_len: bias.map_or(0, <[f32]>::len),
            output: output.as_mut_ptr(),
            output_len: output.len(),
            output_stride,
            memory: ffi::MEM_HOST,
        };
        // SAFETY: every pointer is valid for the lengths given; the call
        // validates them before any access and writes only inside output.
        check(unsafe { ffi::gossmx_mxfp4_matmul(self.ctx.raw, &problem) })
    }

    fn warn_fallback(error: &HipError, role: &str) {
        tracing::warn!(
            projection = role,
            reason = %error,
            "GPU projection failed; recomputing once on CPU (the circuit breaker is open)"
        );
    }

    /// The residual-Q8 branch of `project_mxfp4_batch` for one expert bucket:
    /// `activations` are the bucket's rows (`m` rows of `view.blocks()`
    /// records), `output` is `m * view.rows()` floats with stride `view.rows()`.
    /// `view` is the same expert's CPU view, used by the fallback.
    #[allow(clippy::too_many_arguments)]
    pub fn project_residual_q8(
        &mut self,
        resident: &ResidentMxfp4,
        expert: usize,
        view: Mxfp4MatrixView<'_>,
        activations: &[ResidualQ8Block],
        m: usize,
        bias: &[f32],
        output: &mut [f32],
        role: &str,
    ) -> Result<Projection, LLMError> {
        let records = activations
            .iter()
            .map(|block| ffi::ResidualQ8Record {
                primary: ffi::Q8Record { scale: block.primary.scale, values: block.primary.values },
                residual: ffi::Q8Record { scale: block.residual.scale, values: block.residual.values },
            })
            .collect::<Vec<_>>();
        let rows = view.rows();
        let gpu = self.gpu_matmul(
            resident,
            expert,
            ffi::ACT_RESIDUAL_Q8,
            records.as_ptr().cast(),
            records.len(),
            m,
            Some(bias),
            output,
            rows,
        );
        match gpu {
            Ok(()) => Ok(Projection::Gpu),
            Err(error) if error.is_device_fault() => {
                Self::warn_fallback(&error, role);
                let blocks = view.blocks();
                let acts = ResidualQ8MatrixView::new(activations, m, blocks, blocks).map_err(kernel_error)?;
                let problem =
                    Mxfp4MatmulProblem::new_residual_q8(view, acts, Some(bias), output, rows).map_err(kernel_error)?;
                let requirement = self.cpu_backend.scratch_requirement(&problem).map_err(kernel_error)?;
                let (kernels, backend) = (self.kernels, self.cpu_backend);
                let scratch = self.cpu_scratch(requirement);
                kernels.mxfp4_matmul(backend, problem, scratch).map_err(kernel_error)?;
                Ok(Projection::CpuFallback)
            }
            Err(error) => Err(error.into()),
        }
    }

    /// The Q8 branch of `project_mxfp4_batch` (`cpu_runner.rs:3158-3210`).
    #[allow(clippy::too_many_arguments)]
    pub fn project_q8(
        &mut self,
        resident: &ResidentMxfp4,
        expert: usize,
        view: Mxfp4MatrixView<'_>,
        activations: &[Q8Block],
        m: usize,
        bias: &[f32],
        output: &mut [f32],
        role: &str,
    ) -> Result<Projection, LLMError> {
        let records = activations
            .iter()
            .map(|block| ffi::Q8Record { scale: block.scale, values: block.values })
            .collect::<Vec<_>>();
        let rows = view.rows();
        let gpu = self.gpu_matmul(
            resident,
            expert,
            ffi::ACT_Q8,
            records.as_ptr().cast(),
            records.len(),
            m,
            Some(bias),
            output,
            rows,
        );
        match gpu {
            Ok(()) => Ok(Projection::Gpu),
            Err(error) if error.is_device_fault() => {
                Self::warn_fallback(&error, role);
                let blocks = view.blocks();
                let acts = Q8MatrixView::new(activations, m, blocks, blocks).map_err(kernel_error)?;
                let problem = Mxfp4MatmulProblem::new_q8(view, acts, Some(bias), output, rows).map_err(kernel_error)?;
                let requirement = self.cpu_backend.scratch_requirement(&problem).map_err(kernel_error)?;
                let (kernels, backend) = (self.kernels, self.cpu_backend);
                let scratch = self.cpu_scratch(requirement);
                kernels.mxfp4_matmul(backend, problem, scratch).map_err(kernel_error)?;
                Ok(Projection::CpuFallback)
            }
            Err(error) => Err(error.into()),
        }
    }

    /// `CpuModel::moe_batch` on the GPU for rows `inputs` (each `hidden`
    /// bf16 values): one call runs the router, selection, grouping, both
    /// projections and the combine. `capture[i]` asks for row i's expert
    /// traces. On a device fault the error is returned (the breaker is open
    /// and the caller runs its own `moe_batch` once, as the Xe branch
    /// recomputes on CPU).
    pub fn moe_batch(&self, layer: &MoeLayer<'_>, inputs: &[Vec<bf16>], capture: &[bool]) -> Result<Vec<MoeStep>, HipError> {
        let (m, e, k, h, i) = (inputs.len(), layer.experts, layer.top_k, layer.hidden, layer.intermediate);
        if capture.len() != m || inputs.iter().any(|row| row.len() != h) {
            return Err(HipError { status: Status::InvalidDimensions, message: "invalid CPU MoE batch metadata".into() });
        }
        let mut x = Vec::with_capacity(m * h);
        for row in inputs {
            x.extend(row.iter().map(|value| value.to_bits()));
        }
        let mut logits = vec![0.0_f32; m * e];
        let mut selected = vec![0_u32; m * k];
        let mut weights = vec![0.0_f32; m * k];
        let mut output = vec![0.0_f32; m * h];
        let want_traces = capture.iter().any(|&c| c);
        let mut trace_down = if want_traces { vec![0.0_f32; m * k * h] } else { Vec::new() };
        let mut trace_gate_up = if want_traces { vec![0.0_f32; m * k * 2 * i] } else { Vec::new() };
        let mut trace_swiglu = if want_traces { vec![0.0_f32; m * k * i] } else { Vec::new() };
        let nullable = |v: &mut Vec<f32>| if v.is_empty() { ptr::null_mut() } else { v.as_mut_ptr() };
        let io = ffi::GossmxMoeIo {
            x: x.as_ptr(),
            m,
            injected_logits: ptr::null(),
            router_logits: logits.as_mut_ptr(),
            selected: selected.as_mut_ptr(),
            routing_weights: weights.as_mut_ptr(),
            output: output.as_mut_ptr(),
            route_order: ptr::null_mut(),
            trace_down: nullable(&mut trace_down),
            memory: ffi::MEM_HOST,
            trace_gate_up: nullable(&mut trace_gate_up),
            trace_swiglu: nullable(&mut trace_swiglu),
            output_unrounded: ptr::null_mut(),
        };
        // SAFETY: every array has the size the header states for these m, e, k, h, i.
        check(unsafe { ffi::gossmx_moe_forward(self.ctx.raw, layer.raw, &io) })?;
        Ok((0..m)
            .map(|r| MoeStep {
                router_logits: logits[r * e..(r + 1) * e].to_vec(),
                selected_experts: selected[r * k..(r + 1) * k].iter().map(|&s| s as usize).collect(),
                routing_weights: weights[r * k..(r + 1) * k].to_vec(),
                output: output[r * h..(r + 1) * h].to_vec(),
                traces: if capture[r] {
                    (0..k)
                        .map(|rank| {
                            let slot = r * k + rank;
                            (
                                trace_gate_up[slot * 2 * i..(slot + 1) * 2 * i].to_vec(),
                                trace_swiglu[slot * i..(slot + 1) * i].to_vec(),
                                trace_down[slot * h..(slot + 1) * h].to_vec(),
                            )
                        })
                        .collect()
                } else {
                    Vec::new()
                },
            })
            .collect())
    }
}

fn kernel_error(error: KernelError) -> LLMError {
    LLMError::ModelError(error.to_string())
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn every_status_code_has_its_own_variant() {
        let statuses = (1..=11).map(Status::from_code).collect::<Vec<_>>();
        for (index, status) in statuses.iter().enumerate() {
            assert!(!matches!(status, Status::Unknown(_)), "code {}", index + 1);
            assert_eq!(statuses.iter().filter(|other| *other == status).count(), 1);
        }
        assert_eq!(Status::from_code(42), Status::Unknown(42));
    }

    #[test]
    fn kernel_statuses_map_to_kernel_errors() {
        let error = |status| HipError { status, message: "m".into() };
        assert_eq!(error(Status::InvalidDimensions).kernel_error(), Some(KernelError::InvalidDimensions("m".into())));
        assert_eq!(error(Status::NonFiniteInput).kernel_error(), Some(KernelError::NonFiniteInput));
        assert!(error(Status::Device).is_device_fault());
        assert!(error(Status::CircuitOpen).is_device_fault());
        assert!(!error(Status::NonFiniteInput).is_device_fault());
        assert!(matches!(LLMError::from(error(Status::Device)), LLMError::GpuError(_)));
        assert!(matches!(LLMError::from(error(Status::OutOfMemory)), LLMError::MemoryError(_)));
    }

    /// On a host with a gfx950 device: the injected device fault opens the
    /// breaker and the projection is recomputed on the reference's CPU
    /// kernel, bit-identical to its scalar matmul.
    #[test]
    fn device_fault_falls_back_to_the_cpu_kernel_once() {
        if device_count() == 0 {
            return;
        }
        let (rows, blocks, m) = (16_usize, 2_usize, 3_usize);
        let data = (0..rows * blocks * 17)
            .map(|i| if i % 17 == 0 { 120 + (i / 17 % 5) as u8 } else { (i * 37 % 251) as u8 })
            .collect::<Vec<u8>>();
        let activations = (0..m * blocks)
            .map(|b| ResidualQ8Block {
                primary: Q8Block { scale: 0.01 + b as f32 * 0.001, values: std::array::from_fn(|j| (j as i8) - 16) },
                residual: Q8Block { scale: 0.0001, values: std::array::from_fn(|j| 15 - j as i8) },
            })
            .collect::<Vec<_>>();
        let bias = (0..rows).map(|r| r as f32 * 0.25).collect::<Vec<f32>>();
        let kernels = Kernels::new(gpt_oss_cpu_kernels::KernelPath::Auto).expect("kernels");
        let mut backend = HipMoeBackend::new(0, kernels, Mxfp4MatmulBackend::Scalar).expect("context");
        let resident =
            ResidentMxfp4::upload(backend.context(), &data, 1, rows, blocks, Mxfp4WeightLayout::CanonicalAdjacentV1)
                .expect("upload");
        let view = Mxfp4MatrixView::new(&data, rows, blocks, Mxfp4WeightLayout::CanonicalAdjacentV1).unwrap();
        let mut want = vec![0.0_f32; m * rows];
        let acts = ResidualQ8MatrixView::new(&activations, m, blocks, blocks).unwrap();
        let problem = Mxfp4MatmulProblem::new_residual_q8(view, acts, Some(&bias), &mut want, rows).unwrap();
        kernels.mxfp4_matmul(Mxfp4MatmulBackend::Scalar, problem, &mut []).unwrap();

        let mut got = vec![0.0_f32; m * rows];
        let run = |backend: &mut HipMoeBackend, out: &mut [f32]| {
            backend.project_residual_q8(&resident, 0, view, &activations, m, &bias, out, "gate_up").unwrap()
        };
        assert_eq!(run(&mut backend, &mut got), Projection::Gpu);
        assert_eq!(got.iter().map(|v| v.to_bits()).collect::<Vec<_>>(), want.iter().map(|v| v.to_bits()).collect::<Vec<_>>());
        backend.context().inject_fault(2).unwrap();
        got.fill(f32::NAN);
        assert_eq!(run(&mut backend, &mut got), Projection::CpuFallback);
        assert!(circuit_is_open());
        assert_eq!(got.iter().map(|v| v.to_bits()).collect::<Vec<_>>(), want.iter().map(|v| v.to_bits()).collect::<Vec<_>>());
        assert_eq!(run(&mut backend, &mut got), Projection::CpuFallback); // stays on the CPU while open
        reset_circuit();
        assert_eq!(run(&mut backend, &mut got), Projection::Gpu);
    }
}
