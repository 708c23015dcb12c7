//! The C ABI of libiris_hip, one declaration per function of
//! include/iris_hip.h, in the header's order. The first five are the
//! reference's own extern block (crates/inference/kernels/src/gpu.rs:45-62).

use std::os::raw::{c_char, c_int, c_void};

/// Opaque device matrix (the reference's `DeviceMatrix`, gpu.rs:40-43).
#[repr(C)]
pub struct Q8GpuMatrix {
    _private: [u8; 0],
}

#[repr(C)]
pub struct IrisModel {
    _private: [u8; 0],
}

#[repr(C)]
pub struct IrisSession {
    _private: [u8; 0],
}

pub const IRIS_FAMILY_MISTRAL_DENSE: i32 = 0;
pub const IRIS_FAMILY_GEMMA_DENSE: i32 = 1;
pub const IRIS_NOALLOC_SCRATCH_BYTES: u64 = 32 << 20;

/// Shape scalars (include/iris_hip.h `IrisModelDesc`; the reference's
/// MistralShape / DirectInferShape, crates/inference/artifacts/src/direct.rs:241-290).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct IrisModelDesc {
    pub family: i32,
    pub hidden: u32,
    pub layers: u32,
    pub heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub ffn: u32,
    pub vocab: u32,
    pub norm_eps: i64,
    pub attention_scale_q32: u32,
    pub max_positions: u32,
    pub tied_head: i32,
    pub global_head_dim: u32,
    pub ple_width: u32,
    pub sliding_window: u32,
    pub num_kv_shared_layers: u32,
    pub rope_base_sliding: i64,
    pub rope_base_full: i64,
    pub partial_rotary_q16: i32,
    pub embedding_scale: i32,
    pub ple_embedding_scale: i32,
    pub ple_projection_scalar: i32,
    pub ple_input_scale: i32,
    pub final_logit_softcap: i32,
    pub layer_is_sliding: *const u8,
}

extern "C" {
    pub fn q8gpu_error(code: c_int) -> *const c_char;
    pub fn q8gpu_init() -> c_int;
    pub fn q8gpu_upload(
        weights: *const i8,
        scales: *const i64,
        rows: u32,
        cols: u32,
        out: *mut *mut Q8GpuMatrix,
    ) -> c_int;
    pub fn q8gpu_free(matrix: *mut Q8GpuMatrix);
    pub fn q8gpu_product(matrix: *const Q8GpuMatrix, activations: *const i32, tokens: u32, out: *mut i32) -> c_int;

    pub fn q8gpu_upload_q8_0(blocks: *const u8, rows: u32, cols: u32, out: *mut *mut Q8GpuMatrix) -> c_int;
    pub fn q8gpu_product_device(
        matrix: *const Q8GpuMatrix,
        d_activations: *const i32,
        tokens: u32,
        d_out: *mut i32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn q8gpu_workspace_bytes(matrix: *const Q8GpuMatrix, tokens: u32) -> u64;
    pub fn q8gpu_product_device_ws(
        matrix: *const Q8GpuMatrix,
        d_activations: *const i32,
        tokens: u32,
        d_out: *mut i32,
        d_workspace: *mut c_void,
        workspace_bytes: u64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn q8gpu_prepare_matrix_cores(matrix: *mut Q8GpuMatrix, stream: *mut c_void) -> c_int;
    pub fn q8gpu_product_device_noalloc(
        matrix: *const Q8GpuMatrix,
        d_activations: *const i32,
        tokens: u32,
        d_out: *mut i32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn q8gpu_matrix_info(
        matrix: *const Q8GpuMatrix,
        rows: *mut u32,
        cols: *mut u32,
        scale_mode: *mut c_int,
        bytes: *mut u64,
    ) -> c_int;
    pub fn q8gpu_synchronize() -> c_int;

    pub fn iris_device_malloc(bytes: u64, out: *mut *mut c_void) -> c_int;
    pub fn iris_device_free(ptr: *mut c_void) -> c_int;
    pub fn iris_memcpy_h2d(dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
    pub fn iris_memcpy_d2h(dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
    pub fn iris_memcpy_d2d(dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
    pub fn iris_probe_hbm_read(d_buf: *const c_void, bytes: u64, repeats: u32, gb_per_s: *mut f64) -> c_int;
    pub fn iris_probe_mfma_i8(random_operands: u32, iterations: u32, tops: *mut f64) -> c_int;
    pub fn iris_probe_handoff(workgroups: u32, round_trip_us: *mut f64, atomic_us: *mut f64, barrier_us: *mut f64)
        -> c_int;
    pub fn iris_probe_row_latency(flood_waves: u32, vector_us: *mut f64, scalar_us: *mut f64) -> c_int;
    pub fn iris_time_product(
        matrices: *const *const Q8GpuMatrix,
        count: u32,
        d_activations: *const i32,
        tokens: u32,
        d_out: *mut i32,
        iterations: u32,
        ms_per_product: *mut f64,
    ) -> c_int;
    pub fn iris_time_bcast_product(
        matrices: *const *const Q8GpuMatrix,
        count: u32,
        d_activations: *const i32,
        d_out: *mut i32,
        iterations: u32,
        ms_per_product: *mut f64,
    ) -> c_int;
    pub fn iris_time_product_ws(
        matrix: *const Q8GpuMatrix,
        d_activations: *const i32,
        tokens: u32,
        d_out: *mut i32,
        d_workspace: *mut c_void,
        workspace_bytes: u64,
        iterations: u32,
        ms_per_product: *mut f64,
    ) -> c_int;

    pub fn iris_model_create(desc: *const IrisModelDesc, out: *mut *mut IrisModel) -> c_int;
    pub fn iris_model_set_tensor(
        model: *mut IrisModel,
        name: *const c_char,
        width: i32,
        data: *const c_void,
        rows: u64,
        cols: u64,
    ) -> c_int;
    pub fn iris_model_finalize(model: *mut IrisModel) -> c_int;
    pub fn iris_model_free(model: *mut IrisModel);
    pub fn iris_model_device_bytes(model: *const IrisModel) -> u64;

    pub fn iris_session_create(
        model: *mut IrisModel,
        max_positions: u32,
        max_rows: u32,
        out: *mut *mut IrisSession,
    ) -> c_int;
    pub fn iris_session_free(session: *mut IrisSession);
    pub fn iris_session_generate(
        session: *mut IrisSession,
        prompt: *const i32,
        prompt_len: u32,
        tokens: u32,
        eos_ids: *const i32,
        n_eos: u32,
        out_tokens: *mut i32,
        out_count: *mut u32,
        out_logits: *mut i32,
        use_graph: i32,
    ) -> c_int;
    pub fn iris_session_layer_pass(
        session: *mut IrisSession,
        ids: *const i32,
        count: u32,
        out_rows: *mut i32,
        out_hashes: *mut u8,
    ) -> c_int;
    pub fn iris_session_layer_range(
        session: *mut IrisSession,
        ids: *const i32,
        count: u32,
        start_position: u32,
        out_rows: *mut i32,
        out_hashes: *mut u8,
    ) -> c_int;
    pub fn iris_session_layer_stage(
        session: *mut IrisSession,
        layer: u32,
        in_rows: *const i32,
        count: u32,
        start_position: u32,
        ple_rows: *const i32,
        out_rows: *mut i32,
    ) -> c_int;
    pub fn iris_session_write_kv(
        session: *mut IrisSession,
        layer: u32,
        pos0: u32,
        count: u32,
        k: *const i32,
        v: *const i32,
    ) -> c_int;
    pub fn iris_session_read_kv(
        session: *mut IrisSession,
        layer: u32,
        pos0: u32,
        count: u32,
        k_out: *mut i32,
        v_out: *mut i32,
    ) -> c_int;
    pub fn iris_session_time_decode(
        session: *mut IrisSession,
        prompt: *const i32,
        prompt_len: u32,
        steps: u32,
        ms_per_token: *mut f64,
        prefill_ms: *mut f64,
        out_tokens: *mut i32,
    ) -> c_int;
    pub fn iris_session_time_decode_launches(
        session: *mut IrisSession,
        prompt: *const i32,
        prompt_len: u32,
        steps: u32,
        use_graph: c_int,
        ms_per_token: *mut f64,
        prefill_ms: *mut f64,
        out_tokens: *mut i32,
    ) -> c_int;
    pub fn iris_kernel_tracer_loaded() -> c_int;
    pub fn iris_session_time_pass(session: *mut IrisSession, ids: *const i32, count: u32, ms: *mut f64) -> c_int;
    pub fn iris_attention_numerics(
        diff: *const u32,
        e: *const u64,
        sum: *const u64,
        dot: *const i64,
        scale_q32: u32,
        n: u32,
        exp_out: *mut u64,
        weight_out: *mut i32,
        score_out: *mut i32,
    ) -> c_int;
    pub fn iris_silu_device(x: *const i32, n: u32, out: *mut i32) -> c_int;
    pub fn iris_silu_table_device(x: *const i32, n: u32, out: *mut i32) -> c_int;
    pub fn iris_sha256_bytes(data: *const u8, len: u64, out: *mut u8) -> c_int;
}
