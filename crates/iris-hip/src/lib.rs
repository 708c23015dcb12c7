//! Safe Rust over libiris_hip: exact Q8_0 products and the deterministic
//! token loop on an AMD Instinct MI355X (gfx950).
//!
//! - [`DeviceMatrix`]: a `Q8_0` matrix on the device and its products, the
//!   same values as `det_num::q8::dot_row` for every output.
//! - [`Model`] and [`Session`]: one family's weights on the device and a KV
//!   cache, for greedy generation (`DirectInferenceExecutor::run`,
//!   crates/inference/direct/src/executor.rs:41-290) and the staged
//!   teacher-forced pass over ranges with carried keys
//!   (crates/inference/kernels/src/mistral/stage.rs:172-226).
//!
//! inference-kernels' own `gpu` module (crates/inference/kernels/src/gpu.rs)
//! needs none of this: it links the five `q8gpu_*` symbols of the library
//! unchanged.
//!
//! Every call returns `Err` with the library's own text for any nonzero
//! code; nothing falls back to the CPU here.

pub mod ffi;

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::c_int;

/// A nonzero return code of the library and its text (`q8gpu_error`).
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct Error {
    pub code: i32,
    pub text: String,
    pub what: &'static str,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "{} failed: {} (code {})", self.what, self.text, self.code)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

/// Library codes (negative; positive codes are hipError_t values).
pub const E_INVALID: i32 = -1;
pub const E_SCALE: i32 = -2;
pub const E_NOMEM: i32 = -3;
pub const E_STATE: i32 = -4;
pub const E_RANGE: i32 = -5;
pub const E_SCRATCH: i32 = -6;
pub const E_TRACED: i32 = -7;

pub fn error_text(code: i32) -> String {
    // SAFETY: q8gpu_error returns a static NUL-terminated string for any code.
    unsafe { CStr::from_ptr(ffi::q8gpu_error(code as c_int)) }
        .to_string_lossy()
        .into_owned()
}

fn check(code: c_int, what: &'static str) -> Result<()> {
    if code == 0 {
        Ok(())
    } else {
        Err(Error { code, text: error_text(code), what })
    }
}

/// Creates the device context (`q8gpu_init`).
pub fn init() -> Result<()> {
    // SAFETY: no arguments.
    check(unsafe { ffi::q8gpu_init() }, "q8gpu_init")
}

/// A `Q8_0` matrix on the device.
pub struct DeviceMatrix {
    ptr: *mut ffi::Q8GpuMatrix,
    pub rows: usize,
    pub cols: usize,
}

// SAFETY: the library serialises its host round trip, and a matrix changes
// only through `prepare_matrix_cores`, which takes `&mut self` (no product
// can run on it meanwhile); products may be issued from any thread.
unsafe impl Send for DeviceMatrix {}
unsafe impl Sync for DeviceMatrix {}

impl DeviceMatrix {
    /// From committed `Q8_0` rows (`rows` x `cols/32` blocks of 34 bytes),
    /// in one piece or several whole-block pieces, in order (the reference's
    /// `Q8Source::parts`, crates/inference/kernels/src/tensor.rs:110-115).
    pub fn upload_q8_0(parts: &[&[u8]], rows: usize, cols: usize) -> Result<Self> {
        let bytes: usize = parts.iter().map(|p| p.len()).sum();
        if cols == 0 || cols % 32 != 0 || bytes != rows * cols / 32 * 34 || rows > u32::MAX as usize {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "Q8_0 upload" });
        }
        let joined;
        let data: &[u8] = if parts.len() == 1 {
            parts[0]
        } else {
            joined = parts.concat();
            &joined
        };
        let mut ptr = std::ptr::null_mut();
        // SAFETY: `data` holds exactly rows * cols/32 * 34 bytes.
        check(unsafe { ffi::q8gpu_upload_q8_0(data.as_ptr(), rows as u32, cols as u32, &mut ptr) }, "Q8_0 upload")?;
        Ok(Self { ptr, rows, cols })
    }

    /// The reference device ABI's form: weights `rows*cols` and one Q.24
    /// scale per block (crates/inference/kernels/cuda/q8_product.cu:150-172).
    pub fn upload(weights: &[i8], scales: &[i64], rows: usize, cols: usize) -> Result<Self> {
        if cols % 32 != 0 || weights.len() != rows * cols || scales.len() != rows * cols / 32 {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "upload" });
        }
        let mut ptr = std::ptr::null_mut();
        // SAFETY: the slices hold the sizes the library reads.
        check(
            unsafe { ffi::q8gpu_upload(weights.as_ptr(), scales.as_ptr(), rows as u32, cols as u32, &mut ptr) },
            "upload",
        )?;
        Ok(Self { ptr, rows, cols })
    }

    /// `out[t * rows + r] = dot_row(input[t], W[r])` for `tokens` rows of
    /// `cols` Q16.16 values in host memory (synchronous).
    pub fn product(&self, input: &[i32], tokens: usize) -> Result<Vec<i32>> {
        if input.len() != tokens * self.cols {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "Q8_0 product" });
        }
        let mut out = vec![0i32; tokens * self.rows];
        if tokens == 0 {
            return Ok(out);
        }
        // SAFETY: `input` holds tokens*cols values and `out` tokens*rows.
        check(
            unsafe { ffi::q8gpu_product(self.ptr, input.as_ptr(), tokens as u32, out.as_mut_ptr()) },
            "Q8_0 product",
        )?;
        Ok(out)
    }

    /// Folds a per-block scale matrix for the int8 matrix cores, so that its
    /// multi-token products run there (more device memory, see `info`);
    /// nothing for a row-scale matrix. Synchronous.
    pub fn prepare_matrix_cores(&mut self) -> Result<()> {
        // SAFETY: a live matrix, borrowed mutably: no other call uses it.
        check(unsafe { ffi::q8gpu_prepare_matrix_cores(self.ptr, std::ptr::null_mut()) }, "prepare matrix cores")
    }

    /// (rows, cols, scale layout, device bytes).
    pub fn info(&self) -> Result<(u32, u32, i32, u64)> {
        let (mut r, mut c, mut m, mut b) = (0u32, 0u32, 0 as c_int, 0u64);
        // SAFETY: all out-pointers are valid locals.
        check(unsafe { ffi::q8gpu_matrix_info(self.ptr, &mut r, &mut c, &mut m, &mut b) }, "matrix info")?;
        Ok((r, c, m, b))
    }

    pub fn as_ptr(&self) -> *const ffi::Q8GpuMatrix {
        self.ptr
    }
}

impl Drop for DeviceMatrix {
    fn drop(&mut self) {
        // SAFETY: the pointer came from an upload and is freed once.
        unsafe { ffi::q8gpu_free(self.ptr) }
    }
}

/// Tensor element widths `Model::set_tensor` takes.
#[derive(Clone, Copy, Debug)]
pub enum Width {
    /// Q8_0 rows (rows x cols/32 blocks of 34 bytes).
    Q8_0,
    /// Q16.16 values as i32.
    I32,
    /// i64 values (mistral-dense's `rope_inverse_frequencies`).
    I64,
}

/// One family's weights on the device (`DirectInferenceModel`,
/// crates/inference/direct/src/model.rs:167-677).
pub struct Model {
    ptr: *mut ffi::IrisModel,
    pub desc: ffi::IrisModelDesc,
    _sliding: Vec<u8>,
}

unsafe impl Send for Model {}

impl Model {
    /// `layer_is_sliding` (gemma-dense): one entry per layer.
    pub fn create(mut desc: ffi::IrisModelDesc, layer_is_sliding: &[bool]) -> Result<Self> {
        let sliding: Vec<u8> = layer_is_sliding.iter().map(|&s| s as u8).collect();
        desc.layer_is_sliding = if sliding.is_empty() { std::ptr::null() } else { sliding.as_ptr() };
        let mut ptr = std::ptr::null_mut();
        // SAFETY: desc and the sliding flags outlive the call.
        check(unsafe { ffi::iris_model_create(&desc, &mut ptr) }, "model create")?;
        desc.layer_is_sliding = std::ptr::null();
        Ok(Self { ptr, desc, _sliding: sliding })
    }

    /// Hands one DETWGT tensor to the model by its name; `data` holds its
    /// bytes (Q8_0 rows, or little-endian i32 / i64 values).
    pub fn set_tensor(&mut self, name: &str, width: Width, data: &[u8], rows: u64, cols: u64) -> Result<()> {
        let (w, need) = match width {
            Width::Q8_0 => (8, rows * (cols / 32) * 34),
            Width::I32 => (32, rows * cols * 4),
            Width::I64 => (64, rows * cols * 8),
        };
        if data.len() as u64 != need {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "set tensor" });
        }
        let cname = CString::new(name).map_err(|_| Error { code: E_INVALID, text: error_text(E_INVALID), what: "set tensor" })?;
        // SAFETY: `data` holds the bytes the width and shape describe.
        check(
            unsafe { ffi::iris_model_set_tensor(self.ptr, cname.as_ptr(), w, data.as_ptr().cast(), rows, cols) },
            "set tensor",
        )
    }

    pub fn finalize(&mut self) -> Result<()> {
        // SAFETY: a live model.
        check(unsafe { ffi::iris_model_finalize(self.ptr) }, "model finalize")
    }

    pub fn device_bytes(&self) -> u64 {
        // SAFETY: a live model.
        unsafe { ffi::iris_model_device_bytes(self.ptr) }
    }
}

impl Drop for Model {
    fn drop(&mut self) {
        // SAFETY: freed once; sessions borrow the model, so none outlives it.
        unsafe { ffi::iris_model_free(self.ptr) }
    }
}

/// A KV cache over a model and its passes.
pub struct Session<'m> {
    ptr: *mut ffi::IrisSession,
    model: &'m Model,
    pub max_positions: u32,
}

/// A layer's keys and values of consecutive positions, one row of
/// kv_heads*head_dim values each (the reference's `KeyRow` k and v,
/// raster-stages/prefill-range/src/input.rs:185-189).
#[derive(Clone, Debug, Default, PartialEq, Eq)]
pub struct Keys {
    pub first_position: u32,
    pub k: Vec<Vec<i32>>,
    pub v: Vec<Vec<i32>>,
}

impl<'m> Session<'m> {
    pub fn create(model: &'m Model, max_positions: u32, max_rows: u32) -> Result<Self> {
        let mut ptr = std::ptr::null_mut();
        // SAFETY: a finalized model; the session is freed before it.
        check(unsafe { ffi::iris_session_create(model.ptr, max_positions, max_rows, &mut ptr) }, "session create")?;
        Ok(Self { ptr, model, max_positions })
    }

    /// Greedy generation (executor.rs:143-185): (token ids, the logits each
    /// selection was made from when asked).
    pub fn generate(
        &mut self,
        prompt: &[i32],
        tokens: u32,
        eos: &[i32],
        keep_logits: bool,
    ) -> Result<(Vec<i32>, Option<Vec<i32>>)> {
        let vocab = self.model.desc.vocab as usize;
        let mut out = vec![0i32; tokens.max(1) as usize];
        let mut logits = if keep_logits { Some(vec![0i32; tokens.max(1) as usize * vocab]) } else { None };
        let mut count = 0u32;
        let eos_ptr = if eos.is_empty() { [0i32].as_ptr() } else { eos.as_ptr() };
        // SAFETY: out holds `tokens` ids and logits tokens*vocab values.
        check(
            unsafe {
                ffi::iris_session_generate(
                    self.ptr,
                    prompt.as_ptr(),
                    prompt.len() as u32,
                    tokens,
                    eos_ptr,
                    eos.len() as u32,
                    out.as_mut_ptr(),
                    &mut count,
                    logits.as_mut().map_or(std::ptr::null_mut(), |l| l.as_mut_ptr()),
                    1,
                )
            },
            "generate",
        )?;
        out.truncate(count as usize);
        if let Some(l) = logits.as_mut() {
            l.truncate(count as usize * vocab);
        }
        Ok((out, logits))
    }

    /// Every layer over one range of ids at `start_position`: per-layer
    /// output rows (layers x count x hidden) and SHA-256 of each layer's rows.
    pub fn layer_range(&mut self, ids: &[i32], start_position: u32) -> Result<(Vec<i32>, Vec<[u8; 32]>)> {
        let d = &self.model.desc;
        let mut rows = vec![0i32; d.layers as usize * ids.len() * d.hidden as usize];
        let mut hashes = vec![[0u8; 32]; d.layers as usize];
        // SAFETY: rows and hashes hold what the call writes.
        check(
            unsafe {
                ffi::iris_session_layer_range(
                    self.ptr,
                    ids.as_ptr(),
                    ids.len() as u32,
                    start_position,
                    rows.as_mut_ptr(),
                    hashes.as_mut_ptr().cast(),
                )
            },
            "layer range",
        )?;
        Ok((rows, hashes))
    }

    /// One layer's stage over a range: the layer's rows for `in_rows`
    /// (count x hidden), with its PLE rows for gemma-dense.
    pub fn layer_stage(
        &mut self,
        layer: u32,
        in_rows: &[i32],
        start_position: u32,
        ple_rows: Option<&[i32]>,
    ) -> Result<Vec<i32>> {
        let hidden = self.model.desc.hidden as usize;
        if hidden == 0 || in_rows.len() % hidden != 0 {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "layer stage" });
        }
        let count = in_rows.len() / hidden;
        let mut out = vec![0i32; in_rows.len()];
        // SAFETY: in/out rows hold count*hidden values, ple rows count*ple_width.
        check(
            unsafe {
                ffi::iris_session_layer_stage(
                    self.ptr,
                    layer,
                    in_rows.as_ptr(),
                    count as u32,
                    start_position,
                    ple_rows.map_or(std::ptr::null(), |p| p.as_ptr()),
                    out.as_mut_ptr(),
                )
            },
            "layer stage",
        )?;
        Ok(out)
    }

    /// Carried keys into a layer's cache.
    pub fn write_kv(&mut self, layer: u32, keys: &Keys) -> Result<()> {
        let k: Vec<i32> = keys.k.concat();
        let v: Vec<i32> = keys.v.concat();
        if k.len() != v.len() || keys.k.len() != keys.v.len() {
            return Err(Error { code: E_INVALID, text: error_text(E_INVALID), what: "write kv" });
        }
        // SAFETY: k and v hold count rows of the layer's kv width.
        check(
            unsafe {
                ffi::iris_session_write_kv(
                    self.ptr,
                    layer,
                    keys.first_position,
                    keys.k.len() as u32,
                    k.as_ptr(),
                    v.as_ptr(),
                )
            },
            "write kv",
        )
    }

    /// A layer's cached keys of positions pos0..pos0+count (`kv_width` =
    /// kv_heads * that layer's head_dim).
    pub fn read_kv(&mut self, layer: u32, pos0: u32, count: u32, kv_width: usize) -> Result<Keys> {
        let n = count as usize * kv_width;
        let (mut k, mut v) = (vec![0i32; n], vec![0i32; n]);
        // SAFETY: k and v hold count*kv_width values.
        check(
            unsafe { ffi::iris_session_read_kv(self.ptr, layer, pos0, count, k.as_mut_ptr(), v.as_mut_ptr()) },
            "read kv",
        )?;
        let split = |x: Vec<i32>| x.chunks(kv_width.max(1)).map(|c| c.to_vec()).collect();
        Ok(Keys { first_position: pos0, k: split(k), v: split(v) })
    }
}

impl Drop for Session<'_> {
    fn drop(&mut self) {
        // SAFETY: freed once, before its model.
        unsafe { ffi::iris_session_free(self.ptr) }
    }
}
