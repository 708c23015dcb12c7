//! The drop-in for inference-kernels' `gpu` module on an MI355X: the same
//! `slab_product` contract (crates/inference/kernels/src/gpu.rs:233-309) over
//! `MatrixSource`, with libiris_hip in place of the CUDA library.
//!
//! Differences from the CUDA path, all in how bytes travel, none in values:
//! - a matrix goes up as its committed `Q8_0` parts (`q8gpu_upload_q8_0`),
//!   not de-interleaved weights plus expanded i64 scales;
//! - uploads are kept by `Q8Key` with least-recently-used eviction under
//!   `IRIS_GPU_WEIGHT_BYTES`, as the reference keeps them;
//! - every product is still spot-checked against `row_dot`, and a
//!   disagreement is an error, not a fallback.
//!
//! Wiring (in crates/inference/kernels): `tensor.rs`'s GPU hook
//! (`linear_slab_from_source`, tensor.rs:445-448) calls
//! `iris_hip::backend::slab_product` under the `gpu-kernels` feature.

use std::collections::HashMap;
use std::sync::Mutex;

use anyhow::{bail, Result};
use inference_kernels::tensor::{MatrixSource, Q8Key, Slab};

use crate::DeviceMatrix;

const DEFAULT_MIN_WORK: u64 = 1 << 28;
const DEFAULT_WEIGHT_BYTES: u64 = 64 << 30;
const SPOT_CHECKS: usize = 64;

struct Held {
    matrix: DeviceMatrix,
    bytes: u64,
    last_used: u64,
}

#[derive(Default)]
struct Device {
    ready: bool,
    failed: bool,
    held: HashMap<Q8Key, Held>,
    held_bytes: u64,
    clock: u64,
    sample: u64,
}

static DEVICE: Mutex<Option<Device>> = Mutex::new(None);

fn number(name: &str, default: u64) -> u64 {
    std::env::var(name).ok().and_then(|v| v.parse().ok()).unwrap_or(default)
}

fn enabled() -> bool {
    !std::env::var("IRIS_GPU_KERNELS").is_ok_and(|v| v.eq_ignore_ascii_case("off"))
}

impl Device {
    fn fail(&mut self, what: &str, error: &crate::Error) {
        if !self.failed {
            eprintln!("iris: GPU kernels disabled, continuing on the CPU: {what} failed: {error}");
        }
        self.failed = true;
    }

    fn start(&mut self) -> bool {
        if self.failed {
            return false;
        }
        if !self.ready {
            if let Err(e) = crate::init() {
                self.fail("starting the device", &e);
                return false;
            }
            self.ready = true;
        }
        true
    }

    fn next_sample(&mut self) -> u64 {
        self.sample = self.sample.wrapping_add(0x9E37_79B9_7F4A_7C15);
        let mut z = self.sample;
        z = (z ^ (z >> 30)).wrapping_mul(0xBF58_476D_1CE4_E5B9);
        z = (z ^ (z >> 27)).wrapping_mul(0x94D0_49BB_1331_11EB);
        z ^ (z >> 31)
    }
}

/// `matrix` applied to every row of `input` on the device, or `None` when the
/// product should stay on the CPU (small, not `Q8_0`, or no device).
pub fn slab_product<M: MatrixSource + ?Sized>(input: &Slab, matrix: &M) -> Result<Option<Slab>> {
    if !enabled() {
        return Ok(None);
    }
    let (rows, cols, tokens) = (matrix.rows(), matrix.cols(), input.rows());
    if (tokens as u64) * (rows as u64) * (cols as u64) < number("IRIS_GPU_MIN_WORK", DEFAULT_MIN_WORK) {
        return Ok(None);
    }
    let Some(source) = matrix.q8_source() else {
        return Ok(None);
    };
    if tokens == 0 || rows == 0 || input.cols() != cols || [rows, cols, tokens].iter().any(|c| *c > i32::MAX as usize)
    {
        return Ok(None);
    }
    let mut guard = DEVICE.lock().unwrap_or_else(|p| p.into_inner());
    let device = guard.get_or_insert_with(Device::default);
    if !device.start() {
        return Ok(None);
    }
    device.clock += 1;
    let clock = device.clock;
    if !device.held.contains_key(&source.key) {
        let bytes = (rows * cols / 32 * 34) as u64;
        let budget = number("IRIS_GPU_WEIGHT_BYTES", DEFAULT_WEIGHT_BYTES);
        if bytes > budget {
            return Ok(None);
        }
        while device.held_bytes + bytes > budget {
            let Some(oldest) = device.held.iter().min_by_key(|(_, h)| h.last_used).map(|(k, _)| *k) else {
                break;
            };
            if let Some(evicted) = device.held.remove(&oldest) {
                device.held_bytes -= evicted.bytes;
            }
        }
        match DeviceMatrix::upload_q8_0(&source.parts, rows, cols) {
            Ok(matrix) => {
                device.held.insert(source.key, Held { matrix, bytes, last_used: clock });
                device.held_bytes += bytes;
            }
            // A scale the CPU would reject is the CPU's error to report.
            Err(e) if e.code == crate::E_SCALE => return Ok(None),
            Err(e) => {
                device.fail("uploading weights", &e);
                return Ok(None);
            }
        }
    }
    let held = device.held.get_mut(&source.key).expect("uploaded above");
    held.last_used = clock;
    let values = match held.matrix.product(input.as_flat(), tokens) {
        Ok(v) => v,
        Err(e) => {
            device.fail("a product", &e);
            return Ok(None);
        }
    };
    let mut output = Slab::zeroed(tokens, rows);
    output.as_flat_mut().copy_from_slice(&values);
    let outputs = tokens * rows;
    let picks: Vec<usize> = (0..SPOT_CHECKS).map(|_| (device.next_sample() % outputs as u64) as usize).collect();
    drop(guard);
    for index in picks.into_iter().chain([0, outputs - 1]) {
        let (token, row) = (index / rows, index % rows);
        let expected = matrix.row_dot(row, input.row(token))?;
        let actual = output.row(token)[row];
        if actual != expected {
            bail!(
                "GPU Q8_0 product disagrees with the CPU at token {token}, row {row} of a \
                 {rows}x{cols} matrix: {actual} against {expected}"
            );
        }
    }
    Ok(Some(output))
}
