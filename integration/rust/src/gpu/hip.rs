//! hip — the MI355X (gfx950) backend of the quantized projection path, as a module of the engine
//! crate: `src/gpu/hip.rs`, declared `#[cfg(feature = "hip")] pub mod hip;` in `src/gpu/mod.rs`
//! (Cargo.toml: `hip = []`).
//!
//! A run-time `dlopen` of `libapeiron_hip.so` (the C ABI of `include/apeiron_hip.h` in the
//! apeiron-amd tree) through the `libc` the crate already depends on: no link-time dependency and
//! no new crate.  `Hip::load` returning `Err(String)` is an honest skip — no library, a missing
//! symbol, or no gfx950 device — exactly as `Vk::load` treats a missing Vulkan loader
//! (`src/gpu/vulkan.rs:1097-1106`); the engine then keeps its CPU kernels.
//!
//! Every ABI status maps to exactly one error value (`HipError::from_status`): statuses 1-9 to the
//! nine `MatvecError` variants (`src/engine/ops/matvec.rs:11-48`) with their struct fields filled
//! from the call, 10-11 to `F32Error`, 12-14 to `FfnError`, 20-25 to `HipError::Backend`.
//!
//! Written against the reference tree's types; this repository has no Rust toolchain, so the
//! module is compiled only where it is integrated (its C twin, `tests/cpp/abi_driver.cpp`, runs
//! the same calls against the same library in this repository's tests).
#![allow(unsafe_code, reason = "an FFI boundary: every unsafe block calls into the loaded library")]

use std::collections::HashMap;
use std::ffi::{c_void, CStr};
use std::os::raw::{c_char, c_int};

use crate::engine::loader::PayloadRef;
use crate::engine::num::fp::F32;
use crate::engine::{EngineError, F32Error, FfnError, MatvecError};

/// `ah_ctx` / `ah_tensor` of the C ABI: opaque handles.
#[repr(C)]
pub struct AhCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct AhTensor {
    _p: [u8; 0],
}

/// Status codes of `include/apeiron_hip.h`.
pub const AH_OK: i32 = 0;
pub const AH_ERR_NO_DEVICE: i32 = 20;

type Init = unsafe extern "C" fn(c_int, *mut *mut AhCtx) -> i32;
type Destroy = unsafe extern "C" fn(*mut AhCtx) -> i32;
type StatusStr = unsafe extern "C" fn(i32) -> *const c_char;
type Upload = unsafe extern "C" fn(*mut AhCtx, u32, *const c_void, usize, usize, usize, *mut *mut AhTensor) -> i32;
type FreeTensor = unsafe extern "C" fn(*mut AhCtx, *mut AhTensor) -> i32;
type MatvecQ8 = unsafe extern "C" fn(*mut AhCtx, *const AhTensor, *const i8, *const i64, usize, *mut f32) -> i32;
type MatmatQ8 = unsafe extern "C" fn(*mut AhCtx, *const AhTensor, *const i8, *const i64, usize, *mut f32) -> i32;
type QuantAct = unsafe extern "C" fn(*mut AhCtx, *const i64, usize, *mut i8, *mut i64) -> i32;
type RefusalBits = unsafe extern "C" fn(*mut AhCtx, *mut u32) -> i32;
type ProbeMfma = unsafe extern "C" fn(*mut AhCtx, u32, *mut f64) -> i32;

/// The resolved entry points.
#[derive(Clone, Copy)]
struct Fns {
    destroy: Destroy,
    status_str: StatusStr,
    upload: Upload,
    free_tensor: FreeTensor,
    matvec: MatvecQ8,
    matmat: MatmatQ8,
    quant: QuantAct,
    refusal_bits: RefusalBits,
    probe: ProbeMfma,
}

/// A refusal or failure of a backend call: one value per ABI status.
#[derive(Debug, Clone, PartialEq, Eq)]
pub enum HipError {
    /// Statuses 1-9: the projection contract's own refusal.
    Matvec(MatvecError),
    /// Statuses 10-11: an f32 input the Q32.32 conversion refuses.
    Input(F32Error),
    /// Statuses 12-14: the SwiGLU stage's refusal.
    Ffn(FfnError),
    /// Statuses 20-25 (and any status this build does not know): the backend itself failed —
    /// no device, a bad argument, the HIP runtime, device memory, fixed scratch, a barrier
    /// timeout.  The engine answers these with its CPU path.
    Backend { status: i32, what: String },
}

/// What a call knew about its operands, for the struct-variant fields of `MatvecError`.
#[derive(Clone, Copy, Default)]
pub struct CallShape {
    pub ggml_type: u32,
    pub n_in: usize,
    pub x_len: usize,
    pub need: usize,
    pub have: usize,
}

impl HipError {
    /// The one error value of ABI status `st` (Ok for 0).  `bits` is the f16 scale word behind a
    /// NonFiniteScale refusal (`ah_last_refusal_bits`).
    pub fn from_status(st: i32, shape: CallShape, bits: u16, what: &str) -> Result<(), HipError> {
        let m = |e: MatvecError| Err(HipError::Matvec(e));
        match st {
            0 => Ok(()),
            1 => m(MatvecError::ShapeMismatch { x: shape.x_len, n_in: shape.n_in }),
            2 => m(MatvecError::RowLength { row: 0, weights: 0, n_in: shape.n_in }),
            3 => m(MatvecError::ShortPayload { need: shape.need, have: shape.have }),
            4 => m(MatvecError::LengthOverflow),
            5 => m(MatvecError::UnsupportedQuant { ggml_type: shape.ggml_type }),
            6 => m(MatvecError::Dequant(EngineError::NonFiniteScale { bits })),
            7 => m(MatvecError::Dequant(EngineError::FixedOverflow)),
            8 => m(MatvecError::AccumulatorOverflow),
            9 => m(MatvecError::OutputOverflow),
            10 => Err(HipError::Input(F32Error::NonFinite)),
            11 => Err(HipError::Input(F32Error::OutOfRange)),
            12 => Err(HipError::Ffn(FfnError::Overflow)),
            13 => Err(HipError::Ffn(FfnError::ExpOutOfRange)),
            14 => Err(HipError::Ffn(FfnError::ZeroDenominator)),
            status => Err(HipError::Backend { status, what: what.to_owned() }),
        }
    }
}

/// One device copy of a projection tensor.
struct Resident {
    t: *mut AhTensor,
    ggml_type: u32,
    n_out: usize,
    n_in: usize,
}

/// The loaded backend: one context on one GPU and the engine's resident projection tensors,
/// keyed by directory index.  Not thread-safe (one context, as the reference's pool lock).
pub struct Hip {
    lib: *mut c_void,
    ctx: *mut AhCtx,
    f: Fns,
    tensors: HashMap<usize, Resident>,
}

// SAFETY: the context and tensor handles are plain device-side objects of the library, usable from
// any thread as long as calls on one context do not overlap; the engine keeps `Hip` behind a
// Mutex, which serialises them.
unsafe impl Send for Hip {}

unsafe fn sym<T: Copy>(lib: *mut c_void, name: &[u8]) -> Result<T, String> {
    let p = libc::dlsym(lib, name.as_ptr().cast::<c_char>());
    if p.is_null() {
        let n = CStr::from_bytes_with_nul(name).map(|c| c.to_string_lossy().into_owned()).unwrap_or_default();
        return Err(format!("libapeiron_hip.so: missing symbol {n}"));
    }
    Ok(std::mem::transmute_copy::<*mut c_void, T>(&p))
}

impl Hip {
    /// Load the library and create a context on `device`.  `Err(msg)` = honest skip (no library,
    /// a missing symbol, no gfx950 device), never a hard failure.
    ///
    /// # Safety
    /// Loads and runs foreign code; the library must be the one `include/apeiron_hip.h` describes.
    pub unsafe fn load(device: i32) -> Result<Hip, String> {
        let lib = libc::dlopen(b"libapeiron_hip.so\0".as_ptr().cast::<c_char>(), libc::RTLD_NOW);
        if lib.is_null() {
            return Err("libapeiron_hip.so not found".into());
        }
        let init: Init = match sym(lib, b"ah_init\0") {
            Ok(f) => f,
            Err(e) => {
                libc::dlclose(lib);
                return Err(e);
            }
        };
        let resolved = (|| -> Result<Fns, String> {
            Ok(Fns {
                destroy: sym(lib, b"ah_destroy\0")?,
                status_str: sym(lib, b"ah_status_str\0")?,
                upload: sym(lib, b"ah_upload_weight\0")?,
                free_tensor: sym(lib, b"ah_free_tensor\0")?,
                matvec: sym(lib, b"ah_matvec_q8act\0")?,
                matmat: sym(lib, b"ah_matmat_q8act\0")?,
                quant: sym(lib, b"ah_quant_act\0")?,
                refusal_bits: sym(lib, b"ah_last_refusal_bits\0")?,
                probe: sym(lib, b"ah_probe_mfma_peak\0")?,
            })
        })();
        let f = match resolved {
            Ok(f) => f,
            Err(e) => {
                libc::dlclose(lib);
                return Err(e);
            }
        };
        let mut ctx: *mut AhCtx = std::ptr::null_mut();
        let st = init(device, &mut ctx);
        if st != AH_OK {
            let msg = CStr::from_ptr((f.status_str)(st)).to_string_lossy().into_owned();
            libc::dlclose(lib);
            return Err(format!("ah_init: {msg} (status {st})"));
        }
        Ok(Hip { lib, ctx, f, tensors: HashMap::new() })
    }

    fn check(&self, st: i32, shape: CallShape, what: &str) -> Result<(), HipError> {
        let mut bits = 0u32;
        if st == 6 {
            // SAFETY: ctx is live for &self; the call only reads the context.
            unsafe { (self.f.refusal_bits)(self.ctx, &mut bits) };
        }
        HipError::from_status(st, shape, bits as u16, what)
    }

    /// Upload tensor `idx`'s GGUF payload (`resident()[at.off..at.off + at.len]`, the bytes the
    /// engine's CPU path reads) once at load.  A NonFiniteScale refusal is returned as the
    /// reference's row dequantizer would return it; the engine then keeps that tensor on the CPU.
    pub fn upload(&mut self, idx: usize, ggml_type: u32, file: &[u8], at: PayloadRef, n_out: usize,
                  n_in: usize) -> Result<(), HipError> {
        let raw = at.bytes(file);
        let mut t: *mut AhTensor = std::ptr::null_mut();
        // SAFETY: raw is a live slice for the call; the library copies it to the device.
        let st = unsafe {
            (self.f.upload)(self.ctx, ggml_type, raw.as_ptr().cast::<c_void>(), raw.len(), n_out, n_in, &mut t)
        };
        let shape = CallShape { ggml_type, n_in, x_len: n_in, need: 0, have: raw.len() };
        self.check(st, shape, "ah_upload_weight")?;
        if let Some(old) = self.tensors.insert(idx, Resident { t, ggml_type, n_out, n_in }) {
            // SAFETY: old.t came from ah_upload_weight on this context and is dropped once.
            unsafe { (self.f.free_tensor)(self.ctx, old.t) };
        }
        Ok(())
    }

    /// True when tensor `idx` is resident on the device.
    pub fn has(&self, idx: usize) -> bool {
        self.tensors.contains_key(&idx)
    }

    /// `matvec_q8act` (`src/engine/chart/mod.rs:1887`) of resident tensor `idx` on a QuantAct's
    /// codes and scales (`QuantAct::codes()` / `scales()`), as Q32.32 outputs: `F32::to_q32` of
    /// each f32 row value, within 1e-4 * sum|w * xhat| + 2^-32 of the exact round_shift_32 value.
    pub fn matvec_q8act(&self, idx: usize, codes: &[i8], scales: &[i64]) -> Result<Vec<i64>, HipError> {
        let r = self.tensors.get(&idx).ok_or(HipError::Backend { status: 21, what: "tensor not resident".into() })?;
        let mut y = vec![0f32; r.n_out];
        if scales.len() != codes.len().div_ceil(32) {
            return Err(HipError::Backend { status: 21, what: "scales length".into() });
        }
        // SAFETY: codes, scales and y are live for the call with the lengths passed.
        let st = unsafe { (self.f.matvec)(self.ctx, r.t, codes.as_ptr(), scales.as_ptr(), codes.len(), y.as_mut_ptr()) };
        let shape = CallShape { ggml_type: r.ggml_type, n_in: r.n_in, x_len: codes.len(), need: 0, have: 0 };
        self.check(st, shape, "ah_matvec_q8act")?;
        y.iter().map(|v| F32(v.to_bits()).to_q32().ok_or(HipError::Matvec(MatvecError::OutputOverflow))).collect()
    }

    /// `matmat_q8act` (`src/engine/kern/matmat.rs:134`) of resident tensor `idx` over `qs`
    /// (codes and scales per column), one Q32.32 vector per column.
    pub fn matmat_q8act(&self, idx: usize, qs: &[(&[i8], &[i64])]) -> Result<Vec<Vec<i64>>, HipError> {
        let r = self.tensors.get(&idx).ok_or(HipError::Backend { status: 21, what: "tensor not resident".into() })?;
        let nb = r.n_in.div_ceil(32);
        let mut codes = Vec::with_capacity(qs.len() * r.n_in);
        let mut scales = Vec::with_capacity(qs.len() * nb);
        for (c, s) in qs {
            if c.len() != r.n_in {
                return Err(HipError::Matvec(MatvecError::ShapeMismatch { x: c.len(), n_in: r.n_in }));
            }
            if s.len() != nb {
                return Err(HipError::Backend { status: 21, what: "scales length".into() });
            }
            codes.extend_from_slice(c);
            scales.extend_from_slice(s);
        }
        let mut y = vec![0f32; qs.len() * r.n_out];
        // SAFETY: the buffers are live for the call, token-major [n_tok][n_in] / [n_tok][nb].
        let st = unsafe { (self.f.matmat)(self.ctx, r.t, codes.as_ptr(), scales.as_ptr(), qs.len(), y.as_mut_ptr()) };
        let shape = CallShape { ggml_type: r.ggml_type, n_in: r.n_in, x_len: r.n_in, need: 0, have: 0 };
        self.check(st, shape, "ah_matmat_q8act")?;
        y.chunks(r.n_out.max(1))
            .take(qs.len())
            .map(|col| col.iter().map(|v| F32(v.to_bits()).to_q32().ok_or(HipError::Matvec(MatvecError::OutputOverflow))).collect())
            .collect()
    }

    /// `quant_act` (`src/engine/chart/mod.rs:258`) on the device: bit-identical codes and scales,
    /// `Ok(None)` where the reference returns None (an activation with no Q32.32 value).
    pub fn quant_act(&self, x: &[i64]) -> Result<Option<(Vec<i8>, Vec<i64>)>, HipError> {
        let mut codes = vec![0i8; x.len()];
        let mut scales = vec![0i64; x.len().div_ceil(32)];
        // SAFETY: the buffers are live for the call with the lengths passed.
        let st = unsafe { (self.f.quant)(self.ctx, x.as_ptr(), x.len(), codes.as_mut_ptr(), scales.as_mut_ptr()) };
        match self.check(st, CallShape::default(), "ah_quant_act") {
            Ok(()) => Ok(Some((codes, scales))),
            Err(HipError::Matvec(MatvecError::Dequant(EngineError::FixedOverflow))) => Ok(None),
            Err(e) => Err(e),
        }
    }

    /// The device's measured MFMA-only rate (kind 0: int8 32x32x32, 1: f16 32x32x16), tera-ops/s:
    /// a diagnostic beside the engine's DP4A roofline probe, never on the projection path.
    pub fn probe_mfma_peak(&self, kind: u32) -> Result<f64, HipError> {
        let mut v = 0f64;
        // SAFETY: v is live for the call.
        let st = unsafe { (self.f.probe)(self.ctx, kind, &mut v) };
        self.check(st, CallShape::default(), "ah_probe_mfma_peak")?;
        Ok(v)
    }
}

impl Drop for Hip {
    fn drop(&mut self) {
        // SAFETY: every handle came from this context; the context and library are released last.
        unsafe {
            for (_, r) in self.tensors.drain() {
                (self.f.free_tensor)(self.ctx, r.t);
            }
            (self.f.destroy)(self.ctx);
            libc::dlclose(self.lib);
        }
    }
}
