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
//! Two kinds of call: the host forms (`matvec_q8act`, `matmat_q8act`, `quant_act`: host buffers in
//! and out, each call its own copies), and the device-resident forms (`projections_q8act`,
//! `ffn_q8act`, `matmat_group_q8act`, `ffn_cols_q8act`): one upload of the QuantAct per call into
//! a staging region the module keeps on the device, every projection of the call (and the FFN's
//! hidden activation) on the device, one synchronization, one download of the outputs.
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
// device-pointer forms (`stream` NULL: the context's stream)
type SyncStatus = unsafe extern "C" fn(*mut AhCtx, *mut c_void) -> i32;
type GemvQ8Dev = unsafe extern "C" fn(*mut AhCtx, *const AhTensor, *const i8, *const i64, *mut f32, *mut c_void) -> i32;
type GemmGroupQ8Dev = unsafe extern "C" fn(
    *mut AhCtx, usize, *const *const AhTensor, *const i8, *const i64, usize, *const *mut f32, *mut c_void,
) -> i32;
type FfnQ8Dev = unsafe extern "C" fn(
    *mut AhCtx, *const AhTensor, *const AhTensor, *const AhTensor, *const i8, *const i64, *mut f32, *mut i8,
    *mut i64, *mut c_void,
) -> i32;
type FfnPrefillQ8Dev = unsafe extern "C" fn(
    *mut AhCtx, *const AhTensor, *const AhTensor, *const AhTensor, *const i8, *const i64, usize, *mut f32,
    *mut i8, *mut i64, *mut c_void,
) -> i32;
type DevAlloc = unsafe extern "C" fn(*mut AhCtx, usize, *mut *mut c_void) -> i32;
type DevFree = unsafe extern "C" fn(*mut AhCtx, *mut c_void) -> i32;
type CopyToDev = unsafe extern "C" fn(*mut AhCtx, *mut c_void, *const c_void, usize, *mut c_void) -> i32;
type CopyToHost = unsafe extern "C" fn(*mut AhCtx, *mut c_void, *const c_void, usize, *mut c_void) -> i32;

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
    sync: SyncStatus,
    gemv_q8: GemvQ8Dev,
    gemm_group_q8: GemmGroupQ8Dev,
    ffn_q8: FfnQ8Dev,
    ffn_prefill_q8: FfnPrefillQ8Dev,
    dev_alloc: DevAlloc,
    dev_free: DevFree,
    to_dev: CopyToDev,
    to_host: CopyToHost,
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

/// The device staging region of the device-resident forms: one allocation, grown on demand and
/// carved per call into 256-byte aligned pieces (activation codes and scales in, outputs and the
/// FFN's hidden QuantAct out), so a call allocates nothing once the region has its size.
struct Stage {
    d: *mut c_void,
    bytes: usize,
}

/// Offsets of a call's pieces in the staging region.
struct Carve {
    at: Vec<usize>,
    total: usize,
}

impl Carve {
    fn new(sizes: &[usize]) -> Carve {
        let mut at = Vec::with_capacity(sizes.len());
        let mut total = 0usize;
        for &s in sizes {
            at.push(total);
            total += s.div_ceil(256) * 256;
        }
        Carve { at, total }
    }
}

/// The loaded backend: one context on one GPU and the engine's resident projection tensors,
/// keyed by directory index.  Not thread-safe (one context, as the reference's pool lock).
pub struct Hip {
    lib: *mut c_void,
    ctx: *mut AhCtx,
    f: Fns,
    tensors: HashMap<usize, Resident>,
    stage: Stage,
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
                sync: sym(lib, b"ah_sync_status\0")?,
                gemv_q8: sym(lib, b"ah_gemv_q8_dev\0")?,
                gemm_group_q8: sym(lib, b"ah_gemm_group_q8_dev\0")?,
                ffn_q8: sym(lib, b"ah_ffn_q8_dev\0")?,
                ffn_prefill_q8: sym(lib, b"ah_ffn_prefill_q8_dev\0")?,
                dev_alloc: sym(lib, b"ah_dev_alloc\0")?,
                dev_free: sym(lib, b"ah_dev_free\0")?,
                to_dev: sym(lib, b"ah_copy_to_dev\0")?,
                to_host: sym(lib, b"ah_copy_to_host\0")?,
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
        Ok(Hip { lib, ctx, f, tensors: HashMap::new(), stage: Stage { d: std::ptr::null_mut(), bytes: 0 } })
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

    // ---- device-resident forms ------------------------------------------------------------
    //
    // One upload of the activation per call, every projection of the call on the device, one
    // synchronization and one download of the outputs: the grouped decode projections, the FFN
    // with its hidden activation kept on the device, and the prefill forms.

    fn resident(&self, idx: usize) -> Result<&Resident, HipError> {
        self.tensors.get(&idx).ok_or(HipError::Backend { status: 21, what: "tensor not resident".into() })
    }

    /// The staging region with at least `bytes`, as a base address.
    fn stage(&mut self, bytes: usize) -> Result<*mut u8, HipError> {
        if bytes > self.stage.bytes {
            // SAFETY: the old region came from ah_dev_alloc on this context (ah_dev_free waits for
            // the context's stream first).
            unsafe {
                if !self.stage.d.is_null() {
                    (self.f.dev_free)(self.ctx, self.stage.d);
                }
            }
            self.stage = Stage { d: std::ptr::null_mut(), bytes: 0 };
            let want = bytes + bytes / 4;
            let mut d: *mut c_void = std::ptr::null_mut();
            // SAFETY: d receives a device address or stays null.
            let st = unsafe { (self.f.dev_alloc)(self.ctx, want, &mut d) };
            self.check(st, CallShape::default(), "ah_dev_alloc")?;
            self.stage = Stage { d, bytes: want };
        }
        Ok(self.stage.d.cast::<u8>())
    }

    fn upload_bytes<T>(&self, d: *mut u8, host: &[T]) -> Result<(), HipError> {
        let n = std::mem::size_of_val(host);
        // SAFETY: d has room for n bytes (carved from the staging region); host is live.
        let st = unsafe { (self.f.to_dev)(self.ctx, d.cast::<c_void>(), host.as_ptr().cast::<c_void>(), n, std::ptr::null_mut()) };
        self.check(st, CallShape::default(), "ah_copy_to_dev")
    }

    fn download_bytes<T>(&self, host: &mut [T], d: *const u8) -> Result<(), HipError> {
        let n = std::mem::size_of_val(host);
        // SAFETY: d holds n bytes the call wrote; host is live and exclusively borrowed.
        let st = unsafe { (self.f.to_host)(self.ctx, host.as_mut_ptr().cast::<c_void>(), d.cast::<c_void>(), n, std::ptr::null_mut()) };
        self.check(st, CallShape::default(), "ah_copy_to_host")
    }

    /// The f32 outputs as Q32.32 words (`F32::to_q32`, within the tolerance of the exact value).
    fn to_q32(y: &[f32]) -> Result<Vec<i64>, HipError> {
        y.iter().map(|v| F32(v.to_bits()).to_q32().ok_or(HipError::Matvec(MatvecError::OutputOverflow))).collect()
    }

    /// `projections_q8act_prepared` (`src/engine/chart/ffn.rs:940-954`): the resident projections
    /// `idxs` (one n_in) over ONE QuantAct, uploaded once, one launch each on the device, one
    /// synchronization.  The first refusal in projection-then-row order: when the batch refuses,
    /// the projections run again one at a time to name the first (a rare path: the contract's
    /// refusals are overflows).
    pub fn projections_q8act(&mut self, idxs: &[usize], codes: &[i8], scales: &[i64]) -> Result<Vec<Vec<i64>>, HipError> {
        let mut rs: Vec<(*mut AhTensor, u32, usize, usize)> = Vec::with_capacity(idxs.len());
        for &i in idxs {
            let r = self.resident(i)?;
            if r.n_in != codes.len() {
                return Err(HipError::Matvec(MatvecError::ShapeMismatch { x: codes.len(), n_in: r.n_in }));
            }
            rs.push((r.t, r.ggml_type, r.n_out, r.n_in));
        }
        if scales.len() != codes.len().div_ceil(32) {
            return Err(HipError::Backend { status: 21, what: "scales length".into() });
        }
        let mut sizes = vec![codes.len(), 8 * scales.len()];
        sizes.extend(rs.iter().map(|r| 4 * r.2));
        let c = Carve::new(&sizes);
        let base = self.stage(c.total)?;
        // SAFETY (all pointer arithmetic below): every offset lies inside the carve's total.
        let (dc, ds) = unsafe { (base.add(c.at[0]), base.add(c.at[1])) };
        self.upload_bytes(dc, codes)?;
        self.upload_bytes(ds, scales)?;
        let launch_all = |hip: &Hip, upto: Option<usize>| -> i32 {
            for (k, r) in rs.iter().enumerate() {
                if upto.is_some_and(|u| k != u) {
                    continue;
                }
                // SAFETY: device pointers carved above; the tensor is resident on this context.
                let st = unsafe {
                    (hip.f.gemv_q8)(hip.ctx, r.0, dc.cast::<i8>(), ds.cast::<i64>(), base.add(c.at[2 + k]).cast::<f32>(), std::ptr::null_mut())
                };
                if st != AH_OK {
                    return st;
                }
            }
            // SAFETY: the context is live; NULL is its own stream.
            unsafe { (hip.f.sync)(hip.ctx, std::ptr::null_mut()) }
        };
        let st = launch_all(self, None);
        if st != AH_OK {
            for (k, r) in rs.iter().enumerate() {
                let sk = launch_all(self, Some(k));
                if sk != AH_OK {
                    let shape = CallShape { ggml_type: r.1, n_in: r.3, x_len: codes.len(), need: 0, have: 0 };
                    self.check(sk, shape, "ah_gemv_q8_dev")?;
                }
            }
            self.check(st, CallShape::default(), "ah_gemv_q8_dev")?;
        }
        let mut out = Vec::with_capacity(rs.len());
        for (k, r) in rs.iter().enumerate() {
            let mut y = vec![0f32; r.2];
            // SAFETY: offset inside the carve.
            self.download_bytes(&mut y, unsafe { base.add(c.at[2 + k]) })?;
            out.push(Self::to_q32(&y)?);
        }
        Ok(out)
    }

    /// `ffn_q8act_prepared_into` (`src/engine/chart/ffn.rs:1609`) on the device: gate / up with the
    /// exact SwiGLU and the hidden quant_act in one launch, down from that QuantAct in a second;
    /// the hidden activation never leaves the device.  `codes` / `scales` are `quantize(x)`.
    /// Refusals in the reference FFN's order: a projection's as `HipError::Matvec` (the caller's
    /// `FfnError::Matvec`), the SwiGLU's as `HipError::Ffn`.
    pub fn ffn_q8act(&mut self, gate: usize, up: usize, down: usize, codes: &[i8], scales: &[i64]) -> Result<Vec<i64>, HipError> {
        let (g, u, d) = (self.resident(gate)?.t, self.resident(up)?.t, self.resident(down)?);
        let (dt, n_embd, n_ff, d_type) = (d.t, d.n_out, d.n_in, d.ggml_type);
        if codes.len() != n_embd || scales.len() != n_embd.div_ceil(32) {
            return Err(HipError::Matvec(MatvecError::ShapeMismatch { x: codes.len(), n_in: n_embd }));
        }
        let c = Carve::new(&[codes.len(), 8 * scales.len(), 4 * n_embd, n_ff, 8 * n_ff.div_ceil(32)]);
        let base = self.stage(c.total)?;
        // SAFETY (pointer arithmetic): offsets inside the carve.
        let p = |k: usize| unsafe { base.add(c.at[k]) };
        self.upload_bytes(p(0), codes)?;
        self.upload_bytes(p(1), scales)?;
        // SAFETY: device pointers carved above; the tensors are resident on this context.
        let mut st = unsafe {
            (self.f.ffn_q8)(self.ctx, g, u, dt, p(0).cast::<i8>(), p(1).cast::<i64>(), p(2).cast::<f32>(), p(3).cast::<i8>(),
                            p(4).cast::<i64>(), std::ptr::null_mut())
        };
        if st == AH_OK {
            // SAFETY: the context is live.
            st = unsafe { (self.f.sync)(self.ctx, std::ptr::null_mut()) };
        }
        self.check(st, CallShape { ggml_type: d_type, n_in: n_embd, x_len: codes.len(), need: 0, have: 0 }, "ah_ffn_q8_dev")?;
        let mut y = vec![0f32; n_embd];
        self.download_bytes(&mut y, p(2))?;
        Self::to_q32(&y)
    }

    /// The column path's projection (`proj_cols`, `src/engine/step/cols.rs:485-575`; the grouped
    /// form `gemm_q8_0_group`, `src/engine/kern/gemm.rs:818`): the resident projections `idxs` of
    /// every column `qs[c] = (codes, scales)`, one operand pass and one MFMA launch per run of
    /// projections, one Q32.32 vector per projection and column.  First refusal in
    /// projection-then-column-then-row order.
    pub fn matmat_group_q8act(&mut self, idxs: &[usize], qs: &[(&[i8], &[i64])]) -> Result<Vec<Vec<Vec<i64>>>, HipError> {
        let mut ts: Vec<*const AhTensor> = Vec::with_capacity(idxs.len());
        let mut outs: Vec<usize> = Vec::with_capacity(idxs.len());
        let mut n_in = 0usize;
        for &i in idxs {
            let r = self.resident(i)?;
            if n_in != 0 && r.n_in != n_in {
                return Err(HipError::Backend { status: 21, what: "group n_in".into() });
            }
            n_in = r.n_in;
            ts.push(r.t.cast_const());
            outs.push(r.n_out);
        }
        let nb = n_in.div_ceil(32);
        let k = qs.len();
        let mut codes = Vec::with_capacity(k * n_in);
        let mut scales = Vec::with_capacity(k * nb);
        for (cc, ss) in qs {
            if cc.len() != n_in {
                return Err(HipError::Matvec(MatvecError::ShapeMismatch { x: cc.len(), n_in }));
            }
            if ss.len() != nb {
                return Err(HipError::Backend { status: 21, what: "scales length".into() });
            }
            codes.extend_from_slice(cc);
            scales.extend_from_slice(ss);
        }
        let mut sizes = vec![codes.len(), 8 * scales.len()];
        sizes.extend(outs.iter().map(|&n| 4 * n * k));
        let c = Carve::new(&sizes);
        let base = self.stage(c.total)?;
        // SAFETY (pointer arithmetic): offsets inside the carve.
        let p = |j: usize| unsafe { base.add(c.at[j]) };
        self.upload_bytes(p(0), &codes)?;
        self.upload_bytes(p(1), &scales)?;
        let ys: Vec<*mut f32> = (0..outs.len()).map(|j| p(2 + j).cast::<f32>()).collect();
        // SAFETY: device pointers carved above; tensors resident; ts / ys live for the call.
        let mut st = unsafe {
            (self.f.gemm_group_q8)(self.ctx, ts.len(), ts.as_ptr(), p(0).cast::<i8>(), p(1).cast::<i64>(), k, ys.as_ptr(), std::ptr::null_mut())
        };
        if st == AH_OK {
            // SAFETY: the context is live.
            st = unsafe { (self.f.sync)(self.ctx, std::ptr::null_mut()) };
        }
        self.check(st, CallShape { ggml_type: 0, n_in, x_len: n_in, need: 0, have: 0 }, "ah_gemm_group_q8_dev")?;
        let mut res = Vec::with_capacity(outs.len());
        for (j, &n_out) in outs.iter().enumerate() {
            let mut y = vec![0f32; n_out * k];
            self.download_bytes(&mut y, p(2 + j))?;
            res.push(y.chunks(n_out.max(1)).take(k).map(Self::to_q32).collect::<Result<Vec<_>, _>>()?);
        }
        Ok(res)
    }

    /// The column path's FFN (`src/engine/step/cols.rs:1026-1067`: the `[W_gate; W_up]` GEMM with
    /// the SwiGLU, then the down `proj_cols`) over every column's QuantAct, the hidden columns kept
    /// on the device; one Q32.32 vector of n_embd per column.
    pub fn ffn_cols_q8act(&mut self, gate: usize, up: usize, down: usize, qs: &[(&[i8], &[i64])]) -> Result<Vec<Vec<i64>>, HipError> {
        let (g, u, d) = (self.resident(gate)?.t, self.resident(up)?.t, self.resident(down)?);
        let (dt, n_embd, n_ff) = (d.t, d.n_out, d.n_in);
        let nb = n_embd.div_ceil(32);
        let k = qs.len();
        let mut codes = Vec::with_capacity(k * n_embd);
        let mut scales = Vec::with_capacity(k * nb);
        for (cc, ss) in qs {
            if cc.len() != n_embd || ss.len() != nb {
                return Err(HipError::Matvec(MatvecError::ShapeMismatch { x: cc.len(), n_in: n_embd }));
            }
            codes.extend_from_slice(cc);
            scales.extend_from_slice(ss);
        }
        let c = Carve::new(&[codes.len(), 8 * scales.len(), 4 * n_embd * k, n_ff * k, 8 * n_ff.div_ceil(32) * k]);
        let base = self.stage(c.total)?;
        // SAFETY (pointer arithmetic): offsets inside the carve.
        let p = |j: usize| unsafe { base.add(c.at[j]) };
        self.upload_bytes(p(0), &codes)?;
        self.upload_bytes(p(1), &scales)?;
        // SAFETY: device pointers carved above; tensors resident on this context.
        let mut st = unsafe {
            (self.f.ffn_prefill_q8)(self.ctx, g, u, dt, p(0).cast::<i8>(), p(1).cast::<i64>(), k, p(2).cast::<f32>(),
                                    p(3).cast::<i8>(), p(4).cast::<i64>(), std::ptr::null_mut())
        };
        if st == AH_OK {
            // SAFETY: the context is live.
            st = unsafe { (self.f.sync)(self.ctx, std::ptr::null_mut()) };
        }
        self.check(st, CallShape { ggml_type: 0, n_in: n_embd, x_len: n_embd, need: 0, have: 0 }, "ah_ffn_prefill_q8_dev")?;
        let mut y = vec![0f32; n_embd * k];
        self.download_bytes(&mut y, p(2))?;
        y.chunks(n_embd.max(1)).take(k).map(Self::to_q32).collect()
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
            if !self.stage.d.is_null() {
                (self.f.dev_free)(self.ctx, self.stage.d);
            }
            (self.f.destroy)(self.ctx);
            libc::dlclose(self.lib);
        }
    }
}
