// The engine side of the `hip` backend: what a maintainer adds to the reference's engine so that
// every projection can run on the MI355X.  Four insertions, each an item of its own below, with
// the place it goes; nothing else in the engine changes (the GGUF layouts, the projection entry
// points and the CPU kernels stay as they are, and a machine without the library runs exactly as
// before).
//
// Written against the reference tree's types (src/engine/step.rs, src/engine/loader.rs,
// src/engine/chart/mod.rs); compiled only where it is integrated.

// ---- 1. src/engine/step.rs:211-220 — one more KernelMode arm ---------------------------------
//
// `KernelMode` (Exact, Q8Act) gains:
//
//     /// The int8-activation chart on the MI355X (`crate::gpu::hip`), where the tensor is
//     /// resident there; every other tensor, and every backend failure, takes `Q8Act`.
//     Hip,
//
// and the engine holds the loaded backend beside its resident file (src/engine/loader.rs, the
// `Engine` struct):
//
//     #[cfg(feature = "hip")]
//     hip: std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
//
// (a Mutex: `Hip` is one device context and, like the chart's pool, serves one caller at a time).

// ---- 2. Engine load — upload every projection tensor once -------------------------------------
//
// After the resident file is mapped and the tensor directory read: an honest skip when the
// library or the device is absent, else one upload per 2-D projection tensor of a family the
// backend serves, from the same bytes the CPU path reads (`payload_ref`, loader.rs:1447-1466).

#[cfg(feature = "hip")]
pub(crate) fn load_hip(engine: &crate::engine::Engine, device: i32) -> Option<crate::gpu::hip::Hip> {
    use crate::format::quant;
    // SAFETY: loads libapeiron_hip.so (include/apeiron_hip.h); Err is a skip, never a failure.
    let mut hip = match unsafe { crate::gpu::hip::Hip::load(device) } {
        Ok(h) => h,
        Err(msg) => {
            eprintln!("hip backend skipped: {msg}");
            return None;
        }
    };
    for (idx, t) in engine.table().entries().iter().enumerate() {
        let served = matches!(
            t.ggml_type,
            quant::GGML_TYPE_Q8_0
                | quant::GGML_TYPE_Q5_0
                | quant::GGML_TYPE_Q2_K
                | quant::GGML_TYPE_Q3_K
                | quant::GGML_TYPE_Q4_K
                | quant::GGML_TYPE_Q6_K
        );
        if !served || t.dims.len() != 2 {
            continue;
        }
        let (Ok(n_in), Ok(n_out)) = (usize::try_from(t.dims[0]), usize::try_from(t.dims[1])) else {
            continue;
        };
        let Some(n_bytes) = t.n_bytes else { continue };
        let Ok(at) = engine.payload_ref(t.byte_range.start, n_bytes) else { continue };
        // A refusal (a non-finite scale, a shape past the device limits) keeps this tensor on the
        // CPU path, where the reference's row dequantizer gives its own answer.
        if let Err(e) = hip.upload(idx, t.ggml_type, engine.resident(), at, n_out, n_in) {
            eprintln!("hip backend: tensor {} stays on the CPU ({e:?})", t.name);
        }
    }
    Some(hip)
}

// ---- 3. src/engine/step.rs:346-378 — the projection dispatch ---------------------------------
//
// In `proj_q8act_quantified`, after `let q = quant_act_pooled(x)...?;` and before the CPU call,
// for KernelMode::Hip:
//
//     #[cfg(feature = "hip")]
//     if self.kernel_mode == KernelMode::Hip {
//         if let Some(y) = hip_projection(&self.hip, idx, &q)? {
//             return Ok(y);
//         }
//     }
//
// with the helper below: Some(outputs) when the device served the call, None when the caller
// should take its CPU path (tensor not resident, no backend, a backend failure), and the
// contract's own refusal as the same MatvecError the CPU path would return.

#[cfg(feature = "hip")]
pub(crate) fn hip_projection(
    hip: &std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
    idx: usize,
    q: &crate::engine::chart::QuantAct,
) -> Result<Option<Vec<i64>>, crate::engine::MatvecError> {
    use crate::gpu::hip::HipError;
    let Ok(guard) = hip.lock() else { return Ok(None) };
    let Some(h) = guard.as_ref() else { return Ok(None) };
    if !h.has(idx) {
        return Ok(None);
    }
    match h.matvec_q8act(idx, q.codes(), q.scales()) {
        Ok(y) => Ok(Some(y)),
        Err(HipError::Matvec(e)) => Err(e),
        // f32-input and SwiGLU statuses cannot come from a codes-input projection; backend
        // failures (device lost, memory) fall back to the CPU kernels for this call
        Err(HipError::Input(_) | HipError::Ffn(_) | HipError::Backend { .. }) => Ok(None),
    }
}

// ---- 4. Device-resident forms: the grouped projections, the FFN and the column (prefill) path ---
//
// Each helper below returns Some(outputs) when the device served the call, None when the caller
// keeps its CPU path (a tensor not resident, no backend, a backend failure), and the contract's own
// refusal as the value the CPU path would return.  The activation goes up once per call, every
// projection of the call (and the FFN's hidden activation) stays on the device, and only the
// outputs come back.

/// The backend's answer mapped onto the engine's: Ok(None) = take the CPU path.
#[cfg(feature = "hip")]
fn served<T, E>(r: Result<T, crate::gpu::hip::HipError>, refusal: impl Fn(crate::gpu::hip::HipError) -> Option<E>) -> Result<Option<T>, E> {
    match r {
        Ok(v) => Ok(Some(v)),
        Err(e) => match refusal(e) {
            Some(err) => Err(err),
            None => Ok(None),
        },
    }
}

/// src/engine/step.rs:911-1000 `group_q8act_at` (q/k/v, and gate/up outside the fused FFN) — at
/// the top of its final step, before `projections_q8act(self.resident(), ...)`:
///
///     #[cfg(feature = "hip")]
///     if self.kernel_mode == KernelMode::Hip {
///         if let Some(out) = hip_group(&self.hip, &idxs, x)? {
///             return Ok(out);
///         }
///     }
///
/// `projections_q8act`'s quantization (`quantize(x)`, chart/ffn.rs:236-238) happens here on the
/// host, so its refusal and the QuantAct are the CPU path's; the projections run on the device in
/// projection-then-row refusal order.
#[cfg(feature = "hip")]
pub(crate) fn hip_group(
    hip: &std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
    idxs: &[usize],
    x: &[i64],
) -> Result<Option<Vec<Vec<i64>>>, crate::engine::step::StepError> {
    use crate::engine::step::StepError;
    use crate::engine::{EngineError, MatvecError};
    use crate::gpu::hip::HipError;
    let Ok(mut guard) = hip.lock() else { return Ok(None) };
    let Some(h) = guard.as_mut() else { return Ok(None) };
    if !idxs.iter().all(|&i| h.has(i)) {
        return Ok(None);
    }
    let q = crate::engine::chart::ffn::quant_act_pooled(x)
        .ok_or(StepError::Matvec(MatvecError::Dequant(EngineError::FixedOverflow)))?;
    served(h.projections_q8act(idxs, q.codes(), q.scales()), |e| match e {
        HipError::Matvec(m) => Some(StepError::Matvec(m)),
        HipError::Input(_) | HipError::Ffn(_) | HipError::Backend { .. } => None,
    })
}

/// src/engine/step.rs:1004-1037 `ffn_q8act_at` — before the `ffn_q8act_prepared_into(...)` call
/// (chart/ffn.rs:1609), with `idxs = [li.at(4, layer)?, li.at(5, layer)?, li.at(6, layer)?]`:
///
///     #[cfg(feature = "hip")]
///     if self.kernel_mode == KernelMode::Hip {
///         if let Some(y) = hip_ffn(&self.hip, idxs, x)? {
///             return Ok(y);
///         }
///     }
///
/// gate / up with the exact SwiGLU and the hidden quant_act run in one device launch, down from
/// that QuantAct in a second: the hidden activation never comes back to the host.  Refusals in
/// the reference FFN's order: `quantize(x)`'s, a projection's (`FfnError::Matvec`), the SwiGLU's.
#[cfg(feature = "hip")]
pub(crate) fn hip_ffn(
    hip: &std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
    idxs: [usize; 3],
    x: &[i64],
) -> Result<Option<Vec<i64>>, crate::engine::step::StepError> {
    use crate::engine::step::StepError;
    use crate::engine::{EngineError, FfnError, MatvecError};
    use crate::gpu::hip::HipError;
    let Ok(mut guard) = hip.lock() else { return Ok(None) };
    let Some(h) = guard.as_mut() else { return Ok(None) };
    if !idxs.iter().all(|&i| h.has(i)) {
        return Ok(None);
    }
    let q = crate::engine::chart::ffn::quant_act_pooled(x)
        .ok_or(StepError::Ffn(FfnError::Matvec(MatvecError::Dequant(EngineError::FixedOverflow))))?;
    served(h.ffn_q8act(idxs[0], idxs[1], idxs[2], q.codes(), q.scales()), |e| match e {
        HipError::Matvec(m) => Some(StepError::Ffn(FfnError::Matvec(m))),
        HipError::Ffn(f) => Some(StepError::Ffn(f)),
        HipError::Input(_) | HipError::Backend { .. } => None,
    })
}

/// src/engine/step/cols.rs:485-575 `proj_cols` — in its `xs.len() > 1` branch, once `qs` holds
/// the columns' QuantActs and before the `matmat_q8act(...)` call:
///
///     #[cfg(feature = "hip")]
///     if mode == KernelMode::Hip {
///         if let Some(mut cols) = hip_proj_cols(&self.hip, &[idx], qs)? {
///             return Ok(cols.swap_remove(0));
///         }
///     }
///
/// (the q/k/v group of the column path passes its three indices at once: one operand pass, one
/// MFMA launch, refusals projection-then-column-then-row).
#[cfg(feature = "hip")]
pub(crate) fn hip_proj_cols(
    hip: &std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
    idxs: &[usize],
    qs: &[crate::engine::chart::QuantAct],
) -> Result<Option<Vec<Vec<Vec<i64>>>>, crate::engine::step::StepError> {
    use crate::engine::step::StepError;
    use crate::gpu::hip::HipError;
    let Ok(mut guard) = hip.lock() else { return Ok(None) };
    let Some(h) = guard.as_mut() else { return Ok(None) };
    if !idxs.iter().all(|&i| h.has(i)) {
        return Ok(None);
    }
    let cols: Vec<(&[i8], &[i64])> = qs.iter().map(|q| (q.codes(), q.scales())).collect();
    served(h.matmat_group_q8act(idxs, &cols), |e| match e {
        HipError::Matvec(m) => Some(StepError::Matvec(m)),
        HipError::Input(_) | HipError::Ffn(_) | HipError::Backend { .. } => None,
    })
}

/// src/engine/step/cols.rs:1026-1067 — the column FFN: after `let qs = quant_cols(xs)?;` and
/// before the fused / separate gate-up branch (a recording tap keeps the CPU path, which holds the
/// gate and up words the tap stores):
///
///     #[cfg(feature = "hip")]
///     if mode == KernelMode::Hip && tap.is_none() {
///         let idxs = [li.at(4, layer)?, li.at(5, layer)?, li.at(6, layer)?];
///         if let Some(out) = hip_ffn_cols(&self.hip, idxs, &qs)? {
///             return Ok(out);
///         }
///     }
///
/// gate/up, the exact SwiGLU, the hidden columns' quant_act and down on the device; refusals in
/// the column path's order (gate for every column, then up, then the SwiGLU, then down).
#[cfg(feature = "hip")]
pub(crate) fn hip_ffn_cols(
    hip: &std::sync::Mutex<Option<crate::gpu::hip::Hip>>,
    idxs: [usize; 3],
    qs: &[crate::engine::chart::QuantAct],
) -> Result<Option<Vec<Vec<i64>>>, crate::engine::step::StepError> {
    use crate::engine::step::StepError;
    use crate::gpu::hip::HipError;
    let Ok(mut guard) = hip.lock() else { return Ok(None) };
    let Some(h) = guard.as_mut() else { return Ok(None) };
    if !idxs.iter().all(|&i| h.has(i)) {
        return Ok(None);
    }
    let cols: Vec<(&[i8], &[i64])> = qs.iter().map(|q| (q.codes(), q.scales())).collect();
    served(h.ffn_cols_q8act(idxs[0], idxs[1], idxs[2], &cols), |e| match e {
        // the column path reports a gate / up / down projection's refusal as StepError::Matvec
        // (proj_cols) and the SwiGLU's as StepError::Ffn (swiglu_cols)
        HipError::Matvec(m) => Some(StepError::Matvec(m)),
        HipError::Ffn(f) => Some(StepError::Ffn(f)),
        HipError::Input(_) | HipError::Backend { .. } => None,
    })
}
