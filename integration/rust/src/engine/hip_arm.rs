// The engine side of the `hip` backend: what a maintainer adds to the reference's engine so that
// every projection can run on the MI355X.  Three insertions, each an item of its own below, with
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
            quant::GGML_TYPE_Q8_0 | quant::GGML_TYPE_Q5_0 | quant::GGML_TYPE_Q4_K | quant::GGML_TYPE_Q6_K
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

// The prefill form is the same shape: `matmat_q8act` (src/engine/kern/matmat.rs:134) routes to
// `Hip::matmat_q8act(idx, &cols)` with `cols[c] = (qs[c].codes(), qs[c].scales())`, one Q32.32
// vector per column, under the same Some / None / refusal rule.
