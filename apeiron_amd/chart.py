"""Host-side mirror of apeiron's int8-activation projection interface, backed by the HIP C ABI.

Mirrors, with the same names, argument meaning and refusal behaviour:

* ``QuantAct``          -- chart/mod.rs:67-81 (codes int8 [n_in], scales int64 [ceil(n_in/32)])
* ``quant_act(x)``      -- chart/mod.rs:258 (x: Q32.32 int64); returns None where the reference
                           returns None (an activation with no Q32.32 value)
* ``matvec_q8act``      -- chart/mod.rs:1887 (returns f32 real outputs, see below)
* ``matmat_q8act``      -- kern/matmat.rs:134 (one output vector per column)
* ``MatvecError``       -- ops/matvec.rs:11-48, raised instead of returned

Outputs are f32 real values: the reference's Q32.32 result of row o is
round_shift_32(sum_i w_oi*xhat_i); ours is that sum * 2^-32 from exact integer group dots,
accumulated in f32.  ``to_q32`` converts back to the engine's Q32.32 type where needed.

Device memory here comes from PyTorch (plumbing only); every computation runs in
libapeiron_hip.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib

Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q6_K = 6, 8, 10, 11, 12, 14


class MatvecError(Exception):
    """A refused projection; ``kind`` is the MatvecError variant name (ops/matvec.rs:11-48)."""

    def __init__(self, status: int, where: str = ""):
        self.status = status
        self.kind = _lib.STATUS.get(status, f"status{status}")
        super().__init__(f"{self.kind}{(' in ' + where) if where else ''}")


def _check(status: int, where: str) -> None:
    if status != 0:
        raise MatvecError(status, where)


@dataclass
class QuantAct:
    scales: np.ndarray  # int64 [ceil(n/32)]
    codes: np.ndarray   # int8 [n]

    def __len__(self) -> int:
        return int(self.codes.shape[0])


class Device:
    """One ah_ctx on one GPU (the backend's context; not thread-safe, like the reference pool)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        _check(self.lib.ah_init(device, ctypes.byref(h)), "ah_init")
        self.h = h
        self.device = device

    def close(self) -> None:
        if self.h:
            self.lib.ah_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, ggml_type: int, raw: np.ndarray, n_out: int, n_in: int) -> "Tensor":
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        t = ctypes.c_void_p()
        _check(self.lib.ah_upload_weight(self.h, ggml_type, raw.ctypes.data_as(ctypes.c_void_p),
                                         raw.nbytes, n_out, n_in, ctypes.byref(t)), "upload")
        return Tensor(self, t, ggml_type, n_out, n_in)

    def wrap(self, ggml_type: int, dev_ptr: int, nbytes: int, n_out: int, n_in: int) -> "Tensor":
        t = ctypes.c_void_p()
        _check(self.lib.ah_wrap_weight_dev(self.h, ggml_type, dev_ptr, nbytes, n_out, n_in,
                                           ctypes.byref(t)), "wrap")
        return Tensor(self, t, ggml_type, n_out, n_in)

    def sync_status(self, stream: int | None = None) -> int:
        return self.lib.ah_sync_status(self.h, stream)

    def last_refusal_bits(self) -> int:
        """f16 bits of the scale behind the last NonFiniteScale refusal (NonFiniteScale { bits })."""
        b = ctypes.c_uint32(0)
        _check(self.lib.ah_last_refusal_bits(self.h, ctypes.byref(b)), "last_refusal_bits")
        return b.value

    GEMM_AUTO, GEMM_F16, GEMM_INT8, GEMM_F16_TILE = 0, 1, 2, 3

    def set_gemm_design(self, ggml_type: int, design: int) -> None:
        """The prefill GEMM design of `ggml_type` on this context (ah_set_gemm_design).  AUTO is
        F16 for every type but Q2_K and Q3_K, where it is F16_TILE (the dequantize-once tiles);
        INT8 exists for Q8_0 and Q4_K, F16_TILE for Q4_K, Q2_K and Q3_K; F16 on Q2_K / Q3_K serves the
        prefill as one streaming GEMV per token."""
        _check(self.lib.ah_set_gemm_design(self.h, ggml_type, design), "set_gemm_design")

    FFN_AUTO, FFN_FUSED, FFN_TWO_PASS = 0, 1, 2

    def set_ffn_prefill_form(self, form: int) -> None:
        """The prefill FFN's form (ah_set_ffn_prefill_form): AUTO (two passes), FUSED (one launch
        for Q4_K / Q2_K / Q3_K gate/up) or TWO_PASS."""
        _check(self.lib.ah_set_ffn_prefill_form(self.h, form), "set_ffn_prefill_form")

    def probe_mfma_peak(self, kind: int) -> float:
        """Measured MFMA-only rate in tera-ops/s (kind 0: int8 32x32x32, 1: f16 32x32x16)."""
        out = ctypes.c_double(0.0)
        _check(self.lib.ah_probe_mfma_peak(self.h, kind, ctypes.byref(out)), "probe_mfma_peak")
        return out.value

    # device-pointer forms (enqueue only) -------------------------------------------------
    def quant_act_f32_dev(self, x_ptr: int, n_tok: int, n_in: int, codes_ptr: int,
                          scales_ptr: int, stream: int | None = None) -> None:
        _check(self.lib.ah_quant_act_f32_dev(self.h, x_ptr, n_tok, n_in, codes_ptr, scales_ptr,
                                             stream), "quant_act_f32_dev")

    def quant_act_q32_dev(self, x_ptr: int, n_tok: int, n_in: int, codes_ptr: int,
                          scales_ptr: int, stream: int | None = None) -> None:
        _check(self.lib.ah_quant_act_q32_dev(self.h, x_ptr, n_tok, n_in, codes_ptr, scales_ptr,
                                             stream), "quant_act_q32_dev")

    # host forms -------------------------------------------------------------------------
    def quant_act(self, x) -> QuantAct | None:
        """chart/mod.rs:258: None exactly where the reference refuses."""
        x = np.ascontiguousarray(x, dtype=np.int64)
        n = x.shape[0]
        codes = np.zeros(max(n, 1), np.int8)
        scales = np.zeros(max(-(-n // 32), 1), np.int64)
        st = self.lib.ah_quant_act(self.h, x.ctypes.data_as(ctypes.c_void_p), n,
                                   codes.ctypes.data_as(ctypes.c_void_p),
                                   scales.ctypes.data_as(ctypes.c_void_p))
        if st == 7:
            return None
        _check(st, "quant_act")
        return QuantAct(scales[: -(-n // 32)], codes[:n])


class Tensor:
    """A device-resident GGUF weight (unchanged layout)."""

    def __init__(self, dev: Device, handle: ctypes.c_void_p, ggml_type: int, n_out: int, n_in: int):
        self.dev, self.h = dev, handle
        self.ggml_type, self.n_out, self.n_in = ggml_type, n_out, n_in

    def free(self) -> None:
        if self.h:
            self.dev.lib.ah_free_tensor(self.dev.h, self.h)
            self.h = None

    def __del__(self):
        try:
            if self.dev.h:
                self.free()
        except Exception:
            pass

    def gemv_f32_dev(self, x_ptr: int, y_ptr: int, stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemv_f32_dev(self.dev.h, self.h, x_ptr, y_ptr, stream), "gemv_f32")

    def gemv_q8_dev(self, codes_ptr: int, scales_ptr: int, y_ptr: int, stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemv_q8_dev(self.dev.h, self.h, codes_ptr, scales_ptr, y_ptr, stream),
               "gemv_q8")

    def gemv_q8_dots_dev(self, codes_ptr: int, scales_ptr: int, y_ptr: int, dots_ptr: int,
                         stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemv_q8_dots_dev(self.dev.h, self.h, codes_ptr, scales_ptr, y_ptr,
                                                dots_ptr, stream), "gemv_q8_dots")

    def gemm_f32_dev(self, x_ptr: int, n_tok: int, y_ptr: int, stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemm_f32_dev(self.dev.h, self.h, x_ptr, n_tok, y_ptr, stream), "gemm_f32")

    def gemm_q8_dev(self, codes_ptr: int, scales_ptr: int, n_tok: int, y_ptr: int,
                    stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemm_q8_dev(self.dev.h, self.h, codes_ptr, scales_ptr, n_tok, y_ptr,
                                           stream), "gemm_q8")


def gemm_group_f32_dev(dev: "Device", tensors: list["Tensor"], x_ptr: int, n_tok: int,
                       y_ptrs: list[int], stream: int | None = None) -> None:
    """Prefill over projections of one f32 input [n_tok][n_in] (ah_gemm_group_f32_dev)."""
    n = len(tensors)
    W = (ctypes.c_void_p * n)(*[t.h.value for t in tensors])
    Y = (ctypes.c_void_p * n)(*y_ptrs)
    _check(dev.lib.ah_gemm_group_f32_dev(dev.h, n, W, x_ptr, n_tok, Y, stream), "gemm_group_f32")


def gemm_group_q8_dev(dev: "Device", tensors: list["Tensor"], codes_ptr: int, scales_ptr: int,
                      n_tok: int, y_ptrs: list[int], stream: int | None = None) -> None:
    """Prefill over projections of one quantized input (ah_gemm_group_q8_dev)."""
    n = len(tensors)
    W = (ctypes.c_void_p * n)(*[t.h.value for t in tensors])
    Y = (ctypes.c_void_p * n)(*y_ptrs)
    _check(dev.lib.ah_gemm_group_q8_dev(dev.h, n, W, codes_ptr, scales_ptr, n_tok, Y, stream),
           "gemm_group_q8")


def ffn_gate_up_dev(dev: "Device", gate: "Tensor", up: "Tensor", x_ptr: int, h_codes_ptr: int,
                    h_scales_ptr: int, gate_y_ptr: int | None = None, up_y_ptr: int | None = None,
                    stream: int | None = None) -> None:
    """The fused FFN's gate/up launch with the SwiGLU + hidden requantize epilogue
    (ah_ffn_gate_up_dev): the hidden QuantAct ffn_q8act_prepared_into (chart/ffn.rs:1609) feeds
    its down projection."""
    _check(dev.lib.ah_ffn_gate_up_dev(dev.h, gate.h, up.h, x_ptr, gate_y_ptr, up_y_ptr, h_codes_ptr,
                                      h_scales_ptr, stream), "ffn_gate_up")


def ffn_dev(dev: "Device", gate: "Tensor", up: "Tensor", down: "Tensor", x_ptr: int, y_ptr: int,
            h_codes_ptr: int, h_scales_ptr: int, stream: int | None = None) -> None:
    """The fused FFN, ffn_q8act_prepared_into (chart/ffn.rs:1609): y = down . quant_act(SwiGLU(gate . x,
    up . x)) in two launches (ah_ffn_dev)."""
    _check(dev.lib.ah_ffn_dev(dev.h, gate.h, up.h, down.h, x_ptr, y_ptr, h_codes_ptr, h_scales_ptr, stream),
           "ffn")


def ffn_gate_up_prefill_dev(dev: "Device", gate: "Tensor", up: "Tensor", x_ptr: int, n_tok: int,
                            h_codes_ptr: int, h_scales_ptr: int, gate_y_ptr: int | None = None,
                            up_y_ptr: int | None = None, stream: int | None = None) -> None:
    """The prefill FFN's gate/up with the exact SwiGLU and the hidden quant_act
    (ah_ffn_gate_up_prefill_dev; the column path of step/cols.rs:1026-1067): f32 x[n_tok][n_embd]
    into the hidden QuantAct codes[n_tok][n_ff] / scales[n_tok][ceil(n_ff/32)], optionally the f32
    gate and up values it consumed."""
    _check(dev.lib.ah_ffn_gate_up_prefill_dev(dev.h, gate.h, up.h, x_ptr, n_tok, gate_y_ptr, up_y_ptr,
                                              h_codes_ptr, h_scales_ptr, stream), "ffn_gate_up_prefill")


def ffn_prefill_dev(dev: "Device", gate: "Tensor", up: "Tensor", down: "Tensor", x_ptr: int, n_tok: int,
                    y_ptr: int, h_codes_ptr: int, h_scales_ptr: int, stream: int | None = None) -> None:
    """The prefill FFN, y[n_tok][n_embd] = down . quant_act(SwiGLU(gate . x, up . x)) per token
    (ah_ffn_prefill_dev)."""
    _check(dev.lib.ah_ffn_prefill_dev(dev.h, gate.h, up.h, down.h, x_ptr, n_tok, y_ptr, h_codes_ptr,
                                      h_scales_ptr, stream), "ffn_prefill")


def ffn_q8_dev(dev: "Device", gate: "Tensor", up: "Tensor", down: "Tensor", codes_ptr: int, scales_ptr: int,
               y_ptr: int, h_codes_ptr: int, h_scales_ptr: int, stream: int | None = None) -> None:
    """ffn_dev from a QuantAct (ah_ffn_q8_dev)."""
    _check(dev.lib.ah_ffn_q8_dev(dev.h, gate.h, up.h, down.h, codes_ptr, scales_ptr, y_ptr, h_codes_ptr,
                                 h_scales_ptr, stream), "ffn_q8")


def ffn_prefill_q8_dev(dev: "Device", gate: "Tensor", up: "Tensor", down: "Tensor", codes_ptr: int,
                       scales_ptr: int, n_tok: int, y_ptr: int, h_codes_ptr: int, h_scales_ptr: int,
                       stream: int | None = None) -> None:
    """ffn_prefill_dev from the tokens' QuantActs (ah_ffn_prefill_q8_dev)."""
    _check(dev.lib.ah_ffn_prefill_q8_dev(dev.h, gate.h, up.h, down.h, codes_ptr, scales_ptr, n_tok, y_ptr,
                                         h_codes_ptr, h_scales_ptr, stream), "ffn_prefill_q8")


def swiglu_quant_dev(dev: "Device", gate_ptr: int, up_ptr: int, n_tok: int, n_ff: int, h_codes_ptr: int,
                     h_scales_ptr: int, stream: int | None = None) -> None:
    """swiglu_cols + quant_cols over f32 gate / up [n_tok][n_ff] (ah_swiglu_quant_dev)."""
    _check(dev.lib.ah_swiglu_quant_dev(dev.h, gate_ptr, up_ptr, n_tok, n_ff, h_codes_ptr, h_scales_ptr, stream),
           "swiglu_quant")


class GemvPlan:
    """A grouped GEMV launch over fixed device pointers (ah_gemv_plan_*)."""

    def __init__(self, dev: Device, tensors: list[Tensor], x_ptrs: list[int], y_ptrs: list[int]):
        n = len(tensors)
        W = (ctypes.c_void_p * n)(*[t.h.value for t in tensors])
        X = (ctypes.c_void_p * n)(*x_ptrs)
        Y = (ctypes.c_void_p * n)(*y_ptrs)
        h = ctypes.c_void_p()
        _check(dev.lib.ah_gemv_plan_create(dev.h, n, W, X, Y, ctypes.byref(h)), "gemv_plan_create")
        self.dev, self.h, self.keep = dev, h, tensors

    def run(self, stream: int | None = None) -> None:
        _check(self.dev.lib.ah_gemv_plan_run(self.dev.h, self.h, stream), "gemv_plan_run")

    def free(self) -> None:
        if self.h:
            self.dev.lib.ah_gemv_plan_free(self.dev.h, self.h)
            self.h = None


class Seq:
    """A persistent decode sequence (ah_seq_*): stages run in order in ONE launch, each reading
    outputs of the stages before it.  A stage is ``("gemv", parts)`` with parts a list of
    ``(tensor, x_ptr, y_ptr)`` (f32 input) or ``(tensor, (codes_ptr, scales_ptr), y_ptr)``
    (a QuantAct, e.g. a SwiGLU stage's output), or ``("swiglu", gate_ptr, up_ptr, n, codes_ptr,
    scales_ptr)``: the fused FFN's hidden activation (chart/ffn.rs:1532-1594)."""

    def __init__(self, dev: Device, stages: list):
        n = len(stages)
        arr = (_lib.SeqStage * n)()
        self.keep = []
        for i, st in enumerate(stages):
            S = arr[i]
            if st[0] == "swiglu":
                _, gate, up, width, codes, scales = st
                S.kind, S.gate, S.up, S.n, S.h_codes, S.h_scales = 1, gate, up, width, codes, scales
                continue
            parts = st[1]
            k = len(parts)
            W = (ctypes.c_void_p * k)(*[p[0].h.value for p in parts])
            X = (ctypes.c_void_p * k)(*[p[1] if isinstance(p[1], int) else None for p in parts])
            C = (ctypes.c_void_p * k)(*[p[1][0] if not isinstance(p[1], int) else None for p in parts])
            Sc = (ctypes.c_void_p * k)(*[p[1][1] if not isinstance(p[1], int) else None for p in parts])
            Y = (ctypes.c_void_p * k)(*[p[2] for p in parts])
            self.keep += [W, X, C, Sc, Y, [p[0] for p in parts]]
            S.kind, S.n_parts = 0, k
            S.w, S.x, S.codes, S.scales, S.y = (ctypes.cast(a, ctypes.c_void_p) for a in (W, X, C, Sc, Y))
        h = ctypes.c_void_p()
        _check(dev.lib.ah_seq_create(dev.h, n, ctypes.cast(arr, ctypes.c_void_p), ctypes.byref(h)), "seq_create")
        self.dev, self.h = dev, h

    def run(self, stream: int | None = None) -> None:
        _check(self.dev.lib.ah_seq_run(self.dev.h, self.h, stream), "seq_run")

    def set_spin_limit(self, polls: int) -> None:
        """Polls a grid-barrier wait makes before it gives up (0: the default)."""
        _check(self.dev.lib.ah_seq_set_spin_limit(self.h, polls), "seq_set_spin_limit")

    def sync_status(self, stream: int | None = None) -> tuple[int, int]:
        """(status, stage) of the first refusal since the last call, in stage order."""
        stage = ctypes.c_uint32(0)
        st = self.dev.lib.ah_seq_sync_status(self.dev.h, self.h, stream, ctypes.byref(stage))
        return st, stage.value

    def info(self) -> tuple[int, int]:
        """(resident grid, activation LDS bytes per workgroup)."""
        g, a = ctypes.c_uint32(0), ctypes.c_uint32(0)
        _check(self.dev.lib.ah_seq_info(self.h, ctypes.byref(g), ctypes.byref(a)), "seq_info")
        return g.value, a.value

    def free(self) -> None:
        if self.h:
            self.dev.lib.ah_seq_free(self.dev.h, self.h)
            self.h = None


_default: Device | None = None


def device() -> Device:
    global _default
    if _default is None:
        _default = Device(0)
    return _default


def quant_act(x) -> QuantAct | None:
    return device().quant_act(x)


def matvec_q8act(ggml_type: int, raw: np.ndarray, n_out: int, n_in: int, q: QuantAct) -> np.ndarray:
    """chart/mod.rs:1887 over the GPU: raises MatvecError where the reference returns Err."""
    dev = device()
    if len(q) != n_in:
        raise MatvecError(1, "matvec_q8act")
    w = dev.upload(ggml_type, raw, n_out, n_in)
    try:
        y = np.zeros(max(n_out, 1), np.float32)
        codes = np.ascontiguousarray(q.codes, np.int8)
        scales = np.ascontiguousarray(q.scales, np.int64)
        _check(dev.lib.ah_matvec_q8act(dev.h, w.h, codes.ctypes.data_as(ctypes.c_void_p),
                                       scales.ctypes.data_as(ctypes.c_void_p), len(q),
                                       y.ctypes.data_as(ctypes.c_void_p)), "matvec_q8act")
        return y[:n_out]
    finally:
        w.free()


def matmat_q8act(ggml_type: int, raw: np.ndarray, n_out: int, n_in: int,
                 qs: list[QuantAct]) -> np.ndarray:
    """kern/matmat.rs:134 over the GPU: y[c] = matvec_q8act(..., qs[c]); returns [n_tok][n_out]."""
    dev = device()
    for q in qs:
        if len(q) != n_in:
            raise MatvecError(1, "matmat_q8act")
    n_tok = len(qs)
    w = dev.upload(ggml_type, raw, n_out, n_in)
    try:
        codes = np.ascontiguousarray(np.stack([q.codes for q in qs]) if qs else np.zeros((0, n_in)), np.int8)
        scales = np.ascontiguousarray(np.stack([q.scales for q in qs]) if qs else np.zeros((0, 1)), np.int64)
        y = np.zeros((max(n_tok, 1), max(n_out, 1)), np.float32)
        _check(dev.lib.ah_matmat_q8act(dev.h, w.h, codes.ctypes.data_as(ctypes.c_void_p),
                                       scales.ctypes.data_as(ctypes.c_void_p), n_tok,
                                       y.ctypes.data_as(ctypes.c_void_p)), "matmat_q8act")
        return y[:n_tok, :n_out]
    finally:
        w.free()


def to_q32(y: np.ndarray) -> np.ndarray:
    """f32 real outputs -> the engine's Q32.32 int64 (round half away, as F32::to_q32)."""
    v = np.asarray(y, np.float64) * 4294967296.0
    return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)
