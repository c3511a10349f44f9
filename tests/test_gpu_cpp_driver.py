"""The C++ ABI driver (the C twin of the Rust `hip` module) on the GPU: the host-form calls the
engine integration makes -- ah_upload_weight, ah_matvec_q8act, ah_matmat_q8act, ah_quant_act --
through dlopen'd entry points, against the oracle, for every served GGUF type, plus a
NonFiniteScale refusal carrying its scale bits.

Bar: outputs within 1e-4 * sum|w*xhat| + 2^-32 of the exact contract; quant_act bit-exact.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle
from apeiron_amd import build, synth

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(build.__file__), "libapeiron_hip.so")
TOL = 1e-4
Q32 = 2.0 ** -32


def write_case(path, t, raw, n_out, n_in, codes, scales, x):
    with open(path, "wb") as f:
        f.write(struct.pack("<IQQQQ", t, n_out, n_in, codes.shape[0], raw.nbytes))
        f.write(np.ascontiguousarray(raw, np.uint8).tobytes())
        f.write(np.ascontiguousarray(codes, np.int8).tobytes())
        f.write(np.ascontiguousarray(scales, np.int64).tobytes())
        f.write(np.ascontiguousarray(x, np.int64).tobytes())


def read_out(path, n_out, n_in, n_tok):
    b = open(path, "rb").read()
    o = 0

    def take(dt, n):
        nonlocal o
        a = np.frombuffer(b, dt, n, o)
        o += a.nbytes
        return a

    su = int(take(np.int32, 1)[0])
    sv = int(take(np.int32, 1)[0])
    y0 = take(np.float32, n_out)
    sm = int(take(np.int32, 1)[0])
    Y = take(np.float32, n_tok * n_out).reshape(n_tok, n_out)
    sq = int(take(np.int32, 1)[0])
    qc = take(np.int8, n_in)
    qs = take(np.int64, -(-n_in // 32))
    bits = int(take(np.uint32, 1)[0])
    assert o == len(b)
    return su, sv, y0, sm, Y, sq, qc, qs, bits


def drive(tmp_path, t, raw, n_out, n_in, codes, scales, x):
    assert os.path.exists(build.DRIVER), "build() builds tests/cpp/abi_driver"
    fi, fo = str(tmp_path / "in.bin"), str(tmp_path / "out.bin")
    write_case(fi, t, raw, n_out, n_in, codes, scales, x)
    r = subprocess.run([build.DRIVER, LIB, "run", fi, fo], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("RUN"), r.stdout + r.stderr
    return read_out(fo, n_out, n_in, codes.shape[0])


@pytest.mark.parametrize("t,n_out,n_in", [(6, 100, 896), (8, 77, 300), (10, 40, 300), (11, 64, 1536), (12, 64, 896),
                                         (14, 50, 1536)])
def test_driver_host_forms_vs_oracle(tmp_path, t, n_out, n_in):
    rng = synth.rng_for(7, 1000 * t + n_in)
    raw = synth.payload(t, rng, n_out, n_in)
    n_tok = 5
    x = synth.activations(rng, n_in, n_tok)
    st, codes, scales = oracle.quant_act_f32_batch(x)
    assert st == 0
    xq = (rng.integers(-2 ** 40, 2 ** 40, size=n_in)).astype(np.int64)
    su, sv, y0, sm, Y, sq, qc, qs, bits = drive(tmp_path, t, raw, n_out, n_in, codes, scales, xq)
    assert (su, sv, sm, sq) == (0, 0, 0, 0)
    for c in range(n_tok):
        st1, yref = oracle.matvec_q8act(t, raw, n_out, n_in, codes[c], scales[c])
        st2, absdot = oracle.row_absdot(t, raw, n_out, n_in, codes[c], scales[c])
        assert st1 == 0 and st2 == 0
        ref = yref.astype(np.float64) * Q32
        assert (np.abs(Y[c] - ref) <= TOL * absdot + Q32).all(), (t, c)
        if c == 0:
            assert (np.abs(y0 - ref) <= TOL * absdot + Q32).all(), t
    st, oc, os_ = oracle.quant_act(xq)
    assert st == 0 and (qc == oc).all() and (qs == os_).all()


def test_driver_nonfinite_scale_refusal(tmp_path):
    rng = synth.rng_for(7, 99)
    raw = synth.payload(8, rng, 4, 64)
    raw[34 * 3:34 * 3 + 2] = [0x01, 0x7E]  # NaN scale word 0x7E01 in row 1, block 1
    codes = np.zeros((1, 64), np.int8)
    scales = np.zeros((1, 2), np.int64)
    su, sv, y0, sm, Y, sq, qc, qs, bits = drive(tmp_path, 8, raw, 4, 64, codes, scales, np.zeros(64, np.int64))
    assert su == 6 and bits == 0x7E01  # MatvecError::Dequant(EngineError::NonFiniteScale { bits })


# ---- the device-resident forms the engine binding makes (integration/rust/src/gpu/hip.rs) -------

def write_engine_case(path, gt, dt, n_embd, n_ff, raws, codes, scales):
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQQ", gt, dt, n_embd, n_ff, codes.shape[0]))
        for raw in raws:
            f.write(struct.pack("<Q", raw.nbytes))
            f.write(np.ascontiguousarray(raw, np.uint8).tobytes())
        f.write(np.ascontiguousarray(codes, np.int8).tobytes())
        f.write(np.ascontiguousarray(scales, np.int64).tobytes())


def read_engine_out(path, n_embd, n_ff, n_tok):
    b = open(path, "rb").read()
    o = 0

    def take(dt, n):
        nonlocal o
        a = np.frombuffer(b, dt, n, o)
        o += a.nbytes
        return a

    nbh = -(-n_ff // 32)
    out = {"upload": [int(take(np.int32, 1)[0]) for _ in range(3)]}
    out["proj_st"] = int(take(np.int32, 1)[0])
    out["gate0"], out["up0"] = take(np.float32, n_ff), take(np.float32, n_ff)
    out["ffn_st"] = int(take(np.int32, 1)[0])
    out["y0"], out["hc0"], out["hs0"] = take(np.float32, n_embd), take(np.int8, n_ff), take(np.int64, nbh)
    out["group_st"] = int(take(np.int32, 1)[0])
    out["G"] = take(np.float32, n_tok * n_ff).reshape(n_tok, n_ff)
    out["U"] = take(np.float32, n_tok * n_ff).reshape(n_tok, n_ff)
    out["cols_st"] = int(take(np.int32, 1)[0])
    out["Y"] = take(np.float32, n_tok * n_embd).reshape(n_tok, n_embd)
    out["HC"] = take(np.int8, n_tok * n_ff).reshape(n_tok, n_ff)
    out["HS"] = take(np.int64, n_tok * nbh).reshape(n_tok, nbh)
    assert o == len(b)
    return out


def scaled(raw, t, scale):
    raw = raw.copy()
    qk, bb = synth.GEOM[t]
    blk = raw.reshape(-1, bb)
    for off in (o for o in synth.SCALE_AT[t] if o is not None):
        d = blk[:, off:off + 2].copy().view(np.float16).astype(np.float32) * scale
        blk[:, off:off + 2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw


def close(t, raw, n_out, n_in, codes, scales, y, what):
    st, yref = oracle.matvec_q8act(t, raw, n_out, n_in, codes, scales)
    st2, absdot = oracle.row_absdot(t, raw, n_out, n_in, codes, scales)
    assert st == 0 and st2 == 0, what
    err = np.abs(np.asarray(y, np.float64) - yref.astype(np.float64) * Q32)
    assert (err <= TOL * absdot + Q32).all(), (what, float(err.max()))


@pytest.mark.parametrize("gt,dt,n_embd,n_ff,n_tok", [(12, 14, 1536, 8960, 6), (10, 11, 512, 1000, 5),
                                                    (8, 12, 256, 512, 3)])
def test_driver_device_forms_vs_oracle(tmp_path, gt, dt, n_embd, n_ff, n_tok):
    """The Rust module's device-resident calls (grouped projections, FFN, column projections,
    column FFN) through dlopen'd entry points: projections within tolerance of the contract,
    every hidden QuantAct bit-exact to the oracle's SwiGLU + quant_act of the gate / up values of
    the same grouped GEMM, down within tolerance on that QuantAct."""
    assert os.path.exists(build.DRIVER), "build() builds tests/cpp/abi_driver"
    rng = synth.rng_for(8, 100 * gt + n_ff)
    raws = [scaled(synth.payload(gt, rng, n_ff, n_embd), gt, 1 / 32), scaled(synth.payload(gt, rng, n_ff, n_embd), gt, 1 / 32),
            scaled(synth.payload(dt, rng, n_embd, n_ff), dt, 1 / 32)]
    x = synth.activations(rng, n_embd, n_tok).reshape(n_tok, n_embd)
    st, codes, scales = oracle.quant_act_f32_batch(x)
    assert st == 0
    fi, fo = str(tmp_path / "e_in.bin"), str(tmp_path / "e_out.bin")
    write_engine_case(fi, gt, dt, n_embd, n_ff, raws, codes, scales)
    r = subprocess.run([build.DRIVER, LIB, "engine", fi, fo], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ENGINE"), r.stdout + r.stderr
    out = read_engine_out(fo, n_embd, n_ff, n_tok)
    assert out["upload"] == [0, 0, 0]
    assert (out["proj_st"], out["ffn_st"], out["group_st"], out["cols_st"]) == (0, 0, 0, 0)
    close(gt, raws[0], n_ff, n_embd, codes[0], scales[0], out["gate0"], "projections gate")
    close(gt, raws[1], n_ff, n_embd, codes[0], scales[0], out["up0"], "projections up")
    close(dt, raws[2], n_embd, n_ff, out["hc0"], out["hs0"], out["y0"], "ffn down")
    for t in range(n_tok):
        close(gt, raws[0], n_ff, n_embd, codes[t], scales[t], out["G"][t], f"group gate {t}")
        close(gt, raws[1], n_ff, n_embd, codes[t], scales[t], out["U"][t], f"group up {t}")
        sth, hc, hs, _ = oracle.swiglu_quant_f32(out["G"][t], out["U"][t])
        assert sth == 0 and (out["HC"][t] == hc).all() and (out["HS"][t] == hs).all(), f"column hidden {t}"
        close(dt, raws[2], n_embd, n_ff, out["HC"][t], out["HS"][t], out["Y"][t], f"column down {t}")
