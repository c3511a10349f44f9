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
