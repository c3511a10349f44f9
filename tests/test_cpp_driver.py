"""The C++ ABI driver (tests/cpp/abi_driver.cpp, the C twin of the Rust `hip` module) on the CPU.

Without a GPU it checks what the integration relies on before any compute call: the library
loads by dlopen and exports every entry point the Rust module resolves; every status maps to
exactly one error value, the one the header documents (statuses 1-9 to the nine MatvecError
variants of ops/matvec.rs:11-48, 10-11 to F32Error, 12-14 to FfnError, 20-25 to the backend);
and both skips are honest -- a missing library and a missing gfx950 device each end the driver
with a SKIP line and status 0, as Vk::load's Err does (gpu/vulkan.rs:1097-1106).
"""
import os
import re
import subprocess

import pytest

from apeiron_amd import build

LIB = os.path.join(os.path.dirname(build.__file__), "libapeiron_hip.so")
WANT = {0: "Ok", 1: "Matvec(ShapeMismatch)", 2: "Matvec(RowLength)", 3: "Matvec(ShortPayload)",
        4: "Matvec(LengthOverflow)", 5: "Matvec(UnsupportedQuant)", 6: "Matvec(Dequant(NonFiniteScale))",
        7: "Matvec(Dequant(FixedOverflow))", 8: "Matvec(AccumulatorOverflow)", 9: "Matvec(OutputOverflow)",
        10: "Input(NonFinite)", 11: "Input(OutOfRange)", 12: "Ffn(Overflow)", 13: "Ffn(ExpOutOfRange)",
        14: "Ffn(ZeroDenominator)"}


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("drv") / "abi_driver")
    return build.build_driver(out)


def run(driver, *args):
    r = subprocess.run([driver, *args], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout


def test_status_table_is_one_to_one(driver):
    rc, out = run(driver, LIB, "status")
    assert rc == 0, out
    rows = {}
    for line in out.strip().splitlines():
        m = re.match(r"(\d+) (\S+) \| (.*)$", line)
        assert m, line
        rows[int(m.group(1))] = (m.group(2), m.group(3))
    for st, name in WANT.items():
        assert rows[st][0] == name, (st, rows[st])
    # one error value per status: no two statuses 0-14 share a value
    assert len({rows[s][0] for s in WANT}) == len(WANT)
    # the library names each documented code (20-25 are the backend's own)
    for st in list(WANT) + [20, 21, 22, 23, 24, 25]:
        assert rows[st][1] != "unknown status", st
    assert rows[26][1] == "unknown status"
    # the header documents the same mapping
    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                            "apeiron_hip.h")).read()
    for st, name in ((1, "ShapeMismatch"), (3, "ShortPayload"), (5, "UnsupportedQuant"), (6, "NonFiniteScale"),
                     (8, "AccumulatorOverflow"), (9, "OutputOverflow")):
        assert re.search(rf"#define AH_ERR_\w+ {st}\s+/\*[^*]*{name}", hdr), (st, name)


def test_honest_skips(driver):
    rc, out = run(driver, "/nonexistent/libapeiron_hip.so", "probe")
    assert rc == 0 and out.startswith("SKIP") and "not found" in out
    rc, out = run(driver, LIB, "probe")
    assert rc == 0
    # this container has no GPU: ah_init's honest skip, mapped to the backend class
    if not os.path.exists("/dev/kfd"):
        assert out.startswith("SKIP ah_init: no gfx950 device (status 20, Backend)"), out
