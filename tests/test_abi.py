"""The C-ABI library builds, loads and exports every symbol include/apeiron_hip.h declares.

No compute call runs here (this suite runs without a GPU).
"""
import ctypes
import os
import re

import pytest

from apeiron_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "apeiron_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ah_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert sorted(_lib.EXPORTS) == declared_symbols()


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in declared_symbols():
        assert hasattr(L, name), name


def test_status_codes_match_oracle_and_strings():
    import oracle  # noqa: F401  (the oracle enum mirrors the ABI codes)
    L = _lib.load()
    hdr = open(os.path.join(ROOT, "include", "apeiron_hip.h")).read()
    codes = dict((m[0], int(m[1])) for m in re.findall(r"#define (AH_ERR_\w+|AH_OK) (\d+)", hdr))
    ohdr = open(os.path.join(ROOT, "oracle", "ah_oracle.h")).read()
    ocodes = dict((m[0], int(m[1])) for m in re.findall(r"(AHO_ERR_\w+|AHO_OK) = (\d+)", ohdr))
    for k, v in ocodes.items():
        assert codes[k.replace("AHO_", "AH_")] == v
    for v in codes.values():
        assert L.ah_status_str(v) and L.ah_status_str(v) != b"unknown status"


def test_no_device_is_an_honest_refusal():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    L = _lib.load()
    h = ctypes.c_void_p()
    assert L.ah_init(0, ctypes.byref(h)) == 20  # AH_ERR_NO_DEVICE
