"""The C ABI library loads and exports every symbol include/prism_hip.h declares (no GPU calls)."""

import ctypes
import os

import pytest

import prism_hip


def test_library_exports_every_declared_symbol():
    assert os.path.exists(prism_hip.LIB_PATH), "build libprism_hip.so first (prism-inference_amd/build.py)"
    lib = ctypes.CDLL(prism_hip.LIB_PATH)
    declared = prism_hip.header_symbols()
    assert len(declared) >= 25
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # The binding covers the whole declared surface.
    prism_hip.lib()
    bound = {name for name in declared if getattr(prism_hip.lib(), name).argtypes is not None}
    assert bound == set(declared)


def test_struct_layouts_match_the_reference_blocks():
    # tools/ternary/src/lib.rs:27-39 (292-byte Q8_K) and src/kernels.rs:528-535 (prepared Q8_0)
    assert prism_hip.Q8K_DTYPE.itemsize == 292
    assert prism_hip.Q8K_DTYPE.fields["values"][1] == 4
    assert prism_hip.Q8_DTYPE.itemsize == 40


def test_library_does_not_link_the_oracle():
    with open(prism_hip.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"liboracle" not in blob and b"po_matvec" not in blob
