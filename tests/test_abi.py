"""CPU-side checks of the boundary: the HIP library loads and exports every
symbol include/volta_train.h declares; the header and the ctypes table agree.
No compute call is made (there may be no GPU)."""
import os
import re

import pytest

from volta_amd import HIP_LIB, load_hip
from volta_amd.abi import HEADER_SYMBOLS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(name="volta_train.h"):
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(volta_\w+)\s*\(", text)))


def test_header_and_ctypes_table_agree():
    assert sorted(HEADER_SYMBOLS) == header_functions()


def test_reference_six_symbols_declared():
    for s in ("volta_train_init", "volta_train_step", "volta_train_loss", "volta_train_get_params",
              "volta_train_set_params", "volta_train_free"):
        assert s in header_functions()


@pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")
def test_hip_library_exports_header_symbols():
    lib = load_hip()
    for name in header_functions():
        assert hasattr(lib.lib, name), name


@pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")
def test_hip_library_exports_vt_front_end():
    from volta_amd.abi import VT_SIGNATURES

    assert sorted(VT_SIGNATURES) == header_functions("volta_vt.h")
    lib = load_hip()
    for name in header_functions("volta_vt.h"):
        assert hasattr(lib.lib, name), name


@pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")
def test_hip_spec_parse_without_gpu():
    lib = load_hip()
    s = lib.parse_spec("1024-4096-4096-1024-10:relu:adagrad:ce:eps=1e-10")
    assert s.n_sizes == 5 and s.sizes[4] == 10 and s.loss == 1


@pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")
def test_hip_code_object_is_gfx950():
    """The library's offload bundle names a gfx950 code object and no other
    GPU target (bundle entry ids are 'hipv4-amdgcn-amd-amdhsa--<arch>')."""
    blob = open(HIP_LIB, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx\w+)", blob))
    assert targets == {b"gfx950"}, targets


def test_backend_header_symbols_exported_by_hip_and_oracle():
    """Every function include/volta_backend.h declares (the runtime optimizer
    boundary) is exported by libvolta_hip.so and by the CPU oracle."""
    import ctypes

    from tests.oracle_lib import load_oracle
    from volta_amd.backend import _SIGS

    names = header_functions("volta_backend.h")
    assert sorted(_SIGS) == names
    oracle = load_oracle().lib
    for name in names:
        assert hasattr(oracle, name), name
    if os.path.exists(HIP_LIB):
        hip = ctypes.CDLL(HIP_LIB)
        for name in names:
            assert hasattr(hip, name), name


@pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")
def test_hip_backend_capabilities_without_gpu():
    """The capabilities a HIP backend reports need no device."""
    from volta_amd.backend import capabilities

    caps = capabilities(load_hip().lib)
    assert caps["device_class"] == 1 and caps["vendor"] == 2 and caps["supports_adam"] == 1
    assert caps["default_determinism"] == 0
