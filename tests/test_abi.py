"""CPU checks of the C ABI: the library loads, exports every symbol that
include/nexus_hip.h declares, and its host-only entry points behave (no
compute calls are made without a GPU)."""
import ctypes as C
import os
import re

import pytest

import nexus_amd as nx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "nexus_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(nx_[a-z_0-9]+)\s*\(", src)))


def test_header_declares_the_python_export_list():
    assert header_symbols() == sorted(nx.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = nx.lib()
    for name in header_symbols():
        assert hasattr(L, name), name
        assert C.cast(getattr(L, name), C.c_void_p).value


def test_no_cpu_fallback_symbols():
    """The product library carries no oracle code."""
    data = open(nx.LIB_PATH, "rb").read()
    assert b"nxo_" not in data


def test_quant_bytes_matches_gguf_sizes():
    # src/gguf/mod.rs:262-272
    assert nx.quant_bytes(nx.Q4_K, 300) == 2 * 144
    assert nx.quant_bytes(nx.Q8_0, 33) == 2 * 34
    assert nx.quant_bytes(nx.Q4_0, 32) == 18
    assert nx.quant_bytes(nx.F32, 7) == 28
    with pytest.raises(nx.NexusError) as e:
        nx.quant_bytes(5, 10)
    assert e.value.code == nx.NX_ERR_INVALID_ARG


def test_version_and_null_arguments():
    L = nx.lib()
    assert L.nx_version() == 1
    assert L.nx_ctx_create(0, None) == nx.NX_ERR_INVALID_ARG
    assert b"null" in L.nx_last_error()
    assert L.nx_experts_info(None, None, None, None, None, None, None) == nx.NX_ERR_INVALID_ARG
    assert L.nx_ctx_destroy(None) == nx.NX_OK
    assert L.nx_experts_destroy(None) == nx.NX_OK


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU node is present")
def test_no_device_reports_device_error():
    assert nx.device_count() == 0
    with pytest.raises(nx.NexusError) as e:
        nx.Context(0)
    assert e.value.code == nx.NX_ERR_DEVICE
