"""CPU tests of the C ABI: the library loads, exports exactly what include/arfq.h
declares, and rejects null handles without touching a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

import arf_amd
from arf_amd import arfq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "arfq.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(arfq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert _declared() == arf_amd.exported_symbols()


def test_library_exports_every_declared_symbol():
    L = arf_amd.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", arfq.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (arfq_[a-z0-9_]+)", out))
    for name in _declared():
        assert name in exported, name
        assert getattr(L, name) is not None


def test_version_and_status_strings():
    L = arf_amd.load_library()
    assert L.arfq_version() == 100
    assert L.arfq_status_string(0) == b"ok"
    assert L.arfq_status_string(-2) == b"shape mismatch"


def test_null_handles_are_rejected():
    L = arf_amd.load_library()
    assert L.arfq_ctx_destroy(None) == arfq.ARFQ_E_INVALID
    assert L.arfq_ctx_sync(None) == arfq.ARFQ_E_INVALID
    assert L.arfq_weight_free(None) == arfq.ARFQ_E_INVALID
    assert L.arfq_weight_info(None, None, None, None, None, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_matmul(None, None, 0, 1, None, 0, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_dequant_f32(None, None, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_moe_route(None, None, 1, 8, 2, 1, None, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_moe(None, None, None, None, None, 1, 2, 1, None, 0, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_ctx_create(0, None, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_ctx_set_options(None, 0) == arfq.ARFQ_E_INVALID
    assert L.arfq_moe_add(None, None, None, None, None, 1, 2, 1, None, 0, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_moe_ids_add(None, None, None, None, None, None, 1, 2, None, 0, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_ffn(None, None, None, None, 1, None, None) == arfq.ARFQ_E_INVALID
    assert L.arfq_ffn_act(None, None, None, None, 1, None, None, arfq.ACT_GELU_TANH) == arfq.ARFQ_E_INVALID


def test_no_gpu_here_fails_loudly():
    if os.environ.get("ARFQ_EXPECT_GPU"):
        pytest.skip("GPU box")
    try:
        arf_amd.Context(0)
    except arf_amd.ArfqError as e:
        assert e.status == arfq.ARFQ_E_DEVICE
    else:  # a GPU is present: nothing to check here
        pass


def test_package_has_no_oracle_or_fallback_import():
    # the product path must not route through the CPU checker
    pkg = os.path.join(ROOT, "arf_amd")
    for f in os.listdir(pkg):
        if f.endswith(".py"):
            src = open(os.path.join(pkg, f)).read()
            assert not re.search(r"^\s*(from|import)\s+oracle\b", src, flags=re.M), f
            assert "liboracle" not in src, f
