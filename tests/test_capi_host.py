"""CPU: the C-ABI library loads, exports every entry point include/knj_capi.h
declares, and its host-side gate behaves like the reference's C2 arch guard
(/root/reference/src/device/device_caps.h:100-115): refuse on mismatch, and
refuse an environment override that names another arch."""
import ctypes as C
import os
import re

import pytest

import kanjoos_amd as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "knj_capi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(knj_[a-z0-9_]+)\s*\(", text)))


def test_header_and_python_exports_agree():
    assert sorted(K.EXPORTS) == declared_symbols()


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(K.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_arch_guard_strings():
    L = K.lib()
    assert L.knj_built_arch() == b"gfx950"
    assert L.knj_check_arch(b"gfx950:sramecc+:xnack-", b"gfx950", None) == K.KNJ_OK
    assert L.knj_check_arch(b"gfx950", b"gfx950", b"gfx950") == K.KNJ_OK
    assert L.knj_check_arch(b"gfx942:sramecc+:xnack-", b"gfx950", None) == K.KNJ_E_ARCH
    assert b"gfx942" in L.knj_last_error()
    assert L.knj_check_arch(b"gfx9500", b"gfx950", None) == K.KNJ_E_ARCH
    assert L.knj_check_arch(b"gfx950", b"gfx950", b"gfx1201") == K.KNJ_E_ARCH
    assert L.knj_check_arch(None, b"gfx950", None) == K.KNJ_E_ARCH


def test_calls_before_open_are_refused():
    """Compute entry points refuse until the gate has passed (no GPU touched)."""
    L = K.lib()
    rc = L.knj_gemv(K.TYPE_Q4_K, None, 256, 1, None, None, 1e-6, None, None, None)
    assert rc in (K.KNJ_E_STATE, K.KNJ_E_ARG)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU may be present")
def test_open_without_device_fails_cleanly():
    L = K.lib()
    rc = L.knj_device_open(0)
    assert rc in (K.KNJ_E_ENV, K.KNJ_E_HIP)
