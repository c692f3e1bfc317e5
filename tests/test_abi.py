"""CPU-side checks of the C ABI library: it loads, exports every symbol the
header declares, rejects bad input on the host, and its host utilities agree
with the oracle.  No kernel is launched here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def gnlib():
    from goneuron_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from goneuron_amd import build
        build.build()
    return _lib.lib()


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "goneuron_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(gn_[a-z0-9_]+)\s*\(", txt)))


def test_exports_every_declared_symbol(gnlib):
    syms = declared_symbols()
    assert len(syms) > 30
    missing = [s for s in syms if not hasattr(gnlib, s)]
    assert not missing, missing


def test_bindings_cover_header():
    from goneuron_amd import _lib
    assert set(declared_symbols()) == set(_lib.SIGNATURES), \
        set(declared_symbols()) ^ set(_lib.SIGNATURES)


def test_no_device_is_an_error_not_a_fallback(gnlib):
    if gnlib.gn_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    assert gnlib.gn_init(0, C.byref(h)) == -7
    import goneuron_amd as gn
    with pytest.raises(gn.GNError):
        gn.GetDefaultDevice()


def test_null_context_rejected(gnlib):
    assert gnlib.gn_sync(None) == -1
    assert gnlib.gn_model_step(None) == -1


@pytest.mark.parametrize("kind", ["uniform", "normal", "ids"])
def test_synthetic_data_matches_oracle(gnlib, oracle, kind):
    import goneuron_amd as gn
    n = 10007
    if kind == "uniform":
        np.testing.assert_array_equal(gn.fill_uniform(n, 1001), oracle.fill_uniform(n, 1001))
    elif kind == "normal":
        np.testing.assert_array_equal(gn.fill_normal(n, 1003), oracle.fill_normal(n, 1003))
    else:
        np.testing.assert_array_equal(gn.fill_class_ids(n, 1000, 2003), oracle.fill_class_ids(n, 1000, 2003))


def test_facade_argument_errors():
    import goneuron_amd as gn
    with pytest.raises(gn.GNError):
        gn.Dense(10, gn.ReLU)          # lazy size never built by Sequential.Build
    with pytest.raises(gn.GNError):
        gn.Dropout(0.2)                # NewDropout rejects inSize <= 0
    with pytest.raises(gn.GNError):
        gn.Dropout(1.5, 10)
    d = gn.Dense(128, gn.Ref(gn.Softmax), 64)   # (out, act, in) order
    assert (d.desc.in_size, d.desc.out_size, d.desc.act_is_ptr) == (64, 128, 1)
