"""The C ABI library: it loads, exports every symbol the header declares, and validates
descriptions and reports errors without a GPU (no kernel is launched)."""
import ctypes as C
import os
import re

import pytest

from hydra_amd import _lib as L
from hydra_amd import formats as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "hydra_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hh_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    assert _declared() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in _declared():
        assert hasattr(lib, name), name


@pytest.mark.parametrize("mutate,code", [
    (dict(top_k=9), -3), (dict(top_k=0), -3), (dict(top_k=40), -3),
    (dict(hidden=2880 + 32), -6), (dict(intermediate=100), -6),
    (dict(quant=7), -1), (dict(activation=5), -1), (dict(router=3), -1),
    (dict(experts=0), -1), (dict(experts=600, top_k=4), -1),
    (dict(quant=F.QUANT_MLX4, group_size=32), -6),
])
def test_desc_check_rejects_bad_descriptions(mutate, code):
    d = L.desc_c(F.GPT_OSS_20B.replace(**mutate))
    assert L.lib().hh_desc_check(C.byref(d)) == code
    assert L.lib().hh_last_error()


def test_desc_check_accepts_every_config():
    for desc in F.CONFIGS.values():
        d = L.desc_c(desc)
        assert L.lib().hh_desc_check(C.byref(d)) == 0


def test_blob_layout_matches_python_layout():
    for desc in F.CONFIGS.values():
        off, by, payload, stride = L.blob_layout(desc)
        py = F.blob_layout(desc)
        assert (off, by, payload, stride) == (list(py.offsets), list(py.sizes), py.payload, py.stride)
        if desc.shared_intermediate:
            assert L.blob_layout(desc, desc.shared_intermediate)[3] == F.blob_layout(desc, desc.shared_intermediate).stride


def test_null_arguments_are_errors_not_crashes():
    lib = L.lib()
    assert lib.hh_moe_forward(None, None, None, None, None, 1, None, None, None) == -1
    assert lib.hh_mxfp4_dequant(None, None, None, 1, None) == -1
    assert lib.hh_ctx_create(None, 0) == -1
