"""The C-ABI library: it loads, exports every function that include/ declares, and its host-only
entry points behave like the reference C API (c/src/neighbors/certex.cpp:162-230,
c/src/core/exceptions.hpp:17-33). No GPU is needed: nothing here launches a kernel."""

import ctypes
import glob
import os
import re

import pytest

from libcertex_amd import _capi as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "**", "*.h"), recursive=True):
        text = open(h).read()
        names.update(re.findall(r"CUVS_EXPORT\s+[\w\s\*]+?\b(\w+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert "cuvsCertexSearch" in names and len(names) >= 15 + 7
    lib = ctypes.CDLL(C.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_entry_points_present():
    ref = [
        "cuvsCertexIndexParamsCreate", "cuvsCertexIndexParamsDestroy", "cuvsCertexSearchParamsCreate",
        "cuvsCertexSearchParamsDestroy", "cuvsCertexIndexCreate", "cuvsCertexIndexDestroy",
        "cuvsCertexIndexGetSize", "cuvsCertexIndexGetDim", "cuvsCertexBuild", "cuvsCertexExtend",
        "cuvsCertexRemove", "cuvsCertexSetLabels", "cuvsCertexPartitionByLabels", "cuvsCertexSearch",
        "cuvsCertexSearchWithLabels", "cuvsCertexSerialize", "cuvsCertexDeserialize",
    ]
    assert set(ref) <= set(declared_functions())


def test_parameter_defaults():
    L = C.lib()
    p = ctypes.POINTER(C.IndexParams)()
    C.check(L.cuvsCertexIndexParamsCreate(ctypes.byref(p)))
    v = p.contents
    assert (v.metric, v.width, v.variance, v.anchor_stride, v.pca_sample) == (C.L2Expanded, 0, 0.95, 16, 1_000_000)
    assert (v.host_vectors, v.n_lists, v.local_projections, v.int8_rows) == (False, 0, False, False)
    C.check(L.cuvsCertexIndexParamsDestroy(p))
    s = ctypes.POINTER(C.SearchParams)()
    C.check(L.cuvsCertexSearchParamsCreate(ctypes.byref(s)))
    assert (s.contents.anchors, s.contents.batch_size, s.contents.probe_lists) == (128, 2048, 2)
    C.check(L.cuvsCertexSearchParamsDestroy(s))


def test_errors_become_status_and_text():
    L = C.lib()
    h = ctypes.POINTER(C.IndexHandle)()
    C.check(L.cuvsCertexIndexCreate(ctypes.byref(h)))
    h.contents.dtype = C.DLDataType(C.kDLUInt, 8, 1)
    size = ctypes.c_int64()
    assert L.cuvsCertexIndexGetSize(h, ctypes.byref(size)) == C.CUVS_ERROR
    assert b"empty" in L.cuvsGetLastErrorText()
    with pytest.raises(ValueError, match="empty"):
        C.check(L.cuvsCertexIndexGetSize(h, ctypes.byref(size)))
    h.contents.dtype = C.DLDataType(C.kDLFloat, 64, 1)
    assert L.cuvsCertexIndexGetDim(h, ctypes.byref(size)) == C.CUVS_ERROR
    assert b"float32, float16, bfloat16, int8, or uint8" in L.cuvsGetLastErrorText()
    # a successful call clears the text
    C.check(L.cuvsCertexStatsBegin())
    assert L.cuvsGetLastErrorText() is None
    q, s, v = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    C.check(L.cuvsCertexStatsEnd(ctypes.byref(q), ctypes.byref(s), ctypes.byref(v)))
    assert (q.value, s.value, v.value) == (0, 0, 0)
    h.contents.dtype = C.DLDataType(C.kDLUInt, 8, 1)
    C.check(L.cuvsCertexIndexDestroy(h))


def test_null_resources_rejected():
    L = C.lib()
    assert L.cuvsStreamSync(0) == C.CUVS_ERROR
    assert b"NULL" in L.cuvsGetLastErrorText()
