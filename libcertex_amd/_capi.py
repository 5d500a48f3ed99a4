"""ctypes binding of libcertex_c.so, the C API of the index (include/cuvs/neighbors/certex.h).

Python reaches the index only through these C entry points; tensors cross as DLPack v1.0 structs
that borrow torch's memory (no deleter is called). The library must have been built
(python -m libcertex_amd.build): a missing library is an error, there is no other code path.
"""

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcertex_c.so")

kDLCPU, kDLROCM = 1, 10
kDLInt, kDLUInt, kDLFloat, kDLBfloat = 0, 1, 2, 4
NO_FILTER, BITSET, BITMAP = 0, 1, 2
L2Expanded, CosineExpanded, InnerProduct = 0, 2, 6
CUVS_ERROR, CUVS_SUCCESS = 0, 1

_DL = {
    torch.float32: (kDLFloat, 32),
    torch.float16: (kDLFloat, 16),
    torch.bfloat16: (kDLBfloat, 16),
    torch.int8: (kDLInt, 8),
    torch.uint8: (kDLUInt, 8),
    torch.int64: (kDLInt, 64),
    torch.int32: (kDLInt, 32),
}


class DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int), ("device_id", ctypes.c_int32)]


class DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class DLTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("device", DLDevice),
        ("ndim", ctypes.c_int32),
        ("dtype", DLDataType),
        ("shape", ctypes.POINTER(ctypes.c_int64)),
        ("strides", ctypes.POINTER(ctypes.c_int64)),
        ("byte_offset", ctypes.c_uint64),
    ]


class DLManagedTensor(ctypes.Structure):
    _fields_ = [("dl_tensor", DLTensor), ("manager_ctx", ctypes.c_void_p), ("deleter", ctypes.c_void_p)]


class IndexParams(ctypes.Structure):
    _fields_ = [
        ("metric", ctypes.c_int),
        ("width", ctypes.c_int32),
        ("variance", ctypes.c_double),
        ("anchor_stride", ctypes.c_int32),
        ("pca_sample", ctypes.c_int64),
        ("host_vectors", ctypes.c_bool),
        ("n_lists", ctypes.c_int32),
        ("local_projections", ctypes.c_bool),
        ("int8_rows", ctypes.c_bool),
    ]


class SearchParams(ctypes.Structure):
    _fields_ = [("anchors", ctypes.c_int32), ("batch_size", ctypes.c_int32), ("probe_lists", ctypes.c_int32)]


class IndexHandle(ctypes.Structure):
    _fields_ = [("addr", ctypes.c_size_t), ("dtype", DLDataType)]


class Filter(ctypes.Structure):
    _fields_ = [("addr", ctypes.c_size_t), ("type", ctypes.c_int)]


class CertexError(RuntimeError):
    """An error reported by the C API (its last-error text)."""


_lib = None
_lock = threading.Lock()


def lib():
    """The loaded C library (loaded once; an error if it was not built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build it with `python -m libcertex_amd.build` "
                        "(hipcc, gfx950)"
                    )
                L = ctypes.CDLL(LIB_PATH)
                P = ctypes.POINTER
                vp, i64, i32, err = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int
                sig = {
                    "cuvsResourcesCreate": [P(ctypes.c_size_t)],
                    "cuvsResourcesDestroy": [ctypes.c_size_t],
                    "cuvsStreamSet": [ctypes.c_size_t, vp],
                    "cuvsStreamSync": [ctypes.c_size_t],
                    "cuvsCertexIndexParamsCreate": [P(P(IndexParams))],
                    "cuvsCertexIndexParamsDestroy": [P(IndexParams)],
                    "cuvsCertexSearchParamsCreate": [P(P(SearchParams))],
                    "cuvsCertexSearchParamsDestroy": [P(SearchParams)],
                    "cuvsCertexIndexCreate": [P(P(IndexHandle))],
                    "cuvsCertexIndexDestroy": [P(IndexHandle)],
                    "cuvsCertexIndexGetSize": [P(IndexHandle), P(i64)],
                    "cuvsCertexIndexGetDim": [P(IndexHandle), P(i64)],
                    "cuvsCertexBuild": [ctypes.c_size_t, P(IndexParams), P(DLManagedTensor), P(IndexHandle)],
                    "cuvsCertexExtend": [ctypes.c_size_t, P(DLManagedTensor), P(IndexHandle)],
                    "cuvsCertexRemove": [ctypes.c_size_t, P(DLManagedTensor), P(IndexHandle)],
                    "cuvsCertexSetLabels": [ctypes.c_size_t, P(DLManagedTensor), i64, P(IndexHandle)],
                    "cuvsCertexPartitionByLabels": [ctypes.c_size_t, P(IndexHandle)],
                    "cuvsCertexSearch": [
                        ctypes.c_size_t,
                        P(SearchParams),
                        P(IndexHandle),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        Filter,
                    ],
                    "cuvsCertexSearchNoAlloc": [
                        ctypes.c_size_t,
                        P(SearchParams),
                        P(IndexHandle),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        Filter,
                    ],
                    "cuvsCertexSearchWithLabels": [
                        ctypes.c_size_t,
                        P(SearchParams),
                        P(IndexHandle),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                        P(DLManagedTensor),
                    ],
                    "cuvsCertexSerialize": [ctypes.c_size_t, ctypes.c_char_p, P(IndexHandle)],
                    "cuvsCertexDeserialize": [ctypes.c_size_t, ctypes.c_char_p, P(IndexHandle)],
                    "cuvsCertexIndexGetRemoved": [P(IndexHandle), P(i64)],
                    "cuvsCertexIndexGetCapacity": [P(IndexHandle), P(i64)],
                    "cuvsCertexIndexGetWidth": [P(IndexHandle), P(i32)],
                    "cuvsCertexIndexGetMetric": [P(IndexHandle), P(ctypes.c_int)],
                    "cuvsCertexIndexGetAnchorStride": [P(IndexHandle), P(i32)],
                    "cuvsCertexIndexHasLabels": [P(IndexHandle), P(ctypes.c_bool)],
                    "cuvsCertexIndexGetHostVectors": [P(IndexHandle), P(ctypes.c_bool)],
                    "cuvsCertexIndexGetPartitioned": [P(IndexHandle), P(i64)],
                    "cuvsCertexIndexGetLists": [P(IndexHandle), P(i32), P(i64)],
                    "cuvsCertexReserve": [ctypes.c_size_t, i64, P(IndexHandle)],
                    "cuvsCertexIndexListOrder": [ctypes.c_size_t, P(IndexHandle), P(DLManagedTensor)],
                    "cuvsCertexStatsBegin": [],
                    "cuvsCertexStatsEnd": [P(i64), P(i64), P(i64)],
                    "cuvsCertexTimingShaderClock": [P(ctypes.c_double)],
                    "cuvsCertexTestCaptureBegin": [],
                    "cuvsCertexTestCaptureGet": [ctypes.c_char_p, vp, P(i64)],
                    "cuvsCertexTrimPool": [ctypes.c_size_t],
                    "cuvsCertexTestScratchCap": [ctypes.c_size_t, i64],
                    "cuvsCertexTimingBegin": [],
                    "cuvsCertexTimingEnd": [P(ctypes.c_double), P(i64)],
                }
                for name, args in sig.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = err
                L.cuvsGetLastErrorText.argtypes = []
                L.cuvsGetLastErrorText.restype = ctypes.c_char_p
                _lib = L
    return _lib


def check(status):
    """Raise the C API's last error as a ValueError (argument errors) or CertexError."""
    if status != CUVS_SUCCESS:
        msg = lib().cuvsGetLastErrorText()
        text = msg.decode() if msg else "unknown error"
        if "HIP error" in text or "out of memory" in text:
            raise CertexError(text)
        raise ValueError(text)


class Borrowed:
    """A DLManagedTensor that borrows a contiguous torch tensor (kept alive with it)."""

    def __init__(self, t, dtype_override=None):
        if not t.is_contiguous():
            t = t.contiguous()
        self.t = t
        self.shape = (ctypes.c_int64 * max(1, t.ndim))(*t.shape)
        code, bits = dtype_override if dtype_override is not None else _DL[t.dtype]
        dev = DLDevice(kDLROCM if t.is_cuda else kDLCPU, t.device.index or 0 if t.is_cuda else 0)
        self.m = DLManagedTensor()
        self.m.dl_tensor = DLTensor(
            ctypes.c_void_p(t.data_ptr()),
            dev,
            t.ndim,
            DLDataType(code, bits, 1),
            ctypes.cast(self.shape, ctypes.POINTER(ctypes.c_int64)),
            None,
            0,
        )
        self.m.manager_ctx = None
        self.m.deleter = None

    @property
    def ptr(self):
        return ctypes.byref(self.m)


_tls = threading.local()


def resources():
    """Per-thread, per-device C resources bound to torch's current stream."""
    dev = torch.cuda.current_device()
    stream = torch.cuda.current_stream().cuda_stream
    cache = getattr(_tls, "res", None)
    if cache is None:
        cache = _tls.res = {}
    entry = cache.get(dev)
    if entry is None:
        h = ctypes.c_size_t(0)
        check(lib().cuvsResourcesCreate(ctypes.byref(h)))
        entry = cache[dev] = [h.value, None]
    if entry[1] != stream:
        check(lib().cuvsStreamSet(entry[0], ctypes.c_void_p(stream)))
        entry[1] = stream
    return entry[0]
