"""Interface checks that need no GPU (reference tests/test_api.py:29-63)."""

import pytest
import torch

import libcertex_amd as certex
from libcertex_amd.index import _pack, row_len


def test_version():
    assert certex.__version__.count(".") == 2


def test_rejects_unknown_metric_and_storage():
    with pytest.raises(ValueError):
        certex.Index(8, metric="hamming")
    with pytest.raises(ValueError):
        certex.Index(8, storage="disk")


def test_empty_index():
    idx = certex.Index(8)
    assert idx.ntotal == 0 and idx.info()["width"] is None and idx.dtype is None
    with pytest.raises(ValueError):
        idx.search(torch.zeros(1, 8))


def test_mask_packing():
    m = torch.zeros(70, dtype=torch.bool)
    m[[0, 31, 32, 69]] = True
    w = _pack(m).numpy().view("uint32")
    assert w.tolist() == [1 | 1 << 31, 1, 1 << 5]


def test_row_length():
    assert [row_len(m) for m in (11, 59, 60, 123, 124, 251)] == [64, 64, 128, 128, 256, 256]


def test_auto_width_follows_the_spectrum():
    g = torch.Generator().manual_seed(0)
    low = torch.randn(4000, 8, generator=g) @ torch.randn(8, 256, generator=g)
    assert certex.auto_width(low, "l2") == 59
    full = torch.randn(4000, 256, generator=g)
    assert certex.auto_width(full, "l2") > 200


def test_keycache_argument_checks():
    with pytest.raises(ValueError):
        certex.KeyCache(0, 128)
    with pytest.raises(ValueError):
        certex.KeyCache(8, 128, k=4096)
