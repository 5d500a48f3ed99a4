"""Host-side interface checks (no GPU): argument validation, the filter-word layout, the row length
rule and the width rule. The known answers are the reference's (tests/test_api.py:43-63): the
mask bits [0, 31, 32, 69] pack to [1 | 1 << 31, 1, 1 << 5]; widths 11, 59, 60, 123, 124, 251 give
rows of 64, 64, 128, 128, 256, 256 halves; rank-8 data gets width 59."""

import numpy as np
import pytest
import torch

import libcertex_amd as certex
from libcertex_amd.index import _cast, _pack, row_len


def test_version_string():
    major, minor, patch = certex.__version__.split(".")
    assert all(p.isdigit() for p in (major, minor, patch))


@pytest.mark.parametrize("kw", [{"metric": "hamming"}, {"metric": "L2"}, {"storage": "disk"}])
def test_index_rejects_unknown_options(kw):
    with pytest.raises(ValueError):
        certex.Index(16, **kw)


def test_index_before_the_first_add():
    idx = certex.Index(16)
    info = idx.info()
    assert idx.ntotal == 0 and idx.dtype is None and info["width"] is None and info["n_lists"] == 0
    for call in (lambda: idx.search(torch.zeros(2, 16)), lambda: idx.remove([0]), lambda: idx.list_order()):
        with pytest.raises(ValueError):
            call()


def words(mask):
    return _pack(torch.as_tensor(mask)).numpy().view(np.uint32).tolist()


def test_filter_words_reference_answer():
    m = np.zeros(70, bool)
    m[[0, 31, 32, 69]] = True
    assert words(m) == [1 | 1 << 31, 1, 1 << 5]


def test_filter_words_match_numpy_little_endian_bits():
    """Entry e is bit e % 32 of word e // 32, rows of a bitmap laid out one after the other."""
    m = np.random.default_rng(5).random((3, 101)) < 0.4
    bits = np.packbits(m.reshape(-1), bitorder="little")
    ref = np.pad(bits, (0, (-bits.size) % 4)).view("<u4").tolist()
    assert words(m) == ref
    assert words(np.ones(32, bool)) == [0xFFFFFFFF]
    assert words(np.zeros(1, bool)) == [0]


@pytest.mark.parametrize("m,halves", [(1, 64), (11, 64), (59, 64), (60, 128), (123, 128), (124, 256), (251, 256), (252, 384)])
def test_row_length_rule(m, halves):
    assert row_len(m) == halves


def test_width_rule_follows_the_spectrum():
    g = torch.Generator().manual_seed(3)
    rank8 = torch.randn(3000, 8, generator=g) @ torch.randn(8, 192, generator=g)
    assert certex.auto_width(rank8, "l2") == 59
    assert certex.auto_width(rank8, "ip") == 59
    flat = torch.randn(3000, 192, generator=g)
    assert certex.auto_width(flat, "l2") == 192  # no tile below the dimension holds 95%
    assert certex.auto_width(torch.randn(500, 40, generator=g), "l2") == 40  # capped at the dimension


def test_integer_index_takes_only_integers():
    """Values of an integer index must be integers its type holds (tests/test_exact.py:342-350)."""
    ok = _cast(torch.tensor([[0.0, 255.0]]), torch.uint8)
    assert ok.dtype == torch.uint8 and ok.tolist() == [[0, 255]]
    for bad in ([[0.5, 1.0]], [[256.0, 0.0]], [[-1.0, 3.0]], [[float("nan"), 0.0]]):
        with pytest.raises(ValueError):
            _cast(torch.tensor(bad), torch.uint8)
    with pytest.raises(ValueError):
        _cast(torch.tensor([[200]], dtype=torch.int32), torch.int8)
    assert _cast(torch.tensor([[-128, 127]], dtype=torch.int32), torch.int8).tolist() == [[-128, 127]]


def test_keycache_rejects_bad_shapes():
    for args, kw in (((0, 64), {}), ((4, 0), {}), ((4, 64), {"k": 0}), ((4, 64), {"k": 2049})):
        with pytest.raises(ValueError):
            certex.KeyCache(*args, **kw)
