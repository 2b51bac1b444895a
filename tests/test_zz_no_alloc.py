"""bch_matmul_noalloc (the entry point that allocates nothing) against
bch_matmul through the C ABI: the same kernels and the same column split, so
the outputs must be bit-identical, on two calls in a row (the second smaller,
so the static scratch holds the first call's larger contents), including a
launch whose inputs fill the static scratch almost to its end and a launch
that bch_matmul splits over its columns; a launch whose inputs and split
partials exceed the static scratch must fail with the Argument status."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from bobcat_amd import BobcatError
from bobcat_amd._lib import check, lib
from bobcat_amd.backend import Format, Store, _view
from bobcat_amd.synth import q4k_matrix

pytestmark = pytest.mark.gpu


def both(hip, w, n_rows, n_cols, x, n_tokens, store, prior):
    wb, xb = hip.buffer_from(w), hip.buffer_from(x)
    ya, yb = hip.buffer_from(prior), hip.buffer_from(prior)
    hip.begin()
    check(lib().bch_matmul(hip.handle, int(Format.Q4K), _view(wb.at(0)), n_rows, n_cols, _view(xb.at(0)),
                           _view(ya.at(0)), n_tokens, int(store)))
    check(lib().bch_matmul_noalloc(hip.handle, int(Format.Q4K), _view(wb.at(0)), n_rows, n_cols, _view(xb.at(0)),
                                   _view(yb.at(0)), n_tokens, int(store)))
    hip.end()
    a = hip.read(ya.at(0), np.empty(n_tokens * n_rows, np.float32))
    b = hip.read(yb.at(0), np.empty(n_tokens * n_rows, np.float32))
    return a, b


def test_noalloc_matches_matmul_twice(hip):
    rng = np.random.default_rng(77)
    # (2048, 4096, 2000): 2000·(2·4096 + 4) = 16.39 MB of fp16 inputs, unsplit,
    # within the 16 MiB; (512, 2048, 300): bch_matmul splits its columns.
    for n_rows, n_cols, n_tokens, store in [(2048, 4096, 2000, Store.OVERWRITE), (512, 2048, 300, Store.OVERWRITE),
                                            (256, 1024, 37, Store.ACCUMULATE)]:
        w = q4k_matrix(rng, n_rows, n_cols)
        x = (rng.standard_normal(n_tokens * n_cols) * 3).astype(np.float32)
        prior = rng.standard_normal(n_tokens * n_rows).astype(np.float32)
        a, b = both(hip, w, n_rows, n_cols, x, n_tokens, store, prior)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (n_rows, n_cols, n_tokens)


def test_noalloc_rejects_launches_beyond_its_scratch(hip):
    limit = lib().bch_matmul_noalloc_max_bytes()
    assert limit == 16 << 20
    n_cols = 8192
    n_tokens = limit // (2 * n_cols + 4) + 1  # inputs one token past the limit
    w = hip.new_buffer(16 * (n_cols // 256) * 144)
    x = hip.new_buffer(n_tokens * n_cols * 4)
    y = hip.new_buffer(n_tokens * 16 * 4)
    hip.begin()
    with pytest.raises(BobcatError) as e:
        check(lib().bch_matmul_noalloc(hip.handle, int(Format.Q4K), _view(w.at(0)), 16, n_cols, _view(x.at(0)),
                                       _view(y.at(0)), n_tokens, 0))
    hip.end()
    assert e.value.status == 14  # Argument
    assert "scratch" in str(e.value)
    # Inputs that fit but a column split whose partials do not: 128 rows of
    # 8192 columns at 1000 tokens are 16.4 MB of inputs, and bch_matmul splits
    # the columns 8 ways (4.1 MB of partials).
    n_tokens = 1000
    x = hip.new_buffer(n_tokens * n_cols * 4)
    y = hip.new_buffer(n_tokens * 128 * 4)
    w = hip.new_buffer(128 * (n_cols // 256) * 144)
    hip.begin()
    with pytest.raises(BobcatError) as e:
        check(lib().bch_matmul_noalloc(hip.handle, int(Format.Q4K), _view(w.at(0)), 128, n_cols, _view(x.at(0)),
                                       _view(y.at(0)), n_tokens, 0))
    hip.end()
    assert e.value.status == 14
