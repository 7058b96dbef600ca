"""mk_argmax_top2_noalloc (the allocation-free, context-free greedy selection) against mk_argmax_top2 through the C
ABI: identical ids on two calls in a row, the second with fewer rows (the static scratch keeps the first call's
partials), on the context's stream and on the null stream; no device memory allocated by the calls (free memory
unchanged); more rows than the static scratch holds is an error, not an overrun."""
import ctypes

import numpy as np
import pytest

import malkin_amd as mk_

pytestmark = pytest.mark.gpu


def hip():
    return ctypes.CDLL("libamdhip64.so")


def free_bytes():
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip().hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
    return f.value


def logits(rng, rows, V):
    l = rng.standard_normal((rows, V)).astype(np.float32)
    l[0, [5, V // 2, V - 1]] = 99.0  # a three-way tie: the first index wins, the next is the runner-up
    if rows > 1:
        l[1, :] = 1.0                # all equal
    if rows > 2:
        l[2, V - 1] = 50.0           # the maximum at the last index
    return l


def run_pair(mk, l, stream_of_ctx):
    L = mk_.load()
    rows, V = l.shape
    dl = mk.to_device(l)
    a1, a2, b1, b2 = (mk.alloc(rows * 4) for _ in range(4))
    mk_.check(L.mk_argmax_top2(mk.h, dl.ptr, rows, V, a1.ptr, a2.ptr))
    mk.sync()
    stream = L.mk_stream(mk.h) if stream_of_ctx else None
    if stream is None:
        # The runtime creates the null stream's queue (a few MiB) the first time anything uses that stream; a plain
        # runtime copy on it first, so that the free-memory check below sees only the entry point.
        assert hip().hipMemcpy(b1.ptr, a1.ptr, ctypes.c_size_t(4), 3) == 0
    before = free_bytes()
    print(f"noalloc: rows {rows}, vocab {V}, stream {'context' if stream_of_ctx else 'null'}", flush=True)
    mk_.check(L.mk_argmax_top2_noalloc(stream, dl.ptr, rows, V, b1.ptr, b2.ptr))
    assert hip().hipDeviceSynchronize() == 0
    assert free_bytes() == before
    out = [x.download(np.int32) for x in (a1, a2, b1, b2)]
    for x in (dl, a1, a2, b1, b2):
        x.free()
    return out


@pytest.mark.parametrize("stream_of_ctx", [True, False])
def test_noalloc_matches_the_context_entry_point(mk, stream_of_ctx):
    rng = np.random.default_rng(11)
    for rows, V in ((200, 151936), (5, 3000)):  # second call smaller: stale partials of the first must not leak
        l = logits(rng, rows, V)
        a1, a2, b1, b2 = run_pair(mk, l, stream_of_ctx)
        assert np.array_equal(a1, b1) and np.array_equal(a2, b2), (rows, V)
        assert (a1[0], a2[0]) == (5, V // 2)
        assert a1[1] == 0 and a2[1] == 1
        assert a1[2] == V - 1


def test_noalloc_rejects_more_rows_than_its_scratch(mk):
    L = mk_.load()
    d = mk.alloc(257 * 64 * 4)
    t = mk.alloc(257 * 4)
    rc = L.mk_argmax_top2_noalloc(L.mk_stream(mk.h), d.ptr, 257, 64, t.ptr, None)
    assert rc == mk_.MK_ERR_INVALID
    assert b"256 rows" in L.mk_last_error()
    d.free()
    t.free()
