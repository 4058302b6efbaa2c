"""fl_mean_pool_noalloc (no counterpart in the reference: the mean pool for
callers that cannot allocate device memory) against fl_mean_pool, the entry
point it is a variant of.  Both run the same kernels, so the outputs must be
equal bit for bit, on two calls in a row, the second with a smaller input
(the static scratch array keeps the first call's contents)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def device_free_bytes():
    """hipMemGetInfo's free bytes of the current device (device 0, made
    current on this thread by the library's entry points)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("dtype_name", ["F16", "F32"])
def test_noalloc_pool_matches_fl_mean_pool(ctx, fl, dtype_name):
    dtype = getattr(fl, dtype_name)
    rng = np.random.default_rng(7)
    cases = [
        (np.array([512, 300, 64, 9, 512, 1, 129, 77] * 8, np.int64), 768, True),
        (np.array([33, 5, 200], np.int64), 768, False),
    ]
    for lengths, cols, l2 in cases:
        print(f"noalloc pool dtype={dtype_name} nseq={lengths.size} cols={cols} l2={l2}",
              flush=True)
        x = rng.standard_normal((int(lengths.sum()), cols)).astype(np.float32)
        hid = ctx.tensor(x, dtype)
        want = ctx.mean_pool(hid, lengths, l2=l2)
        out = ctx.empty((lengths.size, cols), fl.F32)
        ctx.synchronize()
        before = ctx.vram_usage()[0]
        free0 = device_free_bytes()
        ctx.mean_pool(hid, lengths, l2=l2, out=out, noalloc=True)
        ctx.synchronize()
        # Neither the library's count nor the device's free memory moves.
        assert ctx.vram_usage()[0] == before
        assert device_free_bytes() == free0
        np.testing.assert_array_equal(out.numpy(), want.numpy())
        for t in (hid, want, out):
            t.free()


def test_noalloc_pool_limits(ctx, fl):
    # More sequences than the kernel arguments carry: refused on the host.
    hid = ctx.empty((513, 8), fl.F32)
    out = ctx.empty((513, 8), fl.F32)
    with pytest.raises(fl.FletcherError, match="sequences"):
        ctx.mean_pool(hid, np.ones(513, np.int64), out=out, noalloc=True)
    ctx.mean_pool(hid, np.ones(512, np.int64), out=out, noalloc=True)
    hid.free()
    out.free()
    # Partial sums past the scratch array: 1 sequence of 65 chunks (4160 rows)
    # x 65536 columns x 4 bytes = 17,039,360 > 16 MiB.  The buffers are as
    # large as the lengths claim, so nothing could be read out of bounds.
    rows, cols = 64 * 65, 65536
    hid = ctx.empty((rows, cols), fl.F16)
    out = ctx.empty((1, cols), fl.F32)
    with pytest.raises(fl.FletcherError, match="scratch array"):
        ctx.mean_pool(hid, np.array([rows], np.int64), out=out, noalloc=True)
    # One chunk fewer fits (64 x 65536 x 4 = 16 MiB exactly).
    ctx.mean_pool(hid, np.array([rows - 64], np.int64), out=out, noalloc=True)
    ctx.synchronize()
    assert not np.any(out.numpy())
    hid.free()
    out.free()


def test_noalloc_pool_two_contexts_in_call_order(fl):
    """Two contexts on one GPU share its scratch array: calls made one after
    the other, without a host synchronisation between them, run in that
    order (the second waits for the first's kernels), so each gets its own
    result."""
    rng = np.random.default_rng(9)
    ca, cb = fl.Context(0), fl.Context(0)
    ts = []
    try:
        la = np.array([512] * 64, np.int64)
        lb = np.array([7, 300, 41], np.int64)
        ha = ca.tensor(rng.standard_normal((int(la.sum()), 768)).astype(np.float32), fl.F16)
        hb = cb.tensor(rng.standard_normal((int(lb.sum()), 768)).astype(np.float32), fl.F16)
        wa, wb = ca.mean_pool(ha, la), cb.mean_pool(hb, lb)
        oa, ob = ca.empty((la.size, 768), fl.F32), cb.empty((lb.size, 768), fl.F32)
        ts = [(ca, t) for t in (ha, wa, oa)] + [(cb, t) for t in (hb, wb, ob)]
        ca.synchronize()
        cb.synchronize()
        for _ in range(3):
            ca.mean_pool(ha, la, out=oa, noalloc=True)
            cb.mean_pool(hb, lb, out=ob, noalloc=True)
            ca.mean_pool(ha, la, out=oa, noalloc=True)
        np.testing.assert_array_equal(ob.numpy(), wb.numpy())
        np.testing.assert_array_equal(oa.numpy(), wa.numpy())
    finally:
        for _, t in ts:
            t.free()
        ca.close()
        cb.close()
