"""The allocation-free max-pool entry point (mpcx_maxpool_eval_noalloc),
through the C ABI: on the same keys and inputs it returns what the allocating
entry point mpcx_maxpool_eval returns, on two calls in a row (the second with a
smaller input, so the static scratch array holds the first call's planes), it
refuses a call whose workspace exceeds the array, and a call from another
stream while the array's last call is still pending (MPCX_EBUSY)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(c, rng, B, N, C):
    bw = c.bw
    mask = (1 << bw) - 1
    v = rng.integers(-(1 << 24), 1 << 24, size=(B, N, C), dtype=np.int64)
    rin = rng.integers(0, 1 << 63, size=v.size, dtype=np.uint64) & np.uint64(mask)
    k0, k1, rout = c.maxpool_keygen(B, N, C, rin, seed=17 + N, gate=3)
    xhat = (v.reshape(-1).astype(np.uint64) + rin) & np.uint64(mask)
    return v, k0, k1, rout, xhat


@pytest.mark.parametrize("bw", [32, 64])
def test_maxpool_noalloc_matches_allocating_entry(bw):
    import mpcx
    c = mpcx.Ctx(bw=bw)
    rng = np.random.default_rng(bw)
    # the affinity pool shape (64 x 140 x 312: at bw=64 its workspace is
    # 67,092,480 bytes of the 64 MiB array), then a smaller call
    for B, N, C in ((64, 140, 312), (3, 7, 5)):
        v, k0, k1, rout, xhat = _case(c, rng, B, N, C)
        c.reset_counters()
        want = c.maxpool_eval(B, N, C, k0, k1, xhat)
        by = c.bytes_exchanged
        c.reset_counters()
        got = c.maxpool_eval_noalloc(B, N, C, k0, k1, xhat)
        assert np.array_equal(got, want)
        assert c.bytes_exchanged == by
        y = (got.astype(np.uint64) - rout.astype(np.uint64)) & np.uint64((1 << bw) - 1)
        y = y.astype(np.int64) if bw == 32 else y.view(np.int64)
        if bw == 32:
            y = np.where(y >= 1 << 31, y - (1 << 32), y)
        assert np.array_equal(y.reshape(B, C), v.max(axis=1))
    c.close()


def test_maxpool_noalloc_refuses_oversized_workspace():
    import mpcx
    c = mpcx.Ctx(bw=64)
    B, N, C = 65, 140, 312  # 68,140,860 bytes of workspace > 64 MiB
    dummy = mpcx.empty_dev(8 * B * N * C)
    out = mpcx.empty_dev(8 * B * C)
    st = c.lib.mpcx_maxpool_eval_noalloc(c.h, B, N, C, mpcx.dptr(dummy), mpcx.dptr(dummy), mpcx.dptr(dummy),
                                         mpcx.dptr(out))
    assert st == 1  # MPCX_EINVAL, before any launch
    assert b"exceeds" in c.lib.mpcx_last_error(c.h)
    c.close()


def test_maxpool_noalloc_refuses_a_second_stream_while_busy():
    """Two contexts (two streams) on one GPU: while the first context's calls on
    the static array are still queued, the second context's call is refused
    with MPCX_EBUSY before any launch; once the first stream has drained, the
    second context's call runs and matches the allocating entry point.  Two
    contexts sharing one stream (mpcx_set_stream) are ordered and never refused."""
    import torch

    import mpcx
    a, b = mpcx.Ctx(bw=64), mpcx.Ctx(bw=64)
    rng = np.random.default_rng(5)
    B, N, C = 64, 140, 312
    v, k0, k1, rout, xhat = _case(a, rng, B, N, C)
    want = a.maxpool_eval(B, N, C, k0, k1, xhat)
    dx = mpcx.to_dev(xhat)
    outs = [mpcx.empty_dev(8 * B * C) for _ in range(2)]
    args = (B, N, C, mpcx.dptr(k0), mpcx.dptr(k1), mpcx.dptr(dx))
    torch.cuda.synchronize()  # the inputs are on torch's stream, the calls on the contexts' own
    for _ in range(6):  # several milliseconds of queued work on a's stream
        assert a.lib.mpcx_maxpool_eval_noalloc(a.h, *args, mpcx.dptr(outs[0])) == 0
    st = b.lib.mpcx_maxpool_eval_noalloc(b.h, *args, mpcx.dptr(outs[1]))
    err = b.lib.mpcx_last_error(b.h)
    a.sync()
    assert st == 6, (st, err)  # MPCX_EBUSY
    assert b"in use" in err
    assert b.lib.mpcx_maxpool_eval_noalloc(b.h, *args, mpcx.dptr(outs[1])) == 0
    b.sync()
    for o in outs:
        assert np.array_equal(mpcx.from_dev(o, np.uint64, B * C), want)
    # both contexts on one stream: ordered, never refused
    shared = torch.cuda.Stream()
    for c in (a, b):
        assert c.lib.mpcx_set_stream(c.h, shared.cuda_stream) == 0
    outs[0].zero_()
    torch.cuda.synchronize()
    assert b.lib.mpcx_maxpool_eval_noalloc(b.h, *args, mpcx.dptr(outs[1])) == 0
    assert a.lib.mpcx_maxpool_eval_noalloc(a.h, *args, mpcx.dptr(outs[0])) == 0
    shared.synchronize()
    assert np.array_equal(mpcx.from_dev(outs[0], np.uint64, B * C), want)
    for c in (a, b):
        assert c.lib.mpcx_set_stream(c.h, None) == 0
    a.close()
    b.close()
