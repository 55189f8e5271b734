"""Ring GEMM kernel paths against the oracle, both rings.

The default path takes, in Z_2^32, the panel kernel wherever it applies (rows
and columns whole 16-byte groups, K within one step or enough workgroups),
the wide-K matrix-core kernel wherever that applies (enough tiles for a
quarter of the CUs, or K within one step) and the tiled matrix-core kernels
elsewhere (long K over few tiles, split-K); MPCX_GEMM=wide skips the panel
kernel and MPCX_GEMM=tiled forces the tiled kernels everywhere.  Z_2^32 SxS
products of both parties take the LDS-staged kernel (k_sxs_staged) where K is
a multiple of 4, on the default and wide paths; MPCX_SXS_STAGED=0 gives them
to the panel and fused kernels as before (the "nostaged" context).  The shapes
below make the panel and wide kernels take every branch: one and several K
steps (a last step of one 16-byte group), steps with masks, party 1's two K
segments, rows read as 16-byte groups or word by word (K not a multiple of
the group), ragged M and N, 16- and 32-column panel workgroups; the SxS
products also take the fused evaluation of both parties with the
reconstruction in the same launch (three panels, or the fused SxS kernel).
Every result is checked bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (M, K, N): single step (K <= 288 words of Z_2^32, 144 of Z_2^64), several
# steps with 64+ tiles, K not a multiple of the 16-byte group, tiny; few-row
# products (split-K with K ending inside an MFMA chunk and ragged N, one chunk,
# 128 rows of a long K, K not a whole number of groups); the dot kernel (N <= 4)
# with two rounds of loads
GEMM_SHAPES = [(3080, 78, 78), (3080, 156, 312), (140, 140, 312), (130, 77, 65), (600, 700, 300), (64, 63, 1),
               (1, 1, 1), (22, 256, 1024), (64, 144, 64), (48, 148, 36), (200, 288, 32), (100, 340, 70),
               (33, 12, 17), (128, 1024, 20), (20, 77, 40), (5, 700, 3)]
# (nb, M, K, N): the affinity model's per-graph products, several masked and
# unmasked steps over 64 tiles, K not a multiple of the group, tiny; the
# panel-pipelined kernel (K within one step; 48-column workgroups at
# 140 x 140 x 312) with 64-row workgroups, K of exactly one step and ragged N
# on 16-column tiles, with rows past M in a partly used workgroup and K inside
# one MFMA chunk, and with 64-row workgroups on 32- and 48-column tiles; the
# staged kernel with odd N (single-word groups along B's rows), K of several
# 48-word steps and a last partial one, rows past M in a 48-row tile
SXS_SHAPES = [(22, 140, 140, 78), (22, 140, 140, 312), (22, 140, 140, 156), (64, 33, 300, 40), (3, 70, 66, 37),
              (5, 100, 148, 64), (2, 5, 63, 3), (1, 1, 1, 1), (2, 200, 144, 68), (3, 37, 20, 100),
              (22, 200, 100, 96), (40, 200, 64, 140), (3, 50, 52, 37), (4, 97, 196, 33)]


PATHS = ("default", "wide", "tiled", "nostaged")  # the contexts of the ctxs fixture, in order


def _check(got, want, path):
    """Bit-exact, naming the GEMM path and the first differing elements."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (path, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, (f"{path}: {bad.size} of {got.size} differ, first at flat index "
                           f"{bad[:8].tolist()}: got {got.ravel()[bad[:4]].tolist()} want {want.ravel()[bad[:4]].tolist()}")


def _mask(bw):
    return np.uint64((1 << bw) - 1) if bw < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)


def _uniform(rng, n, bw):
    return rng.integers(0, np.iinfo(np.uint64).max, size=n, dtype=np.uint64, endpoint=True) & _mask(bw)


def _signed(v, bw):
    v = np.asarray(v, np.uint64) & _mask(bw)
    if bw == 64:
        return v.view(np.int64)
    v = v.astype(np.int64)
    return np.where(v >= 1 << (bw - 1), v - (1 << bw), v)


def _ctx_with(bw, var, val):
    """A context created with the environment variable var set to val."""
    import os
    import mpcx
    old = os.environ.get(var)
    os.environ[var] = val
    try:
        return mpcx.Ctx(bw=bw)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old


@pytest.fixture(scope="module", params=[32, 64])
def ctxs(request):
    """(ring width, contexts on the default, wide, tiled-only and unstaged paths)."""
    import mpcx
    bw = request.param
    cs = (mpcx.Ctx(bw=bw), _ctx_with(bw, "MPCX_GEMM", "wide"), _ctx_with(bw, "MPCX_GEMM", "tiled"),
          _ctx_with(bw, "MPCX_SXS_STAGED", "0"))
    yield bw, cs
    for c in cs:
        c.close()


@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_ring_gemm_paths(ctxs, orc, shape):
    bw, cs = ctxs
    M, K, N = shape
    rng = np.random.default_rng(M + 7 * K + 13 * N + bw)
    A = _uniform(rng, M * K, bw).reshape(M, K)
    B = _uniform(rng, K * N, bw).reshape(K, N)
    want = orc.ring_gemm(bw, A, B)
    for path, c in zip(PATHS, cs):
        _check(c.ring_gemm(A, B).astype(np.uint64), want, path)


@pytest.mark.parametrize("shape", SXS_SHAPES)
def test_sxs_paths(ctxs, orc, shape):
    """Beaver products of both parties, reconstructed: the one-launch paths
    (panels, fused SxS) and the tiled pair launch with a separate reconstruction
    give A.B exactly once the oracle dealer's output mask is removed (the GPU
    dealer's mask is that mask)."""
    bw, cs = ctxs
    nb, Mm, K, N = shape
    rng = np.random.default_rng(nb + Mm + K + N + bw)
    A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))  # |A.B| < 2^31 at K = 300
    B = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
    ra, rb = _uniform(rng, A.size, bw), _uniform(rng, B.size, bw)
    want = np.einsum("bmk,bkn->bmn", A, B)
    ah = (A.ravel().astype(np.uint64) + ra) & _mask(bw)
    bh = (B.ravel().astype(np.uint64) + rb) & _mask(bw)
    _, _, orc_rc = orc.sxs_keygen(4, 2, bw, nb, Mm, K, N, ra, rb)
    for path, c in zip(PATHS, cs):
        g0, g1, grc = c.sxs_keygen(nb, Mm, K, N, ra, rb, seed=4, gate=2)
        _check(grc.astype(np.uint64), orc_rc, path + " keygen")
        got = c.sxs_eval(nb, Mm, K, N, g0, g1, ah, bh)
        _check(_signed(got.astype(np.uint64) - orc_rc, bw).reshape(nb, Mm, N), want, path)


@pytest.mark.parametrize("shape", [(5, 140, 140, 312), (3, 200, 100, 100), (2, 37, 20, 52)])
def test_sxs_panel_forms(orc, shape):
    """The three-panel SxS launch (both parties' Beaver products and their sum)
    in every form, on the same products: the unpipelined panel kernel
    (MPCX_PANEL_PF=0) and the pipelined one on 16-, 32- and 48-column
    workgroups (MPCX_PANEL_NT=1..3), each bit-exact against the oracle (the
    staged kernel, which would take these products, switched off)."""
    import os
    import mpcx
    nb, Mm, K, N = shape
    rng = np.random.default_rng(nb * Mm + K + N)
    A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))
    B = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
    ra, rb = _uniform(rng, A.size, 32), _uniform(rng, B.size, 32)
    want = np.einsum("bmk,bkn->bmn", A, B)
    ah = (A.ravel().astype(np.uint64) + ra) & _mask(32)
    bh = (B.ravel().astype(np.uint64) + rb) & _mask(32)
    _, _, orc_rc = orc.sxs_keygen(4, 2, 32, nb, Mm, K, N, ra, rb)
    forms = [("MPCX_PANEL_PF", "0")] + [("MPCX_PANEL_NT", str(t)) for t in (1, 2, 3)]
    for var, val in forms:
        saved = {v: os.environ.get(v) for v in (var, "MPCX_SXS_STAGED")}
        os.environ[var] = val
        os.environ["MPCX_SXS_STAGED"] = "0"
        try:
            c = mpcx.Ctx(bw=32)
        finally:
            for v, o in saved.items():
                if o is None:
                    del os.environ[v]
                else:
                    os.environ[v] = o
        try:
            g0, g1, _ = c.sxs_keygen(nb, Mm, K, N, ra, rb, seed=4, gate=2)
            got = c.sxs_eval(nb, Mm, K, N, g0, g1, ah, bh)
            _check(_signed(got.astype(np.uint64) - orc_rc, 32).reshape(nb, Mm, N), want, f"{var}={val}")
        finally:
            c.close()
