"""Ring GEMM kernel paths against the oracle, both rings.

The default path takes the wide-K matrix-core kernel wherever it applies
(enough tiles for a quarter of the CUs, or K within one step) and the tiled
matrix-core kernels elsewhere (long K over few tiles, split-K);
MPCX_GEMM=tiled forces the tiled kernels everywhere.  The shapes below make
the wide kernel take every branch: one and several K steps, steps with masks
(half as wide), party 1's two K segments, rows read as 16-byte groups or
word by word (K not a multiple of the group), ragged M and N; the SxS
products also take the fused evaluation of both parties with the
reconstruction in the same launch.  Every result is checked bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (M, K, N): single step (K <= 288 words of Z_2^32, 144 of Z_2^64), several
# steps with 64+ tiles, K not a multiple of the 16-byte group, tiny
GEMM_SHAPES = [(3080, 78, 78), (3080, 156, 312), (140, 140, 312), (130, 77, 65), (600, 700, 300), (64, 63, 1),
               (1, 1, 1), (22, 256, 1024)]
# (nb, M, K, N): the affinity model's per-graph products, several masked and
# unmasked steps over 64 tiles, K not a multiple of the group, tiny
SXS_SHAPES = [(22, 140, 140, 78), (22, 140, 140, 312), (64, 33, 300, 40), (3, 70, 66, 37), (2, 5, 63, 3),
              (1, 1, 1, 1)]


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


@pytest.fixture(scope="module", params=[32, 64])
def ctxs(request):
    """(default-path context, tiled-only context) of one ring width."""
    import os
    import mpcx
    bw = request.param
    old = os.environ.get("MPCX_GEMM")
    auto = mpcx.Ctx(bw=bw)
    os.environ["MPCX_GEMM"] = "tiled"
    try:
        tiled = mpcx.Ctx(bw=bw)
    finally:
        if old is None:
            del os.environ["MPCX_GEMM"]
        else:
            os.environ["MPCX_GEMM"] = old
    yield bw, auto, tiled
    auto.close()
    tiled.close()


@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_ring_gemm_paths(ctxs, orc, shape):
    bw, auto, tiled = ctxs
    M, K, N = shape
    rng = np.random.default_rng(M + 7 * K + 13 * N + bw)
    A = _uniform(rng, M * K, bw).reshape(M, K)
    B = _uniform(rng, K * N, bw).reshape(K, N)
    want = orc.ring_gemm(bw, A, B)
    assert np.array_equal(auto.ring_gemm(A, B).astype(np.uint64), want)
    assert np.array_equal(tiled.ring_gemm(A, B).astype(np.uint64), want)


@pytest.mark.parametrize("shape", SXS_SHAPES)
def test_sxs_paths(ctxs, orc, shape):
    """Beaver products of both parties, reconstructed: the fused launch (default)
    and the tiled pair launch with a separate reconstruction give A.B exactly
    once the oracle dealer's output mask is removed (the GPU dealer's mask is
    that mask)."""
    bw, auto, tiled = ctxs
    nb, Mm, K, N = shape
    rng = np.random.default_rng(nb + Mm + K + N + bw)
    A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))  # |A.B| < 2^31 at K = 300
    B = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
    ra, rb = _uniform(rng, A.size, bw), _uniform(rng, B.size, bw)
    want = np.einsum("bmk,bkn->bmn", A, B)
    ah = (A.ravel().astype(np.uint64) + ra) & _mask(bw)
    bh = (B.ravel().astype(np.uint64) + rb) & _mask(bw)
    _, _, orc_rc = orc.sxs_keygen(4, 2, bw, nb, Mm, K, N, ra, rb)
    for c in (auto, tiled):
        g0, g1, grc = c.sxs_keygen(nb, Mm, K, N, ra, rb, seed=4, gate=2)
        assert np.array_equal(grc.astype(np.uint64), orc_rc)
        got = c.sxs_eval(nb, Mm, K, N, g0, g1, ah, bh)
        assert np.array_equal(_signed(got.astype(np.uint64) - orc_rc, bw).reshape(nb, Mm, N), want)
