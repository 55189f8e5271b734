"""Parity of the HIP path (libmpcx through its C ABI) with the CPU oracle.

For every primitive and gate: the GPU dealer must write byte-identical keys to
the oracle's dealer, the GPU evaluation must reconstruct the same masked
outputs as the oracle's evaluation, and the unmasked outputs must equal the
plaintext function.  Integer work: bit-exact, no tolerance.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

S = 12


@pytest.fixture(scope="module")
def mp():
    import mpcx
    return mpcx


@pytest.fixture(scope="module", params=[32, 64])
def ctx(request, mp):
    c = mp.Ctx(bw=request.param, scale=S)
    yield c
    c.close()


def M(bw):
    return np.uint64((1 << bw) - 1 if bw < 64 else 0xFFFFFFFFFFFFFFFF)


def signed(v, bw):
    v = np.asarray(v, np.uint64) & M(bw)
    if bw == 64:
        return v.view(np.int64)
    v = v.astype(np.int64)
    return np.where(v >= 1 << (bw - 1), v - (1 << bw), v)


def rmask(rng, n, bw):
    return rng.integers(0, np.iinfo(np.uint64).max, size=n, dtype=np.uint64, endpoint=True) & M(bw)


def host(t):
    import mpcx
    return mpcx.from_dev(t, np.uint8)


# ---------------------------------------------------------------------------
def test_prg_hash_matches_oracle(mp, orc):
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(0)
    blocks = rng.integers(0, 2**32, size=(4099, 4), dtype=np.uint64).astype(np.uint32)
    for leaf in (False, True):
        assert np.array_equal(c.prg_hash(blocks, leaf), orc.hash_blocks(blocks, leaf))
    assert np.array_equal(c.prf(77, 5, 0x30, 1000), orc.prf_blocks(77, 5, 0x30, 1000))
    c.close()


@pytest.mark.parametrize("m", [5, 8, 12, 31, 63])
def test_dcf_keys_and_eval(mp, orc, m):
    c = mp.Ctx(bw=64 if m > 31 else 32)
    rng = np.random.default_rng(m)
    n = 3001
    top = (1 << m) - 1
    alpha = rng.integers(0, top, size=n, dtype=np.uint64, endpoint=True)
    alpha[:4] = [0, top, 1, top - 1]
    rb = rng.integers(0, 2, size=n).astype(np.uint8)
    g0, g1 = c.dcf_keygen(m, alpha, rb, seed=31, gate=9)
    o0, o1 = orc.dcf_keygen(31, 9, m, alpha, rbit=rb)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    x = rng.integers(0, top, size=n, dtype=np.uint64, endpoint=True)
    x[:8] = [0, top, alpha[2], alpha[3], alpha[4], alpha[4] - 1 if alpha[4] else 0, top, 0]
    b = c.dcf_eval(0, m, g0, x) ^ c.dcf_eval(1, m, g1, x)
    assert np.array_equal(b, (x < alpha).astype(np.uint8) ^ rb)
    assert np.array_equal(c.dcf_eval(0, m, g0, x), orc.dcf_eval(0, m, o0, x))
    c.close()


@pytest.mark.parametrize("bw,m", [(32, 5), (32, 12), (32, 31), (64, 20), (64, 63)])
def test_dcf_eval_ring_inputs_and_mask(mp, orc, bw, m):
    """mpcx_dcf_eval_ring (the reference's gpuDcf with maskEpilogue,
    gpu_mpc/dpf_dcf_adapter.h:266, 293): ring elements read modulo 2^m (their
    upper bits set at random change nothing), the output bits XORed with a mask
    of 32-bit words; equal to mpcx_dcf_eval on the reduced inputs."""
    c = mp.Ctx(bw=bw)
    rng = np.random.default_rng(bw + m)
    n = 3001  # odd number of 32-bit mask words: the last one partly used
    top = (1 << m) - 1
    alpha = rng.integers(0, top, size=n, dtype=np.uint64, endpoint=True)
    g0, g1 = c.dcf_keygen(m, alpha, None, seed=5, gate=2)
    x = rng.integers(0, top, size=n, dtype=np.uint64, endpoint=True)
    x_ring = x | (rng.integers(0, 1 << (bw - m), size=n, dtype=np.uint64) << np.uint64(m))  # garbage above bit m
    mask = rng.integers(0, 1 << 32, size=(n + 31) // 32, dtype=np.uint64).astype(np.uint32)
    mbits = np.unpackbits(mask.view(np.uint8), bitorder="little")[:n]
    for p, g in ((0, g0), (1, g1)):
        want = c.dcf_eval(p, m, g, x)
        assert np.array_equal(c.dcf_eval_ring(p, m, g, x_ring), want)
        assert np.array_equal(c.dcf_eval_ring(p, m, g, x_ring, mask), want ^ mbits)
    b = c.dcf_eval_ring(0, m, g0, x_ring, mask) ^ c.dcf_eval_ring(1, m, g1, x_ring)
    assert np.array_equal(b, (x < alpha).astype(np.uint8) ^ mbits)
    c.close()


def test_dcf_exhaustive_small_domain(mp):
    c = mp.Ctx(bw=32)
    m, N = 10, 1024
    x = np.arange(N, dtype=np.uint64)
    for alpha in (0, 1, 511, 512, 1023, 777):
        g0, g1 = c.dcf_keygen(m, np.full(N, alpha, np.uint64), None, seed=alpha, gate=1)
        b = c.dcf_eval(0, m, g0, x) ^ c.dcf_eval(1, m, g1, x)
        assert np.array_equal(b, (x < alpha).astype(np.uint8)), alpha
    c.close()


def _tr_inputs(rng, kind, bw, n=4000):
    h = 1 << (bw - 1)
    q = 1 << (bw - 2)
    edge = [-h, -h + 1, -1, 0, 1, h - 1, (1 << S) - 1, 1 << S, -(1 << S), -(1 << S) - 1]
    if kind == 4:
        x = np.concatenate([np.array([-q, -1, 0, 1, q - 1], np.int64), rng.integers(-q, q, size=n, dtype=np.int64)])
        return x, None
    if kind in (9, 15):
        qs = 1 << (bw - 2 - S if kind == 9 else bw - S)
        x = np.concatenate([np.array([-qs, -1, 0, 1, qs - 1], np.int64), rng.integers(-qs, qs, size=n, dtype=np.int64)])
        return x, None
    x = np.concatenate([np.array(edge, np.int64), rng.integers(-(h // 4), h // 4, size=n // 2, dtype=np.int64),
                        rng.integers(-8 << S, 8 << S, size=n // 2)])
    bias = None
    if kind in (1, 2):
        bias = rng.integers(-(1 << 14), 1 << 14, size=37)
        lim = h - (1 << (14 + S)) - 1
        x = np.clip(x, -lim, lim)
    return x, bias


def _tr_expected(kind, x, bias):
    if kind in (1, 2):
        bb = np.resize(bias, x.size)
        t = (x + (bb << S)) >> S
        return t if kind == 1 else np.maximum(t, 0)
    if kind in (3, 9, 15):
        return np.maximum(x, 0)
    return x >> S


@pytest.mark.parametrize("kind", [1, 2, 3, 4, 9, 15])
def test_tr_family_keys_and_eval(ctx, orc, kind):
    bw = ctx.bw
    rng = np.random.default_rng(kind * 100 + bw)
    x, bias = _tr_inputs(rng, kind, bw)
    rin = rmask(rng, x.size, bw)
    g0, g1, grout = ctx.tr_keygen(kind, rin, seed=5, gate=17)
    o0, o1, orout = orc.tr_keygen(5, 17, kind, bw, S, rin)
    assert np.array_equal(grout.astype(np.uint64), orout)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    ctx.reset_counters()
    y = ctx.tr_eval(kind, g0, g1, xhat, bias)
    by = ctx.bytes_exchanged
    be = None if bias is None else np.resize(bias, x.size)
    oy, oby = orc.tr_eval(kind, bw, S, o0, o1, xhat, be)
    assert np.array_equal(y.astype(np.uint64), oy)
    assert by == oby
    assert np.array_equal(signed(y.astype(np.uint64) - orout, bw), _tr_expected(kind, x, bias))


@pytest.mark.parametrize("relu", [False, True])
def test_split_truncation_keys_and_eval(ctx, orc, relu):
    """The exact truncation as two gates, TRMOD (truncate-reduce, s-bit DCF) then
    EXT / EXTRELU (sign extension, (bw-s-1)-bit DCF; gpu_mpc/dpf_dcf_adapter.h:
    225-234, 274-303): both gates' keys byte-identical to the oracle's, each
    revealed value and the exchanged bytes identical, and the unmasked result the
    signed floor (+ bias), and its ReLU, over the whole ring."""
    bw = ctx.bw
    rng = np.random.default_rng(bw * 7 + relu)
    x, bias = _tr_inputs(rng, 1, bw)
    rin = rmask(rng, x.size, bw)
    kind = 14 if relu else 13
    g0, g1, gr1 = ctx.tr_keygen(12, rin, seed=6, gate=30)
    q0, q1, gr2 = ctx.tr_keygen(kind, gr1, seed=6, gate=31)
    o0, o1, or1 = orc.tr_keygen(6, 30, 12, bw, S, rin)
    p0, p1, or2 = orc.tr_keygen(6, 31, kind, bw, S, or1)
    assert np.array_equal(gr1.astype(np.uint64), or1) and np.array_equal(gr2.astype(np.uint64), or2)
    for g, o in ((g0, o0), (g1, o1), (q0, p0), (q1, p1)):
        assert np.array_equal(host(g)[:o.size], o)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    ctx.reset_counters()
    y1 = ctx.tr_eval(12, g0, g1, xhat, bias)
    y2 = ctx.tr_eval(kind, q0, q1, y1)
    by = ctx.bytes_exchanged
    be = np.resize(bias, x.size)
    oy1, b1 = orc.tr_eval(12, bw, S, o0, o1, xhat, be)
    oy2, b2 = orc.tr_eval(kind, bw, S, p0, p1, oy1)
    assert np.array_equal(y1.astype(np.uint64), oy1) and np.array_equal(y2.astype(np.uint64), oy2)
    assert by == b1 + b2
    assert np.array_equal(signed(y2.astype(np.uint64) - or2, bw), _tr_expected(2 if relu else 1, x, bias))


def _num_cu():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("form", ["auto", "block512"])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 255, 256, 257, 511, 513, 1023, 1025, "quad", "quad+1", 40000])
def test_gate_tile_edges(ctx, mp, orc, n, form):
    """One gate launch takes tiles of elements, both parties' threads per tile:
    element counts around the wave and tile sizes give the oracle's outputs
    (EXTRELU after TRMOD, so both DCF widths and both exchanges run).  "auto"
    takes the default forms -- up to 64 elements per CU ("quad": 64 times the
    device's CU count) the quad-lane kernel with 32-element tiles, above it
    ("quad+1") about one workgroup per CU -- and "block512" pins the variant's
    512-thread workgroups (256-element tiles, one lane per element); the form
    each case runs is asserted."""
    if form == "block512":
        ctx = mp.Ctx(bw=ctx.bw)
        ctx.set_aes_variant(0, 512)
    quad_max = 64 * _num_cu()
    n = quad_max if n == "quad" else quad_max + 1 if n == "quad+1" else n
    if form == "block512":
        assert ctx.tr_eval_form(12, n) == ctx.tr_eval_form(14, n) == 0
    elif n <= quad_max:
        assert ctx.tr_eval_form(12, n) == ctx.tr_eval_form(14, n) == 2
    else:
        assert ctx.tr_eval_form(14, n) == 0
    bw = ctx.bw
    rng = np.random.default_rng(n + bw)
    h = 1 << (bw - 1)
    x = rng.integers(-(h // 2), h // 2, size=n, dtype=np.int64)
    rin = rmask(rng, n, bw)
    o0, o1, r1 = orc.tr_keygen(3, 40, 12, bw, S, rin)
    p0, p1, r2 = orc.tr_keygen(3, 41, 14, bw, S, r1)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    y1 = ctx.tr_eval(12, mp.to_dev(o0), mp.to_dev(o1), xhat)
    y2 = ctx.tr_eval(14, mp.to_dev(p0), mp.to_dev(p1), y1)
    oy1, _ = orc.tr_eval(12, bw, S, o0, o1, xhat)
    oy2, _ = orc.tr_eval(14, bw, S, p0, p1, oy1)
    assert np.array_equal(y1.astype(np.uint64), oy1) and np.array_equal(y2.astype(np.uint64), oy2)
    assert np.array_equal(signed(y2.astype(np.uint64) - r2, bw), np.maximum(x >> S, 0))
    if form == "block512":
        ctx.close()


@pytest.mark.parametrize("kind,size", [(4, "ragged"), (9, "ragged"), (15, "ragged"), (13, "ragged"), (14, "whole"),
                                       (14, "ragged")])
def test_gate_both_party_form(ctx, mp, orc, kind, size):
    """At bw=32 a launch of at least 1024 elements per CU ("whole": 1024 times the
    device's CU count) of a gate of at most mpcx_set_both_party_aes AES calls per
    element and party (set to 14 here: TRSLACK, RELUSLACK, RELUPOOL, TRMOD, EXT,
    EXTRELU) runs the both-party form: one thread per element holds both
    parties' keys, runs the two DCF walks side by side and adds the two
    messages.  Outputs identical to the oracle's, on one whole grid pass and on
    a count past it ("ragged": a partial second pass), and the unmasked result
    as the plaintext gate gives it (bw=64 runs the same cases on the one-lane
    kernel); the form is asserted."""
    n = 1024 * _num_cu() + (37751 if size == "ragged" else 0)
    c = mp.Ctx(bw=ctx.bw)
    try:
        c.set_both_party_aes(14)
        for k in ((12, kind) if kind in (13, 14) else (kind,)):
            assert c.tr_eval_form(k, n) == (1 if ctx.bw == 32 else 0), k
        _both_party_case(c, mp, orc, kind, n)
    finally:
        c.close()


@pytest.mark.parametrize("kind,variant", [(1, 0), (2, 0), (3, 0), (11, 0), (3, 1), (2, 3)])
def test_gate_both_party_every_kind(ctx, mp, orc, kind, variant):
    """The both-party form for the longest gates, with mpcx_set_both_party_aes(64)
    (every gate qualifies): TR and TRRELU (both DCF planes in one thread), the
    full-width RELU, DRELU (party 0's message carries the public bit), on the
    default T0/T1 table and on the other AES table layouts (variants 1 and 3,
    whose both-party walks hash the two parties' seeds one after the other);
    bit-exact against the oracle at bw=32 (bw=64 runs the one-lane kernel)."""
    n = 1024 * _num_cu() + 4099
    c = mp.Ctx(bw=ctx.bw)
    try:
        c.set_aes_variant(variant)
        c.set_both_party_aes(64)
        assert c.tr_eval_form(kind, n) == (1 if ctx.bw == 32 else 0)
        if kind == 11:
            bw = c.bw
            rng = np.random.default_rng(bw + 11)
            h = 1 << (bw - 1)
            x = np.concatenate([np.array([-h, -1, 0, 1, h - 1], np.int64),
                                rng.integers(-h, h, size=n - 5, dtype=np.int64)])
            rin = rmask(rng, n, bw)
            o0, o1, kap = orc.tr_keygen(7, 53, 11, bw, S, rin)
            xhat = (x.astype(np.uint64) + rin) & M(bw)
            y = c.tr_eval(11, mp.to_dev(o0), mp.to_dev(o1), xhat)
            oy, _ = orc.tr_eval(11, bw, S, o0, o1, xhat)
            assert np.array_equal(y.astype(np.uint64), oy)
            assert np.array_equal((y.astype(np.uint64) ^ kap.astype(np.uint64)) & np.uint64(1),
                                  (x >= 0).astype(np.uint64))
        else:
            _both_party_case(c, mp, orc, kind, n)
    finally:
        c.close()


def _both_party_case(ctx, mp, orc, kind, n):
    bw = ctx.bw
    rng = np.random.default_rng(kind * 31 + n + bw)
    if kind in (13, 14):  # TRMOD, then EXT or EXTRELU on its output
        x = rng.integers(-(1 << (bw - 3)), 1 << (bw - 3), size=n, dtype=np.int64)
        rin = rmask(rng, n, bw)
        o0, o1, r1 = orc.tr_keygen(7, 50, 12, bw, S, rin)
        p0, p1, r2 = orc.tr_keygen(7, 51, kind, bw, S, r1)
        xhat = (x.astype(np.uint64) + rin) & M(bw)
        y1 = ctx.tr_eval(12, mp.to_dev(o0), mp.to_dev(o1), xhat)
        y2 = ctx.tr_eval(kind, mp.to_dev(p0), mp.to_dev(p1), y1)
        oy1, _ = orc.tr_eval(12, bw, S, o0, o1, xhat)
        oy2, _ = orc.tr_eval(kind, bw, S, p0, p1, oy1)
        assert np.array_equal(y1.astype(np.uint64), oy1) and np.array_equal(y2.astype(np.uint64), oy2)
        want = x >> S if kind == 13 else np.maximum(x >> S, 0)
        assert np.array_equal(signed(y2.astype(np.uint64) - r2, bw), want)
        return
    x, bias = _tr_inputs(rng, kind, bw, n=n)
    rin = rmask(rng, x.size, bw)
    o0, o1, orout = orc.tr_keygen(7, 52, kind, bw, S, rin)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    y = ctx.tr_eval(kind, mp.to_dev(o0), mp.to_dev(o1), xhat, bias)
    oy, _ = orc.tr_eval(kind, bw, S, o0, o1, xhat, None if bias is None else np.resize(bias, x.size))
    assert np.array_equal(y.astype(np.uint64), oy)
    assert np.array_equal(signed(y.astype(np.uint64) - orout, bw), _tr_expected(kind, x, bias))


def test_both_party_setting_checked(ctx):
    """mpcx_set_both_party_aes takes 0..64 and refuses other values."""
    for bad in (-1, 65):
        assert ctx.lib.mpcx_set_both_party_aes(ctx.h, bad) != 0
    assert ctx.lib.mpcx_set_both_party_aes(ctx.h, 6) == 0


def test_local_ars_matches_oracle(ctx, orc):
    """LocalARS (TruncateType::LocalARS, ddg_orca_batched.h:180-199): no key and no
    exchange; output mask and outputs identical to the oracle's, whose closed form
    (carry of the low bits, wrap of x + r) is pinned on the CPU."""
    bw = ctx.bw
    rng = np.random.default_rng(bw + 77)
    x = rng.integers(-(1 << (bw - 3)), 1 << (bw - 3), size=50000, dtype=np.int64)
    bias = rng.integers(-(1 << 14), 1 << 14, size=312)
    rin = rmask(rng, x.size, bw)
    assert ctx.lib.mpcx_tr_key_bytes(ctx.h, 10, x.size) == 0
    g0, g1, grout = ctx.tr_keygen(10, rin)
    _, _, orout = orc.tr_keygen(0, 0, 10, bw, S, rin)
    assert np.array_equal(grout.astype(np.uint64), orout)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    ctx.reset_counters()
    y = ctx.tr_eval(10, g0, g1, xhat, bias)
    assert ctx.bytes_exchanged == 0
    oy, oby = orc.tr_eval(10, bw, S, np.zeros(0, np.uint8), np.zeros(0, np.uint8), xhat, np.resize(bias, x.size))
    assert oby == 0
    assert np.array_equal(y.astype(np.uint64), oy)


def test_drelu_keys_and_eval(ctx, orc):
    """DReLU gate: keys byte-identical to the oracle's, masked bits and exchange
    bytes identical, masked bit XOR mask bit = [x >= 0] (ring edges included)."""
    bw = ctx.bw
    rng = np.random.default_rng(bw + 12)
    h = 1 << (bw - 1)
    x = np.concatenate([np.array([-h, -h + 1, -1, 0, 1, h - 1], np.int64),
                        rng.integers(-h, h, size=20000, dtype=np.int64)])
    rin = rmask(rng, x.size, bw)
    g0, g1, grbit = ctx.tr_keygen(11, rin, seed=4, gate=9)
    o0, o1, orbit = orc.tr_keygen(4, 9, 11, bw, S, rin)
    assert ctx.lib.mpcx_tr_key_bytes(ctx.h, 11, x.size) == o0.size
    assert np.array_equal(grbit.astype(np.uint64), orbit)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    ctx.reset_counters()
    y = ctx.tr_eval(11, g0, g1, xhat)
    oy, oby = orc.tr_eval(11, bw, S, o0, o1, xhat)
    assert ctx.bytes_exchanged == oby
    assert np.array_equal(y.astype(np.uint64), oy)
    assert np.array_equal(y.astype(np.uint64) ^ orbit, (x >= 0).astype(np.uint64))


def test_empty_inputs_are_no_ops(ctx):
    """Every gate entry point over zero elements returns MPCX_OK without reading
    its (null) pointers or counting an exchange; bad kinds are still refused."""
    lib, h, N = ctx.lib, ctx.h, None
    ctx.reset_counters()
    for kind in (1, 2, 3, 4, 9, 10, 11, 12, 13, 14, 15):
        assert ctx.lib.mpcx_tr_key_bytes(h, kind, 0) == 0
        assert lib.mpcx_tr_keygen(h, kind, 0, N, N, 1, 1, N, N) == 0
        assert lib.mpcx_tr_eval(h, kind, 0, N, N, N, N, 0, N) == 0
    assert lib.mpcx_tr_eval(h, 99, 0, N, N, N, N, 0, N) != 0
    assert lib.mpcx_dcf_keygen(h, 31, 0, N, N, 1, 1, N, N) == 0
    assert lib.mpcx_dcf_eval(h, 0, 31, 0, N, N, N) == 0
    assert lib.mpcx_mul_keygen(h, 0, 0, 0, N, N, N, N, N, 1, 1, N, N) == 0
    assert lib.mpcx_mul_eval(h, 0, 0, 0, N, N, N, N, N, N, N) == 0
    assert lib.mpcx_lut8_keygen(h, 0, N, N, 1, 1, N, N) == 0
    assert lib.mpcx_lut8_eval(h, 0, N, N, N, N, N) == 0
    assert lib.mpcx_reveal_keygen(h, 0, N, 1, 1, N, N) == 0
    assert lib.mpcx_reveal_eval(h, 0, N, N, N, N, N) == 0
    assert lib.mpcx_prg_hash(h, 0, 0, N, N) == 0
    assert lib.mpcx_prf(h, 1, 1, 1, 0, N) == 0
    assert lib.mpcx_ring_lincomb(h, 0, 5, 1, N, 0, N, N, 0, N) == 0
    assert ctx.bytes_exchanged == 0 and ctx.lib.mpcx_rounds(h) == 0
    # matrix shapes must be non-empty
    assert lib.mpcx_maxpool_eval(h, 0, 3, 3, N, N, N, N) != 0
    assert lib.mpcx_ring_gemm(h, 0, 3, 3, N, N, N) != 0


def test_all_aes_variants_agree(mp, orc):
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(4)
    x, bias = _tr_inputs(rng, 2, 32, n=3000)
    rin = rmask(rng, x.size, 32)
    o0, o1, orout = orc.tr_keygen(8, 2, 2, 32, S, rin)
    k0, k1 = mp.to_dev(o0), mp.to_dev(o1)
    xhat = (x.astype(np.uint64) + rin) & M(32)
    want = _tr_expected(2, x, bias)
    nvar = c.lib.mpcx_aes_variant_count()
    for v in range(nvar):
        c.set_aes_variant(v)
        y = c.tr_eval(2, k0, k1, xhat, bias)
        assert np.array_equal(signed(y.astype(np.uint64) - orout, 32), want), v
    # explicit workgroup sizes: the gate kernel splits a workgroup into the two
    # parties' halves of whole waves (tiles of block/2 elements, the last one
    # partial here); other sizes are refused when set
    for block in (128, 256, 384, 1024):
        c.set_aes_variant(0, block)
        y = c.tr_eval(2, k0, k1, xhat, bias)
        assert np.array_equal(signed(y.astype(np.uint64) - orout, 32), want), block
    for block in (64, 192, 2048):
        assert c.lib.mpcx_set_aes_variant(c.h, 0, block) != 0
    c.set_aes_variant(0)
    c.close()


def test_mul_keys_and_eval(ctx, orc):
    bw = ctx.bw
    rng = np.random.default_rng(bw)
    nx, ny, nz = 300, 200, 5000
    lim = 1 << (14 if bw == 32 else 30)
    xv = rng.integers(-lim, lim, size=nx)
    yv = rng.integers(-lim, lim, size=ny)
    ia = rng.integers(0, nx, size=nz).astype(np.uint32)
    ib = rng.integers(0, ny, size=nz).astype(np.uint32)
    rx, ry = rmask(rng, nx, bw), rmask(rng, ny, bw)
    g0, g1, grz = ctx.mul_keygen(rx, ry, ia, ib, seed=2, gate=4)
    o0, o1, orz = orc.mul_keygen(2, 4, bw, rx, ry, ia, ib)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    xh = (xv.astype(np.uint64) + rx) & M(bw)
    yh = (yv.astype(np.uint64) + ry) & M(bw)
    z = ctx.mul_eval(g0, g1, xh, yh, ia, ib)
    assert np.array_equal(signed(z.astype(np.uint64) - orz, bw), xv[ia] * yv[ib])


def test_mul_and_reveal_in_place(ctx, orc, mp):
    """Through the C ABI, outputs that overlap an input (the product over its own
    x^ buffer, the reveal over party 0's share) give the same values: the C-ABI
    calls always take the message path (messages, then the reconstruction), so
    no thread writes an output while others still gather inputs.  The model's
    own choice between that path and the one-launch evaluation (by whether the
    output overlaps an input) is covered by the model parity tests, whose
    products and reveals write disjoint buffers."""
    bw = ctx.bw
    rng = np.random.default_rng(bw + 5)
    nx, ny, nz = 3000, 200, 2500
    lim = 1 << (14 if bw == 32 else 30)
    xv = rng.integers(-lim, lim, size=nx)
    yv = rng.integers(-lim, lim, size=ny)
    ia = rng.integers(0, nx, size=nz).astype(np.uint32)
    ib = rng.integers(0, ny, size=nz).astype(np.uint32)
    rx, ry = rmask(rng, nx, bw), rmask(rng, ny, bw)
    g0, g1, grz = ctx.mul_keygen(rx, ry, ia, ib, seed=3, gate=5)
    xh = (xv.astype(np.uint64) + rx) & M(bw)
    yh = (yv.astype(np.uint64) + ry) & M(bw)
    want = ctx.mul_eval(g0, g1, xh, yh, ia, ib)
    d = [mp.to_dev(v) for v in (ia, ib)]
    dx, dy = mp.to_dev(ctx.ring(xh)), mp.to_dev(ctx.ring(yh))
    ctx.check(ctx.lib.mpcx_mul_eval(ctx.h, nx, ny, nz, mp.dptr(d[0]), mp.dptr(d[1]), mp.dptr(g0), mp.dptr(g1),
                                    mp.dptr(dx), mp.dptr(dy), mp.dptr(dx)), "mul_eval")
    got = mp.from_dev(dx, ctx.T, nz)
    assert np.array_equal(got, want)
    assert np.array_equal(signed(got.astype(np.uint64) - grz, bw), xv[ia] * yv[ib])
    n = 777
    r0, r1, rm = ctx.reveal_keygen(n, seed=4, gate=6)
    v = rng.integers(-1000, 1000, size=n)
    v0 = rmask(rng, n, bw)
    v1 = (v.astype(np.uint64) - v0) & M(bw)
    d0, d1 = mp.to_dev(ctx.ring(v0)), mp.to_dev(ctx.ring(v1))
    ctx.check(ctx.lib.mpcx_reveal_eval(ctx.h, n, mp.dptr(r0), mp.dptr(r1), mp.dptr(d0), mp.dptr(d1), mp.dptr(d0)),
              "reveal_eval")
    assert np.array_equal(signed(mp.from_dev(d0, ctx.T, n).astype(np.uint64) - rm, bw), v)


def test_lut8_keys_and_eval(ctx, orc):
    bw = ctx.bw
    rng = np.random.default_rng(9)
    table = orc.invsqrt_table(S, 138)
    x = np.tile(np.arange(256, dtype=np.uint64), 4)
    rin = rmask(rng, x.size, bw)
    g0, g1, grout = ctx.lut8_keygen(rin, seed=4, gate=6)
    o0, o1, orout = orc.lut8_keygen(4, 6, bw, rin)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    y = ctx.lut8_eval(g0, g1, table, (x + rin) & M(bw))
    assert np.array_equal((y.astype(np.uint64) - orout) & M(bw), table[x.astype(np.int64)])


SXS_SHAPES = [(3, 70, 66, 37), (1, 3, 1000, 70), (2, 140, 140, 312), (1, 1, 1, 1), (4, 17, 63, 5)]


@pytest.mark.parametrize("shape", SXS_SHAPES)
def test_sxs_keys_and_eval(ctx, orc, shape):
    """Batched Beaver products: both parties' GEMMs in one launch (party 1 over
    the concatenated K of its two products), split-K shapes included."""
    bw = ctx.bw
    nb, Mm, K, N = shape
    rng = np.random.default_rng(12 + K)
    A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))
    B = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
    ra, rb = rmask(rng, A.size, bw), rmask(rng, B.size, bw)
    g0, g1, grc = ctx.sxs_keygen(nb, Mm, K, N, ra, rb, seed=3, gate=2)
    o0, o1, orc_ = orc.sxs_keygen(3, 2, bw, nb, Mm, K, N, ra, rb)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    ah = (A.ravel().astype(np.uint64) + ra) & M(bw)
    bh = (B.ravel().astype(np.uint64) + rb) & M(bw)
    c = ctx.sxs_eval(nb, Mm, K, N, g0, g1, ah, bh)
    assert np.array_equal(signed(c.astype(np.uint64) - orc_, bw).reshape(nb, Mm, N), np.einsum("bmk,bkn->bmn", A, B))


GEMM_SHAPES = [(130, 77, 65), (64, 1024, 128), (64, 512, 1), (3, 1000, 70), (64, 312, 1024), (1, 1, 1),
               (17, 63, 5), (200, 64, 64), (140, 140, 312)]


@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_ring_gemm(ctx, orc, shape):
    """Square-ish and skinny (FC-layer, split-K with atomic accumulation)
    products mod 2^bw against the oracle's exact ring GEMM, uniform operands
    (every balanced digit value occurs)."""
    bw = ctx.bw
    M, K, N = shape
    rng = np.random.default_rng(M * K + N)
    A = rmask(rng, M * K, bw).reshape(M, K)
    B = rmask(rng, K * N, bw).reshape(K, N)
    assert np.array_equal(ctx.ring_gemm(A, B).astype(np.uint64), orc.ring_gemm(bw, A, B))


@pytest.mark.parametrize("K", [32767, 40000])
def test_ring_gemm64_digit_sum_bound(mp, orc, K):
    """Z_2^64 on the matrix cores keeps the low shifts' int32 digit sums exact
    for K < 2^15: a 1024 x 1024 product (256 tiles: no split-K, the whole K in
    one accumulator) at K = 2^15 - 1 with every digit at -128 (the largest
    sums) equals K a^2 mod 2^64 everywhere; K = 40000 runs on the VALU kernel.
    Uniform operands at both K against the oracle."""
    c = mp.Ctx(bw=64)
    a = 0x8080808080808080
    worst = np.full((1024, K), a, np.uint64)
    got = c.ring_gemm(worst, worst.T.copy()).astype(np.uint64)
    assert np.all(got == np.uint64((K * a * a) % (1 << 64)))
    del worst, got
    rng = np.random.default_rng(K)
    A = rmask(rng, 3 * K, 64).reshape(3, K)
    B = rmask(rng, K * 2, 64).reshape(K, 2)
    assert np.array_equal(c.ring_gemm(A, B).astype(np.uint64), orc.ring_gemm(64, A, B))
    c.close()


def test_ring_gemm_valu_path(mp, orc, monkeypatch):
    """Z_2^32 products on the VALU path (MPCX_GEMM=valu; the default is the
    int8 matrix-core path) agree with the oracle too."""
    monkeypatch.setenv("MPCX_GEMM", "valu")
    c = mp.Ctx(bw=32)
    for M, K, N in [(130, 77, 65), (64, 512, 1), (140, 140, 312)]:
        rng = np.random.default_rng(M + K + N)
        A = rmask(rng, M * K, 32).reshape(M, K)
        B = rmask(rng, K * N, 32).reshape(K, N)
        assert np.array_equal(c.ring_gemm(A, B).astype(np.uint64), orc.ring_gemm(32, A, B))
    c.close()


def test_sxs_valu_path(mp, orc, monkeypatch):
    """The same Beaver products on the VALU GEMM path (two launches for party 1)."""
    monkeypatch.setenv("MPCX_GEMM", "valu")
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(5)
    for nb, Mm, K, N in [(2, 70, 66, 37), (1, 3, 1000, 70)]:
        A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))
        B = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
        ra, rb = rmask(rng, A.size, 32), rmask(rng, B.size, 32)
        g0, g1, grc = c.sxs_keygen(nb, Mm, K, N, ra, rb, seed=3, gate=2)
        _, _, orc_ = orc.sxs_keygen(3, 2, 32, nb, Mm, K, N, ra, rb)
        ah = (A.ravel().astype(np.uint64) + ra) & M(32)
        bh = (B.ravel().astype(np.uint64) + rb) & M(32)
        got = c.sxs_eval(nb, Mm, K, N, g0, g1, ah, bh)
        assert np.array_equal(signed(got.astype(np.uint64) - orc_, 32).reshape(nb, Mm, N),
                              np.einsum("bmk,bkn->bmn", A, B))
    c.close()


def test_reveal_keys_and_eval(ctx, orc):
    bw = ctx.bw
    rng = np.random.default_rng(2)
    n = 1001
    g0, g1, gm = ctx.reveal_keygen(n, seed=1, gate=3)
    o0, o1, om = orc.reveal_keygen(1, 3, bw, n)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(gm.astype(np.uint64), om)
    v = rng.integers(-1000, 1000, size=n)
    v0 = rmask(rng, n, bw)
    v1 = (v.astype(np.uint64) - v0) & M(bw)
    vh = ctx.reveal_eval(g0, g1, v0, v1)
    assert np.array_equal(signed(vh.astype(np.uint64) - om, bw), v)


# ---------------------------------------------------------------------------
def _od(orc, dims):
    return orc.make_dims(bw=dims.bw, s=dims.s, n_nodes=dims.n_nodes, feat=dims.feat, gcn=dims.gcn, dfc=dims.dfc,
                         prot=dims.prot, fus=dims.fus, lut_nmax=dims.lut_nmax, mask_scale=dims.mask_scale,
                         slack=dims.slack)


@pytest.mark.parametrize("bw,slack,ms", [(32, 0, 0), (64, 0, 0), (32, 1, 0), (64, 1, 0), (32, 2, 0), (64, 2, 0),
                                         (32, 0, 12), (32, 0, 25), (64, 0, 55)])
def test_model_keys_and_forward(mp, orc, synth, bw, slack, ms):
    """GPU dealer keys byte-identical to the oracle's, forward bit-exact, same
    exchange bytes; exact, and with the slack truncations of the GCN.  Atom masks
    at scale ms: 12 (the reference's share files) keeps the max-pool's narrow
    sentinel and RELUPOOL gates, 25 (bw=32) and 55 (bw=64) exceed bw-s-1 and take
    the reference's sentinel with full RELU gates."""
    B = 2
    wl = synth.workload(B, synth.Dims(bw=bw, slack=slack, mask_scale=ms), seed=21)
    d = _od(orc, wl.dims)
    mask = wl.mask << ms
    want, code = orc.plain_forward(d, wl.X, wl.A, mask, wl.prot, wl.W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W)
    assert m.key_bytes(B) == orc.model_key_bytes(d, B)
    m.keygen(B, 777)
    o0, o1 = orc.model_keygen(d, B, 777, wl.W)
    assert np.array_equal(m.export_keys(0, B), o0)
    assert np.array_equal(m.export_keys(1, B), o1)
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = synth.share(mask, bw, 5) if ms else wl.shares["m"]
    m.set_inputs(B, x0, x1, a0, a1, m0, m1, wl.prot)
    c.reset_counters()
    m.forward(B)
    got = m.output(B)
    assert np.array_equal(got, want)
    _, oby = orc.model_eval(d, B, wl.W, o0, o1, x0, x1, a0, a1, m0, m1, wl.prot)
    assert c.bytes_exchanged == oby
    m.close()
    c.close()


@pytest.mark.parametrize("bw", [32, 64])
def test_model_local_truncation(mp, orc, synth, bw):
    """slack 3 (every layer truncation LocalARS, the reference's default): GPU
    dealer keys byte-identical to the oracle's, outputs and exchange bytes
    identical to the oracle's two-party evaluation on those keys (not to the
    fixed-point forward: LocalARS is not exact)."""
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw, slack=3), seed=22)
    d = _od(orc, wl.dims)
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W)
    assert m.key_bytes(B) == orc.model_key_bytes(d, B)
    m.keygen(B, 778)
    o0, o1 = orc.model_keygen(d, B, 778, wl.W)
    assert np.array_equal(m.export_keys(0, B), o0)
    assert np.array_equal(m.export_keys(1, B), o1)
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = wl.shares["m"]
    m.set_inputs(B, x0, x1, a0, a1, m0, m1, wl.prot)
    c.reset_counters()
    m.forward(B)
    got = m.output(B)
    want, oby = orc.model_eval(d, B, wl.W, o0, o1, x0, x1, a0, a1, m0, m1, wl.prot)
    assert np.array_equal(got, want)
    assert c.bytes_exchanged == oby
    m.close()
    c.close()


def _tr_gates(dims):
    """DCF gates of one exact forward: the adjacency block's TRSLACK,
    3 x (TRMOD, EXT, TRMOD, EXTRELU), the pool levels, then TRMOD and EXT /
    EXTRELU for the two drug FCs and the hidden fusion layers."""
    R, levels = dims.n_nodes, 0
    while R > 1:
        R, levels = R // 2 + (R & 1), levels + 1
    return 1 + 12 + levels + 2 * (2 + len(dims.fus) - 1)


def _tr_launches(dims, n):
    """DCF-evaluation launches of one exact forward of a lane of n samples with
    resident keys and both parties in one process: a lane of at most 8 samples
    (latency-bound) runs every truncation (TRMOD with its EXT or EXTRELU) as one
    launch, one fewer per truncation than there are gates, and its max-pool
    levels from the third on in one launch; larger lanes pair only the
    truncations of at most 65536 elements (the fully connected layers here)."""
    sizes = [n * dims.n_nodes * f for f in dims.gcn for _ in range(2)]
    sizes += [n * w for w in dims.dfc] + [n * w for w in dims.fus[:-1]]
    assert len(sizes) == 6 + 2 + len(dims.fus) - 1
    R, levels = dims.n_nodes, 0
    while R > 1:
        R, levels = R // 2 + (R & 1), levels + 1
    tail = levels - 2 if n <= 8 and levels - 2 >= 2 else 0  # levels 3.. in one launch
    return _tr_gates(dims) - sum(1 for e in sizes if n <= 8 or e <= 65536) - max(tail - 1, 0)


@pytest.mark.parametrize("bw,B,lanes", [(32, 5, 2), (64, 4, 3), (32, 2, 4), (32, 10, 1), (32, 16, 2)])
def test_model_lanes_keys_and_forward(mp, orc, synth, bw, B, lanes):
    """Concurrent sub-batches: the key arena is the lanes' one-lane key sets
    back to back, each byte-identical to the oracle dealer's under its lane
    seed; each lane's key set evaluates correctly in the oracle; the forward
    gives the plaintext outputs and the lanes' summed exchange bytes; a profiled
    forward (lanes one after another) gives the same outputs and times every
    lane's DCF launches.  B=2 with 4 lanes leaves two lanes empty; a lane of 10
    samples pairs only its small truncations, the smaller lanes pair all (lanes
    of 8 samples pair their GCN-2 and GCN-3 truncations in the both-party
    form)."""
    wl = synth.workload(B, synth.Dims(bw=bw), seed=23)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W, lanes=lanes)
    assert m.lanes == lanes
    split = mp.Model.lane_split(B, lanes)
    assert len(split) == min(B, lanes) and sum(n for _, n in split) == B
    assert m.key_bytes(B) == sum(orc.model_key_bytes(d, n) for _, n in split)
    seed = 901
    m.keygen(B, seed)
    got = [m.export_keys(p, B) for p in (0, 1)]
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = wl.shares["m"]
    o, want_bytes = 0, 0
    for i, (s0, n) in enumerate(split):
        k0, k1 = orc.model_keygen(d, n, mp.Model.lane_seed(seed, i), wl.W)
        assert np.array_equal(got[0][o:o + k0.size], k0)
        assert np.array_equal(got[1][o:o + k1.size], k1)
        o += k0.size
        sl = slice(s0, s0 + n)
        y, by = orc.model_eval(d, n, wl.W, k0, k1, x0[sl], x1[sl], a0[sl], a1[sl], m0[sl], m1[sl], wl.prot[sl])
        assert np.array_equal(y, want[sl])
        want_bytes += by
    assert o == got[0].size
    m.set_inputs(B, x0, x1, a0, a1, m0, m1, wl.prot)
    c.reset_counters()
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    assert c.bytes_exchanged == want_bytes
    m.profile(True)
    m.forward(B)
    prof = m.profile_read()
    m.profile(False)
    assert np.array_equal(m.output(B), want)
    assert prof["launches"] == sum(_tr_launches(wl.dims, n) for _, n in split) and prof["ms"] > 0
    # ring GEMM sections: per lane 3 public GCN products, 3 SxS gates, 2 drug FCs
    # and the fusion layers, with their ring multiply-adds
    dm = wl.dims
    widths = [dm.feat] + list(dm.gcn)
    fc = [(dm.gcn[2], dm.dfc[0]), (dm.dfc[0], dm.dfc[1])]
    fin = dm.dfc[1] + dm.prot
    for w in dm.fus:
        fc.append((fin, w))
        fin = w
    macs = 0
    for _, n in split:
        rows = n * dm.n_nodes
        macs += sum(rows * widths[l] * widths[l + 1] for l in range(3))
        macs += sum(3 * n * dm.n_nodes * dm.n_nodes * f for f in dm.gcn)
        macs += sum(n * a * b for a, b in fc)
    assert prof["gemm_sections"] == (8 + len(dm.fus)) * len(split)
    assert prof["gemm_macs"] == macs and prof["gemm_ms"] > 0
    # lanes back to one: the keys are dropped, a fresh one-lane key set works
    m.set_lanes(1)
    with pytest.raises(mp.MpcxError):
        m.forward(B)
    m.keygen(B, seed)
    m.set_inputs(B, x0, x1, a0, a1, m0, m1, wl.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    m.close()
    c.close()


def test_model_lanes_streamed_keys(mp, orc, synth):
    """Two lanes on host-streamed packed keys (both parties): each lane streams
    its part of the host buffers through its own two slots and expands its
    parties' PRF-drawn planes there."""
    B, bw = 3, 64
    wl = synth.workload(B, synth.Dims(bw=bw), seed=33)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W, lanes=2)
    m.keygen(B, 4321)
    nbytes = m.key_bytes(B)
    h0, hp = mp.PinnedBuffer(m.unique_key_bytes(B, 0)), mp.PinnedBuffer(m.unique_key_bytes(B, 1))
    m.export_unique_keys(0, B, into=h0)
    m.export_unique_keys(1, B, into=hp)
    m.release_arena()
    m.attach_host_keys(B, h0, hp, slot_bytes=nbytes // 6)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    for _ in range(2):
        m.forward(B)
        assert np.array_equal(m.output(B), want)
        st = m.stream_stats()
        # each lane's packed keys start with a 256-byte header that is not copied
        assert st["bytes_h2d"] == h0.nbytes + hp.nbytes - 2 * 2 * 256 and st["chunks"] >= 4
    m.close()
    c.close()
    h0.free()
    hp.free()


def test_model_create_rejects_bad_dims(mp, synth):
    """Model creation checks its dimensions and the weight blob length, and
    the forward refuses to run before keys and inputs are set."""
    import dataclasses
    c = mp.Ctx(bw=32)
    good = synth.Dims(bw=32, n_nodes=8)
    W = np.zeros(sum(i * o + o for i, o in good.layers()), np.int64)
    m = mp.Model(c, good, W)
    with pytest.raises(mp.MpcxError):
        m.forward(2)
    m.close()
    for bad in (dict(n_nodes=256), dict(feat=0), dict(gcn=(8, 0, 8)), dict(fus=(16, 4)),
                dict(mask_scale=30), dict(lut_nmax=300)):
        d = dataclasses.replace(good, **bad)
        Wd = np.zeros(sum(i * o + o for i, o in d.layers()), np.int64)
        with pytest.raises(mp.MpcxError):
            mp.Model(c, d, Wd)
    with pytest.raises(mp.MpcxError):
        mp.Model(c, good, W[:-1])
    c.close()


@pytest.mark.parametrize("bw,lanes", [(32, 1), (64, 2)])
def test_model_extreme_molecule_sizes(mp, orc, synth, bw, lanes):
    """A molecule of one atom (a single real row in the pool tree, all others
    sentinels) next to one that fills all 140 rows (no padding)."""
    dims = synth.Dims(bw=bw)
    X1, A1, m1 = synth.molecules(1, dims, seed=3, min_atoms=1, max_atoms=1)
    X2, A2, m2 = synth.molecules(1, dims, seed=4, min_atoms=140, max_atoms=140)
    X, A, mask = np.concatenate([X1, X2]), np.concatenate([A1, A2]), np.concatenate([m1, m2])
    assert mask[0].sum() == 1 and mask[1].sum() == 140
    W = synth.weights(dims, seed=5)
    prot = synth.protein(2, dims, seed=6)
    d = _od(orc, dims)
    want, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, dims, W, lanes=lanes)
    m.keygen(2, 77)
    sh = [synth.share(v, bw, 20 + k) for k, v in enumerate((X, A, mask))]
    m.set_inputs(2, *sh[0], *sh[1], *sh[2], prot)
    m.forward(2)
    assert np.array_equal(m.output(2), want)
    m.close()
    c.close()


@pytest.mark.parametrize("bw", [32, 64])
def test_model_alone_lane_quad_gates(mp, orc, synth, monkeypatch, bw):
    """A lane that runs alone (one active lane) evaluates its mid-size gates
    (up to 192 elements per CU: on 256 CUs the GCN-2 and GCN-3 gates of one
    molecule, 85 and 171) in the quad-lane form, on 512-thread workgroups; a
    lane beside another does not.  On one two-lane model: B = 1 (alone), B = 2
    (two lanes), B = 1 again (the captured forward is dropped when the lane's
    setting changes); and B = 1 with the wider form off (MPCX_QUAD_ALONE=64).
    Every forward matches the oracle."""
    dims = synth.Dims(bw=bw)
    W = synth.weights(dims, seed=31)
    d = _od(orc, dims)

    def batch(B, seed):
        X, A, mask = synth.molecules(B, dims, seed=seed, min_atoms=100, max_atoms=140)
        prot = synth.protein(B, dims, seed=seed + 1)
        want, code = orc.plain_forward(d, X, A, mask, prot, W)
        assert code == 0
        sh = [synth.share(v, bw, seed + 2 + k) for k, v in enumerate((X, A, mask))]
        return sh, prot, want

    def run(m, B, seed):
        sh, prot, want = batch(B, seed)
        m.keygen(B, 500 + seed)
        m.set_inputs(B, *sh[0], *sh[1], *sh[2], prot)
        m.forward(B)
        assert np.array_equal(m.output(B), want), (B, seed)

    c = mp.Ctx(bw=bw)
    m = mp.Model(c, dims, W, lanes=2)
    for B, seed in ((1, 40), (2, 41), (1, 42)):
        run(m, B, seed)
    m.close()
    c.close()
    monkeypatch.setenv("MPCX_QUAD_ALONE", "64")
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, dims, W)
    run(m, 1, 43)
    m.close()
    c.close()


@pytest.mark.parametrize("lanes", [1, 2])
def test_model_graph_replays(mp, orc, synth, monkeypatch, lanes):
    """Resident-key forwards are captured into a HIP graph once per batch size
    and replayed: four inputs in turn (with synchronised host work and eager
    kernels of the same context between replays), a second batch size (fresh
    keys, a new capture), then the first size again; every replay matches the
    oracle and the eager path (MPCX_GRAPH=0) on the same keys, exchange bytes
    included."""
    dims = synth.Dims(bw=32)
    W = synth.weights(dims, seed=9)
    d = _od(orc, dims)

    def batch(B, seed):
        X, A, mask = synth.molecules(B, dims, seed=seed)
        prot = synth.protein(B, dims, seed=seed + 1)
        want, code = orc.plain_forward(d, X, A, mask, prot, W)
        assert code == 0
        sh = [synth.share(v, 32, seed + 2 + k) for k, v in enumerate((X, A, mask))]
        return sh, prot, want

    c = mp.Ctx(bw=32)
    monkeypatch.setenv("MPCX_GRAPH", "0")
    ce = mp.Ctx(bw=32)
    m = mp.Model(c, dims, W, lanes=lanes)
    me = mp.Model(ce, dims, W, lanes=lanes)
    for B, seeds in ((3, (50, 60, 70, 80)), (5, (90,)), (3, (100,))):
        m.keygen(B, 123 + B)
        me.keygen(B, 123 + B)
        for sd in seeds:
            sh, prot, want = batch(B, sd)
            for mm in (m, me):
                mm.set_inputs(B, *sh[0], *sh[1], *sh[2], prot)
            c.reset_counters()
            ce.reset_counters()
            m.forward(B)
            me.forward(B)
            got = m.output(B)
            assert np.array_equal(got, want) and np.array_equal(me.output(B), want)
            assert c.bytes_exchanged == ce.bytes_exchanged > 0
            # eager work on the same context between replays
            A = rmask(np.random.default_rng(sd), 64 * 64, 32).reshape(64, 64)
            assert np.array_equal(c.ring_gemm(A, A).astype(np.uint64), orc.ring_gemm(32, A, A))
    m.close()
    me.close()
    c.close()
    ce.close()


def test_model_forward_on_oracle_keys_config0(mp, orc, synth):
    """Config 0 shape (B=16, N=140, bw=32): keys from the oracle's dealer,
    online phase on the GPU, outputs equal to the plaintext forward."""
    B = 16
    wl = synth.workload(B, synth.Dims(bw=32), seed=0)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    o0, o1 = orc.model_keygen(d, B, 4242, wl.W)
    c = mp.Ctx(bw=32)
    m = mp.Model(c, wl.dims, wl.W)
    m.import_keys(B, o0, o1)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    # repeated forwards on the same resident keys are deterministic
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    m.close()
    c.close()


@pytest.mark.parametrize("B,N,C", [(1, 1, 3), (3, 7, 4), (2, 140, 6), (4, 2, 33)])
def test_maxpool_keys_and_eval(ctx, orc, B, N, C):
    """Standalone masked max-pool (MaskedMaxPoolLayer, masked_maxpool_layer.h:47-165):
    keys byte-identical to the oracle dealer's, outputs and exchanged bytes
    identical to the oracle's, unmasked output = max over the rows."""
    bw = ctx.bw
    rng = np.random.default_rng(bw + N)
    q = 1 << (bw - 2)
    v = rng.integers(-q, q, size=(B, N, C), dtype=np.int64)
    v[:, :, 0] = rng.integers(-2, 2, size=(B, N))
    rin = rmask(rng, v.size, bw)
    g0, g1, grout = ctx.maxpool_keygen(B, N, C, rin, seed=3, gate=40)
    o0, o1, orout = orc.maxpool_keygen(3, 40, bw, S, B, N, C, rin)
    assert ctx.lib.mpcx_maxpool_key_bytes(ctx.h, B, N, C) == o0.size
    assert ctx.lib.mpcx_maxpool_levels(N) == (int(np.ceil(np.log2(N))) if N > 1 else 0)
    assert np.array_equal(grout.astype(np.uint64), orout)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    xhat = (v.reshape(-1).astype(np.uint64) + rin) & M(bw)
    ctx.reset_counters()
    y = ctx.maxpool_eval(B, N, C, g0, g1, xhat)
    by = ctx.bytes_exchanged
    oy, oby = orc.maxpool_eval(bw, S, B, N, C, o0, o1, xhat)
    assert np.array_equal(y.astype(np.uint64), oy)
    assert by == oby
    assert np.array_equal(signed(y.astype(np.uint64) - orout, bw).reshape(B, C), v.max(axis=1))


def test_maxpool_affinity_pool_shape(mp):
    """The affinity forward's pool at full size (B=64 molecules x 140 atoms x 312
    channels, bw=32, 8 levels): non-negative activations with zeroed padding rows
    (the reference's H (.) mask input), against numpy's max."""
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(5)
    B, N, C = 64, 140, 312
    v = rng.integers(0, 1 << 24, size=(B, N, C), dtype=np.int64)
    real = rng.integers(10, 61, size=B)
    v[np.arange(N)[None, :] >= real[:, None]] = 0
    rin = rmask(rng, v.size, 32)
    k0, k1, rout = c.maxpool_keygen(B, N, C, rin, seed=8, gate=1)
    y = c.maxpool_eval(B, N, C, k0, k1, (v.reshape(-1).astype(np.uint64) + rin) & M(32))
    assert np.array_equal(signed(y.astype(np.uint64) - rout.astype(np.uint64), 32).reshape(B, C), v.max(axis=1))
    c.close()


def test_relu_microbench_slice(mp):
    """Config 1 shape at 2^20 elements: ReLU of uniform fixed-point values in
    [-8, 8), reconstructed against max(x, 0)."""
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(1)
    n = 1 << 20
    x = rng.integers(-8 << S, 8 << S, size=n)
    rin = rmask(rng, n, 32)
    k0, k1, rout = c.tr_keygen(3, rin, seed=11, gate=1)
    y = c.tr_eval(3, k0, k1, (x.astype(np.uint64) + rin) & M(32))
    assert np.array_equal(signed(y.astype(np.uint64) - rout.astype(np.uint64), 32), np.maximum(x, 0))
    c.close()


# ---------------------------------------------------------------------------
# committed fixtures (tests/golden/)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bw", [32, 64])
def test_model_small_fixture(mp, synth, bw):
    import os
    from golden_dims import SMALL
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "model_small.npz"))
    dims = synth.Dims(bw=bw, **SMALL)
    B = f["X"].shape[0]
    sh = {k: synth.share(f[v], bw, 40 + i) for i, (k, v) in enumerate((("x", "X"), ("a", "A"), ("m", "mask")))}
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, dims, f["W"])
    m.keygen(B, 99)
    m.set_inputs(B, *sh["x"], *sh["a"], *sh["m"], f["prot"])
    m.forward(B)
    assert np.array_equal(m.output(B), f[f"want_bw{bw}"])
    m.close()
    c.close()


@pytest.mark.parametrize("bw", [32, 64])
def test_model_default_fixture(mp, synth, bw):
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "model_default.json")) as fh:
        rec = json.load(fh)
    B = rec["B"]
    wl = synth.workload(B, synth.Dims(bw=bw), seed=rec["seed"])
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W)
    m.keygen(B, 2024)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    m.forward(B)
    assert m.output(B).tolist() == rec[f"want_bw{bw}"]
    m.close()
    c.close()


# ---------------------------------------------------------------------------
# standalone secure adjacency normalisation (config 2)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bw", [32, 64])
def test_adjnorm_keys_and_eval(mp, orc, synth, bw):
    B, N = 3, 24
    _, A, _ = synth.molecules(B, synth.Dims(bw=bw, n_nodes=N), seed=5, min_atoms=3, max_atoms=N)
    a0, a1 = synth.share(A, bw, 77)
    c = mp.Ctx(bw=bw)
    g0, g1, gmask = c.adjnorm_keygen(B, N, seed=123)
    o0, o1, omask = orc.adjnorm_keygen(bw, S, B, N, 123)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    assert np.array_equal(mp.from_dev(gmask, c.T, B * N * N).astype(np.uint64), omask)
    c.reset_counters()
    got = c.adjnorm_eval(B, N, 138, g0, g1, a0, a1)
    want, oby = orc.adjnorm_eval(bw, S, B, N, 138, o0, o1, a0, a1)
    assert np.array_equal(got.astype(np.uint64), want)
    assert c.bytes_exchanged == oby
    # the context keeps the prepared maps and scratch between calls: a smaller
    # batch (re-prepared), then the first batch again, on the same context
    g0s, g1s, gms = c.adjnorm_keygen(1, N, seed=124)
    o0s, o1s, _ = orc.adjnorm_keygen(bw, S, 1, N, 124)
    got1 = c.adjnorm_eval(1, N, 138, g0s, g1s, a0[:1], a1[:1])
    want1, _ = orc.adjnorm_eval(bw, S, 1, N, 138, o0s, o1s, a0[:1], a1[:1])
    assert np.array_equal(got1.astype(np.uint64), want1)
    assert np.array_equal(c.adjnorm_eval(B, N, 138, g0, g1, a0, a1).astype(np.uint64), want)
    c.close()


@pytest.mark.parametrize("bw,lanes", [(32, 3), (64, 2)])
def test_adjnorm_lanes(mp, orc, synth, bw, lanes):
    """Concurrent graph groups: the key set is the groups' one-group key sets
    (group i under seed + i * 0x9E3779B97F4A7C15) back to back, byte-identical
    to the oracle dealer's; the outputs and exchange bytes are the groups'."""
    B, N, seed = 5, 20, 321
    _, A, _ = synth.molecules(B, synth.Dims(bw=bw, n_nodes=N), seed=6, min_atoms=3, max_atoms=N)
    a0, a1 = synth.share(A, bw, 78)
    c = mp.Ctx(bw=bw)
    c.set_adjnorm_lanes(lanes)
    g0, g1, gmask = c.adjnorm_keygen(B, N, seed=seed)
    sizes = [B // lanes + (1 if i < B % lanes else 0) for i in range(lanes)]
    ok0, ok1, omask, want, oby, g = [], [], [], [], 0, 0
    for i, Bi in enumerate(sizes):
        si = (seed + i * 0x9E3779B97F4A7C15) % (1 << 64)
        k0, k1, m = orc.adjnorm_keygen(bw, S, Bi, N, si)
        ok0.append(k0)
        ok1.append(k1)
        omask.append(m)
        y, by = orc.adjnorm_eval(bw, S, Bi, N, 138, k0, k1, a0[g:g + Bi], a1[g:g + Bi])
        want.append(y)
        oby += by
        g += Bi
    o0, o1 = np.concatenate(ok0), np.concatenate(ok1)
    assert c.lib.mpcx_adjnorm_key_bytes(c.h, B, N) == o0.size
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    assert np.array_equal(mp.from_dev(gmask, c.T, B * N * N).astype(np.uint64), np.concatenate(omask))
    c.reset_counters()
    for _ in range(2):  # the second call reuses the prepared groups and streams
        got = c.adjnorm_eval(B, N, 138, g0, g1, a0, a1)
        assert np.array_equal(got.astype(np.uint64), np.concatenate(want))
    assert c.bytes_exchanged == 2 * oby
    c.close()


@pytest.mark.parametrize("bw", [32, 64])
def test_adjnorm_max_nodes_and_degrees(mp, orc, bw):
    """N = 255 (the 8-bit degree domain's limit): a star whose centre has degree
    255 (past the table's 138 entries, so T = 0), an isolated atom (self loop
    only, degree 1), a path, random edges, and padding; keys byte-identical,
    every unmasked entry equal to the closed form."""
    B, N = 2, 255
    rng = np.random.default_rng(255)
    A = np.zeros((B, N, N), np.int64)
    A[0, 0, :] = 1
    A[0, :, 0] = 1
    np.fill_diagonal(A[0], 1)  # star: centre degree 255, leaves degree 2
    n1 = 200
    idx = np.arange(n1)
    A[1, idx, idx] = 1
    A[1, idx[1:100], idx[:99]] = 1  # a path over atoms 0..99
    A[1, idx[:99], idx[1:100]] = 1
    for _ in range(300):  # random extra edges among atoms 100..198 (atom 199 stays isolated)
        i, j = rng.integers(100, n1 - 1, size=2)
        A[1, i, j] = A[1, j, i] = 1
    M = (1 << bw) - 1
    a0 = rng.integers(0, 1 << 63, size=A.size, dtype=np.uint64) & np.uint64(M)
    a1 = (A.reshape(-1).astype(np.uint64) - a0) & np.uint64(M)
    c = mp.Ctx(bw=bw)
    g0, g1, gmask = c.adjnorm_keygen(B, N, seed=31)
    o0, o1, omask = orc.adjnorm_keygen(bw, S, B, N, 31)
    assert np.array_equal(host(g0)[:o0.size], o0) and np.array_equal(host(g1)[:o1.size], o1)
    out = c.adjnorm_eval(B, N, 138, g0, g1, a0, a1)
    got = signed(out.astype(np.uint64) - omask, bw)
    want = orc.adj_norm_plain(A).reshape(-1)
    assert np.array_equal(got, want)
    assert want.reshape(B, N, N)[0, 0].sum() == 0  # the degree-255 centre has T = 0
    c.close()


def test_adjnorm_config2_full_size(mp, orc, synth):
    """Config 2: B=1024 graphs of the config-0 distribution, N=140, Z_2^32.
    Every unmasked entry equals A[i,j] * floor(T[d_i] T[d_j] / 2^12)."""
    B, N, bw = 1024, 140, 32
    _, A, _ = synth.molecules(B, synth.Dims(bw=bw), seed=2)
    a0, a1 = synth.share(A, bw, 3)
    c = mp.Ctx(bw=bw)
    k0, k1, mask = c.adjnorm_keygen(B, N, seed=9)
    out = c.adjnorm_eval(B, N, 138, k0, k1, a0, a1, as_device=True)
    got = (mp.from_dev(out, np.uint32, B * N * N) - mp.from_dev(mask, np.uint32, B * N * N)).astype(np.int64)
    want = orc.adj_norm_plain(A).reshape(-1)
    assert np.array_equal(got, want)
    c.close()


# ---------------------------------------------------------------------------
# streamed key arena (config 4 path)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bw", [32, 64])
def test_model_streamed_keys_match_resident(mp, orc, synth, bw):
    """Keys exported to pinned host memory and streamed through two small
    device slots give the same outputs as the resident arena, on two
    consecutive forwards (slot events reused)."""
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw), seed=31)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, wl.dims, wl.W)
    m.keygen(B, 555)
    nbytes = m.key_bytes(B)
    h0, h1 = mp.PinnedBuffer(nbytes), mp.PinnedBuffer(nbytes)
    m.export_keys(0, B, into=h0)
    m.export_keys(1, B, into=h1)
    m.release_arena()
    # a slot smaller than one gate's key is refused; a quarter of the arena
    # (the largest gate, GCN-3's TRRELU, is about a fifth) gives several chunks
    with pytest.raises(mp.MpcxError):
        m.attach_host_keys(B, h0, h1, slot_bytes=4096)
    m.attach_host_keys(B, h0, h1, slot_bytes=nbytes // 4)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    for _ in range(2):
        m.forward(B)
        assert np.array_equal(m.output(B), want)
        st = m.stream_stats()
        # party 1's copy skips the correction/leaf words both parties hold
        assert st["chunks"] >= 4 and nbytes < st["bytes_h2d"] < 1.6 * nbytes
    # party 1's key packed (without the planes it reads from party 0's copy and
    # those drawn from its own PRF key, expanded on the device): same outputs
    m.close()
    m = mp.Model(c, wl.dims, wl.W)
    m.keygen(B, 555)
    hp = mp.PinnedBuffer(m.unique_key_bytes(B, 1))
    assert hp.nbytes < nbytes // 2
    m.export_unique_keys(1, B, into=hp)
    m.release_arena()
    m.attach_host_keys(B, h0, hp, slot_bytes=nbytes // 4)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    hdr = 256  # the packed key's header (the party's PRF key) is not copied
    assert m.stream_stats()["bytes_h2d"] == nbytes + hp.nbytes - hdr
    # a second input batch on the same streamed keys
    wl2 = synth.workload(B, synth.Dims(bw=bw), seed=32)
    want2, code = orc.plain_forward(d, wl2.X, wl2.A, wl2.mask, wl2.prot, wl.W)
    assert code == 0
    m.set_inputs(B, *wl2.shares["x"], *wl2.shares["a"], *wl2.shares["m"], wl2.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want2)
    # back to a resident arena: a fresh dealer run replaces the streamed keys
    m.keygen(B, 556)
    m.forward(B)
    assert np.array_equal(m.output(B), want2)
    assert m.stream_stats()["chunks"] == 0
    # both parties packed: the planes the dealer drew from each party's PRF key
    # are expanded in the device slots after the copies
    hq = mp.PinnedBuffer(m.unique_key_bytes(B, 0))
    hq1 = mp.PinnedBuffer(m.unique_key_bytes(B, 1))
    assert hq.nbytes < 0.95 * nbytes and hq1.nbytes == hp.nbytes
    m.export_unique_keys(0, B, into=hq)
    m.export_unique_keys(1, B, into=hq1)
    m.release_arena()
    m.attach_host_keys(B, hq, hq1, slot_bytes=nbytes // 4)
    m.set_inputs(B, *wl2.shares["x"], *wl2.shares["a"], *wl2.shares["m"], wl2.prot)
    for _ in range(2):
        m.forward(B)
        assert np.array_equal(m.output(B), want2)
        assert m.stream_stats()["bytes_h2d"] == hq.nbytes + hq1.nbytes - 2 * hdr
    # imported keys carry no PRF keys: no packed export
    m.keygen(B, 557)
    k0, k1 = m.export_keys(0, B), m.export_keys(1, B)
    m.import_keys(B, k0, k1)
    with pytest.raises(mp.MpcxError):
        m.export_unique_keys(0, B, into=hq)
    m.close()
    c.close()
    for h in (h0, h1, hp, hq, hq1):
        h.free()


@pytest.mark.parametrize("bw,lanes,packed", [(64, 1, True), (32, 2, False)])
def test_model_key_files(mp, orc, synth, tmp_path, bw, lanes, packed):
    """File-backed keys: three key sets (fresh dealer seeds) appended to two
    files, streamed chunk by chunk through the I/O thread's pinned staging
    buffers; four forwards use sets 0, 1, 2, 0, each on its own inputs, and
    give the plaintext outputs.  Files that do not hold whole key sets are
    refused."""
    B = 3
    c = mp.Ctx(bw=bw)
    wls = [synth.workload(B, synth.Dims(bw=bw), seed=40 + k) for k in range(4)]
    W = wls[0].W
    d = _od(orc, wls[0].dims)
    m = mp.Model(c, wls[0].dims, W, lanes=lanes)
    p0, p1 = tmp_path / "keys0.bin", tmp_path / "keys1.bin"
    for k in range(3):
        m.keygen(B, 1000 + k)
        m.write_keys(0, p0, packed=packed, append=k > 0)
        m.write_keys(1, p1, packed=packed, append=k > 0)
    nbytes = m.key_bytes(B)
    assert p0.stat().st_size == 3 * (m.unique_key_bytes(B, 0) if packed else nbytes)
    assert p1.stat().st_size == 3 * (m.unique_key_bytes(B, 1) if packed else nbytes)
    m.release_arena()
    bad = tmp_path / "short.bin"
    bad.write_bytes(p0.read_bytes()[: p0.stat().st_size // 3 // 2])
    with pytest.raises(mp.MpcxError):
        m.attach_key_files(B, bad, p1, slot_bytes=nbytes // 4)
    with pytest.raises(mp.MpcxError):
        m.attach_key_files(B, tmp_path / "missing.bin", p1, slot_bytes=nbytes // 4)
    m.attach_key_files(B, p0, p1, slot_bytes=nbytes // 4)
    for wl in wls:
        want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, W)
        assert code == 0
        m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
        m.forward(B)
        assert np.array_equal(m.output(B), want)
        assert m.stream_stats()["chunks"] >= 4
    m.close()
    c.close()


def test_relu_config1_full_size(mp):
    """Config 1: 2^24 ReLUs over Z_2^32 of uniform fixed-point values in
    [-8, 8), one 31-bit DCF key per element, against max(x, 0)."""
    c = mp.Ctx(bw=32)
    rng = np.random.default_rng(24)
    n = 1 << 24
    x = rng.integers(-8 << S, 8 << S, size=n)
    rin = rmask(rng, n, 32)
    k0, k1, rout = c.tr_keygen(3, rin, seed=12, gate=1)
    y = c.tr_eval(3, k0, k1, (x.astype(np.uint64) + rin) & M(32))
    assert np.array_equal(signed(y.astype(np.uint64) - rout.astype(np.uint64), 32), np.maximum(x, 0))
    c.close()


# ---------------------------------------------------------------------------
# inputs from the reference's file formats
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bw", [32, 64])
def test_model_on_reference_files(mp, orc, synth, tmp_path, bw):
    """Shares, protein rows and weights written in the reference's layout
    (mask pre-tiled at scale s) load into the model with mask_scale = s and
    reconstruct the plaintext forward exactly."""
    import formats
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw), seed=12)
    bdir = str(tmp_path / "batch")
    formats.write_batch(bdir, wl.X, wl.A, wl.mask, wl.prot, bw=bw, scale=12, pool_dim=312, seed=5)
    wpath = str(tmp_path / "weights.bin")
    formats.write_weights(wpath, wl.W, wl.dims.layers(), scale=12)
    got = formats.read_batch(bdir)
    blob, layers, _ = formats.read_weights(wpath)
    dims = formats.dims_from_weights(layers, n_nodes=140, bw=bw, mask_scale=got["mask_scale"])
    want, code = orc.plain_forward(_od(orc, synth.Dims(bw=bw)), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    c = mp.Ctx(bw=bw)
    m = mp.Model(c, dims, blob)
    m.keygen(B, 8)
    m.set_inputs(B, *got["x"], *got["a"], *got["m"], got["prot"])
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    m.close()
    c.close()


# ---------------------------------------------------------------------------
# command-line driver over the C ABI (the reference's deepdtagen_inference role)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bw", [32, 64])
def test_driver_dealer_then_evaluator(mp, orc, synth, tmp_path, bw):
    """mpcx_infer: the dealer run writes both parties' key files, the evaluator
    run reads them with the reference-format batch and weights and prints one
    AFFINITY line per molecule, equal to the fixed-point forward; the combined
    run (role 2, two lanes) prints the same lines.  The dealer draws its keys
    under the 16-byte secret key of MPCX_DEALER_KEY (other key files than the
    seed alone gives, which it warns about); a key file of another size is
    refused."""
    import os
    import re
    import subprocess
    import formats
    exe = os.path.join(os.path.dirname(mp.__file__), "mpcx_infer")
    assert os.path.exists(exe), "mpcx_infer not built"
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw), seed=14)
    bdir, kdir = tmp_path / "batch", tmp_path / "keys"
    kdir.mkdir()
    formats.write_batch(str(bdir), wl.X, wl.A, wl.mask, wl.prot, bw=bw, scale=12, pool_dim=312, seed=6)
    wpath = str(tmp_path / "weights.bin")
    formats.write_weights(wpath, wl.W, wl.dims.layers(), scale=12)
    want, code = orc.plain_forward(_od(orc, synth.Dims(bw=bw)), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    lines = [f"AFFINITY[{j}]={v / 4096.0:.6f}" for j, v in enumerate(want)]
    env = dict(os.environ, MPCX_WEIGHTS_BIN=wpath)

    def run(role, extra_env=None, full=False):
        r = subprocess.run([exe, str(bw), "12", str(role), str(kdir), str(bdir)], env=dict(env, **(extra_env or {})),
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        return r if full else r.stdout

    # the dealer with its secret key file (MPCX_DEALER_KEY), then without one
    kfile = tmp_path / "dealer.key"
    kfile.write_bytes(bytes(range(7, 23)))
    kenv = {"MPCX_DEALER_KEY": str(kfile)}
    r0 = run(0, kenv, full=True)
    assert "MPCX_DEALER_KEY" not in r0.stderr
    k_keyed = (kdir / f"DeepDTAGen_{bw}_12_party0").read_bytes()
    assert len(k_keyed) > 0
    out = run(1)
    assert re.findall(r"AFFINITY\[\d+\]=\S+", out) == lines
    assert int(re.search(r"Comm \(B\)=(\d+)", out).group(1)) > 0
    r0 = run(0, full=True)
    assert "warning: no MPCX_DEALER_KEY" in r0.stderr
    k_seed = (kdir / f"DeepDTAGen_{bw}_12_party0").read_bytes()
    assert len(k_seed) == len(k_keyed) and k_seed != k_keyed  # the key, not the seed alone, drew the masks
    out = run(1)
    assert re.findall(r"AFFINITY\[\d+\]=\S+", out) == lines
    out2 = run(2, dict(kenv, MPCX_LANES="2"))
    assert re.findall(r"AFFINITY\[\d+\]=\S+", out2) == lines
    kfile.write_bytes(bytes(15))  # not 16 bytes: refused
    bad = subprocess.run([exe, str(bw), "12", "0", str(kdir), str(bdir)], env=dict(env, **kenv),
                         capture_output=True, text=True, timeout=120)
    assert bad.returncode != 0 and "16 bytes" in bad.stderr
    # a batch that does not match the key files is refused
    bad = subprocess.run([exe, str(bw), "12", "1", str(kdir), str(bdir), "2"], env=env, capture_output=True,
                         text=True, timeout=120)
    assert bad.returncode != 0
