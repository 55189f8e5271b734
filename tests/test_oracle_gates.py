"""Pins the oracle's two-party gates against closed forms (CPU only).

Each gate is keyed on a random input mask, evaluated by both parties on the
masked input, reconstructed, unmasked, and compared with the plaintext
function: signed floor(x/2^s) + bias (TrFloor, gpu_mpc/ddg_orca.h:112-123),
max(x, 0) (ddg_orca.h:83-110), x*y (Beaver, secure_adj_norm.h:611-651),
table[x] (DPF LUT, secure_adj_norm.h:495-520), A.B mod 2^bw
(ddg_orca_base.h:170-205).  Boundary values of the signed ring are included.
"""
import numpy as np
import pytest

S = 12


def mod(bw):
    return (1 << bw) - 1


def to_signed(v, bw):
    v = np.asarray(v, np.uint64)
    if bw == 64:
        return v.view(np.int64)
    v = (v & np.uint64(mod(bw))).astype(np.int64)
    return np.where(v >= 1 << (bw - 1), v - (1 << bw), v)


def ring(v, bw):
    return np.asarray(v, np.int64).astype(np.uint64) & np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)


def mask_in(rng, n, bw):
    return rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + rng.integers(0, 2, size=n,
                                                                                       dtype=np.uint64) \
        if bw == 64 else rng.integers(0, 1 << bw, size=n, dtype=np.uint64)


def edge_values(bw, s):
    h = 1 << (bw - 1)
    return [-h, -h + 1, -1, 0, 1, h - 1, (1 << s) - 1, 1 << s, -(1 << s), -(1 << s) - 1, -(1 << s) + 1]


@pytest.mark.parametrize("bw", [32, 64])
@pytest.mark.parametrize("kind", [1, 2, 3])
def test_tr_relu_family(orc, bw, kind):
    rng = np.random.default_rng(bw * 10 + kind)
    n = 3000
    h = 1 << (bw - 1)
    x = np.concatenate([np.array(edge_values(bw, S), np.int64),
                        rng.integers(-(h // 4), h // 4, size=n, dtype=np.int64)])
    x = np.concatenate([x, rng.integers(-5 << S, 5 << S, size=n)])
    N = x.size
    bias = rng.integers(-(1 << 14), 1 << 14, size=N) if kind in (1, 2) else None
    if bias is not None:
        # keep x + bias*2^s inside the signed ring (the bit-exact domain)
        lim = h - (1 << (14 + S)) - 1
        x = np.clip(x, -lim, lim)
    rin = mask_in(rng, N, bw)
    k0, k1, rout = orc.tr_keygen(5, 17, kind, bw, S, rin)
    xhat = (ring(x, bw) + rin) & np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, by = orc.tr_eval(kind, bw, S, k0, k1, xhat, bias)
    got = to_signed(y - rout, bw)
    if kind == 1:
        exp = (x + (bias << S)) >> S
    elif kind == 2:
        exp = np.maximum((x + (bias << S)) >> S, 0)
    else:
        exp = np.maximum(x, 0)
    assert np.array_equal(got, exp)
    nbits = 2 if kind in (1, 2) else 1
    assert by == 2 * (nbits * ((N + 31) // 32) * 4 + N * bw // 8)


@pytest.mark.parametrize("bw", [32, 64])
@pytest.mark.parametrize("relu", [False, True])
def test_split_truncation(orc, bw, relu):
    """TRMOD then EXT (EXTRELU) = signed floor((x + bias*2^s)/2^s), and its ReLU,
    over the whole signed ring (the ring's edges included): the two-gate exact
    truncation with one s-bit and one (bw-s-1)-bit DCF (gpu_mpc/dpf_dcf_adapter.h:
    274-303, ReLU-extend :225-234).  TRMOD alone is exact modulo 2^(bw-s) only;
    EXT reads only the low bw-s bits of its input and of its input mask."""
    rng = np.random.default_rng(bw * 3 + relu)
    n = 4000
    h = 1 << (bw - 1)
    x = np.concatenate([np.array(edge_values(bw, S), np.int64), rng.integers(-h, h - 1, size=n, dtype=np.int64),
                        rng.integers(-5 << S, 5 << S, size=n)])
    N = x.size
    bias = rng.integers(-(1 << 14), 1 << 14, size=N)
    lim = h - (1 << (14 + S)) - 1
    x = np.clip(x, -lim, lim)
    M = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    low = np.uint64((1 << (bw - S)) - 1)
    rin = mask_in(rng, N, bw)
    k0, k1, r1 = orc.tr_keygen(5, 20, 12, bw, S, rin)
    y1, b1 = orc.tr_eval(12, bw, S, k0, k1, (ring(x, bw) + rin) & M, bias)
    exp = (x + (bias << S)) >> S
    assert np.array_equal((y1 - r1) & low, ring(exp, bw) & low)
    assert np.all(y1 <= low)  # revealed reduced to bw-s bits, as the reference's bout = bin - shift
    # only the low bw-s bits are meaningful: move the high bits of the value and
    # of its mask independently
    y1x = (y1 + (rng.integers(0, 1 << S, size=N).astype(np.uint64) << np.uint64(bw - S))) & M
    r1x = (r1 + (rng.integers(0, 1 << S, size=N).astype(np.uint64) << np.uint64(bw - S))) & M
    kind = 14 if relu else 13
    q0, q1, r2 = orc.tr_keygen(5, 21, kind, bw, S, r1x)
    y2, b2 = orc.tr_eval(kind, bw, S, q0, q1, y1x)
    got = to_signed(y2 - r2, bw)
    assert np.array_equal(got, np.maximum(exp, 0) if relu else exp)
    per = 2 * (((N + 31) // 32) * 4 + N * bw // 8)
    # TRMOD's message goes out packed at bw-s bits per element in 64-bit words
    # (gpu_mpc/utils/gpu_comms.h:143-168): at bw=32, 20 bits instead of 32
    packed = 2 * (((N + 31) // 32) * 4 + ((N * (bw - S) + 63) // 64) * 8)
    assert b1 == packed and b2 == per
    split = orc.tr_layout(12, bw, S, N).end + orc.tr_layout(kind, bw, S, N).end
    assert split < orc.tr_layout(2 if relu else 1, bw, S, N).end


@pytest.mark.parametrize("bw", [32, 64])
def test_tr_slack(orc, bw):
    rng = np.random.default_rng(bw)
    q = 1 << (bw - 2)
    x = np.concatenate([np.array([-q, -q + 1, -1, 0, 1, q - 1, (1 << S) - 1, -(1 << S)], np.int64),
                        rng.integers(-q, q, size=4000, dtype=np.int64)])
    rin = mask_in(rng, x.size, bw)
    k0, k1, rout = orc.tr_keygen(9, 3, 4, bw, S, rin)
    xhat = (ring(x, bw) + rin) & np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, _ = orc.tr_eval(4, bw, S, k0, k1, xhat)
    assert np.array_equal(to_signed(y - rout, bw), x >> S)


@pytest.mark.parametrize("bw", [32, 64])
def test_relu_slack(orc, bw):
    """ReLU for |x| < 2^(bw-2-s) with a (bw-2-s)-bit DCF: the domain edges, small
    values around 0 and uniform values; its key is smaller than the full ReLU's."""
    rng = np.random.default_rng(bw + 7)
    q = 1 << (bw - 2 - S)
    x = np.concatenate([np.array([-q, -q + 1, -2, -1, 0, 1, 2, q - 2, q - 1], np.int64),
                        rng.integers(-q, q, size=4000, dtype=np.int64), rng.integers(-40, 40, size=500)])
    rin = mask_in(rng, x.size, bw)
    k0, k1, rout = orc.tr_keygen(9, 4, 9, bw, S, rin)
    xhat = (ring(x, bw) + rin) & np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, by = orc.tr_eval(9, bw, S, k0, k1, xhat)
    assert np.array_equal(to_signed(y - rout, bw), np.maximum(x, 0))
    assert by == 2 * (((x.size + 31) // 32) * 4 + x.size * bw // 8)
    assert orc.tr_layout(9, bw, S, x.size).end < orc.tr_layout(3, bw, S, x.size).end


@pytest.mark.parametrize("bw", [32, 64])
def test_relu_pool(orc, bw):
    """ReLU for |x| < 2^(bw-s) with a (bw-s)-bit DCF (the max-pool differences of
    truncated activations): the domain edges, values around 0, uniform values;
    a value just outside (2^(bw-s)) reads as negative, so the gate really takes
    the sign from bit bw-s."""
    rng = np.random.default_rng(bw + 9)
    q = 1 << (bw - S)
    x = np.concatenate([np.array([-q + 1, -q // 2, -2, -1, 0, 1, 2, q // 2, q - 1], np.int64),
                        rng.integers(-q + 1, q, size=4000, dtype=np.int64), rng.integers(-40, 40, size=500)])
    rin = mask_in(rng, x.size, bw)
    k0, k1, rout = orc.tr_keygen(9, 6, 15, bw, S, rin)
    M = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, by = orc.tr_eval(15, bw, S, k0, k1, (ring(x, bw) + rin) & M)
    assert np.array_equal(to_signed(y - rout, bw), np.maximum(x, 0))
    assert by == 2 * (((x.size + 31) // 32) * 4 + x.size * bw // 8)
    assert orc.tr_layout(15, bw, S, x.size).end < orc.tr_layout(3, bw, S, x.size).end
    xo = np.array([q, q + 5], np.int64)
    ko0, ko1, ro = orc.tr_keygen(9, 7, 15, bw, S, rin[:2])
    yo, _ = orc.tr_eval(15, bw, S, ko0, ko1, (ring(xo, bw) + rin[:2]) & M)
    assert np.array_equal(to_signed(yo - ro, bw), [0, 0])


def test_relu_slack_catches_wrong_sign_bit(orc):
    """A value just outside the domain (x = 2^(bw-2-s)) reads as negative: the
    gate really uses bit bw-2-s, which the in-domain test alone would not show."""
    bw = 32
    q = 1 << (bw - 2 - S)
    x = np.array([q, -q - 1], np.int64)
    rin = np.array([12345, 987654321], np.uint64)
    k0, k1, rout = orc.tr_keygen(9, 5, 9, bw, S, rin)
    y, _ = orc.tr_eval(9, bw, S, k0, k1, (ring(x, bw) + rin) & np.uint64(mod(bw)))
    assert np.array_equal(to_signed(y - rout, bw), [0, -q - 1])


@pytest.mark.parametrize("bw", [32, 64])
def test_mul_index_maps(orc, bw):
    rng = np.random.default_rng(3)
    nx, ny, nz = 50, 40, 500
    lim = 1 << (14 if bw == 32 else 30)  # products stay inside the signed ring
    xv = rng.integers(-lim, lim, size=nx)
    yv = rng.integers(-lim, lim, size=ny)
    ia = rng.integers(0, nx, size=nz).astype(np.uint32)
    ib = rng.integers(0, ny, size=nz).astype(np.uint32)
    rx, ry = mask_in(rng, nx, bw), mask_in(rng, ny, bw)
    k0, k1, rz = orc.mul_keygen(2, 4, bw, rx, ry, ia, ib)
    M = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    z, _ = orc.mul_eval(bw, k0, k1, (ring(xv, bw) + rx) & M, (ring(yv, bw) + ry) & M, ia, ib)
    assert np.array_equal(to_signed(z - rz, bw), xv[ia] * yv[ib])


@pytest.mark.parametrize("bw", [32, 64])
def test_lut8_all_inputs(orc, bw):
    rng = np.random.default_rng(8)
    table = orc.invsqrt_table(S, 138)
    x = np.tile(np.arange(256, dtype=np.uint64), 3)
    rin = mask_in(rng, x.size, bw)
    k0, k1, rout = orc.lut8_keygen(4, 6, bw, rin)
    M = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, _ = orc.lut8_eval(bw, k0, k1, table, (x + rin) & M)
    assert np.array_equal((y - rout) & M, table[x.astype(np.int64)])


def test_invsqrt_table_values(orc):
    # T[k] = llround(2^12/sqrt(k)), T[0] = 0 (secure_adj_norm.h:138-184)
    t = orc.invsqrt_table(12, 138)
    assert list(t[:7]) == [0, 4096, 2896, 2365, 2048, 1832, 1672]
    assert t[138] == round(4096 / 138 ** 0.5) and t[139] == 0 and t[255] == 0


@pytest.mark.parametrize("bw", [32, 64])
def test_sxs_matches_matmul(orc, bw):
    rng = np.random.default_rng(11)
    nb, M_, K, N = 3, 7, 9, 5
    A = rng.integers(-(1 << 12), 1 << 12, size=(nb, M_, K))
    B = rng.integers(-(1 << 12), 1 << 12, size=(nb, K, N))
    ra, rb = mask_in(rng, A.size, bw), mask_in(rng, B.size, bw)
    k0, k1, rc = orc.sxs_keygen(3, 2, bw, nb, M_, K, N, ra, rb)
    MM = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    c, _ = orc.sxs_eval(bw, nb, M_, K, N, k0, k1, (ring(A, bw).ravel() + ra) & MM, (ring(B, bw).ravel() + rb) & MM)
    assert np.array_equal(to_signed(c - rc, bw).reshape(nb, M_, N), np.einsum("bmk,bkn->bmn", A, B))


def test_reveal(orc):
    rng = np.random.default_rng(2)
    bw = 32
    v = rng.integers(-1000, 1000, size=100)
    v0 = rng.integers(0, 1 << 32, size=100, dtype=np.uint64)
    v1 = (ring(v, bw) - v0) & np.uint64(mod(bw))
    k0, k1, m = orc.reveal_keygen(1, 1, bw, 100)
    vh, by = orc.reveal_eval(bw, k0, k1, v0, v1)
    assert np.array_equal(to_signed(vh - m, bw), v)
    assert by == 2 * 100 * 4


def test_gate_keys_deterministic_and_seed_dependent(orc):
    rin = np.arange(100, dtype=np.uint64) * np.uint64(2654435761)
    a0, a1, ra = orc.tr_keygen(1, 2, 2, 32, S, rin)
    b0, b1, rb = orc.tr_keygen(1, 2, 2, 32, S, rin)
    c0, _, rc = orc.tr_keygen(2, 2, 2, 32, S, rin)
    assert np.array_equal(a0, b0) and np.array_equal(a1, b1) and np.array_equal(ra, rb)
    assert not np.array_equal(a0, c0) and not np.array_equal(ra, rc)


@pytest.mark.parametrize("bw", [32, 64])
@pytest.mark.parametrize("B,N,C", [(1, 1, 3), (2, 2, 5), (3, 7, 4), (2, 140, 6), (1, 33, 1)])
def test_maxpool_tree(orc, bw, B, N, C):
    """Masked global max-pool (gpu_mpc/masked_maxpool_layer.h:47-165): the
    reconstructed, unmasked output is the maximum over the N rows of every
    (sample, channel), for signed values whose pairwise differences stay in the
    ring (|v| < 2^(bw-2)); ties, one row and odd levels included."""
    rng = np.random.default_rng(bw + 7 * N + C)
    q = 1 << (bw - 2)
    v = rng.integers(-q, q, size=(B, N, C), dtype=np.int64)
    v[:, :, 0] = rng.integers(-3, 3, size=(B, N))  # many ties
    if N > 2:
        v[0, N - 1, :] = q - 1  # the carried odd row holds the maximum
        v[B - 1, 1, :] = -q     # the ring's lower edge
    rin = mask_in(rng, v.size, bw)
    k0, k1, rout = orc.maxpool_keygen(3, 40, bw, S, B, N, C, rin)
    levels = int(np.ceil(np.log2(N))) if N > 1 else 0
    assert k0.size == orc.lib().orc_maxpool_layout(bw, S, B, N, C, 0)
    assert (k0.size == 0) == (levels == 0)
    xhat = (ring(v.reshape(-1), bw) + rin) & np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    y, by = orc.maxpool_eval(bw, S, B, N, C, k0, k1, xhat)
    got = to_signed(y - rout, bw).reshape(B, C)
    assert np.array_equal(got, v.max(axis=1))
    # every level is one RELU gate over B * pairs * C differences
    want_bytes = 0
    R = N
    while R > 1:
        n = B * (R // 2) * C
        want_bytes += 2 * ((n + 31) // 32) * 4 + 2 * n * (bw // 8)
        R = R // 2 + (R & 1)
    assert by == want_bytes


def test_maxpool_keys_are_the_relu_gates(orc):
    """The pool's key is the sequence of the RELU gates of its levels: level l
    keyed under gate id gate + l on the mask differences r[2j+1] - r[2j]."""
    bw, B, N, C = 32, 2, 5, 3
    rng = np.random.default_rng(1)
    rin = mask_in(rng, B * N * C, bw)
    k0, k1, rout = orc.maxpool_keygen(9, 100, bw, S, B, N, C, rin)
    r = rin.reshape(B, N, C).astype(np.uint64)
    m = np.uint64(mod(bw))
    off, gate = 0, 100
    while r.shape[1] > 1:
        R = r.shape[1]
        d = ((r[:, 1:R - R % 2:2] - r[:, 0:R - R % 2:2]) & m).reshape(-1)
        g0, g1, gout = orc.tr_keygen(9, gate, 3, bw, S, d)
        assert np.array_equal(k0[off:off + g0.size], g0) and np.array_equal(k1[off:off + g1.size], g1)
        off += g0.size
        gate += 1
        nxt = (r[:, 0:R - R % 2:2] + gout.reshape(B, R // 2, C)) & m
        r = np.concatenate([nxt, r[:, R - 1:R]], axis=1) if R % 2 else nxt
    assert off == k0.size
    assert np.array_equal(r.reshape(-1), rout)


def local_ars_expected(x, r, bias, bw, s):
    """floor(x/2^s) + b + e - k 2^(bw-s) (mod 2^bw): e is the carry out of the low
    s bits of x + r, k the wrap of x + r (signed mask r) out of the signed ring."""
    h = 1 << (bw - 1)
    out = []
    for xi, ri, bi in zip(x.tolist(), to_signed(r, bw).tolist(), bias.tolist()):
        tot = xi + ri
        k = 1 if tot >= h else (-1 if tot < -h else 0)
        e = 1 if (xi % (1 << s)) + (ri % (1 << s)) >= (1 << s) else 0
        out.append(((xi >> s) + bi + e - k * (1 << (bw - s))) % (1 << bw))
    return np.array(out, dtype=np.uint64)


@pytest.mark.parametrize("bw", [32, 64])
def test_local_ars(orc, bw):
    """LocalARS (TruncateType::LocalARS, gpu_mpc/ddg_orca_batched.h:180-199): no key
    bytes, no exchange; the unmasked output is floor(x/2^s) + bias up to the carry
    of the low bits and the wrap of x + r, both counted here from their
    definitions (wraps included: |x| up to 2^(bw-3))."""
    rng = np.random.default_rng(bw + 1000)
    h = 1 << (bw - 1)
    x = np.concatenate([np.array([-h // 4, -1, 0, 1, (1 << S) - 1, -(1 << S)], np.int64),
                        rng.integers(-(h // 4), h // 4, size=4000, dtype=np.int64),
                        rng.integers(-8 << S, 8 << S, size=4000)])
    r = mask_in(rng, x.size, bw)
    bias = rng.integers(-(1 << 14), 1 << 14, size=x.size)
    k0, k1, rout = orc.tr_keygen(1, 1, 10, bw, S, r)
    assert k0.size == 0 and k1.size == 0
    full = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    xhat = (ring(x, bw) + r) & full
    y, by = orc.tr_eval(10, bw, S, k0, k1, xhat, bias)
    assert by == 0
    got = (y - rout) & full
    assert np.array_equal(got, local_ars_expected(x, r, bias, bw, S))
    wrapped = np.abs(x.astype(object) + to_signed(r, bw).astype(object)) >= h
    assert wrapped.any() and not wrapped.all()


@pytest.mark.parametrize("bw", [32, 64])
def test_drelu(orc, bw):
    """DReLU (gpuKeyGenDRelu, gpu_mpc/dpf_dcf_adapter.h:32-36, 330): the masked
    public bit XOR the dealer's mask bit is [x >= 0] over the signed ring, edges
    included; one bit plane each way, no ring message."""
    rng = np.random.default_rng(bw + 11)
    h = 1 << (bw - 1)
    x = np.concatenate([np.array([-h, -h + 1, -1, 0, 1, h - 1], np.int64),
                        rng.integers(-h, h, size=3000, dtype=np.int64),
                        rng.integers(-4, 4, size=500)])
    r = mask_in(rng, x.size, bw)
    k0, k1, rbit = orc.tr_keygen(4, 9, 11, bw, S, r)
    assert set(np.unique(rbit).tolist()) <= {0, 1}
    full = np.uint64(mod(bw) if bw < 64 else 0xFFFFFFFFFFFFFFFF)
    xhat = (ring(x, bw) + r) & full
    y, by = orc.tr_eval(11, bw, S, k0, k1, xhat)
    assert np.array_equal(y ^ rbit, (x >= 0).astype(np.uint64))
    assert by == 2 * ((x.size + 31) // 32) * 4
