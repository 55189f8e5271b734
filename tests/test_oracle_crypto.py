"""Pins the oracle's cryptographic building blocks (CPU only).

AES-128: FIPS-197 Appendix B and C.1 vectors (C.1 is also the KAT of the
reference's gpu_mpc/lss/lss_test.cpp:52-70), key expansion vs FIPS-197 A.1.
DCF / DPF: exhaustive closed forms ([x < alpha], one-hot) on small domains and
boundary cases on the 31/63-bit domains the protocol uses.
"""
import numpy as np
import pytest

FIPS_C1_KEY = bytes(range(16))
FIPS_C1_PT = bytes.fromhex("00112233445566778899aabbccddeeff")
FIPS_C1_CT = "69c4e0d86a7b0430d8cdb78070b4c55a"
FIPS_B_KEY = bytes.fromhex("2b7e151628aed2a6abf7158809cf4f3c")
FIPS_B_PT = bytes.fromhex("3243f6a8885a308d313198a2e0370734")
FIPS_B_CT = "3925841d02dc09fbdc118597196a0b32"


@pytest.mark.parametrize("portable", [0, 1])
def test_aes_fips197_vectors(orc, portable):
    orc.lib().orc_aes_force_portable(portable)
    try:
        assert orc.aes_encrypt(FIPS_C1_KEY, FIPS_C1_PT).hex() == FIPS_C1_CT
        assert orc.aes_encrypt(FIPS_B_KEY, FIPS_B_PT).hex() == FIPS_B_CT
    finally:
        orc.lib().orc_aes_force_portable(0)


def test_aes_key_expansion_last_round(orc):
    # FIPS-197 A.1: w40..w43 = d014f9a8 c9ee2589 e13f0cc8 b6630ca6
    rk = np.zeros(176, np.uint8)
    k = np.frombuffer(FIPS_B_KEY, np.uint8).copy()
    orc.lib().orc_aes_expand(orc.ptr(k), orc.ptr(rk))
    assert rk[160:176].tobytes().hex() == "d014f9a8c9ee2589e13f0cc8b6630ca6"


def test_aes_backends_agree(orc):
    rng = np.random.default_rng(5)
    for _ in range(50):
        key = rng.bytes(16)
        pt = rng.bytes(16)
        orc.lib().orc_aes_force_portable(1)
        a = orc.aes_encrypt(key, pt)
        orc.lib().orc_aes_force_portable(0)
        assert orc.aes_encrypt(key, pt) == a


def _blk_bytes(b):
    return np.asarray(b, np.uint32).astype("<u4").tobytes()


def test_hash_definition(orc):
    """H(s) = AES_KH(sigma(s)) ^ sigma(s), sigma(xL||xR) = (xL^xR)||xL."""
    rng = np.random.default_rng(1)
    s = rng.integers(0, 2**32, size=(8, 4), dtype=np.uint64).astype(np.uint32)
    for leaf, key in ((0, b"MI355X-HalfTreeH"), (1, b"MI355X-HalfTreeL")):
        h = orc.hash_blocks(s, leaf=bool(leaf))
        for i in range(s.shape[0]):
            w = s[i]
            sig = np.array([w[2], w[3], w[2] ^ w[0], w[3] ^ w[1]], np.uint32)
            ct = np.frombuffer(orc.aes_encrypt(key, _blk_bytes(sig)), "<u4")
            assert np.array_equal(h[i], ct ^ sig)


def test_prf_is_aes_of_counter(orc):
    seed = 0x1234
    out = orc.prf_blocks(seed, 7, 0x30, 5)
    key = seed.to_bytes(8, "little") + (seed ^ 0x9E3779B97F4A7C15).to_bytes(8, "little")
    for i in range(5):
        blk = np.array([i, 0, 0x30, 7], np.uint32)
        assert np.array_equal(out[i], np.frombuffer(orc.aes_encrypt(key, _blk_bytes(blk)), "<u4"))


def test_prf_under_dealer_key(orc):
    """With the dealer's 16 secret bytes set, the PRF key of a key set is AES
    under those bytes of (seed lo, seed hi, 0x4D415354, 0xFFFFFFFE); the PRF
    blocks change with the key bytes at a fixed seed, and return to the
    seed-only ones when the key is cleared."""
    seed, dk = 0x1234, bytes(range(100, 116))
    plain = orc.prf_blocks(seed, 7, 0x30, 5)
    try:
        orc.set_dealer_key(dk)
        out = orc.prf_blocks(seed, 7, 0x30, 5)
        kset = orc.aes_encrypt(dk, _blk_bytes(np.array([seed, 0, 0x4D415354, 0xFFFFFFFE], np.uint32)))
        for i in range(5):
            blk = np.array([i, 0, 0x30, 7], np.uint32)
            assert np.array_equal(out[i], np.frombuffer(orc.aes_encrypt(kset, _blk_bytes(blk)), "<u4"))
        assert not np.array_equal(out, plain)
        orc.set_dealer_key(bytes(range(101, 117)))
        assert not np.array_equal(orc.prf_blocks(seed, 7, 0x30, 5), out)
    finally:
        orc.set_dealer_key(None)
    assert np.array_equal(orc.prf_blocks(seed, 7, 0x30, 5), plain)


@pytest.mark.parametrize("m", [1, 3, 6, 7, 8, 9, 11])
def test_dcf_exhaustive_small(orc, m):
    rng = np.random.default_rng(m)
    N = 1 << m
    x = np.arange(N, dtype=np.uint64)
    alphas = {0, N - 1, N // 2} | set(int(a) for a in rng.integers(0, N, size=3))
    for alpha in sorted(alphas):
        rb = rng.integers(0, 2, size=N).astype(np.uint8)
        k0, k1 = orc.dcf_keygen(7, 3 + alpha, m, np.full(N, alpha, np.uint64), rbit=rb)
        out = orc.dcf_eval(0, m, k0, x) ^ orc.dcf_eval(1, m, k1, x)
        assert np.array_equal(out, (x < alpha).astype(np.uint8) ^ rb), (m, alpha)


@pytest.mark.parametrize("m", [12, 31, 63])
def test_dcf_wide_boundaries(orc, m):
    rng = np.random.default_rng(100 + m)
    top = (1 << m) - 1
    alphas = np.array([0, 1, top, top - 1, 1 << (m - 1)] + list(rng.integers(0, top, size=11, dtype=np.uint64)),
                      np.uint64)
    xs, als = [], []
    for a in alphas:
        a = int(a)
        for x in (0, 1, top, a, a - 1, a + 1, int(rng.integers(0, top, dtype=np.uint64))):
            if 0 <= x <= top:
                xs.append(x)
                als.append(a)
    xs = np.array(xs, np.uint64)
    als = np.array(als, np.uint64)
    k0, k1 = orc.dcf_keygen(11, 5, m, als)
    out = orc.dcf_eval(0, m, k0, xs) ^ orc.dcf_eval(1, m, k1, xs)
    assert np.array_equal(out, (xs < als).astype(np.uint8))


def test_dcf_single_key_share_looks_balanced(orc):
    """Each party's output alone is not the comparison (it is masked by the
    other share): both values occur for a fixed alpha."""
    m, N = 12, 4096
    k0, _ = orc.dcf_keygen(3, 9, m, np.full(N, 1000, np.uint64))
    b0 = orc.dcf_eval(0, m, k0, np.arange(N, dtype=np.uint64))
    assert 0.2 < b0.mean() < 0.8
