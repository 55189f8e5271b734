"""Party mode: one party per thread or per process, exchanging over a socket
(or, for two threads, an in-process pair linked in memory),
as the reference deploys the two parties (gpu_mpc/run_local_2pc.sh:196-233,
GpuPeer / SigmaPeer in gpu_mpc/utils/gpu_comms.h and sigma_comms.cpp).

Each party evaluates with its own key only and the peer's messages; the
reconstructed outputs must equal the one-process evaluation's (which the
parity suite checks against the oracle) and the plaintext function, and the
bytes that cross the channel must equal what mpcx_bytes_exchanged counts.
"""
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

S = 12


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


TRANSPORTS = ["local", "socket", "local-async"]


def two_parties(bw, fn, transport="local"):
    """Runs fn(ctx, peer, party) for both parties on two threads, each with its
    own context and one end of an in-process pair: linked in memory (device to
    device copies, "local"; "local-async": the party calls also return without
    synchronising the stream, mpcx_set_party_sync(ctx, 0)) or a socket pair
    staged through pinned host memory as between processes ("socket",
    MPCX_PEER_SOCKETPAIR=1); returns both results and the parties' counted and
    channel bytes."""
    import mpcx
    old = os.environ.get("MPCX_PEER_SOCKETPAIR")
    os.environ["MPCX_PEER_SOCKETPAIR"] = "1" if transport == "socket" else "0"
    try:
        p0, p1 = mpcx.Peer.pair(timeout_ms=30000)
    finally:
        if old is None:
            del os.environ["MPCX_PEER_SOCKETPAIR"]
        else:
            os.environ["MPCX_PEER_SOCKETPAIR"] = old
    ctxs = [mpcx.Ctx(bw=bw, scale=S) for _ in range(2)]
    if transport == "local-async":
        for c in ctxs:
            c.set_party_sync(False)

    def run(party):
        c = ctxs[party]
        c.reset_counters()
        out = fn(c, (p0, p1)[party], party)
        return out, c.bytes_exchanged

    with ThreadPoolExecutor(2) as ex:
        f = [ex.submit(run, p) for p in (0, 1)]
        res = [x.result(timeout=120) for x in f]
    wire = (p0.bytes, p1.bytes)
    assert p0.transport == p1.transport == (0 if transport == "socket" else 2)
    for c in ctxs:
        c.close()
    p0.close()
    p1.close()
    return res, wire


@pytest.mark.parametrize("transport", ["local", "socket"])
def test_peer_gone_or_silent(transport):
    """An exchange with a closed peer fails at once, and with a live peer that
    never exchanges fails after the pair's timeout; the channel reports why.
    Both are host-side conditions: the failing end enqueues no wait on the
    peer's events, so the context stays usable."""
    import time
    import mpcx
    old = os.environ.get("MPCX_PEER_SOCKETPAIR")
    os.environ["MPCX_PEER_SOCKETPAIR"] = "1" if transport == "socket" else "0"
    try:
        a0, a1 = mpcx.Peer.pair(timeout_ms=500)
        b0, b1 = mpcx.Peer.pair(timeout_ms=500)
    finally:
        if old is None:
            del os.environ["MPCX_PEER_SOCKETPAIR"]
        else:
            os.environ["MPCX_PEER_SOCKETPAIR"] = old
    c = mpcx.Ctx(bw=32, scale=S)
    v = np.arange(1000, dtype=np.uint32)
    try:
        a1.close()
        t0 = time.perf_counter()
        with pytest.raises(mpcx.MpcxError):
            c.party_reconstruct(a0, v)
        assert time.perf_counter() - t0 < 5
        t0 = time.perf_counter()
        with pytest.raises(mpcx.MpcxError):
            c.party_reconstruct(b0, v)  # b1 is open but never exchanges
        assert 0.3 < time.perf_counter() - t0 < 10
        c.sync()  # nothing left waiting on the stream
    finally:
        for p_ in (a0, b0, b1):
            p_.close()
        c.close()


TR_KINDS = [(3, "RELU"), (12, "TRMOD"), (1, "TR"), (2, "TRRELU"), (4, "TRSLACK"), (15, "RELUPOOL"), (11, "DRELU")]


@pytest.mark.parametrize("transport", TRANSPORTS)
@pytest.mark.parametrize("bw", [32, 64])
@pytest.mark.parametrize("kind,name", TR_KINDS)
def test_party_tr_gates(bw, kind, name, transport):
    """Every truncation / ReLU kind: the two parties' outputs are identical,
    equal to the one-process evaluation on the same keys, and the channel
    carried exactly the counted bytes."""
    import mpcx
    rng = np.random.default_rng(bw * 31 + kind)
    n = 5000 + kind  # not a multiple of 32 or 64: ragged last words of the bit planes
    if kind == 4:
        x = rng.integers(-(1 << (bw - 2)), 1 << (bw - 2), size=n, dtype=np.int64)
    elif kind == 15:
        x = rng.integers(-(1 << (bw - S)), 1 << (bw - S), size=n, dtype=np.int64)
    else:
        x = rng.integers(-(1 << (bw - 3)), 1 << (bw - 3), size=n, dtype=np.int64)
    bias = rng.integers(-(1 << 10), 1 << 10, size=13) if kind in (1, 2, 12) else None
    rin = rmask(rng, n, bw)
    d = mpcx.Ctx(bw=bw, scale=S)
    k0, k1, rout = d.tr_keygen(kind, rin, seed=9, gate=5)
    xhat = (x.astype(np.uint64) + rin) & M(bw)
    d.reset_counters()
    want = d.tr_eval(kind, k0, k1, xhat, bias)
    want_bytes = d.bytes_exchanged
    (r0, r1), wire = two_parties(bw, lambda c, pe, p: c.party_tr_eval(pe, kind, (k0, k1)[p], xhat, bias), transport)
    assert np.array_equal(r0[0], want) and np.array_equal(r1[0], want)
    assert r0[1] == r1[1] == want_bytes
    assert wire[0] == wire[1] == want_bytes
    if kind == 12:
        # TRMOD's output is known modulo 2^(bw-s): revealed, and sent, at bw-s
        # bits per element packed in 64-bit words (gpu_mpc/utils/gpu_comms.h:143-168)
        assert want_bytes == 2 * (((n + 31) // 32) * 4 + ((n * (bw - S) + 63) // 64) * 8)
        assert np.all(want.astype(np.uint64) < np.uint64(1 << (bw - S)))
        exp = (x + (np.resize(bias, n) << S)) >> S
        low = np.uint64((1 << (bw - S)) - 1)
        assert np.array_equal((want.astype(np.uint64) - rout.astype(np.uint64)) & low,
                              exp.astype(np.uint64) & low)
    if kind == 11:  # DRELU: the masked public bit
        assert np.array_equal((want.astype(np.uint64) ^ rout.astype(np.uint64)) & np.uint64(1),
                              (x >= 0).astype(np.uint64))
    elif kind in (3, 15):
        assert np.array_equal(signed(want.astype(np.uint64) - rout.astype(np.uint64), bw), np.maximum(x, 0))
    d.close()


@pytest.mark.parametrize("transport", TRANSPORTS)
@pytest.mark.parametrize("bw", [32, 64])
def test_party_split_truncation_chain(bw, transport):
    """TRMOD (with a bias) then EXTRELU, party by party: the exact ReLU of the
    floor, as the one-process chain."""
    import mpcx
    rng = np.random.default_rng(bw + 3)
    n = 3001
    x = rng.integers(-(1 << (bw - 3)), 1 << (bw - 3), size=n, dtype=np.int64)
    bias = rng.integers(-(1 << 10), 1 << 10, size=7)
    rin = rmask(rng, n, bw)
    d = mpcx.Ctx(bw=bw, scale=S)
    g0, g1, r1 = d.tr_keygen(12, rin, seed=2, gate=1)
    q0, q1, r2 = d.tr_keygen(14, r1, seed=2, gate=2)
    xhat = (x.astype(np.uint64) + rin) & M(bw)

    def fn(c, pe, p):
        y = c.party_tr_eval(pe, 12, (g0, g1)[p], xhat, bias)
        return c.party_tr_eval(pe, 14, (q0, q1)[p], y)

    (a, b), wire = two_parties(bw, fn, transport)
    assert np.array_equal(a[0], b[0])
    want = np.maximum((x + (np.resize(bias, n) << S)) >> S, 0)
    assert np.array_equal(signed(a[0].astype(np.uint64) - r2.astype(np.uint64), bw), want)
    assert wire[0] == a[1]
    d.close()


@pytest.mark.parametrize("transport", TRANSPORTS)
@pytest.mark.parametrize("bw", [32, 64])
def test_party_mul_lut_sxs_reveal(bw, transport):
    """Beaver product, 8-bit DPF table, batched secret x secret GEMM, reveal and
    reconstructInPlace, party by party, against the one-process calls."""
    import mpcx
    rng = np.random.default_rng(bw)
    d = mpcx.Ctx(bw=bw, scale=S)
    # Beaver product with index maps
    nx, ny, nz = 300, 200, 4001
    xv = rng.integers(-(1 << 14), 1 << 14, size=nx)
    yv = rng.integers(-(1 << 14), 1 << 14, size=ny)
    ia = rng.integers(0, nx, size=nz).astype(np.uint32)
    ib = rng.integers(0, ny, size=nz).astype(np.uint32)
    rx, ry = rmask(rng, nx, bw), rmask(rng, ny, bw)
    m0, m1, rz = d.mul_keygen(rx, ry, ia, ib, seed=2, gate=4)
    xh = (xv.astype(np.uint64) + rx) & M(bw)
    yh = (yv.astype(np.uint64) + ry) & M(bw)
    # LUT8
    table = np.zeros(256, np.int64)
    table[1:139] = np.round(4096.0 / np.sqrt(np.arange(1, 139)))
    lx = np.tile(np.arange(256, dtype=np.uint64), 3)
    lin = rmask(rng, lx.size, bw)
    l0, l1, lout = d.lut8_keygen(lin, seed=4, gate=6)
    # SxS
    nb, Mm, K, N = 2, 37, 70, 29
    A = rng.integers(-(1 << 10), 1 << 10, size=(nb, Mm, K))
    Bm = rng.integers(-(1 << 10), 1 << 10, size=(nb, K, N))
    ra, rb = rmask(rng, A.size, bw), rmask(rng, Bm.size, bw)
    s0, s1, rc = d.sxs_keygen(nb, Mm, K, N, ra, rb, seed=3, gate=2)
    ah = (A.ravel().astype(np.uint64) + ra) & M(bw)
    bh = (Bm.ravel().astype(np.uint64) + rb) & M(bw)
    # reveal of additive shares
    n = 777
    e0, e1, em = d.reveal_keygen(n, seed=1, gate=3)
    v = rng.integers(-1000, 1000, size=n)
    v0 = rmask(rng, n, bw)
    v1 = (v.astype(np.uint64) - v0) & M(bw)

    def fn(c, pe, p):
        return (c.party_mul_eval(pe, (m0, m1)[p], xh, yh, ia, ib),
                c.party_lut8_eval(pe, (l0, l1)[p], table, (lx + lin) & M(bw)),
                c.party_sxs_eval(pe, nb, Mm, K, N, (s0, s1)[p], ah, bh),
                c.party_reveal_eval(pe, (e0, e1)[p], (v0, v1)[p]),
                c.party_reconstruct(pe, (v0, v1)[p]))

    (a, b), wire = two_parties(bw, fn, transport)
    for u, w in zip(a[0], b[0]):
        assert np.array_equal(u, w)
    z, ly, cc, vh, vs = a[0]
    assert np.array_equal(signed(z.astype(np.uint64) - rz.astype(np.uint64), bw), xv[ia] * yv[ib])
    assert np.array_equal((ly.astype(np.uint64) - lout.astype(np.uint64)) & M(bw),
                          table[lx.astype(np.int64)].astype(np.uint64))
    assert np.array_equal(signed(cc.astype(np.uint64) - rc.astype(np.uint64), bw).reshape(nb, Mm, N),
                          np.einsum("bmk,bkn->bmn", A, Bm))
    assert np.array_equal(signed(vh.astype(np.uint64) - em.astype(np.uint64), bw), v)
    assert np.array_equal(signed(vs, bw), v)
    elem = bw // 8
    assert a[1] == b[1] == wire[0] == wire[1] == 2 * elem * (nz + 2 * lx.size + nb * Mm * N + 2 * n)
    d.close()


def _od(orc, dims):
    return orc.make_dims(bw=dims.bw, s=dims.s, n_nodes=dims.n_nodes, feat=dims.feat, gcn=dims.gcn, dfc=dims.dfc,
                         prot=dims.prot, fus=dims.fus, lut_nmax=dims.lut_nmax, mask_scale=dims.mask_scale,
                         slack=dims.slack)


@pytest.mark.parametrize("transport", TRANSPORTS)
@pytest.mark.parametrize("bw", [32, 64])
def test_model_party_threads(orc, synth, bw, transport):
    """The affinity forward with the two parties as two threads: each holds its
    key (exported from the dealer's run) and its input shares, party 1 the
    protein embedding; both get the plaintext outputs, and each party counts,
    and its channel carries, the one-process run's exchange bytes."""
    import mpcx
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw), seed=41)
    want, code = orc.plain_forward(_od(orc, wl.dims), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    dc = mpcx.Ctx(bw=bw)
    dm = mpcx.Model(dc, wl.dims, wl.W)
    dm.keygen(B, 99)
    keys = [dm.export_keys(p, B) for p in (0, 1)]
    dm.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    dc.reset_counters()
    dm.forward(B)
    assert np.array_equal(dm.output(B), want)
    one_bytes = dc.bytes_exchanged
    dm.close()
    dc.close()
    sh = wl.shares

    def fn(c, pe, p):
        m = mpcx.Model(c, wl.dims, wl.W)
        m.set_party(pe)
        m.import_party_key(B, keys[p])
        m.set_party_inputs(B, sh["x"][p], sh["a"][p], sh["m"][p], wl.prot if p == 1 else None)
        outs = []
        for _ in range(2):  # two forwards on the same keys
            m.forward(B)
            outs.append(m.output(B))
        m.close()
        return outs

    (a, b), wire = two_parties(bw, fn, transport)
    for outs in (a[0], b[0]):
        for o in outs:
            assert np.array_equal(o, want)
    assert a[1] == b[1] == 2 * one_bytes
    assert wire[0] == wire[1] == 2 * one_bytes


@pytest.mark.parametrize("transport", ["ipc", "socket"])
@pytest.mark.parametrize("bw", [32, 64])
def test_driver_two_processes(orc, synth, tmp_path, bw, transport):
    """The reference's deployment: the dealer run writes both parties' key
    files, then two evaluator processes (mpcx_infer role 3, party 0 and party 1)
    each read their own key file and share files and exchange over a Unix
    socket; both print the plaintext affinities, and the same Comm (B) as the
    one-process evaluator, which is also what crossed each party's channel:
    through device inboxes shared by IPC handles (the default for two
    processes on one GPU) or staged through the socket (MPCX_PEER_IPC=0)."""
    import mpcx
    import formats
    exe = os.path.join(os.path.dirname(mpcx.__file__), "mpcx_infer")
    assert os.path.exists(exe), "mpcx_infer not built"
    B = 3
    wl = synth.workload(B, synth.Dims(bw=bw), seed=15)
    bdir, kdir = tmp_path / "batch", tmp_path / "keys"
    kdir.mkdir()
    formats.write_batch(str(bdir), wl.X, wl.A, wl.mask, wl.prot, bw=bw, scale=12, pool_dim=312, seed=7)
    wpath = str(tmp_path / "weights.bin")
    formats.write_weights(wpath, wl.W, wl.dims.layers(), scale=12)
    want, code = orc.plain_forward(_od(orc, synth.Dims(bw=bw)), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    lines = [f"AFFINITY[{j}]={v / 4096.0:.6f}" for j, v in enumerate(want)]
    env = dict(os.environ, MPCX_WEIGHTS_BIN=wpath)
    args = [exe, str(bw), "12"]
    r = subprocess.run(args + ["0", str(kdir), str(bdir)], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run(args + ["1", str(kdir), str(bdir)], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    one_comm = int(re.search(r"Comm \(B\)=(\d+)", r.stdout).group(1))
    sock = str(tmp_path / "peer.sock")
    print(f"[two-process] bw={bw}: starting party 0 and party 1 on {sock}", file=sys.stderr, flush=True)
    penv = dict(env, MPCX_PEER_IPC="1" if transport == "ipc" else "0")
    procs = [subprocess.Popen(args + ["3", str(kdir), str(bdir)], env=dict(penv, MPCX_PARTY=str(p), MPCX_PEER=sock),
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True) for p in (0, 1)]
    outs = []
    for p in procs:
        try:
            o, e = p.communicate(timeout=120)
        except subprocess.TimeoutExpired:
            for q in procs:
                q.kill()
            raise
        assert p.returncode == 0, e
        outs.append(o)
    for o in outs:
        assert re.findall(r"AFFINITY\[\d+\]=\S+", o) == lines
        assert int(re.search(r"Comm \(B\)=(\d+)", o).group(1)) == one_comm
        assert int(re.search(r"Peer \(B\)=(\d+)", o).group(1)) == one_comm
        assert re.search(r"Peer transport=(\w+)", o).group(1) == transport
