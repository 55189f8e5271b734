"""The benchmarked configurations at their own sizes, through the C ABI.

- Config 3: bw=32, B=64 molecules x 140 atoms, every FSS key resident in HBM,
  three concurrent sub-batches (lanes), the forward captured into a HIP graph
  and replayed -- exactly what bench.py times.  The reference's resident-key
  loop is gpu_mpc/deepdtagen_inference.cu:476-559.
- Config 4: bw=64, one micro-batch of B=256 streamed from both parties'
  packed keys in pinned host memory through two 16 GiB device slots per party
  (bench.py --stream).  The reference's streamed loop is
  gpu_mpc/deepdtagen_inference.cu:608-859.

Outputs must equal the oracle's plaintext fixed-point forward bit for bit, and
the bytes exchanged must equal the oracle's two-party evaluation's count.
This file sorts before the slower parity suite so that both run early.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _od(orc, dims):
    return orc.make_dims(bw=dims.bw, s=dims.s, n_nodes=dims.n_nodes, feat=dims.feat, gcn=dims.gcn, dfc=dims.dfc,
                         prot=dims.prot, fus=dims.fus, lut_nmax=dims.lut_nmax, mask_scale=dims.mask_scale,
                         slack=dims.slack)


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def test_config3_resident_b64_three_lanes_graph(orc, synth):
    """bw=32, B=64, 3 lanes, graph replay: two replays of the same batch and a
    replay on a second batch are bit-exact; exchange bytes equal the sum of the
    oracle's two-party evaluations of the lanes' sub-batches on the lanes' key
    sets (which also reconstruct the plaintext outputs)."""
    import mpcx
    B, lanes, bw = 64, 3, 32
    dims = synth.Dims(bw=bw)
    wl = synth.workload(B, dims, seed=0)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0, orc.domain_msg(code)
    c = mpcx.Ctx(bw=bw)
    m = mpcx.Model(c, wl.dims, wl.W, lanes=lanes)
    seed = 0xC0FFEE
    m.keygen(B, seed)
    _say(f"[config3] keys {2 * m.key_bytes(B) / 1e9:.2f} GB resident")
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    c.reset_counters()
    m.forward(B)  # first forward: capture, then replay
    assert np.array_equal(m.output(B), want)
    got_bytes = c.bytes_exchanged
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    assert c.bytes_exchanged == 2 * got_bytes
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = wl.shares["m"]
    want_bytes = 0
    for i, (s0, n) in enumerate(mpcx.Model.lane_split(B, lanes)):
        k0, k1 = orc.model_keygen(d, n, mpcx.Model.lane_seed(seed, i), wl.W)
        sl = slice(s0, s0 + n)
        y, by = orc.model_eval(d, n, wl.W, k0, k1, x0[sl], x1[sl], a0[sl], a1[sl], m0[sl], m1[sl], wl.prot[sl])
        del k0, k1
        assert np.array_equal(y, want[sl])
        want_bytes += by
        _say(f"[config3] oracle lane {i}: {n} samples checked")
    assert got_bytes == want_bytes
    # a second batch on the same keys (inputs replaced under the captured graph)
    wl2 = synth.workload(B, dims, seed=1)
    want2, code = orc.plain_forward(d, wl2.X, wl2.A, wl2.mask, wl2.prot, wl.W)
    assert code == 0
    m.set_inputs(B, *wl2.shares["x"], *wl2.shares["a"], *wl2.shares["m"], wl2.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want2)
    m.close()
    c.close()


def test_config4_streamed_b256_bw64(orc, synth):
    """bw=64, one micro-batch of B=256 streamed from both parties' packed
    pinned keys through two 16 GiB device slots per party, two micro-batches in
    a row (fresh inputs, the same key set re-streamed); bit-exact.  Exchange
    bytes: every gate's element count at B=256 is a multiple of 32, so the
    count is 16x the oracle's two-party evaluation at B=16 (whose counts are
    too)."""
    import mpcx
    B, bw = 256, 64
    dims = synth.Dims(bw=bw)
    wls = [synth.workload(B, dims, seed=s) for s in (0, 100)]
    W = wls[0].W
    d = _od(orc, dims)
    wants = []
    for wl in wls:
        y, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, W)
        assert code == 0, orc.domain_msg(code)
        wants.append(y)
    c = mpcx.Ctx(bw=bw)
    m = mpcx.Model(c, dims, W)
    m.keygen(B, 0xBEEF)
    h0 = mpcx.PinnedBuffer(m.unique_key_bytes(B, 0))
    h1 = mpcx.PinnedBuffer(m.unique_key_bytes(B, 1))
    m.export_unique_keys(0, B, into=h0)
    m.export_unique_keys(1, B, into=h1)
    m.release_arena()
    _say(f"[config4] packed keys {(h0.nbytes + h1.nbytes) / 1e9:.1f} GB pinned")
    m.attach_host_keys(B, h0, h1, 16 << 30)
    byts = []
    for k, wl in enumerate(wls):
        m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
        c.reset_counters()
        m.forward(B)
        assert np.array_equal(m.output(B), wants[k])
        byts.append(c.bytes_exchanged)
        st = m.stream_stats()
        assert st["chunks"] >= 2 and st["bytes_h2d"] == h0.nbytes + h1.nbytes - 2 * 256
        _say(f"[config4] micro-batch {k}: bit-exact, {st['chunks']} chunks")
    m.close()
    c.close()
    h0.free()
    h1.free()
    assert byts[0] == byts[1]
    Bs = 16
    sl = slice(0, Bs)
    wl = wls[0]
    k0, k1 = orc.model_keygen(d, Bs, 7, W)
    sh = wl.shares
    y, by = orc.model_eval(d, Bs, W, k0, k1, sh["x"][0][sl], sh["x"][1][sl], sh["a"][0][sl], sh["a"][1][sl],
                           sh["m"][0][sl], sh["m"][1][sl], wl.prot[sl])
    assert np.array_equal(y, wants[0][sl])
    assert byts[0] == (B // Bs) * by


@pytest.mark.parametrize("bw", [32, 64])
def test_reference_model_dims_from_weights_file(orc, synth, tmp_path, bw):
    """The model at the dimensions the reference deploys (gpu_mpc/deepdtagen.h:
    12-31: 94 atom features, GCN 94-188-282-376, Nmax = 138, drug FCs 376-1024-128,
    fusion 256-1024-512-256-1), weights read back from a weights.bin written in
    the reference layout (reference/export_weights.py:38-75): the GPU dealer's keys
    reproduce the oracle's, and the forward equals the fixed-point forward."""
    import mpcx
    import formats
    B = 4
    dims = synth.Dims(bw=bw, n_nodes=138, feat=94, gcn=(188, 282, 376), dfc=(1024, 128), prot=128,
                      fus=(1024, 512, 256, 1))
    wl = synth.workload(B, dims, seed=5)
    wpath = str(tmp_path / "weights.bin")
    formats.write_weights(wpath, wl.W, dims.layers(), scale=12)
    W, layers, _ = formats.read_weights(wpath)
    assert layers == dims.layers() and np.array_equal(W, wl.W)
    d = _od(orc, dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, W)
    assert code == 0, orc.domain_msg(code)
    c = mpcx.Ctx(bw=bw)
    m = mpcx.Model(c, dims, W, lanes=2)
    m.keygen(B, 31)
    split = mpcx.Model.lane_split(B, 2)
    k0 = m.export_keys(0, B)
    o0, _ = orc.model_keygen(d, split[0][1], mpcx.Model.lane_seed(31, 0), W)
    assert np.array_equal(k0[:o0.size], o0)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    m.close()
    c.close()


@pytest.mark.parametrize("bw", [32, 64])
def test_dealer_key_bytes(orc, synth, bw):
    """A 16-byte dealer key (mpcx_set_dealer_key): the GPU dealer's keys equal
    the oracle dealer's under the same key bytes, differ from the seed-only keys
    of the same seed, and the forward stays bit-exact."""
    import mpcx
    B = 2
    wl = synth.workload(B, synth.Dims(bw=bw), seed=8)
    d = _od(orc, wl.dims)
    want, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    dk = bytes(range(200, 216))
    c = mpcx.Ctx(bw=bw)
    plain = mpcx.Model(c, wl.dims, wl.W)
    plain.keygen(B, 5)
    k_plain = plain.export_keys(0, B)
    plain.close()
    c.set_dealer_key(dk)
    m = mpcx.Model(c, wl.dims, wl.W)
    m.keygen(B, 5)
    got = [m.export_keys(p, B) for p in (0, 1)]
    try:
        orc.set_dealer_key(dk)
        o0, o1 = orc.model_keygen(d, B, 5, wl.W)
    finally:
        orc.set_dealer_key(None)
    assert np.array_equal(got[0], o0) and np.array_equal(got[1], o1)
    assert not np.array_equal(got[0], k_plain)
    m.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
    m.forward(B)
    assert np.array_equal(m.output(B), want)
    m.close()
    c.close()
