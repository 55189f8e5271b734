"""Pins the oracle's plaintext fixed-point forward and its two-party protocol
(CPU only).

- A_hat closed form: A[i,j]*floor(T[d_i]T[d_j]/2^12) with the hand-checkable
  degree pairs of gpu_mpc/secure_adj_norm.h:138-184,326-365.
- a 2-node model whose every intermediate is computed by hand below (floor
  rounding of a negative product included), following the op order of
  reference/fixed_forward.py:63-95;
- node-permutation invariance and padding invariance (exact);
- agreement with an independent float64 forward of the same network;
- bw=32 and bw=64 agree when nothing wraps (microbench/test_ring32.py:57-66);
- the two-party protocol reconstructs exactly the plaintext outputs.
"""
import numpy as np
import pytest


def test_adj_norm_degree_pairs(orc):
    # graph with nodes of degree (incl. self loop) 1..5 connected as needed
    cases = {(1, 1): 4096, (2, 2): 2047, (2, 3): 1672, (3, 3): 1365, (3, 5): 1057, (4, 4): 1024,
             (5, 5): 819}
    t = orc.invsqrt_table(12, 138)
    for (da, db), want in cases.items():
        assert (int(t[da]) * int(t[db])) >> 12 == want
    # a path 0-1-2 with self loops: degrees 2,3,2
    A = np.zeros((1, 4, 4), np.int64)
    for i, j in ((0, 1), (1, 2)):
        A[0, i, j] = A[0, j, i] = 1
    for v in range(3):
        A[0, v, v] = 1
    Ah = orc.adj_norm_plain(A)[0]
    assert Ah[0, 0] == 2047 and Ah[0, 1] == 1672 and Ah[1, 1] == 1365 and Ah[2, 1] == 1672
    assert Ah[3].sum() == 0 and Ah[:, 3].sum() == 0 and Ah[0, 2] == 0


def _tiny(orc):
    d = orc.make_dims(bw=32, s=12, n_nodes=2, feat=1, gcn=(1, 1, 1), dfc=(1, 1), prot=1, fus=(1, 1))
    W = np.array([
        8192, 2048,      # gcn0: W=2.0, b=0.5
        8192, 2048,      # gcn1
        8192, 2048,      # gcn2
        2048, -4096,     # dfc0: W=0.5, b=-1.0
        -4096, 1024,     # dfc1: W=-1.0, b=0.25
        4096, 4096, 0,   # fus0: W^T=[[1],[1]], b=0
        -8193, 512,      # fus1: W=-2.000244, b=0.125
    ], np.int64)
    assert W.size == orc.weights_len(d)
    X = np.array([[[4096], [0]]], np.int64)
    A = np.array([[[1, 0], [0, 0]]], np.int64)
    mask = np.array([[1, 0]], np.int64)
    prot = np.array([[32768]], np.int64)
    return d, W, X, A, mask, prot


def test_hand_computed_two_node_model(orc):
    """Real atom: H = 2.5, 5.5, 11.5 after the GCNs (A_fx[0,0] = 4096);
    padding atom: H = ReLU(b) = 0.5 (masked out of the pool).
    dfc0: floor(47104*2048/4096) - 4096 = 19456; dfc1: -19456 + 1024 = -18432;
    fus0: floor((-18432 + 32768)*4096/4096) = 14336;
    fus1: floor(14336*-8193/4096) = floor(-28675.5) = -28676, + 512 = -28164."""
    d, W, X, A, mask, prot = _tiny(orc)
    out, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 0
    assert out.tolist() == [-28164]


def _path3(orc):
    """3-node path graph 0-1-2 with self loops (degrees 2, 3, 2), one feature,
    every layer one channel wide. GCN-1 W = 6145 (1.500244), every other weight
    4096 (1.0) or, for the fusion layer, [4096, 8192] on [drug, protein];
    all biases zero; public protein value 1000."""
    d = orc.make_dims(bw=32, s=12, n_nodes=3, feat=1, gcn=(1, 1, 1), dfc=(1, 1), prot=1, fus=(1, 1))
    W = np.array([
        6145, 0,         # gcn0
        4096, 0,         # gcn1
        4096, 0,         # gcn2
        4096, 0,         # dfc0
        4096, 0,         # dfc1
        4096, 8192, 0,   # fus0: W^T = [[1.0], [2.0]] on [drug, protein]
        4096, 0,         # fus1
    ], np.int64)
    assert W.size == orc.weights_len(d)
    A = np.zeros((1, 3, 3), np.int64)
    for i, j in ((0, 0), (1, 1), (2, 2), (0, 1), (1, 0), (1, 2), (2, 1)):
        A[0, i, j] = 1
    X = np.array([[[4097], [-3], [1]]], np.int64)
    mask = np.ones((1, 3), np.int64)
    prot = np.array([[1000]], np.int64)
    return d, W, X, A, mask, prot


def _path3_ints(order):
    """The same forward in Python integers, GCN layers either transform-first
    tr(A.tr(H.W)) or aggregate-first tr(tr(A.H).W); returns (pooled, output)."""
    Af = [[2047, 1672, 0], [1672, 1365, 1672], [0, 1672, 2047]]
    H = [4097, -3, 1]
    for w in (6145, 4096, 4096):
        if order == "transform":
            XW = [(h * w) >> 12 for h in H]
            agg = [sum(Af[i][j] * XW[j] for j in range(3)) >> 12 for i in range(3)]
        else:
            AH = [sum(Af[i][j] * H[j] for j in range(3)) >> 12 for i in range(3)]
            agg = [(a * w) >> 12 for a in AH]
        H = [max(a, 0) for a in agg]
    pooled = max(H)
    h = max((pooled * 4096) >> 12, 0)
    drug = (h * 4096) >> 12
    fus = max((drug * 4096 + 1000 * 8192) >> 12, 0)
    return pooled, (fus * 4096) >> 12


def test_gcn_order_is_transform_first(orc):
    """reference/fixed_forward.py:63-67 runs each GCN layer transform-first,
    H' = ReLU(tr(A_fx . tr(H . W^T)) + b); the C++ path aggregates first
    (gpu_mpc/gcn_layer.h:113-114). On the path graph the two orders differ
    by one LSB. By hand, A_fx = [[2047,1672,0],[1672,1365,1672],[0,1672,2047]]
    (degree pairs (2,2), (2,3), (3,3)), X = [4097, -3, 1], >> is floor:
      layer 1: H.W = [25176065, -18435, 6145] >> 12 = [6146, -5, 1]
               (6146.5, -4.5, 1.5 before the floor);
               A.XW = [12572502, 10270959, -6313] >> 12 = [3069, 2507, -2];
               ReLU -> [3069, 2507, 0]
      layer 2 (W = 1.0, so XW = H): A.XW = [10473947, 8553423, 4191704] >> 12
               = [2557, 2088, 1023]
      layer 3: A.XW = [8725315, 8835880, 5585217] >> 12 = [2130, 2157, 1363];
               pooled max = 2157.
    Aggregate-first: A.X = [8381543, 6847761, -2969] >> 12 = [2046, 1671, -1],
    times 6145 = [12572670, 10268295, -6145] >> 12 = [3069, 2506, -2]; the
    next layers give [2556, 2087, 1022] and [2129, 2156, 1362]: pooled 2156.
    Drug FCs (1.0, no bias) keep 2157; fusion [drug, protein] . [1.0, 2.0]
    = 2157 + 2000 = 4157 (the swapped concat order would give 5314); the
    last layer (1.0) outputs 4157."""
    assert _path3_ints("transform") == (2157, 4157)
    assert _path3_ints("aggregate") == (2156, 4156)
    d, W, X, A, mask, prot = _path3(orc)
    out, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 0
    assert out.tolist() == [4157]
    # the C++ layers' order (orc_dims.gcn_order = 1) gives the aggregate-first 4156
    d.gcn_order = 1
    out, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 0 and out.tolist() == [4156]
    d.gcn_order = 0
    # the two-party protocol reconstructs the same value
    k0, k1 = orc.model_keygen(d, 1, 7, W)
    rng = np.random.default_rng(3)
    shares = []
    for v in (X, A, mask):
        v0 = rng.integers(0, 1 << 32, size=v.size, dtype=np.uint64)
        shares += [v0, (v.ravel().astype(np.uint64) - v0) & np.uint64(0xFFFFFFFF)]
    out2, _ = orc.model_eval(d, 1, W, k0, k1, *shares, prot)
    assert out2.tolist() == [4157]


def test_hand_computed_two_party(orc):
    d, W, X, A, mask, prot = _tiny(orc)
    k0, k1 = orc.model_keygen(d, 1, 99, W)
    rng = np.random.default_rng(0)
    shares = []
    for v in (X, A, mask):
        v0 = rng.integers(0, 1 << 32, size=v.size, dtype=np.uint64)
        shares += [v0, (v.ravel().astype(np.uint64) - v0) & np.uint64(0xFFFFFFFF)]
    out, _ = orc.model_eval(d, 1, W, k0, k1, *shares, prot)
    assert out.tolist() == [-28164]


def test_domain_violation_is_reported(orc):
    d, W, X, A, mask, prot = _tiny(orc)
    W = W.copy()
    W[0] = 1 << 30  # XW product 4096 * 2^30 overflows the 32-bit ring
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 1
    assert "pre-truncation" in orc.domain_msg(code)


def test_slack_domain_violation_is_reported(orc):
    """With slack truncation of the GCN products the bit-exact domain of H.W^T
    is |x| < 2^(bw-2): a product of 2^30 is outside it (code 7) but inside the
    exact truncation's (the first violation, if any, comes later)."""
    d, W, X, A, mask, prot = _tiny(orc)
    W = W.copy()
    W[0] = 1 << 18  # XW product 4096 * 2^18 = 2^30
    d.slack = 1
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 7 and "slack" in orc.domain_msg(code)
    d.slack = 0
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code != 7
    W[0] = (1 << 18) - 1  # just inside the half ring
    d.slack = 1
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code != 7


def test_slack2_aggregation_domain_is_reported(orc):
    """slack = 2 also needs |A.XW + b 2^s| < 2^(bw-2): a bias that pushes the
    aggregation of the first layer past it gives code 8 (and not under slack 1)."""
    d, W, X, A, mask, prot = _tiny(orc)
    W = W.copy()
    W[1] = (1 << 18)  # gcn0 bias: b*2^s = 2^30
    d.slack = 2
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code == 8 and "aggregation" in orc.domain_msg(code)
    d.slack = 1
    _, code = orc.plain_forward(d, X, A, mask, prot, W)
    assert code != 8


def _wl(synth, B, bw=32, seed=0, n_nodes=140, slack=0):
    dims = synth.Dims(bw=bw, n_nodes=n_nodes, slack=slack)
    return synth.workload(B, dims, seed=seed)


def _od(orc, wl):
    d = wl.dims
    return orc.make_dims(bw=d.bw, s=d.s, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                         fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale, slack=d.slack)


def test_permutation_invariance(orc, synth):
    wl = _wl(synth, 3, seed=4)
    d = _od(orc, wl)
    out, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    rng = np.random.default_rng(1)
    X, A, M = wl.X.copy(), wl.A.copy(), wl.mask.copy()
    for b in range(3):
        p = rng.permutation(wl.dims.n_nodes)
        X[b] = wl.X[b][p]
        A[b] = wl.A[b][p][:, p]
        M[b] = wl.mask[b][p]
    out2, code2 = orc.plain_forward(d, X, A, M, wl.prot, wl.W)
    assert code2 == 0 and np.array_equal(out, out2)


def test_padding_invariance(orc, synth):
    wl = _wl(synth, 2, seed=6)
    d = _od(orc, wl)
    out, _ = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    n = 64  # every molecule has <= 60 real atoms
    d2 = orc.make_dims(bw=32, n_nodes=n)
    out2, code = orc.plain_forward(d2, wl.X[:, :n], wl.A[:, :n, :n], wl.mask[:, :n], wl.prot, wl.W)
    assert code == 0 and np.array_equal(out, out2)


def _float_forward(wl):
    """Independent float64 forward of the same network (dequantised weights)."""
    dims = wl.dims
    s = float(1 << dims.s)
    layers = []
    o = 0
    for fin, fout in dims.layers():
        Wt = wl.W[o:o + fin * fout].reshape(fin, fout) / s
        o += fin * fout
        b = wl.W[o:o + fout] / s
        o += fout
        layers.append((Wt, b))
    outs = []
    for bi in range(wl.B):
        A = wl.A[bi].astype(float)
        deg = A.sum(1)
        inv = np.where(deg > 0, 1.0 / np.sqrt(np.maximum(deg, 1)), 0.0)
        Ah = inv[:, None] * A * inv[None, :]
        H = wl.X[bi] / s
        for l in range(3):
            Wt, b = layers[l]
            H = np.maximum(Ah @ (H @ Wt) + b, 0)
        keep = wl.mask[bi] != 0
        p = H[keep].max(0)
        Wt, b = layers[3]
        h = np.maximum(p @ Wt + b, 0)
        Wt, b = layers[4]
        h = np.concatenate([h @ Wt + b, wl.prot[bi] / s])
        for k in range(len(dims.fus)):
            Wt, b = layers[5 + k]
            h = h @ Wt + b
            if k < len(dims.fus) - 1:
                h = np.maximum(h, 0)
        outs.append(h[0])
    return np.array(outs)


def test_close_to_float_model(orc, synth):
    wl = _wl(synth, 6, seed=2)
    d = _od(orc, wl)
    out, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    ref = _float_forward(wl)
    fx = out / 4096.0
    assert np.abs(fx - ref).max() < 0.05, (fx, ref)
    assert np.ptp(ref) > 0.1  # outputs are not degenerate


def test_bw32_equals_bw64_in_domain(orc, synth):
    wl = _wl(synth, 3, seed=8)
    o32, c32 = orc.plain_forward(_od(orc, wl), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    o64, c64 = orc.plain_forward(orc.make_dims(bw=64), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert c32 == 0 and c64 == 0 and np.array_equal(o32, o64)


@pytest.mark.parametrize("bw,slack", [(32, 0), (64, 0), (32, 1), (64, 1), (32, 2), (64, 2)])
def test_two_party_matches_plaintext(orc, synth, bw, slack):
    """Two-party evaluation reconstructs the plaintext forward, with exact and
    with slack truncation of the GCN products (in the slack domain)."""
    wl = _wl(synth, 2, bw=bw, seed=10, slack=slack)
    d = _od(orc, wl)
    out, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    k0, k1 = orc.model_keygen(d, 2, 2024, wl.W)
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = wl.shares["m"]
    o2, by = orc.model_eval(d, 2, wl.W, k0, k1, x0, x1, a0, a1, m0, m1, wl.prot)
    assert np.array_equal(o2, out)
    assert by > 0


@pytest.mark.parametrize("bw,ms", [(32, 12), (32, 19), (32, 20), (32, 25), (64, 51), (64, 55)])
def test_two_party_mask_scales(orc, synth, bw, ms):
    """Atom masks 0 / 2^ms: up to ms = bw-s-1 the max-pool takes the narrow
    sentinel -2^(bw-s-1) and RELUPOOL gates, above it the reference's sentinel
    -2^(bw-2) and RELU gates (a larger key); both reconstruct the plaintext forward,
    whose own sentinel is always -2^(bw-2)."""
    dims = synth.Dims(bw=bw, n_nodes=140, mask_scale=ms)
    wl = synth.workload(2, dims, seed=12)
    d = _od(orc, wl)
    mask = wl.mask << ms
    out, code = orc.plain_forward(d, wl.X, wl.A, mask, wl.prot, wl.W)
    assert code == 0
    k0, k1 = orc.model_keygen(d, 2, 99, wl.W)
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = synth.share(mask, bw, 5)
    o2, _ = orc.model_eval(d, 2, wl.W, k0, k1, x0, x1, a0, a1, m0, m1, wl.prot)
    assert np.array_equal(o2, out)
    narrow = ms <= bw - 12 - 1
    d0 = _od(orc, synth.workload(2, synth.Dims(bw=bw, n_nodes=140, mask_scale=0), seed=12))
    assert (k0.size == orc.model_key_bytes(d0, 2)) == narrow


@pytest.mark.parametrize("bw", [32, 64])
def test_adjnorm_two_party_matches_closed_form(orc, synth, bw):
    """Standalone secure adjacency normalisation (the config-2 pipeline) on
    shares of A reconstructs A (.) floor(T[d_i] T[d_j] / 2^12) exactly."""
    B, N = 3, 24
    _, A, _ = synth.molecules(B, synth.Dims(bw=bw, n_nodes=N), seed=5, min_atoms=3, max_atoms=N)
    a0, a1 = synth.share(A, bw, 77)
    k0, k1, rout = orc.adjnorm_keygen(bw, 12, B, N, 123)
    got, by = orc.adjnorm_eval(bw, 12, B, N, 138, k0, k1, a0, a1)
    mod = (1 << bw) - 1 if bw < 64 else 0xFFFFFFFFFFFFFFFF
    val = (got - rout) & np.uint64(mod)
    want = orc.adj_norm_plain(A).reshape(-1)
    assert np.array_equal(val.astype(np.int64), want)
    # five exchanges of ring elements + one of DCF bit planes
    assert by > 0


@pytest.mark.parametrize("bw", [32, 64])
def test_local_truncation_model(orc, synth, bw):
    """slack 3: every layer truncation is LocalARS (the reference's default,
    gpu_mpc/ddg_orca_batched.h:180-199): no truncation keys (under 85% of the exact
    key set, a RELU key per ReLU layer remains).  At bw=64
    the outputs stay within a few units of 2^-12 of the fixed-point forward; at
    bw=32 masked values wrap (probability ~|x|/2^32 per element) and the outputs
    are far off, as the reference records for bw=32."""
    wl = _wl(synth, 4, bw=bw, seed=10, slack=3)
    d = _od(orc, wl)
    out, code = orc.plain_forward(d, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0
    k0, k1 = orc.model_keygen(d, 4, 2024, wl.W)
    x0, x1 = wl.shares["x"]
    a0, a1 = wl.shares["a"]
    m0, m1 = wl.shares["m"]
    o2, by = orc.model_eval(d, 4, wl.W, k0, k1, x0, x1, a0, a1, m0, m1, wl.prot)
    err = np.abs(o2 - out)
    if bw == 64:
        assert err.max() <= 16
    else:
        assert err.max() > 1 << 12
    d0 = _od(orc, _wl(synth, 4, bw=bw, seed=10, slack=0))
    assert k0.size < 0.85 * orc.model_key_bytes(d0, 4) and by > 0
