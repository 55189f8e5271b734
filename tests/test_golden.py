"""Known-answer vectors of tests/golden/ (CPU): the oracle and the synthetic
generator against the reference's own vectors and closed forms, and the
committed model fixtures against the oracle's plaintext forward."""
import hashlib
import json
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _vectors():
    with open(os.path.join(GOLD, "reference_vectors.json")) as f:
        return json.load(f)


def test_to_fixed_vectors(synth):
    for case in _vectors()["to_fixed"]["cases"]:
        assert synth.to_fixed(case["x"], case["s"]).tolist() == case["want"]


def test_fixed_matmul_vector(orc):
    for case in _vectors()["fixed_matmul"]["cases"]:
        a = np.array(case["a"], np.uint64)
        b = np.array(case["b"], np.uint64)
        prod = orc.ring_gemm(64, a, b).astype(np.int64)
        assert (prod >> case["s"]).tolist() == case["want"]


@pytest.mark.parametrize("portable", [0, 1])
def test_aes_vectors(orc, portable):
    orc.lib().orc_aes_force_portable(portable)
    try:
        for case in _vectors()["aes128"]["cases"]:
            ct = orc.aes_encrypt(bytes.fromhex(case["key"]), bytes.fromhex(case["pt"]))
            assert ct.hex() == case["ct"]
    finally:
        orc.lib().orc_aes_force_portable(0)


def test_invsqrt_table_and_pairs(orc):
    v = _vectors()
    tab = v["invsqrt_table"]
    t = orc.invsqrt_table(tab["s"], tab["nmax"])
    for k, want in tab["T"].items():
        assert int(t[int(k)]) == want, k
    for di, dj, want in v["adj_norm_pairs"]["pairs"]:
        # a star around node 0 gives node 0 degree di (self loop included);
        # node 1's degree is raised to dj with extra neighbours
        N = 16
        A = np.zeros((1, N, N), np.int64)
        for u in range(N):
            A[0, u, u] = 1
        A[0, 0, 1] = A[0, 1, 0] = 1
        nxt = 2
        for _ in range(di - 2):
            A[0, 0, nxt] = A[0, nxt, 0] = 1
            nxt += 1
        for _ in range(dj - 2):
            A[0, 1, nxt] = A[0, nxt, 1] = 1
            nxt += 1
        if di == 1 or dj == 1:  # isolated node pair: use the self loop entry
            A = np.zeros((1, N, N), np.int64)
            A[0, 0, 0] = 1
            assert orc.adj_norm_plain(A)[0, 0, 0] == want
            continue
        deg = A[0].sum(axis=1)
        assert deg[0] == di and deg[1] == dj
        assert orc.adj_norm_plain(A)[0, 0, 1] == want


def test_model_small_fixture(orc, synth):
    f = np.load(os.path.join(GOLD, "model_small.npz"))
    from golden_dims import SMALL
    for bw in (32, 64):
        d = synth.Dims(bw=bw, **SMALL)
        od = orc.make_dims(bw=bw, s=12, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                           fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale)
        y, code = orc.plain_forward(od, f["X"], f["A"], f["mask"], f["prot"], f["W"])
        assert code == 0
        assert np.array_equal(y, f[f"want_bw{bw}"])


def test_model_default_fixture(orc, synth):
    with open(os.path.join(GOLD, "model_default.json")) as fh:
        rec = json.load(fh)
    for bw in (32, 64):
        wl = synth.workload(rec["B"], synth.Dims(bw=bw), seed=rec["seed"])
        h = hashlib.sha256()
        for a in (wl.X, wl.A, wl.mask, wl.prot, wl.W):
            h.update(np.ascontiguousarray(a, np.int64).tobytes())
        assert h.hexdigest() == rec["inputs_sha256"], "synthetic generator changed"
        d = wl.dims
        od = orc.make_dims(bw=bw, s=12, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                           fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale)
        y, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, wl.W)
        assert code == 0
        assert y.tolist() == rec[f"want_bw{bw}"]
