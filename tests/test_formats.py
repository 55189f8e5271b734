"""The reference's file formats (CPU): share files, protein embeddings,
weights blob + manifest, batch manifest; and the oracle's two-party forward on
inputs loaded from them (mask shared at scale s, mask_scale = s)."""
import json
import os

import numpy as np
import pytest


@pytest.fixture()
def fmt():
    import formats
    return formats


def _batch(synth, tmp_path, fmt, bw, B=3, seed=4):
    d = synth.Dims(bw=bw)
    wl = synth.workload(B, d, seed=seed)
    bdir = str(tmp_path / f"batch_bw{bw}")
    fmt.write_batch(bdir, wl.X, wl.A, wl.mask, wl.prot, bw=bw, scale=d.s, pool_dim=d.gcn[2], seed=seed)
    return wl, bdir


@pytest.mark.parametrize("bw", [32, 64])
def test_batch_roundtrip(synth, tmp_path, fmt, bw):
    wl, bdir = _batch(synth, tmp_path, fmt, bw)
    names = sorted(os.listdir(bdir))
    assert names == sorted([f"{t}_share{p}.dat" for t in ("x", "adj", "mask") for p in (0, 1)] +
                           ["protein_emb.dat", "batch_manifest.json"])
    itemsize = bw // 8
    B, N, F = wl.X.shape
    assert os.path.getsize(os.path.join(bdir, "mask_share0.dat")) == B * N * 312 * itemsize  # pre-tiled
    got = fmt.read_batch(bdir)
    mod = (1 << bw) - 1 if bw < 64 else 0xFFFFFFFFFFFFFFFF

    def rec(pair):
        s = (pair[0].astype(np.uint64) + pair[1].astype(np.uint64)) & np.uint64(mod)
        return s.view(np.int64) if bw == 64 else np.where(s >= 1 << 31, s.astype(np.int64) - (1 << 32),
                                                            s.astype(np.int64))
    assert np.array_equal(rec(got["x"]), wl.X)
    assert np.array_equal(rec(got["a"]), wl.A)
    assert np.array_equal(rec(got["m"]), wl.mask << 12)
    assert np.array_equal(got["prot"], wl.prot)
    assert got["mask_scale"] == 12 and got["bw"] == bw
    # shares are not the values themselves
    assert not np.array_equal(got["x"][0].astype(np.int64), wl.X)


def test_weights_roundtrip_and_manifest(synth, tmp_path, fmt):
    d = synth.Dims()
    W = synth.weights(d, seed=3)
    path = str(tmp_path / "weights.bin")
    fmt.write_weights(path, W, d.layers(), scale=12)
    blob, layers, scale = fmt.read_weights(path)
    assert np.array_equal(blob, W) and layers == d.layers() and scale == 12
    man = json.load(open(path + ".json"))
    assert [l["name"] for l in man["layers"]] == ["gcn.0", "gcn.1", "gcn.2", "drug_fc.0", "drug_fc.1", "fusion.0",
                                                   "fusion.1", "fusion.2"]
    assert fmt.dims_from_weights(layers, n_nodes=140) == synth.Dims()
    man["layers"][2]["W_offset"] += 1
    json.dump(man, open(path + ".json", "w"))
    with pytest.raises(ValueError):
        fmt.read_weights(path)


def test_reference_model_shapes(synth, fmt):
    """The reference's own layer table (deepdtagen_inference.cu:121-181:
    94-188-282-376, FC 376-1024-128, fusion 256-1024-512-256-1) maps onto the
    model dimensions."""
    layers = [(94, 188), (188, 282), (282, 376), (376, 1024), (1024, 128), (256, 1024), (1024, 512), (512, 256),
              (256, 1)]
    d = fmt.dims_from_weights(layers, n_nodes=138)
    assert d.gcn == (188, 282, 376) and d.dfc == (1024, 128) and d.prot == 128 and d.fus == (1024, 512, 256, 1)
    assert d.layers() == layers


@pytest.mark.parametrize("bw", [32, 64])
def test_oracle_two_party_on_loaded_batch(orc, synth, tmp_path, fmt, bw):
    wl, bdir = _batch(synth, tmp_path, fmt, bw, B=2, seed=8)
    got = fmt.read_batch(bdir)
    d = synth.Dims(bw=bw, mask_scale=got["mask_scale"])
    od = orc.make_dims(bw=bw, s=12, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot, fus=d.fus,
                       lut_nmax=d.lut_nmax, mask_scale=d.mask_scale)
    want, code = orc.plain_forward(od, wl.X, wl.A, wl.mask << 12, wl.prot, wl.W)
    assert code == 0
    want01, _ = orc.plain_forward(orc.make_dims(bw=bw), wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert np.array_equal(want, want01)
    k0, k1 = orc.model_keygen(od, 2, 61, wl.W)
    out, _ = orc.model_eval(od, 2, wl.W, k0, k1, *got["x"], *got["a"], *got["m"], got["prot"])
    assert np.array_equal(out, want)
