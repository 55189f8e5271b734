"""The reference's on-disk formats for the secure-inference inputs.

Readers (and writers, for tests and tooling) of the files the reference's
offline preparation produces and its evaluator loads:

* ``{x,adj,mask}_share{0,1}.dat`` -- headerless little-endian ring elements
  (``<u4`` at bw=32, ``<u8`` at bw=64), sample-major: x (B, N, feat) at scale s,
  adj (B, N, N) raw 0/1 with self loops at scale 0, mask (B, N, pool_dim) at
  scale s, pre-tiled along the pooled width; each element is an independent
  additive sharing (share 0 = uniform pad, share 1 = value - pad)
  (reference/share_data.py:56-79, :135-159;
  scripts/dev_tools/prepare_batch_samples.py:119-151; read by
  gpu_mpc/deepdtagen_inference.cu:426-432);
* ``protein_emb.dat`` -- (B, prot) ring elements at scale s, public, held by
  party 1 (prepare_batch_samples.py:143-151);
* ``weights.bin`` -- headerless little-endian int64 blob, per layer W^T
  (in x out, row-major) then bias, at scale s, with a ``weights.bin.json``
  manifest of names, shapes and offsets (reference/export_weights.py:38-75);
  the evaluator shifts biases by s itself (deepdtagen_inference.cu:121-181);
* ``batch_manifest.json`` -- batch size, scale, bw, shapes
  (prepare_batch_samples.py:154-177).

The mask file holds 2^s for a real atom: the model takes it with
``mask_scale = s`` (one column of the tiled shares is a sharing of the mask).
"""
import json
import os

import numpy as np

SHARE_TENSORS = ("x", "adj", "mask")
PROTEIN_FILE = "protein_emb.dat"
MANIFEST_FILE = "batch_manifest.json"
WEIGHT_GROUPS = ("gcn", "drug_fc", "fusion")


def share_filename(tensor, party):
    """``{tensor}_share{party}.dat`` (reference/mpc_config.py:14-17)."""
    if party not in (0, 1):
        raise ValueError("party must be 0 or 1")
    return f"{tensor}_share{party}.dat"


def ring_dtype(bw):
    if bw == 32:
        return np.dtype("<u4")
    if bw == 64:
        return np.dtype("<u8")
    raise ValueError("bw must be 32 or 64")


def _ring(v, bw):
    """int64 values -> unsigned bw-bit residues."""
    v = np.asarray(v, dtype=np.int64)
    if bw == 64:
        return v.view(np.uint64)
    return (v & np.int64((1 << bw) - 1)).astype(np.uint32)


def _signed(u, bw):
    u = np.asarray(u)
    return u.view(np.int64) if bw == 64 else u.astype(np.uint32).view(np.int32).astype(np.int64)


def split(values, bw, rng):
    """Additive sharing of integer ring values: (uniform pad, value - pad)."""
    val = _ring(values, bw)
    dt = ring_dtype(bw)
    pad = rng.integers(0, np.iinfo(dt.type).max, size=val.shape, dtype=dt.type, endpoint=True)
    return pad, (val - pad).astype(dt.type)


# ---------------------------------------------------------------------------
# batches
# ---------------------------------------------------------------------------
def write_batch(batch_dir, X, A, mask, prot, bw, scale, pool_dim, seed=0):
    """Write one batch in the reference's layout.  X (B,N,feat) and prot
    (B,prot) are integers at scale s, A (B,N,N) is 0/1 with self loops, mask
    (B,N) is 0/1 (written as 2^s, tiled to pool_dim)."""
    os.makedirs(batch_dir, exist_ok=True)
    X, A, mask, prot = (np.asarray(t, dtype=np.int64) for t in (X, A, mask, prot))
    B, N, feat = X.shape
    tiled = np.broadcast_to((mask << scale).reshape(B, N, 1), (B, N, pool_dim))
    rng = np.random.default_rng(seed)
    dt = ring_dtype(bw)
    for name, val in (("x", X), ("adj", A), ("mask", tiled)):
        s0, s1 = split(val, bw, rng)
        s0.astype(dt).tofile(os.path.join(batch_dir, share_filename(name, 0)))
        s1.astype(dt).tofile(os.path.join(batch_dir, share_filename(name, 1)))
    _ring(prot, bw).astype(dt).tofile(os.path.join(batch_dir, PROTEIN_FILE))
    manifest = {"batch_size": int(B), "scale": int(scale), "bw": int(bw), "raw_adj": True, "adj_scale": 0,
                "nmax": int(N), "feat_dim": int(feat), "pool_dim": int(pool_dim),
                "shapes": {"X": [int(B), int(N), int(feat)], "A_hat": [int(B), int(N), int(N)],
                           "mask": [int(B), int(N), int(pool_dim)], "protein_emb": list(map(int, prot.shape))}}
    with open(os.path.join(batch_dir, MANIFEST_FILE), "w") as f:
        json.dump(manifest, f, indent=2)
    return manifest


def read_batch(batch_dir):
    """Read a batch written by the reference's preparation (or write_batch).

    Returns a dict with both parties' shares as unsigned ring arrays --
    x (B,N,feat), a (B,N,N), m (B,N): column 0 of the tiled mask -- the public
    protein rows as signed int64 at scale s, the manifest, and mask_scale."""
    with open(os.path.join(batch_dir, MANIFEST_FILE)) as f:
        man = json.load(f)
    bw, scale = int(man["bw"]), int(man["scale"])
    if not man.get("raw_adj", False) or int(man.get("adj_scale", 0)) != 0:
        raise ValueError("only the raw-adjacency layout (adj at scale 0, normalised on shares) is supported")
    sh = man["shapes"]
    dt = ring_dtype(bw)
    out = {"manifest": man, "bw": bw, "scale": scale, "mask_scale": scale}
    for name, key, shape in (("x", "x", sh["X"]), ("adj", "a", sh["A_hat"]), ("mask", "m", sh["mask"])):
        parts = []
        for p in (0, 1):
            path = os.path.join(batch_dir, share_filename(name, p))
            arr = np.fromfile(path, dtype=dt)
            if arr.size != int(np.prod(shape)):
                raise ValueError(f"{path}: {arr.size} elements, expected {shape}")
            arr = arr.reshape(shape)
            if name == "mask":
                arr = np.ascontiguousarray(arr[:, :, 0])
            parts.append(arr)
        out[key] = tuple(parts)
    prot = np.fromfile(os.path.join(batch_dir, PROTEIN_FILE), dtype=dt)
    if prot.size != int(np.prod(sh["protein_emb"])):
        raise ValueError(f"{PROTEIN_FILE}: {prot.size} elements, expected {sh['protein_emb']}")
    out["prot"] = _signed(prot, bw).reshape(sh["protein_emb"])
    return out


# ---------------------------------------------------------------------------
# weights
# ---------------------------------------------------------------------------
def weight_layer_names(n_gcn=3, n_drug=2, n_fusion=3):
    return ([f"gcn.{i}" for i in range(n_gcn)] + [f"drug_fc.{i}" for i in range(n_drug)] +
            [f"fusion.{i}" for i in range(n_fusion)])


def write_weights(path, blob, layers, scale):
    """blob: int64 W^T-then-bias per layer; layers: [(in, out)] in blob order
    (3 GCN, 2 drug FC, then the fusion layers)."""
    blob = np.ascontiguousarray(blob, dtype="<i8")
    names = weight_layer_names(n_fusion=len(layers) - 5)
    meta, off = [], 0
    for name, (fin, fout) in zip(names, layers):
        meta.append({"name": name, "W_shape": [int(fin), int(fout)], "b_shape": [int(fout)], "W_offset": off,
                     "b_offset": off + fin * fout})
        off += fin * fout + fout
    if off != blob.size:
        raise ValueError(f"weight blob has {blob.size} elements, layers need {off}")
    blob.tofile(path)
    with open(path + ".json", "w") as f:
        json.dump({"scale": int(scale), "bitwidth": 64, "total_elements": int(blob.size), "layers": meta}, f,
                  indent=2)


def read_weights(path):
    """Returns (int64 blob, [(in, out)] per layer, scale).  The manifest, when
    present, is checked against the blob; the blob is used as stored (biases
    at scale s: the library adds them after the floor shift)."""
    blob = np.fromfile(path, dtype="<i8")
    man_path = path + ".json"
    if not os.path.exists(man_path):
        return blob, None, None
    with open(man_path) as f:
        man = json.load(f)
    layers, off = [], 0
    for layer in man["layers"]:
        fin, fout = layer["W_shape"]
        if layer["W_offset"] != off or layer["b_offset"] != off + fin * fout or layer["b_shape"] != [fout]:
            raise ValueError(f"{man_path}: layer {layer['name']} offsets do not follow the blob order")
        layers.append((int(fin), int(fout)))
        off += fin * fout + fout
    if off != blob.size or man.get("total_elements", off) != blob.size:
        raise ValueError(f"{path}: {blob.size} elements, manifest describes {off}")
    return blob, layers, int(man["scale"])


def dims_from_weights(layers, n_nodes, lut_nmax=138, bw=32, scale=12, mask_scale=0):
    """synth.Dims for a weight manifest's layer shapes (3 GCN, 2 drug FC,
    2..4 fusion layers, the last of width 1)."""
    from synth import Dims
    feat = layers[0][0]
    gcn = tuple(o for _, o in layers[:3])
    dfc = tuple(o for _, o in layers[3:5])
    prot = layers[5][0] - dfc[1]
    fus = tuple(o for _, o in layers[5:])
    return Dims(bw=bw, s=scale, n_nodes=n_nodes, feat=feat, gcn=gcn, dfc=dfc, prot=prot, fus=fus,
                lut_nmax=lut_nmax, mask_scale=mask_scale)
