"""Writes the model fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

model_small.npz -- a reduced-width affinity model (16 atoms, GCN 12->8->12->16,
    FC 16->24->8, protein 8, fusion 16->16->8->1), B=3 molecules, inputs and
    weights stored in full with the expected outputs for bw=32 and bw=64.
model_default.json -- the full-size workload (140 atoms, GCN 78->78->156->312,
    FC 312->1024->128, fusion 256->1024->512->1) for B=4, seed 7: the
    generator seed, a SHA-256 of the generated integer tensors (so that a
    change of the generator is caught) and the expected outputs.

The expected outputs are the oracle's plaintext fixed-point forward; the
oracle itself is pinned by the closed-form and hand-computed tests under
tests/, so these fixtures pin the HIP path and guard against regressions.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [HERE, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "idash26-track3_amd")]

import orc  # noqa: E402
import synth  # noqa: E402

from golden_dims import SMALL  # noqa: E402


def odims(d):
    return orc.make_dims(bw=d.bw, s=d.s, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                         fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale)


def workload_digest(wl):
    h = hashlib.sha256()
    for a in (wl.X, wl.A, wl.mask, wl.prot, wl.W):
        h.update(np.ascontiguousarray(a, np.int64).tobytes())
    return h.hexdigest()


def small():
    out = {}
    d32 = synth.Dims(bw=32, **SMALL)
    wl = synth.molecules(3, d32, seed=21, min_atoms=2, max_atoms=16)
    X, A, mask = wl
    W = synth.weights(d32, seed=22)
    prot = synth.protein(3, d32, seed=23)
    out.update(X=X, A=A, mask=mask, W=W, prot=prot)
    for bw in (32, 64):
        d = synth.Dims(bw=bw, **SMALL)
        y, code = orc.plain_forward(odims(d), X, A, mask, prot, W)
        assert code == 0, orc.domain_msg(code)
        out[f"want_bw{bw}"] = y
    np.savez(os.path.join(HERE, "model_small.npz"), **out)


def default():
    B, seed = 4, 7
    rec = {"B": B, "seed": seed, "dims": "synth.Dims() defaults (bw 32 and 64)"}
    for bw in (32, 64):
        d = synth.Dims(bw=bw)
        wl = synth.workload(B, d, seed=seed)
        y, code = orc.plain_forward(odims(d), wl.X, wl.A, wl.mask, wl.prot, wl.W)
        assert code == 0, orc.domain_msg(code)
        rec[f"want_bw{bw}"] = [int(v) for v in y]
        rec["inputs_sha256"] = workload_digest(wl)
    with open(os.path.join(HERE, "model_default.json"), "w") as f:
        json.dump(rec, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    small()
    default()
    print("wrote", os.listdir(HERE))
