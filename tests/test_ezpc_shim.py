"""The EzPC-named entry points (include/mpcx_ezpc.hpp) and the sytorch Backend<T>
subclasses (include/mpcx_sytorch.hpp), driven from C++ (tests/cpp/ezpc_check.cpp)
through two of the reference's call sequences, one dealer run per party and
the two evaluators as two threads on one channel:
  - ddgSecureAdjNormKeygen / ddgSecureAdjNormEval (gpu_mpc/secure_adj_norm.h:
    203-374, 393-659), against the oracle's closed form of A_norm;
  - a GCN layer's backend calls (gcn_layer.h:107-116, layers.h:67-93: the
    per-graph secret x secret matmul, truncateForward, the public-weight matmul
    with bias, truncateForward, relu, output), against exact integer arithmetic
    on the oracle's A_norm.
"""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "ezpc_check")
S = 12


def test_ezpc_check_built():
    assert os.path.exists(BIN), "tests/cpp/ezpc_check not built (run __graft_entry__.build())"


@pytest.mark.parametrize("bw,bin_,bout,drelu,ok", [
    (32, 32, 32, False, True), (32, 20, 20, False, True), (32, 20, 32, False, True), (64, 52, 52, False, True),
    (32, 21, 21, False, True), (32, 16, 16, False, False), (32, 20, 24, False, False), (64, 31, 31, False, False),
    (32, 32, 1, True, True), (32, 20, 1, True, False)])
def test_shim_relu_widths(bw, bin_, bout, drelu, ok):
    """gpuGenReluKey serves bin = bw (full-width RELU) and bin = bw - scale for
    a context scale 1..bw/2-2 (the narrow gate, the reference's mode-3 ReLU with
    tmpBw = bw - scale, gpu_mpc/ddg_orca.h:229-233); gpuKeyGenDRelu only full
    width. Any other width aborts with a message instead of evaluating a gate
    of another width (checked before any device call: no GPU needed)."""
    args = [BIN, "width", str(bw), str(bin_), str(bout)] + (["drelu"] if drelu else [])
    r = subprocess.run(args, capture_output=True, text=True, timeout=60)
    if ok:
        assert r.returncode == 0 and "width ok" in r.stdout, r.stderr
        if not drelu and bin_ < bw:
            assert f"scale {bw - bin_}" in r.stdout
    else:
        assert r.returncode != 0 and "mpcx_ezpc:" in r.stderr


def _ring(v, bw):
    dt = np.uint32 if bw == 32 else np.uint64
    m = (1 << bw) - 1
    return (np.asarray(v, np.int64).astype(np.uint64) & np.uint64(m)).astype(dt)


def _signed(v, bw):
    v = np.asarray(v).astype(np.uint64)
    if bw == 64:
        return v.view(np.int64)
    v = v.astype(np.int64)
    return np.where(v >= 1 << 31, v - (1 << 32), v)


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [32, 64])
def test_shim_adjnorm_and_gcn_layer(orc, synth, tmp_path, bw):
    B, N, F, O, nmax = 3, 24, 8, 6, 138
    dims = synth.Dims(bw=bw, n_nodes=N)
    _, A, _ = synth.molecules(B, dims, seed=bw, min_atoms=5, max_atoms=N)
    rng = np.random.default_rng(bw + 1)
    X = rng.integers(-(1 << S), 1 << S, size=(B, N, F))
    W = rng.integers(-256, 257, size=(F, O))
    b = rng.integers(-(1 << S), 1 << S, size=O)
    a0, a1 = synth.share(A, bw, 3)
    x0, x1 = synth.share(X, bw, 4)
    d = tmp_path
    (d / "meta.txt").write_text(f"{bw} {B} {N} {F} {O} {S} {nmax}\n")
    for name, v in (("a0", a0), ("a1", a1), ("x0", x0), ("x1", x1), ("w", W), ("b", b << S)):
        _ring(v, bw).tofile(str(d / f"{name}.bin"))
    kfile = d / "dealer.key"  # the dealers draw every key set under this secret key
    kfile.write_bytes(bytes(range(40, 56)))
    r = subprocess.run([BIN, str(d)], capture_output=True, text=True, timeout=180,
                       env=dict(os.environ, MPCX_DEALER_KEY=str(kfile)))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "MPCX_DEALER_KEY" not in r.stderr
    dt = np.uint32 if bw == 32 else np.uint64
    An = orc.adj_norm_plain(A)
    got_an = _signed(np.fromfile(str(d / "adjn.bin"), dt), bw).reshape(B, N, N)
    assert np.array_equal(got_an, An)
    AX = np.floor_divide(np.einsum("bij,bjf->bif", An, X), 1 << S).reshape(B * N, F)
    Z = np.floor_divide(AX @ W + (b << S), 1 << S)
    act = np.maximum(Z, 0)
    got_act = _signed(np.fromfile(str(d / "act.bin"), dt), bw).reshape(B * N, O)
    assert np.array_equal(got_act, act)
    got_out = _signed(np.fromfile(str(d / "out.bin"), dt), bw).reshape(B * N, O)
    assert np.array_equal(got_out, act >> S)
    c0, c1 = (int(v) for v in (d / "comm.txt").read_text().split())
    assert c0 == c1 > 0


def _fwd_expected(A_fx, X, maskT, prot, layers, bw, s=S):
    """The forward in the backend's op order, in exact integers: GCN aggregate
    first (gcn_layer.h:113-114: tr(A.H), then the FC + bias and its
    truncation, ReLU); the mask product truncated once (TrWithSlack); the pool
    a maximum over all node rows (padding rows are 0 after the mask); the drug
    FCs; [drug | protein]; the fusion FCs, the last one truncated by output().
    Checks that every value a ring protocol truncates lies in the signed ring."""
    half = 1 << (bw - 1)

    def tr(v, lim=half):
        assert np.abs(v).max() < lim, "outside the bit-exact domain"
        return np.floor_divide(v, 1 << s)

    H = X
    for W, b in layers[:3]:
        AX = tr(np.matmul(A_fx, H))
        H = np.maximum(tr(np.matmul(AX, W) + (b << s)), 0)
    pooled = tr(H * maskT, 1 << (bw - 2)).max(axis=1)
    (W3, b3), (W4, b4) = layers[3], layers[4]
    d1 = np.maximum(tr(pooled @ W3 + (b3 << s)), 0)
    f = np.concatenate([tr(d1 @ W4 + (b4 << s)), prot], axis=1)
    for i, (W, b) in enumerate(layers[5:]):
        e = tr(f @ W + (b << s))
        f = e if i + 1 == len(layers) - 5 else np.maximum(e, 0)
    return f.reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [32, 64])
def test_shim_whole_forward(orc, synth, tmp_path, bw):
    """The reference's whole online path through the shim and Backend<T>
    (ezpc_check forward): ddgSecureAdjNormEval, then DeepDTAGenAffinity::
    _forward's backend calls, one dealer run per party, the two evaluators as
    two threads on one channel with both key sets resident (initGPUKeyArena);
    both parties' outputs equal the integer forward in that op order."""
    B = 2
    dims = synth.Dims(bw=bw)
    wl = synth.workload(B, dims, seed=23)
    N, C = dims.n_nodes, dims.gcn[2]
    maskT = np.repeat((wl.mask << S)[:, :, None], C, axis=2)  # the pre-tiled mask at scale s
    layers, o = [], 0
    for fin, fout in dims.layers():
        W = wl.W[o:o + fin * fout].reshape(fin, fout)
        b = wl.W[o + fin * fout:o + fin * fout + fout]
        layers.append((W, b))
        o += fin * fout + fout
    want = _fwd_expected(orc.adj_norm_plain(wl.A), wl.X, maskT, wl.prot, layers, bw)
    od = orc.make_dims(bw=bw, s=S, n_nodes=N, feat=dims.feat, gcn=dims.gcn, dfc=dims.dfc, prot=dims.prot,
                       fus=dims.fus, lut_nmax=dims.lut_nmax, gcn_order=1)
    ow, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, wl.W)
    assert code == 0 and np.array_equal(ow, want)  # the oracle's aggregate-first forward agrees
    d = tmp_path
    (d / "meta.txt").write_text(" ".join(str(v) for v in (
        bw, B, N, dims.feat, *dims.gcn, *dims.dfc, dims.prot, len(dims.fus), *dims.fus, S, dims.lut_nmax, 1)) + "\n")
    a0, a1 = synth.share(wl.A, bw, 3)
    x0, x1 = synth.share(wl.X, bw, 4)
    m0, m1 = synth.share(maskT, bw, 5)
    blob = np.concatenate([np.concatenate([W.reshape(-1), b << S]) for W, b in layers])
    for name, v in (("a0", a0), ("a1", a1), ("x0", x0), ("x1", x1), ("m0", m0), ("m1", m1), ("prot", wl.prot),
                    ("w", blob)):
        _ring(v, bw).tofile(str(d / f"{name}.bin"))
    kfile = d / "dealer.key"
    kfile.write_bytes(bytes(range(90, 106)))
    r = subprocess.run([BIN, "forward", str(d)], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, MPCX_DEALER_KEY=str(kfile)))
    assert r.returncode == 0, r.stdout + r.stderr
    dt = np.uint32 if bw == 32 else np.uint64
    got = _signed(np.fromfile(str(d / "out.bin"), dt), bw)
    assert np.array_equal(got, want), (got, want)
    c0, c1 = (int(v) for v in (d / "comm.txt").read_text().split())
    assert c0 == c1 > 0
