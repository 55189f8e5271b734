"""Deterministic synthetic workloads for the secure affinity forward.

Generates integer tensors only (already quantised), so every consumer -- the
GPU path, the CPU oracle, the benchmark -- sees the same bits:

* molecules: B graphs padded to ``n_nodes`` atoms, each with 10..60 real
  atoms; adjacency = random spanning tree with max degree 4 plus 0..3
  ring-closing edges (degree cap respected), symmetric, self loops on real
  atoms (secure_adj_norm.h:20-23 expects them in the input);
* atom features: 78-dim one-hot groups (44 atom types, 11 degrees, 11 H
  counts, 11 valences, 1 aromatic flag), scaled by 2^s;
* weights: Kaiming-normal (sigma = sqrt(2/fan_in)), biases U(-1/sqrt(fan_in),
  1/sqrt(fan_in)), protein embedding N(0,1); all quantised with the
  round-half-away-from-zero rule of reference/fixedpoint.py:28-41;
* additive secret shares over Z_2^bw (reference/share_data.py:56-79 splits
  the same way: uniform share 0, share 1 = value - share 0).

Weight blob layout = weights.bin of gpu_mpc/deepdtagen_inference.cu:121-181:
for each layer W^T (in x out, row-major) then bias (out).
"""
from dataclasses import dataclass, field

import numpy as np

FEAT_GROUPS = (44, 11, 11, 11, 1)


@dataclass
class Dims:
    bw: int = 32
    s: int = 12
    n_nodes: int = 140
    feat: int = 78
    gcn: tuple = (78, 156, 312)
    dfc: tuple = (1024, 128)
    prot: int = 128
    fus: tuple = (1024, 512, 1)
    lut_nmax: int = 138
    mask_scale: int = 0  # the atom mask is 0 or 2^mask_scale
    slack: int = 0  # 0 exact; 1 H.W^T slack-truncated; 2 also A.XW + b (|x| < 2^(bw-2)); 3 LocalARS

    def layers(self):
        """(in, out) of every linear layer in weight-blob order."""
        io = []
        fin = self.feat
        for g in self.gcn:
            io.append((fin, g))
            fin = g
        io.append((self.gcn[2], self.dfc[0]))
        io.append((self.dfc[0], self.dfc[1]))
        fin = self.dfc[1] + self.prot
        for f in self.fus:
            io.append((fin, f))
            fin = f
        return io

    def weights_len(self):
        return sum(i * o + o for i, o in self.layers())


def to_fixed(x, s):
    """round(x * 2^s), half away from zero (reference/fixedpoint.py:28-41)."""
    x = np.asarray(x, dtype=np.float64) * float(1 << s)
    return np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5)).astype(np.int64)


def _graph(rng, n_real, n_nodes, max_deg=4):
    A = np.zeros((n_nodes, n_nodes), np.int64)
    deg = np.zeros(n_nodes, np.int64)
    for v in range(1, n_real):
        cand = [u for u in range(v) if deg[u] < max_deg]
        u = cand[rng.integers(len(cand))]
        A[u, v] = A[v, u] = 1
        deg[u] += 1
        deg[v] += 1
    n_ring = int(rng.integers(0, 4))
    tries = 0
    while n_ring > 0 and tries < 50:
        tries += 1
        i, j = rng.integers(0, n_real, size=2)
        if i == j or A[i, j] or deg[i] >= max_deg or deg[j] >= max_deg:
            continue
        A[i, j] = A[j, i] = 1
        deg[i] += 1
        deg[j] += 1
        n_ring -= 1
    for v in range(n_real):
        A[v, v] = 1
    return A, deg


def molecules(B, dims: Dims, seed=0, min_atoms=10, max_atoms=60):
    """X (B,N,feat) at scale s, A (B,N,N) 0/1 with self loops, mask (B,N)."""
    rng = np.random.default_rng(seed)
    N, s = dims.n_nodes, dims.s
    X = np.zeros((B, N, dims.feat), np.int64)
    A = np.zeros((B, N, N), np.int64)
    mask = np.zeros((B, N), np.int64)
    one = 1 << s
    for b in range(B):
        n_real = int(rng.integers(min_atoms, max_atoms + 1))
        n_real = min(n_real, N)
        A[b], deg = _graph(rng, n_real, N)
        mask[b, :n_real] = 1
        for v in range(n_real):
            off = 0
            for gi, g in enumerate(FEAT_GROUPS):
                if off + g > dims.feat:
                    break
                if gi == 1:
                    k = min(int(deg[v]), g - 1)
                elif g == 1:
                    k = 0 if rng.random() < 0.3 else -1
                else:
                    k = int(rng.integers(g))
                if k >= 0:
                    X[b, v, off + k] = one
                off += g
    return X, A, mask


def weights(dims: Dims, seed=1):
    """Quantised weight blob (int64), W^T then bias per layer."""
    rng = np.random.default_rng(seed)
    parts = []
    for fin, fout in dims.layers():
        W = rng.standard_normal((fin, fout)) * np.sqrt(2.0 / fin)
        bnd = 1.0 / np.sqrt(fin)
        b = rng.uniform(-bnd, bnd, size=fout)
        parts.append(to_fixed(W, dims.s).reshape(-1))
        parts.append(to_fixed(b, dims.s))
    return np.concatenate(parts)


def protein(B, dims: Dims, seed=2):
    rng = np.random.default_rng(seed)
    return to_fixed(rng.standard_normal((B, dims.prot)), dims.s)


def share(v, bw, seed):
    """Additive shares over Z_2^bw: (v0 uniform, v1 = v - v0)."""
    rng = np.random.default_rng(seed)
    v = np.asarray(v, dtype=np.int64)
    mod = np.uint64((1 << bw) - 1) if bw < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)
    v0 = rng.integers(0, np.iinfo(np.uint64).max, size=v.shape, dtype=np.uint64, endpoint=True) & mod
    v1 = (v.astype(np.uint64) - v0) & mod
    return v0, v1


@dataclass
class Workload:
    dims: Dims
    B: int
    X: np.ndarray
    A: np.ndarray
    mask: np.ndarray
    prot: np.ndarray
    W: np.ndarray
    shares: dict = field(default_factory=dict)


def workload(B, dims: Dims = None, seed=0):
    """Everything one forward needs, deterministic in (B, dims, seed)."""
    dims = dims or Dims()
    X, A, mask = molecules(B, dims, seed=seed)
    W = weights(dims, seed=seed + 1)
    prot = protein(B, dims, seed=seed + 2)
    wl = Workload(dims, B, X, A, mask, prot, W)
    for k, (name, v) in enumerate((("x", X), ("a", A), ("m", mask))):
        wl.shares[name] = share(v, dims.bw, seed + 10 + k)
    return wl
