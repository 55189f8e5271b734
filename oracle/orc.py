"""ctypes bindings of the CPU oracle (oracle/_build/liborc.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, never by the product.  Build with
``make -C oracle`` (``__graft_entry__.build()`` does it).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liborc.so")

G_TR, G_TRRELU, G_RELU, G_TRSLACK, G_MUL, G_LUT8, G_SXS, G_REVEAL = 1, 2, 3, 4, 5, 6, 7, 8
F_DCFA, F_DCFB, F_ROUT, F_SPLIT, F_LUTV, F_RIN = 0x10, 0x20, 0x30, 0x40, 0x58, 0x60

_lib = None


class Dims(C.Structure):
    _fields_ = [("bw", C.c_int), ("s", C.c_int), ("n_nodes", C.c_int), ("feat", C.c_int),
                ("gcn", C.c_int * 3), ("dfc", C.c_int * 2), ("prot", C.c_int),
                ("nfus", C.c_int), ("fus", C.c_int * 4), ("lut_nmax", C.c_int),
                ("mask_scale", C.c_int), ("slack", C.c_int), ("gcn_order", C.c_int)]


class DcfLayout(C.Structure):
    _fields_ = [("m", C.c_int), ("L", C.c_int), ("N", C.c_size_t), ("off_root", C.c_size_t),
                ("off_cw", C.c_size_t), ("off_leaf", C.c_size_t), ("off_z", C.c_size_t),
                ("end", C.c_size_t)]


class TrLayout(C.Structure):
    _fields_ = [("kind", C.c_int), ("bw", C.c_int), ("s", C.c_int), ("relu", C.c_int),
                ("N", C.c_size_t), ("a", DcfLayout), ("b", DcfLayout),
                ("off_kappa", C.c_size_t), ("off_g", C.c_size_t), ("ncase", C.c_int),
                ("end", C.c_size_t)]


def make_dims(bw=32, s=12, n_nodes=140, feat=78, gcn=(78, 156, 312), dfc=(1024, 128), prot=128,
              fus=(1024, 512, 1), lut_nmax=138, mask_scale=0, slack=0, gcn_order=0):
    d = Dims()
    d.bw, d.s, d.n_nodes, d.feat = bw, s, n_nodes, feat
    for i, v in enumerate(gcn):
        d.gcn[i] = v
    for i, v in enumerate(dfc):
        d.dfc[i] = v
    d.prot = prot
    d.nfus = len(fus)
    for i, v in enumerate(fus):
        d.fus[i] = v
    d.lut_nmax = lut_nmax
    d.mask_scale = mask_scale
    d.slack = int(slack)
    d.gcn_order = int(gcn_order)  # plain_forward: 0 transform-first, 1 aggregate-first
    return d


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        sz = C.c_size_t
        u64 = C.c_uint64
        u32 = C.c_uint32
        i = C.c_int
        sigs = {
            "orc_aes_expand": (None, [P, P]),
            "orc_aes_encrypt": (None, [P, P, P]),
            "orc_aes_backend": (i, []),
            "orc_aes_force_portable": (None, [i]),
            "orc_H_batch": (None, [sz, P, P, i]),
            "orc_prf_batch": (None, [u64, u32, u32, sz, P]),
            "orc_align": (sz, [sz]),
            "orc_zwords": (sz, [sz]),
            "orc_dcf_layout_make": (DcfLayout, [i, sz, sz, i]),
            "orc_tr_layout_make": (TrLayout, [i, i, i, sz, sz]),
            "orc_dcf_keygen": (None, [u64, u32, u32, i, sz, P, P, P, P, sz]),
            "orc_dcf_eval": (None, [i, i, sz, P, sz, P, P]),
            "orc_tr_keygen": (None, [u64, u32, i, i, i, sz, P, P, P, P, sz]),
            "orc_tr_eval": (None, [i, i, i, sz, P, P, sz, P, P, P, P]),
            "orc_mul_layout": (sz, [i, sz, sz, sz, sz, P, P, P]),
            "orc_mul_keygen": (None, [u64, u32, i, sz, sz, sz, P, P, P, P, P, P, P, sz]),
            "orc_mul_eval": (None, [i, sz, sz, sz, P, P, P, P, sz, P, P, P, P]),
            "orc_lut8_layout": (sz, [i, sz, sz, P, P, P, P]),
            "orc_lut8_keygen": (None, [u64, u32, i, sz, P, P, P, P, sz]),
            "orc_lut8_eval": (None, [i, sz, P, P, sz, P, P, P, P]),
            "orc_sxs_layout": (sz, [i, sz, sz, sz, sz, sz, P, P, P]),
            "orc_sxs_keygen": (None, [u64, u32, i, sz, sz, sz, sz, P, P, P, P, P, sz]),
            "orc_sxs_eval": (None, [i, sz, sz, sz, sz, P, P, sz, P, P, P, P]),
            "orc_reveal_layout": (sz, [i, sz, sz, P]),
            "orc_reveal_keygen": (None, [u64, u32, i, sz, P, P, P, sz]),
            "orc_reveal_eval": (None, [i, sz, P, P, sz, P, P, P, P]),
            "orc_ring_gemm": (None, [i, sz, sz, sz, sz, P, P, P, i]),
            "orc_weights_len": (sz, [P]),
            "orc_invsqrt_table": (None, [i, i, P]),
            "orc_plain_forward": (i, [P, i, P, P, P, P, P, P]),
            "orc_domain_msg": (C.c_char_p, [i]),
            "orc_adj_norm_plain": (None, [i, i, i, P, P]),
            "orc_model_key_bytes": (sz, [P, i]),
            "orc_model_keygen": (i, [P, i, u64, P, P, P]),
            "orc_model_eval": (i, [P, i, P, P, P, P, P, P, P, P, P, P, P, P]),
            "orc_adjnorm_key_bytes": (sz, [i, i, i, i]),
            "orc_adjnorm_keygen": (i, [i, i, i, i, u64, P, P, P]),
            "orc_adjnorm_eval": (i, [i, i, i, i, i, P, P, P, P, P, P]),
            "orc_maxpool_layout": (sz, [i, i, i, i, i, sz]),
            "orc_maxpool_keygen": (None, [u64, u32, i, i, i, i, i, P, P, P, P, sz]),
            "orc_maxpool_eval": (None, [i, i, i, i, i, P, P, sz, P, P, P]),
            "orc_set_threads": (None, [i]),
            "orc_set_dealer_key": (None, [C.c_void_p]),
            "orc_get_threads": (i, []),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _u64(a):
    return np.ascontiguousarray(a, dtype=np.uint64)


def _i64(a):
    return np.ascontiguousarray(a, dtype=np.int64)


# ---------------- AES / PRG ----------------
def aes_encrypt(key16: bytes, block16: bytes) -> bytes:
    rk = np.zeros(176, np.uint8)
    k = np.frombuffer(key16, np.uint8).copy()
    lib().orc_aes_expand(ptr(k), ptr(rk))
    inp = np.frombuffer(block16, np.uint8).copy()
    out = np.zeros(16, np.uint8)
    lib().orc_aes_encrypt(ptr(rk), ptr(inp), ptr(out))
    return out.tobytes()


def hash_blocks(blocks_u32: np.ndarray, leaf=False) -> np.ndarray:
    b = np.ascontiguousarray(blocks_u32, dtype=np.uint32).reshape(-1, 4)
    out = np.zeros_like(b)
    lib().orc_H_batch(b.shape[0], ptr(b), ptr(out), 1 if leaf else 0)
    return out


def prf_blocks(seed, gate, field, n):
    out = np.zeros((n, 4), np.uint32)
    lib().orc_prf_batch(seed, gate, field, n, ptr(out))
    return out


# ---------------- layouts ----------------
def dcf_layout(m, N, base=0, with_z=1):
    return lib().orc_dcf_layout_make(m, N, base, with_z)


def tr_layout(kind, bw, s, N, base=0):
    return lib().orc_tr_layout_make(kind, bw, s, N, base)


# ---------------- DCF ----------------
def dcf_keygen(seed, gate, m, alpha, rbit=None, fbase=F_DCFA):
    alpha = _u64(alpha)
    N = alpha.size
    Lo = dcf_layout(m, N)
    k0 = np.zeros(Lo.end, np.uint8)
    k1 = np.zeros(Lo.end, np.uint8)
    rb = None if rbit is None else np.ascontiguousarray(rbit, dtype=np.uint8)
    lib().orc_dcf_keygen(seed, gate, fbase, m, N, ptr(alpha), ptr(rb), ptr(k0), ptr(k1), 0)
    return k0, k1


def dcf_eval(party, m, key, x):
    x = _u64(x)
    out = np.zeros(x.size, np.uint8)
    lib().orc_dcf_eval(party, m, x.size, ptr(key), 0, ptr(x), ptr(out))
    return out


# ---------------- gates ----------------
def tr_keygen(seed, gate, kind, bw, s, in_mask):
    in_mask = _u64(in_mask)
    N = in_mask.size
    Lo = tr_layout(kind, bw, s, N)
    k0 = np.zeros(Lo.end, np.uint8)
    k1 = np.zeros(Lo.end, np.uint8)
    out_mask = np.zeros(N, np.uint64)
    lib().orc_tr_keygen(seed, gate, kind, bw, s, N, ptr(in_mask), ptr(out_mask), ptr(k0), ptr(k1), 0)
    return k0, k1, out_mask


def tr_eval(kind, bw, s, k0, k1, xhat, bias=None):
    xhat = _u64(xhat)
    N = xhat.size
    b = None if bias is None else _i64(bias)
    y = np.zeros(N, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_tr_eval(kind, bw, s, N, ptr(k0), ptr(k1), 0, ptr(xhat), ptr(b), ptr(y), ptr(by))
    return y, int(by[0])


def mul_keygen(seed, gate, bw, rx, ry, ia, ib):
    rx, ry = _u64(rx), _u64(ry)
    ia = np.ascontiguousarray(ia, np.uint32)
    ib = np.ascontiguousarray(ib, np.uint32)
    nx, ny, nz = rx.size, ry.size, ia.size
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    end = lib().orc_mul_layout(bw, nx, ny, nz, 0, C.byref(a), C.byref(b), C.byref(c))
    k0 = np.zeros(end, np.uint8)
    k1 = np.zeros(end, np.uint8)
    rz = np.zeros(nz, np.uint64)
    lib().orc_mul_keygen(seed, gate, bw, nx, ny, nz, ptr(ia), ptr(ib), ptr(rx), ptr(ry), ptr(rz),
                         ptr(k0), ptr(k1), 0)
    return k0, k1, rz


def mul_eval(bw, k0, k1, xhat, yhat, ia, ib):
    xhat, yhat = _u64(xhat), _u64(yhat)
    ia = np.ascontiguousarray(ia, np.uint32)
    ib = np.ascontiguousarray(ib, np.uint32)
    z = np.zeros(ia.size, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_mul_eval(bw, xhat.size, yhat.size, ia.size, ptr(ia), ptr(ib), ptr(k0), ptr(k1), 0,
                       ptr(xhat), ptr(yhat), ptr(z), ptr(by))
    return z, int(by[0])


def lut8_keygen(seed, gate, bw, in_mask):
    in_mask = _u64(in_mask)
    N = in_mask.size
    D = DcfLayout()
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    end = lib().orc_lut8_layout(bw, N, 0, C.byref(D), C.byref(a), C.byref(b), C.byref(c))
    k0 = np.zeros(end, np.uint8)
    k1 = np.zeros(end, np.uint8)
    out = np.zeros(N, np.uint64)
    lib().orc_lut8_keygen(seed, gate, bw, N, ptr(in_mask), ptr(out), ptr(k0), ptr(k1), 0)
    return k0, k1, out


def lut8_eval(bw, k0, k1, table, xhat):
    xhat = _u64(xhat)
    table = _u64(table)
    y = np.zeros(xhat.size, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_lut8_eval(bw, xhat.size, ptr(k0), ptr(k1), 0, ptr(table), ptr(xhat), ptr(y), ptr(by))
    return y, int(by[0])


def sxs_keygen(seed, gate, bw, nb, M, K, N, ra, rb):
    ra, rb = _u64(ra), _u64(rb)
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    end = lib().orc_sxs_layout(bw, nb, M, K, N, 0, C.byref(a), C.byref(b), C.byref(c))
    k0 = np.zeros(end, np.uint8)
    k1 = np.zeros(end, np.uint8)
    rc = np.zeros(nb * M * N, np.uint64)
    lib().orc_sxs_keygen(seed, gate, bw, nb, M, K, N, ptr(ra), ptr(rb), ptr(rc), ptr(k0), ptr(k1), 0)
    return k0, k1, rc


def sxs_eval(bw, nb, M, K, N, k0, k1, ahat, bhat):
    ahat, bhat = _u64(ahat), _u64(bhat)
    c = np.zeros(nb * M * N, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_sxs_eval(bw, nb, M, K, N, ptr(k0), ptr(k1), 0, ptr(ahat), ptr(bhat), ptr(c), ptr(by))
    return c, int(by[0])


def reveal_keygen(seed, gate, bw, N):
    r = C.c_size_t()
    end = lib().orc_reveal_layout(bw, N, 0, C.byref(r))
    k0 = np.zeros(end, np.uint8)
    k1 = np.zeros(end, np.uint8)
    mask = np.zeros(N, np.uint64)
    lib().orc_reveal_keygen(seed, gate, bw, N, ptr(mask), ptr(k0), ptr(k1), 0)
    return k0, k1, mask


def reveal_eval(bw, k0, k1, v0, v1):
    v0, v1 = _u64(v0), _u64(v1)
    out = np.zeros(v0.size, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_reveal_eval(bw, v0.size, ptr(k0), ptr(k1), 0, ptr(v0), ptr(v1), ptr(out), ptr(by))
    return out, int(by[0])


def ring_gemm(bw, A, B, nb=1, b_batched=False):
    A, B = _u64(A), _u64(B)
    if nb == 1 and A.ndim == 2:
        M, K = A.shape
        N = B.shape[-1]
    else:
        _, M, K = A.shape
        N = B.shape[-1]
    out = np.zeros((nb, M, N), np.uint64)
    lib().orc_ring_gemm(bw, nb, M, K, N, ptr(A), ptr(B), ptr(out), 1 if b_batched else 0)
    return out.reshape((M, N)) if (nb == 1 and A.ndim == 2) else out


def invsqrt_table(s=12, nmax=138):
    t = np.zeros(256, np.uint64)
    lib().orc_invsqrt_table(s, nmax, ptr(t))
    return t


def adj_norm_plain(A, s=12):
    A = _i64(A)
    B, N, _ = A.shape
    out = np.zeros_like(A)
    lib().orc_adj_norm_plain(s, N, B, ptr(A), ptr(out))
    return out


# ---------------- model ----------------
def weights_len(d):
    return lib().orc_weights_len(C.byref(d))


def plain_forward(d, X, A, mask, prot, W):
    X, A, mask, prot, W = _i64(X), _i64(A), _i64(mask), _i64(prot), _i64(W)
    B = A.shape[0]
    out = np.zeros(B, np.int64)
    code = lib().orc_plain_forward(C.byref(d), B, ptr(X), ptr(A), ptr(mask), ptr(prot), ptr(W), ptr(out))
    return out, code


def domain_msg(code):
    return lib().orc_domain_msg(code).decode()


def model_key_bytes(d, B):
    return lib().orc_model_key_bytes(C.byref(d), B)


def model_keygen(d, B, seed, W):
    W = _i64(W)
    n = model_key_bytes(d, B)
    k0 = np.zeros(n, np.uint8)
    k1 = np.zeros(n, np.uint8)
    lib().orc_model_keygen(C.byref(d), B, seed, ptr(W), ptr(k0), ptr(k1))
    return k0, k1


def model_eval(d, B, W, k0, k1, x0, x1, a0, a1, m0, m1, prot):
    W = _i64(W)
    arrs = [_u64(v) for v in (x0, x1, a0, a1, m0, m1)]
    prot = _i64(prot)
    out = np.zeros(B, np.int64)
    by = np.zeros(1, np.uint64)
    lib().orc_model_eval(C.byref(d), B, ptr(W), ptr(k0), ptr(k1), *[ptr(v) for v in arrs], ptr(prot),
                         ptr(out), ptr(by))
    return out, int(by[0])


def adjnorm_keygen(bw, s, B, N, seed):
    n = lib().orc_adjnorm_key_bytes(bw, s, B, N)
    k0 = np.zeros(n, np.uint8)
    k1 = np.zeros(n, np.uint8)
    mask = np.zeros(B * N * N, np.uint64)
    lib().orc_adjnorm_keygen(bw, s, B, N, seed, ptr(mask), ptr(k0), ptr(k1))
    return k0, k1, mask


def adjnorm_eval(bw, s, B, N, nmax, k0, k1, a0, a1):
    a0, a1 = _u64(a0), _u64(a1)
    out = np.zeros(B * N * N, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_adjnorm_eval(bw, s, B, N, nmax, ptr(k0), ptr(k1), ptr(a0), ptr(a1), ptr(out), ptr(by))
    return out, int(by[0])


def maxpool_keygen(seed, gate, bw, s, B, N, C, in_mask):
    in_mask = _u64(in_mask)
    n = lib().orc_maxpool_layout(bw, s, B, N, C, 0)
    k0 = np.zeros(n, np.uint8)
    k1 = np.zeros(n, np.uint8)
    out_mask = np.zeros(B * C, np.uint64)
    lib().orc_maxpool_keygen(seed, gate, bw, s, B, N, C, ptr(in_mask), ptr(out_mask), ptr(k0), ptr(k1), 0)
    return k0, k1, out_mask


def maxpool_eval(bw, s, B, N, C, k0, k1, xhat):
    xhat = _u64(xhat)
    y = np.zeros(B * C, np.uint64)
    by = np.zeros(1, np.uint64)
    lib().orc_maxpool_eval(bw, s, B, N, C, ptr(k0), ptr(k1), 0, ptr(xhat), ptr(y), ptr(by))
    return y, int(by[0])


def set_dealer_key(key16):
    """The dealer's 16 secret key bytes (None: derive keys from the seed alone)."""
    if key16 is None:
        lib().orc_set_dealer_key(None)
        return
    buf = (C.c_uint8 * 16)(*bytes(key16))
    lib().orc_set_dealer_key(C.cast(buf, C.c_void_p))


def set_threads(n):
    lib().orc_set_threads(n)


def get_threads():
    return lib().orc_get_threads()
