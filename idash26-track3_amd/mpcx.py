"""Python binding of libmpcx (ctypes over the C ABI of include/mpcx.h).

Device buffers are torch tensors on the GPU (plumbing only); every kernel runs
in libmpcx.so.  There is no CPU fallback: importing this module on a machine
without the built library or without a GPU raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmpcx.so")

TR, TRRELU, RELU, TRSLACK, RELUSLACK, LOCALARS, DRELU, TRMOD, EXT, EXTRELU, RELUPOOL = \
    1, 2, 3, 4, 9, 10, 11, 12, 13, 14, 15

_lib = None


class ModelDims(C.Structure):
    _fields_ = [("n_nodes", C.c_int), ("feat", C.c_int), ("gcn", C.c_int * 3), ("dfc", C.c_int * 2),
                ("prot", C.c_int), ("nfus", C.c_int), ("fus", C.c_int * 4), ("lut_nmax", C.c_int),
                ("mask_scale", C.c_int), ("slack", C.c_int)]


_SIGS = {
    "mpcx_create": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "mpcx_destroy": (None, [C.c_void_p]),
    "mpcx_last_error": (C.c_char_p, [C.c_void_p]),
    "mpcx_set_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mpcx_synchronize": (C.c_int, [C.c_void_p]),
    "mpcx_aes_variant_count": (C.c_int, []),
    "mpcx_aes_variant_name": (C.c_char_p, [C.c_int]),
    "mpcx_set_aes_variant": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "mpcx_set_party_sync": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_set_both_party_aes": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_aes_variant": (C.c_int, [C.c_void_p]),
    "mpcx_bytes_exchanged": (C.c_uint64, [C.c_void_p]),
    "mpcx_rounds": (C.c_uint64, [C.c_void_p]),
    "mpcx_reset_counters": (None, [C.c_void_p]),
    "mpcx_prg_hash": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p]),
    "mpcx_prf": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_size_t, C.c_void_p]),
    "mpcx_dcf_key_bytes": (C.c_size_t, [C.c_int, C.c_size_t]),
    "mpcx_dcf_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p, C.c_uint64,
                                  C.c_uint32, C.c_void_p, C.c_void_p]),
    "mpcx_dcf_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p,
                                C.c_void_p]),
    "mpcx_dcf_eval_ring": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t] + [C.c_void_p] * 4),
    "mpcx_maxpool_levels": (C.c_int, [C.c_int]),
    "mpcx_maxpool_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "mpcx_maxpool_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_uint64,
                                      C.c_uint32, C.c_void_p, C.c_void_p]),
    "mpcx_maxpool_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]),
    "mpcx_maxpool_eval_noalloc": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                            C.c_void_p, C.c_void_p]),
    "mpcx_tr_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int, C.c_size_t]),
    "mpcx_tr_aes_calls": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_tr_eval_form": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t]),
    "mpcx_tr_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p, C.c_uint64,
                                 C.c_uint32, C.c_void_p, C.c_void_p]),
    "mpcx_tr_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_void_p, C.c_int, C.c_void_p]),
    "mpcx_mul_key_bytes": (C.c_size_t, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t]),
    "mpcx_mul_keygen": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p,
                                  C.c_void_p]),
    "mpcx_mul_eval": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p,
                                C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "mpcx_lut8_key_bytes": (C.c_size_t, [C.c_void_p, C.c_size_t]),
    "mpcx_lut8_keygen": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32,
                                   C.c_void_p, C.c_void_p]),
    "mpcx_lut8_eval": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p]),
    "mpcx_sxs_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int]),
    "mpcx_sxs_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p, C.c_void_p]),
    "mpcx_sxs_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                C.c_void_p, C.c_void_p, C.c_void_p]),
    "mpcx_ring_gemm": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                 C.c_void_p]),
    "mpcx_ring_lincomb": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_uint64, C.c_void_p, C.c_uint64,
                                    C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "mpcx_set_adjnorm_lanes": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_reveal_key_bytes": (C.c_size_t, [C.c_void_p, C.c_size_t]),
    "mpcx_reveal_keygen": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p,
                                     C.c_void_p]),
    "mpcx_reveal_eval": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_void_p]),
    "mpcx_model_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mpcx_model_destroy": (None, [C.c_void_p]),
    "mpcx_model_set_lanes": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_model_write_keys": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_char_p, C.c_int]),
    "mpcx_model_attach_key_files": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_char_p, C.c_size_t]),
    "mpcx_model_lanes": (C.c_int, [C.c_void_p]),
    "mpcx_model_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int]),
    "mpcx_model_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_uint64]),
    "mpcx_model_import_keys": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t]),
    "mpcx_model_export_keys": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
    "mpcx_model_set_inputs": (C.c_int, [C.c_void_p, C.c_int] + [C.c_void_p] * 7),
    "mpcx_model_forward": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_model_output": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
    "mpcx_model_profile": (C.c_int, [C.c_void_p, C.c_int]),
    "mpcx_model_release_arena": (C.c_int, [C.c_void_p]),
    "mpcx_model_attach_host_keys": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p,
                                              C.c_size_t, C.c_size_t]),
    "mpcx_model_unique_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int, C.c_int]),
    "mpcx_model_export_unique_keys": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
    "mpcx_model_stream_stats": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "mpcx_adjnorm_key_bytes": (C.c_size_t, [C.c_void_p, C.c_int, C.c_int]),
    "mpcx_adjnorm_keygen": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_uint64, C.c_void_p, C.c_void_p,
                                      C.c_void_p]),
    "mpcx_adjnorm_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int] + [C.c_void_p] * 5),
    "mpcx_host_alloc": (C.c_int, [C.c_size_t, C.c_void_p]),
    "mpcx_host_free": (None, [C.c_void_p]),
    "mpcx_model_profile_read": (C.c_int, [C.c_void_p] + [C.c_void_p] * 5),
    "mpcx_mul_key_layout": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p]),
    "mpcx_sxs_key_layout": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "mpcx_set_dealer_key": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mpcx_peer_connect": (C.c_int, [C.c_int, C.c_char_p, C.c_int, C.c_void_p]),
    "mpcx_peer_pair": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p]),
    "mpcx_peer_close": (None, [C.c_void_p]),
    "mpcx_peer_party": (C.c_int, [C.c_void_p]),
    "mpcx_peer_bytes": (C.c_uint64, [C.c_void_p]),
    "mpcx_peer_rounds": (C.c_uint64, [C.c_void_p]),
    "mpcx_peer_transport": (C.c_int, [C.c_void_p]),
    "mpcx_peer_error": (C.c_char_p, [C.c_void_p]),
    "mpcx_party_reconstruct": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mpcx_party_tr_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_int, C.c_void_p]),
    "mpcx_party_mul_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t] +
                            [C.c_void_p] * 6),
    "mpcx_party_lut8_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t] + [C.c_void_p] * 4),
    "mpcx_party_sxs_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int] +
                            [C.c_void_p] * 4),
    "mpcx_party_reveal_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t] + [C.c_void_p] * 3),
    "mpcx_model_set_party": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mpcx_model_import_party_key": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
    "mpcx_model_set_party_inputs": (C.c_int, [C.c_void_p, C.c_int] + [C.c_void_p] * 4),
    "mpcx_model_profile_gemm": (C.c_int, [C.c_void_p] + [C.c_void_p] * 3),
}


def load():
    """Load libmpcx.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: build it with `make -C idash26-track3_amd` "
                               "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGS)


class MpcxError(RuntimeError):
    pass


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise MpcxError("no GPU visible: libmpcx has no CPU path")
    return torch


def to_dev(a):
    """numpy array -> GPU tensor with the same bytes (uint64 viewed as int64)."""
    torch = _torch()
    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint64): np.int64, np.dtype(np.uint32): np.int32, np.dtype(np.uint8): np.uint8,
            np.dtype(np.int64): np.int64, np.dtype(np.int32): np.int32}[a.dtype]
    return torch.from_numpy(a.view(view)).cuda()


def empty_dev(nbytes):
    torch = _torch()
    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device="cuda")


def from_dev(t, dtype, count=None):
    torch = _torch()
    torch.cuda.synchronize()
    raw = t.detach().cpu().numpy().view(np.uint8)
    out = raw.view(dtype)
    return out if count is None else out[:count]


def dptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


class Ctx:
    """A libmpcx context (bw-bit ring, fixed-point scale s) on one GPU."""

    def __init__(self, bw=32, scale=12, device=0):
        _torch()
        self.lib = load()
        self.bw, self.s = bw, scale
        self.T = np.uint32 if bw == 32 else np.uint64
        h = C.c_void_p()
        st = self.lib.mpcx_create(bw, scale, device, C.byref(h))
        if st != 0:
            raise MpcxError(f"mpcx_create failed ({st})")
        self.h = h

    def close(self):
        if self.h:
            self.lib.mpcx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, st, what):
        if st != 0:
            raise MpcxError(f"{what}: status {st}: {self.lib.mpcx_last_error(self.h).decode()}")

    def sync(self):
        self.check(self.lib.mpcx_synchronize(self.h), "synchronize")

    def set_party_sync(self, sync):
        """Party-mode calls synchronise the stream (True, the default) or return
        with their work enqueued (False: the methods below then synchronise the
        context themselves before reading their outputs)."""
        self.check(self.lib.mpcx_set_party_sync(self.h, 1 if sync else 0), "set_party_sync")
        self._party_async = not sync

    def _party_out(self, t, n):
        if getattr(self, "_party_async", False):
            self.sync()
        return from_dev(t, self.T, n)

    def set_aes_variant(self, v, block=0):
        self.check(self.lib.mpcx_set_aes_variant(self.h, v, block), "set_aes_variant")

    def tr_eval_form(self, kind, n):
        """Kernel form of tr_eval on n elements: 0 one-lane, 1 both-party, 2 quad-lane."""
        return int(self.lib.mpcx_tr_eval_form(self.h, kind, n))

    def set_both_party_aes(self, max_aes):
        """Longest gate (AES calls per element and party) evaluated in the
        both-party form by large Z_2^32 launches (0: never)."""
        self.check(self.lib.mpcx_set_both_party_aes(self.h, int(max_aes)), "set_both_party_aes")

    def set_dealer_key(self, key16):
        """The dealer's 16 secret key bytes (None: keys from the seed alone)."""
        buf = (C.c_uint8 * 16)(*bytes(key16)) if key16 is not None else None
        self.check(self.lib.mpcx_set_dealer_key(self.h, C.cast(buf, C.c_void_p) if buf is not None else None),
                   "set_dealer_key")

    def aes_variant_name(self):
        return self.lib.mpcx_aes_variant_name(self.lib.mpcx_aes_variant(self.h)).decode()

    @property
    def bytes_exchanged(self):
        return int(self.lib.mpcx_bytes_exchanged(self.h))

    @property
    def rounds(self):
        return int(self.lib.mpcx_rounds(self.h))

    def reset_counters(self):
        self.lib.mpcx_reset_counters(self.h)

    def ring(self, a):
        return np.ascontiguousarray(np.asarray(a).astype(np.uint64) & np.uint64((1 << self.bw) - 1 if self.bw < 64 else 0xFFFFFFFFFFFFFFFF)).astype(self.T)

    # ---------------- PRG ----------------
    def prg_hash(self, blocks_u32, leaf=False):
        b = to_dev(np.ascontiguousarray(blocks_u32, np.uint32).reshape(-1))
        out = empty_dev(b.numel() * 4)
        self.check(self.lib.mpcx_prg_hash(self.h, int(leaf), b.numel() // 4, dptr(b), dptr(out)), "prg_hash")
        return from_dev(out, np.uint32).reshape(-1, 4)

    def prf(self, seed, gate, field, n):
        out = empty_dev(16 * n)
        self.check(self.lib.mpcx_prf(self.h, seed, gate, field, n, dptr(out)), "prf")
        return from_dev(out, np.uint32).reshape(-1, 4)

    # ---------------- DCF ----------------
    def dcf_keygen(self, m, alpha, rbit=None, seed=1, gate=1):
        alpha = np.ascontiguousarray(alpha, np.uint64)
        n = alpha.size
        nb = self.lib.mpcx_dcf_key_bytes(m, n)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        da = to_dev(alpha)
        dr = to_dev(np.ascontiguousarray(rbit, np.uint8)) if rbit is not None else None
        self.check(self.lib.mpcx_dcf_keygen(self.h, m, n, dptr(da), dptr(dr), seed, gate, dptr(k0), dptr(k1)),
                   "dcf_keygen")
        return k0, k1

    def dcf_eval(self, party, m, key, x):
        x = np.ascontiguousarray(x, np.uint64)
        n = x.size
        dx = to_dev(x)
        out = empty_dev(((n + 63) // 64) * 8)
        self.check(self.lib.mpcx_dcf_eval(self.h, party, m, n, dptr(key), dptr(dx), dptr(out)), "dcf_eval")
        words = from_dev(out, np.uint64)
        bits = np.unpackbits(words.view(np.uint8), bitorder="little")[:n]
        return bits

    def dcf_eval_ring(self, party, m, key, x, mask_words=None):
        """mpcx_dcf_eval_ring: x as ring elements of the context's width (read
        modulo 2^m), the output bits XORed with mask_words (uint32, bit i of
        word i/32) if given; returns the n output bits."""
        x = self.ring(x)
        n = x.size
        dx = to_dev(x)
        dm = to_dev(np.ascontiguousarray(mask_words, np.uint32)) if mask_words is not None else None
        out = empty_dev(((n + 63) // 64) * 8)
        self.check(self.lib.mpcx_dcf_eval_ring(self.h, party, m, n, dptr(key), dptr(dx), dptr(dm), dptr(out)),
                   "dcf_eval_ring")
        words = from_dev(out, np.uint64)
        return np.unpackbits(words.view(np.uint8), bitorder="little")[:n]

    # ---------------- gates ----------------
    def tr_keygen(self, kind, in_mask, seed=1, gate=1):
        in_mask = self.ring(in_mask)
        n = in_mask.size
        nb = self.lib.mpcx_tr_key_bytes(self.h, kind, n)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        dm = to_dev(in_mask)
        out = empty_dev(n * in_mask.itemsize)
        self.check(self.lib.mpcx_tr_keygen(self.h, kind, n, dptr(dm), dptr(out), seed, gate, dptr(k0), dptr(k1)),
                   "tr_keygen")
        return k0, k1, from_dev(out, self.T, n)

    def tr_eval(self, kind, k0, k1, xhat, bias=None):
        xhat = self.ring(xhat)
        n = xhat.size
        dx = to_dev(xhat)
        db = to_dev(self.ring(bias)) if bias is not None else None
        ncol = int(np.asarray(bias).size) if bias is not None else 0
        out = empty_dev(n * xhat.itemsize)
        self.check(self.lib.mpcx_tr_eval(self.h, kind, n, dptr(k0), dptr(k1), dptr(dx), dptr(db), ncol, dptr(out)),
                   "tr_eval")
        return from_dev(out, self.T, n)

    def maxpool_keygen(self, B, N, C, in_mask, seed=1, gate=1):
        in_mask = self.ring(in_mask)
        nb = self.lib.mpcx_maxpool_key_bytes(self.h, B, N, C)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        dm = to_dev(in_mask)
        out = empty_dev(B * C * in_mask.itemsize)
        self.check(self.lib.mpcx_maxpool_keygen(self.h, B, N, C, dptr(dm), dptr(out), seed, gate, dptr(k0),
                                                dptr(k1)), "maxpool_keygen")
        return k0, k1, from_dev(out, self.T, B * C)

    def maxpool_eval(self, B, N, C, k0, k1, xhat):
        xhat = self.ring(xhat)
        dx = to_dev(xhat)
        out = empty_dev(B * C * xhat.itemsize)
        self.check(self.lib.mpcx_maxpool_eval(self.h, B, N, C, dptr(k0), dptr(k1), dptr(dx), dptr(out)),
                   "maxpool_eval")
        return from_dev(out, self.T, B * C)

    def maxpool_eval_noalloc(self, B, N, C, k0, k1, xhat):
        """mpcx_maxpool_eval_noalloc: the same evaluation on the library's static
        device scratch array (no allocation inside the call, no synchronisation)."""
        xhat = self.ring(xhat)
        dx = to_dev(xhat)
        out = empty_dev(B * C * xhat.itemsize)
        self.check(self.lib.mpcx_maxpool_eval_noalloc(self.h, B, N, C, dptr(k0), dptr(k1), dptr(dx), dptr(out)),
                   "maxpool_eval_noalloc")
        self.sync()
        return from_dev(out, self.T, B * C)

    def mul_keygen(self, rx, ry, ia, ib, seed=1, gate=1):
        rx, ry = self.ring(rx), self.ring(ry)
        ia = np.ascontiguousarray(ia, np.uint32)
        ib = np.ascontiguousarray(ib, np.uint32)
        nx, ny, nz = rx.size, ry.size, ia.size
        nb = self.lib.mpcx_mul_key_bytes(self.h, nx, ny, nz)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        d = [to_dev(v) for v in (ia, ib, rx, ry)]
        rz = empty_dev(nz * rx.itemsize)
        self.check(self.lib.mpcx_mul_keygen(self.h, nx, ny, nz, *[dptr(v) for v in d], dptr(rz), seed, gate,
                                            dptr(k0), dptr(k1)), "mul_keygen")
        return k0, k1, from_dev(rz, self.T, nz)

    def mul_eval(self, k0, k1, xhat, yhat, ia, ib):
        xhat, yhat = self.ring(xhat), self.ring(yhat)
        ia = np.ascontiguousarray(ia, np.uint32)
        ib = np.ascontiguousarray(ib, np.uint32)
        nz = ia.size
        d = [to_dev(v) for v in (ia, ib)]
        dx, dy = to_dev(xhat), to_dev(yhat)
        out = empty_dev(nz * xhat.itemsize)
        self.check(self.lib.mpcx_mul_eval(self.h, xhat.size, yhat.size, nz, dptr(d[0]), dptr(d[1]), dptr(k0),
                                          dptr(k1), dptr(dx), dptr(dy), dptr(out)), "mul_eval")
        return from_dev(out, self.T, nz)

    def lut8_keygen(self, in_mask, seed=1, gate=1):
        in_mask = self.ring(in_mask)
        n = in_mask.size
        nb = self.lib.mpcx_lut8_key_bytes(self.h, n)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        dm = to_dev(in_mask)
        out = empty_dev(n * in_mask.itemsize)
        self.check(self.lib.mpcx_lut8_keygen(self.h, n, dptr(dm), dptr(out), seed, gate, dptr(k0), dptr(k1)),
                   "lut8_keygen")
        return k0, k1, from_dev(out, self.T, n)

    def lut8_eval(self, k0, k1, table, xhat):
        xhat, table = self.ring(xhat), self.ring(table)
        n = xhat.size
        dx, dt = to_dev(xhat), to_dev(table)
        out = empty_dev(n * xhat.itemsize)
        self.check(self.lib.mpcx_lut8_eval(self.h, n, dptr(k0), dptr(k1), dptr(dt), dptr(dx), dptr(out)),
                   "lut8_eval")
        return from_dev(out, self.T, n)

    def sxs_keygen(self, nb, M, K, N, ra, rb, seed=1, gate=1):
        ra, rb = self.ring(ra), self.ring(rb)
        kb = self.lib.mpcx_sxs_key_bytes(self.h, nb, M, K, N)
        k0, k1 = empty_dev(kb), empty_dev(kb)
        da, db = to_dev(ra), to_dev(rb)
        rc = empty_dev(nb * M * N * ra.itemsize)
        self.check(self.lib.mpcx_sxs_keygen(self.h, nb, M, K, N, dptr(da), dptr(db), dptr(rc), seed, gate,
                                            dptr(k0), dptr(k1)), "sxs_keygen")
        return k0, k1, from_dev(rc, self.T, nb * M * N)

    def sxs_eval(self, nb, M, K, N, k0, k1, ahat, bhat):
        ahat, bhat = self.ring(ahat), self.ring(bhat)
        da, db = to_dev(ahat), to_dev(bhat)
        out = empty_dev(nb * M * N * ahat.itemsize)
        self.check(self.lib.mpcx_sxs_eval(self.h, nb, M, K, N, dptr(k0), dptr(k1), dptr(da), dptr(db), dptr(out)),
                   "sxs_eval")
        return from_dev(out, self.T, nb * M * N)

    def ring_gemm(self, A, B):
        A, B = self.ring(A), self.ring(B)
        M, K = A.shape
        N = B.shape[1]
        da, db = to_dev(A), to_dev(B)
        out = empty_dev(M * N * A.itemsize)
        self.check(self.lib.mpcx_ring_gemm(self.h, M, K, N, dptr(da), dptr(db), dptr(out)), "ring_gemm")
        return from_dev(out, self.T, M * N).reshape(M, N)

    def reveal_keygen(self, n, seed=1, gate=1):
        nb = self.lib.mpcx_reveal_key_bytes(self.h, n)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        mask = empty_dev(n * np.dtype(self.T).itemsize)
        self.check(self.lib.mpcx_reveal_keygen(self.h, n, dptr(mask), seed, gate, dptr(k0), dptr(k1)),
                   "reveal_keygen")
        return k0, k1, from_dev(mask, self.T, n)

    def reveal_eval(self, k0, k1, v0, v1):
        v0, v1 = self.ring(v0), self.ring(v1)
        d0, d1 = to_dev(v0), to_dev(v1)
        out = empty_dev(v0.size * v0.itemsize)
        self.check(self.lib.mpcx_reveal_eval(self.h, v0.size, dptr(k0), dptr(k1), dptr(d0), dptr(d1), dptr(out)),
                   "reveal_eval")
        return from_dev(out, self.T, v0.size)

    # ---------------- party mode (one party per process or thread) ----------------
    def party_tr_eval(self, peer, kind, key, xhat, bias=None):
        xhat = self.ring(xhat)
        n = xhat.size
        dx = to_dev(xhat)
        db = to_dev(self.ring(bias)) if bias is not None else None
        ncol = int(np.asarray(bias).size) if bias is not None else 0
        out = empty_dev(n * xhat.itemsize)
        self.check(self.lib.mpcx_party_tr_eval(self.h, peer.h, kind, n, dptr(key), dptr(dx), dptr(db), ncol,
                                               dptr(out)), "party_tr_eval")
        return self._party_out(out, n)

    def party_mul_eval(self, peer, key, xhat, yhat, ia, ib):
        xhat, yhat = self.ring(xhat), self.ring(yhat)
        ia = np.ascontiguousarray(ia, np.uint32)
        ib = np.ascontiguousarray(ib, np.uint32)
        nz = ia.size
        d = [to_dev(v) for v in (ia, ib)]
        dx, dy = to_dev(xhat), to_dev(yhat)
        out = empty_dev(nz * xhat.itemsize)
        self.check(self.lib.mpcx_party_mul_eval(self.h, peer.h, xhat.size, yhat.size, nz, dptr(d[0]), dptr(d[1]),
                                                dptr(key), dptr(dx), dptr(dy), dptr(out)), "party_mul_eval")
        return self._party_out(out, nz)

    def party_lut8_eval(self, peer, key, table, xhat):
        xhat, table = self.ring(xhat), self.ring(table)
        n = xhat.size
        dx, dt = to_dev(xhat), to_dev(table)
        out = empty_dev(n * xhat.itemsize)
        self.check(self.lib.mpcx_party_lut8_eval(self.h, peer.h, n, dptr(key), dptr(dt), dptr(dx), dptr(out)),
                   "party_lut8_eval")
        return self._party_out(out, n)

    def party_sxs_eval(self, peer, nb, M, K, N, key, ahat, bhat):
        ahat, bhat = self.ring(ahat), self.ring(bhat)
        da, db = to_dev(ahat), to_dev(bhat)
        out = empty_dev(nb * M * N * ahat.itemsize)
        self.check(self.lib.mpcx_party_sxs_eval(self.h, peer.h, nb, M, K, N, dptr(key), dptr(da), dptr(db),
                                                dptr(out)), "party_sxs_eval")
        return self._party_out(out, nb * M * N)

    def party_reveal_eval(self, peer, key, v):
        v = self.ring(v)
        dv = to_dev(v)
        out = empty_dev(v.size * v.itemsize)
        self.check(self.lib.mpcx_party_reveal_eval(self.h, peer.h, v.size, dptr(key), dptr(dv), dptr(out)),
                   "party_reveal_eval")
        return self._party_out(out, v.size)

    def party_reconstruct(self, peer, v):
        v = self.ring(v)
        dv = to_dev(v)
        self.check(self.lib.mpcx_party_reconstruct(self.h, peer.h, v.size, dptr(dv)), "party_reconstruct")
        return self._party_out(dv, v.size)

    # ---------------- adjacency normalisation ----------------
    def set_adjnorm_lanes(self, lanes):
        """Concurrent graph groups of the adjacency normalisation (keygen and eval
        must agree: the key set is the groups' key sets back to back)."""
        self.check(self.lib.mpcx_set_adjnorm_lanes(self.h, int(lanes)), "set_adjnorm_lanes")

    def adjnorm_keygen(self, B, N, seed=1):
        nb = self.lib.mpcx_adjnorm_key_bytes(self.h, B, N)
        k0, k1 = empty_dev(nb), empty_dev(nb)
        mask = empty_dev(B * N * N * np.dtype(self.T).itemsize)
        self.check(self.lib.mpcx_adjnorm_keygen(self.h, B, N, seed, dptr(mask), dptr(k0), dptr(k1)), "adjnorm_keygen")
        return k0, k1, mask

    def adjnorm_eval(self, B, N, nmax, k0, k1, a0, a1, as_device=False):
        """a0, a1: numpy shares or device tensors; returns masked A_norm."""
        d0 = a0 if not isinstance(a0, np.ndarray) else to_dev(self.ring(a0))
        d1 = a1 if not isinstance(a1, np.ndarray) else to_dev(self.ring(a1))
        out = empty_dev(B * N * N * np.dtype(self.T).itemsize)
        self.check(self.lib.mpcx_adjnorm_eval(self.h, B, N, nmax, dptr(k0), dptr(k1), dptr(d0), dptr(d1), dptr(out)),
                   "adjnorm_eval")
        return out if as_device else from_dev(out, self.T, B * N * N)


class Peer:
    """One party's end of the channel between the two parties (party mode)."""

    def __init__(self, handle):
        self.lib = load()
        self.h = handle

    @staticmethod
    def connect(party, path, timeout_ms=60000):
        _torch()  # torch's HIP runtime first, as for a context
        lib = load()
        h = C.c_void_p()
        st = lib.mpcx_peer_connect(int(party), os.fsencode(path), int(timeout_ms), C.byref(h))
        if st != 0:
            raise MpcxError(f"mpcx_peer_connect(party {party}, {path}) failed ({st})")
        return Peer(h)

    @staticmethod
    def pair(timeout_ms=60000):
        """Both ends of one channel (two parties as two threads of this process)."""
        _torch()  # torch's HIP runtime first, as for a context
        lib = load()
        a, b = C.c_void_p(), C.c_void_p()
        st = lib.mpcx_peer_pair(int(timeout_ms), C.byref(a), C.byref(b))
        if st != 0:
            raise MpcxError(f"mpcx_peer_pair failed ({st})")
        return Peer(a), Peer(b)

    @property
    def party(self):
        return int(self.lib.mpcx_peer_party(self.h))

    @property
    def bytes(self):
        return int(self.lib.mpcx_peer_bytes(self.h))

    @property
    def rounds(self):
        return int(self.lib.mpcx_peer_rounds(self.h))

    @property
    def transport(self):
        """2 linked in memory, 1 IPC inboxes, 0 staged through the socket, -1 undecided."""
        return int(self.lib.mpcx_peer_transport(self.h))

    def close(self):
        if self.h:
            self.lib.mpcx_peer_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PinnedBuffer:
    """Page-locked host memory from libmpcx (hipHostMalloc), viewed as uint8."""

    def __init__(self, nbytes):
        self.lib = load()
        p = C.c_void_p()
        st = self.lib.mpcx_host_alloc(int(nbytes), C.byref(p))
        if st != 0:
            raise MpcxError(f"mpcx_host_alloc({nbytes}) failed ({st})")
        self.ptr = p
        self.nbytes = int(nbytes)
        self.array = np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(p.value))

    def free(self):
        if self.ptr:
            self.array = None
            self.lib.mpcx_host_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def model_dims(d):
    """synth.Dims -> ModelDims"""
    md = ModelDims()
    md.n_nodes, md.feat, md.prot, md.lut_nmax = d.n_nodes, d.feat, d.prot, d.lut_nmax
    md.mask_scale = getattr(d, "mask_scale", 0)
    md.slack = int(getattr(d, "slack", 0))
    for i, v in enumerate(d.gcn):
        md.gcn[i] = v
    for i, v in enumerate(d.dfc):
        md.dfc[i] = v
    md.nfus = len(d.fus)
    for i, v in enumerate(d.fus):
        md.fus[i] = v
    return md


class Model:
    """The secure affinity model on one GPU (both parties)."""

    def __init__(self, ctx: Ctx, dims, weights, lanes=1):
        self.ctx = ctx
        self.lib = ctx.lib
        self.dims = dims
        self.md = model_dims(dims)
        w = np.ascontiguousarray(weights, np.int64)
        self._w = w
        h = C.c_void_p()
        ctx.check(self.lib.mpcx_model_create(ctx.h, C.byref(self.md), w.ctypes.data_as(C.c_void_p), w.size,
                                             C.byref(h)), "model_create")
        self.h = h
        if lanes != 1:
            self.set_lanes(lanes)

    def set_lanes(self, lanes):
        """Concurrent sub-batches on their own streams (drops keys and inputs)."""
        self.ctx.check(self.lib.mpcx_model_set_lanes(self.h, int(lanes)), "model_set_lanes")

    @property
    def lanes(self):
        return int(self.lib.mpcx_model_lanes(self.h))

    @staticmethod
    def lane_split(B, lanes):
        """[(sample offset, samples)] of each lane with samples."""
        out, off = [], 0
        for i in range(min(lanes, B)):
            n = B // lanes + (1 if i < B % lanes else 0)
            out.append((off, n))
            off += n
        return out

    @staticmethod
    def lane_seed(seed, i):
        return (int(seed) + i * 0x9E3779B97F4A7C15) % (1 << 64)

    def close(self):
        if self.h:
            self.lib.mpcx_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def key_bytes(self, B):
        return int(self.lib.mpcx_model_key_bytes(self.h, B))

    def keygen(self, B, seed):
        self.ctx.check(self.lib.mpcx_model_keygen(self.h, B, seed), "model_keygen")

    def import_keys(self, B, k0, k1):
        k0 = np.ascontiguousarray(k0, np.uint8)
        k1 = np.ascontiguousarray(k1, np.uint8)
        self.ctx.check(self.lib.mpcx_model_import_keys(self.h, B, k0.ctypes.data_as(C.c_void_p),
                                                       k1.ctypes.data_as(C.c_void_p), k0.size), "import_keys")

    def export_keys(self, party, B, into=None):
        """Copy party's resident key arena to host (a new array, or `into`: a
        PinnedBuffer or uint8 array of key_bytes(B))."""
        n = self.key_bytes(B)
        if into is None:
            out = np.zeros(n, np.uint8)
            ptr = out.ctypes.data_as(C.c_void_p)
        else:
            out = into
            ptr = into.ptr if isinstance(into, PinnedBuffer) else into.ctypes.data_as(C.c_void_p)
        self.ctx.check(self.lib.mpcx_model_export_keys(self.h, party, ptr, n), "export_keys")
        return out

    def release_arena(self):
        self.ctx.check(self.lib.mpcx_model_release_arena(self.h), "release_arena")

    def unique_key_bytes(self, B, party):
        return int(self.lib.mpcx_model_unique_key_bytes(self.h, B, party))

    def export_unique_keys(self, party, B, into=None):
        """Party p's packed key: a 256-byte header with the party's own PRF key,
        then its planes without those it reads from party 0's copy (party 1) and
        without those the dealer drew from its PRF key (expanded on the device
        when streamed).  Keys from keygen only."""
        n = self.unique_key_bytes(B, party)
        out = np.zeros(n, np.uint8) if into is None else into
        ptr = out.ptr if isinstance(out, PinnedBuffer) else out.ctypes.data_as(C.c_void_p)
        self.ctx.check(self.lib.mpcx_model_export_unique_keys(self.h, party, ptr, n), "export_unique_keys")
        return out

    def attach_host_keys(self, B, k0, k1, slot_bytes):
        """Stream keys from host buffers (PinnedBuffer for overlap) through two
        device slots of slot_bytes per party; each of k0, k1 is the party's
        whole arena or its packed key (export_unique_keys)."""
        self._host_keys = (k0, k1)
        p0 = k0.ptr if isinstance(k0, PinnedBuffer) else k0.ctypes.data_as(C.c_void_p)
        p1 = k1.ptr if isinstance(k1, PinnedBuffer) else k1.ctypes.data_as(C.c_void_p)
        n0 = k0.nbytes
        n1 = k1.nbytes
        self.ctx.check(self.lib.mpcx_model_attach_host_keys(self.h, B, p0, n0, p1, n1, int(slot_bytes)),
                       "attach_host_keys")

    def write_keys(self, party, path, packed=False, append=False):
        """Append (or write) the key set of the last keygen for one party to a
        file: the party's arena, or its packed key (packed=True)."""
        self.ctx.check(self.lib.mpcx_model_write_keys(self.h, party, 1 if packed else 0, os.fsencode(path),
                                                      1 if append else 0), "write_keys")

    def attach_key_files(self, B, path0, path1, slot_bytes):
        """Stream key sets from files (one set per forward, cycling) through pinned
        staging buffers filled by an I/O thread and two device slots."""
        self.ctx.check(self.lib.mpcx_model_attach_key_files(self.h, B, os.fsencode(path0), os.fsencode(path1),
                                                            int(slot_bytes)), "attach_key_files")

    def stream_stats(self):
        ch, by = C.c_int(), C.c_uint64()
        self.ctx.check(self.lib.mpcx_model_stream_stats(self.h, C.byref(ch), C.byref(by)), "stream_stats")
        return {"chunks": ch.value, "bytes_h2d": by.value}

    def set_inputs(self, B, x0, x1, a0, a1, m0, m1, prot):
        arrs = [self.ctx.ring(v) for v in (x0, x1, a0, a1, m0, m1)]
        prot = np.ascontiguousarray(prot, np.int64)
        self._inputs = arrs + [prot]
        self.ctx.check(self.lib.mpcx_model_set_inputs(self.h, B, *[a.ctypes.data_as(C.c_void_p) for a in arrs],
                                                      prot.ctypes.data_as(C.c_void_p)), "set_inputs")

    def forward(self, B):
        self.ctx.check(self.lib.mpcx_model_forward(self.h, B), "model_forward")

    def output(self, B):
        out = np.zeros(B, np.int64)
        self.ctx.check(self.lib.mpcx_model_output(self.h, B, out.ctypes.data_as(C.c_void_p)), "model_output")
        return out

    def set_party(self, peer):
        """Party mode: evaluate only peer.party's side, exchanging through peer
        (None: both parties in this process).  Drops keys and inputs."""
        self._peer = peer
        self.ctx.check(self.lib.mpcx_model_set_party(self.h, peer.h if peer is not None else None), "set_party")

    def import_party_key(self, B, key):
        key = np.ascontiguousarray(key, np.uint8)
        self.ctx.check(self.lib.mpcx_model_import_party_key(self.h, B, key.ctypes.data_as(C.c_void_p), key.size),
                       "import_party_key")

    def set_party_inputs(self, B, x, a, m, prot=None):
        arrs = [self.ctx.ring(v) for v in (x, a, m)]
        pr = np.ascontiguousarray(prot, np.int64) if prot is not None else None
        self._inputs = arrs + [pr]
        self.ctx.check(self.lib.mpcx_model_set_party_inputs(
            self.h, B, *[v.ctypes.data_as(C.c_void_p) for v in arrs],
            pr.ctypes.data_as(C.c_void_p) if pr is not None else None), "set_party_inputs")

    def profile(self, on=True):
        self.ctx.check(self.lib.mpcx_model_profile(self.h, 1 if on else 0), "profile")

    def profile_read(self):
        n = C.c_int()
        ms, el, ae, by = C.c_double(), C.c_double(), C.c_double(), C.c_double()
        self.ctx.check(self.lib.mpcx_model_profile_read(self.h, C.byref(n), C.byref(ms), C.byref(el), C.byref(ae),
                                                        C.byref(by)), "profile_read")
        gn, gms, gmac = C.c_int(), C.c_double(), C.c_double()
        self.ctx.check(self.lib.mpcx_model_profile_gemm(self.h, C.byref(gn), C.byref(gms), C.byref(gmac)),
                       "profile_gemm")
        return {"launches": n.value, "ms": ms.value, "elements": el.value, "aes_calls": ae.value,
                "hbm_bytes": by.value, "gemm_sections": gn.value, "gemm_ms": gms.value, "gemm_macs": gmac.value}
