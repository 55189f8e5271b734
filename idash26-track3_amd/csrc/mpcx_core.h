// mpcx_core.h -- host/device definitions shared by every translation unit of
// libmpcx: ring traits, key-block layouts, gate kinds, dealer PRF fields and the
// AES-128 key schedule.
//
// Key-block layouts are the on-HBM format of the FSS key arena: every gate's key
// is a sequence of 256-byte aligned structure-of-arrays planes, so that lane i of
// a wavefront reads element i of a plane (coalesced).  DCF correction words are
// stored level-major (cw[level][element]) for the same reason.  The layout is
// this library's own; the reference's keys are EzPC GPU-MPC byte streams
// (patches/EzPC-GPU-MPC.track3.patch:245-274) that are not reproduced.
#pragma once
#include <cstddef>
#include <cstdint>

namespace mpcx {

constexpr size_t kAlign = 256;
inline constexpr size_t align_up(size_t x) { return (x + (kAlign - 1)) & ~(kAlign - 1); }
// packed-bit plane words (u32), rounded up to whole u64 words
inline constexpr size_t zwords(size_t n) { return ((n + 63) / 64) * 2; }

// kinds of the truncation / ReLU gate family (the MPCX_* codes of mpcx.h)
enum GateKind : int {
  G_TR = 1,          // exact truncation (+bias), full-width sign extension
  G_TRRELU = 2,      // ReLU(trunc(x) + bias)
  G_RELU = 3,        // ReLU without truncation
  G_TRSLACK = 4,     // exact truncation for |x| < 2^(bw-2)
  G_RELUSLACK = 9,   // ReLU for |x| < 2^(bw-2-s): a (bw-2-s)-bit DCF (after TRSLACK)
  G_LOCALARS = 10,   // local arithmetic shift of the masked value and its mask (no key)
  G_DRELU = 11,      // [x >= 0] as a masked public bit: one (bw-1)-bit DCF, one round
  G_TRMOD = 12,      // floor(x/2^s) + bias, exact modulo 2^(bw-s) only: one s-bit DCF
  G_EXT = 13,        // a value known modulo 2^(bw-s) (a TRMOD output) sign-extended to bw bits
  G_EXTRELU = 14,    // ReLU of that value, sign-extended: one (bw-s-1)-bit DCF for both
  G_RELUPOOL = 15    // ReLU for |x| < 2^(bw-s), e.g. the difference of two values in
                     // [-2^(bw-s-1), 2^(bw-s-1)) (truncated ones): a (bw-s)-bit DCF
};

// Gate-kind properties of the truncation family.  A gate reads its public
// input modulo 2^tr_in_bits, shifts it right by tr_shift, and takes the sign
// from bit tr_sign_bit of the input plus 2^tr_sign_bit.
inline bool tr_ext(int kind) { return kind == G_EXT || kind == G_EXTRELU; }
inline int tr_in_bits(int kind, int bw, int s) { return tr_ext(kind) ? bw - s : bw; }
inline int tr_shift(int kind, int s) { return tr_ext(kind) ? 0 : s; }
inline bool tr_has_bias(int kind) { return kind == G_TR || kind == G_TRRELU || kind == G_TRSLACK || kind == G_TRMOD; }
inline bool tr_is_relu(int kind) {
  return kind == G_TRRELU || kind == G_RELU || kind == G_RELUSLACK || kind == G_EXTRELU || kind == G_RELUPOOL;
}
// the (sign-bit)-bit DCF "a" and the s-bit DCF "b"
inline bool tr_uses_a(int kind) { return kind != G_TRSLACK && kind != G_TRMOD && kind != G_LOCALARS; }
inline bool tr_uses_b(int kind) { return tr_has_bias(kind); }
// public cases of the output correction table G
inline int tr_ncase(int kind) {
  switch (kind) {
    case G_TR: case G_TRRELU: case G_TRSLACK: return 8;
    case G_EXT: case G_EXTRELU: return 4;
    case G_RELU: case G_RELUSLACK: case G_RELUPOOL: case G_TRMOD: return 2;
    default: return 0;
  }
}

enum Field : uint32_t {
  F_DCFA = 0x10,   // +0 root seed, +1 delta, +2 z0 bit, +3 output mask bit
  F_DCFB = 0x20,
  F_ROUT = 0x30,   // fresh output mask
  F_SPLIT = 0x40,  // +k: share 0 of plane k
  F_LUTV = 0x58,
  F_RIN = 0x60,    // input masks of reveal gates
  F_PARTY = 0x70   // party p's PRF key: dealer PRF block (p, F_PARTY, gate 0xFFFFFFFF)
};

struct DcfLayout {
  int m = 0, L = 0;
  size_t N = 0;
  size_t off_root = 0, off_cw = 0, off_leaf = 0, off_z = 0, end = 0;
};

inline DcfLayout dcf_layout(int m, size_t N, size_t base, bool with_z) {
  DcfLayout d;
  d.m = m;
  d.L = m > 7 ? m - 7 : 0;
  d.N = N;
  size_t o = align_up(base);
  d.off_root = o;
  o = align_up(o + N * 16);
  d.off_cw = o;
  o = align_up(o + size_t(d.L) * N * 16);
  d.off_leaf = o;
  o = align_up(o + N * 16);
  if (with_z) {
    d.off_z = o;
    o = align_up(o + zwords(N) * 4);
  }
  d.end = o;
  return d;
}

struct TrLayout {
  int kind = 0, bw = 0, s = 0;
  bool relu = false, use_a = false, use_b = false;
  size_t N = 0;
  DcfLayout a, b;
  size_t off_kappa = 0, off_g = 0, end = 0;
  int ncase = 0;
};

// Bit of the shifted input that carries the sign: the top bit of the input
// width, bit bw-2-s for RELUSLACK (inputs |x| < 2^(bw-2-s), e.g. a value
// truncated by TRSLACK) and bit bw-s for RELUPOOL (|x| < 2^(bw-s)).
inline int tr_sign_bit(int kind, int bw, int s) {
  return kind == G_RELUSLACK ? bw - 2 - s : kind == G_RELUPOOL ? bw - s : tr_in_bits(kind, bw, s) - 1;
}

inline TrLayout tr_layout(int kind, int bw, int s, size_t N, size_t base) {
  TrLayout t;
  t.kind = kind;
  t.bw = bw;
  t.s = s;
  t.N = N;
  t.relu = tr_is_relu(kind);
  if (kind == G_LOCALARS) {  // keyless: consumes no key bytes
    t.use_a = t.use_b = false;
    t.ncase = 0;
    t.off_g = t.end = base;
    return t;
  }
  t.use_a = tr_uses_a(kind);
  t.use_b = tr_uses_b(kind);
  const size_t tb = size_t(bw) / 8;
  size_t o = align_up(base);
  if (t.use_a) {
    t.a = dcf_layout(tr_sign_bit(kind, bw, s), N, o, true);
    o = t.a.end;
  }
  if (t.use_b) {
    t.b = dcf_layout(s, N, o, true);
    o = t.b.end;
  }
  if (t.relu) {
    t.off_kappa = o;
    o = align_up(o + N * tb);
  }
  t.ncase = tr_ncase(kind);
  t.off_g = o;
  o = align_up(o + size_t(t.ncase) * N * tb);
  t.end = o;
  return t;
}

struct MulLayout {
  size_t nx = 0, ny = 0, nz = 0;
  size_t off_rx = 0, off_ry = 0, off_c = 0, end = 0;
};
inline MulLayout mul_layout(int bw, size_t nx, size_t ny, size_t nz, size_t base) {
  MulLayout m;
  const size_t tb = size_t(bw) / 8;
  m.nx = nx;
  m.ny = ny;
  m.nz = nz;
  size_t o = align_up(base);
  m.off_rx = o;
  o = align_up(o + nx * tb);
  m.off_ry = o;
  o = align_up(o + ny * tb);
  m.off_c = o;
  o = align_up(o + nz * tb);
  m.end = o;
  return m;
}

struct Lut8Layout {
  DcfLayout dpf;
  size_t off_rv = 0, off_sig = 0, off_c = 0, end = 0;
};
inline Lut8Layout lut8_layout(int bw, size_t N, size_t base) {
  Lut8Layout l;
  const size_t tb = size_t(bw) / 8;
  l.dpf = dcf_layout(8, N, base, false);
  size_t o = l.dpf.end;
  l.off_rv = o;
  o = align_up(o + N * tb);
  l.off_sig = o;
  o = align_up(o + N * tb);
  l.off_c = o;
  o = align_up(o + N * tb);
  l.end = o;
  return l;
}

struct SxsLayout {
  size_t nb = 0, M = 0, K = 0, N = 0;
  size_t off_ra = 0, off_rb = 0, off_c = 0, end = 0;
};
inline SxsLayout sxs_layout(int bw, size_t nb, size_t M, size_t K, size_t N, size_t base) {
  SxsLayout x;
  const size_t tb = size_t(bw) / 8;
  x.nb = nb;
  x.M = M;
  x.K = K;
  x.N = N;
  size_t o = align_up(base);
  x.off_ra = o;
  o = align_up(o + nb * M * K * tb);
  x.off_rb = o;
  o = align_up(o + nb * K * N * tb);
  x.off_c = o;
  o = align_up(o + nb * M * N * tb);
  x.end = o;
  return x;
}

struct RevealLayout {
  size_t N = 0, off_r = 0, end = 0;
};
inline RevealLayout reveal_layout(int bw, size_t N, size_t base) {
  RevealLayout r;
  r.N = N;
  r.off_r = align_up(base);
  r.end = align_up(r.off_r + N * size_t(bw / 8));
  return r;
}

// ---------------- AES-128 key schedule (FIPS-197 5.2) ----------------
// Round keys as little-endian 32-bit column words: word j of round r holds the
// round-key bytes 16r+4j .. 16r+4j+3 with the first byte in the low bits, which
// is the column representation the T-table cipher works on.
struct AesRK {
  uint32_t w[44];
};

extern const uint8_t kSbox[256];
AesRK aes_expand(const uint8_t key[16]);
AesRK dealer_key(uint64_t seed);  // dealer PRF key derived from a 64-bit seed
// Party p's own PRF key (a dealer PRF output): the dealer draws every purely
// random plane of party p's truncation-family keys from it (DCF roots and output
// mask bits; for party 0 also its shares of kappa and of the G table), so that a
// party holding the 16 key bytes can expand those planes itself.
void party_key_bytes(uint64_t seed, int party, uint8_t out[16]);
AesRK party_key(uint64_t seed, int party);
extern const uint8_t kKeyH[16];   // fixed key of the tree hash H
extern const uint8_t kKeyL[16];   // fixed key of the leaf hash HL

}  // namespace mpcx
