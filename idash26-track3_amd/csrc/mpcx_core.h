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
// Bits of a gate's revealed output: a TRMOD output is known modulo 2^(bw-s)
// only, so it is revealed (and sent) reduced to bw - s bits; the others at bw.
inline int tr_out_bits(int kind, int bw, int s) { return kind == G_TRMOD ? bw - s : bw; }
// 64-bit words of n elements packed at m bits each
inline constexpr size_t packed_words(size_t n, int m) { return (n * size_t(m) + 63) / 64; }
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

// The FIPS-197 S-box: the one copy of the library (host key schedules, device T-tables).
constexpr uint8_t kSboxC[256] = {
    0x63, 0x7c, 0x77, 0x7b, 0xf2, 0x6b, 0x6f, 0xc5, 0x30, 0x01, 0x67, 0x2b, 0xfe, 0xd7, 0xab, 0x76,
    0xca, 0x82, 0xc9, 0x7d, 0xfa, 0x59, 0x47, 0xf0, 0xad, 0xd4, 0xa2, 0xaf, 0x9c, 0xa4, 0x72, 0xc0,
    0xb7, 0xfd, 0x93, 0x26, 0x36, 0x3f, 0xf7, 0xcc, 0x34, 0xa5, 0xe5, 0xf1, 0x71, 0xd8, 0x31, 0x15,
    0x04, 0xc7, 0x23, 0xc3, 0x18, 0x96, 0x05, 0x9a, 0x07, 0x12, 0x80, 0xe2, 0xeb, 0x27, 0xb2, 0x75,
    0x09, 0x83, 0x2c, 0x1a, 0x1b, 0x6e, 0x5a, 0xa0, 0x52, 0x3b, 0xd6, 0xb3, 0x29, 0xe3, 0x2f, 0x84,
    0x53, 0xd1, 0x00, 0xed, 0x20, 0xfc, 0xb1, 0x5b, 0x6a, 0xcb, 0xbe, 0x39, 0x4a, 0x4c, 0x58, 0xcf,
    0xd0, 0xef, 0xaa, 0xfb, 0x43, 0x4d, 0x33, 0x85, 0x45, 0xf9, 0x02, 0x7f, 0x50, 0x3c, 0x9f, 0xa8,
    0x51, 0xa3, 0x40, 0x8f, 0x92, 0x9d, 0x38, 0xf5, 0xbc, 0xb6, 0xda, 0x21, 0x10, 0xff, 0xf3, 0xd2,
    0xcd, 0x0c, 0x13, 0xec, 0x5f, 0x97, 0x44, 0x17, 0xc4, 0xa7, 0x7e, 0x3d, 0x64, 0x5d, 0x19, 0x73,
    0x60, 0x81, 0x4f, 0xdc, 0x22, 0x2a, 0x90, 0x88, 0x46, 0xee, 0xb8, 0x14, 0xde, 0x5e, 0x0b, 0xdb,
    0xe0, 0x32, 0x3a, 0x0a, 0x49, 0x06, 0x24, 0x5c, 0xc2, 0xd3, 0xac, 0x62, 0x91, 0x95, 0xe4, 0x79,
    0xe7, 0xc8, 0x37, 0x6d, 0x8d, 0xd5, 0x4e, 0xa9, 0x6c, 0x56, 0xf4, 0xea, 0x65, 0x7a, 0xae, 0x08,
    0xba, 0x78, 0x25, 0x2e, 0x1c, 0xa6, 0xb4, 0xc6, 0xe8, 0xdd, 0x74, 0x1f, 0x4b, 0xbd, 0x8b, 0x8a,
    0x70, 0x3e, 0xb5, 0x66, 0x48, 0x03, 0xf6, 0x0e, 0x61, 0x35, 0x57, 0xb9, 0x86, 0xc1, 0x1d, 0x9e,
    0xe1, 0xf8, 0x98, 0x11, 0x69, 0xd9, 0x8e, 0x94, 0x9b, 0x1e, 0x87, 0xe9, 0xce, 0x55, 0x28, 0xdf,
    0x8c, 0xa1, 0x89, 0x0d, 0xbf, 0xe6, 0x42, 0x68, 0x41, 0x99, 0x2d, 0x0f, 0xb0, 0x54, 0xbb, 0x16};

// FIPS-197 5.2 key expansion: at compile time for the two fixed keys (so that
// every round-key word folds into an instruction literal), at run time for the
// dealer and party keys.
constexpr AesRK aes_expand_c(const uint8_t (&key)[16]) {
  constexpr uint8_t rcon[10] = {0x01, 0x02, 0x04, 0x08, 0x10, 0x20, 0x40, 0x80, 0x1b, 0x36};
  uint8_t b[176] = {};
  for (int i = 0; i < 16; i++) b[i] = key[i];
  for (int i = 4; i < 44; i++) {
    uint8_t t[4] = {b[4 * (i - 1)], b[4 * (i - 1) + 1], b[4 * (i - 1) + 2], b[4 * (i - 1) + 3]};
    if (i % 4 == 0) {
      const uint8_t t0 = t[0];
      t[0] = uint8_t(kSboxC[t[1]] ^ rcon[i / 4 - 1]);
      t[1] = kSboxC[t[2]];
      t[2] = kSboxC[t[3]];
      t[3] = kSboxC[t0];
    }
    for (int j = 0; j < 4; j++) b[4 * i + j] = uint8_t(b[4 * (i - 4) + j] ^ t[j]);
  }
  AesRK rk{};
  for (int j = 0; j < 44; j++)
    rk.w[j] = uint32_t(b[4 * j]) | (uint32_t(b[4 * j + 1]) << 8) | (uint32_t(b[4 * j + 2]) << 16) |
              (uint32_t(b[4 * j + 3]) << 24);
  return rk;
}
constexpr uint8_t kKeyHc[16] = {'M', 'I', '3', '5', '5', 'X', '-', 'H', 'a', 'l', 'f', 'T', 'r', 'e', 'e', 'H'};
constexpr uint8_t kKeyLc[16] = {'M', 'I', '3', '5', '5', 'X', '-', 'H', 'a', 'l', 'f', 'T', 'r', 'e', 'e', 'L'};
inline AesRK aes_expand(const uint8_t key[16]) {
  uint8_t k[16];
  for (int i = 0; i < 16; i++) k[i] = key[i];
  return aes_expand_c(k);
}
struct Launch;
// The dealer's PRF key for a key set: from the 64-bit seed alone (seed, then
// seed XOR 0x9E3779B97F4A7C15, as the key bytes) or, with a 16-byte dealer key
// set on the launch configuration, the AES encryption under that key of the
// block (seed low word, seed high word, 0x4D415354, 0xFFFFFFFE): the seed then
// only names the key set and the keys rest on the 16 secret bytes.
AesRK dealer_key(const Launch &L, uint64_t seed);
// Party p's own PRF key (a dealer PRF output): the dealer draws every purely
// random plane of party p's truncation-family keys from it (DCF roots and output
// mask bits; for party 0 also its shares of kappa and of the G table), so that a
// party holding the 16 key bytes can expand those planes itself.
void party_key_bytes(const Launch &L, uint64_t seed, int party, uint8_t out[16]);
AesRK party_key(const Launch &L, uint64_t seed, int party);

}  // namespace mpcx
