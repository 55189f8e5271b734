/*
 * oracle/orc_fss.c -- function secret sharing and two-party gates, CPU
 * restatement.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * DCF: distributed comparison function [x < alpha] with XOR-shared 1-bit
 * output, evaluated as a DPF path walk that XORs the control bit of every
 * right sibling left behind (the DPF-based DCF the reference selects in
 * gpu_mpc/dpf_dcf_adapter.h:1-12, 97-104 and gpu_mpc/ddg_orca.h:11-12).
 * The DPF tree itself is the half-tree construction (Guo et al., "Half-Tree:
 * Halving the Cost of Tree Expansion in COT and DPF", EUROCRYPT 2023):
 *   sL = H(s) ^ t*CW,  sR = sL ^ s,  t = lsb(s),
 * with a global offset Delta (lsb 1) between the two parties' on-path seeds,
 * one fixed-key AES call per level, and a 128-bit leaf that packs the last
 * 7 levels (the reference's DPF keys likewise hold bin-7 AES-block correction
 * words: patches/EzPC-GPU-MPC.track3.patch:250,267-274).
 *
 * Gates (masked-public convention x^ = x + r, ddg_orca_base.h:167-205):
 *   TR / TRRELU / TRSLACK / RELU  -- ddg_orca.h:83-123 (relu, TrFloor)
 *   MUL                           -- ddg_orca.h:43-63, secure_adj_norm.h:611-651
 *   LUT8                          -- secure_adj_norm.h:495-520
 *   SXS                           -- ddg_orca_base.h:170-205
 *   REVEAL                        -- ddg_orca_base.h:72-89
 * Key coefficients: with x' = x^ + bias*2^s + 2^(n-1), h = msb(x'), rho = msb(r),
 * c = [x' mod 2^(n-1) < r mod 2^(n-1)], d = [x' mod 2^s < r mod 2^s], the wrap of x' - r
 * is w = h ? (rho & c) : (rho | c) and floor(u/2^s) = floor(x'/2^s) - floor(r/2^s) - d
 * + 2^(n-s) w for u = x + bias*2^s + 2^(n-1); the dealer tabulates everything but the
 * public floor(x'/2^s) over the 8 public cases (h, c^, d^).  The ReLU variants multiply by
 * the sign bit h ^ rho ^ c = z ^ kappa (z public, kappa shared).
 */
#include <stdlib.h>
#include <string.h>
#include "orc.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------- small helpers ---------------- */
static inline uint64_t rmask(int bw) { return bw >= 64 ? ~0ull : ((1ull << bw) - 1ull); }
static inline uint64_t ring_of(orc_blk b, int bw) {
  return ((uint64_t)b.w[0] | ((uint64_t)b.w[1] << 32)) & rmask(bw);
}
static inline void put_t(uint8_t *buf, size_t off, size_t i, int bw, uint64_t v) {
  if (bw == 32) {
    uint32_t x = (uint32_t)v;
    memcpy(buf + off + 4 * i, &x, 4);
  } else {
    memcpy(buf + off + 8 * i, &v, 8);
  }
}
static inline uint64_t get_t(const uint8_t *buf, size_t off, size_t i, int bw) {
  if (bw == 32) {
    uint32_t x;
    memcpy(&x, buf + off + 4 * i, 4);
    return x;
  }
  uint64_t v;
  memcpy(&v, buf + off + 8 * i, 8);
  return v;
}
static inline void put_blk(uint8_t *buf, size_t off, size_t i, orc_blk b) {
  memcpy(buf + off + 16 * i, b.w, 16);
}
static inline orc_blk get_blk(const uint8_t *buf, size_t off, size_t i) {
  orc_blk b;
  memcpy(b.w, buf + off + 16 * i, 16);
  return b;
}
static inline orc_blk bxor(orc_blk a, orc_blk b) {
  orc_blk r;
  for (int k = 0; k < 4; k++) r.w[k] = a.w[k] ^ b.w[k];
  return r;
}
static inline orc_blk bsel(int t, orc_blk a) { /* t ? a : 0 */
  orc_blk r;
  uint32_t m = t ? 0xffffffffu : 0u;
  for (int k = 0; k < 4; k++) r.w[k] = a.w[k] & m;
  return r;
}
static inline int getbit(const uint8_t *buf, size_t off, size_t i) {
  uint32_t w;
  memcpy(&w, buf + off + 4 * (i / 32), 4);
  return (int)((w >> (i % 32)) & 1u);
}
static inline void setbit(uint8_t *buf, size_t off, size_t i, int v) {
  uint32_t w;
  memcpy(&w, buf + off + 4 * (i / 32), 4);
  w = (w & ~(1u << (i % 32))) | ((uint32_t)(v & 1) << (i % 32));
  memcpy(buf + off + 4 * (i / 32), &w, 4);
}
static inline int prf_bit(const orc_prf *P, uint32_t g, uint32_t f, uint64_t i) {
  return (int)(orc_prf_blk(P, g, f, i).w[0] & 1u);
}
static inline uint64_t prf_ring(const orc_prf *P, uint32_t g, uint32_t f, uint64_t i, int bw) {
  return ring_of(orc_prf_blk(P, g, f, i), bw);
}
static size_t bitplane_bytes(size_t N) { return ((N + 31) / 32) * 4; }
/* a message of N elements known modulo 2^m (m < bw) goes out packed at m bits
 * per element in 64-bit words (gpu_mpc/utils/gpu_comms.h:143-168: compressMem's
 * ((N m - 1) / 64 + 1) * 8 bytes for a truncate-reduce output revealed at
 * bout = bin - shift bits, gpu_mpc/dpf_dcf_adapter.h:297) */
static uint64_t msg_bytes(size_t N, int m, int bw) {
  return m < bw ? (((uint64_t)N * (uint64_t)m + 63) / 64) * 8 : (uint64_t)N * (uint64_t)(bw / 8);
}

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}
#define OMP_FOR _Pragma("omp parallel for schedule(static) num_threads(orc_get_threads())")

/* ---------------- layouts ---------------- */
size_t orc_align(size_t x) { return (x + (ORC_ALIGN - 1)) & ~(size_t)(ORC_ALIGN - 1); }
size_t orc_zwords(size_t N) { return ((N + 63) / 64) * 2; }

orc_dcf_layout orc_dcf_layout_make(int m, size_t N, size_t base, int with_z) {
  orc_dcf_layout L;
  L.m = m;
  L.L = m > 7 ? m - 7 : 0;
  L.N = N;
  size_t o = orc_align(base);
  L.off_root = o;
  o = orc_align(o + N * 16);
  L.off_cw = o;
  o = orc_align(o + (size_t)L.L * N * 16);
  L.off_leaf = o;
  o = orc_align(o + N * 16);
  if (with_z) {
    L.off_z = o;
    o = orc_align(o + orc_zwords(N) * 4);
  } else {
    L.off_z = 0;
  }
  L.end = o;
  return L;
}

/* EXT kinds read their input modulo 2^(bw-s) and do not shift; every other
 * kind reads all bw bits and shifts by s (the reference's TrFloor is the
 * truncate-reduce then the sign extension, gpu_mpc/dpf_dcf_adapter.h:274-303;
 * its ReLU-extend gpuReluExtend, :225-234, takes bin = bw - scale) */
static int is_ext(int kind) { return kind == ORC_G_EXT || kind == ORC_G_EXTRELU; }
static int in_bits(int kind, int bw, int s) { return is_ext(kind) ? bw - s : bw; }
static int own_shift(int kind, int s) { return is_ext(kind) ? 0 : s; }
static int has_bias(int kind) {
  return kind == ORC_G_TR || kind == ORC_G_TRRELU || kind == ORC_G_TRSLACK || kind == ORC_G_TRMOD;
}
static int uses_a(int kind) { return kind != ORC_G_TRSLACK && kind != ORC_G_TRMOD; }
static int is_relu(int kind) {
  return kind == ORC_G_TRRELU || kind == ORC_G_RELU || kind == ORC_G_RELUSLACK || kind == ORC_G_EXTRELU ||
         kind == ORC_G_RELUPOOL;
}
static int ncase_of(int kind) {
  switch (kind) {
    case ORC_G_TR: case ORC_G_TRRELU: case ORC_G_TRSLACK: return 8;
    case ORC_G_EXT: case ORC_G_EXTRELU: return 4;
    case ORC_G_RELU: case ORC_G_RELUSLACK: case ORC_G_RELUPOOL: case ORC_G_TRMOD: return 2;
    default: return 0;
  }
}

/* bit of the shifted input that carries the sign: the top bit of the input
 * width, bit bw-2-s for RELUSLACK (inputs |x| < 2^(bw-2-s), e.g. a value
 * truncated by TRSLACK) and bit bw-s for RELUPOOL (|x| < 2^(bw-s)) */
int orc_sign_bit(int kind, int bw, int s) {
  return kind == ORC_G_RELUSLACK ? bw - 2 - s : kind == ORC_G_RELUPOOL ? bw - s : in_bits(kind, bw, s) - 1;
}

orc_tr_layout orc_tr_layout_make(int kind, int bw, int s, size_t N, size_t base) {
  orc_tr_layout T;
  memset(&T, 0, sizeof(T));
  T.kind = kind;
  T.bw = bw;
  T.s = s;
  T.N = N;
  T.relu = is_relu(kind);
  if (kind == ORC_G_LOCALARS) { /* keyless: consumes no key bytes */
    T.off_g = T.end = base;
    return T;
  }
  size_t o = orc_align(base);
  size_t tb = (size_t)bw / 8;
  if (uses_a(kind)) {
    T.a = orc_dcf_layout_make(orc_sign_bit(kind, bw, s), N, o, 1);
    o = T.a.end;
  }
  if (has_bias(kind)) {
    T.b = orc_dcf_layout_make(s, N, o, 1);
    o = T.b.end;
  }
  if (T.relu) {
    T.off_kappa = o;
    o = orc_align(o + N * tb);
  }
  T.ncase = ncase_of(kind);
  T.off_g = o;
  o = orc_align(o + (size_t)T.ncase * N * tb);
  T.end = o;
  return T;
}

/* ---------------- DCF ---------------- */
static uint32_t bits_above(int j) { return j >= 31 ? 0u : (0xffffffffu << (j + 1)); }

/* parity of the bits of blk at positions > pos (pos in [0,127]) */
static int parity_above(orc_blk b, int pos) {
  uint32_t acc = 0;
  for (int k = 0; k < 4; k++) {
    int lo = 32 * k;
    uint32_t m;
    if (pos < lo)
      m = 0xffffffffu;
    else if (pos >= lo + 31)
      m = 0u;
    else
      m = bits_above(pos - lo);
    acc ^= b.w[k] & m;
  }
  return __builtin_parity(acc);
}

/* Dealer walk from the parties' roots s0 (lsb 0) and s1 (lsb 1), D = s0 ^ s1. */
static void dcf_gen_roots(orc_blk s0, orc_blk s1, const orc_dcf_layout *L, uint64_t alpha, size_t i,
                          uint8_t *k0, uint8_t *k1) {
  const int m = L->m;
  const orc_blk D = bxor(s0, s1);
  put_blk(k0, L->off_root, i, s0);
  put_blk(k1, L->off_root, i, s1);
  int t0 = 0, t1 = 1;
  for (int l = 0; l < L->L; l++) {
    int a = (int)((alpha >> (m - 1 - l)) & 1u);
    orc_blk h0 = orc_H(s0), h1 = orc_H(s1);
    orc_blk cw = bxor(h0, h1);
    if (!a) cw = bxor(cw, D);
    put_blk(k0, L->off_cw, (size_t)l * L->N + i, cw);
    put_blk(k1, L->off_cw, (size_t)l * L->N + i, cw);
    orc_blk sl0 = bxor(h0, bsel(t0, cw)), sl1 = bxor(h1, bsel(t1, cw));
    if (a) {
      s0 = bxor(sl0, s0);
      s1 = bxor(sl1, s1);
    } else {
      s0 = sl0;
      s1 = sl1;
    }
    t0 = (int)(s0.w[0] & 1u);
    t1 = (int)(s1.w[0] & 1u);
  }
  int pos = (int)(m >= 7 ? (alpha & 127u) : alpha);
  orc_blk lcw = bxor(orc_HL(s0), orc_HL(s1));
  lcw.w[pos / 32] ^= 1u << (pos % 32);
  put_blk(k0, L->off_leaf, i, lcw);
  put_blk(k1, L->off_leaf, i, lcw);
}

/* Roots from the dealer PRF: s0 = PRF(fb) with lsb 0, s1 = s0 ^ D, D = PRF(fb+1) | 1. */
static void dcf_gen1(const orc_prf *P, uint32_t gate, uint32_t fb, const orc_dcf_layout *L,
                     uint64_t alpha, size_t i, uint8_t *k0, uint8_t *k1) {
  orc_blk s0 = orc_prf_blk(P, gate, fb + 0, i);
  s0.w[0] &= ~1u;
  orc_blk D = orc_prf_blk(P, gate, fb + 1, i);
  D.w[0] |= 1u;
  dcf_gen_roots(s0, bxor(s0, D), L, alpha, i, k0, k1);
}

/* Party p's own PRF key: the dealer PRF block (p, ORC_F_PARTY, gate 0xFFFFFFFF)
 * as an AES-128 key.  The dealer draws every purely random plane of party p's
 * truncation-family keys from it (DCF roots and output-mask bits; for party 0
 * also its shares of kappa and of the G table). */
void orc_party_key(uint64_t seed, int party, uint8_t key[16]) {
  orc_prf P;
  orc_prf_init(&P, seed);
  orc_blk b = orc_prf_blk(&P, 0xFFFFFFFFu, ORC_F_PARTY, (uint64_t)party);
  for (int j = 0; j < 4; j++)
    for (int k = 0; k < 4; k++) key[4 * j + k] = (uint8_t)(b.w[j] >> (8 * k));
}
static void party_prf(uint64_t seed, int party, orc_prf *Pp) {
  uint8_t key[16];
  orc_party_key(seed, party, key);
  orc_aes_expand(key, Pp->rk);
}
/* root of party p: its PRF block with lsb = p */
static orc_blk party_root(const orc_prf *Pp, int p, uint32_t gate, uint32_t fb, size_t i) {
  orc_blk s = orc_prf_blk(Pp, gate, fb + 0, i);
  s.w[0] = (s.w[0] & ~1u) | (uint32_t)p;
  return s;
}
/* DCF key of a truncation-family gate: roots and output-mask bits from the
 * parties' own PRF keys (rbit = z0 ^ z1 was computed by the caller the same way) */
static void dcf_keygen_parties(const orc_prf *P0, const orc_prf *P1, uint32_t gate, uint32_t fb, int m,
                               size_t N, const uint64_t *alpha, uint8_t *k0, uint8_t *k1, size_t base) {
  orc_dcf_layout L = orc_dcf_layout_make(m, N, base, 1);
  OMP_FOR
  for (size_t i = 0; i < N; i++)
    dcf_gen_roots(party_root(P0, 0, gate, fb, i), party_root(P1, 1, gate, fb, i), &L, alpha[i], i, k0, k1);
  memset(k0 + L.off_z, 0, orc_zwords(N) * 4);
  memset(k1 + L.off_z, 0, orc_zwords(N) * 4);
  for (size_t i = 0; i < N; i++) {
    setbit(k0, L.off_z, i, prf_bit(P0, gate, fb + 2, i));
    setbit(k1, L.off_z, i, prf_bit(P1, gate, fb + 2, i));
  }
}

void orc_dcf_keygen(uint64_t seed, uint32_t gate, uint32_t fbase, int m, size_t N,
                    const uint64_t *alpha, const uint8_t *rbit, uint8_t *k0, uint8_t *k1,
                    size_t base) {
  orc_prf P;
  orc_prf_init(&P, seed);
  orc_dcf_layout L = orc_dcf_layout_make(m, N, base, 1);
  OMP_FOR
  for (size_t i = 0; i < N; i++) dcf_gen1(&P, gate, fbase, &L, alpha[i], i, k0, k1);
  memset(k0 + L.off_z, 0, orc_zwords(N) * 4);
  memset(k1 + L.off_z, 0, orc_zwords(N) * 4);
  for (size_t i = 0; i < N; i++) {
    int z0 = prf_bit(&P, gate, fbase + 2, i);
    int rb = rbit ? (rbit[i] & 1) : 0;
    setbit(k0, L.off_z, i, z0);
    setbit(k1, L.off_z, i, z0 ^ rb);
  }
}

int orc_dcf_eval1(int party, const uint8_t *key, const orc_dcf_layout *L, size_t i,
                  uint64_t x) {
  const int m = L->m;
  orc_blk s = get_blk(key, L->off_root, i);
  int t = (int)(s.w[0] & 1u);
  (void)party;
  int out = 0;
  for (int l = 0; l < L->L; l++) {
    int bit = (int)((x >> (m - 1 - l)) & 1u);
    orc_blk h = orc_H(s);
    orc_blk sl = bxor(h, bsel(t, get_blk(key, L->off_cw, (size_t)l * L->N + i)));
    int tl = (int)(sl.w[0] & 1u);
    if (!bit) {
      out ^= tl ^ t; /* control bit of the right sibling */
      s = sl;
      t = tl;
    } else {
      s = bxor(sl, s);
      t = tl ^ t;
    }
  }
  orc_blk lb = bxor(orc_HL(s), bsel(t, get_blk(key, L->off_leaf, i)));
  int pos = (int)(m >= 7 ? (x & 127u) : x);
  out ^= parity_above(lb, pos);
  if (L->off_z) out ^= getbit(key, L->off_z, i);
  return out;
}

void orc_dcf_eval(int party, int m, size_t N, const uint8_t *key, size_t base,
                  const uint64_t *x, uint8_t *out) {
  orc_dcf_layout L = orc_dcf_layout_make(m, N, base, 1);
  OMP_FOR
  for (size_t i = 0; i < N; i++) out[i] = (uint8_t)orc_dcf_eval1(party, key, &L, i, x[i]);
}

/* Full-domain DPF expansion: bits[k] for k in [0, 2^m), m >= 7. */
void orc_dpf_full_eval(int party, int m, const uint8_t *key, const orc_dcf_layout *L,
                       size_t i, uint8_t *bits) {
  (void)party;
  int nleaf = 1 << L->L;
  orc_blk *lvl = (orc_blk *)malloc(sizeof(orc_blk) * (size_t)nleaf);
  orc_blk *nxt = (orc_blk *)malloc(sizeof(orc_blk) * (size_t)nleaf);
  lvl[0] = get_blk(key, L->off_root, i);
  int cnt = 1;
  for (int l = 0; l < L->L; l++) {
    orc_blk cw = get_blk(key, L->off_cw, (size_t)l * L->N + i);
    for (int j = 0; j < cnt; j++) {
      orc_blk s = lvl[j];
      int t = (int)(s.w[0] & 1u);
      orc_blk sl = bxor(orc_H(s), bsel(t, cw));
      nxt[2 * j] = sl;
      nxt[2 * j + 1] = bxor(sl, s);
    }
    cnt *= 2;
    orc_blk *tmp = lvl;
    lvl = nxt;
    nxt = tmp;
  }
  orc_blk leaf = get_blk(key, L->off_leaf, i);
  int per = m >= 7 ? 128 : (1 << m);
  for (int j = 0; j < cnt; j++) {
    int t = (int)(lvl[j].w[0] & 1u);
    orc_blk lb = bxor(orc_HL(lvl[j]), bsel(t, leaf));
    for (int k = 0; k < per; k++) bits[j * per + k] = (uint8_t)((lb.w[k / 32] >> (k % 32)) & 1u);
  }
  free(lvl);
  free(nxt);
}

/* ---------------- TR / TRRELU / RELU / TRSLACK ---------------- */
/* Arithmetic right shift by s of a bw-bit ring element (sign-extended from bit
 * bw-1), reduced mod 2^bw. */
static uint64_t ars_bw(uint64_t v, int bw, int s) {
  const int64_t sv = bw >= 64 ? (int64_t)v : (int64_t)(v << (64 - bw)) >> (64 - bw);
  return (uint64_t)(sv >> s) & rmask(bw);
}

/* LocalARS (TruncateType::LocalARS, the default of DDGOrcaBatched::truncateForward,
 * gpu_mpc/ddg_orca_batched.h:180-199 and keygen :273-277): both parties shift the
 * public masked value, the dealer shifts the mask.  No key bytes, no exchange.
 * y^ - r_y = floor(x/2^s) + b + e, e in {0, 1} (the carry of the low s bits of
 * x + r), minus 2^(bw-s) when x + r leaves the signed ring (probability about
 * |x| / 2^bw for a uniform mask). */
static void local_ars_keygen(int bw, int s, size_t N, const uint64_t *in_mask, uint64_t *out_mask) {
  for (size_t i = 0; i < N; i++) out_mask[i] = ars_bw(in_mask[i] & rmask(bw), bw, s);
}
static void local_ars_eval(int bw, int s, size_t N, const uint64_t *xhat, const int64_t *bias_elem,
                           uint64_t *yhat) {
  for (size_t i = 0; i < N; i++)
    yhat[i] = (ars_bw(xhat[i] & rmask(bw), bw, s) + (bias_elem ? (uint64_t)bias_elem[i] : 0)) & rmask(bw);
}

void orc_tr_keygen(uint64_t seed, uint32_t gate, int kind, int bw, int s, size_t N,
                   const uint64_t *in_mask, uint64_t *out_mask, uint8_t *k0, uint8_t *k1,
                   size_t base) {
  if (kind == ORC_G_LOCALARS) {
    local_ars_keygen(bw, s, N, in_mask, out_mask);
    return;
  }
  orc_prf P, P0, P1;
  orc_prf_init(&P, seed);
  party_prf(seed, 0, &P0);
  party_prf(seed, 1, &P1);
  orc_tr_layout T = orc_tr_layout_make(kind, bw, s, N, base);
  const uint64_t M = rmask(bw);
  const int n = bw, sb = orc_sign_bit(kind, bw, s);
  const int m = in_bits(kind, bw, s), sh = own_shift(kind, s);
  const int relu_like = kind == ORC_G_RELU || kind == ORC_G_RELUSLACK || kind == ORC_G_RELUPOOL;
  const int no_b = !has_bias(kind); /* no s-bit DCF */
  const int use_a = uses_a(kind);
  const uint64_t lowmask = (1ull << sb) - 1ull;
  const uint64_t smask = (1ull << s) - 1ull;
  uint64_t *aa = (uint64_t *)calloc(N, 8), *ab = (uint64_t *)calloc(N, 8);
  OMP_FOR
  for (size_t i = 0; i < N; i++) {
    uint64_t r = in_mask[i] & rmask(m);
    int rho = (int)((r >> sb) & 1u);
    uint64_t R = r >> sh;
    /* the DCF output masks: XOR of the parties' own mask bits */
    int rbi = use_a ? prf_bit(&P0, gate, ORC_F_DCFA + 2, i) ^ prf_bit(&P1, gate, ORC_F_DCFA + 2, i) : 0;
    int rdi = !no_b ? prf_bit(&P0, gate, ORC_F_DCFB + 2, i) ^ prf_bit(&P1, gate, ORC_F_DCFB + 2, i) : 0;
    aa[i] = r & lowmask;
    ab[i] = r & smask;
    uint64_t rout = prf_ring(&P, gate, ORC_F_ROUT, i, bw);
    int kappa = rho ^ rbi;
    /* DRELU: the output is the public bit h ^ c^, whose mask is kappa */
    out_mask[i] = kind == ORC_G_DRELU ? (uint64_t)kappa : rout;
    for (int c = 0; c < T.ncase; c++) {
      uint64_t G = 0;
      if (kind == ORC_G_TRMOD) { /* no wrap term: exact modulo 2^(n-s) */
        G = rout - R - (uint64_t)(c ^ rdi);
      } else if (is_ext(kind)) { /* cases (h, c^); the wrap has weight 2^m */
        int h = c >> 1, b = (c & 1) ^ rbi;
        int w = h ? (rho & b) : (rho | b);
        uint64_t cc = kind == ORC_G_EXTRELU ? (uint64_t)(h ^ rho ^ b) : 1u;
        G = rout - cc * R + ((cc * (uint64_t)w) << m);
      } else if (kind == ORC_G_TR || kind == ORC_G_TRRELU) {
        int h = c >> 2, bh = (c >> 1) & 1, dh = c & 1;
        int b = bh ^ rbi, d = dh ^ rdi;
        int w = h ? (rho & b) : (rho | b);
        if (kind == ORC_G_TRRELU) {
          uint64_t cc = (uint64_t)(h ^ rho ^ b);
          G = rout - cc * R - cc * (uint64_t)d + ((cc * (uint64_t)w) << (n - s));
        } else {
          G = rout - R - (uint64_t)d + ((uint64_t)w << (n - s));
        }
      } else if (relu_like) {
        uint64_t cc = (uint64_t)(c ^ kappa);
        G = rout - cc * r;
      } else { /* TRSLACK */
        int Hh = c >> 1, dh = c & 1;
        int d = dh ^ rdi;
        int R2 = (int)(r >> (n - 2));
        int w = Hh < R2;
        G = rout - R - (uint64_t)d + ((uint64_t)w << (n - s));
      }
      G &= M;
      uint64_t g0 = prf_ring(&P0, gate, ORC_F_SPLIT + (uint32_t)c, i, bw);
      put_t(k0, T.off_g, (size_t)c * N + i, bw, g0);
      put_t(k1, T.off_g, (size_t)c * N + i, bw, (G - g0) & M);
    }
    if (T.relu) {
      uint64_t q0 = prf_ring(&P0, gate, ORC_F_SPLIT + 8, i, bw);
      put_t(k0, T.off_kappa, i, bw, q0);
      put_t(k1, T.off_kappa, i, bw, ((uint64_t)kappa - q0) & M);
    }
  }
  if (use_a) dcf_keygen_parties(&P0, &P1, gate, ORC_F_DCFA, sb, N, aa, k0, k1, T.a.off_root);
  if (!no_b) dcf_keygen_parties(&P0, &P1, gate, ORC_F_DCFB, s, N, ab, k0, k1, T.b.off_root);
  free(aa);
  free(ab);
}

void orc_tr_eval(int kind, int bw, int s, size_t N, const uint8_t *k0, const uint8_t *k1,
                 size_t base, const uint64_t *xhat, const int64_t *bias_elem,
                 uint64_t *yhat, uint64_t *bytes) {
  if (kind == ORC_G_LOCALARS) {
    local_ars_eval(bw, s, N, xhat, bias_elem, yhat);
    return;
  }
  orc_tr_layout T = orc_tr_layout_make(kind, bw, s, N, base);
  const uint64_t M = rmask(bw);
  const int n = bw, sb = orc_sign_bit(kind, bw, s);
  const int m = in_bits(kind, bw, s), sh = own_shift(kind, s);
  const int relu_like = kind == ORC_G_RELU || kind == ORC_G_RELUSLACK || kind == ORC_G_RELUPOOL;
  const uint64_t lowmask = (1ull << sb) - 1ull;
  const uint64_t smask = (1ull << s) - 1ull;
  const int use_a = uses_a(kind), use_b = has_bias(kind);
  uint8_t *bb[2], *dd[2];
  for (int p = 0; p < 2; p++) {
    bb[p] = (uint8_t *)calloc(N, 1);
    dd[p] = (uint8_t *)calloc(N, 1);
  }
  const uint8_t *K[2] = {k0, k1};
  /* phase 1: each party evaluates its DCF keys on the public x^' */
  for (int p = 0; p < 2; p++) {
    OMP_FOR
    for (size_t i = 0; i < N; i++) {
      uint64_t b = (use_b && bias_elem) ? ((uint64_t)bias_elem[i] << s) : 0;
      uint64_t xp = (xhat[i] + b + (1ull << sb)) & rmask(m);
      if (use_a) bb[p][i] = (uint8_t)orc_dcf_eval1(p, K[p], &T.a, i, xp & lowmask);
      if (use_b) dd[p][i] = (uint8_t)orc_dcf_eval1(p, K[p], &T.b, i, xp & smask);
    }
  }
  if (bytes) *bytes += 2ull * ((use_a ? bitplane_bytes(N) : 0) + (use_b ? bitplane_bytes(N) : 0));
  /* phase 2: exchange the masked bits, compute the output shares */
  uint64_t *y[2];
  for (int p = 0; p < 2; p++) y[p] = (uint64_t *)calloc(N, 8);
  for (int p = 0; p < 2; p++) {
    OMP_FOR
    for (size_t i = 0; i < N; i++) {
      uint64_t b = (use_b && bias_elem) ? ((uint64_t)bias_elem[i] << s) : 0;
      uint64_t xp = (xhat[i] + b + (1ull << sb)) & rmask(m);
      int h = (int)((xp >> sb) & 1u);
      int bh = bb[0][i] ^ bb[1][i];
      int dh = dd[0][i] ^ dd[1][i];
      uint64_t A = ((xp >> sh) - (1ull << (m - 1 - sh))) & M;
      uint64_t out;
      if (kind == ORC_G_TRMOD) {
        out = (p == 0 ? A : 0) + get_t(K[p], T.off_g, (size_t)dh * N + i, bw);
      } else if (is_ext(kind)) {
        uint64_t G = get_t(K[p], T.off_g, (size_t)(h * 2 + bh) * N + i, bw);
        if (kind == ORC_G_EXTRELU) {
          int z = h ^ bh;
          uint64_t kap = get_t(K[p], T.off_kappa, i, bw);
          uint64_t cp = z ? ((uint64_t)(p == 0) - kap) : kap;
          out = cp * A + G;
        } else {
          out = (p == 0 ? A : 0) + G;
        }
      } else if (kind == ORC_G_TR || kind == ORC_G_TRRELU) {
        int c = h * 4 + bh * 2 + dh;
        uint64_t G = get_t(K[p], T.off_g, (size_t)c * N + i, bw);
        if (kind == ORC_G_TRRELU) {
          int z = h ^ bh;
          uint64_t kap = get_t(K[p], T.off_kappa, i, bw);
          uint64_t cp = z ? ((uint64_t)(p == 0) - kap) : kap;
          out = cp * A + G;
        } else {
          out = (p == 0 ? A : 0) + G;
        }
      } else if (kind == ORC_G_DRELU) { /* public: party 0 carries it, no message */
        out = p == 0 ? (uint64_t)(h ^ bh) : 0;
      } else if (relu_like) {
        int z = h ^ bh;
        uint64_t G = get_t(K[p], T.off_g, (size_t)z * N + i, bw);
        uint64_t kap = get_t(K[p], T.off_kappa, i, bw);
        uint64_t cp = z ? ((uint64_t)(p == 0) - kap) : kap;
        out = cp * xhat[i] + G;
      } else {
        int Hh = (int)(xp >> (n - 2));
        int c = Hh * 2 + dh;
        uint64_t G = get_t(K[p], T.off_g, (size_t)c * N + i, bw);
        out = (p == 0 ? A : 0) + G;
      }
      y[p][i] = out & M;
    }
  }
  /* TRMOD's output is known modulo 2^(n-s) only: revealed (and sent) at n - s bits */
  const int ob = kind == ORC_G_TRMOD ? n - s : n;
  if (bytes && kind != ORC_G_DRELU) *bytes += 2ull * msg_bytes(N, ob, bw);
  for (size_t i = 0; i < N; i++) yhat[i] = (y[0][i] + y[1][i]) & rmask(ob);
  for (int p = 0; p < 2; p++) {
    free(bb[p]);
    free(dd[p]);
    free(y[p]);
  }
}

/* ---------------- Beaver MUL ---------------- */
size_t orc_mul_layout(int bw, size_t nx, size_t ny, size_t nz, size_t base, size_t *off_rx,
                      size_t *off_ry, size_t *off_c) {
  size_t tb = (size_t)bw / 8, o = orc_align(base);
  *off_rx = o;
  o = orc_align(o + nx * tb);
  *off_ry = o;
  o = orc_align(o + ny * tb);
  *off_c = o;
  o = orc_align(o + nz * tb);
  return o;
}

void orc_mul_keygen(uint64_t seed, uint32_t gate, int bw, size_t nx, size_t ny, size_t nz,
                    const uint32_t *ia, const uint32_t *ib, const uint64_t *rx,
                    const uint64_t *ry, uint64_t *rz, uint8_t *k0, uint8_t *k1, size_t base) {
  orc_prf P;
  orc_prf_init(&P, seed);
  const uint64_t M = rmask(bw);
  size_t orx, ory, oc;
  orc_mul_layout(bw, nx, ny, nz, base, &orx, &ory, &oc);
  OMP_FOR
  for (size_t i = 0; i < nx; i++) {
    uint64_t a0 = prf_ring(&P, gate, ORC_F_SPLIT + 0, i, bw);
    put_t(k0, orx, i, bw, a0);
    put_t(k1, orx, i, bw, (rx[i] - a0) & M);
  }
  OMP_FOR
  for (size_t i = 0; i < ny; i++) {
    uint64_t b0 = prf_ring(&P, gate, ORC_F_SPLIT + 1, i, bw);
    put_t(k0, ory, i, bw, b0);
    put_t(k1, ory, i, bw, (ry[i] - b0) & M);
  }
  OMP_FOR
  for (size_t i = 0; i < nz; i++) {
    uint64_t r = prf_ring(&P, gate, ORC_F_ROUT, i, bw);
    rz[i] = r;
    uint64_t C = (rx[ia[i]] * ry[ib[i]] + r) & M;
    uint64_t c0 = prf_ring(&P, gate, ORC_F_SPLIT + 2, i, bw);
    put_t(k0, oc, i, bw, c0);
    put_t(k1, oc, i, bw, (C - c0) & M);
  }
}

void orc_mul_eval(int bw, size_t nx, size_t ny, size_t nz, const uint32_t *ia,
                  const uint32_t *ib, const uint8_t *k0, const uint8_t *k1, size_t base,
                  const uint64_t *xhat, const uint64_t *yhat, uint64_t *zhat,
                  uint64_t *bytes) {
  const uint64_t M = rmask(bw);
  size_t orx, ory, oc;
  orc_mul_layout(bw, nx, ny, nz, base, &orx, &ory, &oc);
  const uint8_t *K[2] = {k0, k1};
  uint64_t *z[2];
  for (int p = 0; p < 2; p++) {
    z[p] = (uint64_t *)calloc(nz, 8);
    OMP_FOR
    for (size_t i = 0; i < nz; i++) {
      uint64_t x = xhat[ia[i]], y = yhat[ib[i]];
      uint64_t v = (p == 0 ? x * y : 0) - x * get_t(K[p], ory, ib[i], bw) -
                   y * get_t(K[p], orx, ia[i], bw) + get_t(K[p], oc, i, bw);
      z[p][i] = v & M;
    }
  }
  if (bytes) *bytes += 2ull * nz * (uint64_t)(bw / 8);
  for (size_t i = 0; i < nz; i++) zhat[i] = (z[0][i] + z[1][i]) & M;
  free(z[0]);
  free(z[1]);
}

/* ---------------- LUT8 ---------------- */
size_t orc_lut8_layout(int bw, size_t N, size_t base, orc_dcf_layout *dpf, size_t *off_rv,
                       size_t *off_sig, size_t *off_c) {
  size_t tb = (size_t)bw / 8;
  *dpf = orc_dcf_layout_make(8, N, base, 0);
  size_t o = dpf->end;
  *off_rv = o;
  o = orc_align(o + N * tb);
  *off_sig = o;
  o = orc_align(o + N * tb);
  *off_c = o;
  o = orc_align(o + N * tb);
  return o;
}

void orc_lut8_keygen(uint64_t seed, uint32_t gate, int bw, size_t N, const uint64_t *in_mask,
                     uint64_t *out_mask, uint8_t *k0, uint8_t *k1, size_t base) {
  orc_prf P;
  orc_prf_init(&P, seed);
  const uint64_t M = rmask(bw);
  orc_dcf_layout D;
  size_t orv, osig, oc;
  orc_lut8_layout(bw, N, base, &D, &orv, &osig, &oc);
  OMP_FOR
  for (size_t i = 0; i < N; i++) {
    uint64_t alpha = in_mask[i] & 255u;
    dcf_gen1(&P, gate, ORC_F_DCFA, &D, alpha, i, k0, k1);
    uint8_t u0[256], u1[256];
    orc_dpf_full_eval(0, 8, k0, &D, i, u0);
    orc_dpf_full_eval(1, 8, k1, &D, i, u1);
    uint64_t sigma = u0[alpha] ? 1u : M; /* +1 or -1 */
    uint64_t rv = prf_ring(&P, gate, ORC_F_LUTV, i, bw);
    uint64_t rout = prf_ring(&P, gate, ORC_F_ROUT, i, bw);
    out_mask[i] = rout;
    uint64_t C = (rout - sigma * rv) & M;
    uint64_t v0 = prf_ring(&P, gate, ORC_F_SPLIT + 0, i, bw);
    uint64_t s0 = prf_ring(&P, gate, ORC_F_SPLIT + 1, i, bw);
    uint64_t c0 = prf_ring(&P, gate, ORC_F_SPLIT + 2, i, bw);
    put_t(k0, orv, i, bw, v0);
    put_t(k1, orv, i, bw, (rv - v0) & M);
    put_t(k0, osig, i, bw, s0);
    put_t(k1, osig, i, bw, (sigma - s0) & M);
    put_t(k0, oc, i, bw, c0);
    put_t(k1, oc, i, bw, (C - c0) & M);
  }
}

void orc_lut8_eval(int bw, size_t N, const uint8_t *k0, const uint8_t *k1, size_t base,
                   const uint64_t *table, const uint64_t *xhat, uint64_t *yhat,
                   uint64_t *bytes) {
  const uint64_t M = rmask(bw);
  orc_dcf_layout D;
  size_t orv, osig, oc;
  orc_lut8_layout(bw, N, base, &D, &orv, &osig, &oc);
  const uint8_t *K[2] = {k0, k1};
  uint64_t *v[2], *y[2];
  for (int p = 0; p < 2; p++) {
    v[p] = (uint64_t *)calloc(N, 8);
    y[p] = (uint64_t *)calloc(N, 8);
    OMP_FOR
    for (size_t i = 0; i < N; i++) {
      uint8_t u[256];
      orc_dpf_full_eval(p, 8, K[p], &D, i, u);
      uint64_t acc = 0, xh = xhat[i] & 255u;
      for (int k = 0; k < 256; k++)
        if (u[k]) acc += table[(xh - (uint64_t)k) & 255u];
      if (p == 1) acc = 0 - acc;
      v[p][i] = (acc + get_t(K[p], orv, i, bw)) & M;
    }
  }
  if (bytes) *bytes += 2ull * N * (uint64_t)(bw / 8);
  for (int p = 0; p < 2; p++) {
    OMP_FOR
    for (size_t i = 0; i < N; i++) {
      uint64_t vh = (v[0][i] + v[1][i]) & M;
      y[p][i] = (vh * get_t(K[p], osig, i, bw) + get_t(K[p], oc, i, bw)) & M;
    }
  }
  if (bytes) *bytes += 2ull * N * (uint64_t)(bw / 8);
  for (size_t i = 0; i < N; i++) yhat[i] = (y[0][i] + y[1][i]) & M;
  for (int p = 0; p < 2; p++) {
    free(v[p]);
    free(y[p]);
  }
}

/* ---------------- ring GEMM ---------------- */
void orc_ring_gemm(int bw, size_t nb, size_t M_, size_t K, size_t N, const uint64_t *A,
                   const uint64_t *B, uint64_t *C, int b_batched) {
  const uint64_t RM = rmask(bw);
  OMP_FOR
  for (size_t bi = 0; bi < nb * M_; bi++) {
    size_t b = bi / M_, i = bi % M_;
    const uint64_t *a = A + (b * M_ + i) * K;
    const uint64_t *bb = B + (b_batched ? b * K * N : 0);
    uint64_t *c = C + (b * M_ + i) * N;
    for (size_t j = 0; j < N; j++) c[j] = 0;
    for (size_t k = 0; k < K; k++) {
      uint64_t av = a[k];
      const uint64_t *brow = bb + k * N;
      for (size_t j = 0; j < N; j++) c[j] += av * brow[j];
    }
    for (size_t j = 0; j < N; j++) c[j] &= RM;
  }
}

/* ---------------- SxS matmul ---------------- */
size_t orc_sxs_layout(int bw, size_t nb, size_t M_, size_t K, size_t N, size_t base,
                      size_t *off_ra, size_t *off_rb, size_t *off_c) {
  size_t tb = (size_t)bw / 8, o = orc_align(base);
  *off_ra = o;
  o = orc_align(o + nb * M_ * K * tb);
  *off_rb = o;
  o = orc_align(o + nb * K * N * tb);
  *off_c = o;
  o = orc_align(o + nb * M_ * N * tb);
  return o;
}

void orc_sxs_keygen(uint64_t seed, uint32_t gate, int bw, size_t nb, size_t M_, size_t K,
                    size_t N, const uint64_t *ra, const uint64_t *rb, uint64_t *rc,
                    uint8_t *k0, uint8_t *k1, size_t base) {
  orc_prf P;
  orc_prf_init(&P, seed);
  const uint64_t RM = rmask(bw);
  size_t ora, orb, oc;
  orc_sxs_layout(bw, nb, M_, K, N, base, &ora, &orb, &oc);
  size_t na = nb * M_ * K, nbb = nb * K * N, nc = nb * M_ * N;
  uint64_t *ra0 = (uint64_t *)malloc(na * 8), *rb0 = (uint64_t *)malloc(nbb * 8);
  uint64_t *t1 = (uint64_t *)malloc(nc * 8), *t2 = (uint64_t *)malloc(nc * 8);
  OMP_FOR
  for (size_t i = 0; i < na; i++) {
    ra0[i] = prf_ring(&P, gate, ORC_F_SPLIT + 0, i, bw);
    put_t(k0, ora, i, bw, ra0[i]);
    put_t(k1, ora, i, bw, (ra[i] - ra0[i]) & RM);
  }
  OMP_FOR
  for (size_t i = 0; i < nbb; i++) {
    rb0[i] = prf_ring(&P, gate, ORC_F_SPLIT + 1, i, bw);
    put_t(k0, orb, i, bw, rb0[i]);
    put_t(k1, orb, i, bw, (rb[i] - rb0[i]) & RM);
  }
  orc_ring_gemm(bw, nb, M_, K, N, ra, rb, t1, 1);
  orc_ring_gemm(bw, nb, M_, K, N, ra0, rb0, t2, 1);
  OMP_FOR
  for (size_t i = 0; i < nc; i++) {
    uint64_t r = prf_ring(&P, gate, ORC_F_ROUT, i, bw);
    rc[i] = r;
    uint64_t C = (t1[i] - t2[i] + r) & RM;
    uint64_t c0 = prf_ring(&P, gate, ORC_F_SPLIT + 2, i, bw);
    put_t(k0, oc, i, bw, c0);
    put_t(k1, oc, i, bw, (C - c0) & RM);
  }
  free(ra0);
  free(rb0);
  free(t1);
  free(t2);
}

void orc_sxs_eval(int bw, size_t nb, size_t M_, size_t K, size_t N, const uint8_t *k0,
                  const uint8_t *k1, size_t base, const uint64_t *ahat,
                  const uint64_t *bhat, uint64_t *chat, uint64_t *bytes) {
  const uint64_t RM = rmask(bw);
  size_t ora, orb, oc;
  orc_sxs_layout(bw, nb, M_, K, N, base, &ora, &orb, &oc);
  size_t na = nb * M_ * K, nbb = nb * K * N, nc = nb * M_ * N;
  uint64_t *A = (uint64_t *)malloc(na * 8), *Bm = (uint64_t *)malloc(nbb * 8);
  uint64_t *z0 = (uint64_t *)malloc(nc * 8), *z1 = (uint64_t *)malloc(nc * 8);
  uint64_t *t = (uint64_t *)malloc(nc * 8);
  /* party 0: (A^ - RA0)(B^ - RB0) + C0 */
  for (size_t i = 0; i < na; i++) A[i] = (ahat[i] - get_t(k0, ora, i, bw)) & RM;
  for (size_t i = 0; i < nbb; i++) Bm[i] = (bhat[i] - get_t(k0, orb, i, bw)) & RM;
  orc_ring_gemm(bw, nb, M_, K, N, A, Bm, z0, 1);
  for (size_t i = 0; i < nc; i++) z0[i] = (z0[i] + get_t(k0, oc, i, bw)) & RM;
  /* party 1: -(A^ RB1 + RA1 B^) + C1 */
  for (size_t i = 0; i < nbb; i++) Bm[i] = get_t(k1, orb, i, bw);
  orc_ring_gemm(bw, nb, M_, K, N, ahat, Bm, z1, 1);
  for (size_t i = 0; i < na; i++) A[i] = get_t(k1, ora, i, bw);
  orc_ring_gemm(bw, nb, M_, K, N, A, bhat, t, 1);
  for (size_t i = 0; i < nc; i++) z1[i] = (get_t(k1, oc, i, bw) - z1[i] - t[i]) & RM;
  if (bytes) *bytes += 2ull * nc * (uint64_t)(bw / 8);
  for (size_t i = 0; i < nc; i++) chat[i] = (z0[i] + z1[i]) & RM;
  free(A);
  free(Bm);
  free(z0);
  free(z1);
  free(t);
}

/* ---------------- reveal ---------------- */
size_t orc_reveal_layout(int bw, size_t N, size_t base, size_t *off_r) {
  size_t o = orc_align(base);
  *off_r = o;
  return orc_align(o + N * (size_t)(bw / 8));
}

void orc_reveal_keygen(uint64_t seed, uint32_t gate, int bw, size_t N, uint64_t *mask,
                       uint8_t *k0, uint8_t *k1, size_t base) {
  orc_prf P;
  orc_prf_init(&P, seed);
  const uint64_t RM = rmask(bw);
  size_t orr;
  orc_reveal_layout(bw, N, base, &orr);
  OMP_FOR
  for (size_t i = 0; i < N; i++) {
    uint64_t r = prf_ring(&P, gate, ORC_F_RIN, i, bw);
    mask[i] = r;
    uint64_t r0 = prf_ring(&P, gate, ORC_F_SPLIT + 0, i, bw);
    put_t(k0, orr, i, bw, r0);
    put_t(k1, orr, i, bw, (r - r0) & RM);
  }
}

void orc_reveal_eval(int bw, size_t N, const uint8_t *k0, const uint8_t *k1, size_t base,
                     const uint64_t *v0, const uint64_t *v1, uint64_t *vhat,
                     uint64_t *bytes) {
  const uint64_t RM = rmask(bw);
  size_t orr;
  orc_reveal_layout(bw, N, base, &orr);
  OMP_FOR
  for (size_t i = 0; i < N; i++) {
    uint64_t m0 = (v0[i] + get_t(k0, orr, i, bw)) & RM;
    uint64_t m1 = (v1[i] + get_t(k1, orr, i, bw)) & RM;
    vhat[i] = (m0 + m1) & RM;
  }
  if (bytes) *bytes += 2ull * N * (uint64_t)(bw / 8);
}
