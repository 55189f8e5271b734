/*
 * oracle/orc_aes.c -- AES-128 per FIPS-197, and the fixed-key hashes /
 * dealer PRF built on it.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * The byte-oriented path is a direct restatement of FIPS-197 sections 5.1
 * (Cipher) and 5.2 (KeyExpansion).  An AES-NI path is used when the host CPU
 * has it; both are checked against the FIPS-197 Appendix C.1 vector, which is
 * also the KAT of gpu_mpc/lss/lss_test.cpp:52-70 in the reference.
 */
#include <string.h>
#include "orc.h"

#if defined(__x86_64__)
#include <immintrin.h>
#endif

static const uint8_t SBOX[256] = {
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

/* FIPS-197 5.2 KeyExpansion, Nk = 4, Nr = 10. */
void orc_aes_expand(const uint8_t key[16], uint8_t rk[176]) {
  static const uint8_t rcon[10] = {0x01, 0x02, 0x04, 0x08, 0x10, 0x20, 0x40, 0x80, 0x1b, 0x36};
  memcpy(rk, key, 16);
  for (int i = 4; i < 44; i++) {
    uint8_t t[4];
    memcpy(t, rk + 4 * (i - 1), 4);
    if (i % 4 == 0) {
      uint8_t t0 = t[0]; /* RotWord then SubWord then Rcon */
      t[0] = (uint8_t)(SBOX[t[1]] ^ rcon[i / 4 - 1]);
      t[1] = SBOX[t[2]];
      t[2] = SBOX[t[3]];
      t[3] = SBOX[t0];
    }
    for (int j = 0; j < 4; j++) rk[4 * i + j] = (uint8_t)(rk[4 * (i - 4) + j] ^ t[j]);
  }
}

static uint8_t xtime(uint8_t a) { return (uint8_t)((a << 1) ^ ((a & 0x80) ? 0x1b : 0)); }

/* FIPS-197 5.1 Cipher on the column-major state s[r + 4c]. */
static void aes_encrypt_bytes(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]) {
  uint8_t s[16], t[16];
  for (int i = 0; i < 16; i++) s[i] = (uint8_t)(in[i] ^ rk[i]);
  for (int round = 1; round <= 10; round++) {
    for (int i = 0; i < 16; i++) s[i] = SBOX[s[i]];           /* SubBytes */
    for (int c = 0; c < 4; c++)                                /* ShiftRows */
      for (int r = 0; r < 4; r++) t[r + 4 * c] = s[r + 4 * ((c + r) & 3)];
    if (round != 10) {                                         /* MixColumns */
      for (int c = 0; c < 4; c++) {
        uint8_t a0 = t[4 * c], a1 = t[4 * c + 1], a2 = t[4 * c + 2], a3 = t[4 * c + 3];
        s[4 * c + 0] = (uint8_t)(xtime(a0) ^ (xtime(a1) ^ a1) ^ a2 ^ a3);
        s[4 * c + 1] = (uint8_t)(a0 ^ xtime(a1) ^ (xtime(a2) ^ a2) ^ a3);
        s[4 * c + 2] = (uint8_t)(a0 ^ a1 ^ xtime(a2) ^ (xtime(a3) ^ a3));
        s[4 * c + 3] = (uint8_t)((xtime(a0) ^ a0) ^ a1 ^ a2 ^ xtime(a3));
      }
    } else {
      memcpy(s, t, 16);
    }
    for (int i = 0; i < 16; i++) s[i] ^= rk[16 * round + i]; /* AddRoundKey */
  }
  memcpy(out, s, 16);
}

static int g_force_portable = 0;

#if defined(__x86_64__)
__attribute__((target("aes,sse2"))) static void aes_encrypt_ni(const uint8_t rk[176],
                                                                const uint8_t in[16],
                                                                uint8_t out[16]) {
  __m128i m = _mm_loadu_si128((const __m128i *)in);
  m = _mm_xor_si128(m, _mm_loadu_si128((const __m128i *)rk));
  for (int r = 1; r < 10; r++) m = _mm_aesenc_si128(m, _mm_loadu_si128((const __m128i *)(rk + 16 * r)));
  m = _mm_aesenclast_si128(m, _mm_loadu_si128((const __m128i *)(rk + 160)));
  _mm_storeu_si128((__m128i *)out, m);
}
static int have_ni(void) {
  static int cached = -1;
  if (cached < 0) cached = __builtin_cpu_supports("aes") ? 1 : 0;
  return cached;
}
#else
static int have_ni(void) { return 0; }
#endif

int orc_aes_backend(void) { return (!g_force_portable && have_ni()) ? 1 : 0; }
void orc_aes_force_portable(int on) { g_force_portable = on; }

void orc_aes_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]) {
#if defined(__x86_64__)
  if (orc_aes_backend()) {
    aes_encrypt_ni(rk, in, out);
    return;
  }
#endif
  aes_encrypt_bytes(rk, in, out);
}

/* ---------------- half-tree hashes ---------------- */
const uint8_t ORC_KEY_H[16] = {'M', 'I', '3', '5', '5', 'X', '-', 'H', 'a', 'l', 'f', 'T', 'r', 'e', 'e', 'H'};
const uint8_t ORC_KEY_L[16] = {'M', 'I', '3', '5', '5', 'X', '-', 'H', 'a', 'l', 'f', 'T', 'r', 'e', 'e', 'L'};

static uint8_t g_rk_h[176], g_rk_l[176];
static int g_rk_init = 0;
static void rk_init(void) {
  if (g_rk_init) return;
  orc_aes_expand(ORC_KEY_H, g_rk_h);
  orc_aes_expand(ORC_KEY_L, g_rk_l);
  g_rk_init = 1;
}

static void blk_to_bytes(orc_blk b, uint8_t o[16]) {
  for (int i = 0; i < 4; i++) {
    o[4 * i + 0] = (uint8_t)(b.w[i]);
    o[4 * i + 1] = (uint8_t)(b.w[i] >> 8);
    o[4 * i + 2] = (uint8_t)(b.w[i] >> 16);
    o[4 * i + 3] = (uint8_t)(b.w[i] >> 24);
  }
}
static orc_blk bytes_to_blk(const uint8_t o[16]) {
  orc_blk b;
  for (int i = 0; i < 4; i++)
    b.w[i] = (uint32_t)o[4 * i] | ((uint32_t)o[4 * i + 1] << 8) | ((uint32_t)o[4 * i + 2] << 16) |
             ((uint32_t)o[4 * i + 3] << 24);
  return b;
}

/* sigma(xL || xR) = (xL ^ xR) || xL; xR = words 0,1 (low 64 bits), xL = words 2,3. */
static orc_blk sigma(orc_blk s) {
  orc_blk r;
  r.w[0] = s.w[2];
  r.w[1] = s.w[3];
  r.w[2] = s.w[2] ^ s.w[0];
  r.w[3] = s.w[3] ^ s.w[1];
  return r;
}

static orc_blk hash_with(const uint8_t *rk, orc_blk s) {
  orc_blk x = sigma(s);
  uint8_t in[16], out[16];
  blk_to_bytes(x, in);
  orc_aes_encrypt(rk, in, out);
  orc_blk y = bytes_to_blk(out);
  for (int i = 0; i < 4; i++) y.w[i] ^= x.w[i];
  return y;
}

orc_blk orc_H(orc_blk s) {
  rk_init();
  return hash_with(g_rk_h, s);
}
orc_blk orc_HL(orc_blk s) {
  rk_init();
  return hash_with(g_rk_l, s);
}

void orc_H_batch(size_t n, const orc_blk *in, orc_blk *out, int leaf) {
  rk_init();
  const uint8_t *rk = leaf ? g_rk_l : g_rk_h;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = hash_with(rk, in[i]);
}

/* ---------------- dealer PRF ---------------- */
/* The dealer's 16 secret key bytes, when set: the PRF key of a key set is then
 * the AES encryption under them of the block (seed low word, seed high word,
 * 0x4D415354, 0xFFFFFFFE); without them it is the seed and seed ^
 * 0x9E3779B97F4A7C15 as the key bytes. */
static int g_has_dealer_key = 0;
static uint8_t g_dealer_rk[176];

void orc_set_dealer_key(const uint8_t *key16) {
  g_has_dealer_key = key16 != NULL;
  if (key16) orc_aes_expand(key16, g_dealer_rk);
}

void orc_prf_init(orc_prf *p, uint64_t seed) {
  uint8_t key[16];
  if (g_has_dealer_key) {
    orc_blk in;
    in.w[0] = (uint32_t)seed;
    in.w[1] = (uint32_t)(seed >> 32);
    in.w[2] = 0x4D415354u;
    in.w[3] = 0xFFFFFFFEu;
    uint8_t b[16];
    blk_to_bytes(in, b);
    orc_aes_encrypt(g_dealer_rk, b, key);
  } else {
    uint64_t a = seed, b = seed ^ 0x9E3779B97F4A7C15ull;
    for (int i = 0; i < 8; i++) {
      key[i] = (uint8_t)(a >> (8 * i));
      key[8 + i] = (uint8_t)(b >> (8 * i));
    }
  }
  orc_aes_expand(key, p->rk);
}

orc_blk orc_prf_blk(const orc_prf *p, uint32_t gate, uint32_t field, uint64_t idx) {
  orc_blk in;
  in.w[0] = (uint32_t)idx;
  in.w[1] = (uint32_t)(idx >> 32);
  in.w[2] = field;
  in.w[3] = gate;
  uint8_t b[16], o[16];
  blk_to_bytes(in, b);
  orc_aes_encrypt(p->rk, b, o);
  return bytes_to_blk(o);
}

void orc_prf_batch(uint64_t seed, uint32_t gate, uint32_t field, size_t n, orc_blk *out) {
  orc_prf p;
  orc_prf_init(&p, seed);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = orc_prf_blk(&p, gate, field, i);
}
