/*
 * oracle/orc.h -- CPU restatement of the secure-inference online path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg use it, and only as the checker (or as the timed CPU baseline).
 *
 * What it restates (reference files, path:line relative to the reference
 * repository):
 *   - fixed-point ring semantics: reference/fixedpoint.py:28-77,
 *     reference/fixed_forward.py:44-117 (to_fixed, truncate, fixed_matmul,
 *     _wrap, _linear, _gcn_layer, _drug_path_fx, _fusion_fx);
 *   - A_hat produced by the secure adjacency normalisation, i.e. the LUT
 *     closed form A[i,j]*floor(T[d_i]*T[d_j]/2^s), T[k]=llround(2^s/sqrt(k)),
 *     T[0]=0: gpu_mpc/secure_adj_norm.h:138-184 and :326-365;
 *   - the masked max-pool (sentinel -2^(bw-2)): fixed_forward.py:33-36,
 *     76-80;
 *   - AES-128 (FIPS-197), used by the FSS PRG; KAT vector of
 *     gpu_mpc/lss/lss_test.cpp:52-70;
 *   - the two-party online protocol itself (DCF/DPF keys, ReLU, truncation,
 *     LUT, Beaver products, max-pool tree) in the same key format as the GPU
 *     implementation, so that keys, exchanged messages and reconstructed
 *     outputs can be compared byte for byte.
 *
 * Every function is checked by tests/ against closed forms, brute force or the
 * known-answer vectors of tests/golden/ (FIPS-197, the reference's fixed-point
 * test vectors and the D^-1/2 table values).
 *
 * Ring elements are carried in uint64_t and reduced mod 2^bw (bw = 32 or 64).
 */
#ifndef ORC_H
#define ORC_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct { uint32_t w[4]; } orc_blk; /* 128-bit block, w[0]=bytes 0..3 LE */

/* ---------------- AES-128, FIPS-197 ---------------- */
void orc_aes_expand(const uint8_t key[16], uint8_t rk[176]);
void orc_aes_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]);
/* 1 when the AES-NI path is active (runtime detected), 0 for the byte path. */
int orc_aes_backend(void);
void orc_aes_force_portable(int on);

/* Fixed-key correlation-robust hashes of the half-tree PRG:
 *   H(s)  = AES_KH(sigma(s)) ^ sigma(s)   (tree levels)
 *   HL(s) = AES_KL(sigma(s)) ^ sigma(s)   (leaf conversion)
 * sigma(xL||xR) = (xL ^ xR) || xL over 64-bit halves. */
orc_blk orc_H(orc_blk s);
orc_blk orc_HL(orc_blk s);
void orc_H_batch(size_t n, const orc_blk *in, orc_blk *out, int leaf);
extern const uint8_t ORC_KEY_H[16];
extern const uint8_t ORC_KEY_L[16];

/* Dealer PRF: AES_Kd(idx_lo, idx_hi, field, gate); Kd derived from seed. */
typedef struct { uint8_t rk[176]; } orc_prf;
void orc_prf_init(orc_prf *p, uint64_t seed);
/* The dealer's 16 secret key bytes (NULL: the seed alone derives the PRF key). */
void orc_set_dealer_key(const uint8_t *key16);
orc_blk orc_prf_blk(const orc_prf *p, uint32_t gate, uint32_t field, uint64_t idx);
void orc_prf_batch(uint64_t seed, uint32_t gate, uint32_t field, size_t n, orc_blk *out);

/* ---------------- key layout ---------------- */
#define ORC_ALIGN 256
size_t orc_align(size_t x);
size_t orc_zwords(size_t N); /* packed-bit words (u32), rounded to u64 */

typedef struct {
  int m;            /* input domain bits */
  int L;            /* tree levels = max(m-7,0) */
  size_t N;
  size_t off_root;  /* N x 16 B */
  size_t off_cw;    /* L x N x 16 B, level-major */
  size_t off_leaf;  /* N x 16 B */
  size_t off_z;     /* zwords(N) x 4 B (output mask bit shares), 0 if none */
  size_t end;
} orc_dcf_layout;
orc_dcf_layout orc_dcf_layout_make(int m, size_t N, size_t base, int with_z);

/* Gate kinds (shared with the GPU implementation). */
enum {
  ORC_G_TR = 1,       /* exact truncation + bias, full sign extension   */
  ORC_G_TRRELU = 2,   /* ReLU(trunc(x)+bias), fused                     */
  ORC_G_RELU = 3,     /* ReLU without truncation                        */
  ORC_G_TRSLACK = 4,  /* exact truncation, |x| < 2^(bw-2)                */
  ORC_G_MUL = 5,      /* Beaver elementwise product (index maps)        */
  ORC_G_LUT8 = 6,     /* 8-bit DPF lookup table                         */
  ORC_G_SXS = 7,      /* batched secret x secret ring GEMM              */
  ORC_G_REVEAL = 8,   /* additive shares -> masked public               */
  ORC_G_RELUSLACK = 9, /* ReLU for |x| < 2^(bw-2-s) (a (bw-2-s)-bit DCF) */
  ORC_G_LOCALARS = 10, /* local arithmetic shift of the masked value and of
                          its mask: no key, no exchange, error +1 or a wrap */
  ORC_G_DRELU = 11,    /* [x >= 0] as a masked public bit (0/1 ring element),
                          mask bit returned by keygen: one (bw-1)-bit DCF */
  ORC_G_TRMOD = 12,    /* floor(x/2^s) + bias modulo 2^(bw-s): one s-bit DCF */
  ORC_G_EXT = 13,      /* a value known modulo 2^(bw-s) sign-extended to bw bits:
                          one (bw-s-1)-bit DCF */
  ORC_G_EXTRELU = 14,  /* ReLU of that value, sign-extended: the same one DCF */
  ORC_G_RELUPOOL = 15  /* ReLU for |x| < 2^(bw-s): a (bw-s)-bit DCF */
};

/* Dealer randomness fields. */
enum {
  ORC_F_DCFA = 0x10, /* +0 root seed, +1 delta, +2 z0 bit, +3 mask bit */
  ORC_F_DCFB = 0x20,
  ORC_F_ROUT = 0x30, /* fresh output mask */
  ORC_F_SPLIT = 0x40, /* +k: share-0 of plane k */
  ORC_F_LUTV = 0x58,
  ORC_F_RIN = 0x60,  /* input masks of reveal gates */
  ORC_F_PARTY = 0x70 /* +0: the parties' own PRF keys (gate 0xFFFFFFFF, index p) */
};

typedef struct {
  int kind, bw, s, relu;
  size_t N;
  orc_dcf_layout a, b; /* a: (bw-1)-bit DCF, b: s-bit DCF */
  size_t off_kappa;    /* N x T (relu kinds) */
  size_t off_g;        /* ncase x N x T */
  int ncase;
  size_t end;
} orc_tr_layout;
int orc_sign_bit(int kind, int bw, int s);
orc_tr_layout orc_tr_layout_make(int kind, int bw, int s, size_t N, size_t base);

/* ---------------- gates (keygen + two-party eval) ----------------
 * All arrays of ring elements are uint64_t reduced mod 2^bw.
 * Keys are written into per-party byte buffers at the layout offsets.
 * Eval functions evaluate BOTH parties, exchange through memory and return
 * the reconstructed masked output; bytes sent by each party are added to
 * *bytes (both directions counted). */

/* DCF [x < alpha] over m bits, XOR-shared and masked with a random bit. */
void orc_dcf_keygen(uint64_t seed, uint32_t gate, uint32_t fbase, int m, size_t N,
                    const uint64_t *alpha, const uint8_t *rbit,
                    uint8_t *k0, uint8_t *k1, size_t base);
int orc_dcf_eval1(int party, const uint8_t *key, const orc_dcf_layout *L, size_t i,
                  uint64_t x);
void orc_dcf_eval(int party, int m, size_t N, const uint8_t *key, size_t base,
                  const uint64_t *x, uint8_t *out);

/* Party p's own PRF key (16 bytes): the truncation-family keygen draws party p's
 * DCF roots and output-mask bits (party 0: also its kappa and G shares) from it. */
void orc_party_key(uint64_t seed, int party, uint8_t key[16]);

/* Truncation / ReLU family.  bias: per element (scale s) or NULL.
 * in_mask: mask of the gate input; out_mask: output mask (written). */
void orc_tr_keygen(uint64_t seed, uint32_t gate, int kind, int bw, int s, size_t N,
                   const uint64_t *in_mask, uint64_t *out_mask,
                   uint8_t *k0, uint8_t *k1, size_t base);
void orc_tr_eval(int kind, int bw, int s, size_t N, const uint8_t *k0, const uint8_t *k1,
                 size_t base, const uint64_t *xhat, const int64_t *bias_elem,
                 uint64_t *yhat, uint64_t *bytes);

/* Beaver product z[i] = x[ia[i]] * y[ib[i]]. */
size_t orc_mul_layout(int bw, size_t nx, size_t ny, size_t nz, size_t base,
                      size_t *off_rx, size_t *off_ry, size_t *off_c);
void orc_mul_keygen(uint64_t seed, uint32_t gate, int bw, size_t nx, size_t ny, size_t nz,
                    const uint32_t *ia, const uint32_t *ib, const uint64_t *rx,
                    const uint64_t *ry, uint64_t *rz, uint8_t *k0, uint8_t *k1, size_t base);
void orc_mul_eval(int bw, size_t nx, size_t ny, size_t nz, const uint32_t *ia,
                  const uint32_t *ib, const uint8_t *k0, const uint8_t *k1, size_t base,
                  const uint64_t *xhat, const uint64_t *yhat, uint64_t *zhat,
                  uint64_t *bytes);

/* 8-bit DPF lookup table, public 256-entry table. */
size_t orc_lut8_layout(int bw, size_t N, size_t base, orc_dcf_layout *dpf,
                       size_t *off_rv, size_t *off_sig, size_t *off_c);
void orc_lut8_keygen(uint64_t seed, uint32_t gate, int bw, size_t N, const uint64_t *in_mask,
                     uint64_t *out_mask, uint8_t *k0, uint8_t *k1, size_t base);
void orc_lut8_eval(int bw, size_t N, const uint8_t *k0, const uint8_t *k1, size_t base,
                   const uint64_t *table, const uint64_t *xhat, uint64_t *yhat,
                   uint64_t *bytes);
void orc_dpf_full_eval(int party, int m, const uint8_t *key, const orc_dcf_layout *L,
                       size_t i, uint8_t *bits /* 2^m */);

/* Batched SxS ring GEMM: per batch C(MxN) = A(MxK) . B(KxN). */
size_t orc_sxs_layout(int bw, size_t nb, size_t M, size_t K, size_t N, size_t base,
                      size_t *off_ra, size_t *off_rb, size_t *off_c);
void orc_sxs_keygen(uint64_t seed, uint32_t gate, int bw, size_t nb, size_t M, size_t K,
                    size_t N, const uint64_t *ra, const uint64_t *rb, uint64_t *rc,
                    uint8_t *k0, uint8_t *k1, size_t base);
void orc_sxs_eval(int bw, size_t nb, size_t M, size_t K, size_t N, const uint8_t *k0,
                  const uint8_t *k1, size_t base, const uint64_t *ahat,
                  const uint64_t *bhat, uint64_t *chat, uint64_t *bytes);

/* Reveal: additive shares v0+v1 -> v + r. */
size_t orc_reveal_layout(int bw, size_t N, size_t base, size_t *off_r);
void orc_reveal_keygen(uint64_t seed, uint32_t gate, int bw, size_t N, uint64_t *mask,
                       uint8_t *k0, uint8_t *k1, size_t base);
void orc_reveal_eval(int bw, size_t N, const uint8_t *k0, const uint8_t *k1, size_t base,
                     const uint64_t *v0, const uint64_t *v1, uint64_t *vhat,
                     uint64_t *bytes);

/* Plain ring GEMM on public/mask operands, mod 2^bw, batched. */
void orc_ring_gemm(int bw, size_t nb, size_t M, size_t K, size_t N, const uint64_t *A,
                   const uint64_t *B, uint64_t *C, int b_batched);

/* ---------------- model ---------------- */
typedef struct {
  int bw, s;
  int n_nodes;    /* padded atoms N */
  int feat;       /* input feature width */
  int gcn[3];     /* GCN output widths */
  int dfc[2];     /* drug FC widths: pool->dfc0->dfc1 */
  int prot;       /* protein embedding width */
  int nfus;       /* number of fusion layers (last has width 1) */
  int fus[4];     /* fusion widths */
  int lut_nmax;   /* largest degree with a table entry (mpc_config.py NMAX) */
  int mask_scale; /* the atom mask is 0 or 2^mask_scale (0; s for the reference's files) */
  int slack;      /* 0: exact truncations over the signed ring; 1: the GCN products
                     H.W^T are truncated with TRSLACK (exact for |H.W^T| < 2^(bw-2));
                     2: also A.XW + bias: TRSLACK then RELUSLACK (|A.XW + b 2^s| < 2^(bw-2));
                     3: every layer truncation is LocalARS (local shift, no key), followed
                     by a RELU gate on ReLU layers: not bit-exact with orc_plain_forward */
  int gcn_order;  /* orc_plain_forward only: 0 transform-first, H' = ReLU(tr(A.tr(H.W^T)) + b)
                     (reference/fixed_forward.py:63-67); 1 aggregate-first, the order of the
                     C++ layers, H' = ReLU(tr(tr(A.H).W^T + b 2^s)) (gpu_mpc/gcn_layer.h:113-114) */
} orc_dims;

/* Weights: for each linear layer in order gcn0..2, dfc0..1, fus0..nfus-1:
 * Wt (in x out, row-major, scale s) followed by bias (out, scale s), int64.
 * This is the weights.bin order of gpu_mpc/deepdtagen_inference.cu:121-181. */
size_t orc_weights_len(const orc_dims *d);

/* Inverse-sqrt degree table T[256] (secure_adj_norm.h:138-184). */
void orc_invsqrt_table(int s, int nmax, uint64_t *table);

/* Plaintext fixed-point forward (fixed_forward.py semantics, LUT A_hat).
 * X: B x N x feat, A: B x N x N (0/1 incl. self loops), mask: B x N,
 * prot: B x prot.  out: B int64.  Returns 0, or a positive code naming the
 * first value that left the bit-exact domain (see orc_domain_msg). */
int orc_plain_forward(const orc_dims *d, int B, const int64_t *X, const int64_t *A,
                      const int64_t *mask, const int64_t *prot, const int64_t *W,
                      int64_t *out);
const char *orc_domain_msg(int code);
/* A_hat of the secure path (scale s), B x N x N. */
void orc_adj_norm_plain(int s, int N, int B, const int64_t *A, int64_t *Ahat);

/* Two-party protocol (dealer + both evaluators), both parties in one process. */
size_t orc_model_key_bytes(const orc_dims *d, int B);
int orc_model_keygen(const orc_dims *d, int B, uint64_t seed, const int64_t *W,
                     uint8_t *k0, uint8_t *k1);
int orc_model_eval(const orc_dims *d, int B, const int64_t *W, const uint8_t *k0,
                   const uint8_t *k1, const uint64_t *x0, const uint64_t *x1,
                   const uint64_t *a0, const uint64_t *a1, const uint64_t *m0,
                   const uint64_t *m1, const int64_t *prot, int64_t *out,
                   uint64_t *bytes);
/* Standalone secure adjacency normalisation (gpu_mpc/secure_adj_norm.h:203-374,
 * 393-659): A (B x N x N, 0/1 with self loops) as additive shares a0, a1 ->
 * masked A_norm = A (.) floor(T[d_i] T[d_j] / 2^s) + out_mask. */
size_t orc_adjnorm_key_bytes(int bw, int s, int B, int N);
int orc_adjnorm_keygen(int bw, int s, int B, int N, uint64_t seed, uint64_t *out_mask, uint8_t *k0,
                       uint8_t *k1);
int orc_adjnorm_eval(int bw, int s, int B, int N, int nmax, const uint8_t *k0, const uint8_t *k1,
                     const uint64_t *a0, const uint64_t *a1, uint64_t *out_masked, uint64_t *bytes);

/* Standalone masked global max-pool (gpu_mpc/masked_maxpool_layer.h:47-165):
 * masked-public (B*N x C, sample-major) -> (B x C) maximum over the N rows, a
 * tree of max(a, b) = a + ReLU(b - a) over pairs (2j, 2j+1), the odd last row
 * carried; keys of the levels back to back from base, gate ids gate, gate+1, ... */
size_t orc_maxpool_layout(int bw, int s, int B, int N, int C, size_t base);
void orc_maxpool_keygen(uint64_t seed, uint32_t gate, int bw, int s, int B, int N, int C,
                        const uint64_t *in_mask, uint64_t *out_mask, uint8_t *k0, uint8_t *k1,
                        size_t base);
void orc_maxpool_eval(int bw, int s, int B, int N, int C, const uint8_t *k0, const uint8_t *k1,
                      size_t base, const uint64_t *xhat, uint64_t *yhat, uint64_t *bytes);

/* Optional trace of reconstructed masked values (for debugging parity):
 * when set, each gate's public output is copied to the callback. */
typedef void (*orc_trace_fn)(uint32_t gate, size_t n, const uint64_t *vals);
void orc_set_trace(orc_trace_fn fn);

void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
