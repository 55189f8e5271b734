/*
 * oracle/orc_model.c -- plaintext fixed-point affinity forward and the
 * two-party protocol over the whole model.  TEST INFRASTRUCTURE ONLY.
 *
 * Plaintext semantics follow reference/fixed_forward.py:
 *   _wrap            :44-52  (signed reduction mod 2^bw)
 *   _linear          :55-61  (wrap(tr(x W^T)) then wrap(+b))
 *   _gcn_layer       :63-67  (transform first: wrap(tr(A_fx . wrap(tr(H W^T)))) + b)
 *   _drug_path_fx    :70-85  (3x GCN + ReLU, sentinel max-pool, drug FCs)
 *   _fusion_fx       :88-95  (concat [drug, protein], ReLU on all but last)
 * with fixed_matmul = exact product, floor(./2^s) (reference/fixedpoint.py:61-77),
 * and A_fx taken from the secure normalisation's closed form
 * A[i,j]*floor(T[d_i]*T[d_j]/2^s) (gpu_mpc/secure_adj_norm.h:138-184,326-365)
 * instead of to_fixed(A_hat) (fixed_forward.py:72), because the secure path
 * computes exactly that.
 *
 * Weights are the weights.bin layout of gpu_mpc/deepdtagen_inference.cu:121-181:
 * per layer W^T (in x out, row-major) then bias (out), int64 at scale s.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "orc.h"

typedef __int128 i128;
typedef unsigned __int128 u128;

static inline uint64_t rmask(int bw) { return bw >= 64 ? ~0ull : ((1ull << bw) - 1ull); }

static orc_trace_fn g_trace = 0;
void orc_set_trace(orc_trace_fn fn) { g_trace = fn; }
static void trace(uint32_t g, size_t n, const uint64_t *v) {
  if (g_trace) g_trace(g, n, v);
}

/* ---------------- dims / weights ---------------- */
static int nlayers(const orc_dims *d) { return 5 + d->nfus; }
/* slack 3: every layer truncation is LocalARS (the reference's default,
 * gpu_mpc/ddg_orca_batched.h:180-199): a local shift, then a RELU gate where the
 * layer has a ReLU; not bit-exact with the fixed-point forward */
static int local_trunc(const orc_dims *d) { return d->slack == 3; }
/* the GCN products H.W^T: TRSLACK when d->slack is 1 or 2, else the layer
 * truncation (exact: TRMOD then EXT) */
static int xw_slack(const orc_dims *d) { return d->slack == 1 || d->slack == 2; }
/* the GCN aggregation A.XW + bias then ReLU: the layer truncation with ReLU
 * (exact: TRMOD then EXTRELU), or (d->slack == 2) TRSLACK (with the bias)
 * followed by RELUSLACK on the truncated value */
static int agg_split(const orc_dims *d) { return d->slack == 2; }
/* the max-pool: exact and slack truncations leave activations in
 * [0, 2^(bw-s-1)), so the sentinel -2^(bw-s-1) keeps every pool value in
 * [-2^(bw-s-1), 2^(bw-s-1)) and a (bw-s)-bit DCF (RELUPOOL) decides each pair; the
 * maximum over a sample with a real atom equals the one the reference's sentinel
 * -2^(bw-2) gives (fixed_forward.py:33-36).  Local truncation (activations up to
 * 2^(bw-1)) or a mask scale above bw-s-1: the sentinel -2^(bw-2) and RELU. */
static int pool_narrow(const orc_dims *d) { return !local_trunc(d) && d->mask_scale <= d->bw - d->s - 1; }
static int pool_kind(const orc_dims *d) { return pool_narrow(d) ? ORC_G_RELUPOOL : ORC_G_RELU; }
static int pool_sentinel_bit(const orc_dims *d) { return pool_narrow(d) ? d->bw - d->s - 1 : d->bw - 2; }
static size_t trunc_layout(const orc_dims *d, int relu, size_t n, size_t o);
static void layer_io(const orc_dims *d, int l, int *in, int *out) {
  if (l < 3) {
    *in = l == 0 ? d->feat : d->gcn[l - 1];
    *out = d->gcn[l];
  } else if (l < 5) {
    *in = l == 3 ? d->gcn[2] : d->dfc[0];
    *out = d->dfc[l - 3];
  } else {
    int k = l - 5;
    *in = k == 0 ? d->dfc[1] + d->prot : d->fus[k - 1];
    *out = d->fus[k];
  }
}
static size_t layer_off(const orc_dims *d, int l) {
  size_t o = 0;
  for (int j = 0; j < l; j++) {
    int in, out;
    layer_io(d, j, &in, &out);
    o += (size_t)in * out + (size_t)out;
  }
  return o;
}
size_t orc_weights_len(const orc_dims *d) { return layer_off(d, nlayers(d)); }

void orc_invsqrt_table(int s, int nmax, uint64_t *table) {
  for (int k = 0; k < 256; k++) table[k] = 0;
  double q = ldexp(1.0, s);
  for (int k = 1; k <= nmax && k < 256; k++) table[k] = (uint64_t)llround(q / sqrt((double)k));
}

/* ---------------- plaintext forward ---------------- */
static const char *DOMAIN_MSG[] = {
    "ok",
    "pre-truncation product outside the signed ring",
    "product + bias*2^s outside the signed ring",
    "max-pool input >= 2^(bw-2) (sentinel headroom)",
    "sample without a real atom",
    "node degree outside the 8-bit LUT domain",
    "adjacency or mask entry not 0/1",
    "GCN product H.W^T outside the slack truncation's domain (|x| < 2^(bw-2))",
    "GCN aggregation A.XW + bias*2^s outside the slack truncation's domain (|x| < 2^(bw-2))",
};
const char *orc_domain_msg(int code) {
  if (code < 0 || code > 8) return "unknown";
  return DOMAIN_MSG[code];
}

typedef struct {
  int bw, s;
  int err;
} fx;

static int fits(const fx *f, i128 v) {
  i128 h = (i128)1 << (f->bw - 1);
  return v >= -h && v < h;
}
static int64_t wrapv(const fx *f, i128 v) {
  if (f->bw >= 64) return (int64_t)v;
  uint64_t m = (uint64_t)v & rmask(f->bw);
  uint64_t half = 1ull << (f->bw - 1);
  return m >= half ? (int64_t)m - (int64_t)(1ull << f->bw) : (int64_t)m;
}
static void seterr(fx *f, int code) {
  if (!f->err) f->err = code;
}
/* exact  sum_k a[k*as] * b[k*bs]  as a 128-bit integer */
static i128 dot(const int64_t *a, size_t as, const int64_t *b, size_t bs, size_t K) {
  u128 acc = 0;
  for (size_t k = 0; k < K; k++) acc += (u128)((i128)a[k * as] * (i128)b[k * bs]);
  return (i128)acc;
}
/* y(MxN) = wrap(tr(X(MxK) . B(KxN))); optional bias check for the fused gate;
 * slack_code != 0: the truncated value (product, plus bias*2^s when bias_check is
 * given) must also lie in [-2^(bw-2), 2^(bw-2)) (TRSLACK), else that code */
static void fixed_mm(fx *f, const int64_t *X, const int64_t *Bm, size_t M, size_t K, size_t N,
                     const int64_t *bias_check, int slack_code, int64_t *Y) {
  for (size_t i = 0; i < M; i++)
    for (size_t j = 0; j < N; j++) {
      i128 P = dot(X + i * K, 1, Bm + j, N, K);
      if (!fits(f, P)) seterr(f, 1);
      if (slack_code) {
        const i128 v = P + (bias_check ? ((i128)bias_check[j] << f->s) : 0);
        if (!(v >= -((i128)1 << (f->bw - 2)) && v < ((i128)1 << (f->bw - 2)))) seterr(f, slack_code);
      }
      if (bias_check && !fits(f, P + ((i128)bias_check[j] << f->s))) seterr(f, 2);
      Y[i * N + j] = wrapv(f, P >> f->s);
    }
}

void orc_adj_norm_plain(int s, int N, int B, const int64_t *A, int64_t *Ahat) {
  uint64_t T[256];
  orc_invsqrt_table(s, 138, T);
  for (int b = 0; b < B; b++) {
    const int64_t *a = A + (size_t)b * N * N;
    int64_t *o = Ahat + (size_t)b * N * N;
    int *deg = (int *)calloc((size_t)N, sizeof(int));
    for (int i = 0; i < N; i++)
      for (int j = 0; j < N; j++) deg[i] += (int)a[(size_t)i * N + j];
    for (int i = 0; i < N; i++)
      for (int j = 0; j < N; j++) {
        uint64_t ti = deg[i] >= 0 && deg[i] < 256 ? T[deg[i]] : 0;
        uint64_t tj = deg[j] >= 0 && deg[j] < 256 ? T[deg[j]] : 0;
        o[(size_t)i * N + j] = a[(size_t)i * N + j] * (int64_t)((ti * tj) >> s);
      }
    free(deg);
  }
}

static void adj_norm_tab(const orc_dims *d, const int64_t *a, int64_t *o, fx *f) {
  const int N = d->n_nodes;
  uint64_t T[256];
  orc_invsqrt_table(d->s, d->lut_nmax, T);
  int *deg = (int *)calloc((size_t)N, sizeof(int));
  for (int i = 0; i < N; i++)
    for (int j = 0; j < N; j++) {
      int64_t v = a[(size_t)i * N + j];
      if (v != 0 && v != 1) seterr(f, 6);
      deg[i] += (int)v;
    }
  for (int i = 0; i < N; i++)
    if (deg[i] < 0 || deg[i] > 255) seterr(f, 5);
  for (int i = 0; i < N; i++)
    for (int j = 0; j < N; j++) {
      uint64_t ti = T[deg[i] & 255], tj = T[deg[j] & 255];
      o[(size_t)i * N + j] = a[(size_t)i * N + j] * (int64_t)((ti * tj) >> d->s);
    }
  free(deg);
}

int orc_plain_forward(const orc_dims *d, int B, const int64_t *X, const int64_t *A,
                      const int64_t *mask, const int64_t *prot, const int64_t *W,
                      int64_t *out) {
  const int N = d->n_nodes, bw = d->bw, s = d->s;
  int err_all = 0;
#pragma omp parallel for schedule(dynamic) num_threads(orc_get_threads())
  for (int b = 0; b < B; b++) {
    fx f = {bw, s, 0};
    int maxw = d->feat;
    for (int l = 0; l < nlayers(d); l++) {
      int in, o;
      layer_io(d, l, &in, &o);
      if (o > maxw) maxw = o;
      if (in > maxw) maxw = in;
    }
    int64_t *Af = (int64_t *)malloc(sizeof(int64_t) * (size_t)N * N);
    int64_t *H = (int64_t *)malloc(sizeof(int64_t) * (size_t)N * maxw);
    int64_t *XW = (int64_t *)malloc(sizeof(int64_t) * (size_t)N * maxw);
    int64_t *Hn = (int64_t *)malloc(sizeof(int64_t) * (size_t)N * maxw);
    adj_norm_tab(d, A + (size_t)b * N * N, Af, &f);
    int fin = d->feat;
    memcpy(H, X + (size_t)b * N * fin, sizeof(int64_t) * (size_t)N * fin);
    for (int l = 0; l < 3; l++) {
      int fo = d->gcn[l];
      const int64_t *Wt = W + layer_off(d, l);
      const int64_t *bias = Wt + (size_t)fin * fo;
      if (d->gcn_order == 1) { /* aggregate first: tr(A.H), then tr(AH.W^T) (+ b below) */
        fixed_mm(&f, Af, H, (size_t)N, (size_t)N, (size_t)fin, NULL, 0, XW);
        fixed_mm(&f, XW, Wt, (size_t)N, (size_t)fin, (size_t)fo, bias, 0, Hn);
      } else {
        fixed_mm(&f, H, Wt, (size_t)N, (size_t)fin, (size_t)fo, NULL, xw_slack(d) ? 7 : 0,
                 XW); /* XW */
        fixed_mm(&f, Af, XW, (size_t)N, (size_t)N, (size_t)fo, bias, agg_split(d) ? 8 : 0, Hn); /* A.XW */
      }
      for (int i = 0; i < N; i++)
        for (int j = 0; j < fo; j++) {
          int64_t v = wrapv(&f, (i128)Hn[(size_t)i * fo + j] + bias[j]);
          H[(size_t)i * fo + j] = v > 0 ? v : 0;
        }
      fin = fo;
    }
    /* masked global max-pool, sentinel -2^(bw-2) */
    const int C = d->gcn[2];
    const int64_t sentinel = -(int64_t)(1ull << (bw - 2));
    int64_t *pooled = (int64_t *)malloc(sizeof(int64_t) * (size_t)C);
    int nreal = 0;
    for (int i = 0; i < N; i++) {
      int64_t mv = mask[(size_t)b * N + i];
      if (mv != 0 && mv != ((int64_t)1 << d->mask_scale)) f.err = f.err ? f.err : 6;
      nreal += mv != 0;
    }
    if (nreal == 0) seterr(&f, 4);
    for (int c = 0; c < C; c++) {
      int64_t best = sentinel;
      for (int i = 0; i < N; i++) {
        int64_t v = H[(size_t)i * C + c];
        if (v >= (int64_t)(1ull << (bw - 2))) seterr(&f, 3);
        int64_t mv = mask[(size_t)b * N + i] != 0 ? v : sentinel;
        if (mv > best) best = mv;
      }
      pooled[c] = best;
    }
    /* drug FCs */
    int64_t *h1 = (int64_t *)malloc(sizeof(int64_t) * (size_t)maxw);
    int64_t *h2 = (int64_t *)malloc(sizeof(int64_t) * (size_t)maxw * 2);
    {
      const int64_t *Wt = W + layer_off(d, 3);
      const int64_t *bias = Wt + (size_t)C * d->dfc[0];
      fixed_mm(&f, pooled, Wt, 1, (size_t)C, (size_t)d->dfc[0], bias, 0, h1);
      for (int j = 0; j < d->dfc[0]; j++) {
        int64_t v = wrapv(&f, (i128)h1[j] + bias[j]);
        h1[j] = v > 0 ? v : 0;
      }
      Wt = W + layer_off(d, 4);
      bias = Wt + (size_t)d->dfc[0] * d->dfc[1];
      fixed_mm(&f, h1, Wt, 1, (size_t)d->dfc[0], (size_t)d->dfc[1], bias, 0, h2);
      for (int j = 0; j < d->dfc[1]; j++) h2[j] = wrapv(&f, (i128)h2[j] + bias[j]);
    }
    /* fusion: concat [drug, protein] (fixed_forward.py:89) */
    int width = d->dfc[1] + d->prot;
    for (int j = 0; j < d->prot; j++) h2[d->dfc[1] + j] = prot[(size_t)b * d->prot + j];
    for (int k = 0; k < d->nfus; k++) {
      const int64_t *Wt = W + layer_off(d, 5 + k);
      int fo = d->fus[k];
      const int64_t *bias = Wt + (size_t)width * fo;
      fixed_mm(&f, h2, Wt, 1, (size_t)width, (size_t)fo, bias, 0, h1);
      for (int j = 0; j < fo; j++) {
        int64_t v = wrapv(&f, (i128)h1[j] + bias[j]);
        h2[j] = (k < d->nfus - 1 && v < 0) ? 0 : v;
      }
      width = fo;
    }
    out[b] = h2[0];
    free(Af);
    free(H);
    free(XW);
    free(Hn);
    free(pooled);
    free(h1);
    free(h2);
    if (f.err) {
#pragma omp critical
      {
        if (!err_all) err_all = f.err;
      }
    }
  }
  return err_all;
}

/* ---------------- two-party model ---------------- */
typedef struct {
  size_t off;
  uint32_t gate;
} walker;

static size_t pairs_of(int N) { return (size_t)N * (N + 1) / 2; }
static size_t pidx(int N, int i, int j) { /* i <= j */
  return (size_t)i * N - (size_t)i * (i - 1) / 2 + (size_t)(j - i);
}

/* pool tree: returns the number of levels, fills pairs per level */
static int pool_levels(int N, int *pairs) {
  int R = N, L = 0;
  while (R > 1) {
    pairs[L++] = R / 2;
    R = R / 2 + (R & 1);
  }
  return L;
}

static void build_maps(int B, int N, uint32_t *oa, uint32_t *ob, uint32_t *wa, uint32_t *wb) {
  size_t P = pairs_of(N);
  for (int b = 0; b < B; b++) {
    size_t q = (size_t)b * P;
    for (int i = 0; i < N; i++)
      for (int j = i; j < N; j++) {
        oa[q] = (uint32_t)(b * N + i);
        ob[q] = (uint32_t)(b * N + j);
        q++;
      }
    for (int i = 0; i < N; i++)
      for (int j = 0; j < N; j++) {
        size_t e = ((size_t)b * N + i) * N + j;
        wa[e] = (uint32_t)e;
        wb[e] = (uint32_t)((size_t)b * P + (i <= j ? pidx(N, i, j) : pidx(N, j, i)));
      }
  }
}

/* Masked global max-pool tree, shared by the model and the standalone entry
 * points (gpu_mpc/masked_maxpool_layer.h:47-165): planes V (B x R x C,
 * sample-major, masked-public) shrink to (B x 1 x C).  Per level the pair
 * differences V[2j+1] - V[2j] (:91-112), one RELU gate (:114-118) and
 * V[2j] + ReLU(.) (:120-124), the odd last row carried forward (:140-147).
 * The dealer runs the same linear steps on the masks.  V is overwritten (its
 * first B*C words hold the result); t1, t2: scratch of B*N*C words. */
static size_t pool_keygen_blk(uint64_t seed, uint32_t *g, int kind, int bw, int s, int B, int N, int C,
                              uint64_t *rV, uint64_t *t1, uint64_t *t2, uint8_t *k0, uint8_t *k1, size_t o) {
  const uint64_t M = rmask(bw);
  int pairs[32];
  int L = pool_levels(N, pairs), R = N;
  for (int l = 0; l < L; l++) {
    int pr = pairs[l];
    size_t E = (size_t)B * pr * C;
    for (int b = 0; b < B; b++)
      for (int j = 0; j < pr; j++)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * pr + j) * C + c] =
              (rV[((size_t)b * R + 2 * j + 1) * C + c] - rV[((size_t)b * R + 2 * j) * C + c]) & M;
    orc_tr_keygen(seed, (*g)++, kind, bw, s, E, t1, t2, k0, k1, o);
    o = orc_tr_layout_make(kind, bw, s, E, o).end;
    int Rn = pr + (R & 1);
    for (int b = 0; b < B; b++) {
      for (int j = 0; j < pr; j++)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * Rn + j) * C + c] =
              (rV[((size_t)b * R + 2 * j) * C + c] + t2[((size_t)b * pr + j) * C + c]) & M;
      if (R & 1)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * Rn + pr) * C + c] = rV[((size_t)b * R + R - 1) * C + c];
    }
    memcpy(rV, t1, 8 * (size_t)B * Rn * C);
    R = Rn;
  }
  return o;
}

static size_t pool_eval_blk(uint32_t *g, int kind, int bw, int s, int B, int N, int C, const uint8_t *k0,
                            const uint8_t *k1, size_t o, uint64_t *V, uint64_t *t1, uint64_t *t2, uint64_t *bytes) {
  const uint64_t M = rmask(bw);
  int pairs[32];
  int L = pool_levels(N, pairs), R = N;
  for (int l = 0; l < L; l++) {
    int pr = pairs[l];
    size_t E = (size_t)B * pr * C;
    for (int b = 0; b < B; b++)
      for (int j = 0; j < pr; j++)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * pr + j) * C + c] =
              (V[((size_t)b * R + 2 * j + 1) * C + c] - V[((size_t)b * R + 2 * j) * C + c]) & M;
    orc_tr_eval(kind, bw, s, E, k0, k1, o, t1, NULL, t2, bytes);
    trace((*g)++, E, t2);
    o = orc_tr_layout_make(kind, bw, s, E, o).end;
    int Rn = pr + (R & 1);
    for (int b = 0; b < B; b++) {
      for (int j = 0; j < pr; j++)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * Rn + j) * C + c] =
              (V[((size_t)b * R + 2 * j) * C + c] + t2[((size_t)b * pr + j) * C + c]) & M;
      if (R & 1)
        for (int c = 0; c < C; c++)
          t1[((size_t)b * Rn + pr) * C + c] = V[((size_t)b * R + R - 1) * C + c];
    }
    memcpy(V, t1, 8 * (size_t)B * Rn * C);
    R = Rn;
  }
  return o;
}

size_t orc_maxpool_layout(int bw, int s, int B, int N, int C, size_t base) {
  int pairs[32];
  int L = pool_levels(N, pairs);
  for (int l = 0; l < L; l++) base = orc_tr_layout_make(ORC_G_RELU, bw, s, (size_t)B * pairs[l] * C, base).end;
  return base;
}

void orc_maxpool_keygen(uint64_t seed, uint32_t gate, int bw, int s, int B, int N, int C, const uint64_t *in_mask,
                        uint64_t *out_mask, uint8_t *k0, uint8_t *k1, size_t base) {
  const size_t n = (size_t)B * N * C;
  uint64_t *rV = (uint64_t *)malloc(8 * n), *t1 = (uint64_t *)malloc(8 * n), *t2 = (uint64_t *)malloc(8 * n);
  memcpy(rV, in_mask, 8 * n);
  pool_keygen_blk(seed, &gate, ORC_G_RELU, bw, s, B, N, C, rV, t1, t2, k0, k1, base);
  memcpy(out_mask, rV, 8 * (size_t)B * C);
  free(rV);
  free(t1);
  free(t2);
}

void orc_maxpool_eval(int bw, int s, int B, int N, int C, const uint8_t *k0, const uint8_t *k1, size_t base,
                      const uint64_t *xhat, uint64_t *yhat, uint64_t *bytes) {
  const size_t n = (size_t)B * N * C;
  uint64_t *V = (uint64_t *)malloc(8 * n), *t1 = (uint64_t *)malloc(8 * n), *t2 = (uint64_t *)malloc(8 * n);
  uint32_t g = 0;
  memcpy(V, xhat, 8 * n);
  pool_eval_blk(&g, ORC_G_RELU, bw, s, B, N, C, k0, k1, base, V, t1, t2, bytes);
  memcpy(yhat, V, 8 * (size_t)B * C);
  free(V);
  free(t1);
  free(t2);
}

/* Secure adjacency normalisation block, shared by the model and the standalone
 * entry points (gpu_mpc/secure_adj_norm.h:203-374 keygen, :393-659 eval):
 *   reveal A; reveal the degrees (row sums of the A shares, :421-493);
 *   LUT8 -> T[d] (:495-520); MUL T[d_i]*T[d_j] over the upper triangle;
 *   TRSLACK (one truncation); MUL A (.) W  (:569-651). */
static size_t adjnorm_layout(int bw, int s, int B, int N, size_t o) {
  size_t r1, r2, r3;
  orc_dcf_layout D;
  const size_t BN = (size_t)B * N, BNN = BN * N, BP = (size_t)B * pairs_of(N);
  o = orc_reveal_layout(bw, BNN, o, &r1);
  o = orc_reveal_layout(bw, BN, o, &r1);
  o = orc_lut8_layout(bw, BN, o, &D, &r1, &r2, &r3);
  o = orc_mul_layout(bw, BN, BN, BP, o, &r1, &r2, &r3);
  o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, BP, o).end;
  o = orc_mul_layout(bw, BNN, BP, BNN, o, &r1, &r2, &r3);
  return o;
}

/* rA (BNN): mask of the revealed A; rN (BNN): mask of A_norm. */
static size_t adjnorm_keygen_blk(int bw, int s, int B, int N, uint64_t seed, uint32_t *g, size_t o,
                                 uint64_t *rA, uint64_t *rN, uint8_t *k0, uint8_t *k1) {
  size_t r1, r2, r3;
  orc_dcf_layout D;
  const size_t BN = (size_t)B * N, BNN = BN * N, BP = (size_t)B * pairs_of(N);
  uint64_t *rd = (uint64_t *)malloc(8 * BN), *rinv = (uint64_t *)malloc(8 * BN);
  uint64_t *rP = (uint64_t *)malloc(8 * BP), *rW = (uint64_t *)malloc(8 * BP);
  uint32_t *oa = (uint32_t *)malloc(4 * BP), *ob = (uint32_t *)malloc(4 * BP);
  uint32_t *wa = (uint32_t *)malloc(4 * BNN), *wb = (uint32_t *)malloc(4 * BNN);
  build_maps(B, N, oa, ob, wa, wb);
  orc_reveal_keygen(seed, (*g)++, bw, BNN, rA, k0, k1, o);
  o = orc_reveal_layout(bw, BNN, o, &r1);
  orc_reveal_keygen(seed, (*g)++, bw, BN, rd, k0, k1, o);
  o = orc_reveal_layout(bw, BN, o, &r1);
  orc_lut8_keygen(seed, (*g)++, bw, BN, rd, rinv, k0, k1, o);
  o = orc_lut8_layout(bw, BN, o, &D, &r1, &r2, &r3);
  orc_mul_keygen(seed, (*g)++, bw, BN, BN, BP, oa, ob, rinv, rinv, rP, k0, k1, o);
  o = orc_mul_layout(bw, BN, BN, BP, o, &r1, &r2, &r3);
  orc_tr_keygen(seed, (*g)++, ORC_G_TRSLACK, bw, s, BP, rP, rW, k0, k1, o);
  o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, BP, o).end;
  orc_mul_keygen(seed, (*g)++, bw, BNN, BP, BNN, wa, wb, rA, rW, rN, k0, k1, o);
  o = orc_mul_layout(bw, BNN, BP, BNN, o, &r1, &r2, &r3);
  free(rd);
  free(rinv);
  free(rP);
  free(rW);
  free(oa);
  free(ob);
  free(wa);
  free(wb);
  return o;
}

/* Ah (BNN): revealed A (A + rA); An (BNN): A_norm + rN. */
static size_t adjnorm_eval_blk(int bw, int s, int B, int N, int nmax, uint32_t *g, size_t o,
                               const uint8_t *k0, const uint8_t *k1, const uint64_t *a0,
                               const uint64_t *a1, uint64_t *Ah, uint64_t *An, uint64_t *by) {
  size_t r1, r2, r3;
  orc_dcf_layout D;
  const uint64_t M = rmask(bw);
  const size_t BN = (size_t)B * N, BNN = BN * N, BP = (size_t)B * pairs_of(N);
  uint64_t *dg0 = (uint64_t *)calloc(BN, 8), *dg1 = (uint64_t *)calloc(BN, 8);
  uint64_t *dh = (uint64_t *)malloc(8 * BN), *inv = (uint64_t *)malloc(8 * BN);
  uint64_t *Ph = (uint64_t *)malloc(8 * BP), *Wh = (uint64_t *)malloc(8 * BP);
  uint32_t *oa = (uint32_t *)malloc(4 * BP), *ob = (uint32_t *)malloc(4 * BP);
  uint32_t *wa = (uint32_t *)malloc(4 * BNN), *wb = (uint32_t *)malloc(4 * BNN);
  uint64_t T[256];
  build_maps(B, N, oa, ob, wa, wb);
  orc_invsqrt_table(s, nmax, T);
  orc_reveal_eval(bw, BNN, k0, k1, o, a0, a1, Ah, by);
  trace((*g)++, BNN, Ah);
  o = orc_reveal_layout(bw, BNN, o, &r1);
  for (size_t r = 0; r < BN; r++) {
    for (int j = 0; j < N; j++) {
      dg0[r] += a0[r * N + j];
      dg1[r] += a1[r * N + j];
    }
    dg0[r] &= M;
    dg1[r] &= M;
  }
  orc_reveal_eval(bw, BN, k0, k1, o, dg0, dg1, dh, by);
  trace((*g)++, BN, dh);
  o = orc_reveal_layout(bw, BN, o, &r1);
  orc_lut8_eval(bw, BN, k0, k1, o, T, dh, inv, by);
  trace((*g)++, BN, inv);
  o = orc_lut8_layout(bw, BN, o, &D, &r1, &r2, &r3);
  orc_mul_eval(bw, BN, BN, BP, oa, ob, k0, k1, o, inv, inv, Ph, by);
  trace((*g)++, BP, Ph);
  o = orc_mul_layout(bw, BN, BN, BP, o, &r1, &r2, &r3);
  orc_tr_eval(ORC_G_TRSLACK, bw, s, BP, k0, k1, o, Ph, NULL, Wh, by);
  trace((*g)++, BP, Wh);
  o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, BP, o).end;
  orc_mul_eval(bw, BNN, BP, BNN, wa, wb, k0, k1, o, Ah, Wh, An, by);
  trace((*g)++, BNN, An);
  o = orc_mul_layout(bw, BNN, BP, BNN, o, &r1, &r2, &r3);
  free(dg0);
  free(dg1);
  free(dh);
  free(inv);
  free(Ph);
  free(Wh);
  free(oa);
  free(ob);
  free(wa);
  free(wb);
  return o;
}

size_t orc_adjnorm_key_bytes(int bw, int s, int B, int N) { return adjnorm_layout(bw, s, B, N, 0); }

int orc_adjnorm_keygen(int bw, int s, int B, int N, uint64_t seed, uint64_t *out_mask, uint8_t *k0,
                       uint8_t *k1) {
  uint32_t g = 1;
  uint64_t *rA = (uint64_t *)malloc(8 * (size_t)B * N * N);
  adjnorm_keygen_blk(bw, s, B, N, seed, &g, 0, rA, out_mask, k0, k1);
  free(rA);
  return 0;
}

int orc_adjnorm_eval(int bw, int s, int B, int N, int nmax, const uint8_t *k0, const uint8_t *k1,
                     const uint64_t *a0, const uint64_t *a1, uint64_t *out_masked, uint64_t *bytes) {
  uint32_t g = 1;
  uint64_t by = 0;
  uint64_t *Ah = (uint64_t *)malloc(8 * (size_t)B * N * N);
  adjnorm_eval_blk(bw, s, B, N, nmax, &g, 0, k0, k1, a0, a1, Ah, out_masked, &by);
  free(Ah);
  if (bytes) *bytes = by;
  return 0;
}

size_t orc_model_key_bytes(const orc_dims *d, int B) {
  const int bw = d->bw, s = d->s, N = d->n_nodes;
  size_t o = 0, r1, r2, r3;
  o = orc_reveal_layout(bw, (size_t)B * N * d->feat, o, &r1);
  o = orc_reveal_layout(bw, (size_t)B * N, o, &r1);
  o = adjnorm_layout(bw, s, B, N, o);
  for (int l = 0; l < 3; l++) {
    size_t E = (size_t)B * N * d->gcn[l];
    o = xw_slack(d) ? orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end : trunc_layout(d, 0, E, o);
    o = orc_sxs_layout(bw, (size_t)B, (size_t)N, (size_t)N, (size_t)d->gcn[l], o, &r1, &r2, &r3);
    if (agg_split(d)) {
      o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end;
      o = orc_tr_layout_make(ORC_G_RELUSLACK, bw, s, E, o).end;
    } else {
      o = trunc_layout(d, 1, E, o);
    }
  }
  int pairs[32];
  int L = pool_levels(N, pairs);
  for (int l = 0; l < L; l++)
    o = orc_tr_layout_make(pool_kind(d), bw, s, (size_t)B * pairs[l] * d->gcn[2], o).end;
  o = trunc_layout(d, 1, (size_t)B * d->dfc[0], o);
  o = trunc_layout(d, 0, (size_t)B * d->dfc[1], o);
  for (int k = 0; k < d->nfus - 1; k++) o = trunc_layout(d, 1, (size_t)B * d->fus[k], o);
  o = orc_reveal_layout(bw, (size_t)B * d->fus[d->nfus - 1], o, &r1);
  return o;
}

/* y (rows x fo) = x (rows x fi) . Wt mod 2^bw, with Wt int64 */
static void pub_gemm(int bw, size_t rows, int fi, int fo, const uint64_t *x, const int64_t *Wt,
                     uint64_t *y) {
  orc_ring_gemm(bw, 1, rows, (size_t)fi, (size_t)fo, x, (const uint64_t *)Wt, y, 0);
}

/* A layer truncation by s (+ bias in eval) and, for relu, the ReLU.  Exact: the
 * truncate-reduce TRMOD (one s-bit DCF, output exact modulo 2^(bw-s)), revealed,
 * then EXT or EXTRELU (one (bw-s-1)-bit DCF for the sign and the wrap) -- the
 * reference's TrFloor as truncate-reduce plus sign extension
 * (gpu_mpc/dpf_dcf_adapter.h:274-303) with the ReLU fused into the extension
 * (gpuReluExtend, :225-234).  With local truncation: the local shift (no key, no
 * gate id) and, for relu, a RELU gate.  Keygen maps the mask rin to rout (rin
 * may be overwritten); eval maps x (may be overwritten) to y.  Return the key end. */
static size_t trunc_layout(const orc_dims *d, int relu, size_t n, size_t o) {
  const int bw = d->bw, s = d->s;
  if (local_trunc(d)) return relu ? orc_tr_layout_make(ORC_G_RELU, bw, s, n, o).end : o;
  o = orc_tr_layout_make(ORC_G_TRMOD, bw, s, n, o).end;
  return orc_tr_layout_make(relu ? ORC_G_EXTRELU : ORC_G_EXT, bw, s, n, o).end;
}
static size_t trunc_keygen(const orc_dims *d, uint64_t seed, uint32_t *g, int relu, size_t n, uint64_t *rin,
                           uint64_t *rout, uint8_t *k0, uint8_t *k1, size_t o) {
  const int bw = d->bw, s = d->s;
  int kind = relu ? ORC_G_EXTRELU : ORC_G_EXT;
  if (local_trunc(d)) {
    orc_tr_keygen(0, 0, ORC_G_LOCALARS, bw, s, n, rin, relu ? rin : rout, NULL, NULL, o);
    if (!relu) return o;
    kind = ORC_G_RELU;
  } else {
    orc_tr_keygen(seed, (*g)++, ORC_G_TRMOD, bw, s, n, rin, rin, k0, k1, o);
    o = orc_tr_layout_make(ORC_G_TRMOD, bw, s, n, o).end;
  }
  orc_tr_keygen(seed, (*g)++, kind, bw, s, n, rin, rout, k0, k1, o);
  return orc_tr_layout_make(kind, bw, s, n, o).end;
}
static size_t trunc_eval(const orc_dims *d, uint32_t *g, int relu, size_t n, const uint8_t *k0, const uint8_t *k1,
                         size_t o, uint64_t *x, const int64_t *be, uint64_t *y, uint64_t *by) {
  const int bw = d->bw, s = d->s;
  int kind = relu ? ORC_G_EXTRELU : ORC_G_EXT;
  if (local_trunc(d)) {
    orc_tr_eval(ORC_G_LOCALARS, bw, s, n, NULL, NULL, o, x, be, relu ? x : y, by);
    if (!relu) return o;
    kind = ORC_G_RELU;
  } else {
    orc_tr_eval(ORC_G_TRMOD, bw, s, n, k0, k1, o, x, be, x, by);
    trace((*g)++, n, x);
    o = orc_tr_layout_make(ORC_G_TRMOD, bw, s, n, o).end;
  }
  orc_tr_eval(kind, bw, s, n, k0, k1, o, x, NULL, y, by);
  trace((*g)++, n, y);
  return orc_tr_layout_make(kind, bw, s, n, o).end;
}

int orc_model_keygen(const orc_dims *d, int B, uint64_t seed, const int64_t *W, uint8_t *k0,
                     uint8_t *k1) {
  const int bw = d->bw, s = d->s, N = d->n_nodes;
  const uint64_t M = rmask(bw);
  size_t o = 0, r1, r2, r3;
  uint32_t g = 1;
  const size_t BN = (size_t)B * N, BNN = BN * N;
  int maxw = d->feat;
  for (int l = 0; l < nlayers(d); l++) {
    int in, out;
    layer_io(d, l, &in, &out);
    if (out > maxw) maxw = out;
    if (in > maxw) maxw = in;
  }
  uint64_t *rX = (uint64_t *)malloc(8 * BN * maxw);
  uint64_t *rA = (uint64_t *)malloc(8 * BNN), *rm = (uint64_t *)malloc(8 * BN);
  uint64_t *rN = (uint64_t *)malloc(8 * BNN);
  uint64_t *t1 = (uint64_t *)malloc(8 * BN * maxw), *t2 = (uint64_t *)malloc(8 * BN * maxw);

  orc_reveal_keygen(seed, g++, bw, BN * d->feat, rX, k0, k1, o);
  o = orc_reveal_layout(bw, BN * d->feat, o, &r1);
  orc_reveal_keygen(seed, g++, bw, BN, rm, k0, k1, o);
  o = orc_reveal_layout(bw, BN, o, &r1);
  o = adjnorm_keygen_blk(bw, s, B, N, seed, &g, o, rA, rN, k0, k1);

  /* GCN stack: rX holds the running H mask */
  int fin = d->feat;
  for (int l = 0; l < 3; l++) {
    int fo = d->gcn[l];
    size_t E = BN * fo;
    pub_gemm(bw, BN, fin, fo, rX, W + layer_off(d, l), t1); /* mask of H.Wt */
    if (xw_slack(d)) {
      orc_tr_keygen(seed, g++, ORC_G_TRSLACK, bw, s, E, t1, t2, k0, k1, o);
      o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end;
    } else {
      o = trunc_keygen(d, seed, &g, 0, E, t1, t2, k0, k1, o);
    }
    orc_sxs_keygen(seed, g++, bw, (size_t)B, (size_t)N, (size_t)N, (size_t)fo, rN, t2, t1, k0, k1, o);
    o = orc_sxs_layout(bw, (size_t)B, (size_t)N, (size_t)N, (size_t)fo, o, &r1, &r2, &r3);
    if (agg_split(d)) {
      orc_tr_keygen(seed, g++, ORC_G_TRSLACK, bw, s, E, t1, t2, k0, k1, o);
      o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end;
      orc_tr_keygen(seed, g++, ORC_G_RELUSLACK, bw, s, E, t2, rX, k0, k1, o);
      o = orc_tr_layout_make(ORC_G_RELUSLACK, bw, s, E, o).end;
    } else {
      o = trunc_keygen(d, seed, &g, 1, E, t1, rX, k0, k1, o);
    }
    fin = fo;
  }
  /* pool: V = H3 + S*m - S, mask rH3 + S*rm */
  const int C = d->gcn[2];
  /* V = H + 2^(q-ms) m - 2^q: the sentinel -2^q on padding rows for a mask of 0
   * or 2^ms (ms = mask_scale, q = pool_sentinel_bit) */
  const uint64_t Sm = 1ull << (pool_sentinel_bit(d) - d->mask_scale);
  for (size_t r = 0; r < BN; r++)
    for (int c = 0; c < C; c++) rX[r * C + c] = (rX[r * C + c] + Sm * rm[r]) & M;
  o = pool_keygen_blk(seed, &g, pool_kind(d), bw, s, B, N, C, rX, t1, t2, k0, k1, o);
  /* drug FCs on the pooled (B x C) mask in rX */
  pub_gemm(bw, (size_t)B, C, d->dfc[0], rX, W + layer_off(d, 3), t1);
  o = trunc_keygen(d, seed, &g, 1, (size_t)B * d->dfc[0], t1, t2, k0, k1, o);
  pub_gemm(bw, (size_t)B, d->dfc[0], d->dfc[1], t2, W + layer_off(d, 4), t1);
  o = trunc_keygen(d, seed, &g, 0, (size_t)B * d->dfc[1], t1, t2, k0, k1, o);
  /* concat [drug (mask t2), protein (public, mask 0)] */
  int width = d->dfc[1] + d->prot;
  for (int b = 0; b < B; b++)
    for (int j = 0; j < width; j++)
      rX[(size_t)b * width + j] = j < d->dfc[1] ? t2[(size_t)b * d->dfc[1] + j] : 0;
  for (int k = 0; k < d->nfus; k++) {
    int fo = d->fus[k];
    pub_gemm(bw, (size_t)B, width, fo, rX, W + layer_off(d, 5 + k), t1);
    if (k < d->nfus - 1) {
      o = trunc_keygen(d, seed, &g, 1, (size_t)B * fo, t1, rX, k0, k1, o);
    } else {
      /* output mask given to both evaluators in the clear (ddg_orca_base.h:296-302,511-517) */
      size_t orr;
      orc_reveal_layout(bw, (size_t)B * fo, o, &orr);
      for (size_t i = 0; i < (size_t)B * fo; i++) {
        uint64_t v = t1[i] & M;
        if (bw == 32) {
          uint32_t x = (uint32_t)v;
          memcpy(k0 + orr + 4 * i, &x, 4);
          memcpy(k1 + orr + 4 * i, &x, 4);
        } else {
          memcpy(k0 + orr + 8 * i, &v, 8);
          memcpy(k1 + orr + 8 * i, &v, 8);
        }
      }
      o = orc_reveal_layout(bw, (size_t)B * fo, o, &r1);
      g++;
    }
    width = fo;
  }
  free(rX);
  free(rA);
  free(rm);
  free(rN);
  free(t1);
  free(t2);
  return 0;
}

int orc_model_eval(const orc_dims *d, int B, const int64_t *W, const uint8_t *k0,
                   const uint8_t *k1, const uint64_t *x0, const uint64_t *x1,
                   const uint64_t *a0, const uint64_t *a1, const uint64_t *m0,
                   const uint64_t *m1, const int64_t *prot, int64_t *out, uint64_t *bytes) {
  const int bw = d->bw, s = d->s, N = d->n_nodes;
  const uint64_t M = rmask(bw);
  size_t o = 0, r1, r2, r3;
  uint32_t g = 1;
  const size_t BN = (size_t)B * N, BNN = BN * N;
  int maxw = d->feat;
  for (int l = 0; l < nlayers(d); l++) {
    int in, outw;
    layer_io(d, l, &in, &outw);
    if (outw > maxw) maxw = outw;
    if (in > maxw) maxw = in;
  }
  uint64_t *H = (uint64_t *)malloc(8 * BN * maxw);
  uint64_t *Ah = (uint64_t *)malloc(8 * BNN), *mh = (uint64_t *)malloc(8 * BN);
  uint64_t *An = (uint64_t *)malloc(8 * BNN);
  uint64_t *t1 = (uint64_t *)malloc(8 * BN * maxw), *t2 = (uint64_t *)malloc(8 * BN * maxw);
  int64_t *be = (int64_t *)malloc(8 * BN * maxw);
  uint64_t by = 0;

  orc_reveal_eval(bw, BN * d->feat, k0, k1, o, x0, x1, H, &by);
  trace(g++, BN * d->feat, H);
  o = orc_reveal_layout(bw, BN * d->feat, o, &r1);
  orc_reveal_eval(bw, BN, k0, k1, o, m0, m1, mh, &by);
  trace(g++, BN, mh);
  o = orc_reveal_layout(bw, BN, o, &r1);
  o = adjnorm_eval_blk(bw, s, B, N, d->lut_nmax, &g, o, k0, k1, a0, a1, Ah, An, &by);

  int fin = d->feat;
  for (int l = 0; l < 3; l++) {
    int fo = d->gcn[l];
    size_t E = BN * fo;
    const int64_t *Wt = W + layer_off(d, l);
    const int64_t *bias = Wt + (size_t)fin * fo;
    pub_gemm(bw, BN, fin, fo, H, Wt, t1);
    if (xw_slack(d)) {
      orc_tr_eval(ORC_G_TRSLACK, bw, s, E, k0, k1, o, t1, NULL, t2, &by);
      trace(g++, E, t2);
      o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end;
    } else {
      o = trunc_eval(d, &g, 0, E, k0, k1, o, t1, NULL, t2, &by);
    }
    orc_sxs_eval(bw, (size_t)B, (size_t)N, (size_t)N, (size_t)fo, k0, k1, o, An, t2, t1, &by);
    trace(g++, E, t1);
    o = orc_sxs_layout(bw, (size_t)B, (size_t)N, (size_t)N, (size_t)fo, o, &r1, &r2, &r3);
    for (size_t e = 0; e < E; e++) be[e] = bias[e % fo];
    if (!agg_split(d)) {
      o = trunc_eval(d, &g, 1, E, k0, k1, o, t1, be, H, &by);
    } else {
      orc_tr_eval(ORC_G_TRSLACK, bw, s, E, k0, k1, o, t1, be, t2, &by);
      trace(g++, E, t2);
      o = orc_tr_layout_make(ORC_G_TRSLACK, bw, s, E, o).end;
      orc_tr_eval(ORC_G_RELUSLACK, bw, s, E, k0, k1, o, t2, NULL, H, &by);
      trace(g++, E, H);
      o = orc_tr_layout_make(ORC_G_RELUSLACK, bw, s, E, o).end;
    }
    fin = fo;
  }
  const int C = d->gcn[2];
  const uint64_t S = 1ull << pool_sentinel_bit(d), Sm = 1ull << (pool_sentinel_bit(d) - d->mask_scale);
  for (size_t r = 0; r < BN; r++)
    for (int c = 0; c < C; c++) H[r * C + c] = (H[r * C + c] + Sm * mh[r] - S) & M;
  o = pool_eval_blk(&g, pool_kind(d), bw, s, B, N, C, k0, k1, o, H, t1, t2, &by);
  {
    const int64_t *Wt = W + layer_off(d, 3);
    const int64_t *bias = Wt + (size_t)C * d->dfc[0];
    pub_gemm(bw, (size_t)B, C, d->dfc[0], H, Wt, t1);
    for (size_t e = 0; e < (size_t)B * d->dfc[0]; e++) be[e] = bias[e % d->dfc[0]];
    o = trunc_eval(d, &g, 1, (size_t)B * d->dfc[0], k0, k1, o, t1, be, t2, &by);
    Wt = W + layer_off(d, 4);
    bias = Wt + (size_t)d->dfc[0] * d->dfc[1];
    pub_gemm(bw, (size_t)B, d->dfc[0], d->dfc[1], t2, Wt, t1);
    for (size_t e = 0; e < (size_t)B * d->dfc[1]; e++) be[e] = bias[e % d->dfc[1]];
    o = trunc_eval(d, &g, 0, (size_t)B * d->dfc[1], k0, k1, o, t1, be, t2, &by);
  }
  int width = d->dfc[1] + d->prot;
  for (int b = 0; b < B; b++)
    for (int j = 0; j < width; j++)
      H[(size_t)b * width + j] = j < d->dfc[1] ? t2[(size_t)b * d->dfc[1] + j]
                                               : ((uint64_t)prot[(size_t)b * d->prot + j - d->dfc[1]] & M);
  /* the protein embedding is revealed by its owner (deepdtagen.h:60-67): one
   * message of B x prot ring elements each way */
  by += 2ull * (size_t)B * d->prot * (uint64_t)(bw / 8);
  for (int k = 0; k < d->nfus; k++) {
    int fo = d->fus[k];
    const int64_t *Wt = W + layer_off(d, 5 + k);
    const int64_t *bias = Wt + (size_t)width * fo;
    pub_gemm(bw, (size_t)B, width, fo, H, Wt, t1);
    if (k < d->nfus - 1) {
      for (size_t e = 0; e < (size_t)B * fo; e++) be[e] = bias[e % fo];
      o = trunc_eval(d, &g, 1, (size_t)B * fo, k0, k1, o, t1, be, H, &by);
    } else {
      size_t orr;
      orc_reveal_layout(bw, (size_t)B * fo, o, &orr);
      for (int b = 0; b < B; b++) {
        uint64_t rz;
        if (bw == 32) {
          uint32_t x;
          memcpy(&x, k0 + orr + 4 * (size_t)b * fo, 4);
          rz = x;
        } else {
          memcpy(&rz, k0 + orr + 8 * (size_t)b * fo, 8);
        }
        uint64_t z = (t1[(size_t)b * fo] - rz) & M;
        int64_t zs = bw == 32 ? (int64_t)(int32_t)(uint32_t)z : (int64_t)z;
        int64_t y = (zs >> s) + bias[0];
        if (bw == 32) y = (int64_t)(int32_t)(uint32_t)((uint64_t)y & M);
        out[b] = y;
      }
      trace(g++, (size_t)B * fo, t1);
      o = orc_reveal_layout(bw, (size_t)B * fo, o, &r1);
    }
    width = fo;
  }
  if (bytes) *bytes = by;
  free(H);
  free(Ah);
  free(mh);
  free(An);
  free(t1);
  free(t2);
  free(be);
  return 0;
}
