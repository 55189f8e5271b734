// kernels.h -- host-side launchers of the libmpcx HIP kernels.
//
// Every launcher enqueues on the given stream and returns the launch status.
// Two-party kernels take both parties' key blocks: blockIdx.y selects the party
// and a party's threads read only that party's key planes; exchanged messages
// are written to per-party device buffers and read back by the peer's kernels
// (the online exchange through device memory).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "mpcx_core.h"

namespace mpcx {

constexpr int kBothAesAlone = 6, kBothAesLanes = 14;
constexpr int kBothMinAlone = 1024, kBothMinLanes = 512;
struct Launch {
  hipStream_t stream = nullptr;
  int num_cu = 256;
  int aes_variant = 0;  // LDS T-table layout, see aes_variants()
  int aes_block = 0;    // threads per block for AES kernels (0 = variant default)
  // The one-launch gate kernel spreads a small gate over the CUs (smaller
  // workgroups, about one per CU).  A caller whose other streams keep the GPU
  // busy clears it: the spread workgroups would take LDS from theirs.
  bool spread_small = true;
  // Longest gate (AES calls per element and party) whose launches of at least
  // both_min elements per CU run in the both-party form over Z_2^32: one thread
  // per element holds both parties' keys (0 = never).  Gates of up to 6 calls
  // gain alone and beside other streams' work; up to 14 only beside other
  // streams' work (a model's lanes), and lose alone.  Alone a launch needs 1024
  // elements per CU to give every CU a 1024-thread workgroup; beside other
  // lanes' work 512 measured best (they fill the CUs it leaves).
  int both_aes = kBothAesAlone;
  int both_min = kBothMinAlone;
  // Launches of a profiled forward use a separately named instantiation of the
  // DCF-evaluation kernel (same code), so kernel traces can tell them apart.
  bool profiled = false;
  // ring GEMM path: 0 = int8 matrix cores, in Z_2^32 the panel kernel where it
  // applies (use_panels), else the wide-K / fused SxS kernels where they apply
  // and the tiled kernels elsewhere; 3 = the same without the panel kernel;
  // 1 = VALU; 2 = tiled matrix-core kernels only.  Z_2^64 products with
  // K >= 2^15 take the VALU path always.
  int gemm = 0;
  // two- and three-panel Z_2^32 products with K in one step run on the
  // panel kernel pipelined across panels (k_panels_pf); 0: k_panels
  int panel_pf = 1;
  // columns per k_panels_pf workgroup in 16-column tiles (1..3); 0: by rounds
  int panel_nt = 0;
  // Z_2^32 SxS pairs (both parties) in the LDS-staged kernel (k_sxs_staged)
  int sxs_staged = 1;
  // party-mode gate calls synchronise the stream before returning (0: they
  // return with their work enqueued, for callers that order by stream)
  int party_sync = 1;
  // model forwards with resident keys are captured once per batch size into a
  // HIP graph and replayed (0 = enqueue every kernel each time)
  int graph = 1;
  // the dealer's 16-byte key (dealer_key): set, or the seed alone
  bool has_dealer_key = false;
  uint8_t dealer_key[16] = {};
  // Model lanes of a few samples run the max-pool levels from this index on
  // (0 = the first level) in one launch (launch_tr_eval_pool_tail); -1: every
  // level alone.
  int pool_tail = 2;
  // gates of at most this many elements per CU take the quad-lane form
  // (at least 64: two 256-thread workgroups per CU; above, 512-thread ones)
  int quad_per_cu = 64;
  // the same in a model lane that runs alone (ModelBase::set_alone): gates of
  // up to 192 elements per CU, in two rounds of two 512-thread workgroups, are
  // shorter chains than the one-lane kernel's (B = 1: 0.496-0.497 against
  // 0.522-0.525 ms at 64); beside other lanes the larger workgroups keep those
  // lanes' gates off the CUs (B = 8 in 3 lanes: 4% slower at 128)
  int quad_alone = 192;
  // -1: two-party kernels evaluate both parties (blockIdx.y = party).  0 or 1:
  // only that party (one process per party): the launchers take the party's own
  // key (and input share, message buffer) in both party slots and launch one
  // party row of workgroups.
  int party = -1;
};

struct AesVariant {
  int nt, rep, block;
  const char *name;
};
const AesVariant *aes_variants(int *count);

// ---------------- PRG ----------------
hipError_t launch_hash(const Launch &L, int leaf, size_t n, const uint4 *in, uint4 *out);
hipError_t launch_prf(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, uint4 *out);

// ---------------- standalone DCF ----------------
hipError_t launch_dcf_keygen(const Launch &L, uint64_t seed, uint32_t gate, uint32_t fbase, int m, size_t n,
                             const uint64_t *alpha, const uint8_t *rbit, uint8_t *k0, uint8_t *k1, size_t base);
hipError_t launch_dcf_eval(const Launch &L, int party, int m, size_t n, const uint8_t *key, size_t base,
                           const uint64_t *x, uint64_t *out_bits);
// The same on ring elements x (reduced to the m-bit domain in the kernel), the
// output bits XORed with mask (32-bit words, bit i of word i/32) when mask is
// not null: the reference's gpuDcf<T, 1, idPrologue, maskEpilogue>.
template <typename T>
hipError_t launch_dcf_eval_ring(const Launch &L, int m, size_t n, const uint8_t *key, const T *x,
                                const uint32_t *mask, uint64_t *out_bits);

// ---------------- truncation / ReLU family ----------------
template <typename T>
struct TrPlan {
  TrLayout lay;
  const uint8_t *key[2];
};

template <typename T>
hipError_t launch_tr_keygen(const Launch &L, const TrLayout &lay, uint64_t seed, uint32_t gate, const T *in_mask,
                            T *out_mask, uint8_t *k0, uint8_t *k1);
// Regenerates into key (laid out by lay) the planes of party p's key of a
// truncation-family gate that keygen drew from the party's own PRF key
// (party_key): its DCF roots and output-mask bits, and for party 0 its shares
// of kappa and of the G table.
template <typename T>
hipError_t launch_tr_expand(const Launch &L, const TrLayout &lay, const uint8_t party_key16[16], uint32_t gate,
                            int party, uint8_t *key);
// The kernel form launch_tr_eval takes for a gate on this launch configuration
// (the same decision the launcher makes).
constexpr int kFormOneLane = 0, kFormBoth = 1, kFormQuad = 2;
int tr_eval_form(const Launch &L, const TrLayout &lay);
// Evaluation of a truncation-family gate by both parties in one launch: the DCF
// walks, the exchange of the masked DCF output bits, the output messages and
// their sum, the revealed output yhat (N words; may alias xhat).
template <typename T>
hipError_t launch_tr_eval(const Launch &L, const TrLayout &lay, const uint8_t *k0, const uint8_t *k1,
                          const T *xhat, const T *bias, int bias_ncol, T *yhat);

// One level of the max-pool tree, max(a, b) = a + ReLU(b - a), as one gate
// launch of both parties: the gate (lay, N = B (R/2) C elements) evaluates the
// pair differences V[b][2j+1][c] - V[b][2j][c] of the R rows of C words of each
// of B blocks, and party 0's threads write V[b][2j][c] + y into row j of Vn
// (R/2 + R%2 rows per block; an odd level's last row is carried).  Requires
// B R C < 2^32; V and Vn distinct.
template <typename T>
hipError_t launch_tr_eval_pool(const Launch &L, const TrLayout &lay, const uint8_t *k0, const uint8_t *k1, int B,
                               int R, int C, const T *V, T *Vn);

// The last nlev levels of the max-pool tree in one launch: lay[l] is level l's
// gate (one RELU kind, N = B (R_l/2) C with R_0 = R0 and R_{l+1} = R_l/2 +
// R_l%2, ending at one row), the keys of every level relative to k0 / k1; V
// holds B blocks of R0 rows of C words, out receives B rows of C words (each
// column's maximum).  Each workgroup takes whole columns and keeps them in LDS
// across the levels (quad-lane gates, both parties).  B R0 C < 2^31.
template <typename T>
hipError_t launch_tr_eval_pool_tail(const Launch &L, const TrLayout *lay, int nlev, const uint8_t *k0,
                                   const uint8_t *k1, int B, int R0, int C, const T *V, T *out);

// Two gates of the same element count in one launch: lay on xhat (with the
// bias), then lay2 on lay's revealed output, which never leaves the launch;
// lay2's revealed output in out.  The model's truncations (TRMOD, then EXT or
// EXTRELU) with resident keys.
template <typename T>
hipError_t launch_tr_eval2(const Launch &L, const TrLayout &lay, const TrLayout &lay2, const uint8_t *k0,
                           const uint8_t *k1, const T *xhat, const T *bias, int bias_ncol, T *out);

// Party mode (L.party = p), the same gate in two launches around the two
// exchanges.  Phase 1: party p's masked DCF output bits, one bit per element,
// packed 64 per word: plane a at bits[0, W), plane b at bits[W, 2W), W = ceil(N/64)
// (lay.use_a / lay.use_b tell which planes the gate has).
template <typename T>
hipError_t launch_tr_party_bits(const Launch &L, const TrLayout &lay, const uint8_t *key, const T *xhat,
                                const T *bias, int bias_ncol, uint64_t *bits);
// Phase 2, after the planes are exchanged: party p's output message msg (N
// words) from its own and the peer's planes.  For G_DRELU the output bit is
// public after phase 1: msg receives it directly (no second exchange).
template <typename T>
hipError_t launch_tr_party_msg(const Launch &L, const TrLayout &lay, const uint8_t *key, const T *xhat,
                               const T *bias, int bias_ncol, const uint64_t *own, const uint64_t *peer, T *msg);

// out = m0 + m1 (reconstruction of a revealed value from both parties' messages)
template <typename T>
hipError_t launch_reconstruct(const Launch &L, size_t n, const T *m0, const T *m1, T *out);
// Reduced-width wire form (party mode) of a message known modulo 2^m, 1 <= m <
// bits of T: element i at bits [i m, i m + m) of packed_words(n, m) 64-bit words.
template <typename T>
hipError_t launch_pack_bits(const Launch &L, size_t n, int m, const T *v, uint64_t *words);
// out[i] = (own[i] + element i of the peer's packed message) mod 2^m
template <typename T>
hipError_t launch_unpack_reconstruct(const Launch &L, size_t n, int m, const T *own, const uint64_t *peer, T *out);
// LocalARS: y[i] = (signed x[i]) >> s + (bias ? bias[i % ncol] : 0), mod 2^bw (bw = 8 sizeof(T))
template <typename T>
hipError_t launch_local_ars(const Launch &L, size_t n, int s, const T *x, const T *bias, int ncol, T *y);

// ---------------- reveal ----------------
template <typename T>
hipError_t launch_reveal_keygen(const Launch &L, const RevealLayout &lay, uint64_t seed, uint32_t gate, T *mask,
                                uint8_t *k0, uint8_t *k1);
// msg_p = v_p + R_p ; if rowlen > 0, v_p[i] is the row sum of a_p (degree shares)
template <typename T>
hipError_t launch_reveal_eval(const Launch &L, const RevealLayout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *v0, const T *v1, int rowlen, T *msg0, T *msg1);
// Both parties in this process: out = msg0 + msg1 from one launch (each party's
// message formed from its own share and key; no message planes in HBM).
template <typename T>
hipError_t launch_reveal_sum(const Launch &L, const RevealLayout &lay, const uint8_t *k0, const uint8_t *k1,
                             const T *v0, const T *v1, int rowlen, T *out);

// ---------------- Beaver product ----------------
// Operand indices of z[k] = x[a(k)] * y[b(k)]: explicit index arrays, or one of
// the two maps of the adjacency normalisation, computed on the fly (N nodes
// per graph, P = N(N+1)/2 node pairs i <= j per graph, pair index
// pidx(i, j) = i*N - i(i-1)/2 + j - i):
//   OUTER_TRI     k = g*P + pidx(i, j)        -> a = g*N + i, b = g*N + j
//   SYM_HADAMARD  k = (g*N + i)*N + j         -> a = k, b = g*P + pidx(min(i,j), max(i,j))
struct MulMap {
  enum Kind { EXPLICIT = 0, OUTER_TRI = 1, SYM_HADAMARD = 2 };
  int kind = EXPLICIT;
  const uint32_t *ia = nullptr, *ib = nullptr;
  uint32_t N = 0;
  static MulMap explicit_maps(const uint32_t *a, const uint32_t *b) {
    MulMap m;
    m.ia = a;
    m.ib = b;
    return m;
  }
  static MulMap of(int kind, int n) {
    MulMap m;
    m.kind = kind;
    m.N = uint32_t(n);
    return m;
  }
};

template <typename T>
hipError_t launch_mul_keygen(const Launch &L, const MulLayout &lay, uint64_t seed, uint32_t gate, const MulMap &map,
                             const T *rx, const T *ry, T *rz, uint8_t *k0, uint8_t *k1);
template <typename T>
hipError_t launch_mul_eval(const Launch &L, const MulLayout &lay, const uint8_t *k0, const uint8_t *k1,
                           const MulMap &map, const T *xhat, const T *yhat, T *msg0, T *msg1);
// Both parties in this process: the revealed product msg0 + msg1 from one launch.
template <typename T>
hipError_t launch_mul_eval_sum(const Launch &L, const MulLayout &lay, const uint8_t *k0, const uint8_t *k1,
                               const MulMap &map, const T *xhat, const T *yhat, T *out);

// ---------------- LUT8 ----------------
template <typename T>
hipError_t launch_lut8_keygen(const Launch &L, const Lut8Layout &lay, uint64_t seed, uint32_t gate,
                              const T *in_mask, T *out_mask, uint8_t *k0, uint8_t *k1);
template <typename T>
hipError_t launch_lut8_phase1(const Launch &L, const Lut8Layout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *table, const T *xhat, T *msg0, T *msg1);
template <typename T>
hipError_t launch_lut8_phase2(const Launch &L, const Lut8Layout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *vhat, T *msg0, T *msg1);

// ---------------- SxS keys ----------------
template <typename T>
hipError_t launch_split(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, const T *v,
                        T *p0, T *p1, T *share0_copy);
template <typename T>
hipError_t launch_prf_ring(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, T *out);

// ---------------- elementwise ----------------
template <typename T>
hipError_t launch_axpby(const Launch &L, size_t n, T a, const T *x, T b, const T *y, T c, T *out);
// out[r*cols+c] = a*x + b*y + (v[c] << shift); x, y, v may be null
template <typename T>
hipError_t launch_lincomb(const Launch &L, size_t rows, size_t cols, T a, const T *x, T b, const T *y, const T *v,
                          int shift, T *out);
// Levels of the pairwise max tree over N rows (pairs (2j, 2j+1), an odd last
// row carried to the next level); pairs[l] = pairs at level l (31 levels at most).
inline int pool_levels(int N, int *pairs) {
  int R = N, L = 0;
  while (R > 1) {
    pairs[L++] = R / 2;
    R = R / 2 + (R & 1);
  }
  return L;
}
// pool prep: V[r*C+c] = H[r*C+c] + S*m[r] + off
template <typename T>
hipError_t launch_pool_prep(const Launch &L, size_t rows, int C, const T *H, const T *m, T S, T off, T *V);
// D[(b*pr+j)*C+c] = V[(b*R+2j+1)*C+c] - V[(b*R+2j)*C+c]
template <typename T>
hipError_t launch_pool_diff(const Launch &L, int B, int R, int C, const T *V, T *D);
// Vn[(b*Rn+j)*C+c] = V[(b*R+2j)*C+c] + y0[..] (+ y1[..]); carry the odd row
template <typename T>
hipError_t launch_pool_combine(const Launch &L, int B, int R, int C, const T *V, const T *y0, const T *y1, T *Vn);
// concat rows: out[b*(w1+w2)+j] = j<w1 ? a[b*w1+j] : (bzero ? 0 : b[b*w2+j-w1])
template <typename T>
hipError_t launch_concat(const Launch &L, int B, int w1, int w2, const T *a, const T *b, T *out);
// output: out[b] = wrap((signed(zhat[b]-rz[b]) >> s) + bias)
template <typename T>
hipError_t launch_output(const Launch &L, int B, int bw, int s, const T *zhat, const T *rz, int64_t bias,
                         int64_t *out);
template <typename T>
hipError_t launch_rowsum(const Launch &L, size_t rows, int len, const T *a, T *out);

}  // namespace mpcx
