// gates.hip -- the truncation / ReLU gate family (the FSS gates of the online
// path): dealer keygen, the one-launch evaluation of both parties, party mode's
// two phases, and the expansion of seed-compressed keys.
//
// Reference interfaces: gpuRelu / gpuGenReluKey (gpu_mpc/ddg_orca.h:103-104,233),
// gpuTruncate / genGPUTruncateKey (gpu_mpc/ddg_orca.h:116-118,240), the DCF of
// gpuDcf / gpuKeyGenDCF underneath (gpu_mpc/dpf_dcf_adapter.h:266,372).
// Gate algebra (masked-public x^ = x + r): the truncation family evaluates two DCFs on
// x' = x^ + bias*2^s + 2^(n-1), c = [x' mod 2^(n-1) < r mod 2^(n-1)] and
// d = [x' mod 2^s < r mod 2^s], then floor(u/2^s) = floor(x'/2^s) - floor(r/2^s) - d
// + 2^(n-s)*w with the wrap w = msb(x') ? (msb(r) & c) : (msb(r) | c); the dealer
// tabulates all but the public floor(x'/2^s) over the 8 public cases.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "dcf_dev.h"
#include "kernels.h"
#include "launch_util.h"

namespace mpcx {

// ---------------------------------------------------------------------------
// truncation / ReLU family
// ---------------------------------------------------------------------------
template <typename T>
struct TrArgs {
  AesRK kd;
  AesRK kp[2];  // the parties' own PRF keys (keygen and seeded-plane expansion)
  int kind, n, s;
  int sb;        // sign bit of the shifted input (tr_sign_bit)
  int m, sh;     // input width (tr_in_bits) and the gate's own shift (tr_shift)
  int ncase;     // cases of the G table
  int relu;      // the gate carries kappa shares
  int has_bias;  // the bias is added before the shift
  size_t N;
  const uint8_t *k0, *k1;
  uint8_t *w0, *w1;  // writable keys (keygen)
  DcfLayout a, b;
  size_t off_kappa, off_g;
  int use_a, use_b;
  const T *xhat;
  const T *bias;
  int bias_ncol;
  T *out;  // revealed output (eval)
  const T *in_mask;
  T *out_mask;
  uint32_t gate;
  int prio;  // eval: the launch's waves raise their issue priority (a small gate)
};

// A gate evaluation in the max-pool form: element i is pair j of block b, column
// c (i = (b pr + j) C + c) of the level's rows v (R rows of C per block); its
// masked input is v[2j+1] - v[2j] and party 0 writes v[2j] + y into row j of the
// next level vn (R / 2 + R % 2 rows per block), the odd last row carried.  The
// regular instances take no such argument and compile without it.
template <typename T>
struct TrPool {
  uint32_t R = 0, C = 0, pr = 0, B = 0;
  const T *v = nullptr;
  T *vn = nullptr;
};
// offset of row 2j of element i's pair in v, and of its row j in vn
template <typename T>
__device__ __forceinline__ uint32_t pool_src(const TrPool<T> &q, uint32_t i, uint32_t *o) {
  const uint32_t C = q.C, pr = q.pr, Rn = pr + (q.R & 1u);
  const uint32_t bj = i / C, c = i - bj * C, b = bj / pr, j = bj - b * pr;
  *o = (b * Rn + j) * C + c;
  return (b * q.R + 2 * j) * C + c;
}
// The carried last rows of an odd level (all threads of the launch share them).
template <typename T>
__device__ __forceinline__ void pool_carry(const TrPool<T> &q) {
  if (!(q.R & 1u)) return;
  const uint32_t C = q.C, pr = q.pr, Rn = pr + 1, nc = q.B * C;
  for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < nc; k += gridDim.x * blockDim.x) {
    const uint32_t b = k / C, c = k - b * C;
    q.vn[(b * Rn + pr) * C + c] = q.v[(b * q.R + q.R - 1) * C + c];
  }
}

__device__ __forceinline__ bool relu_like(int kind) {
  return kind == G_RELU || kind == G_RELUSLACK || kind == G_RELUPOOL;
}

// v mod 2^m for 1 <= m <= bits of T
template <typename T>
__device__ __forceinline__ T low_bits(T v, int m) {
  return m >= int(8 * sizeof(T)) ? v : T(v & ((T(1) << m) - T(1)));
}

// the shifted input of element i from its masked input xh = x^[i]
template <typename T>
__device__ __forceinline__ T tr_shifted_input(const TrArgs<T> &a, size_t i, T xh) {
  T x = xh;
  if (a.has_bias && a.bias) x += T(a.bias[uint32_t(i % uint32_t(a.bias_ncol))]) << a.s;
  return low_bits<T>(x + (T(1) << a.sb), a.m);
}

// Party p's masked DCF output bits of element i (the gate's planes a and b):
// the DCF walks over the shifted input xp with the party's roots and mask bits
// (K) and the correction and leaf words, which are the same in both parties'
// keys (KC: any party's copy).
template <typename T, class Aes>
__device__ __forceinline__ void tr_dcf_bits(Aes &aes, const TrArgs<T> &a, const uint8_t *K,
                                            const uint8_t *KC, size_t i, T xp, uint32_t *ra, uint32_t *rb) {
  const T lowmask = (T(1) << a.sb) - T(1);
  const T smask = (T(1) << a.s) - T(1);
  if (a.use_a) {
    *ra = dcf_eval_walk(aes, reinterpret_cast<const uint4 *>(K + a.a.off_root)[i], a.a.m, a.a.L,
                        reinterpret_cast<const uint4 *>(KC + a.a.off_cw) + i, a.N,
                        reinterpret_cast<const uint4 *>(KC + a.a.off_leaf)[i], uint64_t(xp & lowmask));
    *ra ^= get_bit(reinterpret_cast<const uint64_t *>(K + a.a.off_z), i);
  }
  if (a.use_b) {
    *rb = dcf_eval_walk(aes, reinterpret_cast<const uint4 *>(K + a.b.off_root)[i], a.b.m, a.b.L,
                        reinterpret_cast<const uint4 *>(KC + a.b.off_cw) + i, a.N,
                        reinterpret_cast<const uint4 *>(KC + a.b.off_leaf)[i], uint64_t(xp & smask));
    *rb ^= get_bit(reinterpret_cast<const uint64_t *>(K + a.b.off_z), i);
  }
}

// Party p's output message for element i once the masked DCF outputs are
// public: hb the sign-position bit of the shifted input, bh and dh the
// reconstructed masked bits of planes a and b.  The two parties' messages add
// up to the masked output.
template <typename T>
__device__ __forceinline__ T tr_out_share(const TrArgs<T> &a, int p, const uint8_t *K, size_t i, T xh, T xp,
                                          uint32_t hb, uint32_t bh, uint32_t dh) {
  const T *G = reinterpret_cast<const T *>(K + a.off_g);
  const T *kap = reinterpret_cast<const T *>(K + a.off_kappa);
  const T one0 = p == 0 ? T(1) : T(0);
  const T A = (xp >> a.sh) - (T(1) << (a.m - 1 - a.sh));
  if (a.kind == G_TRMOD) return one0 * A + G[size_t(dh) * a.N + i];  // exact modulo 2^(n-s): no wrap term
  if (a.kind == G_EXT) return one0 * A + G[size_t(hb * 2 + bh) * a.N + i];
  if (a.kind == G_EXTRELU || a.kind == G_TRRELU) {
    const uint32_t z = hb ^ bh;
    const T k = kap[i];
    const T cp = z ? T(one0 - k) : k;
    const size_t c = a.kind == G_EXTRELU ? hb * 2 + bh : hb * 4 + bh * 2 + dh;
    return cp * A + G[c * a.N + i];
  }
  if (a.kind == G_TR) return one0 * A + G[size_t(hb * 4 + bh * 2 + dh) * a.N + i];
  if (a.kind == G_DRELU) return one0 * T(hb ^ bh);  // the public masked bit; party 0 carries it
  if (relu_like(a.kind)) {
    const uint32_t z = hb ^ bh;
    const T k = kap[i];
    const T cp = z ? T(one0 - k) : k;
    return cp * xh + G[size_t(z) * a.N + i];
  }
  // G_TRSLACK
  const uint32_t Hh = uint32_t(xp >> (a.n - 2)) & 3u;
  return one0 * A + G[size_t(Hh * 2 + dh) * a.N + i];
}

// The revealed output from the two parties' messages: their sum, reduced to
// bw - s bits for TRMOD (tr_out_bits), whose output is known only modulo
// 2^(bw-s) and is revealed at that width.
template <typename T>
__device__ __forceinline__ T tr_reveal_sum(const TrArgs<T> &a, T m0, T m1) {
  const T y = m0 + m1;
  return a.kind == G_TRMOD ? low_bits<T>(y, a.n - a.s) : y;
}

// One launch evaluates a gate for both parties.  A workgroup of 2h threads
// takes tiles of h elements: its first h threads are party 0, the last h party
// 1, each evaluating its own keys on the same elements.  The two exchanges of
// the protocol go through LDS: the masked DCF output bits (one ballot word per
// wave and DCF), then the output messages, which party 0's threads add into the
// revealed output.  TAG = 1 marks the launches of a profiled forward (identical
// code, its own name in kernel traces).
constexpr int kTrMaxTile = 512;  // elements per tile (workgroups of up to 1024 threads)

// The exchange buffers of a workgroup: per party, the ballot words of the two
// DCF planes (one per wave) and the output messages.
template <typename T>
struct TrXchg {
  uint64_t xa[2][kTrMaxTile / 64], xb[2][kTrMaxTile / 64];
  T xm[2][kTrMaxTile];
};

// Gate a on element i of a tile (element e of the tile, wave wv of its party's
// half, masked input xh): party p's DCF walks, the exchange of the masked DCF
// output bits, party p's output message, the exchange of the messages.  Every
// thread of the workgroup calls it (the exchanges synchronise the workgroup);
// it returns the revealed output of element i to both parties' threads.
template <typename T, class Aes>
__device__ __forceinline__ T tr_tile(Aes &aes, const TrArgs<T> &a, TrXchg<T> &x, int p, int e, int wv,
                                     const uint8_t *K, const uint8_t *KC, size_t i, bool in, T xh) {
  uint32_t ra = 0, rb = 0;
  T xp = 0;
  if (in) {
    xp = tr_shifted_input(a, i, xh);
    tr_dcf_bits(aes, a, K, KC, i, xp, &ra, &rb);
  }
  // exchange 1: the masked DCF output bits
  const uint64_t wa = __ballot(ra), wb = __ballot(rb);
  if (lane_id() == 0) {
    x.xa[p][wv] = wa;
    x.xb[p][wv] = wb;
  }
  __syncthreads();
  if (in) {
    const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
    const uint32_t bh = a.use_a ? uint32_t((x.xa[0][wv] ^ x.xa[1][wv]) >> lane_id()) & 1u : 0u;
    const uint32_t dh = a.use_b ? uint32_t((x.xb[0][wv] ^ x.xb[1][wv]) >> lane_id()) & 1u : 0u;
    x.xm[p][e] = tr_out_share(a, p, K, i, xh, xp, hb, bh, dh);  // exchange 2: the output messages
  }
  __syncthreads();
  const T y = in ? tr_reveal_sum<T>(a, x.xm[0][e], x.xm[1][e]) : T(0);
  __syncthreads();  // the next gate or tile reuses the exchange buffers
  return y;
}

// The tiles of one launch: gate a on x^, then (TWO) gate a2 on a's revealed
// output, which both parties hold once it is revealed; party 0's threads write
// the last gate's revealed output.
template <typename T, int NT, int REP, bool TWO, bool POOL>
__device__ __forceinline__ void tr_eval_tiles(const TrArgs<T> &a, const TrArgs<T> &a2, const TrPool<T> &q) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  __shared__ TrXchg<T> x;
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const int h = int(blockDim.x) / 2;
  const int p = int(threadIdx.x) >= h ? 1 : 0;
  const int e = int(threadIdx.x) - p * h;  // element of the tile
  const int wv = e >> 6;                   // wave of the party's half
  // The correction words and leaf words of a DCF key are the same for both
  // parties (public to both); both parties read party 0's planes, so one copy
  // serves the two evaluations (and a streamed arena moves it once).
  const uint8_t *K = p ? a.k1 : a.k0, *KC = a.k0;
  const size_t stride = size_t(gridDim.x) * size_t(h);
  for (size_t base = size_t(blockIdx.x) * h; base < a.N; base += stride) {
    const size_t i = base + size_t(e);
    const bool in = i < a.N;
    T xin = 0, v0 = 0;
    uint32_t o = 0;
    if (in) {
      if constexpr (POOL) {
        const uint32_t s0 = pool_src(q, uint32_t(i), &o);
        v0 = q.v[s0];
        xin = q.v[s0 + q.C] - v0;
      } else {
        xin = a.xhat[i];
      }
    }
    T y = tr_tile(aes, a, x, p, e, wv, K, KC, i, in, xin);
    if constexpr (TWO) y = tr_tile(aes, a2, x, p, e, wv, K, KC, i, in, y);
    if (p == 0 && in) {
      if constexpr (POOL)
        q.vn[o] = v0 + y;
      else
        a.out[i] = y;
    }
  }
  if constexpr (POOL) pool_carry(q);
}

// ---- both-party form (throughput launches) ----
// Gate a on element i for both parties in one thread: the two parties' DCF
// walks side by side (dcf_eval_walk2: two independent AES chains, each level's
// correction word read once), their masked bits combined in registers, and the
// sum of the two output messages, the revealed output.  The same keys and
// algebra as tr_tile, with no exchange buffers and no barriers.
template <typename T, class Aes>
__device__ __forceinline__ T tr_both(const Aes &aes, const TrArgs<T> &a, size_t i, T xh) {
  const T xp = tr_shifted_input(a, i, xh);
  const T lowmask = (T(1) << a.sb) - T(1);
  const T smask = (T(1) << a.s) - T(1);
  uint32_t bh = 0, dh = 0;
  if (a.use_a) {
    bh = dcf_eval_walk2(aes, reinterpret_cast<const uint4 *>(a.k0 + a.a.off_root)[i],
                        reinterpret_cast<const uint4 *>(a.k1 + a.a.off_root)[i], a.a.m, a.a.L,
                        reinterpret_cast<const uint4 *>(a.k0 + a.a.off_cw) + i, a.N,
                        reinterpret_cast<const uint4 *>(a.k0 + a.a.off_leaf)[i], uint64_t(xp & lowmask));
    bh ^= get_bit(reinterpret_cast<const uint64_t *>(a.k0 + a.a.off_z), i) ^
          get_bit(reinterpret_cast<const uint64_t *>(a.k1 + a.a.off_z), i);
  }
  if (a.use_b) {
    dh = dcf_eval_walk2(aes, reinterpret_cast<const uint4 *>(a.k0 + a.b.off_root)[i],
                        reinterpret_cast<const uint4 *>(a.k1 + a.b.off_root)[i], a.b.m, a.b.L,
                        reinterpret_cast<const uint4 *>(a.k0 + a.b.off_cw) + i, a.N,
                        reinterpret_cast<const uint4 *>(a.k0 + a.b.off_leaf)[i], uint64_t(xp & smask));
    dh ^= get_bit(reinterpret_cast<const uint64_t *>(a.k0 + a.b.off_z), i) ^
          get_bit(reinterpret_cast<const uint64_t *>(a.k1 + a.b.off_z), i);
  }
  const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
  return tr_reveal_sum<T>(a, tr_out_share(a, 0, a.k0, i, xh, xp, hb, bh, dh),
                          tr_out_share(a, 1, a.k1, i, xh, xp, hb, bh, dh));
}

// The elements of a both-party launch, one per thread (grid-stride): gate a,
// then (TWO) gate a2 on its revealed output, or (POOL) a max-pool level.
template <typename T, int NT, int REP, bool TWO, bool POOL>
__device__ __forceinline__ void tr_eval_both(const TrArgs<T> &a, const TrArgs<T> &a2, const TrPool<T> &q) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  const AesLds<NT, REP> aes(lds);
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < a.N; i += stride) {
    T xin, v0 = 0;
    uint32_t o = 0;
    if constexpr (POOL) {
      const uint32_t s0 = pool_src(q, uint32_t(i), &o);
      v0 = q.v[s0];
      xin = q.v[s0 + q.C] - v0;
    } else {
      xin = a.xhat[i];
    }
    T y = tr_both(aes, a, i, xin);
    if constexpr (TWO) y = tr_both(aes, a2, i, y);
    if constexpr (POOL)
      q.vn[o] = v0 + y;
    else
      a.out[i] = y;
  }
  if constexpr (POOL) pool_carry(q);
}

// ---- quad-lane form (latency-bound launches, AesPerm2 table) ----
// The DCF walks of tr_dcf_bits with four lanes per element and party (lane j of
// the quad reads word j of the roots, correction words and leaves).
template <typename T>
__device__ __forceinline__ void tr_dcf_bits_quad(const AesQuad &aes, const AesQuad::Keys &kH,
                                                 const AesQuad::Keys &kL, const TrArgs<T> &a, const uint8_t *K,
                                                 const uint8_t *KC, size_t i, T xp, uint32_t *ra, uint32_t *rb) {
  const T lowmask = (T(1) << a.sb) - T(1);
  const T smask = (T(1) << a.s) - T(1);
  const size_t w = 4 * i + aes.j, sw = 4 * a.N;
  if (a.use_a) {
    *ra = dcf_eval_walk_quad(aes, kH, kL, reinterpret_cast<const uint32_t *>(K + a.a.off_root)[w], a.a.m, a.a.L,
                             reinterpret_cast<const uint32_t *>(KC + a.a.off_cw) + w, sw,
                             reinterpret_cast<const uint32_t *>(KC + a.a.off_leaf)[w], uint64_t(xp & lowmask));
    *ra ^= get_bit(reinterpret_cast<const uint64_t *>(K + a.a.off_z), i);
  }
  if (a.use_b) {
    *rb = dcf_eval_walk_quad(aes, kH, kL, reinterpret_cast<const uint32_t *>(K + a.b.off_root)[w], a.b.m, a.b.L,
                             reinterpret_cast<const uint32_t *>(KC + a.b.off_cw) + w, sw,
                             reinterpret_cast<const uint32_t *>(KC + a.b.off_leaf)[w], uint64_t(xp & smask));
    *rb ^= get_bit(reinterpret_cast<const uint64_t *>(K + a.b.off_z), i);
  }
}

// tr_tile with a quad of lanes per element and party: the quad's lanes carry the
// same bits, so an element's bit in a ballot word is at its quad's first lane;
// every lane of the quad forms the message, the first one writes it.
template <typename T>
__device__ __forceinline__ T tr_tile_quad(const AesQuad &aes, const AesQuad::Keys &kH, const AesQuad::Keys &kL,
                                          const TrArgs<T> &a, TrXchg<T> &x, int p, int e, int wv, const uint8_t *K,
                                          const uint8_t *KC, size_t i, bool in, T xh) {
  uint32_t ra = 0, rb = 0;
  T xp = 0;
  if (in) {
    xp = tr_shifted_input(a, i, xh);
    tr_dcf_bits_quad(aes, kH, kL, a, K, KC, i, xp, &ra, &rb);
  }
  const uint64_t wa = __ballot(ra), wb = __ballot(rb);
  if (lane_id() == 0) {
    x.xa[p][wv] = wa;
    x.xb[p][wv] = wb;
  }
  __syncthreads();
  const uint32_t q0 = lane_id() & ~3u;
  if (in) {
    const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
    const uint32_t bh = a.use_a ? uint32_t((x.xa[0][wv] ^ x.xa[1][wv]) >> q0) & 1u : 0u;
    const uint32_t dh = a.use_b ? uint32_t((x.xb[0][wv] ^ x.xb[1][wv]) >> q0) & 1u : 0u;
    const T msg = tr_out_share(a, p, K, i, xh, xp, hb, bh, dh);
    if ((lane_id() & 3u) == 0) x.xm[p][e] = msg;
  }
  __syncthreads();
  const T y = in ? tr_reveal_sum<T>(a, x.xm[0][e], x.xm[1][e]) : T(0);
  __syncthreads();
  return y;
}

// The tiles of a quad-lane launch: a workgroup of 2 * 4h threads takes tiles of
// h elements, the first 4h threads party 0 (four consecutive lanes per element),
// the last 4h party 1.
template <typename T, bool TWO, bool POOL>
__device__ __forceinline__ void tr_eval_tiles_quad(const TrArgs<T> &a, const TrArgs<T> &a2, const TrPool<T> &q) {
  __shared__ __align__(16) uint32_t lds[AesPerm2::kWords];
  __shared__ TrXchg<T> x;
  AesPerm2::fill(lds);
  const AesPerm2 tab(lds);
  const AesQuad aes(tab);
  const AesQuad::Keys kH = aes.keys(c_rkH), kL = aes.keys(c_rkL);
  const int hq = int(blockDim.x) / 2, h = hq / 4;
  const int p = int(threadIdx.x) >= hq ? 1 : 0;
  const int lt = int(threadIdx.x) - p * hq;  // thread of the party's half
  const int e = lt >> 2, wv = lt >> 6;
  const uint8_t *K = p ? a.k1 : a.k0, *KC = a.k0;
  const size_t stride = size_t(gridDim.x) * size_t(h);
  for (size_t base = size_t(blockIdx.x) * h; base < a.N; base += stride) {
    const size_t i = base + size_t(e);
    const bool in = i < a.N;
    T xin = 0, v0 = 0;
    uint32_t o = 0;
    if (in) {
      if constexpr (POOL) {
        const uint32_t s0 = pool_src(q, uint32_t(i), &o);
        v0 = q.v[s0];
        xin = q.v[s0 + q.C] - v0;
      } else {
        xin = a.xhat[i];
      }
    }
    T y = tr_tile_quad(aes, kH, kL, a, x, p, e, wv, K, KC, i, in, xin);
    if constexpr (TWO) y = tr_tile_quad(aes, kH, kL, a2, x, p, e, wv, K, KC, i, in, y);
    if (p == 0 && in && (lt & 3) == 0) {
      if constexpr (POOL)
        q.vn[o] = v0 + y;
      else
        a.out[i] = y;
    }
  }
  if constexpr (POOL) pool_carry(q);
}

template <typename T, int TAG>
__global__ void k_tr_eval_q(TrArgs<T> a) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles_quad<T, false, false>(a, a, TrPool<T>{});
}
template <typename T, int TAG>
__global__ void k_tr_eval2_q(TrArgs<T> a, TrArgs<T> a2) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles_quad<T, true, false>(a, a2, TrPool<T>{});
}
template <typename T, int TAG>
__global__ void k_tr_eval_pool_q(TrArgs<T> a, TrPool<T> q) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles_quad<T, false, true>(a, a, q);
}

// ---- the last levels of a max-pool tree in one launch (latency-bound lanes) ----
// Levels 0..nlev-1 of the tail, each a gate of one RELU kind over the pairs of
// the level (element i = (b pr + j) C + c, the layout of a level launched
// alone; N, the sign DCF and the G / kappa planes per level, the rest shared).
constexpr int kTailMaxLevels = 8;
template <typename T>
struct TrTail {
  TrArgs<T> a;
  int nlev = 0;
  size_t N[kTailMaxLevels] = {};
  DcfLayout dcf[kTailMaxLevels];
  size_t off_kappa[kTailMaxLevels] = {}, off_g[kTailMaxLevels] = {};
  int B = 0, R0 = 0, C = 0, ncol = 0;  // ncol: columns (b, c) per workgroup
  const T *v = nullptr;                // R0 rows of C words per block b
  T *out = nullptr;                    // one row of C words per block b
};

// A workgroup owns columns g0 .. g0 + ncol - 1 (g = b C + c) for the whole tail:
// their R0 values sit in LDS, and every level evaluates the columns' pairs in
// tiles of h elements with the quad-lane gate (both parties, the exchanges in
// LDS), party 0 writing V[2j] + y into row j of the other LDS buffer (an odd
// level's last row carried).  No level waits for another workgroup, so the
// levels run back to back in one launch.
template <typename T, int TAG>
__global__ void k_tr_eval_pool_tail_q(TrTail<T> t) {
  if (t.a.prio) __builtin_amdgcn_s_setprio(2);
  __shared__ __align__(16) uint32_t lds[AesPerm2::kWords];
  __shared__ TrXchg<T> x;
  extern __shared__ __align__(16) unsigned char tail_lds[];
  AesPerm2::fill(lds);
  const AesPerm2 tab(lds);
  const AesQuad aes(tab);
  const AesQuad::Keys kH = aes.keys(c_rkH), kL = aes.keys(c_rkL);
  const int hq = int(blockDim.x) / 2, h = hq / 4;
  const int p = int(threadIdx.x) >= hq ? 1 : 0;
  const int lt = int(threadIdx.x) - p * hq;
  const int e = lt >> 2, wv = lt >> 6;
  const uint8_t *K = p ? t.a.k1 : t.a.k0, *KC = t.a.k0;
  const int R0 = t.R0, C = t.C;
  const int g0 = int(blockIdx.x) * t.ncol;
  const int nc = min(t.ncol, t.B * C - g0);
  T *vin = reinterpret_cast<T *>(tail_lds), *vout = vin + t.ncol * R0;
  for (int k = int(threadIdx.x); k < nc * R0; k += int(blockDim.x)) {
    const int cc = k / R0, r = k - cc * R0, g = g0 + cc, b = g / C, c = g - b * C;
    vin[k] = t.v[(size_t(b) * R0 + r) * C + c];
  }
  __syncthreads();
  int R = R0;
  for (int l = 0; l < t.nlev; l++) {
    TrArgs<T> a = t.a;
    a.N = t.N[l];
    a.a = t.dcf[l];
    a.off_kappa = t.off_kappa[l];
    a.off_g = t.off_g[l];
    const int pr = R / 2, tot = nc * pr;
    for (int base = 0; base < tot; base += h) {  // uniform over the workgroup
      const int idx = base + e;
      const bool in = idx < tot;
      T v0 = 0, xin = 0;
      size_t i = 0;
      int cc = 0, j = 0;
      if (in) {
        cc = idx / pr;
        j = idx - cc * pr;
        const int g = g0 + cc, b = g / C, c = g - b * C;
        i = (size_t(b) * pr + j) * C + c;
        v0 = vin[cc * R0 + 2 * j];
        xin = vin[cc * R0 + 2 * j + 1] - v0;
      }
      const T y = tr_tile_quad(aes, kH, kL, a, x, p, e, wv, K, KC, i, in, xin);
      if (p == 0 && in && (lt & 3) == 0) vout[cc * R0 + j] = v0 + y;
    }
    if (R & 1)
      for (int k = int(threadIdx.x); k < nc; k += int(blockDim.x)) vout[k * R0 + pr] = vin[k * R0 + R - 1];
    __syncthreads();
    T *tmp = vin;
    vin = vout;
    vout = tmp;
    R = pr + (R & 1);
  }
  for (int k = int(threadIdx.x); k < nc; k += int(blockDim.x)) t.out[g0 + k] = vin[k * R0];
}

template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval(TrArgs<T> a) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles<T, NT, REP, false, false>(a, a, TrPool<T>{});
}

// The max-pool form (TrPool) of k_tr_eval.
template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval_pool(TrArgs<T> a, TrPool<T> q) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles<T, NT, REP, false, true>(a, a, q);
}

// Two gates of one element count in one launch (a truncation and its extension):
// the second gate's masked input is the first's revealed output, element by
// element, so no workgroup waits on another and the intermediate stays in
// registers.  Output in a.out.
template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval2(TrArgs<T> a, TrArgs<T> a2) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_tiles<T, NT, REP, true, false>(a, a2, TrPool<T>{});
}

// Both-party forms: one thread per element for both parties.
template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval_b(TrArgs<T> a) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_both<T, NT, REP, false, false>(a, a, TrPool<T>{});
}
template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval2_b(TrArgs<T> a, TrArgs<T> a2) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  tr_eval_both<T, NT, REP, true, false>(a, a2, TrPool<T>{});
}

// Party mode, phase 1: party p's masked DCF output bits (one ballot word per
// wave and plane).  a.k0 = a.k1 = the party's own key.
template <typename T, int NT, int REP>
__global__ void k_tr_party_bits(TrArgs<T> a, uint64_t *bits) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const size_t W = (a.N + 63) / 64;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t base = size_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u); base < a.N; base += stride) {
    const size_t i = base + lane_id();
    uint32_t ra = 0, rb = 0;
    if (i < a.N) tr_dcf_bits(aes, a, a.k0, a.k0, i, tr_shifted_input(a, i, a.xhat[i]), &ra, &rb);
    const uint64_t wa = __ballot(ra), wb = __ballot(rb);
    if (lane_id() == 0) {
      if (a.use_a) bits[base >> 6] = wa;
      if (a.use_b) bits[W + (base >> 6)] = wb;
    }
  }
}

// Party mode, phase 2: party p's output message from the reconstructed bits
// (own XOR peer); for G_DRELU the public output bit itself.
template <typename T>
__global__ void k_tr_party_msg(TrArgs<T> a, int p, const uint64_t *own, const uint64_t *peer, T *msg) {
  const size_t W = (a.N + 63) / 64;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < a.N; i += size_t(gridDim.x) * blockDim.x) {
    const T xh = a.xhat[i];
    const T xp = tr_shifted_input(a, i, xh);
    const size_t w = i >> 6;
    const uint32_t sh = uint32_t(i & 63u);
    const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
    const uint32_t bh = a.use_a ? uint32_t((own[w] ^ peer[w]) >> sh) & 1u : 0u;
    const uint32_t dh = a.use_b ? uint32_t((own[W + w] ^ peer[W + w]) >> sh) & 1u : 0u;
    msg[i] = a.kind == G_DRELU ? T(hb ^ bh) : tr_out_share(a, p, a.k0, i, xh, xp, hb, bh, dh);
  }
}

template <typename T, int NT, int REP>
__global__ void k_tr_keygen(TrArgs<T> a) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  const int n = a.n, s = a.s;
  const T lowmask = (T(1) << a.sb) - T(1);
  const T smask = (T(1) << s) - T(1);
  const int wsh = a.m - a.sh;  // weight of the wrap bit after the shift
  T *G0 = reinterpret_cast<T *>(a.w0 + a.off_g);
  T *G1 = reinterpret_cast<T *>(a.w1 + a.off_g);
  const int ncase = a.ncase;
  for (size_t base = size_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u); base < a.N; base += stride) {
    const size_t i = base + lane_id();
    uint32_t za0 = 0, za1 = 0, zb0 = 0, zb1 = 0;
    if (i < a.N) {
      const T r = low_bits<T>(a.in_mask[i], a.m);
      const uint32_t rho = uint32_t(r >> a.sb) & 1u;
      const T R = r >> a.sh;
      // each party's output-mask bit of a DCF comes from its own PRF key; the
      // DCF output mask is their XOR
      if (a.use_a) {
        za0 = aes.prf(a.kp[0], a.gate, F_DCFA + 2, i).x & 1u;
        za1 = aes.prf(a.kp[1], a.gate, F_DCFA + 2, i).x & 1u;
      }
      if (a.use_b) {
        zb0 = aes.prf(a.kp[0], a.gate, F_DCFB + 2, i).x & 1u;
        zb1 = aes.prf(a.kp[1], a.gate, F_DCFB + 2, i).x & 1u;
      }
      const uint32_t rbi = za0 ^ za1, rdi = zb0 ^ zb1;
      const T rout = ring_of<T>(aes.prf(a.kd, a.gate, F_ROUT, i));
      const uint32_t kappa = rho ^ rbi;
      a.out_mask[i] = a.kind == G_DRELU ? T(kappa) : rout;  // DRELU: the mask of the output bit
      for (int c = 0; c < ncase; c++) {
        T Gv;
        if (a.kind == G_TRMOD) {
          Gv = rout - R - T(uint32_t(c) ^ rdi);
        } else if (a.kind == G_EXT || a.kind == G_EXTRELU) {
          const uint32_t h = uint32_t(c) >> 1, b = (uint32_t(c) & 1u) ^ rbi;
          const uint32_t w = h ? (rho & b) : (rho | b);
          if (a.kind == G_EXTRELU) {
            const T cc = T(h ^ rho ^ b);
            Gv = rout - cc * R + ((cc * T(w)) << wsh);
          } else {
            Gv = rout - R + (T(w) << wsh);
          }
        } else if (a.kind == G_TR || a.kind == G_TRRELU) {
          const uint32_t h = uint32_t(c) >> 2, bh = (uint32_t(c) >> 1) & 1u, dh = uint32_t(c) & 1u;
          const uint32_t b = bh ^ rbi, d = dh ^ rdi;
          const uint32_t w = h ? (rho & b) : (rho | b);
          if (a.kind == G_TRRELU) {
            const T cc = T(h ^ rho ^ b);
            Gv = rout - cc * R - cc * T(d) + ((cc * T(w)) << (n - s));
          } else {
            Gv = rout - R - T(d) + (T(w) << (n - s));
          }
        } else if (relu_like(a.kind)) {
          const T cc = T(uint32_t(c) ^ kappa);
          Gv = rout - cc * r;
        } else {
          const uint32_t Hh = uint32_t(c) >> 1, dh = uint32_t(c) & 1u;
          const uint32_t d = dh ^ rdi;
          const uint32_t R2 = uint32_t(r >> (n - 2)) & 3u;
          const uint32_t w = Hh < R2 ? 1u : 0u;
          Gv = rout - R - T(d) + (T(w) << (n - s));
        }
        const T g0 = ring_of<T>(aes.prf(a.kp[0], a.gate, F_SPLIT + uint32_t(c), i));
        G0[size_t(c) * a.N + i] = g0;
        G1[size_t(c) * a.N + i] = Gv - g0;
      }
      if (a.relu) {
        const T q0 = ring_of<T>(aes.prf(a.kp[0], a.gate, F_SPLIT + 8, i));
        reinterpret_cast<T *>(a.w0 + a.off_kappa)[i] = q0;
        reinterpret_cast<T *>(a.w1 + a.off_kappa)[i] = T(kappa) - q0;
      }
      if (a.use_a)
        dcf_gen_roots(aes, party_root(aes, a.kp[0], 0, a.gate, F_DCFA, i),
                      party_root(aes, a.kp[1], 1, a.gate, F_DCFA, i), a.a.m, a.a.L, uint64_t(r & lowmask), i, a.N,
                      a.w0, a.w1, a.a.off_root, a.a.off_cw, a.a.off_leaf);
      if (a.use_b)
        dcf_gen_roots(aes, party_root(aes, a.kp[0], 0, a.gate, F_DCFB, i),
                      party_root(aes, a.kp[1], 1, a.gate, F_DCFB, i), a.b.m, a.b.L, uint64_t(r & smask), i, a.N,
                      a.w0, a.w1, a.b.off_root, a.b.off_cw, a.b.off_leaf);
    }
    const uint64_t wa0 = __ballot(za0), wa1 = __ballot(za1), wb0 = __ballot(zb0), wb1 = __ballot(zb1);
    if (lane_id() == 0) {
      if (a.use_a) {
        reinterpret_cast<uint64_t *>(a.w0 + a.a.off_z)[base >> 6] = wa0;
        reinterpret_cast<uint64_t *>(a.w1 + a.a.off_z)[base >> 6] = wa1;
      }
      if (a.use_b) {
        reinterpret_cast<uint64_t *>(a.w0 + a.b.off_z)[base >> 6] = wb0;
        reinterpret_cast<uint64_t *>(a.w1 + a.b.off_z)[base >> 6] = wb1;
      }
    }
  }
}

template <typename T>
static TrArgs<T> tr_args(const TrLayout &lay) {
  TrArgs<T> a{};
  a.kind = lay.kind;
  a.n = lay.bw;
  a.s = lay.s;
  a.sb = tr_sign_bit(lay.kind, lay.bw, lay.s);
  a.m = tr_in_bits(lay.kind, lay.bw, lay.s);
  a.sh = tr_shift(lay.kind, lay.s);
  a.ncase = lay.ncase;
  a.relu = lay.relu;
  a.has_bias = tr_has_bias(lay.kind);
  a.N = lay.N;
  a.a = lay.a;
  a.b = lay.b;
  a.off_kappa = lay.off_kappa;
  a.off_g = lay.off_g;
  a.use_a = lay.use_a;
  a.use_b = lay.use_b;
  a.bias_ncol = 1;
  return a;
}

template <typename T>
hipError_t launch_tr_keygen(const Launch &L, const TrLayout &lay, uint64_t seed, uint32_t gate, const T *in_mask,
                            T *out_mask, uint8_t *k0, uint8_t *k1) {
  if (lay.bw != int(8 * sizeof(T))) return hipErrorInvalidValue;
  TrArgs<T> a = tr_args<T>(lay);
  a.kd = dealer_key(L, seed);
  a.kp[0] = party_key(L, seed, 0);
  a.kp[1] = party_key(L, seed, 1);
  a.gate = gate;
  a.w0 = k0;
  a.w1 = k1;
  a.in_mask = in_mask;
  a.out_mask = out_mask;
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_tr_keygen<T, NT, REP>, block, lay.N, L.num_cu);
    hipLaunchKernelGGL((k_tr_keygen<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, a);
    return hipGetLastError();
  });
}

// Workgroup of a gate evaluation: the context's explicit size, else the
// variant's; a launch of at least 2^22 elements on the default 512-thread
// variant takes 1024 threads (one T-table per 16 waves).  Measured: 3.28
// against 3.11 G DCF evals/s on 2^24 ReLUs, while the model's launches (up to
// 10^6 elements) and the adjacency normalisation's (3.4 * 10^6) lose 6-10% at
// 1024 and keep 512.
// A gate evaluation of fewer elements than this is latency-bound (a few
// thousand wavefronts of one dependent AES chain each) and sits on its lane's
// critical path while other lanes' large gates fill the GPU: its waves take the
// SIMDs' issue slots first.
constexpr size_t kTrPrioN = size_t(1) << 17;
// Threads per workgroup of the one-launch gate kernel (both parties' threads for
// block/2 elements).  A small gate spreads over the CUs: with the variant's block
// its few workgroups put 8 waves on each CU they land on, and a CU's LDS serves
// one 64-lane table read per two clocks, so every AES round of those waves waits
// on one CU's LDS while the other CUs idle; about one workgroup per CU, of at
// least one wave per party, divides the reads among the CUs (Launch::spread_small).
static int tr_eval_block(const Launch &L, size_t n) {
  const int b = variant_block(L);
  if (L.aes_block != 0) return b;
  if (b == 512 && n >= (size_t(1) << 22)) return 1024;
  if (!L.spread_small) return b;
  const size_t per_cu = (n + size_t(L.num_cu) - 1) / size_t(L.num_cu);
  const size_t h = std::max<size_t>(64, (per_cu + 63) / 64 * 64);
  return int(std::min<size_t>(size_t(b), 2 * h));
}

// Quad-lane evaluation: a launch with the default T0/T1 table whose elements fit
// two 256-thread workgroups (32 elements each; both fit a CU's LDS) per CU, so
// that every element's AES rounds run on four lanes (at B = 1: 0.566 ms per
// forward against 0.609 with one workgroup per CU and 0.570 with four).  Large
// lanes take it too: their smallest gates (the last pool levels, two fully
// connected gates) run at the end of a forward, when the lanes' large gates are
// done (bw=64, B=64: +1.2-1.7%; bw=32 unchanged).
// Above 64 elements per CU (up to L.quad_per_cu) the workgroups are of 512
// threads (64 elements): two still fit a CU (LDS 2 x 68 KiB, 96 VGPRs).
constexpr int kQuadBlock = 256, kQuadElems = kQuadBlock / 8;
static bool use_quad(const Launch &L, size_t n) {
  if (L.aes_block != 0) return false;
  int nv;
  const AesVariant *v = aes_variants(&nv);
  const int vi = L.aes_variant >= 0 && L.aes_variant < nv ? L.aes_variant : 0;
  return v[vi].nt == 2 && v[vi].rep == 32 && n <= size_t(L.num_cu) * size_t(std::max(2 * kQuadElems, L.quad_per_cu));
}
static int quad_block(const Launch &L, size_t n) {
  return n <= size_t(L.num_cu) * 2 * kQuadElems ? kQuadBlock : 2 * kQuadBlock;
}
static int quad_grid(const Launch &L, size_t n) {
  const size_t h = size_t(quad_block(L, n) / 8);
  return int(std::max<size_t>(1, (n + h - 1) / h));
}

// The both-party form (one thread per element for both parties, 1024-thread
// workgroups: one per CU at 68 VGPRs, 64 KiB of LDS) for gates of at most
// L.both_aes AES calls per element and party over Z_2^32 (the launcher's only
// instance), in launches of at least L.both_min elements per CU.  Interleaved
// on one box against the one-lane kernel: affinity B = 64 in 3 lanes +4.6%
// (gates up to 14 calls, 1024 elements per CU), in 1 lane -3.8% with gates up
// to 14 calls and unchanged up to 6; adjacency normalisation B = 1024 (6-call
// gates) +10% in 3 groups, +7.5% in one.  In lanes 512 elements per CU gains
// again (B = 64 +1.4%, B = 32 +2.5%; 384 and 256 lose at B = 32).  Also
// measured: every gate launch in this form (B = 64 -0.6%), 512, 768 and 896
// threads, bw = 64 (2-3% slower), the 25-call RELU of 2^24 elements alone (6%
// slower).  A truncation pair in this form (k_tr_eval2_b, lanes of at most 8
// samples): B = 16 +4%, B = 24 +2%; a max-pool level in this form measured no
// gain.
template <typename T>
static int both_block(const Launch &L, const TrArgs<T> &a) {
  const int aes = (a.use_a ? a.a.L + 1 : 0) + (a.use_b ? a.b.L + 1 : 0);
  if (L.aes_block != 0 || aes > L.both_aes) return 0;
  return a.N >= size_t(L.num_cu) * size_t(L.both_min) ? 1024 : 0;
}

// The kernel form of a gate evaluation outside the max-pool form: the
// quad-lane form, the both-party form, or the one-lane kernel.
template <typename T>
static int tr_form(const Launch &L, const TrArgs<T> &a) {
  if (use_quad(L, a.N)) return kFormQuad;
  if constexpr (sizeof(T) == 4)
    if (both_block(L, a)) return kFormBoth;
  return kFormOneLane;
}
int tr_eval_form(const Launch &L, const TrLayout &lay) {
  return lay.bw == 32 ? tr_form<uint32_t>(L, tr_args<uint32_t>(lay)) : tr_form<uint64_t>(L, tr_args<uint64_t>(lay));
}

// One gate evaluation of both parties with prepared arguments: the regular
// kernels, or (q set) their max-pool form.
template <typename T>
static hipError_t tr_eval_launch(const Launch &L, const TrArgs<T> &a, const TrPool<T> *q) {
  if (tr_form(L, a) == kFormQuad) {
    const dim3 grid(quad_grid(L, a.N)), block(quad_block(L, a.N));
    if (q && L.profiled)
      hipLaunchKernelGGL((k_tr_eval_pool_q<T, 1>), grid, block, 0, L.stream, a, *q);
    else if (q)
      hipLaunchKernelGGL((k_tr_eval_pool_q<T, 0>), grid, block, 0, L.stream, a, *q);
    else if (L.profiled)
      hipLaunchKernelGGL((k_tr_eval_q<T, 1>), grid, block, 0, L.stream, a);
    else
      hipLaunchKernelGGL((k_tr_eval_q<T, 0>), grid, block, 0, L.stream, a);
    return hipGetLastError();
  }
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    if constexpr (sizeof(T) == 4) {
      const int block = !q && tr_form(L, a) == kFormBoth ? both_block(L, a) : 0;
      if (block) {
        const int grid = grid_for(k_tr_eval_b<T, NT, REP, 0>, block, a.N, L.num_cu);
        if (L.profiled)
          hipLaunchKernelGGL((k_tr_eval_b<T, NT, REP, 1>), dim3(grid), dim3(block), 0, L.stream, a);
        else
          hipLaunchKernelGGL((k_tr_eval_b<T, NT, REP, 0>), dim3(grid), dim3(block), 0, L.stream, a);
        return hipGetLastError();
      }
    }
    const int block = tr_eval_block(L, a.N);
    // a workgroup holds both parties' threads for block/2 elements
    if (block < 128 || block > 2 * kTrMaxTile || block % 128 != 0) return hipErrorInvalidConfiguration;
    const int grid = grid_for(k_tr_eval<T, NT, REP, 0>, block, 2 * a.N, L.num_cu);
    if (q && L.profiled)
      hipLaunchKernelGGL((k_tr_eval_pool<T, NT, REP, 1>), dim3(grid), dim3(block), 0, L.stream, a, *q);
    else if (q)
      hipLaunchKernelGGL((k_tr_eval_pool<T, NT, REP, 0>), dim3(grid), dim3(block), 0, L.stream, a, *q);
    else if (L.profiled)
      hipLaunchKernelGGL((k_tr_eval<T, NT, REP, 1>), dim3(grid), dim3(block), 0, L.stream, a);
    else
      hipLaunchKernelGGL((k_tr_eval<T, NT, REP, 0>), dim3(grid), dim3(block), 0, L.stream, a);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t launch_tr_eval(const Launch &L, const TrLayout &lay, const uint8_t *k0, const uint8_t *k1, const T *xhat,
                          const T *bias, int bias_ncol, T *out) {
  if (lay.bw != int(8 * sizeof(T))) return hipErrorInvalidValue;
  TrArgs<T> a = tr_args<T>(lay);
  a.k0 = k0;
  a.k1 = k1;
  a.xhat = xhat;
  a.bias = bias;
  a.bias_ncol = bias_ncol > 0 ? bias_ncol : 1;
  a.out = out;
  a.prio = lay.N < kTrPrioN;
  return tr_eval_launch<T>(L, a, nullptr);
}

template <typename T>
hipError_t launch_tr_eval_pool(const Launch &L, const TrLayout &lay, const uint8_t *k0, const uint8_t *k1, int B,
                               int R, int C, const T *V, T *Vn) {
  if (lay.bw != int(8 * sizeof(T)) || B < 1 || R < 2 || C < 1 || lay.N != size_t(B) * (R / 2) * C ||
      size_t(B) * R * C >= (size_t(1) << 32))
    return hipErrorInvalidValue;
  TrArgs<T> a = tr_args<T>(lay);
  a.k0 = k0;
  a.k1 = k1;
  a.bias_ncol = 1;
  a.prio = lay.N < kTrPrioN;
  TrPool<T> q;
  q.B = uint32_t(B);
  q.R = uint32_t(R);
  q.C = uint32_t(C);
  q.pr = uint32_t(R / 2);
  q.v = V;
  q.vn = Vn;
  return tr_eval_launch<T>(L, a, &q);
}

template <typename T>
hipError_t launch_tr_eval_pool_tail(const Launch &L, const TrLayout *lay, int nlev, const uint8_t *k0,
                                   const uint8_t *k1, int B, int R0, int C, const T *V, T *out) {
  if (nlev < 1 || nlev > kTailMaxLevels || B < 1 || R0 < 2 || C < 1 || size_t(B) * R0 * C >= (size_t(1) << 31))
    return hipErrorInvalidValue;
  TrTail<T> t;
  t.a = tr_args<T>(lay[0]);
  t.a.k0 = k0;
  t.a.k1 = k1;
  t.a.bias_ncol = 1;
  t.a.prio = 1;
  int R = R0;
  for (int l = 0; l < nlev; l++) {  // one RELU kind, sign DCF only, the pairs of level l
    const TrLayout &y = lay[l];
    if (y.bw != int(8 * sizeof(T)) || y.kind != lay[0].kind || y.s != lay[0].s || !y.use_a || y.use_b ||
        !tr_is_relu(y.kind) || R < 2 || y.N != size_t(B) * (R / 2) * C)
      return hipErrorInvalidValue;
    t.N[l] = y.N;
    t.dcf[l] = y.a;
    t.off_kappa[l] = y.off_kappa;
    t.off_g[l] = y.off_g;
    R = R / 2 + (R & 1);
  }
  if (R != 1) return hipErrorInvalidValue;  // the tail ends with one row
  t.nlev = nlev;
  t.B = B;
  t.R0 = R0;
  t.C = C;
  t.v = V;
  t.out = out;
  // about one workgroup per CU; per workgroup h elements per tile (a multiple
  // of 16, so that each party's 4h threads are whole waves)
  const int cols = B * C;
  t.ncol = std::max(1, (cols + L.num_cu - 1) / L.num_cu);
  const int grid = (cols + t.ncol - 1) / t.ncol;
  const int h = std::min(64, std::max(16, (t.ncol * (R0 / 2) + 15) / 16 * 16));
  const size_t shm = 2 * size_t(t.ncol) * size_t(R0) * sizeof(T);
  if (shm > (size_t(64) << 10)) return hipErrorInvalidValue;  // beside the 64 KiB table and the exchange buffers
  if (L.profiled)
    hipLaunchKernelGGL((k_tr_eval_pool_tail_q<T, 1>), dim3(grid), dim3(8 * h), shm, L.stream, t);
  else
    hipLaunchKernelGGL((k_tr_eval_pool_tail_q<T, 0>), dim3(grid), dim3(8 * h), shm, L.stream, t);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_tr_eval2(const Launch &L, const TrLayout &lay, const TrLayout &lay2, const uint8_t *k0,
                           const uint8_t *k1, const T *xhat, const T *bias, int bias_ncol, T *out) {
  if (lay.bw != int(8 * sizeof(T)) || lay2.bw != lay.bw || lay2.N != lay.N) return hipErrorInvalidValue;
  TrArgs<T> a = tr_args<T>(lay), a2 = tr_args<T>(lay2);
  a.k0 = a2.k0 = k0;
  a.k1 = a2.k1 = k1;
  a.xhat = xhat;
  a.bias = bias;
  a.bias_ncol = bias_ncol > 0 ? bias_ncol : 1;
  a.out = out;
  a.prio = lay.N < kTrPrioN;
  if (use_quad(L, lay.N)) {
    if (L.profiled)
      hipLaunchKernelGGL((k_tr_eval2_q<T, 1>), dim3(quad_grid(L, lay.N)), dim3(quad_block(L, lay.N)), 0, L.stream, a,
                         a2);
    else
      hipLaunchKernelGGL((k_tr_eval2_q<T, 0>), dim3(quad_grid(L, lay.N)), dim3(quad_block(L, lay.N)), 0, L.stream, a,
                         a2);
    return hipGetLastError();
  }
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    if constexpr (sizeof(T) == 4) {
      const int bb = both_block(L, a) ? both_block(L, a2) : 0;
      if (bb) {
        const int grid = grid_for(k_tr_eval2_b<T, NT, REP, 0>, bb, lay.N, L.num_cu);
        if (L.profiled)
          hipLaunchKernelGGL((k_tr_eval2_b<T, NT, REP, 1>), dim3(grid), dim3(bb), 0, L.stream, a, a2);
        else
          hipLaunchKernelGGL((k_tr_eval2_b<T, NT, REP, 0>), dim3(grid), dim3(bb), 0, L.stream, a, a2);
        return hipGetLastError();
      }
    }
    const int block = tr_eval_block(L, lay.N);
    if (block < 128 || block > 2 * kTrMaxTile || block % 128 != 0) return hipErrorInvalidConfiguration;
    const int grid = grid_for(k_tr_eval2<T, NT, REP, 0>, block, 2 * lay.N, L.num_cu);
    if (L.profiled)
      hipLaunchKernelGGL((k_tr_eval2<T, NT, REP, 1>), dim3(grid), dim3(block), 0, L.stream, a, a2);
    else
      hipLaunchKernelGGL((k_tr_eval2<T, NT, REP, 0>), dim3(grid), dim3(block), 0, L.stream, a, a2);
    return hipGetLastError();
  });
}

template <typename T>
static TrArgs<T> tr_party_args(const TrLayout &lay, const uint8_t *key, const T *xhat, const T *bias,
                               int bias_ncol) {
  TrArgs<T> a = tr_args<T>(lay);
  a.k0 = key;  // the party's own key in both slots
  a.k1 = key;
  a.xhat = xhat;
  a.bias = bias;
  a.bias_ncol = bias_ncol > 0 ? bias_ncol : 1;
  return a;
}

template <typename T>
hipError_t launch_tr_party_bits(const Launch &L, const TrLayout &lay, const uint8_t *key, const T *xhat,
                                const T *bias, int bias_ncol, uint64_t *bits) {
  if (lay.bw != int(8 * sizeof(T)) || L.party < 0) return hipErrorInvalidValue;
  if (lay.N == 0) return hipSuccess;
  const TrArgs<T> a = tr_party_args<T>(lay, key, xhat, bias, bias_ncol);
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    const int block = variant_block(L);
    const int grid = grid_for(k_tr_party_bits<T, NT, REP>, block, lay.N, L.num_cu);
    hipLaunchKernelGGL((k_tr_party_bits<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, a, bits);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t launch_tr_party_msg(const Launch &L, const TrLayout &lay, const uint8_t *key, const T *xhat,
                               const T *bias, int bias_ncol, const uint64_t *own, const uint64_t *peer, T *msg) {
  if (lay.bw != int(8 * sizeof(T)) || L.party < 0) return hipErrorInvalidValue;
  if (lay.N == 0) return hipSuccess;
  const TrArgs<T> a = tr_party_args<T>(lay, key, xhat, bias, bias_ncol);
  const int block = 256;
  const int grid = grid_for(k_tr_party_msg<T>, block, lay.N, L.num_cu);
  hipLaunchKernelGGL((k_tr_party_msg<T>), dim3(grid), dim3(block), 0, L.stream, a, L.party, own, peer, msg);
  return hipGetLastError();
}

template <typename T, int NT, int REP>
__global__ void k_tr_expand(TrArgs<T> a, int p) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const AesRK &kp = a.kp[0];
  uint8_t *w = a.w0;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  const int ncase = a.ncase;
  const bool kappa = a.relu;
  for (size_t base = size_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u); base < a.N; base += stride) {
    const size_t i = base + lane_id();
    uint32_t za = 0, zb = 0;
    if (i < a.N) {
      if (a.use_a) {
        reinterpret_cast<uint4 *>(w + a.a.off_root)[i] = party_root(aes, kp, p, a.gate, F_DCFA, i);
        za = aes.prf(kp, a.gate, F_DCFA + 2, i).x & 1u;
      }
      if (a.use_b) {
        reinterpret_cast<uint4 *>(w + a.b.off_root)[i] = party_root(aes, kp, p, a.gate, F_DCFB, i);
        zb = aes.prf(kp, a.gate, F_DCFB + 2, i).x & 1u;
      }
      if (p == 0) {
        T *G0 = reinterpret_cast<T *>(w + a.off_g);
        for (int c = 0; c < ncase; c++)
          G0[size_t(c) * a.N + i] = ring_of<T>(aes.prf(kp, a.gate, F_SPLIT + uint32_t(c), i));
        if (kappa) reinterpret_cast<T *>(w + a.off_kappa)[i] = ring_of<T>(aes.prf(kp, a.gate, F_SPLIT + 8, i));
      }
    }
    const uint64_t wa = __ballot(za), wb = __ballot(zb);
    if (lane_id() == 0) {
      if (a.use_a) reinterpret_cast<uint64_t *>(w + a.a.off_z)[base >> 6] = wa;
      if (a.use_b) reinterpret_cast<uint64_t *>(w + a.b.off_z)[base >> 6] = wb;
    }
  }
}

template <typename T>
hipError_t launch_tr_expand(const Launch &L, const TrLayout &lay, const uint8_t party_key16[16], uint32_t gate,
                            int party, uint8_t *key) {
  if (lay.bw != int(8 * sizeof(T)) || (party != 0 && party != 1)) return hipErrorInvalidValue;
  if (lay.N == 0 || lay.kind == G_LOCALARS) return hipSuccess;
  TrArgs<T> a = tr_args<T>(lay);
  a.kp[0] = aes_expand(party_key16);
  a.gate = gate;
  a.w0 = key;
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_tr_expand<T, NT, REP>, block, lay.N, L.num_cu);
    hipLaunchKernelGGL((k_tr_expand<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, a, party);
    return hipGetLastError();
  });
}


#define INST(T)                                                                                                       \
  template hipError_t launch_tr_keygen<T>(const Launch &, const TrLayout &, uint64_t, uint32_t, const T *, T *,       \
                                          uint8_t *, uint8_t *);                                                      \
  template hipError_t launch_tr_expand<T>(const Launch &, const TrLayout &, const uint8_t *, uint32_t, int,           \
                                          uint8_t *);                                                                 \
  template hipError_t launch_tr_eval<T>(const Launch &, const TrLayout &, const uint8_t *, const uint8_t *,           \
                                        const T *, const T *, int, T *);                                              \
  template hipError_t launch_tr_eval_pool<T>(const Launch &, const TrLayout &, const uint8_t *, const uint8_t *, int, \
                                             int, int, const T *, T *);                                               \
  template hipError_t launch_tr_eval_pool_tail<T>(const Launch &, const TrLayout *, int, const uint8_t *,           \
                                                  const uint8_t *, int, int, int, const T *, T *);                    \
  template hipError_t launch_tr_eval2<T>(const Launch &, const TrLayout &, const TrLayout &, const uint8_t *,         \
                                         const uint8_t *, const T *, const T *, int, T *);                            \
  template hipError_t launch_tr_party_bits<T>(const Launch &, const TrLayout &, const uint8_t *, const T *,           \
                                              const T *, int, uint64_t *);                                            \
  template hipError_t launch_tr_party_msg<T>(const Launch &, const TrLayout &, const uint8_t *, const T *,            \
                                             const T *, int, const uint64_t *, const uint64_t *, T *);

INST(uint32_t)
INST(uint64_t)

}  // namespace mpcx
