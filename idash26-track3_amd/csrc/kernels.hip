// kernels.hip -- HIP kernels of the secure-inference online path for gfx950.
//
// Reference interfaces these kernels stand behind (EzPC GPU-MPC, called from the
// reference's backend; signatures reconstructed from the call sites):
//   DCF eval / keygen ........ gpuDcf / gpuKeyGenDCF    (gpu_mpc/dpf_dcf_adapter.h:266,372)
//   ReLU ..................... gpuRelu / gpuGenReluKey   (gpu_mpc/ddg_orca.h:103-104,233)
//   exact truncation ......... gpuTruncate / genGPUTruncateKey (gpu_mpc/ddg_orca.h:116-118,240)
//   Beaver product ........... gpuMul / gpuKeygenMul    (gpu_mpc/secure_adj_norm.h:611-651,326-365)
//   8-bit DPF LUT ............ gpuDpfLUT / gpuKeyGenLUT (gpu_mpc/secure_adj_norm.h:510-520,270-279)
//   ring GEMM ................ gpuMatmul / gpuKeygenMatmul (gpu_mpc/ddg_orca_base.h:170-271,394-469)
//   reveal ................... reconstructInPlace       (gpu_mpc/utils/gpu_comms.h:290-302)
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

namespace mpcx {

// ---------------------------------------------------------------------------
// AES LDS variants
// ---------------------------------------------------------------------------
// 0 (default): T0 and T1 interleaved, 32 copies each (AesPerm2); 1, 2: T0 alone,
// 64 copies (AesPerm); 3: four tables, 32 copies, shift/mask addressing.
static const AesVariant kVariants[] = {
    {2, 32, 512, "perm32x2_b512"},
    {0, 64, 512, "perm64_b512"},
    {0, 64, 1024, "perm64_b1024"},
    {4, 32, 1024, "t4_rep32_b1024"},
};
const AesVariant *aes_variants(int *count) {
  *count = int(sizeof(kVariants) / sizeof(kVariants[0]));
  return kVariants;
}

template <int NT, int REP>
struct V {
  static constexpr int nt = NT, rep = REP;
};

template <class Fn>
static hipError_t with_variant(const Launch &L, Fn &&fn) {
  switch (L.aes_variant) {
    case 0: return fn(V<2, 32>{});
    case 1: return fn(V<0, 64>{});
    case 2: return fn(V<0, 64>{});
    case 3: return fn(V<4, 32>{});
    default: return hipErrorInvalidValue;
  }
}
// Rows of workgroups of a two-party kernel (blockIdx.y + party_base = party):
// both parties, or only L.party in party mode.
static unsigned party_rows(const Launch &L) { return L.party < 0 ? 2u : 1u; }
static int party_base(const Launch &L) { return L.party < 0 ? 0 : L.party; }
static int variant_block(const Launch &L) {
  if (L.aes_block > 0) return L.aes_block;
  int n;
  const AesVariant *v = aes_variants(&n);
  return (L.aes_variant >= 0 && L.aes_variant < n) ? v[L.aes_variant].block : 256;
}

template <typename K>
static int grid_for(K kernel, int block, size_t n, int num_cu) {
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, block, 0) != hipSuccess || occ < 1) occ = 1;
  size_t need = (n + block - 1) / block;
  size_t cap = size_t(occ) * size_t(num_cu);
  size_t g = need < cap ? need : cap;
  return int(g < 1 ? 1 : g);
}


__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

template <typename T>
__device__ __forceinline__ T ring_of(uint4 b) {
  if constexpr (sizeof(T) == 4)
    return T(b.x);
  else
    return T(uint64_t(b.x) | (uint64_t(b.y) << 32));
}

__device__ __forceinline__ uint32_t get_bit(const uint64_t *plane, size_t i) {
  return uint32_t(plane[i >> 6] >> (i & 63)) & 1u;
}

// ---------------------------------------------------------------------------
// PRG probes
// ---------------------------------------------------------------------------
template <int NT, int REP>
__global__ void k_hash(int leaf, size_t n, const uint4 *in, uint4 *out) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    out[i] = leaf ? aes.hash(in[i], c_rkL) : aes.hash(in[i], c_rkH);
}

hipError_t launch_hash(const Launch &L, int leaf, size_t n, const uint4 *in, uint4 *out) {
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_hash<NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_hash<NT, REP>), dim3(grid), dim3(block), 0, L.stream, leaf, n, in, out);
    return hipGetLastError();
  });
}

template <int NT, int REP>
__global__ void k_prf(AesRK kd, uint32_t gate, uint32_t field, size_t n, uint4 *out) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    out[i] = aes.prf(kd, gate, field, i);
}

hipError_t launch_prf(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, uint4 *out) {
  const AesRK kd = dealer_key(L, seed);
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_prf<NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_prf<NT, REP>), dim3(grid), dim3(block), 0, L.stream, kd, gate, field, n, out);
    return hipGetLastError();
  });
}

// ---------------------------------------------------------------------------
// standalone DCF (gpuKeyGenDCF / gpuDcf)
// ---------------------------------------------------------------------------
struct DcfGenArgs {
  AesRK kd;
  uint32_t gate, fb;
  int m, L;
  size_t n;
  const uint64_t *alpha;
  const uint8_t *rbit;
  uint8_t *k0, *k1;
  size_t off_root, off_cw, off_leaf, off_z;
};

template <int NT, int REP>
__global__ void k_dcf_keygen(DcfGenArgs a) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t base = size_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u); base < a.n; base += stride) {
    const size_t i = base + lane_id();
    uint32_t z0 = 0, z1 = 0;
    if (i < a.n) {
      dcf_gen_walk(aes, a.kd, a.gate, a.fb, a.m, a.L, a.alpha[i], i, a.n, a.k0, a.k1, a.off_root,
                   a.off_cw, a.off_leaf);
      z0 = aes.prf(a.kd, a.gate, a.fb + 2, i).x & 1u;
      z1 = z0 ^ (a.rbit ? (a.rbit[i] & 1u) : 0u);
    }
    const uint64_t w0 = __ballot(z0), w1 = __ballot(z1);
    if (lane_id() == 0) {
      reinterpret_cast<uint64_t *>(a.k0 + a.off_z)[base >> 6] = w0;
      reinterpret_cast<uint64_t *>(a.k1 + a.off_z)[base >> 6] = w1;
    }
  }
}

hipError_t launch_dcf_keygen(const Launch &L, uint64_t seed, uint32_t gate, uint32_t fbase, int m, size_t n,
                             const uint64_t *alpha, const uint8_t *rbit, uint8_t *k0, uint8_t *k1, size_t base) {
  DcfLayout lay = dcf_layout(m, n, base, true);
  DcfGenArgs a;
  a.kd = dealer_key(L, seed);
  a.gate = gate;
  a.fb = fbase;
  a.m = m;
  a.L = lay.L;
  a.n = n;
  a.alpha = alpha;
  a.rbit = rbit;
  a.k0 = k0;
  a.k1 = k1;
  a.off_root = lay.off_root;
  a.off_cw = lay.off_cw;
  a.off_leaf = lay.off_leaf;
  a.off_z = lay.off_z;
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_dcf_keygen<NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_dcf_keygen<NT, REP>), dim3(grid), dim3(block), 0, L.stream, a);
    return hipGetLastError();
  });
}

struct DcfEvalArgs {
  int m, L;
  size_t n;
  const uint8_t *key;
  size_t off_root, off_cw, off_leaf, off_z;
  const uint64_t *x;
  uint64_t *out;
};

template <int NT, int REP>
__global__ void k_dcf_eval(DcfEvalArgs a) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  const uint4 *root = reinterpret_cast<const uint4 *>(a.key + a.off_root);
  const uint4 *cw = reinterpret_cast<const uint4 *>(a.key + a.off_cw);
  const uint4 *leaf = reinterpret_cast<const uint4 *>(a.key + a.off_leaf);
  const uint64_t *zp = reinterpret_cast<const uint64_t *>(a.key + a.off_z);
  for (size_t base = size_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u); base < a.n; base += stride) {
    const size_t i = base + lane_id();
    uint32_t b = 0;
    if (i < a.n) {
      b = dcf_eval_walk(aes, root[i], a.m, a.L, cw + i, a.n, leaf[i], a.x[i]);
      b ^= get_bit(zp, i);
    }
    const uint64_t w = __ballot(b);
    if (lane_id() == 0) a.out[base >> 6] = w;
  }
}

hipError_t launch_dcf_eval(const Launch &L, int party, int m, size_t n, const uint8_t *key, size_t base,
                           const uint64_t *x, uint64_t *out_bits) {
  (void)party;
  DcfLayout lay = dcf_layout(m, n, base, true);
  DcfEvalArgs a;
  a.m = m;
  a.L = lay.L;
  a.n = n;
  a.key = key;
  a.off_root = lay.off_root;
  a.off_cw = lay.off_cw;
  a.off_leaf = lay.off_leaf;
  a.off_z = lay.off_z;
  a.x = x;
  a.out = out_bits;
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_dcf_eval<NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_dcf_eval<NT, REP>), dim3(grid), dim3(block), 0, L.stream, a);
    return hipGetLastError();
  });
}

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

__device__ __forceinline__ bool relu_like(int kind) {
  return kind == G_RELU || kind == G_RELUSLACK || kind == G_RELUPOOL;
}

// v mod 2^m for 1 <= m <= bits of T
template <typename T>
__device__ __forceinline__ T low_bits(T v, int m) {
  return m >= int(8 * sizeof(T)) ? v : T(v & ((T(1) << m) - T(1)));
}

template <typename T>
__device__ __forceinline__ T tr_shifted_input(const TrArgs<T> &a, size_t i) {
  T x = a.xhat[i];
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
__device__ __forceinline__ T tr_out_share(const TrArgs<T> &a, int p, const uint8_t *K, size_t i, T xp, uint32_t hb,
                                          uint32_t bh, uint32_t dh) {
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
    return cp * a.xhat[i] + G[size_t(z) * a.N + i];
  }
  // G_TRSLACK
  const uint32_t Hh = uint32_t(xp >> (a.n - 2)) & 3u;
  return one0 * A + G[size_t(Hh * 2 + dh) * a.N + i];
}

// One launch evaluates a gate for both parties.  A workgroup of 2h threads
// takes tiles of h elements: its first h threads are party 0, the last h party
// 1, each evaluating its own keys on the same elements.  The two exchanges of
// the protocol go through LDS: the masked DCF output bits (one ballot word per
// wave and DCF), then the output messages, which party 0's threads add into the
// revealed output.  TAG = 1 marks the launches of a profiled forward (identical
// code, its own name in kernel traces).
constexpr int kTrMaxTile = 512;  // elements per tile (workgroups of up to 1024 threads)

template <typename T, int NT, int REP, int TAG>
__global__ void k_tr_eval(TrArgs<T> a) {
  if (a.prio) __builtin_amdgcn_s_setprio(2);
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  __shared__ uint64_t xa[2][kTrMaxTile / 64], xb[2][kTrMaxTile / 64];
  __shared__ T xm[2][kTrMaxTile];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const int h = int(blockDim.x) / 2;
  const int p = int(threadIdx.x) >= h ? 1 : 0;
  const int e = int(threadIdx.x) - p * h;  // element of the tile
  const int wv = e >> 6;                   // wave of the party's half
  const uint8_t *K = p ? a.k1 : a.k0;
  // The correction words and leaf words of a DCF key are the same for both
  // parties (public to both); both parties read party 0's planes, so one copy
  // serves the two evaluations (and a streamed arena moves it once).
  const uint8_t *KC = a.k0;
  const size_t stride = size_t(gridDim.x) * size_t(h);
  for (size_t base = size_t(blockIdx.x) * h; base < a.N; base += stride) {
    const size_t i = base + size_t(e);
    const bool in = i < a.N;
    uint32_t ra = 0, rb = 0;
    T xp = 0;
    if (in) {
      xp = tr_shifted_input(a, i);
      tr_dcf_bits(aes, a, K, KC, i, xp, &ra, &rb);
    }
    // exchange 1: the masked DCF output bits
    const uint64_t wa = __ballot(ra), wb = __ballot(rb);
    if (lane_id() == 0) {
      xa[p][wv] = wa;
      xb[p][wv] = wb;
    }
    __syncthreads();
    if (in) {
      const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
      const uint32_t bh = a.use_a ? uint32_t((xa[0][wv] ^ xa[1][wv]) >> lane_id()) & 1u : 0u;
      const uint32_t dh = a.use_b ? uint32_t((xb[0][wv] ^ xb[1][wv]) >> lane_id()) & 1u : 0u;
      xm[p][e] = tr_out_share(a, p, K, i, xp, hb, bh, dh);  // exchange 2: the output messages
    }
    __syncthreads();
    if (p == 0 && in) a.out[i] = xm[0][e] + xm[1][e];
    __syncthreads();  // the next tile reuses the exchange buffers
  }
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
    if (i < a.N) tr_dcf_bits(aes, a, a.k0, a.k0, i, tr_shifted_input(a, i), &ra, &rb);
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
    const T xp = tr_shifted_input(a, i);
    const size_t w = i >> 6;
    const uint32_t sh = uint32_t(i & 63u);
    const uint32_t hb = uint32_t(xp >> a.sb) & 1u;
    const uint32_t bh = a.use_a ? uint32_t((own[w] ^ peer[w]) >> sh) & 1u : 0u;
    const uint32_t dh = a.use_b ? uint32_t((own[W + w] ^ peer[W + w]) >> sh) & 1u : 0u;
    msg[i] = a.kind == G_DRELU ? T(hb ^ bh) : tr_out_share(a, p, a.k0, i, xp, hb, bh, dh);
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
static int tr_eval_block(const Launch &L, size_t n) {
  const int b = variant_block(L);
  return (L.aes_block == 0 && b == 512 && n >= (size_t(1) << 22)) ? 1024 : b;
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
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    const int block = tr_eval_block(L, lay.N);
    // a workgroup holds both parties' threads for block/2 elements
    if (block < 128 || block > 2 * kTrMaxTile || block % 128 != 0) return hipErrorInvalidConfiguration;
    const int grid = grid_for(k_tr_eval<T, NT, REP, 0>, block, 2 * lay.N, L.num_cu);
    if (L.profiled)
      hipLaunchKernelGGL((k_tr_eval<T, NT, REP, 1>), dim3(grid), dim3(block), 0, L.stream, a);
    else
      hipLaunchKernelGGL((k_tr_eval<T, NT, REP, 0>), dim3(grid), dim3(block), 0, L.stream, a);
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

// ---------------------------------------------------------------------------
// reconstruct / reveal
// ---------------------------------------------------------------------------
template <typename T>
__global__ void k_reconstruct(size_t n, const T *m0, const T *m1, T *out) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    out[i] = m0[i] + m1[i];
}
template <typename T>
hipError_t launch_reconstruct(const Launch &L, size_t n, const T *m0, const T *m1, T *out) {
  const int block = 256;
  int grid = grid_for(k_reconstruct<T>, block, n, L.num_cu);
  hipLaunchKernelGGL((k_reconstruct<T>), dim3(grid), dim3(block), 0, L.stream, n, m0, m1, out);
  return hipGetLastError();
}

// LocalARS (TruncateType::LocalARS, gpu_mpc/ddg_orca_batched.h:180-199): the
// masked value and (at keygen) its mask are shifted locally, no key, no exchange.
template <typename T>
__global__ void k_local_ars(size_t n, int s, const T *x, const T *bias, uint32_t ncol, T *y) {
  using S = std::make_signed_t<T>;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    T v = T(S(x[i]) >> s);
    if (bias) v += bias[uint32_t(i % ncol)];
    y[i] = v;
  }
}
template <typename T>
hipError_t launch_local_ars(const Launch &L, size_t n, int s, const T *x, const T *bias, int ncol, T *y) {
  if (n == 0) return hipSuccess;
  if (bias && ncol < 1) return hipErrorInvalidValue;
  const int block = 256;
  int grid = grid_for(k_local_ars<T>, block, n, L.num_cu);
  hipLaunchKernelGGL((k_local_ars<T>), dim3(grid), dim3(block), 0, L.stream, n, s, x, bias,
                     uint32_t(bias ? ncol : 1), y);
  return hipGetLastError();
}

template <typename T, int NT, int REP>
__global__ void k_split(AesRK kd, uint32_t gate, uint32_t field, size_t n, const T *v, T *p0, T *p1, T *copy0,
                        T *mask_out) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    T val;
    if (v) {
      val = v[i];
    } else {  // fresh reveal mask
      val = ring_of<T>(aes.prf(kd, gate, F_RIN, i));
      mask_out[i] = val;
    }
    const T s0 = ring_of<T>(aes.prf(kd, gate, field, i));
    p0[i] = s0;
    p1[i] = val - s0;
    if (copy0) copy0[i] = s0;
  }
}

template <typename T>
static hipError_t split_impl(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, const T *v,
                             T *p0, T *p1, T *copy0, T *mask_out) {
  const AesRK kd = dealer_key(L, seed);
  return with_variant(L, [&](auto vv) {
    constexpr int NT = decltype(vv)::nt, REP = decltype(vv)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_split<T, NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_split<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, kd, gate, field, n, v, p0, p1,
                       copy0, mask_out);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t launch_split(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, const T *v, T *p0,
                        T *p1, T *share0_copy) {
  return split_impl<T>(L, seed, gate, field, n, v, p0, p1, share0_copy, nullptr);
}

template <typename T>
hipError_t launch_reveal_keygen(const Launch &L, const RevealLayout &lay, uint64_t seed, uint32_t gate, T *mask,
                                uint8_t *k0, uint8_t *k1) {
  return split_impl<T>(L, seed, gate, F_SPLIT + 0, lay.N, nullptr, reinterpret_cast<T *>(k0 + lay.off_r),
                       reinterpret_cast<T *>(k1 + lay.off_r), nullptr, mask);
}

template <typename T>
__global__ void k_reveal_eval(size_t n, const T *R0, const T *R1, const T *v0, const T *v1, int rowlen, T *msg0,
                              T *msg1, int pbase) {
  const int p = int(blockIdx.y) + pbase;
  const T *R = p ? R1 : R0;
  const T *v = p ? v1 : v0;
  T *msg = p ? msg1 : msg0;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    T x;
    if (rowlen > 0) {
      x = 0;
      const T *row = v + i * size_t(rowlen);
      for (int j = 0; j < rowlen; j++) x += row[j];
    } else {
      x = v[i];
    }
    msg[i] = x + R[i];
  }
}

// Row-sum reveal: one wavefront per row of rowlen contiguous elements, lanes
// read the row coalesced and reduce across the wave (sums mod 2^bw do not
// depend on the order).
template <typename T>
__global__ void k_reveal_rowsum(size_t n, const T *R0, const T *R1, const T *v0, const T *v1, int rowlen, T *msg0,
                                T *msg1, int pbase) {
  const int p = int(blockIdx.y) + pbase;
  const T *R = p ? R1 : R0;
  const T *v = p ? v1 : v0;
  T *msg = p ? msg1 : msg0;
  const int lane = int(threadIdx.x & 63u);
  const size_t wave = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const size_t nwaves = (size_t(gridDim.x) * blockDim.x) >> 6;
  for (size_t r = wave; r < n; r += nwaves) {  // uniform across the wave
    const T *row = v + r * size_t(rowlen);
    T x = 0;
    for (int j = lane; j < rowlen; j += 64) x += row[j];
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    if (lane == 0) msg[r] = x + R[r];
  }
}

template <typename T>
hipError_t launch_reveal_eval(const Launch &L, const RevealLayout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *v0, const T *v1, int rowlen, T *msg0, T *msg1) {
  const int block = 256;
  if (rowlen > 0) {
    int grid = grid_for(k_reveal_rowsum<T>, block, lay.N * 64, L.num_cu);
    hipLaunchKernelGGL((k_reveal_rowsum<T>), dim3(grid, party_rows(L)), dim3(block), 0, L.stream, lay.N,
                       reinterpret_cast<const T *>(k0 + lay.off_r), reinterpret_cast<const T *>(k1 + lay.off_r), v0,
                       v1, rowlen, msg0, msg1, party_base(L));
    return hipGetLastError();
  }
  int grid = grid_for(k_reveal_eval<T>, block, lay.N, L.num_cu);
  hipLaunchKernelGGL((k_reveal_eval<T>), dim3(grid, party_rows(L)), dim3(block), 0, L.stream, lay.N,
                     reinterpret_cast<const T *>(k0 + lay.off_r), reinterpret_cast<const T *>(k1 + lay.off_r), v0,
                     v1, rowlen, msg0, msg1, party_base(L));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Beaver product
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pair_row_start(uint32_t N, uint32_t i) { return i * N - (i * (i - 1)) / 2; }

// Operands of product k (MulMap in kernels.h).  The pair row i of a pair index
// r is the largest i with pair_row_start(i) <= r: a float estimate from the
// quadratic, then exact integer corrections.
__device__ __forceinline__ void mul_operands(const MulMap &m, size_t k, uint32_t *a, uint32_t *b) {
  if (m.kind == MulMap::EXPLICIT) {
    *a = m.ia[k];
    *b = m.ib[k];
    return;
  }
  const uint32_t N = m.N, P = N * (N + 1) / 2;
  const uint32_t k32 = uint32_t(k);
  if (m.kind == MulMap::OUTER_TRI) {
    const uint32_t g = k32 / P, r = k32 - g * P;
    const float q = float(2 * N + 1);
    int ie = int((q - sqrtf(q * q - 8.0f * float(r))) * 0.5f);
    uint32_t i = uint32_t(ie < 0 ? 0 : (ie > int(N) - 1 ? int(N) - 1 : ie));
    while (i + 1 < N && pair_row_start(N, i + 1) <= r) i++;
    while (i > 0 && pair_row_start(N, i) > r) i--;
    const uint32_t j = i + (r - pair_row_start(N, i));
    *a = g * N + i;
    *b = g * N + j;
  } else {  // SYM_HADAMARD
    const uint32_t NN = N * N, g = k32 / NN, rem = k32 - g * NN;
    const uint32_t i = rem / N, j = rem - i * N;
    const uint32_t lo = i < j ? i : j, hi = i < j ? j : i;
    *a = k32;
    *b = g * P + pair_row_start(N, lo) + (hi - lo);
  }
}
template <typename T, int NT, int REP>
__global__ void k_mul_keygen_c(AesRK kd, uint32_t gate, size_t nz, MulMap map, const T *rx, const T *ry, T *rz,
                               T *C0, T *C1) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nz; i += size_t(gridDim.x) * blockDim.x) {
    const T r = ring_of<T>(aes.prf(kd, gate, F_ROUT, i));
    rz[i] = r;
    uint32_t a, b;
    mul_operands(map, i, &a, &b);
    const T C = rx[a] * ry[b] + r;
    const T c0 = ring_of<T>(aes.prf(kd, gate, F_SPLIT + 2, i));
    C0[i] = c0;
    C1[i] = C - c0;
  }
}

template <typename T>
hipError_t launch_mul_keygen(const Launch &L, const MulLayout &lay, uint64_t seed, uint32_t gate, const MulMap &map,
                             const T *rx, const T *ry, T *rz, uint8_t *k0, uint8_t *k1) {
  hipError_t e = launch_split<T>(L, seed, gate, F_SPLIT + 0, lay.nx, rx, reinterpret_cast<T *>(k0 + lay.off_rx),
                                 reinterpret_cast<T *>(k1 + lay.off_rx), nullptr);
  if (e != hipSuccess) return e;
  e = launch_split<T>(L, seed, gate, F_SPLIT + 1, lay.ny, ry, reinterpret_cast<T *>(k0 + lay.off_ry),
                      reinterpret_cast<T *>(k1 + lay.off_ry), nullptr);
  if (e != hipSuccess) return e;
  const AesRK kd = dealer_key(L, seed);
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_mul_keygen_c<T, NT, REP>, block, lay.nz, L.num_cu);
    hipLaunchKernelGGL((k_mul_keygen_c<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, kd, gate, lay.nz, map,
                       rx, ry, rz, reinterpret_cast<T *>(k0 + lay.off_c), reinterpret_cast<T *>(k1 + lay.off_c));
    return hipGetLastError();
  });
}

template <typename T>
__global__ void k_mul_eval(size_t nz, const T *Rx0, const T *Rx1, const T *Ry0, const T *Ry1, const T *C0,
                           const T *C1, MulMap map, const T *xhat, const T *yhat, T *msg0, T *msg1, int pbase) {
  const int p = int(blockIdx.y) + pbase;
  const T *Rx = p ? Rx1 : Rx0;
  const T *Ry = p ? Ry1 : Ry0;
  const T *Cc = p ? C1 : C0;
  T *msg = p ? msg1 : msg0;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nz; i += size_t(gridDim.x) * blockDim.x) {
    uint32_t a, b;
    mul_operands(map, i, &a, &b);
    const T x = xhat[a], y = yhat[b];
    T z = Cc[i] - x * Ry[b] - y * Rx[a];
    if (p == 0) z += x * y;
    msg[i] = z;
  }
}

// A (.) W with W symmetric, stored as its upper triangle (SYM_HADAMARD): one
// workgroup per (graph, tile of TI rows, party).  The tile's W entries are
// staged in LDS as a dense TI x N block so that every global read is a
// contiguous run: row i of the triangle for columns j >= i, and for j < i the
// run of entries (j, i0..i0+TI-1) of triangle row j.  The tile's outputs are
// then consecutive elements of A_norm, read and written coalesced.
template <typename T, int TI>
__global__ void k_mul_eval_sym(uint32_t N, const T *Rx0, const T *Rx1, const T *Ry0, const T *Ry1, const T *C0,
                               const T *C1, const T *xhat, const T *yhat, T *msg0, T *msg1, int pbase) {
  extern __shared__ unsigned char lds_raw[];
  T *Wy = reinterpret_cast<T *>(lds_raw);
  T *Wr = Wy + TI * N;
  const int p = int(blockIdx.y) + pbase;
  const T *Rx = p ? Rx1 : Rx0;
  const T *Ry = p ? Ry1 : Ry0;
  const T *Cc = p ? C1 : C0;
  T *msg = p ? msg1 : msg0;
  const uint32_t tiles = (N + TI - 1) / TI, P = N * (N + 1) / 2;
  const uint32_t g = blockIdx.x / tiles, i0 = (blockIdx.x - g * tiles) * TI;
  const uint32_t ni = N - i0 < uint32_t(TI) ? N - i0 : uint32_t(TI);
  const T *yg = yhat + size_t(g) * P, *rg = Ry + size_t(g) * P;
  // columns j >= i: triangle row i
  for (uint32_t ii = 0; ii < ni; ii++) {
    const uint32_t i = i0 + ii, base = pair_row_start(N, i) - i;
    for (uint32_t j = i + threadIdx.x; j < N; j += blockDim.x) {
      Wy[ii * N + j] = yg[base + j];
      Wr[ii * N + j] = rg[base + j];
    }
  }
  // columns j < i: entry (j, i) of triangle row j, tile rows fastest
  const uint32_t nj = i0 + ni - 1;
  for (uint32_t t = threadIdx.x; t < nj * TI; t += blockDim.x) {
    const uint32_t j = t / TI, ii = t - j * TI, i = i0 + ii;
    if (ii < ni && j < i) {
      const uint32_t q = pair_row_start(N, j) + (i - j);
      Wy[ii * N + j] = yg[q];
      Wr[ii * N + j] = rg[q];
    }
  }
  __syncthreads();
  const size_t kb = (size_t(g) * N + i0) * N;
  for (uint32_t t = threadIdx.x; t < ni * N; t += blockDim.x) {
    const size_t k = kb + t;
    const T x = xhat[k], y = Wy[t];
    T z = Cc[k] - x * Wr[t] - y * Rx[k];
    if (p == 0) z += x * y;
    msg[k] = z;
  }
}

template <typename T>
hipError_t launch_mul_eval(const Launch &L, const MulLayout &lay, const uint8_t *k0, const uint8_t *k1,
                           const MulMap &map, const T *xhat, const T *yhat, T *msg0, T *msg1) {
  const int block = 256;
  if (map.kind == MulMap::SYM_HADAMARD) {
    constexpr int TI = sizeof(T) == 4 ? 16 : 8;
    const size_t N = map.N, NN = N * N, P = N * (N + 1) / 2;
    if (N == 0 || lay.nz % NN != 0 || lay.nx != lay.nz || lay.ny != (lay.nz / NN) * P) return hipErrorInvalidValue;
    const size_t tiles = (N + TI - 1) / TI, blocks = (lay.nz / NN) * tiles;
    if (blocks >= (size_t(1) << 31)) return hipErrorInvalidValue;
    const size_t lds = 2 * TI * N * sizeof(T);
    hipLaunchKernelGGL((k_mul_eval_sym<T, TI>), dim3(unsigned(blocks), party_rows(L)), dim3(block), lds, L.stream,
                       uint32_t(N), reinterpret_cast<const T *>(k0 + lay.off_rx),
                       reinterpret_cast<const T *>(k1 + lay.off_rx), reinterpret_cast<const T *>(k0 + lay.off_ry),
                       reinterpret_cast<const T *>(k1 + lay.off_ry), reinterpret_cast<const T *>(k0 + lay.off_c),
                       reinterpret_cast<const T *>(k1 + lay.off_c), xhat, yhat, msg0, msg1, party_base(L));
    return hipGetLastError();
  }
  int grid = grid_for(k_mul_eval<T>, block, lay.nz, L.num_cu);
  hipLaunchKernelGGL((k_mul_eval<T>), dim3(grid, party_rows(L)), dim3(block), 0, L.stream, lay.nz,
                     reinterpret_cast<const T *>(k0 + lay.off_rx), reinterpret_cast<const T *>(k1 + lay.off_rx),
                     reinterpret_cast<const T *>(k0 + lay.off_ry), reinterpret_cast<const T *>(k1 + lay.off_ry),
                     reinterpret_cast<const T *>(k0 + lay.off_c), reinterpret_cast<const T *>(k1 + lay.off_c), map,
                     xhat, yhat, msg0, msg1, party_base(L));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// 8-bit DPF lookup table
// ---------------------------------------------------------------------------
template <typename T, int NT, int REP>
__global__ void k_lut8_keygen(AesRK kd, uint32_t gate, Lut8Layout lay, const T *in_mask,
                              T *out_mask, uint8_t *k0, uint8_t *k1) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const size_t N = lay.dpf.N;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < N; i += size_t(gridDim.x) * blockDim.x) {
    const uint64_t alpha = uint64_t(in_mask[i]) & 255u;
    const DcfGenOut g = dcf_gen_walk(aes, kd, gate, F_DCFA, 8, lay.dpf.L, alpha, i, N, k0, k1,
                                     lay.dpf.off_root, lay.dpf.off_cw, lay.dpf.off_leaf);
    const uint4 lb = xor4(aes.hash(g.s0, c_rkL), and4(g.leafcw, 0u - g.t0));
    const uint32_t pos = uint32_t(alpha & 127u);
    const uint32_t wsel = pos >> 5;
    const uint32_t word = wsel == 0 ? lb.x : wsel == 1 ? lb.y : wsel == 2 ? lb.z : lb.w;
    const uint32_t u0 = (word >> (pos & 31u)) & 1u;
    const T sigma = u0 ? T(1) : T(0) - T(1);
    const T rv = ring_of<T>(aes.prf(kd, gate, F_LUTV, i));
    const T rout = ring_of<T>(aes.prf(kd, gate, F_ROUT, i));
    out_mask[i] = rout;
    const T C = rout - sigma * rv;
    const T v0 = ring_of<T>(aes.prf(kd, gate, F_SPLIT + 0, i));
    const T s0 = ring_of<T>(aes.prf(kd, gate, F_SPLIT + 1, i));
    const T c0 = ring_of<T>(aes.prf(kd, gate, F_SPLIT + 2, i));
    reinterpret_cast<T *>(k0 + lay.off_rv)[i] = v0;
    reinterpret_cast<T *>(k1 + lay.off_rv)[i] = rv - v0;
    reinterpret_cast<T *>(k0 + lay.off_sig)[i] = s0;
    reinterpret_cast<T *>(k1 + lay.off_sig)[i] = sigma - s0;
    reinterpret_cast<T *>(k0 + lay.off_c)[i] = c0;
    reinterpret_cast<T *>(k1 + lay.off_c)[i] = C - c0;
  }
}

template <typename T>
hipError_t launch_lut8_keygen(const Launch &L, const Lut8Layout &lay, uint64_t seed, uint32_t gate,
                              const T *in_mask, T *out_mask, uint8_t *k0, uint8_t *k1) {
  const AesRK kd = dealer_key(L, seed);
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_lut8_keygen<T, NT, REP>, block, lay.dpf.N, L.num_cu);
    hipLaunchKernelGGL((k_lut8_keygen<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, kd, gate, lay,
                       in_mask, out_mask, k0, k1);
    return hipGetLastError();
  });
}

// Phase 1: full-domain expansion of the 8-bit DPF (1 tree level + two 128-bit
// leaves) and the signed inner product with the public table rotated by x^.
template <typename T, int NT, int REP>
__global__ void k_lut8_phase1(Lut8Layout lay, const uint8_t *k0, const uint8_t *k1,
                              const T *table, const T *xhat, T *msg0, T *msg1, int pbase) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  __shared__ T tab[256];
  for (int k = threadIdx.x; k < 256; k += blockDim.x) tab[k] = table[k];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  const int p = int(blockIdx.y) + pbase;
  const uint8_t *K = p ? k1 : k0;
  T *msg = p ? msg1 : msg0;
  const size_t N = lay.dpf.N;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < N; i += size_t(gridDim.x) * blockDim.x) {
    const uint4 s = reinterpret_cast<const uint4 *>(K + lay.dpf.off_root)[i];
    // correction and leaf words are common to both parties: read party 0's
    const uint4 cw = reinterpret_cast<const uint4 *>(k0 + lay.dpf.off_cw)[i];
    const uint4 leaf = reinterpret_cast<const uint4 *>(k0 + lay.dpf.off_leaf)[i];
    const uint32_t t = s.x & 1u;
    const uint4 sl = xor4(aes.hash(s, c_rkH), and4(cw, 0u - t));
    const uint4 sr = xor4(sl, s);
    const uint32_t tl = sl.x & 1u, tr = tl ^ t;
    const uint4 L0 = xor4(aes.hash(sl, c_rkL), and4(leaf, 0u - tl));
    const uint4 L1 = xor4(aes.hash(sr, c_rkL), and4(leaf, 0u - tr));
    const uint32_t w[8] = {L0.x, L0.y, L0.z, L0.w, L1.x, L1.y, L1.z, L1.w};
    const uint32_t xh = uint32_t(xhat[i]) & 255u;
    T acc = 0;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      uint32_t bits = w[q];
      while (bits) {
        const int b = __ffs(bits) - 1;
        bits &= bits - 1;
        acc += tab[(xh - uint32_t(q * 32 + b)) & 255u];
      }
    }
    if (p == 1) acc = T(0) - acc;
    msg[i] = acc + reinterpret_cast<const T *>(K + lay.off_rv)[i];
  }
}

template <typename T>
hipError_t launch_lut8_phase1(const Launch &L, const Lut8Layout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *table, const T *xhat, T *msg0, T *msg1) {
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_lut8_phase1<T, NT, REP>, block, lay.dpf.N, L.num_cu);
    hipLaunchKernelGGL((k_lut8_phase1<T, NT, REP>), dim3(grid, party_rows(L)), dim3(block), 0, L.stream, lay, k0,
                       k1, table, xhat, msg0, msg1, party_base(L));
    return hipGetLastError();
  });
}

template <typename T>
__global__ void k_lut8_phase2(Lut8Layout lay, const uint8_t *k0, const uint8_t *k1, const T *vhat, T *msg0,
                              T *msg1, int pbase) {
  const int p = int(blockIdx.y) + pbase;
  const uint8_t *K = p ? k1 : k0;
  T *msg = p ? msg1 : msg0;
  const size_t N = lay.dpf.N;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < N; i += size_t(gridDim.x) * blockDim.x)
    msg[i] = vhat[i] * reinterpret_cast<const T *>(K + lay.off_sig)[i] + reinterpret_cast<const T *>(K + lay.off_c)[i];
}

template <typename T>
hipError_t launch_lut8_phase2(const Launch &L, const Lut8Layout &lay, const uint8_t *k0, const uint8_t *k1,
                              const T *vhat, T *msg0, T *msg1) {
  const int block = 256;
  int grid = grid_for(k_lut8_phase2<T>, block, lay.dpf.N, L.num_cu);
  hipLaunchKernelGGL((k_lut8_phase2<T>), dim3(grid, party_rows(L)), dim3(block), 0, L.stream, lay, k0, k1, vhat, msg0,
                     msg1, party_base(L));
  return hipGetLastError();
}

template <typename T, int NT, int REP>
__global__ void k_prf_ring(AesRK kd, uint32_t gate, uint32_t field, size_t n, T *out) {
  __shared__ __align__(16) uint32_t lds[AesLds<NT, REP>::kWords];
  AesLds<NT, REP>::fill(lds);
  AesLds<NT, REP> aes(lds);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    out[i] = ring_of<T>(aes.prf(kd, gate, field, i));
}
template <typename T>
hipError_t launch_prf_ring(const Launch &L, uint64_t seed, uint32_t gate, uint32_t field, size_t n, T *out) {
  const AesRK kd = dealer_key(L, seed);
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_prf_ring<T, NT, REP>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_prf_ring<T, NT, REP>), dim3(grid), dim3(block), 0, L.stream, kd, gate, field, n, out);
    return hipGetLastError();
  });
}

// ---------------------------------------------------------------------------
// elementwise helpers
// ---------------------------------------------------------------------------
template <typename T>
__global__ void k_axpby(size_t n, T a, const T *x, T b, const T *y, T c, T *out) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    T v = c;
    if (x) v += a * x[i];
    if (y) v += b * y[i];
    out[i] = v;
  }
}
template <typename T>
hipError_t launch_axpby(const Launch &L, size_t n, T a, const T *x, T b, const T *y, T c, T *out) {
  const int block = 256;
  int grid = grid_for(k_axpby<T>, block, n, L.num_cu);
  hipLaunchKernelGGL((k_axpby<T>), dim3(grid), dim3(block), 0, L.stream, n, a, x, b, y, c, out);
  return hipGetLastError();
}

template <typename T>
__global__ void k_lincomb(size_t rows, size_t cols, T a, const T *x, T b, const T *y, const T *v, int shift, T *out) {
  const size_t n = rows * cols;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    T r = 0;
    if (x) r += a * x[i];
    if (y) r += b * y[i];
    if (v) r += v[i % cols] << shift;
    out[i] = r;
  }
}
template <typename T>
hipError_t launch_lincomb(const Launch &L, size_t rows, size_t cols, T a, const T *x, T b, const T *y, const T *v,
                          int shift, T *out) {
  const int block = 256;
  int grid = grid_for(k_lincomb<T>, block, rows * cols, L.num_cu);
  hipLaunchKernelGGL((k_lincomb<T>), dim3(grid), dim3(block), 0, L.stream, rows, cols, a, x, b, y, v, shift, out);
  return hipGetLastError();
}

template <typename T>
__global__ void k_pool_prep(size_t rows, int C, const T *H, const T *m, T S, T off, T *V) {
  const size_t n = rows * size_t(C);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    V[i] = H[i] + S * m[i / size_t(C)] + off;
}
template <typename T>
hipError_t launch_pool_prep(const Launch &L, size_t rows, int C, const T *H, const T *m, T S, T off, T *V) {
  const int block = 256;
  int grid = grid_for(k_pool_prep<T>, block, rows * size_t(C), L.num_cu);
  hipLaunchKernelGGL((k_pool_prep<T>), dim3(grid), dim3(block), 0, L.stream, rows, C, H, m, S, off, V);
  return hipGetLastError();
}

template <typename T>
__global__ void k_pool_diff(int B, int R, int C, const T *V, T *D) {
  const int pr = R / 2;
  const size_t n = size_t(B) * pr * C;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const size_t c = i % C, bj = i / C;
    const size_t b = bj / pr, j = bj % pr;
    const size_t e = (b * R + 2 * j) * C + c;
    D[i] = V[e + C] - V[e];
  }
}
template <typename T>
hipError_t launch_pool_diff(const Launch &L, int B, int R, int C, const T *V, T *D) {
  const int block = 256;
  int grid = grid_for(k_pool_diff<T>, block, size_t(B) * (R / 2) * C, L.num_cu);
  hipLaunchKernelGGL((k_pool_diff<T>), dim3(grid), dim3(block), 0, L.stream, B, R, C, V, D);
  return hipGetLastError();
}

template <typename T>
__global__ void k_pool_combine(int B, int R, int C, const T *V, const T *y0, const T *y1, T *Vn) {
  const int pr = R / 2, Rn = pr + (R & 1);
  const size_t n = size_t(B) * Rn * C;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const size_t c = i % C, bj = i / C;
    const size_t b = bj / Rn, j = bj % Rn;
    if (int(j) < pr) {
      const size_t yi = (b * pr + j) * C + c;
      T v = V[(b * R + 2 * j) * C + c] + y0[yi];
      if (y1) v += y1[yi];
      Vn[i] = v;
    } else {
      Vn[i] = V[(b * R + R - 1) * C + c];
    }
  }
}
template <typename T>
hipError_t launch_pool_combine(const Launch &L, int B, int R, int C, const T *V, const T *y0, const T *y1, T *Vn) {
  const int block = 256;
  const int Rn = R / 2 + (R & 1);
  int grid = grid_for(k_pool_combine<T>, block, size_t(B) * Rn * C, L.num_cu);
  hipLaunchKernelGGL((k_pool_combine<T>), dim3(grid), dim3(block), 0, L.stream, B, R, C, V, y0, y1, Vn);
  return hipGetLastError();
}

template <typename T>
__global__ void k_concat(int B, int w1, int w2, const T *a, const T *b, T *out) {
  const int w = w1 + w2;
  const size_t n = size_t(B) * w;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / w;
    const int j = int(i % w);
    out[i] = j < w1 ? a[r * w1 + j] : (b ? b[r * w2 + (j - w1)] : T(0));
  }
}
template <typename T>
hipError_t launch_concat(const Launch &L, int B, int w1, int w2, const T *a, const T *b, T *out) {
  const int block = 256;
  int grid = grid_for(k_concat<T>, block, size_t(B) * (w1 + w2), L.num_cu);
  hipLaunchKernelGGL((k_concat<T>), dim3(grid), dim3(block), 0, L.stream, B, w1, w2, a, b, out);
  return hipGetLastError();
}

template <typename T>
__global__ void k_output(int B, int bw, int s, const T *zhat, const T *rz, int64_t bias, int64_t *out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const T z = zhat[b] - rz[b];
  int64_t zs;
  if constexpr (sizeof(T) == 4)
    zs = int64_t(int32_t(z));
  else
    zs = int64_t(z);
  int64_t y = (zs >> s) + bias;
  if (bw == 32) y = int64_t(int32_t(uint32_t(uint64_t(y))));
  out[b] = y;
}
template <typename T>
hipError_t launch_output(const Launch &L, int B, int bw, int s, const T *zhat, const T *rz, int64_t bias,
                         int64_t *out) {
  hipLaunchKernelGGL((k_output<T>), dim3((B + 255) / 256), dim3(256), 0, L.stream, B, bw, s, zhat, rz, bias, out);
  return hipGetLastError();
}

template <typename T>
__global__ void k_rowsum(size_t rows, int len, const T *a, T *out) {
  for (size_t r = size_t(blockIdx.x) * blockDim.x + threadIdx.x; r < rows; r += size_t(gridDim.x) * blockDim.x) {
    T acc = 0;
    for (int j = 0; j < len; j++) acc += a[r * len + j];
    out[r] = acc;
  }
}
template <typename T>
hipError_t launch_rowsum(const Launch &L, size_t rows, int len, const T *a, T *out) {
  const int block = 256;
  int grid = grid_for(k_rowsum<T>, block, rows, L.num_cu);
  hipLaunchKernelGGL((k_rowsum<T>), dim3(grid), dim3(block), 0, L.stream, rows, len, a, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// explicit instantiations
// ---------------------------------------------------------------------------
#define INST(T)                                                                                                      \
  template hipError_t launch_tr_keygen<T>(const Launch &, const TrLayout &, uint64_t, uint32_t, const T *, T *,      \
                                          uint8_t *, uint8_t *);                                                     \
  template hipError_t launch_tr_expand<T>(const Launch &, const TrLayout &, const uint8_t *, uint32_t, int,          \
                                          uint8_t *);                                                                \
  template hipError_t launch_tr_eval<T>(const Launch &, const TrLayout &, const uint8_t *, const uint8_t *,          \
                                        const T *, const T *, int, T *);                                             \
  template hipError_t launch_tr_party_bits<T>(const Launch &, const TrLayout &, const uint8_t *, const T *,         \
                                              const T *, int, uint64_t *);                                           \
  template hipError_t launch_tr_party_msg<T>(const Launch &, const TrLayout &, const uint8_t *, const T *,          \
                                             const T *, int, const uint64_t *, const uint64_t *, T *);               \
  template hipError_t launch_reconstruct<T>(const Launch &, size_t, const T *, const T *, T *);                      \
  template hipError_t launch_local_ars<T>(const Launch &, size_t, int, const T *, const T *, int, T *);              \
  template hipError_t launch_reveal_keygen<T>(const Launch &, const RevealLayout &, uint64_t, uint32_t, T *,         \
                                              uint8_t *, uint8_t *);                                                 \
  template hipError_t launch_reveal_eval<T>(const Launch &, const RevealLayout &, const uint8_t *, const uint8_t *,  \
                                            const T *, const T *, int, T *, T *);                                    \
  template hipError_t launch_mul_keygen<T>(const Launch &, const MulLayout &, uint64_t, uint32_t, const MulMap &,   \
                                           const T *, const T *, T *, uint8_t *, uint8_t *);                         \
  template hipError_t launch_mul_eval<T>(const Launch &, const MulLayout &, const uint8_t *, const uint8_t *,        \
                                         const MulMap &, const T *, const T *, T *, T *);                            \
  template hipError_t launch_lut8_keygen<T>(const Launch &, const Lut8Layout &, uint64_t, uint32_t, const T *, T *, \
                                            uint8_t *, uint8_t *);                                                   \
  template hipError_t launch_lut8_phase1<T>(const Launch &, const Lut8Layout &, const uint8_t *, const uint8_t *,    \
                                            const T *, const T *, T *, T *);                                         \
  template hipError_t launch_lut8_phase2<T>(const Launch &, const Lut8Layout &, const uint8_t *, const uint8_t *,    \
                                            const T *, T *, T *);                                                    \
  template hipError_t launch_split<T>(const Launch &, uint64_t, uint32_t, uint32_t, size_t, const T *, T *, T *,     \
                                      T *);                                                                          \
  template hipError_t launch_prf_ring<T>(const Launch &, uint64_t, uint32_t, uint32_t, size_t, T *);                \
  template hipError_t launch_axpby<T>(const Launch &, size_t, T, const T *, T, const T *, T, T *);                   \
  template hipError_t launch_lincomb<T>(const Launch &, size_t, size_t, T, const T *, T, const T *, const T *, int,   \
                                        T *);                                                                        \
  template hipError_t launch_pool_prep<T>(const Launch &, size_t, int, const T *, const T *, T, T, T *);            \
  template hipError_t launch_pool_diff<T>(const Launch &, int, int, int, const T *, T *);                            \
  template hipError_t launch_pool_combine<T>(const Launch &, int, int, int, const T *, const T *, const T *, T *);   \
  template hipError_t launch_concat<T>(const Launch &, int, int, int, const T *, const T *, T *);                    \
  template hipError_t launch_output<T>(const Launch &, int, int, int, const T *, const T *, int64_t, int64_t *);     \
  template hipError_t launch_rowsum<T>(const Launch &, size_t, int, const T *, T *);

INST(uint32_t)
INST(uint64_t)

}  // namespace mpcx
