// kernels.hip -- HIP kernels of the secure-inference online path for gfx950
// (the truncation / ReLU gate family is in gates.hip, the ring GEMMs in gemm.hip).
//
// Reference interfaces these kernels stand behind (EzPC GPU-MPC, called from the
// reference's backend; signatures reconstructed from the call sites):
//   DCF eval / keygen ........ gpuDcf / gpuKeyGenDCF    (gpu_mpc/dpf_dcf_adapter.h:266,372)
//   Beaver product ........... gpuMul / gpuKeygenMul    (gpu_mpc/secure_adj_norm.h:611-651,326-365)
//   8-bit DPF LUT ............ gpuDpfLUT / gpuKeyGenLUT (gpu_mpc/secure_adj_norm.h:510-520,270-279)
//   reveal ................... reconstructInPlace       (gpu_mpc/utils/gpu_comms.h:290-302)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "dcf_dev.h"
#include "kernels.h"
#include "launch_util.h"

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

// Inputs of type X (uint64_t, or the ring's element type) reduced to the m-bit
// domain; mask: optional 32-bit words of bits XORed into the output (the
// reference's maskEpilogue, bit i of word i/32), or null.
template <typename X>
struct DcfEvalArgs {
  int m, L;
  size_t n;
  const uint8_t *key;
  size_t off_root, off_cw, off_leaf, off_z;
  const X *x;
  uint64_t xmask;
  const uint32_t *mask;
  uint64_t *out;
};

template <int NT, int REP, typename X>
__global__ void k_dcf_eval(DcfEvalArgs<X> a) {
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
      b = dcf_eval_walk(aes, root[i], a.m, a.L, cw + i, a.n, leaf[i], uint64_t(a.x[i]) & a.xmask);
      b ^= get_bit(zp, i);
      if (a.mask) b ^= (a.mask[i >> 5] >> (i & 31)) & 1u;
    }
    const uint64_t w = __ballot(b);
    if (lane_id() == 0) a.out[base >> 6] = w;
  }
}

template <typename X>
hipError_t launch_dcf_eval_x(const Launch &L, int m, size_t n, const uint8_t *key, size_t base, const X *x,
                             const uint32_t *mask, uint64_t *out_bits) {
  DcfLayout lay = dcf_layout(m, n, base, true);
  DcfEvalArgs<X> a;
  a.m = m;
  a.L = lay.L;
  a.n = n;
  a.key = key;
  a.off_root = lay.off_root;
  a.off_cw = lay.off_cw;
  a.off_leaf = lay.off_leaf;
  a.off_z = lay.off_z;
  a.x = x;
  a.xmask = m >= 64 ? ~0ull : ((1ull << m) - 1ull);
  a.mask = mask;
  a.out = out_bits;
  return with_variant(L, [&](auto v) {
    constexpr int NT = decltype(v)::nt, REP = decltype(v)::rep;
    int block = variant_block(L);
    int grid = grid_for(k_dcf_eval<NT, REP, X>, block, n, L.num_cu);
    hipLaunchKernelGGL((k_dcf_eval<NT, REP, X>), dim3(grid), dim3(block), 0, L.stream, a);
    return hipGetLastError();
  });
}

hipError_t launch_dcf_eval(const Launch &L, int party, int m, size_t n, const uint8_t *key, size_t base,
                           const uint64_t *x, uint64_t *out_bits) {
  (void)party;
  return launch_dcf_eval_x<uint64_t>(L, m, n, key, base, x, nullptr, out_bits);
}
template <typename T>
hipError_t launch_dcf_eval_ring(const Launch &L, int m, size_t n, const uint8_t *key, const T *x,
                                const uint32_t *mask, uint64_t *out_bits) {
  return launch_dcf_eval_x<T>(L, m, n, key, 0, x, mask, out_bits);
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

// Reduced-width wire form of a revealed value known modulo 2^m (m < bits of T):
// element i occupies bits [i m, i m + m) of a little-endian stream of 64-bit
// words, ceil(n m / 64) words in all (the reference sends truncate-reduce
// outputs at bout bits the same way, gpu_mpc/utils/gpu_comms.h:143-168).
// One thread per word: the word's first element may start in the previous
// word, the others follow every m bits.
template <typename T>
__global__ void k_pack_bits(size_t n, int m, const T *v, uint64_t *words, size_t nw) {
  const uint64_t vm = (m >= 64) ? ~0ull : ((1ull << m) - 1ull);
  for (size_t w = size_t(blockIdx.x) * blockDim.x + threadIdx.x; w < nw; w += size_t(gridDim.x) * blockDim.x) {
    const uint64_t bit0 = uint64_t(w) * 64u;
    size_t e = size_t(bit0 / uint64_t(m));
    const int off = int(bit0 - uint64_t(e) * uint64_t(m));  // bits of element e already in word w - 1
    uint64_t acc = (uint64_t(v[e]) & vm) >> off;
    int pos = m - off;
    for (++e; pos < 64 && e < n; ++e, pos += m) acc |= (uint64_t(v[e]) & vm) << pos;
    words[w] = acc;
  }
}
// out[i] = (own[i] + the peer's packed element i) mod 2^m
template <typename T>
__global__ void k_unpack_reconstruct(size_t n, int m, const T *own, const uint64_t *peer, T *out) {
  const uint64_t vm = (1ull << m) - 1ull;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const uint64_t bit = uint64_t(i) * uint64_t(m);
    const size_t w = size_t(bit >> 6);
    const int off = int(bit & 63u);
    uint64_t v = peer[w] >> off;
    if (off + m > 64) v |= peer[w + 1] << (64 - off);  // the element runs into the next word
    out[i] = T((uint64_t(own[i]) + v) & vm);
  }
}
template <typename T>
hipError_t launch_pack_bits(const Launch &L, size_t n, int m, const T *v, uint64_t *words) {
  if (m < 1 || m >= int(8 * sizeof(T))) return hipErrorInvalidValue;
  const size_t nw = packed_words(n, m);
  if (nw == 0) return hipSuccess;
  const int block = 256;
  int grid = grid_for(k_pack_bits<T>, block, nw, L.num_cu);
  hipLaunchKernelGGL((k_pack_bits<T>), dim3(grid), dim3(block), 0, L.stream, n, m, v, words, nw);
  return hipGetLastError();
}
template <typename T>
hipError_t launch_unpack_reconstruct(const Launch &L, size_t n, int m, const T *own, const uint64_t *peer, T *out) {
  if (m < 1 || m >= int(8 * sizeof(T))) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const int block = 256;
  int grid = grid_for(k_unpack_reconstruct<T>, block, n, L.num_cu);
  hipLaunchKernelGGL((k_unpack_reconstruct<T>), dim3(grid), dim3(block), 0, L.stream, n, m, own, peer, out);
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

// Both parties in this process: each thread forms party 0's message v0 + R0 and
// party 1's v1 + R1 from each party's own share and key, and writes their sum,
// the revealed value; the message planes never reach HBM and no reconstruction
// launch follows.
template <typename T>
__global__ void k_reveal_sum(size_t n, const T *R0, const T *R1, const T *v0, const T *v1, T *out) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const T m0 = v0[i] + R0[i], m1 = v1[i] + R1[i];
    out[i] = m0 + m1;
  }
}
// The row-sum reveal (degrees) in the same form: 16 lanes per row of rowlen
// contiguous words, each lane adding its words of both parties' rows (16-byte
// loads where rows are whole 16-byte groups), then a 16-lane reduction; lane 0
// of the group adds both parties' masks.  The two messages are sums, so adding
// the parties' partial sums before the reduction gives the same revealed value.
constexpr int kRowLanes = 16;
template <typename T, bool VEC>
__global__ void k_reveal_rowsum_sum(size_t n, const T *R0, const T *R1, const T *v0, const T *v1, int rowlen,
                                    T *out) {
  const int sub = int(threadIdx.x) % kRowLanes;
  const size_t grp = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) / kRowLanes;
  const size_t ngrp = size_t(gridDim.x) * blockDim.x / kRowLanes;
  const size_t rows = (n + ngrp - 1) / ngrp * ngrp;  // every group runs the same trip count
  for (size_t r = grp; r < rows; r += ngrp) {
    T x = 0;
    if (r < n) {
      const T *a = v0 + r * size_t(rowlen), *b = v1 + r * size_t(rowlen);
      if constexpr (VEC) {
        constexpr int W = 16 / int(sizeof(T));
        const int ng = rowlen / W;
        for (int g = sub; g < ng; g += kRowLanes) {
          const uint4 pa = reinterpret_cast<const uint4 *>(a)[g], pb = reinterpret_cast<const uint4 *>(b)[g];
          if constexpr (sizeof(T) == 4) {
            x += (pa.x + pa.y + pa.z + pa.w) + (pb.x + pb.y + pb.z + pb.w);
          } else {
            x += ((uint64_t(pa.y) << 32 | pa.x) + (uint64_t(pa.w) << 32 | pa.z)) +
                 ((uint64_t(pb.y) << 32 | pb.x) + (uint64_t(pb.w) << 32 | pb.z));
          }
        }
      } else {
        for (int j = sub; j < rowlen; j += kRowLanes) x += a[j] + b[j];
      }
    }
#pragma unroll
    for (int o = kRowLanes / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, kRowLanes);
    if (r < n && sub == 0) {
      const T m0 = R0[r], m1 = R1[r];
      out[r] = x + m0 + m1;
    }
  }
}

template <typename T>
hipError_t launch_reveal_sum(const Launch &L, const RevealLayout &lay, const uint8_t *k0, const uint8_t *k1,
                             const T *v0, const T *v1, int rowlen, T *out) {
  const int block = 256;
  const T *R0 = reinterpret_cast<const T *>(k0 + lay.off_r), *R1 = reinterpret_cast<const T *>(k1 + lay.off_r);
  if (rowlen > 0) {
    const bool vec = (size_t(rowlen) * sizeof(T)) % 16 == 0 && (reinterpret_cast<uintptr_t>(v0) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(v1) & 15) == 0;
    if (vec) {
      const int grid = grid_for(k_reveal_rowsum_sum<T, true>, block, lay.N * kRowLanes, L.num_cu);
      hipLaunchKernelGGL((k_reveal_rowsum_sum<T, true>), dim3(grid), dim3(block), 0, L.stream, lay.N, R0, R1, v0, v1,
                         rowlen, out);
    } else {
      const int grid = grid_for(k_reveal_rowsum_sum<T, false>, block, lay.N * kRowLanes, L.num_cu);
      hipLaunchKernelGGL((k_reveal_rowsum_sum<T, false>), dim3(grid), dim3(block), 0, L.stream, lay.N, R0, R1, v0,
                         v1, rowlen, out);
    }
    return hipGetLastError();
  }
  const int grid = grid_for(k_reveal_sum<T>, block, lay.N, L.num_cu);
  hipLaunchKernelGGL((k_reveal_sum<T>), dim3(grid), dim3(block), 0, L.stream, lay.N, R0, R1, v0, v1, out);
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

// Both parties in this process: each thread forms party 0's message
// x^y^ - x^ ry0 - y^ rx0 + c0 and party 1's - x^ ry1 - y^ rx1 + c1, each from the
// party's own key, and writes their sum, the revealed product (the operands are
// read once, no message planes, no reconstruction launch).
template <typename T>
__global__ void k_mul_eval_sum(size_t nz, const T *Rx0, const T *Rx1, const T *Ry0, const T *Ry1, const T *C0,
                               const T *C1, MulMap map, const T *xhat, const T *yhat, T *out) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nz; i += size_t(gridDim.x) * blockDim.x) {
    uint32_t a, b;
    mul_operands(map, i, &a, &b);
    const T x = xhat[a], y = yhat[b];
    const T z0 = C0[i] - x * Ry0[b] - y * Rx0[a] + x * y;
    const T z1 = C1[i] - x * Ry1[b] - y * Rx1[a];
    out[i] = z0 + z1;
  }
}

// A (.) W with W symmetric (SYM_HADAMARD) in the same form: one workgroup per
// (graph, tile of TI rows).  The tile's W entries and both parties' masks of W
// are staged in LDS as dense TI x N blocks (contiguous global runs: row i of the
// triangle for j >= i, entries (j, i0..i0+TI-1) of triangle row j for j < i), in
// batches of kStage slots per thread whose loads all go out before any store;
// then the tile's outputs, consecutive elements of A_norm, are read and written
// coalesced.
constexpr int kStage = 8;
template <typename T, int TI>
__global__ void k_mul_eval_sym_sum(uint32_t N, const T *Rx0, const T *Rx1, const T *Ry0, const T *Ry1, const T *C0,
                                   const T *C1, const T *xhat, const T *yhat, T *out) {
  extern __shared__ unsigned char lds_raw[];
  T *Wy = reinterpret_cast<T *>(lds_raw);
  T *W0 = Wy + TI * N, *W1 = W0 + TI * N;
  const uint32_t tiles = (N + TI - 1) / TI, P = N * (N + 1) / 2;
  const uint32_t g = blockIdx.x / tiles, i0 = (blockIdx.x - g * tiles) * TI;
  const uint32_t ni = N - i0 < uint32_t(TI) ? N - i0 : uint32_t(TI);
  const T *yg = yhat + size_t(g) * P, *r0g = Ry0 + size_t(g) * P, *r1g = Ry1 + size_t(g) * P;
  // staging slots: [0, ni N) row-major over (ii, j), taken where j >= i; then
  // [ni N, ni N + nj TI) over (j, ii) with tile rows fastest, taken where j < i
  const uint32_t n1 = ni * N, nj = i0 + ni - 1, n2 = nj * TI;
  for (uint32_t t0 = threadIdx.x; t0 < n1 + n2; t0 += kStage * blockDim.x) {
    T vy[kStage], v0[kStage], v1[kStage];
    uint32_t dst[kStage];
#pragma unroll
    for (int u = 0; u < kStage; u++) {
      const uint32_t t = t0 + uint32_t(u) * blockDim.x;
      uint32_t q = 0, d = ~0u;
      if (t < n1) {
        const uint32_t ii = t / N, j = t - ii * N, i = i0 + ii;
        if (j >= i) {
          q = pair_row_start(N, i) + (j - i);
          d = ii * N + j;
        }
      } else if (t < n1 + n2) {
        const uint32_t tt = t - n1, j = tt / TI, ii = tt - j * TI, i = i0 + ii;
        if (ii < ni && j < i) {
          q = pair_row_start(N, j) + (i - j);
          d = ii * N + j;
        }
      }
      dst[u] = d;
      vy[u] = d != ~0u ? yg[q] : T(0);
      v0[u] = d != ~0u ? r0g[q] : T(0);
      v1[u] = d != ~0u ? r1g[q] : T(0);
    }
#pragma unroll
    for (int u = 0; u < kStage; u++)
      if (dst[u] != ~0u) {
        Wy[dst[u]] = vy[u];
        W0[dst[u]] = v0[u];
        W1[dst[u]] = v1[u];
      }
  }
  __syncthreads();
  const size_t kb = (size_t(g) * N + i0) * N;
  for (uint32_t t = threadIdx.x; t < ni * N; t += blockDim.x) {
    const size_t k = kb + t;
    const T x = xhat[k], y = Wy[t];
    const T z0 = C0[k] - x * W0[t] - y * Rx0[k] + x * y;
    const T z1 = C1[k] - x * W1[t] - y * Rx1[k];
    out[k] = z0 + z1;
  }
}

template <typename T>
hipError_t launch_mul_eval_sum(const Launch &L, const MulLayout &lay, const uint8_t *k0, const uint8_t *k1,
                               const MulMap &map, const T *xhat, const T *yhat, T *out) {
  const T *Rx0 = reinterpret_cast<const T *>(k0 + lay.off_rx), *Rx1 = reinterpret_cast<const T *>(k1 + lay.off_rx);
  const T *Ry0 = reinterpret_cast<const T *>(k0 + lay.off_ry), *Ry1 = reinterpret_cast<const T *>(k1 + lay.off_ry);
  const T *C0 = reinterpret_cast<const T *>(k0 + lay.off_c), *C1 = reinterpret_cast<const T *>(k1 + lay.off_c);
  const int block = 256;
  constexpr int TI = sizeof(T) == 4 ? 16 : 8;
  // the staged tile fits 64 KiB of LDS up to N = 341; larger graphs gather W in
  // the generic kernel (the same map, computed per product)
  if (map.kind == MulMap::SYM_HADAMARD && 3 * TI * size_t(map.N) * sizeof(T) <= 65536) {
    const size_t N = map.N, NN = N * N, P = N * (N + 1) / 2;
    if (N == 0 || lay.nz % NN != 0 || lay.nx != lay.nz || lay.ny != (lay.nz / NN) * P) return hipErrorInvalidValue;
    const size_t tiles = (N + TI - 1) / TI, blocks = (lay.nz / NN) * tiles;
    if (blocks >= (size_t(1) << 31)) return hipErrorInvalidValue;
    const size_t lds = 3 * TI * N * sizeof(T);
    hipLaunchKernelGGL((k_mul_eval_sym_sum<T, TI>), dim3(unsigned(blocks)), dim3(block), lds, L.stream, uint32_t(N),
                       Rx0, Rx1, Ry0, Ry1, C0, C1, xhat, yhat, out);
    return hipGetLastError();
  }
  const int grid = grid_for(k_mul_eval_sum<T>, block, lay.nz, L.num_cu);
  hipLaunchKernelGGL((k_mul_eval_sum<T>), dim3(grid), dim3(block), 0, L.stream, lay.nz, Rx0, Rx1, Ry0, Ry1, C0, C1, map,
                     xhat, yhat, out);
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
#define INST(T)                                                                                                       \
  template hipError_t launch_reconstruct<T>(const Launch &, size_t, const T *, const T *, T *);                       \
  template hipError_t launch_dcf_eval_ring<T>(const Launch &, int, size_t, const uint8_t *, const T *,              \
                                              const uint32_t *, uint64_t *);                                          \
  template hipError_t launch_pack_bits<T>(const Launch &, size_t, int, const T *, uint64_t *);                        \
  template hipError_t launch_unpack_reconstruct<T>(const Launch &, size_t, int, const T *, const uint64_t *, T *);    \
  template hipError_t launch_local_ars<T>(const Launch &, size_t, int, const T *, const T *, int, T *);               \
  template hipError_t launch_reveal_keygen<T>(const Launch &, const RevealLayout &, uint64_t, uint32_t, T *,          \
                                              uint8_t *, uint8_t *);                                                  \
  template hipError_t launch_reveal_eval<T>(const Launch &, const RevealLayout &, const uint8_t *, const uint8_t *,   \
                                            const T *, const T *, int, T *, T *);                                     \
  template hipError_t launch_mul_keygen<T>(const Launch &, const MulLayout &, uint64_t, uint32_t, const MulMap &,     \
                                           const T *, const T *, T *, uint8_t *, uint8_t *);                          \
  template hipError_t launch_mul_eval<T>(const Launch &, const MulLayout &, const uint8_t *, const uint8_t *,         \
                                         const MulMap &, const T *, const T *, T *, T *);                             \
  template hipError_t launch_mul_eval_sum<T>(const Launch &, const MulLayout &, const uint8_t *, const uint8_t *,     \
                                             const MulMap &, const T *, const T *, T *);                              \
  template hipError_t launch_reveal_sum<T>(const Launch &, const RevealLayout &, const uint8_t *, const uint8_t *,    \
                                           const T *, const T *, int, T *);                                           \
  template hipError_t launch_lut8_keygen<T>(const Launch &, const Lut8Layout &, uint64_t, uint32_t, const T *, T *,   \
                                            uint8_t *, uint8_t *);                                                    \
  template hipError_t launch_lut8_phase1<T>(const Launch &, const Lut8Layout &, const uint8_t *, const uint8_t *,     \
                                            const T *, const T *, T *, T *);                                          \
  template hipError_t launch_lut8_phase2<T>(const Launch &, const Lut8Layout &, const uint8_t *, const uint8_t *,     \
                                            const T *, T *, T *);                                                     \
  template hipError_t launch_split<T>(const Launch &, uint64_t, uint32_t, uint32_t, size_t, const T *, T *, T *,      \
                                      T *);                                                                           \
  template hipError_t launch_prf_ring<T>(const Launch &, uint64_t, uint32_t, uint32_t, size_t, T *);                  \
  template hipError_t launch_axpby<T>(const Launch &, size_t, T, const T *, T, const T *, T, T *);                    \
  template hipError_t launch_lincomb<T>(const Launch &, size_t, size_t, T, const T *, T, const T *, const T *, int,   \
                                        T *);                                                                         \
  template hipError_t launch_pool_prep<T>(const Launch &, size_t, int, const T *, const T *, T, T, T *);              \
  template hipError_t launch_pool_diff<T>(const Launch &, int, int, int, const T *, T *);                             \
  template hipError_t launch_pool_combine<T>(const Launch &, int, int, int, const T *, const T *, const T *, T *);    \
  template hipError_t launch_concat<T>(const Launch &, int, int, int, const T *, const T *, T *);                     \
  template hipError_t launch_output<T>(const Launch &, int, int, int, const T *, const T *, int64_t, int64_t *);      \
  template hipError_t launch_rowsum<T>(const Launch &, size_t, int, const T *, T *);
INST(uint32_t)
INST(uint64_t)

}  // namespace mpcx
