// dcf_dev.h -- device-side half-tree DPF/DCF walks (evaluation and dealer).
//
// Evaluation of the comparison [x < alpha] (m-bit x): walk the DPF tree of the
// point alpha along the bits of x, MSB first.  At every level where the bit of x
// is 0 the right sibling's control bit is XORed into the output: the two parties'
// control bits differ exactly on the path of alpha, so the XOR of both outputs is
// 1 iff the path of alpha leaves the path of x to the right, i.e. x < alpha.  The
// 128-bit leaf holds the last 7 levels as a one-hot block, and the bits above
// the low 7 bits of x are folded in with a parity.  This is the DPF-based DCF the
// reference builds on (gpu_mpc/dpf_dcf_adapter.h:1-12, gpu_mpc/ddg_orca.h:11-12).
//
// The tree is the half-tree one (Guo et al., EUROCRYPT 2023): one fixed-key AES
// call per level,  sL = H(s) ^ t*CW,  sR = sL ^ s,  t = lsb(s).
#pragma once
#include <type_traits>

#include "aes_dev.h"

namespace mpcx {

template <class A>
__device__ __forceinline__ uint32_t dcf_eval_walk(const A &aes, uint4 s,
                                                  int m, int L, const uint4 *__restrict__ cw, size_t stride,
                                                  uint4 leaf, uint64_t x) {
  uint32_t t = s.x & 1u, out = 0;
  uint4 cnext = L > 0 ? cw[0] : make_uint4(0, 0, 0, 0);
  // the path bits of x, MSB first: levels consume x >> (m-1-l); for m <= 32 the
  // walk stays in 32-bit registers
  const bool wide = m > 32;
  const uint32_t xlo = uint32_t(x);
  for (int l = 0; l < L; l++) {
    const uint4 c = cnext;
    if (l + 1 < L) cnext = cw[size_t(l + 1) * stride];
    const int sh = m - 1 - l;
    const uint32_t bit = wide ? uint32_t(x >> sh) & 1u : (xlo >> sh) & 1u;
    const uint4 h = aes.hash(s, c_rkH);
    const uint4 sl = xor_and4(h, c, 0u - t);
    const uint32_t tl = sl.x & 1u;
    out ^= (bit ^ 1u) & (tl ^ t);
    s = xor_and4(sl, s, 0u - bit);
    t = tl ^ (t & bit);
  }
  const uint4 lb = xor_and4(aes.hash(s, c_rkL), leaf, 0u - t);
  const uint32_t pos = m >= 7 ? uint32_t(x & 127u) : uint32_t(x);
  return out ^ parity_above(lb, pos);
}

// Both parties' hashes of a level: side by side on the T0/T1 table, one after
// the other on the other layouts.
template <class A>
__device__ __forceinline__ void hash_pair(const A &aes, uint4 s, uint4 u, const AesRK &rk, uint4 *hs, uint4 *hu) {
  if constexpr (std::is_same<A, AesPerm2>::value) {
    aes.hash2(s, u, rk, hs, hu);
  } else {
    *hs = aes.hash(s, rk);
    *hu = aes.hash(u, rk);
  }
}

// Both parties' walks of one element in one thread, from their roots s0 and s1
// (the correction words and the leaf are common to the two keys): the XOR of
// the two parties' outputs, i.e. the reconstructed bit.  Each level hashes the
// two seeds side by side and reads its correction word once.
template <class A>
__device__ __forceinline__ uint32_t dcf_eval_walk2(const A &aes, uint4 s0, uint4 s1, int m, int L,
                                                   const uint4 *__restrict__ cw, size_t stride, uint4 leaf,
                                                   uint64_t x) {
  uint32_t t0 = s0.x & 1u, t1 = s1.x & 1u, out = 0;
  uint4 cnext = L > 0 ? cw[0] : make_uint4(0, 0, 0, 0);
  const bool wide = m > 32;
  const uint32_t xlo = uint32_t(x);
  for (int l = 0; l < L; l++) {
    const uint4 c = cnext;
    if (l + 1 < L) cnext = cw[size_t(l + 1) * stride];
    const int sh = m - 1 - l;
    const uint32_t bit = wide ? uint32_t(x >> sh) & 1u : (xlo >> sh) & 1u;
    uint4 h0, h1;
    hash_pair(aes, s0, s1, c_rkH, &h0, &h1);
    const uint4 sl0 = xor_and4(h0, c, 0u - t0), sl1 = xor_and4(h1, c, 0u - t1);
    const uint32_t tl0 = sl0.x & 1u, tl1 = sl1.x & 1u;
    out ^= (bit ^ 1u) & (tl0 ^ t0 ^ tl1 ^ t1);
    s0 = xor_and4(sl0, s0, 0u - bit);
    s1 = xor_and4(sl1, s1, 0u - bit);
    t0 = tl0 ^ (t0 & bit);
    t1 = tl1 ^ (t1 & bit);
  }
  uint4 l0, l1;
  hash_pair(aes, s0, s1, c_rkL, &l0, &l1);
  const uint4 lb = xor4(xor_and4(l0, leaf, 0u - t0), xor_and4(l1, leaf, 0u - t1));
  const uint32_t pos = m >= 7 ? uint32_t(x & 127u) : uint32_t(x);
  return out ^ parity_above(lb, pos);
}

// The same walk on the quad-lane AES (latency-bound launches): lane j of a quad
// holds word j of the seed, of every correction word (cw: the lane's word of
// level 0, levels stride_words apart) and of the leaf; the control bits are bit
// 0 of word 0 (lane 0's), and the leaf's parity above pos is the xor of the four
// lanes' parities of their 32 bits.  Every lane of the quad returns the bit.
__device__ __forceinline__ uint32_t dcf_eval_walk_quad(const AesQuad &aes, const AesQuad::Keys &kH,
                                                       const AesQuad::Keys &kL, uint32_t s, int m, int L,
                                                       const uint32_t *__restrict__ cw, size_t stride_words,
                                                       uint32_t leaf, uint64_t x) {
  uint32_t t = AesQuad::lane0(s) & 1u, out = 0;
  uint32_t cnext = L > 0 ? cw[0] : 0u;
  const bool wide = m > 32;
  const uint32_t xlo = uint32_t(x);
  for (int l = 0; l < L; l++) {
    const uint32_t c = cnext;
    if (l + 1 < L) cnext = cw[size_t(l + 1) * stride_words];
    const int sh = m - 1 - l;
    const uint32_t bit = wide ? uint32_t(x >> sh) & 1u : (xlo >> sh) & 1u;
    const uint32_t sl = xor_and(aes.hash(s, kH), c, 0u - t);
    const uint32_t tl = AesQuad::lane0(sl) & 1u;
    out ^= (bit ^ 1u) & (tl ^ t);
    s = xor_and(sl, s, 0u - bit);
    t = tl ^ (t & bit);
  }
  const uint32_t lb = xor_and(aes.hash(s, kL), leaf, 0u - t);
  const uint32_t pos = m >= 7 ? uint32_t(x & 127u) : uint32_t(x);
  const uint32_t lo = 32u * aes.j;
  const uint32_t msk = pos < lo ? 0xffffffffu : (pos >= lo + 31 ? 0u : 0xffffffffu << (pos - lo + 1));
  return out ^ (AesQuad::quad_xor(__popc(lb & msk) & 1u) & 1u);
}

struct DcfGenOut {
  uint4 s0;      // party 0's final on-path seed
  uint32_t t0;   // party 0's final on-path control bit
  uint4 leafcw;  // leaf correction word
};

// Dealer walk for one element from the parties' root seeds s0 (lsb 0) and s1
// (lsb 1): writes the roots, the level correction words (level-major, stride N)
// and the leaf correction word of both parties.
template <class A>
__device__ __forceinline__ DcfGenOut dcf_gen_roots(const A &aes, uint4 s0, uint4 s1, int m, int L, uint64_t alpha,
                                                   size_t i, size_t N, uint8_t *k0, uint8_t *k1, size_t off_root,
                                                   size_t off_cw, size_t off_leaf) {
  const uint4 D = xor4(s0, s1);
  reinterpret_cast<uint4 *>(k0 + off_root)[i] = s0;
  reinterpret_cast<uint4 *>(k1 + off_root)[i] = s1;
  uint32_t t0 = 0, t1 = 1;
  uint4 *c0 = reinterpret_cast<uint4 *>(k0 + off_cw) + i;
  uint4 *c1 = reinterpret_cast<uint4 *>(k1 + off_cw) + i;
  for (int l = 0; l < L; l++) {
    const uint32_t a = uint32_t(alpha >> (m - 1 - l)) & 1u;
    const uint4 h0 = aes.hash(s0, c_rkH);
    const uint4 h1 = aes.hash(s1, c_rkH);
    const uint4 cw = xor4(xor4(h0, h1), and4(D, a - 1u));  // a ? 0 : D
    c0[size_t(l) * N] = cw;
    c1[size_t(l) * N] = cw;
    const uint4 sl0 = xor4(h0, and4(cw, 0u - t0));
    const uint4 sl1 = xor4(h1, and4(cw, 0u - t1));
    s0 = xor4(sl0, and4(s0, 0u - a));
    s1 = xor4(sl1, and4(s1, 0u - a));
    t0 = s0.x & 1u;
    t1 = s1.x & 1u;
  }
  const uint32_t pos = m >= 7 ? uint32_t(alpha & 127u) : uint32_t(alpha);
  uint4 lcw = xor4(aes.hash(s0, c_rkL), aes.hash(s1, c_rkL));
  const uint32_t bitv = 1u << (pos & 31u);
  lcw.x ^= (pos >> 5) == 0 ? bitv : 0u;
  lcw.y ^= (pos >> 5) == 1 ? bitv : 0u;
  lcw.z ^= (pos >> 5) == 2 ? bitv : 0u;
  lcw.w ^= (pos >> 5) == 3 ? bitv : 0u;
  reinterpret_cast<uint4 *>(k0 + off_leaf)[i] = lcw;
  reinterpret_cast<uint4 *>(k1 + off_leaf)[i] = lcw;
  DcfGenOut o;
  o.s0 = s0;
  o.t0 = t0;
  o.leafcw = lcw;
  return o;
}

// The same with the roots drawn from the dealer PRF: s0 = PRF(fb) with lsb 0,
// s1 = s0 ^ D, D = PRF(fb + 1) with lsb 1.
template <class A>
__device__ __forceinline__ DcfGenOut dcf_gen_walk(const A &aes, const AesRK &kd, uint32_t gate, uint32_t fb, int m, int L,
                                                  uint64_t alpha, size_t i, size_t N, uint8_t *k0,
                                                  uint8_t *k1, size_t off_root, size_t off_cw,
                                                  size_t off_leaf) {
  uint4 s0 = aes.prf(kd, gate, fb + 0, i);
  s0.x &= ~1u;
  uint4 D = aes.prf(kd, gate, fb + 1, i);
  D.x |= 1u;
  return dcf_gen_roots(aes, s0, xor4(s0, D), m, L, alpha, i, N, k0, k1, off_root, off_cw, off_leaf);
}

// Root seed of party p for a DCF drawn from the party's own PRF key: lsb = p.
template <class A>
__device__ __forceinline__ uint4 party_root(const A &aes, const AesRK &kp, int p, uint32_t gate, uint32_t fb,
                                            size_t i) {
  uint4 s = aes.prf(kp, gate, fb + 0, i);
  s.x = (s.x & ~1u) | uint32_t(p);
  return s;
}

}  // namespace mpcx
