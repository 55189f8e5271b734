// aes_dev.h -- AES-128 encryption on CDNA4 with T-tables staged in LDS, and the
// half-tree hashes / dealer PRF built on it.
//
// State: four little-endian 32-bit columns (c_j = byte 4j | byte 4j+1 << 8 | ...).
// One round:  n_j = T0[b0(c_j)] ^ T1[b1(c_j+1)] ^ T2[b2(c_j+2)] ^ T3[b3(c_j+3)] ^ rk_j
// with T0[x] = (2S[x], S[x], S[x], 3S[x]) as bytes 0..3 and T_k = rotl(T0, 8k).
// The last round reads S[x] out of the byte of T_(r+3)%4 that holds it.
//
// LDS layout: NT tables (1 = T0 only, rotations computed; 4 = all four), each
// entry replicated REP times and interleaved so that word address of entry e,
// copy c is e*REP + c.  Lane l reads copy (l % REP), so with REP equal to the
// number of LDS banks the 64 lanes of a wavefront never collide on a bank.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mpcx_core.h"

namespace mpcx {

struct T0Table {
  uint32_t v[256];
};

constexpr uint8_t xtime_c(uint8_t a) { return uint8_t((a << 1) ^ ((a & 0x80) ? 0x1b : 0)); }
constexpr T0Table make_t0() {
  T0Table t{};
  for (int x = 0; x < 256; x++) {
    uint8_t s = kSboxC[x];
    uint8_t s2 = xtime_c(s);
    uint8_t s3 = uint8_t(s2 ^ s);
    t.v[x] = uint32_t(s2) | (uint32_t(s) << 8) | (uint32_t(s) << 16) | (uint32_t(s3) << 24);
  }
  return t;
}

__device__ __constant__ const T0Table c_T0 = make_t0();

__device__ __constant__ const AesRK c_rkH = aes_expand_c(kKeyHc);  // tree hash H
__device__ __constant__ const AesRK c_rkL = aes_expand_c(kKeyLc);  // leaf hash HL

__device__ __forceinline__ uint32_t rotl32(uint32_t v, int k) {
  return k == 0 ? v : ((v << k) | (v >> (32 - k)));
}

// a ^ b ^ c in one v_bitop3_b32 (truth table 0x96 = 0xf0 ^ 0xcc ^ 0xaa).
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

template <int NT, int REP>
struct AesTab {
  static_assert(NT == 1 || NT == 4, "NT");  // NT == 0: AesPerm
  static_assert(REP >= 1 && REP <= 64 && (REP & (REP - 1)) == 0, "REP");
  static constexpr int kWords = NT * 256 * REP;
  static constexpr int kBytes = kWords * 4;
  static constexpr int kLogRep = REP == 1 ? 0 : REP == 2 ? 1 : REP == 4 ? 2 : REP == 8 ? 3 : REP == 16 ? 4 : REP == 32 ? 5 : 6;

  const char *base;
  uint32_t laneoff;

  // Fill the replicated tables; must be called by every thread of the block.
  __device__ static void fill(uint32_t *lds) {
    for (int w = threadIdx.x; w < kWords; w += blockDim.x) {
      int e = w >> kLogRep;
      int k = e >> 8, x = e & 255;
      lds[w] = rotl32(c_T0.v[x], 8 * k);
    }
    __syncthreads();
  }

  __device__ AesTab(const uint32_t *lds) : base((const char *)lds) {
    laneoff = (threadIdx.x & (REP - 1)) * 4u;
  }

  __device__ __forceinline__ uint32_t T(int k, uint32_t x) const {
    if constexpr (NT == 4) {
      return *(const uint32_t *)(base + k * (256 * REP * 4) + (x << (2 + kLogRep)) + laneoff);
    } else {
      uint32_t v = *(const uint32_t *)(base + (x << (2 + kLogRep)) + laneoff);
      return rotl32(v, 8 * k);
    }
  }

  __device__ __forceinline__ uint4 enc(uint4 in, const AesRK &rk) const {
    uint32_t c0 = in.x ^ rk.w[0], c1 = in.y ^ rk.w[1], c2 = in.z ^ rk.w[2], c3 = in.w ^ rk.w[3];
#pragma unroll
    for (int r = 1; r < 10; r++) {
      uint32_t n0 = xor3(xor3(T(0, c0 & 255u), T(1, (c1 >> 8) & 255u), T(2, (c2 >> 16) & 255u)), T(3, c3 >> 24), rk.w[4 * r + 0]);
      uint32_t n1 = xor3(xor3(T(0, c1 & 255u), T(1, (c2 >> 8) & 255u), T(2, (c3 >> 16) & 255u)), T(3, c0 >> 24), rk.w[4 * r + 1]);
      uint32_t n2 = xor3(xor3(T(0, c2 & 255u), T(1, (c3 >> 8) & 255u), T(2, (c0 >> 16) & 255u)), T(3, c1 >> 24), rk.w[4 * r + 2]);
      uint32_t n3 = xor3(xor3(T(0, c3 & 255u), T(1, (c0 >> 8) & 255u), T(2, (c1 >> 16) & 255u)), T(3, c2 >> 24), rk.w[4 * r + 3]);
      c0 = n0;
      c1 = n1;
      c2 = n2;
      c3 = n3;
    }
    uint4 o;
    o.x = ((T(3, c0 & 255u) & 0xffu) | (T(0, (c1 >> 8) & 255u) & 0xff00u) | (T(1, (c2 >> 16) & 255u) & 0xff0000u) |
           (T(2, c3 >> 24) & 0xff000000u)) ^ rk.w[40];
    o.y = ((T(3, c1 & 255u) & 0xffu) | (T(0, (c2 >> 8) & 255u) & 0xff00u) | (T(1, (c3 >> 16) & 255u) & 0xff0000u) |
           (T(2, c0 >> 24) & 0xff000000u)) ^ rk.w[41];
    o.z = ((T(3, c2 & 255u) & 0xffu) | (T(0, (c3 >> 8) & 255u) & 0xff00u) | (T(1, (c0 >> 16) & 255u) & 0xff0000u) |
           (T(2, c1 >> 24) & 0xff000000u)) ^ rk.w[42];
    o.w = ((T(3, c3 & 255u) & 0xffu) | (T(0, (c0 >> 8) & 255u) & 0xff00u) | (T(1, (c1 >> 16) & 255u) & 0xff0000u) |
           (T(2, c2 >> 24) & 0xff000000u)) ^ rk.w[43];
    return o;
  }

  // H(s) = AES_k(sigma(s)) ^ sigma(s), sigma(xL||xR) = (xL^xR)||xL, xR = words 0,1.
  __device__ __forceinline__ uint4 hash(uint4 s, const AesRK &rk) const {
    uint4 x;
    x.x = s.z;
    x.y = s.w;
    x.z = s.z ^ s.x;
    x.w = s.w ^ s.y;
    uint4 y = enc(x, rk);
    y.x ^= x.x;
    y.y ^= x.y;
    y.z ^= x.z;
    y.w ^= x.w;
    return y;
  }

  // Dealer PRF block AES_kd(idx_lo, idx_hi, field, gate).
  __device__ __forceinline__ uint4 prf(const AesRK &kd, uint32_t gate, uint32_t field, uint64_t idx) const {
    uint4 b;
    b.x = uint32_t(idx);
    b.y = uint32_t(idx >> 32);
    b.z = field;
    b.w = gate;
    return enc(b, kd);
  }
};

// T0 alone, 64 copies per entry: entry x, copy j at byte address 256*x + 4*j.
// Lane l reads copy l mod 64, so a wavefront never has two lanes on one bank,
// and the byte address of "T0[byte k of c]" for this lane is one v_perm_b32 of
// (c, lane word): byte 0 = (lane*4) mod 256, byte 1 = byte k of c, bytes 2..3 = 0.
// T1..T3 are rotations of T0 (v_alignbit_b32), three-input XORs are
// v_bitop3_b32, and the last round gathers the S-box bytes (byte 1 of T0) with
// v_perm_b32.  The hash folds sigma into the first AddRoundKey and the
// feed-forward into the last one.  (Holding T1 as a second 64 KiB table saves
// two rotations per column but leaves room for only one workgroup per CU; it
// measured slower.)
struct AesPerm {
  static constexpr int kWords = 256 * 64;
  static constexpr int kBytes = kWords * 4;

  const char *base;
  uint32_t lane4;  // (lane * 4) mod 256

  // 16-byte stores: 16 per entry (its 64 copies), kWords / 4 in all
  __device__ static void fill(uint32_t *lds) {
    uint4 *l4 = reinterpret_cast<uint4 *>(lds);
    for (int q = threadIdx.x; q < kWords / 4; q += blockDim.x) {
      const uint32_t v = c_T0.v[q >> 4];
      l4[q] = make_uint4(v, v, v, v);
    }
    __syncthreads();
  }

  __device__ AesPerm(const uint32_t *lds) : base((const char *)lds) { lane4 = (threadIdx.x & 63u) * 4u; }

  // T0[byte K of c]
  template <int t, int K>
  __device__ __forceinline__ uint32_t L(uint32_t c) const {
    static_assert(t == 0, "one table");
    const uint32_t addr = __builtin_amdgcn_perm(c, lane4, 0x0c0c0000u | ((4u + K) << 8));
    return *(const uint32_t *)(base + addr);
  }
  // rotl(v, 8k) as a funnel shift
  template <int K>
  __device__ __forceinline__ static uint32_t rot(uint32_t v) {
    return K == 0 ? v : __builtin_amdgcn_alignbit(v, v, 32 - 8 * K);
  }
  __device__ __forceinline__ uint32_t col(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t k) const {
    return xor3(xor3(L<0, 0>(a), rot<1>(L<0, 1>(b)), rot<2>(L<0, 2>(c))), rot<3>(L<0, 3>(d)), k);
  }
  // S[byte 0 of a] | S[byte 1 of b] << 8 | S[byte 2 of c] << 16 | S[byte 3 of d] << 24
  __device__ __forceinline__ uint32_t last(uint32_t a, uint32_t b, uint32_t c, uint32_t d) const {
    const uint32_t lo = __builtin_amdgcn_perm(L<0, 1>(b), L<0, 0>(a), 0x0c0c0501u);
    const uint32_t hi = __builtin_amdgcn_perm(L<0, 3>(d), L<0, 2>(c), 0x0c0c0501u);
    return (hi << 16) | lo;
  }

  // rounds 1..9 on the whitened state
  __device__ __forceinline__ void rounds(uint32_t &c0, uint32_t &c1, uint32_t &c2, uint32_t &c3,
                                         const AesRK &rk) const {
#pragma unroll
    for (int r = 1; r < 10; r++) {
      const uint32_t n0 = col(c0, c1, c2, c3, rk.w[4 * r + 0]);
      const uint32_t n1 = col(c1, c2, c3, c0, rk.w[4 * r + 1]);
      const uint32_t n2 = col(c2, c3, c0, c1, rk.w[4 * r + 2]);
      const uint32_t n3 = col(c3, c0, c1, c2, rk.w[4 * r + 3]);
      c0 = n0;
      c1 = n1;
      c2 = n2;
      c3 = n3;
    }
  }

  __device__ __forceinline__ uint4 enc(uint4 in, const AesRK &rk) const {
    uint32_t c0 = in.x ^ rk.w[0], c1 = in.y ^ rk.w[1], c2 = in.z ^ rk.w[2], c3 = in.w ^ rk.w[3];
    rounds(c0, c1, c2, c3, rk);
    uint4 o;
    o.x = last(c0, c1, c2, c3) ^ rk.w[40];
    o.y = last(c1, c2, c3, c0) ^ rk.w[41];
    o.z = last(c2, c3, c0, c1) ^ rk.w[42];
    o.w = last(c3, c0, c1, c2) ^ rk.w[43];
    return o;
  }

  // H(s) = AES_k(sigma(s)) ^ sigma(s), sigma(xL||xR) = (xL^xR)||xL, xR = words 0,1
  __device__ __forceinline__ uint4 hash(uint4 s, const AesRK &rk) const {
    uint32_t c0 = s.z ^ rk.w[0], c1 = s.w ^ rk.w[1];
    uint32_t c2 = xor3(s.z, s.x, rk.w[2]), c3 = xor3(s.w, s.y, rk.w[3]);
    rounds(c0, c1, c2, c3, rk);
    uint4 o;
    o.x = xor3(last(c0, c1, c2, c3), rk.w[40], s.z);
    o.y = xor3(last(c1, c2, c3, c0), rk.w[41], s.w);
    o.z = xor3(last(c2, c3, c0, c1), rk.w[42], s.z) ^ s.x;
    o.w = xor3(last(c3, c0, c1, c2), rk.w[43], s.w) ^ s.y;
    return o;
  }

  // Dealer PRF block AES_kd(idx_lo, idx_hi, field, gate).
  __device__ __forceinline__ uint4 prf(const AesRK &kd, uint32_t gate, uint32_t field, uint64_t idx) const {
    uint4 b;
    b.x = uint32_t(idx);
    b.y = uint32_t(idx >> 32);
    b.z = field;
    b.w = gate;
    return enc(b, kd);
  }
};

// T0 and T1 = rotl(T0, 8) in one 64 KiB table, 32 copies each: entry x holds
// T0[x] at byte address 256*x + 4*j and T1[x] at 256*x + 128 + 4*j, copy j.
// Lane l reads copy l mod 32, so the two half-waves, which the LDS serves in
// turn, never have two lanes on one bank.  One v_perm_b32 gives the address of
// "T0[byte k of c]" (byte 0 = 4 (lane mod 32), byte 1 = byte k of c); T1 is the
// same address plus the read's immediate offset 128.  A column is then
// T0[a] ^ T1[b] ^ rotl(T0[c] ^ T1[d] ^ rotl(k, 16), 16): 4 address permutes, one
// rotation and two three-input XORs (28 VALU per round against 36 with T0 alone).
struct AesPerm2 {
  static constexpr int kWords = 256 * 64;
  static constexpr int kBytes = kWords * 4;

  const char *base;
  uint32_t lane4;  // (lane * 4) mod 128

  // 16-byte stores: entry x is 8 stores of T0[x], then 8 of T1[x]
  __device__ static void fill(uint32_t *lds) {
    uint4 *l4 = reinterpret_cast<uint4 *>(lds);
    for (int q = threadIdx.x; q < kWords / 4; q += blockDim.x) {
      const uint32_t t = c_T0.v[q >> 4];
      const uint32_t v = (q & 8) ? rotl32(t, 8) : t;
      l4[q] = make_uint4(v, v, v, v);
    }
    __syncthreads();
  }

  __device__ AesPerm2(const uint32_t *lds) : base((const char *)lds) { lane4 = (threadIdx.x & 31u) * 4u; }

  // byte address of entry (byte K of c), copy lane mod 32
  template <int K>
  __device__ __forceinline__ uint32_t adr(uint32_t c) const {
    return __builtin_amdgcn_perm(c, lane4, 0x0c0c0000u | ((4u + K) << 8));
  }
  template <int K>
  __device__ __forceinline__ uint32_t t0(uint32_t c) const {
    return *(const uint32_t *)(base + adr<K>(c));
  }
  template <int K>
  __device__ __forceinline__ uint32_t t1(uint32_t c) const {
    return *(const uint32_t *)(base + adr<K>(c) + 128);
  }
  // rotl(T0[c] ^ T1[d] ^ rotl(k, 16), 16) = T2[c] ^ T3[d] ^ k; the round key is
  // uniform, so its rotation is scalar work
  __device__ __forceinline__ uint32_t col(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t k) const {
    const uint32_t h = xor3(t0<2>(c), t1<3>(d), (k << 16) | (k >> 16));
    return xor3(t0<0>(a), t1<1>(b), __builtin_amdgcn_alignbit(h, h, 16));
  }
  // S[byte 0 of a] | S[byte 1 of b] << 8 | S[byte 2 of c] << 16 | S[byte 3 of d] << 24
  // (S[x] is byte 1 of T0[x])
  __device__ __forceinline__ uint32_t last(uint32_t a, uint32_t b, uint32_t c, uint32_t d) const {
    const uint32_t lo = __builtin_amdgcn_perm(t0<1>(b), t0<0>(a), 0x0c0c0501u);
    const uint32_t hi = __builtin_amdgcn_perm(t0<3>(d), t0<2>(c), 0x0c0c0501u);
    return (hi << 16) | lo;
  }

  __device__ __forceinline__ void rounds(uint32_t &c0, uint32_t &c1, uint32_t &c2, uint32_t &c3,
                                         const AesRK &rk) const {
#pragma unroll
    for (int r = 1; r < 10; r++) {
      const uint32_t n0 = col(c0, c1, c2, c3, rk.w[4 * r + 0]);
      const uint32_t n1 = col(c1, c2, c3, c0, rk.w[4 * r + 1]);
      const uint32_t n2 = col(c2, c3, c0, c1, rk.w[4 * r + 2]);
      const uint32_t n3 = col(c3, c0, c1, c2, rk.w[4 * r + 3]);
      c0 = n0;
      c1 = n1;
      c2 = n2;
      c3 = n3;
    }
  }

  __device__ __forceinline__ uint4 enc(uint4 in, const AesRK &rk) const {
    uint32_t c0 = in.x ^ rk.w[0], c1 = in.y ^ rk.w[1], c2 = in.z ^ rk.w[2], c3 = in.w ^ rk.w[3];
    rounds(c0, c1, c2, c3, rk);
    uint4 o;
    o.x = last(c0, c1, c2, c3) ^ rk.w[40];
    o.y = last(c1, c2, c3, c0) ^ rk.w[41];
    o.z = last(c2, c3, c0, c1) ^ rk.w[42];
    o.w = last(c3, c0, c1, c2) ^ rk.w[43];
    return o;
  }

  // H(s) = AES_k(sigma(s)) ^ sigma(s), sigma(xL||xR) = (xL^xR)||xL, xR = words 0,1
  __device__ __forceinline__ uint4 hash(uint4 s, const AesRK &rk) const {
    uint32_t c0 = s.z ^ rk.w[0], c1 = s.w ^ rk.w[1];
    uint32_t c2 = xor3(s.z, s.x, rk.w[2]), c3 = xor3(s.w, s.y, rk.w[3]);
    rounds(c0, c1, c2, c3, rk);
    uint4 o;
    o.x = xor3(last(c0, c1, c2, c3), rk.w[40], s.z);
    o.y = xor3(last(c1, c2, c3, c0), rk.w[41], s.w);
    o.z = xor3(last(c2, c3, c0, c1), rk.w[42], s.z) ^ s.x;
    o.w = xor3(last(c3, c0, c1, c2), rk.w[43], s.w) ^ s.y;
    return o;
  }

  // hash of two independent blocks, their rounds side by side: one thread's
  // two AES chains give the scheduler table reads of one to issue while the
  // other's XORs wait
  __device__ __forceinline__ void hash2(uint4 s, uint4 u, const AesRK &rk, uint4 *hs, uint4 *hu) const {
    uint32_t a0 = s.z ^ rk.w[0], a1 = s.w ^ rk.w[1];
    uint32_t a2 = xor3(s.z, s.x, rk.w[2]), a3 = xor3(s.w, s.y, rk.w[3]);
    uint32_t b0 = u.z ^ rk.w[0], b1 = u.w ^ rk.w[1];
    uint32_t b2 = xor3(u.z, u.x, rk.w[2]), b3 = xor3(u.w, u.y, rk.w[3]);
#pragma unroll
    for (int r = 1; r < 10; r++) {
      const uint32_t n0 = col(a0, a1, a2, a3, rk.w[4 * r + 0]);
      const uint32_t m0 = col(b0, b1, b2, b3, rk.w[4 * r + 0]);
      const uint32_t n1 = col(a1, a2, a3, a0, rk.w[4 * r + 1]);
      const uint32_t m1 = col(b1, b2, b3, b0, rk.w[4 * r + 1]);
      const uint32_t n2 = col(a2, a3, a0, a1, rk.w[4 * r + 2]);
      const uint32_t m2 = col(b2, b3, b0, b1, rk.w[4 * r + 2]);
      const uint32_t n3 = col(a3, a0, a1, a2, rk.w[4 * r + 3]);
      const uint32_t m3 = col(b3, b0, b1, b2, rk.w[4 * r + 3]);
      a0 = n0, a1 = n1, a2 = n2, a3 = n3;
      b0 = m0, b1 = m1, b2 = m2, b3 = m3;
    }
    hs->x = xor3(last(a0, a1, a2, a3), rk.w[40], s.z);
    hu->x = xor3(last(b0, b1, b2, b3), rk.w[40], u.z);
    hs->y = xor3(last(a1, a2, a3, a0), rk.w[41], s.w);
    hu->y = xor3(last(b1, b2, b3, b0), rk.w[41], u.w);
    hs->z = xor3(last(a2, a3, a0, a1), rk.w[42], s.z) ^ s.x;
    hu->z = xor3(last(b2, b3, b0, b1), rk.w[42], u.z) ^ u.x;
    hs->w = xor3(last(a3, a0, a1, a2), rk.w[43], s.w) ^ s.y;
    hu->w = xor3(last(b3, b0, b1, b2), rk.w[43], u.w) ^ u.y;
  }

  // Dealer PRF block AES_kd(idx_lo, idx_hi, field, gate).
  __device__ __forceinline__ uint4 prf(const AesRK &kd, uint32_t gate, uint32_t field, uint64_t idx) const {
    uint4 b;
    b.x = uint32_t(idx);
    b.y = uint32_t(idx >> 32);
    b.z = field;
    b.w = gate;
    return enc(b, kd);
  }
};

// Quad-lane AES on the AesPerm2 table, for latency-bound launches: four
// consecutive lanes (a quad) hold one block, lane j its column c_j.  A round has
// each lane look up its own column's four bytes -- A = T0[b0], B = T1[b1],
// C = T0[b2], D = T1[b3] -- and take the other three terms of its new column from
// the quad's other lanes (DPP quad permutes):
//   n_j = A_j ^ B_(j+1) ^ rotl(C_(j+2) ^ D_(j+3) ^ rotl(k_j, 16), 16),
// 10 VALU instructions and 4 table reads per lane and round instead of 28 and 16
// for one lane per block, so a round's dependent chain is shorter.  Every lane of
// a quad must run the same code (the permutes read the other three lanes).
struct AesQuad {
  const AesPerm2 &t;
  uint32_t j;  // the lane's column (lane mod 4)
  __device__ AesQuad(const AesPerm2 &tab) : t(tab), j(threadIdx.x & 3u) {}

  // DPP quad permutes: the value of lane (j + d) mod 4 of the quad
  __device__ __forceinline__ static uint32_t from1(uint32_t v) { return __builtin_amdgcn_mov_dpp(int(v), 0x39, 0xf, 0xf, false); }
  __device__ __forceinline__ static uint32_t from2(uint32_t v) { return __builtin_amdgcn_mov_dpp(int(v), 0x4e, 0xf, 0xf, false); }
  __device__ __forceinline__ static uint32_t from3(uint32_t v) { return __builtin_amdgcn_mov_dpp(int(v), 0x93, 0xf, 0xf, false); }
  // the value of the quad's lane 0, and the xor over the quad
  __device__ __forceinline__ static uint32_t lane0(uint32_t v) { return __builtin_amdgcn_mov_dpp(int(v), 0x00, 0xf, 0xf, false); }
  __device__ __forceinline__ static uint32_t quad_xor(uint32_t v) {
    v ^= __builtin_amdgcn_mov_dpp(int(v), 0xb1, 0xf, 0xf, false);  // lanes 1,0,3,2
    return v ^ __builtin_amdgcn_mov_dpp(int(v), 0x4e, 0xf, 0xf, false);
  }

  // The lane's round-key words of rk: k[0] and k[10] as they are, k[1..9]
  // rotated by 16 (the rotation the round folds in).
  struct Keys {
    uint32_t k[11];
  };
  __device__ __forceinline__ Keys keys(const AesRK &rk) const {
    Keys o;
#pragma unroll
    for (int r = 0; r < 11; r++) {
      const uint32_t w = rk.w[4 * r + int(j)];
      o.k[r] = (r == 0 || r == 10) ? w : ((w << 16) | (w >> 16));
    }
    return o;
  }

  __device__ __forceinline__ uint32_t enc(uint32_t c, const Keys &k) const {
    c ^= k.k[0];
#pragma unroll
    for (int r = 1; r < 10; r++) {
      const uint32_t a = t.t0<0>(c), b = t.t1<1>(c), cc = t.t0<2>(c), d = t.t1<3>(c);
      const uint32_t h = xor3(from2(cc), from3(d), k.k[r]);
      c = xor3(a, from1(b), __builtin_amdgcn_alignbit(h, h, 16));
    }
    // last round: S[x] is byte 1 of T0[x]; the lane packs the S bytes of its own
    // column, byte i of the new column comes from lane j + i
    const uint32_t lo = __builtin_amdgcn_perm(t.t0<1>(c), t.t0<0>(c), 0x0c0c0501u);
    const uint32_t hi = __builtin_amdgcn_perm(t.t0<3>(c), t.t0<2>(c), 0x0c0c0501u);
    const uint32_t P = (hi << 16) | lo;
    const uint32_t x01 = __builtin_amdgcn_perm(from1(P), P, 0x0c0c0500u);       // bytes 0 (own), 1 (lane j+1)
    const uint32_t x23 = __builtin_amdgcn_perm(from3(P), from2(P), 0x07020c0cu);  // bytes 2 (lane j+2), 3 (j+3)
    return (x01 | x23) ^ k.k[10];
  }

  // H(s) = AES_k(sigma(s)) ^ sigma(s), sigma(xL||xR) = (xL^xR)||xL, xR = words 0,1:
  // sigma_j = s_(j^2), and ^ s_j for j >= 2
  __device__ __forceinline__ uint32_t hash(uint32_t s, const Keys &k) const {
    const uint32_t sg = from2(s) ^ ((j & 2u) ? s : 0u);
    return enc(sg, k) ^ sg;
  }
};

// NT = 0 selects the permute-addressed single table (REP must be 64); NT = 2
// (REP 32) the interleaved pair.
template <int NT, int REP>
struct AesSel {
  using type = AesTab<NT, REP>;
};
template <>
struct AesSel<0, 64> {
  using type = AesPerm;
};
// NT = 2, REP = 32: T0 and T1 interleaved in one table (AesPerm2)
template <>
struct AesSel<2, 32> {
  using type = AesPerm2;
};
template <int NT, int REP>
using AesLds = typename AesSel<NT, REP>::type;

// a ^ (b & m) in one v_bitop3_b32 (truth table 0x78 = 0xf0 ^ (0xcc & 0xaa))
__device__ __forceinline__ uint32_t xor_and(uint32_t a, uint32_t b, uint32_t m) {
  return __builtin_amdgcn_bitop3_b32(a, b, m, 0x78);
}
__device__ __forceinline__ uint4 xor_and4(uint4 a, uint4 b, uint32_t m) {
  return make_uint4(xor_and(a.x, b.x, m), xor_and(a.y, b.y, m), xor_and(a.z, b.z, m), xor_and(a.w, b.w, m));
}
__device__ __forceinline__ uint4 xor4(uint4 a, uint4 b) {
  return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w);
}
__device__ __forceinline__ uint4 and4(uint4 a, uint32_t m) {
  return make_uint4(a.x & m, a.y & m, a.z & m, a.w & m);
}

// parity of the bits of b at positions > pos, pos in [0, 127]
__device__ __forceinline__ uint32_t parity_above(uint4 b, uint32_t pos) {
  uint32_t acc = 0;
  const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    uint32_t lo = 32u * k;
    uint32_t m;
    if (pos < lo)
      m = 0xffffffffu;
    else if (pos >= lo + 31)
      m = 0u;
    else
      m = 0xffffffffu << (pos - lo + 1);
    acc ^= w[k] & m;
  }
  return __popc(acc) & 1u;
}

}  // namespace mpcx
