// gemm.h -- host-side launchers of the ring GEMMs (gemm.hip).
#pragma once
#include "kernels.h"

namespace mpcx {

// ---------------- ring GEMM ----------------
// C[b] = Cin[b] + sign * (A1[b] - A2[b]) (B1[b] - B2[b]) mod 2^bw.
// Any of A2, B2, Cin may be null.  Batch strides in elements (0 = shared).
template <typename T>
struct GemmArgs {
  int M = 0, N = 0, K = 0, batch = 1;
  const T *A1 = nullptr, *A2 = nullptr, *B1 = nullptr, *B2 = nullptr, *Cin = nullptr;
  T *C = nullptr;
  size_t sA = 0, sB = 0, sC = 0;
  int sign = 1;
  int ksplit = 1;  // set by launch_gemm: K slices accumulated with atomic adds
  // C already holds zeros (Cin null): split-K slices add into it without a
  // clearing launch first
  bool c_zero = false;
  // optional second K segment of the same shapes and strides:
  // C = Cin + sign * ((A1 - A2)(B1 - B2) + A1b B1b)
  const T *A1b = nullptr, *B1b = nullptr;
};
template <typename T>
hipError_t launch_gemm(const Launch &L, const GemmArgs<T> &g);
// Two independent products in one launch where the matrix-core path applies
// (the Beaver products of both parties of an SxS gate), else one after another.
template <typename T>
hipError_t launch_gemm_pair(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1);
// Both parties' products of an SxS gate, reconstructed: out = C0 + C1 (batch x
// M x N, contiguous).  One launch (k_sxs_fused) for the pair as the SxS gates
// form it; otherwise launch_gemm_pair into g0.C and g1.C, then the sum.
template <typename T>
hipError_t launch_gemm_pair_sum(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1, T *out);

// ---------------- Z_2^32 SxS gate on balanced-digit planes ----------------
// Both parties' Beaver products of an SxS gate and their sum, with party 0's
// product expanded ((A^ - RA0)(B^ - RB0) = A^ B^ - A^ RB0 - RA0 B^ + RA0 RB0):
//   party 0:  A^ B^ - A^ RB0 - RA0 B^ + K0,   K0 = RA0 RB0 + C0
//   party 1:  C1 - A^ RB1 - RA1 B^
// as five products summed in the same accumulators, C = party 0 + party 1.
// A^ ([batch][M][K]) and B^ ([batch][K][N]) are the gate's ring words; the key
// operands are planes of balanced base-256 digits (ring_digits) formed from
// each party's key once per key set: na = digits of -RA0, -RA1 ([batch][M][K]),
// nb = digits of -RB0, -RB1 transposed ([batch][N][K]); k0 = K0 and c1 = C1
// ([batch][M][N]).  K a multiple of 4.
struct SxsDigitArgs {
  int M = 0, N = 0, K = 0, batch = 0;
  const uint32_t *ahat = nullptr, *bhat = nullptr;
  const uint32_t *na[2] = {nullptr, nullptr};
  const uint32_t *nb[2] = {nullptr, nullptr};
  const uint32_t *k0 = nullptr, *c1 = nullptr;
  uint32_t *C = nullptr;
};
hipError_t launch_sxs_digits(const Launch &L, const SxsDigitArgs &g);
// dst[i] = digits of src[i] (of -src[i] when neg), n words
hipError_t launch_ring_digits(const Launch &L, size_t n, const uint32_t *src, bool neg, uint32_t *dst);
// dst[b][j][i] = digits of src[b][i][j] (of its negation when neg): batch
// matrices of R x Ccols words, transposed
hipError_t launch_ring_digits_t(const Launch &L, int batch, int R, int Ccols, const uint32_t *src, bool neg,
                                uint32_t *dst);

}  // namespace mpcx
