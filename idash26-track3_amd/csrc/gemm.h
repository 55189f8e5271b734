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

}  // namespace mpcx
