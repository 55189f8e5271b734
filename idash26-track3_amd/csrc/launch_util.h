// launch_util.h -- helpers shared by the kernel files of libmpcx: the AES LDS
// variant dispatch, the two-party workgroup rows, grid sizing and small
// device-side accessors.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace mpcx {

template <int NT, int REP>
struct V {
  static constexpr int nt = NT, rep = REP;
};

template <class Fn>
inline hipError_t with_variant(const Launch &L, Fn &&fn) {
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
inline unsigned party_rows(const Launch &L) { return L.party < 0 ? 2u : 1u; }
inline int party_base(const Launch &L) { return L.party < 0 ? 0 : L.party; }
inline int variant_block(const Launch &L) {
  if (L.aes_block > 0) return L.aes_block;
  int n;
  const AesVariant *v = aes_variants(&n);
  return (L.aes_variant >= 0 && L.aes_variant < n) ? v[L.aes_variant].block : 256;
}

template <typename K>
inline int grid_for(K kernel, int block, size_t n, int num_cu) {
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

}  // namespace mpcx
