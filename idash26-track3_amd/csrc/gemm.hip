// gemm.hip -- ring GEMMs of the secure-inference online path on the int8 matrix
// cores of gfx950 (and a VALU fallback), both rings.
//
// Reference interface: gpuMatmul / gpuKeygenMatmul behind DDGOrcaBase::matmul
// (gpu_mpc/ddg_orca_base.h:170-271, 394-469), the per-sample SxS loop of
// sytorch's _MatMul (layers.h:67-93).  A product C = Cin + sign (A1 - A2)(B1 - B2)
// (+ A1b B1b) mod 2^bw with optional masks, a second K segment and batches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "gemm.h"
#include "launch_util.h"

namespace mpcx {

// ---------------------------------------------------------------------------
// ring GEMM: 64x64 tile per 256-thread block, 4x4 outputs per thread,
// K staged through LDS in slices of 16.  Integer multiply-add on the VALU
// (v_mul_lo_u32 / v_mad_u64_u32); operand differences are applied on load.
// Skinny products (the FC layers: M = batch) would leave most CUs idle, so K is
// split across blocks (gridDim.z = batch * ksplit) and the partial sums are
// added with atomics into C, which is first set to Cin (or 0): addition mod
// 2^bw is associative and commutative, so the result does not depend on the
// order in which the slices land.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs<T> g) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ T As[BK][BM + 1];
  __shared__ T Bs[BK][BN + 1];
  const int bz = blockIdx.z / g.ksplit, kz = blockIdx.z % g.ksplit;
  const int kchunk = ((g.K + g.ksplit - 1) / g.ksplit + BK - 1) / BK * BK;
  const int kbeg = kz * kchunk, kend = min(g.K, kbeg + kchunk);
  const T *A1 = g.A1 + size_t(bz) * g.sA;
  const T *A2 = g.A2 ? g.A2 + size_t(bz) * g.sA : nullptr;
  const T *B1 = g.B1 + size_t(bz) * g.sB;
  const T *B2 = g.B2 ? g.B2 + size_t(bz) * g.sB : nullptr;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int tid = threadIdx.x;
  const int tr = tid / 16, tc = tid % 16;  // 16 x 16 thread grid, 4 x 4 each
  T acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0;
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int e = tid + r * 256;  // 0..1023
      // A tile: 64 rows x 16 cols, row-major source
      const int am = e / BK, ak = e % BK;
      const int gm = m0 + am, gk = k0 + ak;
      T av = 0;
      if (gm < g.M && gk < kend) {
        const size_t idx = size_t(gm) * g.K + gk;
        av = A1[idx];
        if (A2) av -= A2[idx];
      }
      As[ak][am] = av;
      // B tile: 16 rows x 64 cols
      const int bk = e / BN, bn = e % BN;
      const int gk2 = k0 + bk, gn = n0 + bn;
      T bv = 0;
      if (gk2 < kend && gn < g.N) {
        const size_t idx = size_t(gk2) * g.N + gn;
        bv = B1[idx];
        if (B2) bv -= B2[idx];
      }
      Bs[bk][bn] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk++) {
      T a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = As[kk][tr * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = Bs[kk][tc * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
  T *C = g.C + size_t(bz) * g.sC;
  const T *Cin = g.Cin ? g.Cin + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int gm = m0 + tr * 4 + i;
    if (gm >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int gn = n0 + tc * 4 + j;
      if (gn >= g.N) continue;
      const size_t idx = size_t(gm) * g.N + gn;
      const T v = g.sign < 0 ? T(T(0) - acc[i][j]) : acc[i][j];
      if (g.ksplit > 1) {
        if constexpr (sizeof(T) == 4)
          atomicAdd(reinterpret_cast<unsigned int *>(&C[idx]), static_cast<unsigned int>(v));
        else
          atomicAdd(reinterpret_cast<unsigned long long *>(&C[idx]), static_cast<unsigned long long>(v));
      } else {
        C[idx] = Cin ? T(v + Cin[idx]) : v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// ring GEMM over Z_2^32 on the int8 matrix cores (v_mfma_i32_16x16x64_i8).
// Balanced base-256 digits: the bytes of y = (a + 0x80808080) ^ 0x80808080,
// read as signed int8 d_0..d_3 in [-128, 127], satisfy a = sum_p d_p 2^(8p)
// mod 2^32 (y - 0x80808080 = a, and byte ^ 0x80 read as int8 is byte - 128).
// Hence a*b mod 2^32 = sum_{s<4} 2^(8s) sum_{p+q=s} a_p b_q.  One MFMA takes 16
// operand words per row and column (4 digit bytes each); with the row words'
// digits permuted to (a_s, a_{s-1}, .., a_0, 0, ..) it returns the shift-s sum
// over those 16 words, so four MFMAs (s = 0..3) cover 16 k.  The int32
// accumulators wrap, and only acc_s mod 2^(32-8s) enters the result.
// Tile: 64 x 64 per 256-thread block; wave w owns rows 16w..16w+15 and the four
// 16-column MFMA tiles; K staged through LDS in slices of 64 words (A as
// [m][k], B transposed to [n][k], rows padded to 68 words).  Split-K and the
// epilogue follow k_gemm.
// ---------------------------------------------------------------------------
typedef int v4i_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t ring_digits(uint32_t a) { return (a + 0x80808080u) ^ 0x80808080u; }

// One 64 x 64 output tile of problem g; z = batch * ksplit + K slice.  A second
// K segment (A1b, B1b) starts at the K tile after the first segment's last one,
// so every 64-wide K tile reads one segment only.  VA / VB: rows of A / B are
// read as 16-byte words (K resp. N a multiple of 4, operands 16-byte aligned).
template <bool VA, bool VB>
__device__ __forceinline__ void gemm_mfma_tile(const GemmArgs<uint32_t> &g, int z, uint32_t *As, uint32_t *Bt) {
  constexpr int BM = 64, BN = 64, BK = 64, LD = BK + 4;
  const int Kp = (g.K + BK - 1) / BK * BK;
  const int Kt = g.A1b ? Kp + g.K : g.K;
  const int bz = z / g.ksplit, kz = z % g.ksplit;
  const int kchunk = ((Kt + g.ksplit - 1) / g.ksplit + BK - 1) / BK * BK;
  const int kbeg = kz * kchunk, kend = min(Kt, kbeg + kchunk);
  const uint32_t *A1 = g.A1 + size_t(bz) * g.sA;
  const uint32_t *A2 = g.A2 ? g.A2 + size_t(bz) * g.sA : nullptr;
  const uint32_t *B1 = g.B1 + size_t(bz) * g.sB;
  const uint32_t *B2 = g.B2 ? g.B2 + size_t(bz) * g.sB : nullptr;
  const uint32_t *A1b = g.A1b ? g.A1b + size_t(bz) * g.sA : nullptr;
  const uint32_t *B1b = g.B1b ? g.B1b + size_t(bz) * g.sB : nullptr;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  if (m0 >= g.M || n0 >= g.N) return;  // the grid spans the larger of two problems
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  v4i_t acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int q = 0; q < 4; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
  // Each thread stages 16 words of the A tile and 16 of the B tile (B stored
  // transposed, Bt[n][k]).  Scalar layout: word r at row hb + 4r, column lo;
  // 16-byte layout: words 4r..4r+3 at row (tid >> 4) + 16r, columns 4 (tid & 15) + 0..3.
  // The next K tile is loaded into registers (addresses clamped in bounds, the
  // masking and the A1 - A2 difference applied when stored to LDS) while the
  // matrix cores work on the current one.
  uint32_t ra[16], ra2[16], rb[16], rb2[16];
  const int lo = tid & 63, hb = tid >> 6, vq = tid & 15, vr = tid >> 4;
  struct Seg {
    const uint32_t *a1, *a2, *b1, *b2;
    int kk, klim;
  };
  auto seg_of = [&](int k0) {
    const bool second = k0 >= Kp;  // uniform over the block
    Seg sg;
    sg.a1 = second ? A1b : A1;
    sg.a2 = second ? nullptr : A2;
    sg.b1 = second ? B1b : B1;
    sg.b2 = second ? nullptr : B2;
    sg.kk = second ? k0 - Kp : k0;
    sg.klim = min(g.K, kend - (second ? Kp : 0));
    return sg;
  };
  // (row, column) of staged word r of A and of B, relative to the tile origin
  auto a_rc = [&](int r, int &row, int &col) {
    if constexpr (VA) {
      row = vr + 16 * (r >> 2);
      col = 4 * vq + (r & 3);
    } else {
      row = hb + 4 * r;
      col = lo;
    }
  };
  auto b_rc = [&](int r, int &row, int &col) {  // row = k, col = n
    if constexpr (VB) {
      row = vr + 16 * (r >> 2);
      col = 4 * vq + (r & 3);
    } else {
      row = hb + 4 * r;
      col = lo;
    }
  };
  auto load = [&](int k0) {
    const Seg sg = seg_of(k0);
#pragma unroll
    for (int r = 0; r < 16; r += VA ? 4 : 1) {
      int row, col;
      a_rc(r, row, col);
      const int gm = m0 + row, gk = sg.kk + col;
      const size_t idx = (gm < g.M && gk < sg.klim) ? size_t(gm) * g.K + gk : 0;
      if constexpr (VA) {
        const uint4 v = *reinterpret_cast<const uint4 *>(sg.a1 + idx);
        ra[r] = v.x, ra[r + 1] = v.y, ra[r + 2] = v.z, ra[r + 3] = v.w;
      } else {
        ra[r] = sg.a1[idx];
      }
    }
    if (sg.a2) {
#pragma unroll
      for (int r = 0; r < 16; r += VA ? 4 : 1) {
        int row, col;
        a_rc(r, row, col);
        const int gm = m0 + row, gk = sg.kk + col;
        const size_t idx = (gm < g.M && gk < sg.klim) ? size_t(gm) * g.K + gk : 0;
        if constexpr (VA) {
          const uint4 v = *reinterpret_cast<const uint4 *>(sg.a2 + idx);
          ra2[r] = v.x, ra2[r + 1] = v.y, ra2[r + 2] = v.z, ra2[r + 3] = v.w;
        } else {
          ra2[r] = sg.a2[idx];
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) ra2[r] = 0;
    }
#pragma unroll
    for (int r = 0; r < 16; r += VB ? 4 : 1) {
      int row, col;
      b_rc(r, row, col);
      const int gk = sg.kk + row, gn = n0 + col;
      const size_t idx = (gk < sg.klim && gn < g.N) ? size_t(gk) * g.N + gn : 0;
      if constexpr (VB) {
        const uint4 v = *reinterpret_cast<const uint4 *>(sg.b1 + idx);
        rb[r] = v.x, rb[r + 1] = v.y, rb[r + 2] = v.z, rb[r + 3] = v.w;
      } else {
        rb[r] = sg.b1[idx];
      }
    }
    if (sg.b2) {
#pragma unroll
      for (int r = 0; r < 16; r += VB ? 4 : 1) {
        int row, col;
        b_rc(r, row, col);
        const int gk = sg.kk + row, gn = n0 + col;
        const size_t idx = (gk < sg.klim && gn < g.N) ? size_t(gk) * g.N + gn : 0;
        if constexpr (VB) {
          const uint4 v = *reinterpret_cast<const uint4 *>(sg.b2 + idx);
          rb2[r] = v.x, rb2[r + 1] = v.y, rb2[r + 2] = v.z, rb2[r + 3] = v.w;
        } else {
          rb2[r] = sg.b2[idx];
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) rb2[r] = 0;
    }
  };
  // K columns past klim and rows past M / N are staged as zeros
  auto store = [&](int k0) {
    const Seg sg = seg_of(k0);
#pragma unroll
    for (int r = 0; r < 16; r++) {
      int row, col;
      a_rc(r, row, col);
      const bool in = m0 + row < g.M && sg.kk + col < sg.klim;
      As[row * LD + col] = in ? ring_digits(ra[r] - ra2[r]) : 0u;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      int row, col;
      b_rc(r, row, col);
      const bool in = sg.kk + row < sg.klim && n0 + col < g.N;
      Bt[col * LD + row] = in ? ring_digits(rb[r] - rb2[r]) : 0u;
    }
  };
  if (kbeg < kend) load(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    store(k0);
    __syncthreads();
    if (k0 + BK < kend) load(k0 + BK);
#pragma unroll
    for (int kc = 0; kc < BK / 16; kc++) {
      const uint4 a = *reinterpret_cast<const uint4 *>(&As[(wave * 16 + li) * LD + kc * 16 + lg * 4]);
      v4i_t as[4];
      // byte p of the shift-s word: digit s-p of the row word (0x0c selects a zero byte)
      constexpr uint32_t sel[4] = {0x0c0c0c00u, 0x0c0c0001u, 0x0c000102u, 0x00010203u};
#pragma unroll
      for (int q = 0; q < 4; q++)
        as[q] = v4i_t{int(__builtin_amdgcn_perm(0u, a.x, sel[q])), int(__builtin_amdgcn_perm(0u, a.y, sel[q])),
                      int(__builtin_amdgcn_perm(0u, a.z, sel[q])), int(__builtin_amdgcn_perm(0u, a.w, sel[q]))};
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[(t * 16 + li) * LD + kc * 16 + lg * 4]);
        const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
        for (int q = 0; q < 4; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  uint32_t *C = g.C + size_t(bz) * g.sC;
  const uint32_t *Cin = g.Cin ? g.Cin + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int gn = n0 + t * 16 + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      // accumulator register r of lane (li, lg): row 4*lg + r, column li of the tile
      const int gm = m0 + wave * 16 + lg * 4 + r;
      if (gm >= g.M || gn >= g.N) continue;
      uint32_t v = uint32_t(acc[t][0][r]) + (uint32_t(acc[t][1][r]) << 8) + (uint32_t(acc[t][2][r]) << 16) +
                   (uint32_t(acc[t][3][r]) << 24);
      if (g.sign < 0) v = 0u - v;
      const size_t idx = size_t(gm) * g.N + gn;
      if (g.ksplit > 1)
        atomicAdd(reinterpret_cast<unsigned int *>(&C[idx]), static_cast<unsigned int>(v));
      else
        C[idx] = Cin ? v + Cin[idx] : v;
    }
  }
}

// blockIdx.z < nz0: problem g0, else problem g1 (nz = batch * ksplit of each)
template <bool VA, bool VB>
__global__ __launch_bounds__(256) void k_gemm_mfma(GemmArgs<uint32_t> g0, GemmArgs<uint32_t> g1, int nz0) {
  __shared__ __align__(16) uint32_t As[64 * 68];
  __shared__ __align__(16) uint32_t Bt[64 * 68];
  const int z = int(blockIdx.z);
  const bool second = z >= nz0;
  gemm_mfma_tile<VA, VB>(second ? g1 : g0, second ? z - nz0 : z, As, Bt);
}

// ---------------------------------------------------------------------------
// ring GEMM over Z_2^64 on the int8 matrix cores.  Eight balanced base-256
// digits per word (the bytes of (a + 0x8080..80) ^ 0x8080..80 read as int8):
// a*b mod 2^64 = sum_{s<8} 2^(8s) sum_{p+q=s} a_p b_q.  One MFMA takes 8
// operand words per row and column (8 digit bytes each); with each row word's
// digits permuted to (a_s, .., a_0, 0, ..) it returns the shift-s sum over those
// 8 words, so eight MFMAs (s = 0..7) cover 8 k.  acc_s enters bits 8s..63 of the
// result, so for s < 4 it must be exact in int32: |acc_s| <= K * 4 * 2^14, i.e.
// K < 2^15 per product (launch_gemm keeps larger K on the VALU kernel).
// Tile 64 x 64 per 256-thread block as in the Z_2^32 kernel; K slices of 32
// words (64 u32 of LDS per row, B transposed).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t ring_digits64(uint64_t a) {
  return (a + 0x8080808080808080ull) ^ 0x8080808080808080ull;
}
// v_perm_b32 selector of output bytes j0..j0+3 for shift s: digit s - j (bytes
// 0..3 of the low source word, 4..7 of the high one), 0x0c (zero) when s < j
constexpr uint32_t digit_sel(int s, int j0) {
  uint32_t v = 0;
  for (int j = 0; j < 4; j++) v |= uint32_t(s - (j0 + j) >= 0 ? s - (j0 + j) : 0x0c) << (8 * j);
  return v;
}

__device__ __forceinline__ void gemm_mfma64_tile(const GemmArgs<uint64_t> &g, int z, uint32_t *As, uint32_t *Bt) {
  constexpr int BM = 64, BN = 64, BK = 32, LD = 2 * BK + 4;  // LD in 32-bit words
  const int Kp = (g.K + BK - 1) / BK * BK;
  const int Kt = g.A1b ? Kp + g.K : g.K;
  const int bz = z / g.ksplit, kz = z % g.ksplit;
  const int kchunk = ((Kt + g.ksplit - 1) / g.ksplit + BK - 1) / BK * BK;
  const int kbeg = kz * kchunk, kend = min(Kt, kbeg + kchunk);
  const uint64_t *A1 = g.A1 + size_t(bz) * g.sA;
  const uint64_t *A2 = g.A2 ? g.A2 + size_t(bz) * g.sA : nullptr;
  const uint64_t *B1 = g.B1 + size_t(bz) * g.sB;
  const uint64_t *B2 = g.B2 ? g.B2 + size_t(bz) * g.sB : nullptr;
  const uint64_t *A1b = g.A1b ? g.A1b + size_t(bz) * g.sA : nullptr;
  const uint64_t *B1b = g.B1b ? g.B1b + size_t(bz) * g.sB : nullptr;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  if (m0 >= g.M || n0 >= g.N) return;  // the grid spans the larger of two problems
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  v4i_t acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int q = 0; q < 8; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
  // staged word r (r < 8) of A: row (tid >> 5) + 8r, column tid & 31; of B:
  // k (tid >> 6) + 4r, column tid & 63 (B stored transposed, Bt[n][k]); rows of
  // 32 consecutive 8-byte words per 32 threads.  The next K slice is loaded into
  // registers while the matrix cores work on the current one.
  uint64_t ra[8], ra2[8], rb[8], rb2[8];
  const int ar = tid >> 5, ac = tid & 31, bk = tid >> 6, bn = tid & 63;
  struct Seg {
    const uint64_t *a1, *a2, *b1, *b2;
    int kk, klim;
  };
  auto seg_of = [&](int k0) {
    const bool second = k0 >= Kp;  // uniform over the block
    Seg sg;
    sg.a1 = second ? A1b : A1;
    sg.a2 = second ? nullptr : A2;
    sg.b1 = second ? B1b : B1;
    sg.b2 = second ? nullptr : B2;
    sg.kk = second ? k0 - Kp : k0;
    sg.klim = min(g.K, kend - (second ? Kp : 0));
    return sg;
  };
  auto load = [&](int k0) {
    const Seg sg = seg_of(k0);
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int gm = m0 + ar + 8 * r, gk = sg.kk + ac;
      const size_t idx = (gm < g.M && gk < sg.klim) ? size_t(gm) * g.K + gk : 0;
      ra[r] = sg.a1[idx];
      ra2[r] = sg.a2 ? sg.a2[idx] : 0ull;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int gk = sg.kk + bk + 4 * r, gn = n0 + bn;
      const size_t idx = (gk < sg.klim && gn < g.N) ? size_t(gk) * g.N + gn : 0;
      rb[r] = sg.b1[idx];
      rb2[r] = sg.b2 ? sg.b2[idx] : 0ull;
    }
  };
  // K columns past klim and rows past M / N are staged as zeros
  auto store = [&](int k0) {
    const Seg sg = seg_of(k0);
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int row = ar + 8 * r;
      const bool in = m0 + row < g.M && sg.kk + ac < sg.klim;
      const uint64_t v = in ? ring_digits64(ra[r] - ra2[r]) : 0ull;
      *reinterpret_cast<uint2 *>(&As[row * LD + 2 * ac]) = make_uint2(uint32_t(v), uint32_t(v >> 32));
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int k = bk + 4 * r;
      const bool in = sg.kk + k < sg.klim && n0 + bn < g.N;
      const uint64_t v = in ? ring_digits64(rb[r] - rb2[r]) : 0ull;
      *reinterpret_cast<uint2 *>(&Bt[bn * LD + 2 * k]) = make_uint2(uint32_t(v), uint32_t(v >> 32));
    }
  };
  if (kbeg < kend) load(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    store(k0);
    __syncthreads();
    if (k0 + BK < kend) load(k0 + BK);
#pragma unroll
    for (int kc = 0; kc < BK / 8; kc++) {
      // lane (li, lg): words 2 lg, 2 lg + 1 of the 8-word step, as (lo, hi) pairs
      const uint4 a = *reinterpret_cast<const uint4 *>(&As[(wave * 16 + li) * LD + kc * 16 + lg * 4]);
      v4i_t as[8];
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const uint32_t lo = digit_sel(q, 0), hi = digit_sel(q, 4);
        as[q] = v4i_t{int(__builtin_amdgcn_perm(a.y, a.x, lo)), int(__builtin_amdgcn_perm(a.y, a.x, hi)),
                      int(__builtin_amdgcn_perm(a.w, a.z, lo)), int(__builtin_amdgcn_perm(a.w, a.z, hi))};
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[(t * 16 + li) * LD + kc * 16 + lg * 4]);
        const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
        for (int q = 0; q < 8; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  uint64_t *C = g.C + size_t(bz) * g.sC;
  const uint64_t *Cin = g.Cin ? g.Cin + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int gn = n0 + t * 16 + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      // accumulator register r of lane (li, lg): row 4*lg + r, column li of the tile
      const int gm = m0 + wave * 16 + lg * 4 + r;
      if (gm >= g.M || gn >= g.N) continue;
      uint64_t v = 0;
#pragma unroll
      for (int q = 0; q < 8; q++) v += uint64_t(int64_t(acc[t][q][r])) << (8 * q);
      if (g.sign < 0) v = 0ull - v;
      const size_t idx = size_t(gm) * g.N + gn;
      if (g.ksplit > 1)
        atomicAdd(reinterpret_cast<unsigned long long *>(&C[idx]), static_cast<unsigned long long>(v));
      else
        C[idx] = Cin ? v + Cin[idx] : v;
    }
  }
}

// blockIdx.z < nz0: problem g0, else problem g1 (nz = batch * ksplit of each)
__global__ __launch_bounds__(256) void k_gemm_mfma64(GemmArgs<uint64_t> g0, GemmArgs<uint64_t> g1, int nz0) {
  __shared__ __align__(16) uint32_t As[64 * 68];
  __shared__ __align__(16) uint32_t Bt[64 * 68];
  const int z = int(blockIdx.z);
  const bool second = z >= nz0;
  gemm_mfma64_tile(second ? g1 : g0, second ? z - nz0 : z, As, Bt);
}

// MFMA row operands of one 16-byte LDS read (16 Z_2^32 or 8 Z_2^64 words of a
// row, balanced digits): shift s takes digit s - j of each word at byte j
template <typename T>
__device__ __forceinline__ void digit_shifts(uint4 a, v4i_t (&as)[sizeof(T)]) {
  if constexpr (sizeof(T) == 4) {
    constexpr uint32_t sel[4] = {0x0c0c0c00u, 0x0c0c0001u, 0x0c000102u, 0x00010203u};
#pragma unroll
    for (int q = 0; q < 4; q++)
      as[q] = v4i_t{int(__builtin_amdgcn_perm(0u, a.x, sel[q])), int(__builtin_amdgcn_perm(0u, a.y, sel[q])),
                    int(__builtin_amdgcn_perm(0u, a.z, sel[q])), int(__builtin_amdgcn_perm(0u, a.w, sel[q]))};
  } else {
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const uint32_t lo = digit_sel(q, 0), hi = digit_sel(q, 4);
      as[q] = v4i_t{int(__builtin_amdgcn_perm(a.y, a.x, lo)), int(__builtin_amdgcn_perm(a.y, a.x, hi)),
                    int(__builtin_amdgcn_perm(a.w, a.z, lo)), int(__builtin_amdgcn_perm(a.w, a.z, hi))};
    }
  }
}
// digit_shifts for Z_2^32 with the byte selectors in scalar registers (set
// once per kernel by pan_shift_selectors): VOP3 takes no literal operand, so
// constant selectors are otherwise rematerialised in vector registers
struct ShiftSel {
  uint32_t s[4];
};
__device__ __forceinline__ ShiftSel pan_shift_selectors() {
  ShiftSel r;
  asm("s_mov_b32 %0, 0x0c0c0c00" : "=s"(r.s[0]));
  asm("s_mov_b32 %0, 0x0c0c0001" : "=s"(r.s[1]));
  asm("s_mov_b32 %0, 0x0c000102" : "=s"(r.s[2]));
  asm("s_mov_b32 %0, 0x00010203" : "=s"(r.s[3]));
  return r;
}
__device__ __forceinline__ void digit_shifts_s(uint4 a, const ShiftSel &sel, v4i_t (&as)[4]) {
#pragma unroll
  for (int q = 0; q < 4; q++)
    as[q] = v4i_t{int(__builtin_amdgcn_perm(0u, a.x, sel.s[q])), int(__builtin_amdgcn_perm(0u, a.y, sel.s[q])),
                  int(__builtin_amdgcn_perm(0u, a.z, sel.s[q])), int(__builtin_amdgcn_perm(0u, a.w, sel.s[q]))};
}
// the ring word of accumulator register r (shift sums acc[q][r])
template <typename T>
__device__ __forceinline__ T digit_fold(const v4i_t (&acc)[sizeof(T)], int r) {
  T v = 0;
#pragma unroll
  for (int q = 0; q < int(sizeof(T)); q++) {
    if constexpr (sizeof(T) == 4) v += uint32_t(acc[q][r]) << (8 * q);
    else v += uint64_t(int64_t(acc[q][r])) << (8 * q);
  }
  return v;
}

// Workgroup p of a one-dimensional launch of W runs on XCD p mod 8 (the
// dispatcher deals workgroups to the eight XCDs in turn); renumbering so that
// each XCD takes a contiguous range of W / 8 logical workgroups keeps a batch
// entry's tiles, which share their operands, in one XCD's L2.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_swizzle(int p, int W) {
  const int xcd = p % kXcds, q = p / kXcds, base = W / kXcds, rem = W % kXcds;
  return (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + q;
}
// ---------------------------------------------------------------------------
// Wide-K ring GEMM on the int8 matrix cores (both rings, the digit algebra of
// the two kernels above).  Those walk K in 64-word (Z_2^32) or 32-word (Z_2^64)
// steps and wait for a round trip to memory at every step, with about one
// 4-wave block per CU on this path's shapes (K = 78..312 words per segment,
// 140 x 140 per-graph blocks), so a tile costs a few memory latencies.  Here a
// 512-thread block stages KW 32-bit words of K per step (kWideK words of
// Z_2^32, half as many of Z_2^64): every load of a step is in flight at once,
// and the next step's loads are issued before the current step's MFMAs, so a
// segment of at most KW words costs one round trip.  LDS as above: A as [m][k],
// B transposed to [n][k], rows of KW + 4 words (16-byte reads by 8 consecutive
// lanes of consecutive rows fall in distinct bank groups).  Wave w computes
// rows 16 (w & 3) .. + 15 and columns 32 (w >> 2) .. + 31 of the 64 x 64 tile
// (two 16 x 16 MFMA tiles).  One step covers one segment only; a problem's
// steps run first segment first.  C = Cin + sign * (products).
// ---------------------------------------------------------------------------
constexpr int kWideK = 288;        // 32-bit words of K per step (LDS: 2 * 64 * 292 * 4 = 149.5 KB)
// The same kernel with 96- and 160-word steps (LDS 50 and 82 KB) for problems
// whose K takes as many steps of them as of kWideK (the public-weight products
// with K = 78 and 156): a thread stages, converts and stores 3 or 5 groups per
// operand instead of 9
constexpr int kWideKShort = 96, kWideKMid = 160;
constexpr int kWideThreads = 512;  // 8 waves

template <typename T>
struct WideStep {
  const T *a, *a2, *b, *b2;  // segment operands of batch entry bz (a2, b2: masks or null)
  int kb, klen;              // K range [kb, kb + klen) of the segment
};
// K words of a step: a segment with masks stages four operands, so its steps
// are half as wide (the staging registers hold two operand panels of KW words)
template <typename T, int KW>
__host__ __device__ __forceinline__ int wide_kt(bool masked) {
  return (masked ? KW / 2 : KW) * 4 / int(sizeof(T));
}
template <typename T, int KW>
__host__ __device__ __forceinline__ int wide_steps(const GemmArgs<T> &g) {
  const int k0 = wide_kt<T, KW>(g.A2 || g.B2), k1 = wide_kt<T, KW>(false);
  return (g.K + k0 - 1) / k0 + (g.A1b ? (g.K + k1 - 1) / k1 : 0);
}
template <typename T, int KW>
__device__ __forceinline__ WideStep<T> wide_step(const GemmArgs<T> &g, int bz, int i) {
  const bool masked = g.A2 || g.B2;
  const int k0 = wide_kt<T, KW>(masked), n0 = (g.K + k0 - 1) / k0;
  const bool seg = i >= n0;
  const int kt = seg ? wide_kt<T, KW>(false) : k0;
  WideStep<T> w;
  w.kb = (seg ? i - n0 : i) * kt;
  w.klen = min(kt, g.K - w.kb);
  w.a = (seg ? g.A1b : g.A1) + size_t(bz) * g.sA;
  w.b = (seg ? g.B1b : g.B1) + size_t(bz) * g.sB;
  w.a2 = (!seg && g.A2) ? g.A2 + size_t(bz) * g.sA : nullptr;
  w.b2 = (!seg && g.B2) ? g.B2 + size_t(bz) * g.sB : nullptr;
  return w;
}
// balanced digits of a 16-byte group (four Z_2^32 words or two Z_2^64 words) of x - y
template <typename T>
__device__ __forceinline__ uint4 wide_digits(uint4 x, uint4 y) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(ring_digits(x.x - y.x), ring_digits(x.y - y.y), ring_digits(x.z - y.z), ring_digits(x.w - y.w));
  } else {
    const uint64_t lo = ring_digits64(((uint64_t(x.y) << 32) | x.x) - ((uint64_t(y.y) << 32) | y.x));
    const uint64_t hi = ring_digits64(((uint64_t(x.w) << 32) | x.z) - ((uint64_t(y.w) << 32) | y.z));
    return make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
  }
}
template <typename T>
__device__ __forceinline__ uint4 wide_pack(const T (&v)[16 / sizeof(T)]) {
  if constexpr (sizeof(T) == 4) return make_uint4(v[0], v[1], v[2], v[3]);
  else return make_uint4(uint32_t(v[0]), uint32_t(v[0] >> 32), uint32_t(v[1]), uint32_t(v[1] >> 32));
}
// 16-byte group kv .. kv + WPG - 1 of row `row` of a row-major matrix with
// `ld` words per row, zero where out of [0, klen) (in = the row exists)
template <typename T, bool VA>
__device__ __forceinline__ uint4 wide_row_group(const T *p, size_t row, int ld, int kb, int kv, int klen, bool in) {
  constexpr int WPG = 16 / int(sizeof(T));
  uint4 r = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (VA) {  // ld, kb and klen are multiples of WPG
    if (in && kv < klen) r = *reinterpret_cast<const uint4 *>(p + row * ld + kb + kv);
  } else {
    T x[WPG];
    const T *q = p + row * ld + kb + kv;
#pragma unroll
    for (int e = 0; e < WPG; e++) {
      x[e] = 0;
      if (in && kv + e < klen) x[e] = q[e];
    }
    r = wide_pack<T>(x);
  }
  return r;
}
// WPG consecutive k (from kb + kv) of column `col` of a row-major K x ld matrix
template <typename T>
__device__ __forceinline__ uint4 wide_col_group(const T *p, int col, int ld, int kb, int kv, int klen, bool in) {
  constexpr int WPG = 16 / int(sizeof(T));
  T x[WPG];
  const T *q = p + size_t(kb + kv) * ld + col;
#pragma unroll
  for (int e = 0; e < WPG; e++) {
    x[e] = 0;
    if (in && kv + e < klen) x[e] = q[size_t(e) * ld];
  }
  return wide_pack<T>(x);
}

template <typename T, int KW, bool VA>
__global__ __launch_bounds__(kWideThreads) void k_gemm_wide(GemmArgs<T> g) {
  constexpr int LDK = KW + 4, WPG = 16 / int(sizeof(T)), NQ = int(sizeof(T));
  // plain and masked steps (KW, KW / 2 words) are whole 16-word MFMA chunks
  static_assert(KW % 32 == 0, "step widths a whole number of MFMA chunks");
  // 16-byte groups per thread and operand panel: NJ in a plain step, NJM in a
  // masked one (then slots NJM.. hold the masks' groups)
  constexpr int NJ = (KW / 4 + 7) / 8, NJM = (KW / 8 + 7) / 8, NS = NJ > 2 * NJM ? NJ : 2 * NJM;
  __shared__ __align__(16) uint32_t As[64 * LDK];
  __shared__ __align__(16) uint32_t Bt[64 * LDK];
  const int M = g.M, N = g.N, K = g.K;
  // one-dimensional launch, renumbered per XCD: column tile fastest, batch entry slowest
  const int gx = (N + 63) / 64, gy = (M + 63) / 64, lw = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const int bz = lw / (gx * gy), m0 = (lw / gx) % gy * 64, n0 = lw % gx * 64;
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4, rg = wave & 3, cg = wave >> 2;
  // staging: A group j of thread tid is row tid >> 3, 16-byte group (tid & 7) + 8j
  // of the step; B group j is column tid & 63, k words WPG ((tid >> 6) + 8j) + e
  const int arow = tid >> 3, bn = tid & 63, ag = tid & 7, bg = tid >> 6;
  const bool arow_ok = m0 + arow < M, bn_ok = n0 + bn < N;
  uint4 ra[NS], rb[NS];
  bool masked = false;  // the staged step's kind (uniform)
  auto load = [&](const WideStep<T> &w) {
    masked = w.a2 || w.b2;
    const size_t row = size_t(m0 + arow);
    const T *a2 = w.a2 ? w.a2 : w.a, *b2 = w.b2 ? w.b2 : w.b;  // a missing mask reads as zero below
    if (masked) {
#pragma unroll
      for (int j = 0; j < NJM; j++) {
        const int gi = ag + 8 * j;
        const bool in = arow_ok && gi < KW / 8;
        ra[j] = wide_row_group<T, VA>(w.a, row, K, w.kb, gi * WPG, w.klen, in);
        ra[NJM + j] = wide_row_group<T, VA>(a2, row, K, w.kb, gi * WPG, w.klen, in && w.a2);
      }
#pragma unroll
      for (int j = 0; j < NJM; j++) {
        const int gi = bg + 8 * j;
        const bool in = bn_ok && gi < KW / 8;
        rb[j] = wide_col_group<T>(w.b, n0 + bn, N, w.kb, gi * WPG, w.klen, in);
        rb[NJM + j] = wide_col_group<T>(b2, n0 + bn, N, w.kb, gi * WPG, w.klen, in && w.b2);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int gi = ag + 8 * j;
        ra[j] = wide_row_group<T, VA>(w.a, row, K, w.kb, gi * WPG, w.klen, arow_ok && gi < KW / 4);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int gi = bg + 8 * j;
        rb[j] = wide_col_group<T>(w.b, n0 + bn, N, w.kb, gi * WPG, w.klen, bn_ok && gi < KW / 4);
      }
    }
  };
  // every word of the step's rows is written (zeros past klen, M and N)
  auto store = [&]() {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    if (masked) {
#pragma unroll
      for (int j = 0; j < NJM; j++) {
        const int ga = ag + 8 * j, gb = bg + 8 * j;
        if (ga < KW / 8) *reinterpret_cast<uint4 *>(&As[arow * LDK + 4 * ga]) = wide_digits<T>(ra[j], ra[NJM + j]);
        if (gb < KW / 8) *reinterpret_cast<uint4 *>(&Bt[bn * LDK + 4 * gb]) = wide_digits<T>(rb[j], rb[NJM + j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int ga = ag + 8 * j, gb = bg + 8 * j;
        if (ga < KW / 4) *reinterpret_cast<uint4 *>(&As[arow * LDK + 4 * ga]) = wide_digits<T>(ra[j], z);
        if (gb < KW / 4) *reinterpret_cast<uint4 *>(&Bt[bn * LDK + 4 * gb]) = wide_digits<T>(rb[j], z);
      }
    }
  };
  v4i_t acc[2][NQ];
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int q = 0; q < NQ; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
  const int nsteps = wide_steps<T, KW>(g);
  WideStep<T> cur = wide_step<T, KW>(g, bz, 0);
  load(cur);
  for (int i = 0; i < nsteps; i++) {
    store();
    __syncthreads();
    const int nkc = (cur.klen * int(sizeof(T) / 4) + 15) / 16;
    if (i + 1 < nsteps) {
      cur = wide_step<T, KW>(g, bz, i + 1);
      load(cur);
    }
    for (int kc = 0; kc < nkc; kc++) {
      v4i_t as[NQ];
      digit_shifts<T>(*reinterpret_cast<const uint4 *>(&As[(16 * rg + li) * LDK + 16 * kc + 4 * lg]), as);
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[(32 * cg + 16 * t + li) * LDK + 16 * kc + 4 * lg]);
        const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
        for (int q = 0; q < NQ; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  T *C = g.C + size_t(bz) * g.sC;
  const T *Cin = g.Cin ? g.Cin + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int gn = n0 + 32 * cg + 16 * t + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      // accumulator register r of lane (li, lg): row 4 lg + r, column li of the MFMA tile
      const int gm = m0 + 16 * rg + 4 * lg + r;
      if (gm >= M || gn >= N) continue;
      const size_t idx = size_t(gm) * N + gn;
      const T v = digit_fold<T>(acc[t], r);
      C[idx] = (Cin ? Cin[idx] : T(0)) + (g.sign < 0 ? T(0) - v : v);
    }
  }
}

// ---------------------------------------------------------------------------
// Both parties' Beaver products of an SxS gate on one GPU, reconstructed, per
// 48 x 32 output tile: party 0's C0 + (A^ - RA0)(B^ - RB0) and party 1's
// C1 - (A^ RB1 + RA1 B^), written as their sum (the masked product both
// parties reveal).  Each K phase (144 words of Z_2^32, 48 of Z_2^64) stages all
// six operand panels at once -- A^, RA0, RA1 rows and B^, RB0, RB1 columns, as
// digits of A^ - RA0, A^, RA1 and of B^ - RB0, RB1, B^ in LDS -- so the
// per-graph products of the affinity model (140 x 140 by 140 x N) cost one
// memory round trip (three for Z_2^64); the next phase's loads are issued before
// the current phase's MFMAs.  Six waves, one 16 x 16 MFMA tile each (rows
// 16 (w % 3), columns 16 (w / 3)), with party 0's and party 1's accumulators.
// The 48-row tiles cover 140 rows as 48 + 48 + 44.
// ---------------------------------------------------------------------------
constexpr int kSxsTM = 48, kSxsTN = 32, kSxsThreads = 384;
// 32-bit words of K per phase, a multiple of 16 (the MFMA chunk): 144 in
// Z_2^32 (142 KB of LDS, one workgroup per CU, the affinity model's products in
// one phase), 96 in Z_2^64 (its staging registers and eight-shift accumulators
// leave room for two thirds of the width; three phases).  Measured alternative:
// 80-word phases in Z_2^32 (two workgroups per CU, 168 VGPRs) were slower,
// 17.7 / 26.6 / 38.5 against 11.8 / 23.5 / 35.7 us for N = 78 / 156 / 312.
template <typename T>
constexpr int sxs_kc() {
  return sizeof(T) == 4 ? 144 : 96;
}

template <typename T, bool VA>
__global__ __launch_bounds__(kSxsThreads) void k_sxs_fused(GemmArgs<T> g0, GemmArgs<T> g1) {
  constexpr int KC = sxs_kc<T>(), WPG = 16 / int(sizeof(T)), NQ = int(sizeof(T)), LDK = KC + 4, GR = KC / 4;
  constexpr int KT = KC * 4 / int(sizeof(T));  // words of T per phase
  constexpr int NA = (kSxsTM * GR + kSxsThreads - 1) / kSxsThreads;
  constexpr int NB = (kSxsTN * GR + kSxsThreads - 1) / kSxsThreads;
  // the MFMA loop reads whole 16-word chunks of a row: KC a multiple of 16 keeps
  // them inside the staged words (zeros past the phase's K); rows of KC + 4
  // words put 16-byte reads of consecutive rows in distinct bank groups
  static_assert(KC % 16 == 0, "phase width a whole number of MFMA chunks");
  __shared__ __align__(16) uint32_t As[3 * kSxsTM * LDK];  // digits of A^ - RA0, A^, RA1
  __shared__ __align__(16) uint32_t Bt[3 * kSxsTN * LDK];  // digits of B^ - RB0, RB1, B^ (as [n][k])
  const int M = g0.M, N = g0.N, K = g0.K;
  // one-dimensional launch, renumbered per XCD: column tile fastest, graph slowest
  const int gx = (N + kSxsTN - 1) / kSxsTN, gy = (M + kSxsTM - 1) / kSxsTM;
  const int lw = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const int bz = lw / (gx * gy), m0 = (lw / gx) % gy * kSxsTM, n0 = lw % gx * kSxsTN;
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4, rg = wave % 3, cg = wave / 3;
  const T *Ah = g0.A1 + size_t(bz) * g0.sA, *RA0 = g0.A2 + size_t(bz) * g0.sA, *RA1 = g1.A1b + size_t(bz) * g1.sA;
  const T *Bh = g0.B1 + size_t(bz) * g0.sB, *RB0 = g0.B2 + size_t(bz) * g0.sB, *RB1 = g1.B1 + size_t(bz) * g1.sB;
  // this lane's four outputs: rows 4 lg + r of the wave's MFMA tile, column li
  const int on = n0 + 16 * cg + li;
  T cin[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int om = m0 + 16 * rg + 4 * lg + r;
    cin[r] = 0;
    if (om < M && on < N) {
      const size_t idx = size_t(om) * N + on;
      if (g0.Cin) cin[r] += g0.Cin[size_t(bz) * g0.sC + idx];
      if (g1.Cin) cin[r] += g1.Cin[size_t(bz) * g1.sC + idx];
    }
  }
  uint4 xa[NA], xa0[NA], xa1[NA], xb[NB], xb0[NB], xb1[NB];
  auto load = [&](int kb) {
    const int klen = min(KT, K - kb);
#pragma unroll
    for (int j = 0; j < NA; j++) {
      const int f = tid + kSxsThreads * j, r = f / GR, gi = f % GR;
      const bool in = f < kSxsTM * GR && m0 + r < M;
      const size_t row = size_t(m0 + r);
      xa[j] = wide_row_group<T, VA>(Ah, row, K, kb, gi * WPG, klen, in);
      xa0[j] = wide_row_group<T, VA>(RA0, row, K, kb, gi * WPG, klen, in);
      xa1[j] = wide_row_group<T, VA>(RA1, row, K, kb, gi * WPG, klen, in);
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int f = tid + kSxsThreads * j, n = f % kSxsTN, gi = f / kSxsTN;
      const bool in = f < kSxsTN * GR && n0 + n < N;
      xb[j] = wide_col_group<T>(Bh, n0 + n, N, kb, gi * WPG, klen, in);
      xb0[j] = wide_col_group<T>(RB0, n0 + n, N, kb, gi * WPG, klen, in);
      xb1[j] = wide_col_group<T>(RB1, n0 + n, N, kb, gi * WPG, klen, in);
    }
  };
  // every word of the panels' rows is written (zeros past K, M and N)
  auto store = [&]() {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < NA; j++) {
      const int f = tid + kSxsThreads * j, r = f / GR, gi = f % GR;
      if (f < kSxsTM * GR) {
        uint32_t *p = &As[r * LDK + 4 * gi];
        *reinterpret_cast<uint4 *>(p) = wide_digits<T>(xa[j], xa0[j]);
        *reinterpret_cast<uint4 *>(p + kSxsTM * LDK) = wide_digits<T>(xa[j], z);
        *reinterpret_cast<uint4 *>(p + 2 * kSxsTM * LDK) = wide_digits<T>(xa1[j], z);
      }
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int f = tid + kSxsThreads * j, n = f % kSxsTN, gi = f / kSxsTN;
      if (f < kSxsTN * GR) {
        uint32_t *p = &Bt[n * LDK + 4 * gi];
        *reinterpret_cast<uint4 *>(p) = wide_digits<T>(xb[j], xb0[j]);
        *reinterpret_cast<uint4 *>(p + kSxsTN * LDK) = wide_digits<T>(xb1[j], z);
        *reinterpret_cast<uint4 *>(p + 2 * kSxsTN * LDK) = wide_digits<T>(xb[j], z);
      }
    }
  };
  // one accumulator set, folded into ring words after each party's MFMAs of a
  // phase (a phase's shift sums are exact, far below 2^15 words of K)
  v4i_t acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; q++) acc[q] = v4i_t{0, 0, 0, 0};
  T vs0[4] = {0, 0, 0, 0}, vs1[4] = {0, 0, 0, 0};
  auto fold = [&](T (&vs)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      vs[r] += digit_fold<T>(acc, r);
#pragma unroll
      for (int q = 0; q < NQ; q++) acc[q][r] = 0;
    }
  };
  // acc += (row panel pa) . (column panel pb)^T over the phase's nkc 16-word chunks
  auto mfma_panel = [&](int pa, int pb, int nkc) {
    const int ar = pa * kSxsTM * LDK + (16 * rg + li) * LDK + 4 * lg;
    const int br = pb * kSxsTN * LDK + (16 * cg + li) * LDK + 4 * lg;
    for (int kc = 0; kc < nkc; kc++) {
      v4i_t as[NQ];
      const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[br + 16 * kc]);
      const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
      digit_shifts<T>(*reinterpret_cast<const uint4 *>(&As[ar + 16 * kc]), as);
#pragma unroll
      for (int q = 0; q < NQ; q++) acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[q], 0, 0, 0);
    }
  };
  load(0);
  for (int kb = 0; kb < K; kb += KT) {
    store();
    __syncthreads();
    const int nkc = (min(KT, K - kb) * int(sizeof(T) / 4) + 15) / 16;
    if (kb + KT < K) load(kb + KT);
    mfma_panel(0, 0, nkc);  // party 0: (A^ - RA0)(B^ - RB0)
    fold(vs0);
    mfma_panel(1, 1, nkc);  // party 1: A^ RB1 + RA1 B^
    mfma_panel(2, 2, nkc);
    fold(vs1);
    __syncthreads();
  }
  T *C = g0.C + size_t(bz) * g0.sC;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int om = m0 + 16 * rg + 4 * lg + r;
    if (om >= M || on >= N) continue;
    // party 0's share (sign +1) plus party 1's (sign -1)
    C[size_t(om) * N + on] = cin[r] + vs0[r] - vs1[r];
  }
}

// ---------------------------------------------------------------------------
// Panel products on buffer loads (both rings, the digit algebra above):
// C[b] = Cin0[b] + Cin1[b] + sum_p sign_p (A_p1 - A_p2)[b] (B_p1 - B_p2)[b] over
// NP <= 3 panels of one shape (M x K by K x N per batch entry; A_p2, B_p2, Cin
// may be null).  An SxS gate is three panels -- party 0's (A^ - RA0)(B^ - RB0)
// + C0 and party 1's C1 - A^ RB1 - RA1 B^ -- whose sum is the masked product
// both parties reveal.  The kernel is meant to share CUs with the DCF gate
// kernels of other lanes: 21 KB of LDS, three waves per workgroup, and a raised
// wave priority (a short product on a lane's critical path).
// Every operand load is a buffer load: the matrix of the batch entry is a buffer
// resource in scalar registers, a lane supplies one 32-bit byte offset per step
// and each MFMA chunk adds an immediate, and an element outside the matrix is
// read through an offset past the resource's end, which the hardware returns as
// zero (no address arithmetic in 64 bits, no exec-mask branches).
// Workgroup: RW waves, 16 NT output columns; wave w owns the 16-row MFMA tile
// at rows m0 + 16 w and keeps its A operands of a step in registers, in the
// MFMA layout (row li, 16-byte group lg of each chunk), as balanced digits; the
// workgroup stages the step's B rows as digits in LDS as [k][n] (LDN words per
// row: the four k rows one lane reads for a chunk fall in distinct bank groups),
// one 16-byte group per thread and operand.  A step is KPW 32-bit words of K of
// one panel; the shift sums are folded into ring words after every step (a
// step's int32 sums are exact, so Z_2^64 has no bound on K here).
// Requires rows of A and B readable as 16-byte groups: K and N multiples of the
// group, 16-byte aligned operands and batch strides (launch_gemm checks).
// ---------------------------------------------------------------------------
template <typename T>
struct PanelArgs {
  int M = 0, N = 0, K = 0, batch = 1, np = 1;
  const T *a1[3] = {}, *a2[3] = {}, *b1[3] = {}, *b2[3] = {};
  int sign[3] = {1, 1, 1};
  size_t sA = 0, sB = 0, sC = 0;
  const T *cin0 = nullptr, *cin1 = nullptr;
  T *C = nullptr;
};
constexpr int kPanKPW = 144;           // 32-bit words of K per step: 9 MFMA chunks (K = 140 in one step)
constexpr uint32_t kPanOob = 0x80000000u;  // a byte offset past every resource (matrices below 2 GiB)
constexpr int kPanRsrcWord3 = 0x00020000;  // gfx9 buffer resource word 3: 32-bit data format

typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pan_rsrc(const void *p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(bytes), kPanRsrcWord3);
}
__device__ __forceinline__ uint4 pan_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const v4u_t v = __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t pan_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, int(off), 0, 0);
}

// Waves per SIMD the register budget is set for: three in Z_2^32 (measured
// faster than two even where a few registers spill), two in Z_2^64.
template <typename T, int RW, int NT>
constexpr int pan_waves() {
  return sizeof(T) == 4 ? 3 : 2;
}
template <typename T, int NP, int RW, int NT>
__global__ __launch_bounds__(64 * RW, (pan_waves<T, RW, NT>())) void k_panels(PanelArgs<T> g) {
  constexpr int KPW = kPanKPW, NTH = 64 * RW, TN = 16 * NT, NQ = int(sizeof(T)), NC = KPW / 16;
  constexpr int WPG = 16 / int(sizeof(T)), KT = KPW * 4 / int(sizeof(T));
  constexpr int LDK = KPW + 4;                    // 32-bit words per LDS row (one column of B)
  constexpr int GPR = TN / WPG;                   // 16-byte groups per B row of the tile
  constexpr int NB = (KT * GPR + NTH - 1) / NTH;  // B groups per thread and operand
  static_assert(KPW % 16 == 0, "whole MFMA chunks");
  __shared__ __align__(16) uint32_t Bt[TN * LDK];  // B of a step as [n][k] digits
  __builtin_amdgcn_s_setprio(2);
  const int M = g.M, N = g.N, K = g.K;
  const int gx = (N + TN - 1) / TN, gy = (M + 16 * RW - 1) / (16 * RW);
  const int lw = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const int bz = lw / (gx * gy), m0 = (lw / gx) % gy * 16 * RW, n0 = lw % gx * TN;
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
  const int arow = m0 + 16 * wave + li;
  const bool wave_ok = m0 + 16 * wave < M;
  const size_t abytes = size_t(M) * K * sizeof(T), bbytes = size_t(K) * N * sizeof(T);
  // byte offset of this lane's A row (past the resource if the row is past M)
  const uint32_t arow_off = arow < M ? uint32_t(arow) * uint32_t(K) * uint32_t(sizeof(T)) : kPanOob;
  const int ksteps = (K + KT - 1) / KT;
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  v4i_t acc[NT][NQ];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int q = 0; q < NQ; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
  T vs[NT][4];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) vs[t][r] = 0;
#pragma unroll
  for (int p = 0; p < NP; p++) {
    // masks (uniform): only panel 0 may have them (party 0's product, or a
    // product's first K segment), so later panels compile without
    const bool ma = p == 0 && g.a2[0] != nullptr, mb = p == 0 && g.b2[0] != nullptr;
    const __amdgpu_buffer_rsrc_t ra1 = pan_rsrc(g.a1[p] + size_t(bz) * g.sA, abytes);
    const __amdgpu_buffer_rsrc_t rb1 = pan_rsrc(g.b1[p] + size_t(bz) * g.sB, bbytes);
    const __amdgpu_buffer_rsrc_t ra2 = pan_rsrc(ma ? g.a2[0] + size_t(bz) * g.sA : g.a1[p], abytes);
    const __amdgpu_buffer_rsrc_t rb2 = pan_rsrc(mb ? g.b2[0] + size_t(bz) * g.sB : g.b1[p], bbytes);
    for (int ks = 0; ks < ksteps; ks++) {
      const int kb = ks * KT, klen = min(KT, K - kb);
      // B groups: k row kr of the step, 16-byte group q of the tile's columns
      uint4 xb[NB], yb[NB];
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int f = tid + NTH * j, kr = f / GPR, q = f % GPR, n = n0 + q * WPG;
        const uint32_t off = (f < KT * GPR && kr < klen && n < N)
                                 ? (uint32_t(kb + kr) * uint32_t(N) + uint32_t(n)) * uint32_t(sizeof(T))
                                 : kPanOob;
        xb[j] = pan_load(rb1, off);
        yb[j] = mb ? pan_load(rb2, off) : z4;
      }
      // A groups of this lane: chunk c covers words (4c + lg) WPG .. of the step
      uint4 xa[NC], ya[NC];
      const uint32_t abase = arow_off + uint32_t(kb + lg * WPG) * uint32_t(sizeof(T));
      const int kfull = klen / (4 * WPG);  // chunks whose 16 words are all inside the step
#pragma unroll
      for (int c = 0; c < NC; c++) {
        uint32_t off = abase + uint32_t(c) * 64u;
        if (c >= kfull && (4 * c + lg) * WPG >= klen) off = kPanOob;
        xa[c] = pan_load(ra1, off);
        ya[c] = ma ? pan_load(ra2, off) : z4;
      }
      // the B groups' digits, transposed into the [n][k] rows (one element per write)
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int f = tid + NTH * j, kr = f / GPR, q = f % GPR;
        if (f < KT * GPR) {
          const uint4 d = wide_digits<T>(xb[j], yb[j]);
          if constexpr (sizeof(T) == 4) {
            uint32_t *bp = &Bt[(4 * q) * LDK + kr];
            bp[0] = d.x;
            bp[LDK] = d.y;
            bp[2 * LDK] = d.z;
            bp[3 * LDK] = d.w;
          } else {
            uint32_t *bp = &Bt[(2 * q) * LDK + 2 * kr];
            *reinterpret_cast<uint2 *>(bp) = make_uint2(d.x, d.y);
            *reinterpret_cast<uint2 *>(bp + LDK) = make_uint2(d.z, d.w);
          }
        }
      }
      __syncthreads();
      const int nkc = (klen * NQ / 4 + 15) / 16;
      if (wave_ok) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
          if (c < nkc) {
            v4i_t as[NQ];
            digit_shifts<T>(wide_digits<T>(xa[c], ya[c]), as);
#pragma unroll
            for (int t = 0; t < NT; t++) {
              const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[(16 * t + li) * LDK + 16 * c + 4 * lg]);
              const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
              for (int q = 0; q < NQ; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const T v = digit_fold<T>(acc[t], r);
          vs[t][r] += g.sign[p] < 0 ? T(0) - v : v;
#pragma unroll
          for (int q = 0; q < NQ; q++) acc[t][q][r] = 0;
        }
      __syncthreads();  // Bt is rewritten by the next step
    }
  }
  T *C = g.C + size_t(bz) * g.sC;
  const T *c0 = g.cin0 ? g.cin0 + size_t(bz) * g.sC : nullptr, *c1 = g.cin1 ? g.cin1 + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int on = n0 + 16 * t + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      // accumulator register r of lane (li, lg): row 4 lg + r, column li of the MFMA tile
      const int om = m0 + 16 * wave + 4 * lg + r;
      if (om >= M || on >= N) continue;
      const size_t idx = size_t(om) * N + on;
      C[idx] = (c0 ? c0[idx] : T(0)) + (c1 ? c1[idx] : T(0)) + vs[t][r];
    }
  }
}

// XOR applied to the word index k of B's LDS row n in k_panels_pf: it flips
// bits 2-3 only (k stays in its 16-word chunk, 16-byte groups stay whole).
// With 148-word rows, a wave's one-word column writes (lanes: 4-column groups
// of a K row, then the next rows) fall on three times fewer bank conflicts,
// and its 16-byte reads (16 rows, 4 groups) stay conflict-free.
__device__ __forceinline__ int pf_swz(int n) { return 4 * ((n >> 3) & 3); }
// k_panels for Z_2^32 with K within one step (K <= kPanKPW words) and at
// least two panels, software-pipelined across the panels: panel p + 1's B
// groups are loaded as soon as panel p's B is in LDS, its A groups as soon as
// panel p's MFMAs have read theirs (under the fold, the barrier and the next
// B staging), and the epilogue's Cin words before the last panel's products.
// A wave's chain (its products and the digit work beside them issue in turn)
// sets a workgroup's time whatever the load on its SIMD, so a launch costs
// about one chain per round of resident workgroups: two waves per SIMD hold
// two workgroups of three or four waves per CU, and the launcher picks the
// columns per workgroup (16, 32 or 48) that give the fewest rounds times chain
// length (22 graphs of 140 x 140 x 312: 462 workgroups of 48 columns, one
// round, against 660 of 32 in two).
template <int NP, int RW, int NT>
__global__ __launch_bounds__(64 * RW, 2) void k_panels_pf(PanelArgs<uint32_t> g) {
  using T = uint32_t;
  constexpr int KT = kPanKPW, NTH = 64 * RW, TN = 16 * NT, NQ = 4, NC = KT / 16, WPG = 4;
  constexpr int LDK = KT + 4;                     // 32-bit words per LDS row (one column of B)
  constexpr int GPR = TN / WPG;                   // 16-byte groups per B row of the tile
  constexpr int NB = (KT * GPR + NTH - 1) / NTH;  // B groups per thread
  static_assert(NP >= 2 && NP <= 3, "pipelined across two or three panels");
  __shared__ __align__(16) uint32_t Bt[TN * LDK];  // B of a panel as [n][k] digits
  __builtin_amdgcn_s_setprio(2);
  const int M = g.M, N = g.N, K = g.K;
  const int gx = (N + TN - 1) / TN, gy = (M + 16 * RW - 1) / (16 * RW);
  const int lw = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const int bz = lw / (gx * gy), m0 = (lw / gx) % gy * 16 * RW, n0 = lw % gx * TN;
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
  const int arow = m0 + 16 * wave + li;
  const bool wave_ok = m0 + 16 * wave < M;
  const size_t abytes = size_t(M) * K * sizeof(T), bbytes = size_t(K) * N * sizeof(T);
  const uint32_t arow_off = arow < M ? uint32_t(arow) * uint32_t(K) * uint32_t(sizeof(T)) : kPanOob;
  const int kfull = K / (4 * WPG);  // chunks whose 16 words are all inside K
  const int nkc = (K + 15) / 16;    // chunks holding any word of K
  const bool ma = g.a2[0] != nullptr, mb = g.b2[0] != nullptr;  // masks: panel 0 only
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  const ShiftSel sel = pan_shift_selectors();

  // operands of panel p (p and the mask flags fold after unrolling)
  auto load_b = [&](int p, uint4(&xb)[NB], uint4(&yb)[NB]) {
    const __amdgpu_buffer_rsrc_t rb1 = pan_rsrc(g.b1[p] + size_t(bz) * g.sB, bbytes);
    const __amdgpu_buffer_rsrc_t rb2 = pan_rsrc(p == 0 && mb ? g.b2[0] + size_t(bz) * g.sB : g.b1[p], bbytes);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int f = tid + NTH * j, kr = f / GPR, q = f % GPR, n = n0 + q * WPG;
      const uint32_t off = (f < KT * GPR && kr < K && n < N) ? (uint32_t(kr) * uint32_t(N) + uint32_t(n)) * 4u : kPanOob;
      xb[j] = pan_load(rb1, off);
      if (p == 0 && mb) yb[j] = pan_load(rb2, off);
    }
  };
  auto load_a = [&](int p, uint4(&xa)[NC], uint4(&ya)[NC]) {
    const __amdgpu_buffer_rsrc_t ra1 = pan_rsrc(g.a1[p] + size_t(bz) * g.sA, abytes);
    const __amdgpu_buffer_rsrc_t ra2 = pan_rsrc(p == 0 && ma ? g.a2[0] + size_t(bz) * g.sA : g.a1[p], abytes);
    const uint32_t abase = arow_off + uint32_t(lg * WPG) * 4u;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      uint32_t off = abase + uint32_t(c) * 64u;
      if (c >= kfull && (4 * c + lg) * WPG >= K) off = kPanOob;
      xa[c] = pan_load(ra1, off);
      if (p == 0 && ma) ya[c] = pan_load(ra2, off);
    }
  };

  v4i_t acc[NT][NQ];
  T vs[NT][4];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) vs[t][r] = 0;
  uint4 xa[NC], ya[NC], xb[NB], yb[NB];
#pragma unroll
  for (int c = 0; c < NC; c++) ya[c] = z4;
#pragma unroll
  for (int j = 0; j < NB; j++) yb[j] = z4;
  load_a(0, xa, ya);
  load_b(0, xb, yb);
  T cin[NT][4];
  T *C = g.C + size_t(bz) * g.sC;
  const T *c0 = g.cin0 ? g.cin0 + size_t(bz) * g.sC : nullptr, *c1 = g.cin1 ? g.cin1 + size_t(bz) * g.sC : nullptr;
#pragma unroll
  for (int p = 0; p < NP; p++) {
    // panel p's B digits, transposed into the [n][k] rows (one element per
    // write); word k of row n sits at k ^ pf_swz(n), which spreads a wave's
    // column writes over the banks and keeps the 16-byte reads contiguous
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int f = tid + NTH * j, kr = f / GPR, q = f % GPR;
      if (f < KT * GPR) {
        const uint4 d = wide_digits<T>(xb[j], p == 0 ? yb[j] : z4);
        uint32_t *bp = &Bt[(4 * q) * LDK + (kr ^ pf_swz(4 * q))];  // pf_swz is the same for rows 4q .. 4q + 3
        bp[0] = d.x;
        bp[LDK] = d.y;
        bp[2 * LDK] = d.z;
        bp[3 * LDK] = d.w;
      }
    }
    if (p + 1 < NP) load_b(p + 1, xb, yb);
    __syncthreads();
    if (p == NP - 1) {
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int on = n0 + 16 * t + li, om = m0 + 16 * wave + 4 * lg + r;
          const size_t idx = size_t(om) * N + on;
          const bool in = om < M && on < N;
          cin[t][r] = (in && c0 ? c0[idx] : T(0)) + (in && c1 ? c1[idx] : T(0));
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int q = 0; q < NQ; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
    // one chunk's products: A digits shifted per shift sum, B from LDS
    auto chunk = [&](int c) {
      v4i_t as[NQ];
      digit_shifts_s(wide_digits<T>(xa[c], p == 0 ? ya[c] : z4), sel, as);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int n = 16 * t + li;
        const uint4 b = *reinterpret_cast<const uint4 *>(&Bt[n * LDK + ((16 * c + 4 * lg) ^ pf_swz(n))]);
        const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
        for (int q = 0; q < NQ; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
      }
    };
    if (wave_ok) {
      if (nkc == NC) {
        // every chunk holds words of K: one basic block, so the scheduler can
        // put a chunk's digit work beside the previous chunk's MFMAs
#pragma unroll
        for (int c = 0; c < NC; c++) chunk(c);
      } else {
#pragma unroll
        for (int c = 0; c < NC; c++)
          if (c < nkc) chunk(c);
      }
    }
    if (p + 1 < NP) load_a(p + 1, xa, ya);  // the next panel's A into the same registers
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const T v = digit_fold<T>(acc[t], r);
        vs[t][r] += g.sign[p] < 0 ? T(0) - v : v;
      }
    if (p + 1 < NP) __syncthreads();  // Bt is rewritten by the next panel
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int on = n0 + 16 * t + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int om = m0 + 16 * wave + 4 * lg + r;
      if (om >= M || on >= N) continue;
      C[size_t(om) * N + on] = cin[t][r] + vs[t][r];
    }
  }
}

// C[b] = Cin[b] (or 0) before the split-K slices are added
template <typename T>
__global__ void k_gemm_init(int M, int N, int batch, size_t sC, const T *Cin, T *C) {
  const size_t per = size_t(M) * N, n = per * batch;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const size_t b = i / per, r = i % per;
    C[b * sC + r] = Cin ? Cin[b * sC + r] : T(0);
  }
}

// ---------------------------------------------------------------------------
// Products of at most kDotMaxN columns (the last fully connected layer of the
// affinity model: 22 x 512 x 1 per lane): a 64 x 64 matrix tile would compute
// mostly padding, and the tiled kernel splits K over a few workgroups that add
// with atomics.  Here one wave per output element: lane l multiplies k = l,
// l + 64, .. on the VALU (ring arithmetic wraps mod 2^bw), a butterfly over the
// wave adds the partial sums, lane 0 writes C = Cin + sign * sum.  A lane loads
// kDotUnroll of its k at once, so K up to 64 * kDotUnroll = 512 costs one
// memory round trip.
// ---------------------------------------------------------------------------
constexpr int kDotMaxN = 4, kDotMaxK = 8192, kDotUnroll = 8;
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    if constexpr (sizeof(T) == 4) {
      v += T(__shfl_xor(int(v), off, 64));
    } else {
      const uint32_t lo = uint32_t(__shfl_xor(int(uint32_t(v)), off, 64));
      const uint32_t hi = uint32_t(__shfl_xor(int(uint32_t(v >> 32)), off, 64));
      v += (uint64_t(hi) << 32) | lo;
    }
  }
  return v;
}
template <typename T>
__global__ __launch_bounds__(256) void k_gemm_dot(GemmArgs<T> g) {
  const size_t per = size_t(g.M) * g.N, e = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (e >= per * size_t(g.batch)) return;  // uniform over the wave
  const int lane = int(threadIdx.x & 63);
  const size_t bz = e / per, mn = e % per, m = mn / size_t(g.N), n = mn % size_t(g.N);
  const size_t ao = bz * g.sA + m * size_t(g.K), bo = bz * g.sB + n, ld = size_t(g.N);
  T s = 0;
  for (int k0 = lane; k0 < g.K; k0 += 64 * kDotUnroll) {
    T a[kDotUnroll], b[kDotUnroll];
#pragma unroll
    for (int u = 0; u < kDotUnroll; u++) {  // k past K reads k = 0 (loads without branches) and adds 0
      const int k = k0 + 64 * u < g.K ? k0 + 64 * u : 0;
      a[u] = g.A1[ao + k];
      b[u] = g.B1[bo + size_t(k) * ld];
    }
#pragma unroll
    for (int u = 0; u < kDotUnroll; u++) s += k0 + 64 * u < g.K ? a[u] * b[u] : T(0);
  }
  s = wave_sum(s);
  if (lane == 0) {
    const size_t ci = bz * g.sC + mn;
    g.C[ci] = (g.Cin ? g.Cin[ci] : T(0)) + (g.sign < 0 ? T(0) - s : s);
  }
}
// the dot kernel: automatic path selection, a plain product (no masks, one K
// segment), at most kDotMaxN columns, K within kDotMaxK (16 rounds of loads)
template <typename T>
static bool use_dot(const Launch &L, const GemmArgs<T> &g) {
  return L.gemm == 0 && !g.A2 && !g.B2 && !g.A1b && g.N <= kDotMaxN && g.K <= kDotMaxK &&
         (size_t(g.M) * g.N * g.batch + 3) / 4 <= size_t(INT32_MAX);
}
template <typename T>
static hipError_t launch_dot(const Launch &L, const GemmArgs<T> &g) {
  const unsigned blocks = unsigned((size_t(g.M) * g.N * g.batch + 3) / 4);
  hipLaunchKernelGGL((k_gemm_dot<T>), dim3(blocks), dim3(256), 0, L.stream, g);
  return hipGetLastError();
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// rows of A (resp. B) can be read as 16-byte words
static bool gemm_vec_a(const GemmArgs<uint32_t> &g) {
  return g.K % 4 == 0 && (g.batch == 1 || g.sA % 4 == 0) && aligned16(g.A1) && aligned16(g.A2) && aligned16(g.A1b);
}
static bool gemm_vec_b(const GemmArgs<uint32_t> &g) {
  return g.N % 4 == 0 && (g.batch == 1 || g.sB % 4 == 0) && aligned16(g.B1) && aligned16(g.B2) && aligned16(g.B1b);
}
static hipError_t launch_mfma(const Launch &L, dim3 grid, const GemmArgs<uint64_t> &g0,
                              const GemmArgs<uint64_t> &g1, int nz0) {
  hipLaunchKernelGGL(k_gemm_mfma64, grid, dim3(256), 0, L.stream, g0, g1, nz0);
  return hipGetLastError();
}
static hipError_t launch_mfma(const Launch &L, dim3 grid, const GemmArgs<uint32_t> &g0,
                              const GemmArgs<uint32_t> &g1, int nz0) {
  const bool va = gemm_vec_a(g0) && gemm_vec_a(g1), vb = gemm_vec_b(g0) && gemm_vec_b(g1);
  if (va && vb)
    hipLaunchKernelGGL((k_gemm_mfma<true, true>), grid, dim3(256), 0, L.stream, g0, g1, nz0);
  else if (va)
    hipLaunchKernelGGL((k_gemm_mfma<true, false>), grid, dim3(256), 0, L.stream, g0, g1, nz0);
  else if (vb)
    hipLaunchKernelGGL((k_gemm_mfma<false, true>), grid, dim3(256), 0, L.stream, g0, g1, nz0);
  else
    hipLaunchKernelGGL((k_gemm_mfma<false, false>), grid, dim3(256), 0, L.stream, g0, g1, nz0);
  return hipGetLastError();
}

// K slice of the matrix-core kernels: 64 words (Z_2^32), 32 (Z_2^64)
template <typename T>
constexpr int mfma_bk() {
  return sizeof(T) == 4 ? 64 : 32;
}
// the matrix-core path: selected (not MPCX_GEMM=valu), and for Z_2^64 a total K
// below 2^15 (the low shifts' int32 sums stay exact)
template <typename T>
static bool use_mfma(const Launch &L, const GemmArgs<T> &g) {
  if (L.gemm == 1) return false;
  constexpr int bk = mfma_bk<T>();
  const int Kt = g.A1b ? (g.K + bk - 1) / bk * bk + g.K : g.K;
  return sizeof(T) == 4 || Kt < (1 << 15);
}
// split-K factor: enough K slices that the launch has about two tiles per CU
template <typename T>
static int gemm_ksplit(const Launch &L, const GemmArgs<T> &g, int tiles, bool mfma) {
  constexpr int bk = mfma_bk<T>();
  const int Kt = g.A1b ? (g.K + bk - 1) / bk * bk + g.K : g.K;
  if (tiles >= L.num_cu || Kt < 64) return 1;
  const int want = (2 * L.num_cu + tiles - 1) / tiles;
  return std::max(1, std::min(want, mfma ? (Kt + bk - 1) / bk : Kt / 32));
}
template <typename T>
static int gemm_tiles(const GemmArgs<T> &g) {
  return ((g.N + 63) / 64) * ((g.M + 63) / 64) * g.batch;
}
template <typename T>
static hipError_t gemm_init(const Launch &L, const GemmArgs<T> &g) {
  if (g.ksplit <= 1 || g.C == g.Cin || (g.c_zero && !g.Cin)) return hipSuccess;
  const int block = 256;
  int grid = grid_for(k_gemm_init<T>, block, size_t(g.M) * g.N * g.batch, L.num_cu);
  hipLaunchKernelGGL((k_gemm_init<T>), dim3(grid), dim3(block), 0, L.stream, g.M, g.N, g.batch, g.sC, g.Cin, g.C);
  return hipGetLastError();
}

// The wide-K kernel: automatic path selection, the matrix-core path, and either
// enough tiles to occupy a quarter of the CUs, or K within one tiled K slice, or
// K within one wide step where a split-K launch would first need a clearing
// launch (C not known to hold zeros).  A longer K over few tiles (the fully
// connected layers: 22 rows, K = 256..1024, outputs cleared once per forward) is
// spread over more CUs by the split-K tiled kernel (K = 256 by 1024 columns: 16
// wide workgroups took 8.3 us, the split-K launch's 64 about 6).
template <typename T>
static bool use_wide(const Launch &L, const GemmArgs<T> &g) {
  if ((L.gemm != 0 && L.gemm != 3) || !use_mfma(L, g)) return false;
  constexpr int KT = kWideK * 4 / int(sizeof(T));
  const bool zeroed = g.c_zero && !g.Cin;
  return gemm_tiles(g) >= L.num_cu / 4 || g.K <= mfma_bk<T>() || (g.K <= KT && !zeroed);
}
// rows of A (and of the masks and second segment) read as 16-byte groups
template <typename T>
static bool wide_vec_a(const GemmArgs<T> &g) {
  constexpr int wpg = 16 / int(sizeof(T));
  return g.K % wpg == 0 && (g.batch == 1 || g.sA % wpg == 0) && aligned16(g.A1) && aligned16(g.A2) &&
         aligned16(g.A1b);
}
template <typename T, int KW>
static void launch_wide_kw(const Launch &L, dim3 grid, const GemmArgs<T> &g) {
  if (wide_vec_a(g))
    hipLaunchKernelGGL((k_gemm_wide<T, KW, true>), grid, dim3(kWideThreads), 0, L.stream, g);
  else
    hipLaunchKernelGGL((k_gemm_wide<T, KW, false>), grid, dim3(kWideThreads), 0, L.stream, g);
}
template <typename T>
static hipError_t launch_wide(const Launch &L, const GemmArgs<T> &g) {
  const size_t wgs = size_t((g.N + 63) / 64) * size_t((g.M + 63) / 64) * size_t(g.batch);
  if (wgs > size_t(INT32_MAX)) return hipErrorInvalidValue;  // one-dimensional, XCD-ordered launch
  const dim3 grid{unsigned(wgs), 1u, 1u};
  const int steps = wide_steps<T, kWideK>(g);  // the narrowest step width that takes no more steps
  if (wide_steps<T, kWideKShort>(g) == steps)
    launch_wide_kw<T, kWideKShort>(L, grid, g);
  else if (wide_steps<T, kWideKMid>(g) == steps)
    launch_wide_kw<T, kWideKMid>(L, grid, g);
  else
    launch_wide_kw<T, kWideK>(L, grid, g);
  return hipGetLastError();
}

// The panel kernel: automatic path selection (MPCX_GEMM=auto), operands whose
// rows and columns are whole 16-byte groups at 16-byte aligned addresses,
// matrices below 2 GiB per batch entry, and either K within one step or enough
// workgroups for half the CUs at 16 columns; a long K over few tiles (the fully
// connected layers: 22 rows, K = 312..1024) goes to the split-K tiled kernel.
// Workgroups of 3 waves (48 rows: a 140-row product as 48 + 48 + 44) for short
// matrices, else 4; in Z_2^32 32 columns per workgroup when that still gives a
// workgroup per CU, else 16 (Z_2^64: 16).
template <typename T>
static bool pan_vec(const T *p, size_t stride, int batch) {
  constexpr int wpg = 16 / int(sizeof(T));
  return aligned16(p) && (batch == 1 || stride % wpg == 0);
}
template <typename T>
static int pan_rw(int M) {
  return M <= 160 ? 3 : 4;
}
template <typename T>
static bool use_panels(const Launch &L, const PanelArgs<T> &r) {
  // Z_2^32 only: in Z_2^64 the eight-shift products measured slower here than
  // on the wide-K and fused kernels (GEMM time per bw=64 forward 0.99 against
  // 0.78 ms)
  if (sizeof(T) != 4 || L.gemm != 0 || r.M <= 0 || r.N <= 0 || r.K <= 0 || r.batch <= 0) return false;
  constexpr int wpg = 16 / int(sizeof(T)), KT = kPanKPW * 4 / int(sizeof(T));
  bool ok = r.K % wpg == 0 && r.N % wpg == 0 && size_t(r.M) * r.K * sizeof(T) < size_t(kPanOob) &&
            size_t(r.K) * r.N * sizeof(T) < size_t(kPanOob);
  for (int p = 0; p < r.np; p++)
    ok = ok && pan_vec(r.a1[p], r.sA, r.batch) && pan_vec(r.a2[p], r.sA, r.batch) &&
         pan_vec(r.b1[p], r.sB, r.batch) && pan_vec(r.b2[p], r.sB, r.batch) &&
         (p == 0 || (!r.a2[p] && !r.b2[p]));  // masks on the first panel only
  const int rw = pan_rw<T>(r.M);
  const size_t wgs = size_t((r.N + 15) / 16) * ((r.M + 16 * rw - 1) / (16 * rw)) * r.batch;
  return ok && (r.K <= KT || wgs >= size_t(L.num_cu / 2));
}
template <typename T, int NP, int RW, int NT>
static hipError_t launch_panels_v(const Launch &L, const PanelArgs<T> &r) {
  const size_t wgs = size_t((r.N + 16 * NT - 1) / (16 * NT)) * size_t((r.M + 16 * RW - 1) / (16 * RW)) * r.batch;
  if (wgs > size_t(INT32_MAX)) return hipErrorInvalidValue;  // one-dimensional, XCD-ordered launch
  hipLaunchKernelGGL((k_panels<T, NP, RW, NT>), dim3(unsigned(wgs)), dim3(64 * RW), 0, L.stream, r);
  return hipGetLastError();
}
template <int NP, int RW, int NT>
static hipError_t launch_panels_pf(const Launch &L, const PanelArgs<uint32_t> &r) {
  const size_t wgs = size_t((r.N + 16 * NT - 1) / (16 * NT)) * size_t((r.M + 16 * RW - 1) / (16 * RW)) * r.batch;
  if (wgs > size_t(INT32_MAX)) return hipErrorInvalidValue;  // one-dimensional, XCD-ordered launch
  hipLaunchKernelGGL((k_panels_pf<NP, RW, NT>), dim3(unsigned(wgs)), dim3(64 * RW), 0, L.stream, r);
  return hipGetLastError();
}
template <typename T, int NP>
static hipError_t launch_panels_np(const Launch &L, const PanelArgs<T> &r) {
  const int rw = pan_rw<T>(r.M);
  const size_t groups = size_t((r.M + 16 * rw - 1) / (16 * rw)) * r.batch;
  if constexpr (sizeof(T) == 4 && NP >= 2) {
    if (L.panel_pf && r.K <= kPanKPW) {
      // 16, 32 or 48 columns per workgroup: the fewest rounds of resident
      // workgroups (two per CU) times the chain, which grows with the columns
      // (one step per column tile plus about one for the loads and stagings)
      int nt = L.panel_nt;
      if (nt < 1 || nt > 3) {
        size_t best = SIZE_MAX;
        for (int t = 1; t <= 3; t++) {
          const size_t wgs = size_t((r.N + 16 * t - 1) / (16 * t)) * groups, slots = size_t(2) * L.num_cu;
          const size_t cost = (wgs + slots - 1) / slots * size_t(1 + t);
          if (cost < best) best = cost, nt = t;
        }
      }
      if (rw == 3)
        return nt == 1 ? launch_panels_pf<NP, 3, 1>(L, r) : nt == 2 ? launch_panels_pf<NP, 3, 2>(L, r)
                                                                    : launch_panels_pf<NP, 3, 3>(L, r);
      return nt == 1 ? launch_panels_pf<NP, 4, 1>(L, r) : nt == 2 ? launch_panels_pf<NP, 4, 2>(L, r)
                                                                  : launch_panels_pf<NP, 4, 3>(L, r);
    }
  }
  if constexpr (sizeof(T) == 4) {
    if (size_t((r.N + 31) / 32) * groups >= size_t(L.num_cu))
      return rw == 3 ? launch_panels_v<T, NP, 3, 2>(L, r) : launch_panels_v<T, NP, 4, 2>(L, r);
  }
  return rw == 3 ? launch_panels_v<T, NP, 3, 1>(L, r) : launch_panels_v<T, NP, 4, 1>(L, r);
}
template <typename T>
static hipError_t launch_panels(const Launch &L, const PanelArgs<T> &r) {
  if constexpr (sizeof(T) != 4) {
    return hipErrorInvalidValue;  // use_panels refuses Z_2^64
  } else {
    switch (r.np) {
      case 1: return launch_panels_np<T, 1>(L, r);
      case 2: return launch_panels_np<T, 2>(L, r);
      case 3: return launch_panels_np<T, 3>(L, r);
      default: return hipErrorInvalidValue;
    }
  }
}
// GemmArgs as panels: (A1 - A2)(B1 - B2), then A1b B1b, both with g.sign
template <typename T>
static void panels_add(PanelArgs<T> &r, const GemmArgs<T> &g) {
  r.a1[r.np] = g.A1;
  r.a2[r.np] = g.A2;
  r.b1[r.np] = g.B1;
  r.b2[r.np] = g.B2;
  r.sign[r.np++] = g.sign;
  if (g.A1b) {
    r.a1[r.np] = g.A1b;
    r.b1[r.np] = g.B1b;
    r.sign[r.np++] = g.sign;
  }
}
template <typename T>
static PanelArgs<T> panels_of(const GemmArgs<T> &g) {
  PanelArgs<T> r;
  r.M = g.M;
  r.N = g.N;
  r.K = g.K;
  r.batch = g.batch;
  r.np = 0;
  r.sA = g.sA;
  r.sB = g.sB;
  r.sC = g.sC;
  r.cin0 = g.Cin;
  r.C = g.C;
  panels_add(r, g);
  return r;
}

// A single product whose K fits one wide step of at most kWideKMid words and
// whose 64 x 64 tiles occupy at least half the CUs runs faster on the wide
// kernel than on the panel kernel (3080 x 156 x 312, the GCN-3 public-weight
// product of 22 graphs: 8.3 against 10.0 us); smaller launches keep the panel
// kernel's smaller workgroups (140 x 156 x 312: 5.6 against 7.6 us).
template <typename T>
static bool prefer_wide(const Launch &L, const GemmArgs<T> &g) {
  return !g.A2 && !g.B2 && !g.A1b && use_wide(L, g) && wide_steps<T, kWideKMid>(g) == 1 &&
         gemm_tiles(g) >= L.num_cu / 2;
}
template <typename T>
hipError_t launch_gemm(const Launch &L, const GemmArgs<T> &g0) {
  if (g0.M <= 0 || g0.N <= 0 || g0.batch <= 0) return hipSuccess;
  if (use_dot(L, g0)) return launch_dot<T>(L, g0);
  {
    const PanelArgs<T> r = panels_of(g0);
    if (use_panels(L, r) && !prefer_wide(L, g0)) return launch_panels<T>(L, r);
  }
  if (use_wide(L, g0)) return launch_wide<T>(L, g0);
  const bool mfma = use_mfma(L, g0);
  if (g0.A1b && !mfma) {
    // the VALU kernel takes one K segment: add the second product in a second launch
    GemmArgs<T> a = g0, b = g0;
    a.A1b = a.B1b = nullptr;
    b.A1 = g0.A1b;
    b.B1 = g0.B1b;
    b.A2 = b.B2 = b.A1b = b.B1b = nullptr;
    b.Cin = b.C;
    hipError_t e = launch_gemm<T>(L, a);
    return e != hipSuccess ? e : launch_gemm<T>(L, b);
  }
  GemmArgs<T> g = g0;
  g.ksplit = gemm_ksplit(L, g, gemm_tiles(g), mfma);
  hipError_t e = gemm_init(L, g);
  if (e != hipSuccess) return e;
  dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, g.batch * g.ksplit);
  if (mfma) return launch_mfma(L, grid, g, g, int(grid.z));
  hipLaunchKernelGGL((k_gemm<T>), grid, dim3(256), 0, L.stream, g);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_gemm_pair(const Launch &L, const GemmArgs<T> &p0, const GemmArgs<T> &p1) {
  const bool empty0 = p0.M <= 0 || p0.N <= 0 || p0.batch <= 0;
  const bool empty1 = p1.M <= 0 || p1.N <= 0 || p1.batch <= 0;
  if (empty0 || empty1 || !use_mfma(L, p0) || !use_mfma(L, p1)) {
    hipError_t e = launch_gemm<T>(L, p0);
    return e != hipSuccess ? e : launch_gemm<T>(L, p1);
  }
  GemmArgs<T> g0 = p0, g1 = p1;
  const int tiles = gemm_tiles(g0) + gemm_tiles(g1);
  g0.ksplit = gemm_ksplit(L, g0, tiles, true);
  g1.ksplit = gemm_ksplit(L, g1, tiles, true);
  hipError_t e = gemm_init(L, g0);
  if (e == hipSuccess) e = gemm_init(L, g1);
  if (e != hipSuccess) return e;
  const int nz0 = g0.batch * g0.ksplit;
  dim3 grid((std::max(g0.N, g1.N) + 63) / 64, (std::max(g0.M, g1.M) + 63) / 64, nz0 + g1.batch * g1.ksplit);
  return launch_mfma(L, grid, g0, g1, nz0);
}

// k_sxs_fused applies to the Beaver pair as the SxS gates form it: party 0
// (A1 - A2)(B1 - B2) + Cin with sign +1, party 1 with the same A1 in its first
// segment, the same B1 in its second, no masks, sign -1; the same shapes and
// strides; enough tiles for a quarter of the CUs or K within one phase.
template <typename T>
static bool use_sxs_fused(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1) {
  if ((L.gemm != 0 && L.gemm != 3) || !use_mfma(L, g0) || !use_mfma(L, g1)) return false;
  const bool form = g0.A2 && g0.B2 && !g0.A1b && g0.sign == 1 && g1.A1 == g0.A1 && g1.B1b == g0.B1 && g1.A1b &&
                    g1.B1 && !g1.A2 && !g1.B2 && g1.sign == -1;
  const bool shape = g0.M == g1.M && g0.N == g1.N && g0.K == g1.K && g0.batch == g1.batch && g0.sA == g1.sA &&
                     g0.sB == g1.sB && g0.sC == size_t(g0.M) * g0.N && g1.sC == g0.sC;
  const int tiles = ((g0.N + kSxsTN - 1) / kSxsTN) * ((g0.M + kSxsTM - 1) / kSxsTM) * g0.batch;
  return form && shape && (tiles >= L.num_cu / 4 || g0.K <= sxs_kc<T>() * 4 / int(sizeof(T)));
}

// ---------------------------------------------------------------------------
// SxS gate (Z_2^32 or Z_2^64), both parties' products and their sum, staged
// through LDS in steps of K (the oracle's three products, one set of shift sums):
//   C = C0 + (A^ - RA0)(B^ - RB0)  +  C1 + A^ (-RB1) + (-RA1) B^
// Workgroup: three waves on a 48-row x 16 CT-column tile, wave w owning rows
// 16 w.. of it and all its columns (CT 16-column MFMA tiles), so a wave's
// A-side operands (three planes, one byte-shifted copy per digit shift) serve
// CT tiles.  A step stages 192 bytes of K (48 words of Z_2^32, 24 of Z_2^64):
// A^, RA0, RA1 rows as the digits of A^ - RA0, A^ and -RA1 ([m][k]); B^, RB0,
// RB1 rows as the digits of B^ - RB0, -RB1 and B^, as [k / KPC][n][k % KPC]
// (a lane's KPC = 16 / sizeof(T) k words of a column are one 16-byte cell: one
// LDS read per MFMA operand).  The digits, differences and negations are
// formed once per workgroup as the words go to LDS; a staging thread loads KPC
// k rows of VW columns (VW divides N), coalesced along the rows.  The next
// step's loads are in flight while this step's MFMAs run, C0 + C1 are loaded
// before the first step; 48 KB of LDS.  Rows of 52 32-bit words put the
// 16-byte A reads of consecutive rows in distinct bank groups.  Outside the
// matrices every load reads zero (offsets past the buffer resource) and every
// store is dropped.
// ---------------------------------------------------------------------------
constexpr int kStgRows = 48, kStgKW = 48, kStgLDK = kStgKW + 4, kStgThreads = 192;

template <int NW>
__device__ __forceinline__ void stg_load(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t (&v)[NW]) {
  if constexpr (NW == 4) {
    const v4u_t x = __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0);
    v[0] = x[0], v[1] = x[1], v[2] = x[2], v[3] = x[3];
  } else if constexpr (NW == 2) {
    typedef unsigned v2u_t __attribute__((ext_vector_type(2)));
    const v2u_t x = __builtin_amdgcn_raw_buffer_load_b64(r, int(off), 0, 0);
    v[0] = x[0], v[1] = x[1];
  } else {
    v[0] = __builtin_amdgcn_raw_buffer_load_b32(r, int(off), 0, 0);
  }
}
// one ring word (T) at a byte offset: zero past the resource
template <typename T>
__device__ __forceinline__ T stg_word(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  uint32_t v[sizeof(T) / 4];
  stg_load<sizeof(T) / 4>(r, off, v);
  if constexpr (sizeof(T) == 4) return v[0];
  else return (uint64_t(v[1]) << 32) | v[0];
}
template <typename T>
__device__ __forceinline__ void stg_store_word(__amdgpu_buffer_rsrc_t r, uint32_t off, T x) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(x, r, int(off), 0, 0);
  } else {
    typedef unsigned v2u_t __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(v2u_t{uint32_t(x), uint32_t(x >> 32)}, r, int(off), 0, 0);
  }
}

// T: the ring (Z_2^32 or Z_2^64); CT: 16-column MFMA tiles per wave; VW: ring
// words per B load along a row (VW divides N).  A 16-byte group holds KPC =
// 16 / sizeof(T) words; a step is 192 bytes of K (48 or 24 words, three 64-byte
// MFMA chunks); shift s of the sizeof(T) digit shifts pairs digit j of an A word
// with digit s - j of the B word.
template <typename T, int CT, int VW>
__global__ __launch_bounds__(kStgThreads, 2) void k_sxs_staged(GemmArgs<T> g0, GemmArgs<T> g1) {
  constexpr int WB = int(sizeof(T)), NQ = WB, KPC = 16 / WB, KW = 192 / WB, TN = 16 * CT, GR = 12;
  constexpr int NG = TN / VW, NV = VW * WB / 4;  // B groups per k row, 32-bit words per B load
  constexpr int SA = kStgRows * GR / kStgThreads;  // A groups (row, 16 bytes) per thread and plane
  constexpr int SB = GR * NG / kStgThreads;        // B blocks (KPC k rows, VW columns) per thread and plane
  static_assert(kStgRows * GR % kStgThreads == 0 && GR * NG % kStgThreads == 0, "whole slots");
  static_assert(NV >= 1 && NV <= 4, "B loads of 4, 8 or 16 bytes");
  constexpr int APL = kStgRows * kStgLDK, BPL = GR * TN * 4;  // 32-bit words per A and B plane
  __shared__ __align__(16) uint32_t As[3 * APL];  // A^ - RA0, A^, -RA1 as [m][k] (52 words a row)
  __shared__ __align__(16) uint32_t Bs[3 * BPL];  // B^ - RB0, -RB1, B^ as [k / KPC][n][k % KPC]
  const int M = g0.M, N = g0.N, K = g0.K;
  const int gx = (N + TN - 1) / TN, gy = (M + kStgRows - 1) / kStgRows;
  const int lw = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const int bz = lw / (gx * gy), m0 = (lw / gx) % gy * kStgRows, n0 = lw % gx * TN;
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
  const size_t mk = size_t(M) * K, kn = size_t(K) * N, mn = size_t(M) * N;
  const __amdgpu_buffer_rsrc_t rah = pan_rsrc(g0.A1 + size_t(bz) * g0.sA, mk * WB);
  const __amdgpu_buffer_rsrc_t ra0 = pan_rsrc(g0.A2 + size_t(bz) * g0.sA, mk * WB);
  const __amdgpu_buffer_rsrc_t ra1 = pan_rsrc(g1.A1b + size_t(bz) * g1.sA, mk * WB);
  const __amdgpu_buffer_rsrc_t rbh = pan_rsrc(g0.B1 + size_t(bz) * g0.sB, kn * WB);
  const __amdgpu_buffer_rsrc_t rb0 = pan_rsrc(g0.B2 + size_t(bz) * g0.sB, kn * WB);
  const __amdgpu_buffer_rsrc_t rb1 = pan_rsrc(g1.B1 + size_t(bz) * g1.sB, kn * WB);
  // this lane's outputs (rows m0 + 16 wave + 4 lg + r, columns n0 + 16 t + li)
  // and their C0 + C1, loaded first so that they arrive during the products
  const __amdgpu_buffer_rsrc_t rc0 = pan_rsrc(g0.Cin + size_t(bz) * g0.sC, mn * WB);
  const __amdgpu_buffer_rsrc_t rc1 = pan_rsrc(g1.Cin + size_t(bz) * g1.sC, mn * WB);
  uint32_t co[CT][4];
  T c0v[CT][4], c1v[CT][4];
#pragma unroll
  for (int t = 0; t < CT; t++) {
    const int on = n0 + 16 * t + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int om = m0 + 16 * wave + 4 * lg + r;
      co[t][r] = (uint32_t(om < M ? om : 0) * uint32_t(N) + uint32_t(on < N ? on : 0)) * uint32_t(WB) |
                 (om < M && on < N ? 0u : kPanOob);
      c0v[t][r] = stg_word<T>(rc0, co[t][r]);
      c1v[t][r] = stg_word<T>(rc1, co[t][r]);
    }
  }
  // staging slots: A group (row f / GR, bytes 16 (f % GR)..) and B block (k rows
  // KPC (f / NG).. + KPC - 1, columns VW (f % NG)..)
  uint32_t aoff[SA], aoob[SA], boff[SB], boob[SB];
#pragma unroll
  for (int j = 0; j < SA; j++) {
    const int f = tid + kStgThreads * j, r = f / GR;
    aoob[j] = m0 + r < M ? 0u : kPanOob;
    aoff[j] = (uint32_t(m0 + r < M ? m0 + r : 0) * uint32_t(K) + uint32_t(KPC * (f % GR))) * uint32_t(WB);
  }
#pragma unroll
  for (int j = 0; j < SB; j++) {
    const int f = tid + kStgThreads * j, n = n0 + VW * (f % NG);
    boob[j] = n < N ? 0u : kPanOob;
    boff[j] = (uint32_t(KPC * (f / NG)) * uint32_t(N) + uint32_t(n < N ? n : 0)) * uint32_t(WB);
  }
  uint32_t xa[SA][3][4], xb[SB][3][KPC][NV];
  auto load = [&](int kb) {
#pragma unroll
    for (int j = 0; j < SA; j++) {
      const int f = tid + kStgThreads * j;
      const uint32_t o =
          (aoff[j] + uint32_t(kb) * uint32_t(WB)) | aoob[j] | (kb + KPC * (f % GR) < K ? 0u : kPanOob);
      stg_load<4>(rah, o, xa[j][0]);
      stg_load<4>(ra0, o, xa[j][1]);
      stg_load<4>(ra1, o, xa[j][2]);
    }
#pragma unroll
    for (int j = 0; j < SB; j++) {
      const int f = tid + kStgThreads * j, k = kb + KPC * (f / NG);  // K % KPC == 0: all rows inside K, or none
      const uint32_t o =
          (boff[j] + uint32_t(kb) * uint32_t(N) * uint32_t(WB)) | boob[j] | (k < K ? 0u : kPanOob);
#pragma unroll
      for (int i = 0; i < KPC; i++) {
        const uint32_t oi = o + uint32_t(i) * uint32_t(N) * uint32_t(WB);
        stg_load<NV>(rbh, oi, xb[j][0][i]);
        stg_load<NV>(rb0, oi, xb[j][1][i]);
        stg_load<NV>(rb1, oi, xb[j][2][i]);
      }
    }
  };
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  auto u4 = [](const uint32_t (&v)[4]) { return make_uint4(v[0], v[1], v[2], v[3]); };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < SA; j++) {
      const int f = tid + kStgThreads * j;
      uint32_t *p = &As[(f / GR) * kStgLDK + 4 * (f % GR)];
      const uint4 ah = u4(xa[j][0]);
      *reinterpret_cast<uint4 *>(p) = wide_digits<T>(ah, u4(xa[j][1]));
      *reinterpret_cast<uint4 *>(p + APL) = wide_digits<T>(ah, z4);
      *reinterpret_cast<uint4 *>(p + 2 * APL) = wide_digits<T>(z4, u4(xa[j][2]));
    }
#pragma unroll
    for (int j = 0; j < SB; j++) {
      const int f = tid + kStgThreads * j;
#pragma unroll
      for (int e = 0; e < VW; e++) {  // column VW (f % NG) + e: its KPC k words as one 16-byte cell
        uint32_t *p = &Bs[((f / NG) * TN + VW * (f % NG) + e) * 4];
        uint32_t c[3][4];
#pragma unroll
        for (int q = 0; q < 3; q++)
#pragma unroll
          for (int i = 0; i < KPC; i++)
#pragma unroll
            for (int h = 0; h < WB / 4; h++) c[q][i * (WB / 4) + h] = xb[j][q][i][e * (WB / 4) + h];
        const uint4 bh = u4(c[0]);
        *reinterpret_cast<uint4 *>(p) = wide_digits<T>(bh, u4(c[1]));
        *reinterpret_cast<uint4 *>(p + BPL) = wide_digits<T>(z4, u4(c[2]));
        *reinterpret_cast<uint4 *>(p + 2 * BPL) = wide_digits<T>(bh, z4);
      }
    }
  };
  const ShiftSel sel = pan_shift_selectors();
  v4i_t acc[CT][NQ];
#pragma unroll
  for (int t = 0; t < CT; t++)
#pragma unroll
    for (int q = 0; q < NQ; q++) acc[t][q] = v4i_t{0, 0, 0, 0};
  // a step's three chunks: A plane p against B plane p (p = 0, 1, 2)
  auto compute = [&]() {
    const int ar = (16 * wave + li) * kStgLDK + 4 * lg;
#pragma unroll
    for (int c = 0; c < 3; c++)
#pragma unroll
      for (int p = 0; p < 3; p++) {  // (A^ - RA0)(B^ - RB0), A^ (-RB1), (-RA1) B^
        v4i_t as[NQ];
        const uint4 a = *reinterpret_cast<const uint4 *>(&As[p * APL + ar + 16 * c]);
        if constexpr (sizeof(T) == 4)
          digit_shifts_s(a, sel, as);
        else
          digit_shifts<T>(a, as);
#pragma unroll
        for (int t = 0; t < CT; t++) {
          const uint4 b = *reinterpret_cast<const uint4 *>(&Bs[p * BPL + ((4 * c + lg) * TN + 16 * t + li) * 4]);
          const v4i_t bv = v4i_t{int(b.x), int(b.y), int(b.z), int(b.w)};
#pragma unroll
          for (int q = 0; q < NQ; q++) acc[t][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[q], bv, acc[t][q], 0, 0, 0);
        }
      }
  };
  load(0);
  for (int kb = 0; kb < K; kb += KW) {
    store();
    __syncthreads();
    if (kb + KW < K) load(kb + KW);  // in flight during this step's MFMAs
    compute();
    __syncthreads();
  }
  const __amdgpu_buffer_rsrc_t rc = pan_rsrc(g0.C + size_t(bz) * mn, mn * WB);
#pragma unroll
  for (int t = 0; t < CT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++)  // outside the matrix: dropped by the range check
      stg_store_word<T>(rc, co[t][r], T(c0v[t][r] + c1v[t][r] + digit_fold<T>(acc[t], r)));
}

// An SxS pair in the staged kernel's form: party 0's (A^ - RA0)(B^ - RB0) + C0
// and party 1's C1 - (A^ RB1 + RA1 B^) on one shape, K a whole number of
// 16-byte groups, 16-byte aligned operands, every matrix of a batch entry below
// 2 GiB; in Z_2^64 K below 2^15 (the shift sums' int32 range).
template <typename T>
static bool use_sxs_staged(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1) {
  constexpr size_t KPC = 16 / sizeof(T), WB = sizeof(T);
  if (!L.sxs_staged || (L.gemm != 0 && L.gemm != 3)) return false;
  const bool form = g0.A2 && g0.B2 && !g0.A1b && g0.sign == 1 && g1.A1 == g0.A1 && g1.B1b == g0.B1 && g1.A1b &&
                    g1.B1 && !g1.A2 && !g1.B2 && g1.sign == -1 && g0.Cin && g1.Cin && g0.C;
  const bool shape = g0.M == g1.M && g0.N == g1.N && g0.K == g1.K && g0.batch == g1.batch && g0.sA == g1.sA &&
                     g0.sB == g1.sB && g0.sC == size_t(g0.M) * g0.N && g1.sC == g0.sC;
  if (!form || !shape || g0.K % KPC != 0 || g0.sA % KPC != 0 || g0.sB % KPC != 0) return false;
  if (sizeof(T) == 8 && g0.K >= (1 << 15)) return false;
  const size_t lim = size_t(kPanOob);
  if (size_t(g0.M) * g0.K * WB >= lim || size_t(g0.K) * g0.N * WB >= lim || size_t(g0.M) * g0.N * WB >= lim)
    return false;
  for (const void *q : {(const void *)g0.A1, (const void *)g0.A2, (const void *)g1.A1b, (const void *)g0.B1,
                        (const void *)g0.B2, (const void *)g1.B1})
    if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return false;
  return true;
}
template <typename T, int CT, int VW>
static hipError_t launch_sxs_staged_at(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1, T *out) {
  const size_t wgs = size_t((g0.N + 16 * CT - 1) / (16 * CT)) * size_t((g0.M + kStgRows - 1) / kStgRows) * g0.batch;
  if (wgs > size_t(INT32_MAX)) return hipErrorInvalidValue;
  GemmArgs<T> a = g0;
  a.C = out;
  hipLaunchKernelGGL((k_sxs_staged<T, CT, VW>), dim3(unsigned(wgs)), dim3(kStgThreads), 0, L.stream, a, g1);
  return hipGetLastError();
}
// 32 columns per workgroup; groups of 2 or 1 words along B's rows, whichever
// divides N
template <typename T>
static hipError_t launch_sxs_staged(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1, T *out) {
  return g0.N % 2 == 0 ? launch_sxs_staged_at<T, 2, 2>(L, g0, g1, out) : launch_sxs_staged_at<T, 2, 1>(L, g0, g1, out);
}

template <typename T>
hipError_t launch_gemm_pair_sum(const Launch &L, const GemmArgs<T> &g0, const GemmArgs<T> &g1, T *out) {
  if (g0.M <= 0 || g0.N <= 0 || g0.batch <= 0) return hipSuccess;
  if (use_sxs_staged(L, g0, g1)) return launch_sxs_staged<T>(L, g0, g1, out);
  const bool same = g0.M == g1.M && g0.N == g1.N && g0.K == g1.K && g0.batch == g1.batch && g0.sA == g1.sA &&
                    g0.sB == g1.sB && g0.sC == size_t(g0.M) * g0.N && g1.sC == g0.sC;
  if (same && (g0.A1b ? 2 : 1) + (g1.A1b ? 2 : 1) <= 3) {  // both parties' products and the sum in one launch
    PanelArgs<T> r = panels_of(g0);
    panels_add(r, g1);
    r.cin1 = g1.Cin;
    r.C = out;
    if (use_panels(L, r)) return launch_panels<T>(L, r);
  }
  if (use_sxs_fused(L, g0, g1)) {
    GemmArgs<T> a = g0;
    a.C = out;
    const size_t wgs = size_t((g0.N + kSxsTN - 1) / kSxsTN) * size_t((g0.M + kSxsTM - 1) / kSxsTM) * size_t(g0.batch);
    if (wgs > size_t(INT32_MAX)) return hipErrorInvalidValue;  // one-dimensional, XCD-ordered launch
    const dim3 grid{unsigned(wgs), 1u, 1u};
    if (wide_vec_a(g0) && wide_vec_a(g1))
      hipLaunchKernelGGL((k_sxs_fused<T, true>), grid, dim3(kSxsThreads), 0, L.stream, a, g1);
    else
      hipLaunchKernelGGL((k_sxs_fused<T, false>), grid, dim3(kSxsThreads), 0, L.stream, a, g1);
    return hipGetLastError();
  }
  hipError_t e = launch_gemm_pair<T>(L, g0, g1);
  if (e != hipSuccess) return e;
  return launch_reconstruct<T>(L, size_t(g0.batch) * g0.M * g0.N, g0.C, g1.C, out);
}


#define INST(T)                                                                                                      \
  template hipError_t launch_gemm<T>(const Launch &, const GemmArgs<T> &);                                           \
  template hipError_t launch_gemm_pair<T>(const Launch &, const GemmArgs<T> &, const GemmArgs<T> &);                \
  template hipError_t launch_gemm_pair_sum<T>(const Launch &, const GemmArgs<T> &, const GemmArgs<T> &, T *);

INST(uint32_t)
INST(uint64_t)

}  // namespace mpcx
