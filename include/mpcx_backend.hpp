// mpcx_backend.hpp -- header-only C++ backend over the libmpcx C ABI with the
// operation set of the reference's sytorch Backend<T> (the virtuals that
// DDGOrcaBase<T> / DDGOrca<T> / DDGOrcaBatched<T> implement for evaluation and
// the ...Keygen classes for the dealer: gpu_mpc/ddg_orca_base.h:170-322,
// 326-526; gpu_mpc/ddg_orca.h:43-139, 169-268).
//
// One object runs in one of two modes, as the reference's two backend families
// do: the dealer walks the model with tensors holding MASKS and appends both
// parties' keys at a cursor; the evaluator walks it again with tensors holding
// MASKED VALUES (x + r, the same for both parties) and consumes the keys in the
// same order.  Both parties are evaluated by every call (one process, one GPU).
//
// Tensor requirements (duck-typed, as sytorch's Tensor / Tensor2D): a device
// pointer member `d_data` (T*), `size()` (element count); 2-D operands of matmul
// also `d1`, `d2` (rows, cols).  MpcxTensor below is a minimal such type.
// Outputs whose d_data is null are allocated by the backend (hipMalloc) and
// freed with it, like the reference's gpuMalloc'd outputs.  Work is enqueued on
// the context's stream; callers that touch the tensors with other streams or
// plain hipMemcpy call mpcx_synchronize first.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "mpcx.h"

namespace mpcx {

template <typename T>
struct MpcxTensor {
  T *d_data = nullptr;
  size_t d1 = 0, d2 = 1;
  size_t size() const { return d1 * d2; }
};

// Both parties' device key arenas and the shared cursor.
struct KeyArena {
  uint8_t *d_key[2] = {nullptr, nullptr};
  size_t capacity = 0;
  size_t offset = 0;
};

template <typename T>
class SecureBackend {
 public:
  enum class Mode { Dealer, Evaluator };

  SecureBackend(mpcx_ctx *ctx, Mode mode, KeyArena *arena, uint64_t seed = 1)
      : ctx_(ctx), mode_(mode), arena_(arena), seed_(seed) {
    if (!ctx_ || !arena_) throw std::invalid_argument("SecureBackend: null context or arena");
    if (mpcx_bw(ctx_) != int(8 * sizeof(T))) throw std::invalid_argument("SecureBackend: T does not match bw");
    scale_ = mpcx_scale(ctx_);
  }
  ~SecureBackend() {
    for (void *p : owned_) (void)hipFree(p);
  }
  SecureBackend(const SecureBackend &) = delete;
  SecureBackend &operator=(const SecureBackend &) = delete;

  bool dealer() const { return mode_ == Mode::Dealer; }
  size_t key_offset() const { return arena_->offset; }

  // ---- reveal of a secret-shared leaf (revealIfLeaf, ddg_orca_base.h:72-89) ----
  // Dealer: `out` receives the input mask.  Evaluator: the parties' additive
  // shares s0, s1 -> masked value in `out`.
  template <class TS, class TO>
  void reveal(const TS &s0, const TS &s1, TO &out) {
    const size_t n = s0.size();
    ensure(out, n);
    const size_t kb = mpcx_reveal_key_bytes(ctx_, n);
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer())
      check(mpcx_reveal_keygen(ctx_, n, out.d_data, seed_, gate_++, k0, k1));
    else
      check(mpcx_reveal_eval(ctx_, n, k0, k1, s0.d_data, s1.d_data, out.d_data));
  }

  // ---- secret x secret matmul, c = a . b (ddg_orca_base.h:170-205 / 394-410) ----
  template <class TA, class TB, class TC>
  void matmul(const TA &a, const TB &b, TC &c) {
    const int M = int(a.d1), K = int(a.d2), N = int(b.d2);
    if (size_t(K) != b.d1) throw std::invalid_argument("matmul: inner dimensions differ");
    ensure(c, size_t(M) * N);
    const size_t kb = mpcx_sxs_key_bytes(ctx_, 1, M, K, N);
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer())
      check(mpcx_sxs_keygen(ctx_, 1, M, K, N, a.d_data, b.d_data, c.d_data, seed_, gate_++, k0, k1));
    else
      check(mpcx_sxs_eval(ctx_, 1, M, K, N, k0, k1, a.d_data, b.d_data, c.d_data));
  }

  // ---- secret x public matmul with optional bias (ddg_orca_base.h:208-271) ----
  // W (K x N, public ring weights on the device); bias (N, scale s) is added at
  // scale 2s (<< s) by the evaluator only: a public addend has mask 0.
  template <class TA, class TW, class TC, class TD>
  void matmul(const TA &a, const TW &W, TC &c, bool useBias, const TD &bias, bool /*isFirst*/) {
    const int M = int(a.d1), K = int(a.d2), N = int(W.d2);
    if (size_t(K) != W.d1) throw std::invalid_argument("matmul: inner dimensions differ");
    ensure(c, size_t(M) * N);
    check(mpcx_ring_gemm(ctx_, M, K, N, a.d_data, W.d_data, c.d_data));
    if (useBias && !dealer())
      check(mpcx_ring_lincomb(ctx_, size_t(M), size_t(N), 1, c.d_data, 0, nullptr, bias.d_data, scale(),
                              c.d_data));
  }

  // ---- element-wise fixed-point product (ddg_orca.h:43-63, keygen :176-193):
  // Beaver product with identity maps, then truncation by the scale with slack
  // (the reference's TrWithSlack: MPCX_TRSLACK, exact for |a*b| < 2^(bw-2)) ----
  template <class TA, class TB, class TO>
  void mul(const TA &a, const TB &b, TO &out) {
    const size_t n = a.size();
    if (b.size() != n) throw std::invalid_argument("mul: shape mismatch");
    ensure(out, n);
    const uint32_t *idx = identity(n);
    const size_t kb = mpcx_mul_key_bytes(ctx_, n, n, n);
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer())
      check(mpcx_mul_keygen(ctx_, n, n, n, idx, idx, a.d_data, b.d_data, out.d_data, seed_, gate_++, k0, k1));
    else
      check(mpcx_mul_eval(ctx_, n, n, n, idx, idx, k0, k1, a.d_data, b.d_data, out.d_data));
    gate(MPCX_TRSLACK, out, out, nullptr, 0);
  }

  // ---- local linear ops (no key, no exchange) ----
  template <class TX, class TY>
  void scalarmul(const TX &x, T scalar, TY &y) {  // ddg_orca.h:65-71
    ensure(y, x.size());
    check(mpcx_ring_lincomb(ctx_, 1, x.size(), uint64_t(scalar), x.d_data, 0, nullptr, nullptr, 0, y.d_data));
  }
  template <class TB, class TA, class TO>
  void sub(const TB &b, const TA &a, TO &out) {  // out = b - a, ddg_orca.h:73-81
    ensure(out, b.size());
    check(mpcx_ring_lincomb(ctx_, 1, b.size(), 1, b.d_data, ~uint64_t(0), a.d_data, nullptr, 0, out.d_data));
  }
  template <class TI, class TO>
  void add(const std::vector<TI *> &in, TO &out) {  // ddg_orca_base.h:304-314
    if (in.empty()) throw std::invalid_argument("add: no inputs");
    const size_t n = in[0]->size();
    ensure(out, n);
    check(mpcx_ring_lincomb(ctx_, 1, n, 1, in[0]->d_data, 0, nullptr, nullptr, 0, out.d_data));
    for (size_t i = 1; i < in.size(); i++)
      check(mpcx_ring_lincomb(ctx_, 1, n, 1, out.d_data, 1, in[i]->d_data, nullptr, 0, out.d_data));
  }

  // ---- ReLU (ddg_orca.h:83-110): one (bw-1)-bit DCF + select, two rounds ----
  template <class TI, class TO>
  void relu(const TI &in, TO &out) {
    gate(MPCX_RELU, in, out, nullptr, 0);
  }

  // ---- masked global max-pool (MaskedMaxPoolLayer<T>(B, Nmax, F)::_forward,
  // masked_maxpool_layer.h:47-165): in (B*N, C) sample-major -> out (B, C), a
  // tree of max(a, b) = a + ReLU(b - a), two rounds per level ----
  template <class TI, class TO>
  void maxpool(const TI &in, TO &out, int B, int N, int C) {
    if (in.size() != size_t(B) * N * C) throw std::invalid_argument("maxpool: input is not (B*N, C)");
    ensure(out, size_t(B) * C);
    const size_t kb = mpcx_maxpool_key_bytes(ctx_, B, N, C);
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer()) {
      check(mpcx_maxpool_keygen(ctx_, B, N, C, in.d_data, out.d_data, seed_, gate_, k0, k1));
      gate_ += uint32_t(mpcx_maxpool_levels(N));
    } else {
      check(mpcx_maxpool_eval(ctx_, B, N, C, k0, k1, in.d_data, out.d_data));
    }
  }

  // ---- truncation by the scale: exact (ddg_orca.h:112-123, TrFloor) by default,
  // as TrFloor composes it: the truncate-reduce MPCX_TRMOD then the sign
  // extension MPCX_EXT (dpf_dcf_adapter.h:274-303);
  // set_truncation(MPCX_LOCALARS) selects the reference batched backend's default
  // local shift (ddg_orca_batched.h:180-199: no key, no exchange, not exact) and
  // MPCX_TRSLACK the exact truncation for |x| < 2^(bw-2).  The dealer and the
  // evaluator must select the same kind (the reference reads DDG_EXACT_TRUNC on
  // both sides, ddg_orca_batched.h:133-134, 239-240). ----
  void set_truncation(int kind) {
    if (kind != MPCX_TR && kind != MPCX_TRSLACK && kind != MPCX_LOCALARS)
      throw std::invalid_argument("set_truncation: MPCX_TR, MPCX_TRSLACK or MPCX_LOCALARS");
    trunc_kind_ = kind;
  }
  template <class TI>
  void truncateForward(TI &in, uint64_t shift, uint8_t /*mode*/ = 0) {
    if (int(shift) != scale()) throw std::invalid_argument("truncateForward: shift must equal the scale");
    if (trunc_kind_ == MPCX_TR) {
      gate(MPCX_TRMOD, in, in, nullptr, 0);
      gate(MPCX_EXT, in, in, nullptr, 0);
    } else {
      gate(trunc_kind_, in, in, nullptr, 0);
    }
  }

  // ---- truncation + bias + ReLU: the truncate-reduce, then the ReLU fused into
  // the sign extension (gpuReluExtend, dpf_dcf_adapter.h:225-234), four rounds ----
  template <class TI, class TO, class TD>
  void truncate_bias_relu(const TI &in, TO &out, const TD &bias) {
    gate(MPCX_TRMOD, in, out, bias.d_data, int(bias.size()));
    gate(MPCX_EXTRELU, out, out, nullptr, 0);
  }

  // ---- output (ddg_orca_base.h:296-302 / 511-517) ----
  // Dealer: writes the output mask (in the clear) into both keys.  Evaluator:
  // unmasks, shifts right by the scale (floor), copies to h_out (int64).
  template <class TA>
  void output(const TA &a, int64_t *h_out = nullptr) {
    const size_t n = a.size(), tb = sizeof(T);
    const size_t kb = (n * tb + 255) / 256 * 256;
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer()) {
      // the mask may still be in flight on the context's stream
      check(mpcx_synchronize(ctx_));
      check_hip(hipMemcpy(k0, a.d_data, n * tb, hipMemcpyDeviceToDevice));
      check_hip(hipMemcpy(k1, a.d_data, n * tb, hipMemcpyDeviceToDevice));
      return;
    }
    check(mpcx_ring_lincomb(ctx_, 1, n, 1, a.d_data, ~uint64_t(0), k0, nullptr, 0, a.d_data));
    check(mpcx_synchronize(ctx_));
    if (h_out) {
      std::vector<T> v(n);
      check_hip(hipMemcpy(v.data(), a.d_data, n * tb, hipMemcpyDeviceToHost));
      for (size_t i = 0; i < n; i++) {
        int64_t x = sizeof(T) == 4 ? int64_t(int32_t(uint32_t(v[i]))) : int64_t(v[i]);
        h_out[i] = x >> scale();
      }
    }
  }

 private:
  int scale() const { return scale_; }

  template <class TI, class TO>
  void gate(int kind, const TI &in, TO &out, const T *bias, int ncol) {
    const size_t n = in.size();
    ensure(out, n);
    const size_t kb = mpcx_tr_key_bytes(ctx_, kind, n);
    uint8_t *k0, *k1;
    take(kb, &k0, &k1);
    if (dealer())
      check(mpcx_tr_keygen(ctx_, kind, n, in.d_data, out.d_data, seed_, gate_++, k0, k1));
    else
      check(mpcx_tr_eval(ctx_, kind, n, k0, k1, in.d_data, bias, ncol, out.d_data));
  }

  void take(size_t bytes, uint8_t **k0, uint8_t **k1) {
    if (arena_->offset + bytes > arena_->capacity) throw std::length_error("SecureBackend: key arena exhausted");
    *k0 = arena_->d_key[0] + arena_->offset;
    *k1 = arena_->d_key[1] + arena_->offset;
    arena_->offset += bytes;
  }

  template <class TO>
  void ensure(TO &t, size_t n) {
    if (t.d_data) return;
    void *p = nullptr;
    check_hip(hipMalloc(&p, n * sizeof(T)));
    owned_.push_back(p);
    t.d_data = static_cast<T *>(p);
  }

  const uint32_t *identity(size_t n) {
    if (n > ident_n_) {
      std::vector<uint32_t> h(n);
      for (size_t i = 0; i < n; i++) h[i] = uint32_t(i);
      void *p = nullptr;
      check_hip(hipMalloc(&p, n * 4));
      owned_.push_back(p);
      check_hip(hipMemcpy(p, h.data(), n * 4, hipMemcpyHostToDevice));
      ident_ = static_cast<uint32_t *>(p);
      ident_n_ = n;
    }
    return ident_;
  }

  void check(mpcx_status st) {
    if (st != MPCX_OK) throw std::runtime_error(std::string("libmpcx: ") + mpcx_last_error(ctx_));
  }
  static void check_hip(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e));
  }

  mpcx_ctx *ctx_;
  Mode mode_;
  KeyArena *arena_;
  uint64_t seed_;
  uint32_t gate_ = 1;
  int scale_ = 12;
  int trunc_kind_ = MPCX_TR;
  std::vector<void *> owned_;
  uint32_t *ident_ = nullptr;
  size_t ident_n_ = 0;
};

}  // namespace mpcx
