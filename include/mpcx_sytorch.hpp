// mpcx_sytorch.hpp -- sytorch Backend<T> subclasses over libmpcx, with the
// virtual signatures of the reference's backends:
//   MpcxOrca<T>        the evaluator, DDGOrcaBase<T> + DDGOrca<T>
//                      (gpu_mpc/ddg_orca_base.h:37-322, gpu_mpc/ddg_orca.h:30-139)
//   MpcxOrcaKeygen<T>  the dealer, DDGOrcaBaseKeygen<T> + DDGOrcaKeygen<T>
//                      (gpu_mpc/ddg_orca_base.h:326-526, gpu_mpc/ddg_orca.h:141-268)
// Include sytorch's backend and tensor declarations first (sytorch/backend/backend.h);
// the layers (_MatMul, FC, ReLU, GCNLayer, MaskedMaxPoolLayer, ...) then run on
// these backends unchanged, one process per party as the reference deploys them.
// Key files: the dealer appends every layer's key for its party to a host key
// buffer and writes <keyFile>_inference_key<party>.dat at close(); the
// evaluator reads that file and consumes the keys in the same order (the two
// passes stay in step because every key size is a function of the tensor sizes).
// The primitives are those of mpcx_ezpc.hpp; the differences from the
// reference's backends are:
//   - the public-weight matmul needs no key and no exchange: the dealer, which
//     holds the weights, sets the output mask to r_A . W (the key keeps the party's
//     share of r_A, for a leaf input's reveal);
//   - truncateForward is the exact truncation (truncate-reduce + sign extension,
//     the reference's TrFloor) for every mode, and optimize() leaves the graph as
//     it is (no ReluExtend fusion pass);
//   - errors abort with a message (the reference's checkCudaErrors / assert).
#pragma once
#include <chrono>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "mpcx_ezpc.hpp"

namespace mpcx_sytorch {
constexpr size_t kKeyBufBytes = size_t(1) << 30;  // dealer key buffer (host), grown never: 1 GiB

template <typename T>
inline T *dev_alloc(u64 n) {
  return reinterpret_cast<T *>(gpuMalloc(n * sizeof(T)));
}
enum : uint32_t { R_SXP_PUBLIC = 100 };

// Public weights and biases kept on the device across calls (a layer's weights
// do not change between forwards): keyed by the host array and its size, and
// checked against a host copy on every call, so weights changed in place are
// uploaded again.  Saves the upload and, above all, the hipMalloc / hipFree
// pair per call (hipFree waits for the whole device).
template <typename T>
class Resident {
 public:
  Resident() = default;
  Resident(const Resident &) = delete;
  Resident &operator=(const Resident &) = delete;
  ~Resident() {
    for (auto &kv : m_) gpuFree(kv.second.d);
  }
  const T *get(const T *h, u64 n) {
    Entry &e = m_[{h, n}];
    if (e.d && std::memcmp(e.host.data(), h, n * sizeof(T)) == 0) return e.d;
    if (!e.d) e.d = dev_alloc<T>(n);
    e.host.assign(h, h + n);
    mpcx_ezpc::hip_check(hipMemcpy(e.d, h, n * sizeof(T), hipMemcpyHostToDevice), "weights to device");
    return e.d;
  }

 private:
  struct Entry {
    std::vector<T> host;
    T *d = nullptr;
  };
  std::map<std::pair<const T *, u64>, Entry> m_;
};
}  // namespace mpcx_sytorch

// ===========================================================================
// evaluator
// ===========================================================================
template <typename T>
class MpcxOrca : public Backend<T> {
 public:
  u8 *startPtr = nullptr;
  u8 *keyBuf = nullptr;
  size_t keySize = 0;
  GpuPeer *peer = nullptr;
  int party = -1;
  Stats s;
  int bw = 0;
  int scale = 0;
  AESGlobalContext g;
  std::set<void *> unrevealedLeaves;

  void registerLeaf(void *d_ptr) { unrevealedLeaves.insert(d_ptr); }
  void resetLeaves() { unrevealedLeaves.clear(); }
  // A secret leaf (an additive share) becomes masked public on first use: add
  // this party's share of its mask, then reconstruct (ddg_orca_base.h:72-80).
  bool revealIfLeaf(T *d_data, T *d_mask, int bw_, u64 size) {
    if (!unrevealedLeaves.count(d_data)) return false;
    gpuLinearComb(bw_, size, d_data, T(1), d_data, T(1), d_mask);
    peer->reconstructInPlace(d_data, bw_, size, &s);
    unrevealedLeaves.erase(d_data);
    return true;
  }
  // Public leaf held by one party (the other holds 0): reconstruct (ddg_orca_base.h:84-89).
  void revealPublicLeaf(T *d_data, int bw_, u64 size) {
    if (unrevealedLeaves.count(d_data)) {
      peer->reconstructInPlace(d_data, bw_, size, &s);
      unrevealedLeaves.erase(d_data);
    }
  }

  // party, peer address (see SigmaPeer::connect), ring width and scale, and the
  // dealer's key file prefix (ddg_orca_base.h:93-116).
  MpcxOrca(int party_, std::string ip, int bw_, int scale_, std::string keyFile = "", bool compress = true)
      : party(party_), bw(mpcx_ezpc::bw_of<T>(bw_)), scale(scale_) {
    initAESContext(&g);
    initGPUMemPool();
    if (!keyFile.empty()) {
      const std::string fn = keyFile + "_inference_key" + std::to_string(party) + ".dat";
      keySize = std::filesystem::file_size(fn);
      getAlignedBuf(&keyBuf, keySize, false);
      std::ifstream f(fn, std::ios::binary);
      if (!f.read(reinterpret_cast<char *>(keyBuf), std::streamsize(keySize))) mpcx_ezpc::die("cannot read " + fn);
      startPtr = keyBuf;
    }
    peer = new GpuPeer(compress);
    if (!ip.empty()) peer->connect(party, ip);
    owns_channel_ = true;
  }
  // Both parties as two threads of one process: an end of mpcx_peer_pair and
  // this party's key bytes.
  MpcxOrca(int party_, mpcx_peer *end, int bw_, int scale_, u8 *keys, size_t bytes)
      : party(party_), bw(mpcx_ezpc::bw_of<T>(bw_)), scale(scale_) {
    initAESContext(&g);
    keyBuf = startPtr = keys;
    keySize = bytes;
    peer = new GpuPeer(false);
    peer->attach(end);
  }
  ~MpcxOrca() override {
    if (peer && !owns_channel_) peer->h = nullptr;  // an attached end stays with its owner
    delete peer;
    if (keyBuf && owns_channel_ && startPtr) cpuFree(startPtr, false);
  }
  void close() { peer->close(); }

  // secret x secret (the per-sample loop of _MatMul, layers.h:67-93, calls it per sample)
  void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c) override {
    const auto t0 = std::chrono::high_resolution_clock::now();
    MatmulParams p;
    p.M = int(a.d1);
    p.K = int(a.d2);
    p.N = int(b.d2);
    p.batchSz = 1;
    stdInit(p, bw, 0);
    auto k = readGPUMatmulKey<T>(p, TruncateType::None, &keyBuf);
    T *d_mask_A = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(k.A), k.mem_size_A, &s));
    T *d_mask_B = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(k.B), k.mem_size_B, &s));
    revealIfLeaf(a.d_data, d_mask_A, bw, p.size_A);
    revealIfLeaf(b.d_data, d_mask_B, bw, p.size_B);
    gpuFree(d_mask_B);
    c.d_data = gpuMatmul(peer, party, p, k, a.d_data, b.d_data, (T *)nullptr, TruncateType::None, &g, &s, true,
                         d_mask_A);
    gpuFree(d_mask_A);
    s.matmul_time += elapsed_us(t0);
  }

  // secret x public (FC): masked A times the public weights, + bias; no exchange.
  void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c, bool useBias, Tensor1D<T> &d,
              bool isFirst) override {
    const auto t0 = std::chrono::high_resolution_clock::now();
    auto r = mpcx_ezpc::take(&keyBuf, mpcx_sytorch::R_SXP_PUBLIC, "matmul (public weights)");
    const u64 M = a.d1, K = a.d2, N = b.d2;
    if (u64(r.h.p[0]) != M || u64(r.h.p[1]) != K || u64(r.h.p[2]) != N) mpcx_ezpc::die("matmul: key of another layer");
    if (isFirst || unrevealedLeaves.count(a.d_data)) {
      T *d_mask_A = reinterpret_cast<T *>(moveToGPU(r.payload, M * K * sizeof(T), &s));
      unrevealedLeaves.insert(a.d_data);
      revealIfLeaf(a.d_data, d_mask_A, bw, M * K);
      gpuFree(d_mask_A);
    }
    mpcx_ctx *cx = mpcx_ezpc::ctx(bw);
    const T *d_W = weights_.get(b.data, K * N);
    T *out = mpcx_sytorch::dev_alloc<T>(M * N);
    mpcx_ezpc::check(cx, mpcx_ring_gemm(cx, int(M), int(K), int(N), a.d_data, d_W, out), "matmul");
    if (useBias)
      mpcx_ezpc::check(cx, mpcx_ring_lincomb(cx, M, N, 1, out, 0, nullptr, weights_.get(d.data, N), 0, out),
                       "matmul bias");
    c.d_data = out;
    s.matmul_time += elapsed_us(t0);
  }

  // element-wise secret x secret, then the slack truncation (ddg_orca.h:43-63)
  void mul(const Tensor<T> &a, const Tensor<T> &b, Tensor<T> &out) override {
    const int N = int(a.size());
    if (!a.is_same_shape(b) || !a.is_same_shape(out)) mpcx_ezpc::die("mul: shape mismatch");
    auto k = readGPUMulKey<T>(&keyBuf, u64(N), u64(N), u64(N), TruncateType::TrWithSlack);
    T *d_mask_a = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(k.a), N * sizeof(T), &s));
    T *d_mask_b = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(k.b), N * sizeof(T), &s));
    revealIfLeaf(a.d_data, d_mask_a, bw, u64(N));
    revealIfLeaf(b.d_data, d_mask_b, bw, u64(N));
    gpuFree(d_mask_a);
    gpuFree(d_mask_b);
    out.d_data = gpuMul(peer, party, bw, scale, N, k, a.d_data, b.d_data, TruncateType::TrWithSlack, &g, &s);
  }

  void scalarmul(Tensor<T> &x, T scalar, Tensor<T> &y) override {
    y.d_data = mpcx_sytorch::dev_alloc<T>(x.size());
    gpuLinearComb(bw, x.size(), y.d_data, scalar, x.d_data);
  }
  void sub(Tensor<T> &b, Tensor<T> &a, Tensor<T> &out) override {
    out.d_data = mpcx_sytorch::dev_alloc<T>(b.size());
    gpuLinearComb(bw, b.size(), out.d_data, T(1), b.d_data, T(0) - T(1), a.d_data);
  }
  void add(const std::vector<Tensor<T> *> &in, Tensor<T> &out) override {
    std::vector<T *> d;
    for (auto *t : in) d.push_back(t->d_data);
    out.d_data = gpuAdd(bw, in[0]->size(), d);
  }

  // mode 2: ReLU of a truncate-reduced value, extended to bw bits; else ReLU
  // (ddg_orca.h:83-110)
  void relu(Tensor<T> &in, Tensor<T> &out, const Tensor<T> &drelu, u64 scale_, int mode) override {
    const auto t0 = std::chrono::high_resolution_clock::now();
    (void)drelu;
    (void)scale_;
    if (mode == 2) {
      auto k = readGPUReluExtendKey<T>(&keyBuf);
      out.d_data = gpuReluExtend(peer, party, k, in.d_data, &g, &s).second;
      s.reluext_time += elapsed_us(t0);
    } else {
      auto k = readReluKey<T>(&keyBuf);
      out.d_data = gpuRelu<T, T, 0, 0, false>(peer, party, k, in.d_data, &g, &s);
      s.relu_time += elapsed_us(t0);
    }
  }

  // exact floor(x / 2^shift), in place (ddg_orca.h:112-123)
  void truncateForward(Tensor<T> &in, u64 shift, u8 mode = 0) override {
    const auto t0 = std::chrono::high_resolution_clock::now();
    (void)mode;
    auto k = readGPUTruncateKey<T>(TruncateType::TrFloor, &keyBuf);
    T *y = gpuTruncate<T, T>(bw, bw, TruncateType::TrFloor, k, int(shift), peer, party, int(in.size()), in.d_data, &g,
                             &s);
    gpuFree(in.d_data);
    in.d_data = y;
    s.truncate_time += elapsed_us(t0);
  }

  // sign extension of a value held in its low bw - scale bits (ddg_orca.h:125-138)
  void signext(Tensor<T> &x, u64 scale_) override {
    const auto t0 = std::chrono::high_resolution_clock::now();
    auto k = readGPUSignExtendKey<T>(&keyBuf);
    T *y = gpuSignExtend<T, T>(party, peer, bw - int(scale_), bw, int(x.size()), k, x.d_data, &g, &s);
    gpuFree(x.d_data);
    x.d_data = y;
    s.signext_time += elapsed_us(t0);
  }

  // unmask with the dealer's clear output mask, local shift by the scale, to host
  // (ddg_orca_base.h:296-302)
  void output(Tensor<T> &a) override {
    const u64 N = a.size();
    unmaskValues(bw, N, a.d_data, reinterpret_cast<T *>(keyBuf), &s);
    gpuLocalTr<T, T, ars>(party, bw, scale, N, a.d_data, true);
    moveIntoCPUMem(reinterpret_cast<u8 *>(a.data), reinterpret_cast<u8 *>(a.d_data), N * sizeof(T), &s);
  }

  void optimize(LayerGraphNode<T> *root) override { (void)root; }

 private:
  bool owns_channel_ = false;
  mpcx_sytorch::Resident<T> weights_;  // the public weights and biases on the device
  static u64 elapsed_us(std::chrono::high_resolution_clock::time_point t0) {
    return u64(std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::high_resolution_clock::now() - t0)
                   .count());
  }
};

// ===========================================================================
// dealer: the same walk on the masks, appending this party's keys
// ===========================================================================
template <typename T>
class MpcxOrcaKeygen : public Backend<T> {
 public:
  u8 *startPtr = nullptr;
  u8 *keyBuf = nullptr;
  size_t keyBufSize = 0;
  int party = -1;
  std::string keyFile;
  int scale = 0;
  int bw = 0;
  AESGlobalContext g;

  // (ddg_orca_base.h:338-355); both parties' keygen runs reset the dealer's
  // randomness to the same seed, so their keys are consistent
  MpcxOrcaKeygen(int party_, int bw_, int scale_, std::string keyFile_, size_t bufBytes = mpcx_sytorch::kKeyBufBytes)
      : party(party_), keyFile(std::move(keyFile_)), scale(scale_), bw(mpcx_ezpc::bw_of<T>(bw_)) {
    initAESContext(&g);
    initGPURandomness();
    initGPUMemPool();
    keyBufSize = bufBytes;
    getAlignedBuf(&keyBuf, keyBufSize, false);
    startPtr = keyBuf;
  }
  ~MpcxOrcaKeygen() override { cpuFree(startPtr, false); }
  size_t keyBytes() const { return size_t(keyBuf - startPtr); }
  // Writes <keyFile>_inference_key<party>.dat (padded to 4 KiB, ddg_orca_base.h:357-372).
  void close() {
    size_t n = keyBytes();
    const size_t pad = (4096 - n % 4096) % 4096;
    std::memset(keyBuf, 0, pad);
    n += pad;
    if (n > keyBufSize) mpcx_ezpc::die("key buffer overflow");
    if (keyFile.empty()) return;
    std::ofstream f(keyFile + "_inference_key" + std::to_string(party) + ".dat", std::ios::binary);
    if (!f.write(reinterpret_cast<const char *>(startPtr), std::streamsize(n))) mpcx_ezpc::die("cannot write keys");
  }

  void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c) override {
    MatmulParams p;
    p.M = int(a.d1);
    p.K = int(a.d2);
    p.N = int(b.d2);
    p.batchSz = 1;
    stdInit(p, bw, 0);
    c.d_data = gpuKeygenMatmul<T>(&keyBuf, party, p, a.d_data, b.d_data, (T *)nullptr, TruncateType::None, &g, true);
  }

  // public weights: output mask r_A . W; the key keeps this party's share of r_A
  void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c, bool useBias, Tensor1D<T> &d,
              bool isFirst) override {
    (void)useBias;
    (void)d;
    (void)isFirst;
    const u64 M = a.d1, K = a.d2, N = b.d2;
    mpcx_ctx *cx = mpcx_ezpc::ctx(bw);
    T *s0 = mpcx_sytorch::dev_alloc<T>(M * K), *s1 = mpcx_sytorch::dev_alloc<T>(M * K);
    mpcx_ezpc::split<T>(cx, M * K, a.d_data, s0, s1);
    mpcx_ezpc::append(&keyBuf, mpcx_sytorch::R_SXP_PUBLIC, {int64_t(M), int64_t(K), int64_t(N)},
                      {{party == SERVER0 ? s0 : s1, M * K * sizeof(T)}});
    gpuFree(s0);
    gpuFree(s1);
    T *out = mpcx_sytorch::dev_alloc<T>(M * N);
    mpcx_ezpc::check(cx, mpcx_ring_gemm(cx, int(M), int(K), int(N), a.d_data, weights_.get(b.data, K * N), out),
                     "matmul keygen");
    c.d_data = out;
  }

  void mul(const Tensor<T> &a, const Tensor<T> &b, Tensor<T> &out) override {
    const int N = int(a.size());
    if (!a.is_same_shape(b) || !a.is_same_shape(out)) mpcx_ezpc::die("mul keygen: shape mismatch");
    out.d_data = gpuKeygenMul<T>(&keyBuf, party, bw, scale, N, a.d_data, b.d_data, TruncateType::TrWithSlack, &g);
  }
  void scalarmul(Tensor<T> &x, T scalar, Tensor<T> &y) override {
    y.d_data = mpcx_sytorch::dev_alloc<T>(x.size());
    gpuLinearComb(bw, x.size(), y.d_data, scalar, x.d_data);
  }
  void sub(Tensor<T> &b, Tensor<T> &a, Tensor<T> &out) override {
    out.d_data = mpcx_sytorch::dev_alloc<T>(b.size());
    gpuLinearComb(bw, b.size(), out.d_data, T(1), b.d_data, T(0) - T(1), a.d_data);
  }
  void add(const std::vector<Tensor<T> *> &in, Tensor<T> &out) override {
    std::vector<T *> d;
    for (auto *t : in) d.push_back(t->d_data);
    out.d_data = gpuAdd(bw, in[0]->size(), d);
  }
  void relu(Tensor<T> &in, Tensor<T> &out, const Tensor<T> &drelu, u64 scale_, int mode) override {
    (void)drelu;
    if (mode == 2) {
      out.d_data = gpuKeygenReluExtend<T>(&keyBuf, party, bw - int(scale_), bw, int(in.size()), in.d_data, &g).second;
    } else {
      const int tmpBw = mode == 3 ? bw - int(scale_) : bw;
      out.d_data = gpuGenReluKey<T, T, 0, 0, false>(&keyBuf, party, tmpBw, tmpBw, int(in.size()), in.d_data, &g);
    }
  }
  void truncateForward(Tensor<T> &in, u64 shift, u8 mode = 0) override {
    (void)mode;
    T *m = genGPUTruncateKey<T, T>(&keyBuf, party, TruncateType::TrFloor, bw, bw, int(shift), int(in.size()),
                                   in.d_data, &g);
    gpuFree(in.d_data);
    in.d_data = m;
  }
  void signext(Tensor<T> &x, u64 scale_) override {
    T *m = genGPUSignExtendKey<T, T>(&keyBuf, party, bw - int(scale_), bw, int(x.size()), x.d_data, &g);
    gpuFree(x.d_data);
    x.d_data = m;
  }
  // the clear output mask for the evaluator (ddg_orca_base.h:511-517)
  void output(Tensor<T> &a) override {
    const size_t n = a.size() * sizeof(T);
    moveIntoCPUMem(keyBuf, reinterpret_cast<u8 *>(a.d_data), n, nullptr);
    keyBuf += n;
  }
  void optimize(LayerGraphNode<T> *root) override { (void)root; }

 private:
  mpcx_sytorch::Resident<T> weights_;  // the public weights on the device
};
