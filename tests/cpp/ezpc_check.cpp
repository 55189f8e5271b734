// ezpc_check.cpp -- replays two of the reference's call sequences through the
// EzPC-named shim (include/mpcx_ezpc.hpp) and the sytorch Backend<T> subclasses
// (include/mpcx_sytorch.hpp), with the two parties as two threads of this
// process on one channel:
//   1. ddgSecureAdjNormKeygen / ddgSecureAdjNormEval (gpu_mpc/secure_adj_norm.h:
//      203-374, 393-659): row sums of the A shares and of its mask, writeShares,
//      gpuKeyGenLUT / readGPULUTKey / gpuDpfLUT, the tiled inverse degrees,
//      gpuKeygenMul / readGPUMulKey / gpuMul (no truncation, then TrFloor),
//      revealing A through the first product key's mask share;
//   2. a GCN layer through the backend (gcn_layer.h:107-116 with the _MatMul
//      per-sample loop, layers.h:67-93): matmul(A_norm_b, X_b) per graph (X a
//      secret leaf), truncateForward, matmul with public weights and bias,
//      truncateForward, relu; then output().
// The dealer runs once per party (initGPURandomness resets its randomness, so
// the two runs write consistent keys), the evaluators run concurrently.
// Usage: ezpc_check <dir>: reads meta.txt (bw B N F O s nmax), a0.bin a1.bin
// (A shares, B*N*N), x0.bin x1.bin (X shares, B*N*F), w.bin (F*O), b.bin (O,
// at scale 2s); writes adjn.bin (A_norm, unmasked), act.bin (the layer's output,
// unmasked), out.bin (output(): act >> s), comm.txt (bytes on each party's
// channel).  Exit status 0 when both parties agree.
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <deque>
#include <fstream>
#include <iterator>
#include <string>
#include <thread>
#include <vector>

#include <sytorch/backend/backend.h>

#include "mpcx_sytorch.hpp"

namespace {

std::vector<uint8_t> slurp(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) mpcx_ezpc::die("cannot open " + path);
  return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}
template <typename T>
std::vector<T> load(const std::string &path, size_t n) {
  auto b = slurp(path);
  if (b.size() != n * sizeof(T)) mpcx_ezpc::die(path + ": wrong size");
  std::vector<T> v(n);
  std::memcpy(v.data(), b.data(), b.size());
  return v;
}
template <typename T>
void store(const std::string &path, const T *d, size_t n, bool device) {
  std::vector<T> h(n);
  if (device)
    mpcx_ezpc::hip_check(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "store");
  else
    std::memcpy(h.data(), d, n * sizeof(T));
  std::ofstream f(path, std::ios::binary);
  f.write(reinterpret_cast<const char *>(h.data()), std::streamsize(n * sizeof(T)));
}
template <typename T>
T *to_dev(const std::vector<T> &h) {
  T *d = reinterpret_cast<T *>(gpuMalloc(h.size() * sizeof(T)));
  mpcx_ezpc::hip_check(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "to_dev");
  return d;
}

// Ring helpers on the shim's context: row sums (A . 1), row tiling (v 1^T) and
// column tiling (1 v_b^T per graph) -- the reference's ddgAdjRowSumKernel and
// ddgTileInvDegreeKernel, here as ring GEMMs with a ones vector.
template <typename T>
struct Ones {
  T *d;
  explicit Ones(int n) : d(to_dev(std::vector<T>(size_t(n), T(1)))) {}
  ~Ones() { gpuFree(d); }
};
template <typename T>
T *rowsum(const T *d_A, int B, int N) {
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  Ones<T> one(N);
  T *out = reinterpret_cast<T *>(gpuMalloc(size_t(B) * N * sizeof(T)));
  mpcx_ezpc::check(c, mpcx_ring_gemm(c, B * N, N, 1, d_A, one.d, out), "rowsum");
  return out;
}
template <typename T>
void tile(const T *d_v, int B, int N, T **row, T **col) {
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  Ones<T> one(N);
  const size_t NN = size_t(N) * N;
  *row = reinterpret_cast<T *>(gpuMalloc(size_t(B) * NN * sizeof(T)));
  *col = reinterpret_cast<T *>(gpuMalloc(size_t(B) * NN * sizeof(T)));
  mpcx_ezpc::check(c, mpcx_ring_gemm(c, B * N, 1, N, d_v, one.d, *row), "tile rows");
  for (int b = 0; b < B; b++)
    mpcx_ezpc::check(c, mpcx_ring_gemm(c, N, 1, N, one.d, d_v + size_t(b) * N, *col + size_t(b) * NN), "tile columns");
}
template <typename T>
T *inv_sqrt_table(int s, int nmax) {
  std::vector<T> t(256, T(0));
  for (int k = 1; k <= nmax && k < 256; k++) t[size_t(k)] = T(std::llround(std::ldexp(1.0, s) / std::sqrt(double(k))));
  return to_dev(t);
}

struct Dims {
  int bw, B, N, F, O, s, nmax;
};

// ---------------- 1. the adjacency normalisation, dealer side ----------------
template <typename T>
T *adjnorm_keygen(u8 **kb, int party, const Dims &d, T *d_A_mask, AESGlobalContext *g) {
  const int degN = d.B * d.N, adjN = d.B * d.N * d.N;
  T *d_degree_mask = rowsum(d_A_mask, d.B, d.N);
  writeShares<T, T>(kb, party, u64(degN), d_degree_mask, d.bw);
  T *d_inv_mask = gpuKeyGenLUT<T, T>(kb, party, 8, d.bw, degN, d_degree_mask, g);
  T *d_row, *d_col;
  tile(d_inv_mask, d.B, d.N, &d_row, &d_col);
  T *d_left_mask = gpuKeygenMul<T>(kb, party, d.bw, d.s, adjN, d_A_mask, d_row, TruncateType::None, g);
  T *d_norm_mask = gpuKeygenMul<T>(kb, party, d.bw, d.s, adjN, d_left_mask, d_col, TruncateType::TrFloor, g);
  for (T *p : {d_degree_mask, d_inv_mask, d_row, d_col, d_left_mask}) gpuFree(p);
  return d_norm_mask;
}

// ---------------- 1. the adjacency normalisation, evaluator side ----------------
template <typename T>
T *adjnorm_eval(u8 **kb, GpuPeer *peer, int party, const Dims &d, AESGlobalContext *g, Stats *s, T *d_A_share) {
  const int degN = d.B * d.N, adjN = d.B * d.N * d.N;
  T *d_degree_share = rowsum(d_A_share, d.B, d.N);
  T *h_degree_mask_share = reinterpret_cast<T *>(*kb);
  *kb += size_t(degN) * sizeof(T);
  T *d_degree_mask_share =
      reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(h_degree_mask_share), size_t(degN) * sizeof(T), s));
  gpuLinearComb(d.bw, u64(degN), d_degree_share, T(1), d_degree_share, T(1), d_degree_mask_share);
  gpuFree(d_degree_mask_share);
  peer->reconstructInPlace(d_degree_share, d.bw, u64(degN), s);
  auto lutKey = readGPULUTKey<T>(kb);
  T *d_table = inv_sqrt_table<T>(d.s, d.nmax);
  T *d_inv = gpuDpfLUT<T, T>(lutKey, peer, party, d_degree_share, d_table, g, s, true);
  gpuFree(d_degree_share);
  gpuFree(d_table);
  T *d_row, *d_col;
  tile(d_inv, d.B, d.N, &d_row, &d_col);
  auto mul1Key = readGPUMulKey<T>(kb, u64(adjN), u64(adjN), u64(adjN), TruncateType::None);
  T *d_A_mask_share = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(mul1Key.a), size_t(adjN) * sizeof(T), s));
  gpuLinearComb(d.bw, u64(adjN), d_A_share, T(1), d_A_share, T(1), d_A_mask_share);
  gpuFree(d_A_mask_share);
  peer->reconstructInPlace(d_A_share, d.bw, u64(adjN), s);
  T *d_left = gpuMul<T>(peer, party, d.bw, d.s, adjN, mul1Key, d_A_share, d_row, TruncateType::None, g, s);
  auto mul2Key = readGPUMulKey<T>(kb, u64(adjN), u64(adjN), u64(adjN), TruncateType::TrFloor);
  T *d_norm = gpuMul<T>(peer, party, d.bw, d.s, adjN, mul2Key, d_left, d_col, TruncateType::TrFloor, g, s);
  for (T *p : {d_inv, d_row, d_col, d_left}) gpuFree(p);
  return d_norm;
}

// ---------------- 2. a GCN layer through a backend ----------------
// A: (B*N, N) A_norm rows (per graph N x N blocks), X: (B*N, F); returns act (B*N, O).
template <typename T, class BE>
Tensor<T> *gcn_layer(BE &be, const Dims &d, Tensor<T> &A, Tensor<T> &X, Tensor<T> &W, Tensor1D<T> &bias) {
  const u64 N = u64(d.N), F = u64(d.F), O = u64(d.O), BN = u64(d.B) * N;
  auto *AX = new Tensor<T>({BN, F});
  AX->d_data = reinterpret_cast<T *>(gpuMalloc(BN * F * sizeof(T)));
  for (int b = 0; b < d.B; b++) {  // _MatMul's per-sample loop
    Tensor2D<T> A_slice(A.data + b * N * N, A.d_data + b * N * N, N, N);
    Tensor2D<T> X_slice(X.data + b * N * F, X.d_data + b * N * F, N, F);
    Tensor2D<T> out_slice(AX->data + b * N * F, nullptr, N, F);
    be.matmul(A_slice, X_slice, out_slice);
    mpcx_ezpc::hip_check(hipMemcpy(AX->d_data + b * N * F, out_slice.d_data, N * F * sizeof(T), hipMemcpyDeviceToDevice),
                         "fold");
    gpuFree(out_slice.d_data);
  }
  be.truncateForward(*AX, u64(d.s));
  auto *Z = new Tensor<T>({BN, O});
  Tensor2D<T> AX2 = AX->as_2d(), W2 = W.as_2d(), Z2 = Z->as_2d();
  be.matmul(AX2, W2, Z2, true, bias, false);
  Z->d_data = Z2.d_data;
  be.truncateForward(*Z, u64(d.s));
  auto *act = new Tensor<T>({BN, O});
  Tensor<T> drelu({BN, O});
  be.relu(*Z, *act, drelu, u64(d.s), 0);
  gpuFree(AX->d_data);
  gpuFree(Z->d_data);
  delete AX;
  delete Z;
  return act;
}

template <typename T>
int run(const std::string &dir, const Dims &d) {
  const size_t NN = size_t(d.N) * d.N, adjN = size_t(d.B) * NN, BN = size_t(d.B) * d.N;
  std::vector<T> a[2] = {load<T>(dir + "/a0.bin", adjN), load<T>(dir + "/a1.bin", adjN)};
  std::vector<T> x[2] = {load<T>(dir + "/x0.bin", BN * d.F), load<T>(dir + "/x1.bin", BN * d.F)};
  const std::vector<T> w = load<T>(dir + "/w.bin", size_t(d.F) * d.O), bias = load<T>(dir + "/b.bin", size_t(d.O));

  // ---- dealer: one run per party (the reference runs one keygen process per party)
  std::vector<u8 *> keys(2);
  std::vector<size_t> key_bytes(2);
  T *norm_mask = nullptr, *act_mask = nullptr;
  for (int party = 0; party < 2; party++) {
    MpcxOrcaKeygen<T> kg(party, d.bw, d.s, "");
    T *d_A_mask = randomGEOnGpu<T>(adjN, d.bw);  // the input masks of this key set
    T *d_X_mask = randomGEOnGpu<T>(BN * d.F, d.bw);
    T *nm = adjnorm_keygen<T>(&kg.keyBuf, party, d, d_A_mask, &kg.g);
    Tensor<T> A({BN, u64(d.N)}), X({BN, u64(d.F)}), W({u64(d.F), u64(d.O)});
    Tensor1D<T> b(u64(d.O));
    A.d_data = nm;
    X.d_data = d_X_mask;
    std::memcpy(W.data, w.data(), w.size() * sizeof(T));
    std::memcpy(b.data, bias.data(), bias.size() * sizeof(T));
    Tensor<T> *act = gcn_layer<T>(kg, d, A, X, W, b);
    kg.output(*act);
    key_bytes[size_t(party)] = kg.keyBytes();
    keys[size_t(party)] = cpuMalloc(kg.keyBytes(), false);
    std::memcpy(keys[size_t(party)], kg.startPtr, kg.keyBytes());
    if (party == 0) {
      norm_mask = nm;
      act_mask = act->d_data;
    } else {
      // the second dealer run must have drawn the same masks
      std::vector<T> m0(adjN), m1(adjN);
      mpcx_ezpc::hip_check(hipMemcpy(m0.data(), norm_mask, adjN * sizeof(T), hipMemcpyDeviceToHost), "mask");
      mpcx_ezpc::hip_check(hipMemcpy(m1.data(), nm, adjN * sizeof(T), hipMemcpyDeviceToHost), "mask");
      if (m0 != m1) mpcx_ezpc::die("the two dealer runs drew different masks");
      gpuFree(nm);
      gpuFree(act->d_data);
    }
    gpuFree(d_A_mask);
    gpuFree(d_X_mask);
    delete act;
  }

  // ---- the two evaluators, concurrently
  mpcx_peer *ends[2];
  if (mpcx_peer_pair(60000, &ends[0], &ends[1]) != MPCX_OK) mpcx_ezpc::die("mpcx_peer_pair");
  std::vector<T> norm_out[2], act_out[2], out_host[2];
  u64 comm[2] = {0, 0};
  auto party_main = [&](int party) {
    MpcxOrca<T> be(party, ends[party], d.bw, d.s, keys[size_t(party)], key_bytes[size_t(party)]);
    T *d_A = to_dev(a[party]);
    T *d_norm = adjnorm_eval<T>(&be.keyBuf, be.peer, party, d, &be.g, &be.s, d_A);
    Tensor<T> A({BN, u64(d.N)}), X({BN, u64(d.F)}), W({u64(d.F), u64(d.O)});
    Tensor1D<T> b(u64(d.O));
    A.d_data = d_norm;
    X.d_data = to_dev(x[party]);
    be.registerLeaf(X.d_data);  // each graph's slice is revealed when its product first uses it
    for (int g = 0; g < d.B; g++) be.registerLeaf(X.d_data + size_t(g) * d.N * d.F);
    std::memcpy(W.data, w.data(), w.size() * sizeof(T));
    std::memcpy(b.data, bias.data(), bias.size() * sizeof(T));
    Tensor<T> *act = gcn_layer<T>(be, d, A, X, W, b);
    norm_out[party].resize(adjN);
    act_out[party].resize(BN * d.O);
    mpcx_ezpc::hip_check(hipMemcpy(norm_out[party].data(), d_norm, adjN * sizeof(T), hipMemcpyDeviceToHost), "out");
    mpcx_ezpc::hip_check(hipMemcpy(act_out[party].data(), act->d_data, BN * d.O * sizeof(T), hipMemcpyDeviceToHost),
                         "out");
    be.output(*act);
    out_host[party].assign(act->data, act->data + BN * d.O);
    comm[party] = mpcx_peer_bytes(ends[party]);
    gpuFree(d_A);
    gpuFree(d_norm);
    gpuFree(X.d_data);
    gpuFree(act->d_data);
    delete act;
  };
  std::thread t0(party_main, 0), t1(party_main, 1);
  t0.join();
  t1.join();
  if (norm_out[0] != norm_out[1] || act_out[0] != act_out[1] || out_host[0] != out_host[1])
    mpcx_ezpc::die("the two parties' outputs differ");
  // unmask with the dealer's masks
  std::vector<T> nm(adjN), am(BN * d.O);
  mpcx_ezpc::hip_check(hipMemcpy(nm.data(), norm_mask, adjN * sizeof(T), hipMemcpyDeviceToHost), "mask");
  mpcx_ezpc::hip_check(hipMemcpy(am.data(), act_mask, BN * d.O * sizeof(T), hipMemcpyDeviceToHost), "mask");
  for (size_t i = 0; i < adjN; i++) nm[i] = norm_out[0][i] - nm[i];
  for (size_t i = 0; i < am.size(); i++) am[i] = act_out[0][i] - am[i];
  store(dir + "/adjn.bin", nm.data(), nm.size(), false);
  store(dir + "/act.bin", am.data(), am.size(), false);
  store(dir + "/out.bin", out_host[0].data(), out_host[0].size(), false);
  std::ofstream(dir + "/comm.txt") << comm[0] << " " << comm[1] << "\n";
  mpcx_peer_close(ends[0]);
  mpcx_peer_close(ends[1]);
  std::printf("ezpc_check: both parties agree (%zu key bytes per party)\n", key_bytes[0]);
  return 0;
}

// ---------------- 3. the whole affinity forward through a backend ----------------
// DeepDTAGenAffinity::_forward (gpu_mpc/deepdtagen.h:183-222) as its layers
// call the backend: per GCN layer _MatMul's per-sample secret x secret loop
// (layers.h:67-93) and its truncation, the FC with public weights and bias and
// its truncation, ReLU (mode 0: every layer full width, ddg_orca_opt.h:47-77);
// the mask product (_Mul, backend mul with TrWithSlack, layers.h:318-346);
// MaskedMaxPoolLayer::_forward (masked_maxpool_layer.h:47-165); the drug FCs;
// GPUConcat (deepdtagen.h:45-101: the protein leaf revealed, rows interleaved);
// the fusion FCs, the last one untruncated; output() (ddg_orca_base.h:296-302).
struct FDims {
  int bw, B, N, F, gcn[3], dfc[2], prot, nfus, fus[4], s, nmax, reps, stop = 0;
  std::vector<std::pair<u64, u64>> layers() const {
    std::vector<std::pair<u64, u64>> io;
    u64 fin = u64(F);
    for (int g : gcn) io.push_back({fin, u64(g)}), fin = u64(g);
    io.push_back({u64(gcn[2]), u64(dfc[0])});
    io.push_back({u64(dfc[0]), u64(dfc[1])});
    fin = u64(dfc[1] + prot);
    for (int i = 0; i < nfus; i++) io.push_back({fin, u64(fus[i])}), fin = u64(fus[i]);
    return io;
  }
};

// A linear layer's public weights (in x out) and bias (at scale 2s), held the
// way FC<T> holds them: host arrays that live as long as the model.
template <typename T>
struct Lin {
  Tensor<T> W;
  Tensor1D<T> b;
  Lin(u64 in, u64 out, const T *w, const T *bias) : W({in, out}), b(out) {
    std::memcpy(W.data, w, in * out * sizeof(T));
    std::memcpy(b.data, bias, out * sizeof(T));
  }
};

// FC<T>::_forward: x . W + b, then the layer truncation (all but the last layer)
template <typename T, class BE>
Tensor<T> *fc(BE &be, Tensor<T> &x, Lin<T> &L, int s, bool trunc) {
  const u64 out = L.W.shape[1], M = x.size() / L.W.shape[0];
  auto *z = new Tensor<T>({M, out});
  Tensor2D<T> x2(x.data, x.d_data, M, L.W.shape[0]), z2 = z->as_2d();
  Tensor2D<T> w2 = L.W.as_2d();
  be.matmul(x2, w2, z2, true, L.b, false);
  z->d_data = z2.d_data;
  if (trunc) be.truncateForward(*z, u64(s));
  return z;
}
// ReLU<T>::_forward in mode 0 (full width)
template <typename T, class BE>
Tensor<T> *relu(BE &be, Tensor<T> *x, int s) {
  auto *y = new Tensor<T>(x->shape);
  Tensor<T> drelu(x->shape);
  be.relu(*x, *y, drelu, u64(s), 0);
  gpuFree(x->d_data);
  delete x;
  return y;
}
// GCNLayer::_forward (gcn_layer.h:107-116): aggregate first, then the FC, ReLU
template <typename T, class BE>
Tensor<T> *gcn(BE &be, int B, int N, Tensor<T> &A, Tensor<T> &H, Lin<T> &L, int s) {
  const u64 K = L.W.shape[0], Nn = u64(N), BN = u64(B) * Nn;
  auto *AX = new Tensor<T>({BN, K});
  AX->d_data = reinterpret_cast<T *>(gpuMalloc(BN * K * sizeof(T)));
  for (int b = 0; b < B; b++) {  // _MatMul's per-sample loop
    Tensor2D<T> A_slice(A.data + b * Nn * Nn, A.d_data + b * Nn * Nn, Nn, Nn);
    Tensor2D<T> X_slice(H.data + b * Nn * K, H.d_data + b * Nn * K, Nn, K);
    Tensor2D<T> out_slice(AX->data + b * Nn * K, nullptr, Nn, K);
    be.matmul(A_slice, X_slice, out_slice);
    mpcx_ezpc::hip_check(hipMemcpy(AX->d_data + b * Nn * K, out_slice.d_data, Nn * K * sizeof(T),
                                   hipMemcpyDeviceToDevice), "fold");
    gpuFree(out_slice.d_data);
  }
  be.truncateForward(*AX, u64(s));
  Tensor<T> *Z = fc(be, *AX, L, s, true);
  gpuFree(AX->d_data);
  delete AX;
  return relu(be, Z, s);
}
// MaskedMaxPoolLayer::_forward: node-major planes, then per level
// scalarmul(even, -1), add(., odd), relu, add(even, .), the odd plane carried
template <typename T, class BE>
Tensor<T> *maxpool(BE &be, Tensor<T> &masked, int B, int N, int F, int s) {
  const u64 plane = u64(B) * u64(F);
  T *d_buf = reinterpret_cast<T *>(gpuMalloc(u64(N) * plane * sizeof(T)));
  for (int b = 0; b < B; b++)
    mpcx_ezpc::hip_check(hipMemcpy2D(d_buf + u64(b) * F, plane * sizeof(T), masked.d_data + u64(b) * N * F,
                                     u64(F) * sizeof(T), u64(F) * sizeof(T), u64(N), hipMemcpyDeviceToDevice),
                         "pool planes");
  u64 cur = u64(N);
  T *d_cur = d_buf;
  while (cur > 1) {
    const u64 pairs = cur / 2, rem = cur % 2, n = pairs * plane;
    T *d_even = reinterpret_cast<T *>(gpuMalloc(n * sizeof(T)));
    T *d_odd = reinterpret_cast<T *>(gpuMalloc(n * sizeof(T)));
    for (u64 p = 0; p < pairs; p++) {
      mpcx_ezpc::hip_check(hipMemcpy(d_even + p * plane, d_cur + 2 * p * plane, plane * sizeof(T),
                                     hipMemcpyDeviceToDevice), "even plane");
      mpcx_ezpc::hip_check(hipMemcpy(d_odd + p * plane, d_cur + (2 * p + 1) * plane, plane * sizeof(T),
                                     hipMemcpyDeviceToDevice), "odd plane");
    }
    Tensor<T> t_even(nullptr, d_even, {n}), t_odd(nullptr, d_odd, {n});
    Tensor<T> t_neg({n}), t_diff({n}), t_drelu({n}), t_relu({n}), t_res({n});
    be.scalarmul(t_even, T(0) - T(1), t_neg);  // ring negation, no truncation
    std::vector<Tensor<T> *> in1 = {&t_neg, &t_odd};
    be.add(in1, t_diff);
    be.relu(t_diff, t_relu, t_drelu, u64(s), 0);
    std::vector<Tensor<T> *> in2 = {&t_even, &t_relu};
    be.add(in2, t_res);
    T *d_next = reinterpret_cast<T *>(gpuMalloc((pairs + rem) * plane * sizeof(T)));
    mpcx_ezpc::hip_check(hipMemcpy(d_next, t_res.d_data, n * sizeof(T), hipMemcpyDeviceToDevice), "level");
    if (rem)
      mpcx_ezpc::hip_check(hipMemcpy(d_next + n, d_cur + (cur - 1) * plane, plane * sizeof(T),
                                     hipMemcpyDeviceToDevice), "carry");
    for (T *q : {d_even, d_odd, t_neg.d_data, t_diff.d_data, t_relu.d_data, t_res.d_data, d_cur}) gpuFree(q);
    d_cur = d_next;
    cur = pairs + rem;
  }
  auto *out = new Tensor<T>({u64(B), u64(F)});
  out->d_data = d_cur;
  return out;
}
// GPUConcat::_forward: reveal the public leaves, then rows [t0[b] | t1[b]]
template <typename T>
void reveal_public(MpcxOrca<T> &be, Tensor<T> &t) {
  be.revealPublicLeaf(t.d_data, be.bw, t.size());
}
template <typename T>
void reveal_public(MpcxOrcaKeygen<T> &, Tensor<T> &) {}
template <typename T, class BE>
Tensor<T> *concat(BE &be, Tensor<T> &a, Tensor<T> &b) {
  reveal_public(be, a);
  reveal_public(be, b);
  const u64 wa = a.shape.back(), wb = b.shape.back(), rows = a.size() / wa, w = wa + wb;
  auto *o = new Tensor<T>({rows, w});
  o->d_data = reinterpret_cast<T *>(gpuMalloc(rows * w * sizeof(T)));
  for (u64 r = 0; r < rows; r++) {
    mpcx_ezpc::hip_check(hipMemcpy(o->d_data + r * w, a.d_data + r * wa, wa * sizeof(T), hipMemcpyDeviceToDevice),
                         "concat");
    mpcx_ezpc::hip_check(hipMemcpy(o->d_data + r * w + wa, b.d_data + r * wb, wb * sizeof(T),
                                   hipMemcpyDeviceToDevice), "concat");
  }
  return o;
}
// The model's forward on masked-public A_norm (B*N x N), X (B*N x F), the
// tiled mask leaf (B*N x gcn[2]) and the protein leaf (B x prot); returns the
// last layer's output (B x 1), not yet output().
// stop > 0 returns the tensor after that stage instead (1-3 the GCN layers, 4
// the mask product, 5 the pool, 6 and 7 the drug FCs, 8 the concat): a
// diagnostic cut that the dealer and the evaluators make alike.
template <typename T, class BE>
Tensor<T> *affinity_forward(BE &be, const FDims &d, std::deque<Lin<T>> &L, Tensor<T> &A, Tensor<T> &X,
                            Tensor<T> &maskT, Tensor<T> &prot, int stop = 0) {
  Tensor<T> *h = gcn(be, d.B, d.N, A, X, L[0], d.s);
  for (int l = 1; l < 3; l++) {
    if (stop == l) return h;
    Tensor<T> *h2 = gcn(be, d.B, d.N, A, *h, L[size_t(l)], d.s);
    gpuFree(h->d_data);
    delete h;
    h = h2;
  }
  if (stop == 3) return h;
  auto *masked = new Tensor<T>(h->shape);
  be.mul(*h, maskT, *masked);
  gpuFree(h->d_data);
  delete h;
  if (stop == 4) return masked;
  Tensor<T> *pooled = maxpool(be, *masked, d.B, d.N, d.gcn[2], d.s);
  gpuFree(masked->d_data);
  delete masked;
  if (stop == 5) return pooled;
  Tensor<T> *d1 = relu(be, fc(be, *pooled, L[3], d.s, true), d.s);
  gpuFree(pooled->d_data);
  delete pooled;
  if (stop == 6) return d1;
  Tensor<T> *d2 = fc(be, *d1, L[4], d.s, true);
  gpuFree(d1->d_data);
  delete d1;
  if (stop == 7) return d2;
  Tensor<T> *f = concat(be, *d2, prot);
  gpuFree(d2->d_data);
  delete d2;
  if (stop == 8) return f;
  for (int i = 0; i < d.nfus; i++) {
    const bool last = i + 1 == d.nfus;
    Tensor<T> *e = fc(be, *f, L[size_t(5 + i)], d.s, !last);
    if (!last) e = relu(be, e, d.s);
    gpuFree(f->d_data);
    delete f;
    f = e;
  }
  return f;
}

template <typename T>
int run_forward(const std::string &dir, const FDims &d) {
  const u64 N = u64(d.N), NN = N * N, BN = u64(d.B) * N, adjN = u64(d.B) * NN;
  const u64 C = u64(d.gcn[2]);
  std::vector<T> a[2] = {load<T>(dir + "/a0.bin", adjN), load<T>(dir + "/a1.bin", adjN)};
  std::vector<T> x[2] = {load<T>(dir + "/x0.bin", BN * d.F), load<T>(dir + "/x1.bin", BN * d.F)};
  std::vector<T> m[2] = {load<T>(dir + "/m0.bin", BN * C), load<T>(dir + "/m1.bin", BN * C)};
  const std::vector<T> prot = load<T>(dir + "/prot.bin", u64(d.B) * d.prot);
  size_t wlen = 0;
  for (auto &io : d.layers()) wlen += io.first * io.second + io.second;
  const std::vector<T> w = load<T>(dir + "/w.bin", wlen);
  auto make_layers = [&]() {
    std::deque<Lin<T>> L;  // FC<T> holds its weights in place: no copies
    size_t o = 0;
    for (auto &io : d.layers()) {
      L.emplace_back(io.first, io.second, w.data() + o, w.data() + o + io.first * io.second);
      o += io.first * io.second + io.second;
    }
    return L;
  };
  Dims ad{d.bw, d.B, d.N, d.F, 0, d.s, d.nmax};

  // ---- dealer: one run per party; both keys go into one host buffer, which
  // becomes the device key arena (initGPUKeyArena) for the evaluators
  const size_t cap = size_t(d.B) * (size_t(d.bw) << 22) + (size_t(256) << 20);
  std::vector<std::vector<u8>> kh(2);
  std::vector<T> out_mask(size_t(d.B));
  for (int party = 0; party < 2; party++) {
    MpcxOrcaKeygen<T> kg(party, d.bw, d.s, "", cap);
    std::deque<Lin<T>> L = make_layers();
    T *d_A_mask = randomGEOnGpu<T>(adjN, d.bw);
    T *d_X_mask = randomGEOnGpu<T>(BN * d.F, d.bw);
    T *d_M_mask = randomGEOnGpu<T>(BN * C, d.bw);
    T *nm = adjnorm_keygen<T>(&kg.keyBuf, party, ad, d_A_mask, &kg.g);
    Tensor<T> A({BN, N}), X({BN, u64(d.F)}), MT({BN, C}), P({u64(d.B), u64(d.prot)});
    A.d_data = nm;
    X.d_data = d_X_mask;
    MT.d_data = d_M_mask;
    P.d_data = to_dev(std::vector<T>(P.size(), T(0)));  // the protein leaf: mask 0 (public)
    Tensor<T> *out = affinity_forward<T>(kg, d, L, A, X, MT, P, d.stop);
    kg.output(*out);
    kh[size_t(party)].assign(kg.startPtr, kg.keyBuf);
    for (T *q : {d_A_mask, d_X_mask, d_M_mask, nm, P.d_data, out->d_data}) gpuFree(q);
    delete out;
  }
  const size_t k0 = kh[0].size(), k1 = kh[1].size(), off1 = (k0 + 4095) / 4096 * 4096;
  u8 *keys = cpuMalloc(off1 + k1, false);
  std::memcpy(keys, kh[0].data(), k0);
  std::memcpy(keys + off1, kh[1].data(), k1);
  kh[0].clear(), kh[0].shrink_to_fit(), kh[1].clear(), kh[1].shrink_to_fit();
  initGPUKeyArena(keys, off1 + k1);

  // ---- the two evaluators, concurrently, reps forwards on the same keys
  mpcx_peer *ends[2];
  if (mpcx_peer_pair(120000, &ends[0], &ends[1]) != MPCX_OK) mpcx_ezpc::die("mpcx_peer_pair");
  std::vector<T> out_host[2];
  std::vector<double> ms[2];
  u64 comm[2] = {0, 0}, aes[2] = {0, 0}, rounds[2] = {0, 0};
  Stats st[2];
  std::atomic<int> ready{0};
  auto party_main = [&](int party) {
    u8 *mine = party ? keys + off1 : keys;
    MpcxOrca<T> be(party, ends[party], d.bw, d.s, mine, party ? k1 : k0);
    std::deque<Lin<T>> L = make_layers();
    for (int r = 0; r < d.reps; r++) {
      be.keyBuf = be.startPtr;  // the same key set for every forward (timing only)
      be.resetLeaves();
      T *d_A = to_dev(a[party]);
      Tensor<T> X({BN, u64(d.F)}), MT({BN, C}), P({u64(d.B), u64(d.prot)});
      X.d_data = to_dev(x[party]);
      MT.d_data = to_dev(m[party]);
      P.d_data = to_dev(party ? prot : std::vector<T>(P.size(), T(0)));  // party 1 holds the protein embedding
      // start together: each forward is timed from here to its output
      const int gen = 2 * (r + 1);
      ready.fetch_add(1);
      while (ready.load() < gen) std::this_thread::yield();
      const u64 b0 = mpcx_peer_bytes(ends[party]), aes0 = mpcx_ezpc::aes_calls(), r0 = mpcx_peer_rounds(ends[party]);
      be.s = Stats();
      const auto t0 = std::chrono::steady_clock::now();
      T *d_norm = adjnorm_eval<T>(&be.keyBuf, be.peer, party, ad, &be.g, &be.s, d_A);
      Tensor<T> A({BN, N});
      A.d_data = d_norm;
      for (int g = 0; g < d.B; g++) be.registerLeaf(X.d_data + size_t(g) * N * d.F);  // _MatMul's slices
      be.registerLeaf(MT.d_data);
      be.registerLeaf(P.d_data);
      Tensor<T> *out = affinity_forward<T>(be, d, L, A, X, MT, P, d.stop);
      be.output(*out);
      ms[party].push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
      comm[party] = mpcx_peer_bytes(ends[party]) - b0;
      aes[party] = mpcx_ezpc::aes_calls() - aes0;
      rounds[party] = mpcx_peer_rounds(ends[party]) - r0;
      st[party] = be.s;
      out_host[party].assign(out->data, out->data + out->size());
      for (T *q : {d_A, d_norm, X.d_data, MT.d_data, P.d_data, out->d_data}) gpuFree(q);
      delete out;
    }
  };
  std::thread t0(party_main, 0), t1(party_main, 1);
  t0.join();
  t1.join();
  if (out_host[0] != out_host[1]) mpcx_ezpc::die("the two parties' outputs differ");
  store(dir + "/out.bin", out_host[0].data(), out_host[0].size(), false);
  std::ofstream(dir + "/comm.txt") << comm[0] << " " << comm[1] << "\n";
  std::ofstream tf(dir + "/time.txt");
  for (int r = 0; r < d.reps; r++) tf << std::max(ms[0][size_t(r)], ms[1][size_t(r)]) << "\n";
  std::ofstream(dir + "/keys.txt") << k0 << " " << k1 << "\n";
  std::ofstream(dir + "/aes.txt") << aes[0] << " " << aes[1] << "\n";
  {  // party 0's backend timers of the last forward (us) and its exchange rounds
    std::ofstream f(dir + "/stats.txt");
    f << "rounds " << rounds[0] << "\nmatmul_us " << st[0].matmul_time << "\nrelu_us " << st[0].relu_time
      << "\ntruncate_us " << st[0].truncate_time << "\n";
  }
  mpcx_peer_close(ends[0]);
  mpcx_peer_close(ends[1]);
  freeGPUKeyArena();
  cpuFree(keys, false);
  std::printf("ezpc_check forward: both parties agree (%zu key bytes per party), %.2f ms last forward\n", k0,
              std::max(ms[0].back(), ms[1].back()));
  return 0;
}

}  // namespace

// `ezpc_check width <bw> <bin> <bout> [drelu]`: a ReLU (or DReLU) keygen for
// bin-bit inputs; widths the gates cannot serve abort with a message before
// any device call (no GPU needed), the others print "width ok".
template <typename T>
int width_check(int bin, int bout, bool drelu) {
  if (drelu) {
    if (bin != 8 * int(sizeof(T))) gpuKeyGenDRelu<T>(nullptr, 0, bin, 0, nullptr, nullptr);
  } else {
    const int bw = 8 * int(sizeof(T));
    const int sc = mpcx_ezpc::relu_scale(bw, bin, bout);
    std::printf("width ok: scale %d\n", sc);
    return 0;
  }
  std::printf("width ok\n");
  return 0;
}

int main(int argc, char **argv) {
  if (argc >= 5 && std::string(argv[1]) == "width") {
    const int bw = std::atoi(argv[2]), bin = std::atoi(argv[3]), bout = std::atoi(argv[4]);
    const bool drelu = argc >= 6 && std::string(argv[5]) == "drelu";
    return bw == 32 ? width_check<uint32_t>(bin, bout, drelu) : width_check<uint64_t>(bin, bout, drelu);
  }
  if (argc >= 3 && std::string(argv[1]) == "forward") {
    const std::string dir = argv[2];
    FDims d{};
    std::ifstream meta(dir + "/meta.txt");
    if (!(meta >> d.bw >> d.B >> d.N >> d.F >> d.gcn[0] >> d.gcn[1] >> d.gcn[2] >> d.dfc[0] >> d.dfc[1] >> d.prot >>
          d.nfus))
      mpcx_ezpc::die("bad meta.txt");
    if (d.nfus < 1 || d.nfus > 4) mpcx_ezpc::die("meta.txt: 1 to 4 fusion layers");
    for (int i = 0; i < d.nfus; i++) meta >> d.fus[i];
    if (!(meta >> d.s >> d.nmax >> d.reps) || d.reps < 1) mpcx_ezpc::die("bad meta.txt");
    if (!(meta >> d.stop)) d.stop = 0;  // optional: the diagnostic stage cut
    return d.bw == 32 ? run_forward<uint32_t>(dir, d) : run_forward<uint64_t>(dir, d);
  }
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s <dir> | forward <dir> | width <bw> <bin> <bout> [drelu]\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  Dims d{};
  std::ifstream meta(dir + "/meta.txt");
  if (!(meta >> d.bw >> d.B >> d.N >> d.F >> d.O >> d.s >> d.nmax)) mpcx_ezpc::die("bad meta.txt");
  return d.bw == 32 ? run<uint32_t>(dir, d) : run<uint64_t>(dir, d);
}
