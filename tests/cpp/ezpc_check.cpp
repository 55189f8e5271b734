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
#include <cmath>
#include <cstdio>
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
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s <dir> | width <bw> <bin> <bout> [drelu]\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  Dims d{};
  std::ifstream meta(dir + "/meta.txt");
  if (!(meta >> d.bw >> d.B >> d.N >> d.F >> d.O >> d.s >> d.nmax)) mpcx_ezpc::die("bad meta.txt");
  return d.bw == 32 ? run<uint32_t>(dir, d) : run<uint64_t>(dir, d);
}
