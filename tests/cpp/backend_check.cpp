// backend_check.cpp -- drives include/mpcx_backend.hpp through a dealer pass and
// an evaluator pass of a small network and compares the reconstructed outputs
// with exact integer arithmetic on the host:
//   h = reveal(x);  z = h . W + b (bias at scale 2s);  truncateForward(z);
//   y = relu(z);  u = 3y - y (= 2y, local ops);  v = floor(u (.) y / 2^s) (the fixed-point
//   product: Beaver, then the slack truncation);  output(v) -> floor(v / 2^s);
//   p = maxpool of y over its M rows (one sample, N channels);  output(p) -> floor(p / 2^s)
// Usage: backend_check <bw: 32|64> [local].  With "local" both passes select the
// LocalARS truncation (set_truncation(MPCX_LOCALARS)) and every output may differ
// from the exact one by 1 (the carry of a local shift; run at bw=64, where masked
// values do not wrap in practice).  Exit status 0 on success.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "mpcx_backend.hpp"

template <typename T>
static int run(int bw, bool local) {
  const int s = 12, M = 37, K = 53, N = 29;
  mpcx_ctx *ctx = nullptr;
  if (mpcx_create(bw, s, 0, &ctx) != MPCX_OK) {
    std::fprintf(stderr, "mpcx_create failed\n");
    return 2;
  }
  std::mt19937_64 rng(7);
  auto uni = [&](int64_t lo, int64_t hi) { return lo + int64_t(rng() % uint64_t(hi - lo + 1)); };
  std::vector<int64_t> x(size_t(M) * K), W(size_t(K) * N), b(N);
  // magnitudes keep every intermediate inside the signed 32-bit ring, and the
  // product inside the slack truncation's domain: |x W| <= 53 * 2^12 * 2^8 < 2^25.8,
  // |b 2^s| <= 2^23, so 0 <= y < 2^14 and 2y * y < 2^29 < 2^(bw-2)
  for (auto &v : x) v = uni(-(1 << s), 1 << s);
  for (auto &v : W) v = uni(-(1 << s), 1 << s) / 16;
  for (auto &v : b) v = uni(-(1 << s), 1 << s) / 2;
  // plaintext reference
  std::vector<int64_t> want(size_t(M) * N), ymax(N, 0);
  for (int i = 0; i < M; i++)
    for (int j = 0; j < N; j++) {
      __int128 acc = 0;
      for (int k = 0; k < K; k++) acc += __int128(x[size_t(i) * K + k]) * W[size_t(k) * N + j];
      int64_t z = int64_t((acc + (__int128(b[j]) << s)) >> s);
      int64_t y = z > 0 ? z : 0;
      ymax[j] = y > ymax[j] ? y : ymax[j];
      int64_t u = 2 * y;
      want[size_t(i) * N + j] = int64_t(((__int128(u) * y) >> s) >> s);
    }
  // shares of x, public W and b on the device
  std::vector<T> x0(x.size()), x1(x.size()), hW(W.size()), hb(b.size());
  for (size_t i = 0; i < x.size(); i++) {
    x0[i] = T(rng());
    x1[i] = T(uint64_t(x[i])) - x0[i];
  }
  for (size_t i = 0; i < W.size(); i++) hW[i] = T(uint64_t(W[i]));
  for (size_t i = 0; i < b.size(); i++) hb[i] = T(uint64_t(b[i]));
  using Tn = mpcx::MpcxTensor<T>;
  auto dev = [](const std::vector<T> &h, size_t d1, size_t d2) {
    Tn t;
    t.d1 = d1;
    t.d2 = d2;
    (void)hipMalloc(&t.d_data, h.size() * sizeof(T));
    (void)hipMemcpy(t.d_data, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice);
    return t;
  };
  Tn X0 = dev(x0, M, K), X1 = dev(x1, M, K), Wt = dev(hW, K, N), Bt = dev(hb, N, 1);
  mpcx::KeyArena arena;
  arena.capacity = size_t(64) << 20;
  for (int p = 0; p < 2; p++) (void)hipMalloc(&arena.d_key[p], arena.capacity);

  std::vector<int64_t> got(size_t(M) * N), gotp(N);
  for (int pass = 0; pass < 2; pass++) {
    const bool dealer = pass == 0;
    arena.offset = 0;
    mpcx::SecureBackend<T> be(ctx, dealer ? mpcx::SecureBackend<T>::Mode::Dealer
                                          : mpcx::SecureBackend<T>::Mode::Evaluator,
                              &arena, 4242);
    if (local) be.set_truncation(MPCX_LOCALARS);
    Tn h{nullptr, size_t(M), size_t(K)}, z{nullptr, size_t(M), size_t(N)}, y{nullptr, size_t(M), size_t(N)};
    Tn t3{nullptr, size_t(M), size_t(N)}, u{nullptr, size_t(M), size_t(N)}, v{nullptr, size_t(M), size_t(N)};
    Tn pl{nullptr, 1, size_t(N)};
    be.reveal(X0, X1, h);
    be.matmul(h, Wt, z, true, Bt, true);
    be.truncateForward(z, s);
    be.relu(z, y);
    be.scalarmul(y, T(3), t3);
    be.sub(t3, y, u);
    be.mul(u, y, v);
    be.output(v, dealer ? nullptr : got.data());
    be.maxpool(y, pl, 1, M, N);
    be.output(pl, dealer ? nullptr : gotp.data());
    std::printf("bw=%d %s pass: %zu key bytes per party\n", bw, dealer ? "dealer" : "evaluator", arena.offset);
  }
  const int64_t tol = local ? 1 : 0;
  auto off = [tol](int64_t a, int64_t b) { return a - b > tol || b - a > tol; };
  int bad = 0;
  for (size_t i = 0; i < got.size(); i++)
    if (off(got[i], want[i]) && bad++ < 5)
      std::fprintf(stderr, "mismatch at %zu: got %lld want %lld\n", i, (long long)got[i], (long long)want[i]);
  for (int j = 0; j < N; j++)
    if (off(gotp[j], ymax[j] >> s) && bad++ < 5)
      std::fprintf(stderr, "pool mismatch at %d: got %lld want %lld\n", j, (long long)gotp[j],
                   (long long)(ymax[j] >> s));
  for (Tn *t : {&X0, &X1, &Wt, &Bt}) (void)hipFree(t->d_data);
  for (int p = 0; p < 2; p++) (void)hipFree(arena.d_key[p]);
  mpcx_destroy(ctx);
  std::printf("bw=%d%s: %s (%zu outputs, %d pooled)\n", bw, local ? " local truncation" : "",
              bad ? "MISMATCH" : (local ? "within 1" : "bit-exact"), got.size(), N);
  return bad ? 1 : 0;
}

int main(int argc, char **argv) {
  const int bw = argc > 1 ? std::atoi(argv[1]) : 32;
  const bool local = argc > 2 && std::string(argv[2]) == "local";
  try {
    return bw == 64 ? run<uint64_t>(64, local) : run<uint32_t>(32, local);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 3;
  }
}
