// model.hip -- dealer (keygen) and online forward of the secure affinity model.
// See model.h for the reference mapping.  The gate sequence, gate ids and key
// arena offsets are a pure function of (dims, B): keygen and forward walk the
// same sequence with a cursor, so the key arena needs no index.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>

#include "model.h"

namespace mpcx {

void Phase1Timer::reset() {
  for (auto e : ev) (void)hipEventDestroy(e);
  ev.clear();
  elems.clear();
  levels.clear();
  bytes.clear();
}

#define TRY(x)                           \
  do {                                   \
    hipError_t e_ = (x);                 \
    if (e_ != hipSuccess) return e_;     \
  } while (0)

namespace {

struct Cursor {
  size_t off = 0;
  uint32_t gate = 1;
};

inline size_t pairs_of(int N) { return size_t(N) * (N + 1) / 2; }
inline size_t pidx(int N, int i, int j) { return size_t(i) * N - size_t(i) * (i - 1) / 2 + size_t(j - i); }

int pool_levels(int N, int *pairs) {
  int R = N, L = 0;
  while (R > 1) {
    pairs[L++] = R / 2;
    R = R / 2 + (R & 1);
  }
  return L;
}

template <typename T>
struct DevBuf {
  T *p = nullptr;
  size_t n = 0;
  hipError_t alloc(size_t count) {
    if (count <= n) return hipSuccess;
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
    hipError_t e = hipMalloc((void **)&p, std::max<size_t>(count, 1) * sizeof(T));
    if (e == hipSuccess) n = count;
    return e;
  }
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

}  // namespace

template <typename T>
class Model final : public ModelBase {
 public:
  Model(int bw, int s, const ModelDims &d, const Launch &L) : bw_(bw), s_(s), d_(d), L_(L) {}
  ~Model() override {
    for (int p = 0; p < 2; p++)
      if (arena_[p]) (void)hipFree(arena_[p]);
    timer.reset();
  }

  // ---------------- weights ----------------
  int nlayers() const { return 5 + d_.nfus; }
  void layer_io(int l, int *in, int *out) const {
    if (l < 3) {
      *in = l == 0 ? d_.feat : d_.gcn[l - 1];
      *out = d_.gcn[l];
    } else if (l < 5) {
      *in = l == 3 ? d_.gcn[2] : d_.dfc[0];
      *out = d_.dfc[l - 3];
    } else {
      int k = l - 5;
      *in = k == 0 ? d_.dfc[1] + d_.prot : d_.fus[k - 1];
      *out = d_.fus[k];
    }
  }
  size_t weights_len() const {
    size_t o = 0;
    for (int l = 0; l < nlayers(); l++) {
      int in, out;
      layer_io(l, &in, &out);
      o += size_t(in) * out + out;
    }
    return o;
  }
  hipError_t set_weights(const int64_t *W) {
    size_t o = 0;
    wt_.resize(nlayers());
    bias_.resize(nlayers());
    hbias_.resize(nlayers());
    for (int l = 0; l < nlayers(); l++) {
      int in, out;
      layer_io(l, &in, &out);
      std::vector<T> w(size_t(in) * out), b(out);
      for (size_t i = 0; i < w.size(); i++) w[i] = T(uint64_t(W[o + i]));
      o += w.size();
      hbias_[l].assign(W + o, W + o + out);
      for (int i = 0; i < out; i++) b[i] = T(uint64_t(W[o + i]));
      o += out;
      TRY(wt_[l].alloc(w.size()));
      TRY(bias_[l].alloc(b.size()));
      TRY(hipMemcpy(wt_[l].p, w.data(), w.size() * sizeof(T), hipMemcpyHostToDevice));
      TRY(hipMemcpy(bias_[l].p, b.data(), b.size() * sizeof(T), hipMemcpyHostToDevice));
    }
    std::vector<T> tab(256, T(0));
    const double q = std::ldexp(1.0, s_);
    for (int k = 1; k <= d_.lut_nmax && k < 256; k++) tab[k] = T(std::llround(q / std::sqrt(double(k))));
    TRY(table_.alloc(256));
    TRY(hipMemcpy(table_.p, tab.data(), 256 * sizeof(T), hipMemcpyHostToDevice));
    return hipSuccess;
  }

  // ---------------- plan sizes ----------------
  size_t key_bytes(int B) const override {
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N, BNN = BN * N, P = pairs_of(N);
    size_t o = 0;
    o = reveal_layout(bw_, BN * d_.feat, o).end;
    o = reveal_layout(bw_, BNN, o).end;
    o = reveal_layout(bw_, BN, o).end;
    o = reveal_layout(bw_, BN, o).end;
    o = lut8_layout(bw_, BN, o).end;
    o = mul_layout(bw_, BN, BN, size_t(B) * P, o).end;
    o = tr_layout(G_TRSLACK, bw_, s_, size_t(B) * P, o).end;
    o = mul_layout(bw_, BNN, size_t(B) * P, BNN, o).end;
    for (int l = 0; l < 3; l++) {
      size_t E = BN * d_.gcn[l];
      o = tr_layout(G_TR, bw_, s_, E, o).end;
      o = sxs_layout(bw_, B, N, N, d_.gcn[l], o).end;
      o = tr_layout(G_TRRELU, bw_, s_, E, o).end;
    }
    int pairs[32];
    int Lv = pool_levels(N, pairs);
    for (int l = 0; l < Lv; l++) o = tr_layout(G_RELU, bw_, s_, size_t(B) * pairs[l] * d_.gcn[2], o).end;
    o = tr_layout(G_TRRELU, bw_, s_, size_t(B) * d_.dfc[0], o).end;
    o = tr_layout(G_TR, bw_, s_, size_t(B) * d_.dfc[1], o).end;
    for (int k = 0; k < d_.nfus - 1; k++) o = tr_layout(G_TRRELU, bw_, s_, size_t(B) * d_.fus[k], o).end;
    o = reveal_layout(bw_, size_t(B) * d_.fus[d_.nfus - 1], o).end;
    return o;
  }

  uint8_t *arena(int party) override { return arena_[party]; }

  hipError_t ensure_arena(int B) {
    size_t need = key_bytes(B);
    if (need <= arena_bytes_) return hipSuccess;
    for (int p = 0; p < 2; p++) {
      if (arena_[p]) (void)hipFree(arena_[p]);
      arena_[p] = nullptr;
    }
    arena_bytes_ = 0;
    for (int p = 0; p < 2; p++) TRY(hipMalloc((void **)&arena_[p], need));
    arena_bytes_ = need;
    return hipSuccess;
  }

  size_t emax(int B) const {
    const int N = d_.n_nodes;
    size_t m = size_t(B) * N * std::max(d_.feat, std::max(d_.gcn[0], std::max(d_.gcn[1], d_.gcn[2])));
    m = std::max(m, size_t(B) * N * N);
    m = std::max(m, size_t(B) * pairs_of(N));
    int fw = std::max(d_.dfc[0], d_.dfc[1] + d_.prot);
    for (int k = 0; k < d_.nfus; k++) fw = std::max(fw, d_.fus[k]);
    m = std::max(m, size_t(B) * fw);
    return m;
  }

  hipError_t ensure_work(int B) {
    if (B == work_B_) return hipSuccess;
    const int N = d_.n_nodes;
    const size_t E = emax(B), BN = size_t(B) * N, BNN = BN * N, BP = size_t(B) * pairs_of(N);
    for (auto *b : {&bA_, &bB_, &bC_, &msg0_, &msg1_}) TRY(b->alloc(E));
    for (auto *b : {&ba0_, &ba1_, &bb0_, &bb1_}) TRY(b->alloc((E + 63) / 64));
    TRY(Ah_.alloc(BNN));
    TRY(An_.alloc(BNN));
    TRY(mh_.alloc(BN));
    TRY(dh_.alloc(BN));
    TRY(inv_.alloc(BN));
    TRY(vh_.alloc(BN));
    TRY(Ph_.alloc(BP));
    TRY(Wh_.alloc(BP));
    TRY(V0_.alloc(BN * d_.gcn[2]));
    TRY(V1_.alloc(BN * d_.gcn[2]));
    TRY(out_.alloc(B));
    // index maps of the adjacency normalisation (outer product, A (.) W)
    const size_t P = pairs_of(N);
    std::vector<uint32_t> oa(B * P), ob(B * P), wa(BNN), wb(BNN);
    for (int b = 0; b < B; b++) {
      size_t q = size_t(b) * P;
      for (int i = 0; i < N; i++)
        for (int j = i; j < N; j++) {
          oa[q] = uint32_t(b * N + i);
          ob[q] = uint32_t(b * N + j);
          q++;
        }
      for (int i = 0; i < N; i++)
        for (int j = 0; j < N; j++) {
          size_t e = (size_t(b) * N + i) * N + j;
          wa[e] = uint32_t(e);
          wb[e] = uint32_t(size_t(b) * P + (i <= j ? pidx(N, i, j) : pidx(N, j, i)));
        }
    }
    TRY(oa_.alloc(oa.size()));
    TRY(ob_.alloc(ob.size()));
    TRY(wa_.alloc(wa.size()));
    TRY(wb_.alloc(wb.size()));
    TRY(hipMemcpy(oa_.p, oa.data(), oa.size() * 4, hipMemcpyHostToDevice));
    TRY(hipMemcpy(ob_.p, ob.data(), ob.size() * 4, hipMemcpyHostToDevice));
    TRY(hipMemcpy(wa_.p, wa.data(), wa.size() * 4, hipMemcpyHostToDevice));
    TRY(hipMemcpy(wb_.p, wb.data(), wb.size() * 4, hipMemcpyHostToDevice));
    work_B_ = B;
    return hipSuccess;
  }

  // ---------------- dealer ----------------
  hipError_t keygen(int B, uint64_t seed) override {
    TRY(ensure_arena(B));
    TRY(ensure_work(B));
    const int N = d_.n_nodes, bw = bw_, s = s_;
    const size_t BN = size_t(B) * N, BNN = BN * N, P = pairs_of(N), BP = size_t(B) * P;
    const size_t E = emax(B);
    uint8_t *K0 = arena_[0], *K1 = arena_[1];
    DevBuf<T> rX, t1, t2, rA, rN, rm, rd, rinv, rP, rW, sa0, sb0, gt;
    TRY(rX.alloc(E));
    TRY(t1.alloc(E));
    TRY(t2.alloc(E));
    TRY(rA.alloc(BNN));
    TRY(rN.alloc(BNN));
    TRY(rm.alloc(BN));
    TRY(rd.alloc(BN));
    TRY(rinv.alloc(BN));
    TRY(rP.alloc(BP));
    TRY(rW.alloc(BP));
    TRY(sa0.alloc(BNN));
    TRY(sb0.alloc(E));
    TRY(gt.alloc(E));
    Cursor c;
    auto reveal = [&](size_t n, T *mask) -> hipError_t {
      RevealLayout lay = reveal_layout(bw, n, c.off);
      TRY(launch_reveal_keygen<T>(L_, lay, seed, c.gate, mask, K0, K1));
      c.off = lay.end;
      c.gate++;
      return hipSuccess;
    };
    auto tr = [&](int kind, size_t n, const T *in, T *out) -> hipError_t {
      TrLayout lay = tr_layout(kind, bw, s, n, c.off);
      TRY(launch_tr_keygen<T>(L_, lay, seed, c.gate, in, out, K0, K1));
      c.off = lay.end;
      c.gate++;
      return hipSuccess;
    };
    auto pub_gemm = [&](const T *x, int l, size_t rows, T *y) -> hipError_t {
      int in, out;
      layer_io(l, &in, &out);
      GemmArgs<T> g;
      g.M = int(rows);
      g.K = in;
      g.N = out;
      g.A1 = x;
      g.B1 = wt_[l].p;
      g.C = y;
      return launch_gemm<T>(L_, g);
    };

    TRY(reveal(BN * d_.feat, rX.p));
    TRY(reveal(BNN, rA.p));
    TRY(reveal(BN, rm.p));
    TRY(reveal(BN, rd.p));
    {
      Lut8Layout lay = lut8_layout(bw, BN, c.off);
      TRY(launch_lut8_keygen<T>(L_, lay, seed, c.gate, rd.p, rinv.p, K0, K1));
      c.off = lay.end;
      c.gate++;
    }
    {
      MulLayout lay = mul_layout(bw, BN, BN, BP, c.off);
      TRY(launch_mul_keygen<T>(L_, lay, seed, c.gate, oa_.p, ob_.p, rinv.p, rinv.p, rP.p, K0, K1));
      c.off = lay.end;
      c.gate++;
    }
    TRY(tr(G_TRSLACK, BP, rP.p, rW.p));
    {
      MulLayout lay = mul_layout(bw, BNN, BP, BNN, c.off);
      TRY(launch_mul_keygen<T>(L_, lay, seed, c.gate, wa_.p, wb_.p, rA.p, rW.p, rN.p, K0, K1));
      c.off = lay.end;
      c.gate++;
    }
    // GCN stack; rX holds the running activation mask
    for (int l = 0; l < 3; l++) {
      const int fo = d_.gcn[l];
      const size_t En = BN * fo;
      TRY(pub_gemm(rX.p, l, BN, t1.p));
      TRY(tr(G_TR, En, t1.p, t2.p));
      {  // SxS: C = rA.rB - RA0.RB0 + rC
        SxsLayout lay = sxs_layout(bw, B, N, N, fo, c.off);
        T *RA0 = reinterpret_cast<T *>(K0 + lay.off_ra), *RA1 = reinterpret_cast<T *>(K1 + lay.off_ra);
        T *RB0 = reinterpret_cast<T *>(K0 + lay.off_rb), *RB1 = reinterpret_cast<T *>(K1 + lay.off_rb);
        TRY(launch_split<T>(L_, seed, c.gate, F_SPLIT + 0, BNN, rN.p, RA0, RA1, nullptr));
        TRY(launch_split<T>(L_, seed, c.gate, F_SPLIT + 1, En, t2.p, RB0, RB1, nullptr));
        TRY(launch_prf_ring<T>(L_, seed, c.gate, F_ROUT, En, t1.p));  // rC (output mask)
        GemmArgs<T> g;
        g.M = N;
        g.K = N;
        g.N = fo;
        g.batch = B;
        g.sA = size_t(N) * N;
        g.sB = size_t(N) * fo;
        g.sC = size_t(N) * fo;
        g.A1 = rN.p;
        g.B1 = t2.p;
        g.Cin = t1.p;
        g.C = gt.p;
        TRY(launch_gemm<T>(L_, g));  // rA.rB + rC
        g.A1 = RA0;
        g.B1 = RB0;
        g.Cin = gt.p;
        g.C = gt.p;
        g.sign = -1;
        TRY(launch_gemm<T>(L_, g));  // - RA0.RB0
        TRY(launch_split<T>(L_, seed, c.gate, F_SPLIT + 2, En, gt.p, reinterpret_cast<T *>(K0 + lay.off_c),
                            reinterpret_cast<T *>(K1 + lay.off_c), nullptr));
        c.off = lay.end;
        c.gate++;
      }
      TRY(tr(G_TRRELU, En, t1.p, rX.p));
    }
    // pool
    const int C = d_.gcn[2];
    const T S = T(1) << (bw - 2);
    TRY(launch_pool_prep<T>(L_, BN, C, rX.p, rm.p, S, T(0), t2.p));  // rV in t2
    T *cur = t2.p, *nxt = rX.p;
    int pairs[32];
    const int Lv = pool_levels(N, pairs);
    int R = N;
    for (int l = 0; l < Lv; l++) {
      const int pr = pairs[l];
      const size_t En = size_t(B) * pr * C;
      TRY(launch_pool_diff<T>(L_, B, R, C, cur, t1.p));
      TRY(tr(G_RELU, En, t1.p, gt.p));
      TRY(launch_pool_combine<T>(L_, B, R, C, cur, gt.p, nullptr, nxt));
      std::swap(cur, nxt);
      R = pr + (R & 1);
    }
    // drug FCs
    TRY(pub_gemm(cur, 3, B, t1.p));
    TRY(tr(G_TRRELU, size_t(B) * d_.dfc[0], t1.p, gt.p));
    TRY(pub_gemm(gt.p, 4, B, t1.p));
    TRY(tr(G_TR, size_t(B) * d_.dfc[1], t1.p, gt.p));
    TRY(launch_concat<T>(L_, B, d_.dfc[1], d_.prot, gt.p, nullptr, nxt));
    T *h = nxt, *h2 = cur;
    for (int k = 0; k < d_.nfus; k++) {
      TRY(pub_gemm(h, 5 + k, B, t1.p));
      if (k < d_.nfus - 1) {
        TRY(tr(G_TRRELU, size_t(B) * d_.fus[k], t1.p, h2));
        std::swap(h, h2);
      } else {
        RevealLayout lay = reveal_layout(bw, size_t(B) * d_.fus[k], c.off);
        TRY(hipMemcpyAsync(K0 + lay.off_r, t1.p, lay.N * sizeof(T), hipMemcpyDeviceToDevice, L_.stream));
        TRY(hipMemcpyAsync(K1 + lay.off_r, t1.p, lay.N * sizeof(T), hipMemcpyDeviceToDevice, L_.stream));
        c.off = lay.end;
        c.gate++;
      }
    }
    TRY(hipStreamSynchronize(L_.stream));
    keyed_B_ = B;
    return hipSuccess;
  }

  hipError_t import_keys(int B, const void *k0, const void *k1, size_t bytes) override {
    if (bytes != key_bytes(B)) return hipErrorInvalidValue;
    TRY(ensure_arena(B));
    TRY(hipMemcpy(arena_[0], k0, bytes, hipMemcpyHostToDevice));
    TRY(hipMemcpy(arena_[1], k1, bytes, hipMemcpyHostToDevice));
    keyed_B_ = B;
    return hipSuccess;
  }
  hipError_t export_keys(int party, void *dst, size_t bytes) override {
    if (!arena_[party] || bytes > arena_bytes_) return hipErrorInvalidValue;
    return hipMemcpy(dst, arena_[party], bytes, hipMemcpyDeviceToHost);
  }

  hipError_t set_inputs(int B, const void *x0, const void *x1, const void *a0, const void *a1, const void *m0,
                        const void *m1, const int64_t *prot) override {
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N, nx = BN * d_.feat, na = BN * N;
    TRY(x0_.alloc(nx));
    TRY(x1_.alloc(nx));
    TRY(a0_.alloc(na));
    TRY(a1_.alloc(na));
    TRY(m0_.alloc(BN));
    TRY(m1_.alloc(BN));
    TRY(prot_.alloc(size_t(B) * d_.prot));
    TRY(hipMemcpy(x0_.p, x0, nx * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(x1_.p, x1, nx * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(a0_.p, a0, na * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(a1_.p, a1, na * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(m0_.p, m0, BN * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(m1_.p, m1, BN * sizeof(T), hipMemcpyHostToDevice));
    std::vector<T> pr(size_t(B) * d_.prot);
    for (size_t i = 0; i < pr.size(); i++) pr[i] = T(uint64_t(prot[i]));
    TRY(hipMemcpy(prot_.p, pr.data(), pr.size() * sizeof(T), hipMemcpyHostToDevice));
    input_B_ = B;
    return hipSuccess;
  }

  // ---------------- online ----------------
  hipError_t tr_eval(Cursor &c, int kind, size_t n, const T *x, const T *bias, int ncol, T *out) {
    TrLayout lay = tr_layout(kind, bw_, s_, n, c.off);
    const uint8_t *K0 = arena_[0], *K1 = arena_[1];
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (timer.on) {
      TRY(hipEventCreate(&e0));
      TRY(hipEventCreate(&e1));
      TRY(hipEventRecord(e0, L_.stream));
    }
    TRY(launch_tr_phase1<T>(L_, lay, K0, K1, x, bias, ncol, ba0_.p, ba1_.p, bb0_.p, bb1_.p));
    if (timer.on) {
      TRY(hipEventRecord(e1, L_.stream));
      timer.ev.push_back(e0);
      timer.ev.push_back(e1);
      timer.elems.push_back(n);
      timer.levels.push_back((lay.use_a ? lay.a.L + 1 : 0) + (lay.use_b ? lay.b.L + 1 : 0));
      // per element and party: the masked input, and for every DCF the root,
      // correction words and leaf (16 B each), the output-mask bit read and the
      // message bit written (the bias vector is ncol words, cache resident)
      double per = double(sizeof(T));
      if (lay.use_a) per += 16.0 * (lay.a.L + 2) + 0.125 + 0.125;
      if (lay.use_b) per += 16.0 * (lay.b.L + 2) + 0.125 + 0.125;
      timer.bytes.push_back(2.0 * per * double(n));
    }
    counters.bitplanes(n, int(lay.use_a) + int(lay.use_b));
    TRY(launch_tr_phase2<T>(L_, lay, K0, K1, x, bias, ncol, ba0_.p, ba1_.p, bb0_.p, bb1_.p, msg0_.p, msg1_.p));
    counters.msg(n, bw_);
    TRY(launch_reconstruct<T>(L_, n, msg0_.p, msg1_.p, out));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }

  hipError_t forward(int B) override {
    if (keyed_B_ != B || input_B_ != B) return hipErrorInvalidValue;
    TRY(ensure_work(B));
    const int N = d_.n_nodes, bw = bw_;
    const size_t BN = size_t(B) * N, BNN = BN * N, P = pairs_of(N), BP = size_t(B) * P;
    const uint8_t *K0 = arena_[0], *K1 = arena_[1];
    T *m0 = msg0_.p, *m1 = msg1_.p;
    Cursor c;
    auto reveal = [&](size_t n, const T *v0, const T *v1, int rowlen, T *out) -> hipError_t {
      RevealLayout lay = reveal_layout(bw, n, c.off);
      TRY(launch_reveal_eval<T>(L_, lay, K0, K1, v0, v1, rowlen, m0, m1));
      counters.msg(n, bw);
      TRY(launch_reconstruct<T>(L_, n, m0, m1, out));
      c.off = lay.end;
      c.gate++;
      return hipSuccess;
    };
    auto pub_gemm = [&](const T *x, int l, size_t rows, T *y) -> hipError_t {
      int in, out;
      layer_io(l, &in, &out);
      GemmArgs<T> g;
      g.M = int(rows);
      g.K = in;
      g.N = out;
      g.A1 = x;
      g.B1 = wt_[l].p;
      g.C = y;
      return launch_gemm<T>(L_, g);
    };
    T *H = bA_.p, *Z = bB_.p, *XW = bC_.p;

    TRY(reveal(BN * d_.feat, x0_.p, x1_.p, 0, H));
    TRY(reveal(BNN, a0_.p, a1_.p, 0, Ah_.p));
    TRY(reveal(BN, m0_.p, m1_.p, 0, mh_.p));
    TRY(reveal(BN, a0_.p, a1_.p, N, dh_.p));  // degree = row sums of the A shares
    {
      Lut8Layout lay = lut8_layout(bw, BN, c.off);
      TRY(launch_lut8_phase1<T>(L_, lay, K0, K1, table_.p, dh_.p, m0, m1));
      counters.msg(BN, bw);
      TRY(launch_reconstruct<T>(L_, BN, m0, m1, vh_.p));
      TRY(launch_lut8_phase2<T>(L_, lay, K0, K1, vh_.p, m0, m1));
      counters.msg(BN, bw);
      TRY(launch_reconstruct<T>(L_, BN, m0, m1, inv_.p));
      c.off = lay.end;
      c.gate++;
    }
    {
      MulLayout lay = mul_layout(bw, BN, BN, BP, c.off);
      TRY(launch_mul_eval<T>(L_, lay, K0, K1, oa_.p, ob_.p, inv_.p, inv_.p, m0, m1));
      counters.msg(BP, bw);
      TRY(launch_reconstruct<T>(L_, BP, m0, m1, Ph_.p));
      c.off = lay.end;
      c.gate++;
    }
    TRY(tr_eval(c, G_TRSLACK, BP, Ph_.p, nullptr, 1, Wh_.p));
    {
      MulLayout lay = mul_layout(bw, BNN, BP, BNN, c.off);
      TRY(launch_mul_eval<T>(L_, lay, K0, K1, wa_.p, wb_.p, Ah_.p, Wh_.p, m0, m1));
      counters.msg(BNN, bw);
      TRY(launch_reconstruct<T>(L_, BNN, m0, m1, An_.p));
      c.off = lay.end;
      c.gate++;
    }
    for (int l = 0; l < 3; l++) {
      const int fo = d_.gcn[l];
      const size_t En = BN * fo;
      TRY(pub_gemm(H, l, BN, Z));
      TRY(tr_eval(c, G_TR, En, Z, nullptr, 1, XW));
      {
        SxsLayout lay = sxs_layout(bw, B, N, N, fo, c.off);
        GemmArgs<T> g;
        g.M = N;
        g.K = N;
        g.N = fo;
        g.batch = B;
        g.sA = size_t(N) * N;
        g.sB = size_t(N) * fo;
        g.sC = size_t(N) * fo;
        // party 0: (A^ - RA0)(B^ - RB0) + C0
        g.A1 = An_.p;
        g.A2 = reinterpret_cast<const T *>(K0 + lay.off_ra);
        g.B1 = XW;
        g.B2 = reinterpret_cast<const T *>(K0 + lay.off_rb);
        g.Cin = reinterpret_cast<const T *>(K0 + lay.off_c);
        g.C = m0;
        TRY(launch_gemm<T>(L_, g));
        // party 1: C1 - A^ RB1 - RA1 B^
        GemmArgs<T> h = g;
        h.A2 = nullptr;
        h.B2 = nullptr;
        h.B1 = reinterpret_cast<const T *>(K1 + lay.off_rb);
        h.Cin = reinterpret_cast<const T *>(K1 + lay.off_c);
        h.C = m1;
        h.sign = -1;
        TRY(launch_gemm<T>(L_, h));
        h.A1 = reinterpret_cast<const T *>(K1 + lay.off_ra);
        h.B1 = XW;
        h.Cin = m1;
        TRY(launch_gemm<T>(L_, h));
        counters.msg(En, bw);
        TRY(launch_reconstruct<T>(L_, En, m0, m1, Z));
        c.off = lay.end;
        c.gate++;
      }
      TRY(tr_eval(c, G_TRRELU, En, Z, bias_[l].p, fo, H));
    }
    // masked max-pool: V = H + S*m^ - S, then a tree of max(a,b) = a + ReLU(b-a)
    const int C = d_.gcn[2];
    const T S = T(1) << (bw - 2);
    TRY(launch_pool_prep<T>(L_, BN, C, H, mh_.p, S, T(0) - S, V0_.p));
    T *cur = V0_.p, *nxt = V1_.p;
    int pairs[32];
    const int Lv = pool_levels(N, pairs);
    int R = N;
    for (int l = 0; l < Lv; l++) {
      const int pr = pairs[l];
      const size_t En = size_t(B) * pr * C;
      TRY(launch_pool_diff<T>(L_, B, R, C, cur, Z));
      TRY(tr_eval(c, G_RELU, En, Z, nullptr, 1, XW));
      TRY(launch_pool_combine<T>(L_, B, R, C, cur, XW, nullptr, nxt));
      std::swap(cur, nxt);
      R = pr + (R & 1);
    }
    // drug FCs
    TRY(pub_gemm(cur, 3, B, Z));
    TRY(tr_eval(c, G_TRRELU, size_t(B) * d_.dfc[0], Z, bias_[3].p, d_.dfc[0], XW));
    TRY(pub_gemm(XW, 4, B, Z));
    TRY(tr_eval(c, G_TR, size_t(B) * d_.dfc[1], Z, bias_[4].p, d_.dfc[1], XW));
    // concat [drug, protein]; the protein embedding owner reveals it (one message)
    counters.msg(size_t(B) * d_.prot, bw);
    TRY(launch_concat<T>(L_, B, d_.dfc[1], d_.prot, XW, prot_.p, H));
    T *h = H, *h2 = XW;
    for (int k = 0; k < d_.nfus; k++) {
      TRY(pub_gemm(h, 5 + k, B, Z));
      if (k < d_.nfus - 1) {
        TRY(tr_eval(c, G_TRRELU, size_t(B) * d_.fus[k], Z, bias_[5 + k].p, d_.fus[k], h2));
        std::swap(h, h2);
      } else {
        RevealLayout lay = reveal_layout(bw, size_t(B) * d_.fus[k], c.off);
        TRY(launch_output<T>(L_, B, bw, s_, Z, reinterpret_cast<const T *>(K0 + lay.off_r), hbias_[5 + k][0],
                             out_.p));
        c.off = lay.end;
        c.gate++;
      }
    }
    return hipGetLastError();
  }

  hipError_t output(int64_t *h_out, int B) override {
    TRY(hipStreamSynchronize(L_.stream));
    return hipMemcpy(h_out, out_.p, size_t(B) * sizeof(int64_t), hipMemcpyDeviceToHost);
  }

 private:
  int bw_, s_;
  ModelDims d_;
  Launch L_;
  std::vector<DevBuf<T>> wt_, bias_;
  std::vector<std::vector<int64_t>> hbias_;
  DevBuf<T> table_;
  uint8_t *arena_[2] = {nullptr, nullptr};
  size_t arena_bytes_ = 0;
  int keyed_B_ = -1, input_B_ = -1, work_B_ = -1;
  DevBuf<T> x0_, x1_, a0_, a1_, m0_, m1_, prot_;
  DevBuf<T> bA_, bB_, bC_, msg0_, msg1_, Ah_, An_, mh_, dh_, inv_, vh_, Ph_, Wh_, V0_, V1_;
  DevBuf<uint64_t> ba0_, ba1_, bb0_, bb1_;
  DevBuf<uint32_t> oa_, ob_, wa_, wb_;
  DevBuf<int64_t> out_;
};

ModelBase *make_model(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L,
                      std::string *err) {
  if (d.nfus < 1 || d.nfus > 4 || d.fus[d.nfus - 1] != 1) {
    *err = "last fusion layer must have width 1";
    return nullptr;
  }
  if (d.n_nodes < 1 || d.n_nodes > 255) {
    *err = "n_nodes must be in [1, 255] (8-bit degree LUT domain)";
    return nullptr;
  }
  ModelBase *m = nullptr;
  if (bw == 32) {
    auto *mm = new Model<uint32_t>(bw, s, d, L);
    if (nW != mm->weights_len()) {
      *err = "weight blob length mismatch";
      delete mm;
      return nullptr;
    }
    if (mm->set_weights(W) != hipSuccess) {
      *err = "weight upload failed";
      delete mm;
      return nullptr;
    }
    m = mm;
  } else if (bw == 64) {
    auto *mm = new Model<uint64_t>(bw, s, d, L);
    if (nW != mm->weights_len()) {
      *err = "weight blob length mismatch";
      delete mm;
      return nullptr;
    }
    if (mm->set_weights(W) != hipSuccess) {
      *err = "weight upload failed";
      delete mm;
      return nullptr;
    }
    m = mm;
  } else {
    *err = "bw must be 32 or 64";
  }
  return m;
}

}  // namespace mpcx
