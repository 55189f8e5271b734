// model.hip -- dealer (keygen) and online forward of the secure affinity model,
// and the standalone secure adjacency normalisation.  See model.h for the
// reference mapping.  The gate sequence, gate ids and key offsets are a pure
// function of (dims, B): keygen and forward walk the same sequence with a
// cursor, so the key arena needs no index; plan() lists the gates' key ranges
// and the forward checks every gate against it.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>

#include "model.h"
#include "peer.h"

namespace mpcx {

void Phase1Timer::reset() {
  for (auto e : ev) (void)hipEventDestroy(e);
  for (auto e : gev) (void)hipEventDestroy(e);
  ev.clear();
  elems.clear();
  levels.clear();
  bytes.clear();
  gev.clear();
  gmacs.clear();
}

namespace {
// A model lane of at most this many samples runs in the latency-bound form
// (small gates spread over the CUs, truncation pairs in one launch).
constexpr int kFewLaneB = 8;
constexpr size_t kFuseSmallN = 65536;
// Events of the profiled forward only time work: they are read after a stream
// synchronisation, so they skip the system-scope fence (an L2 writeback and
// invalidation at every record, which would also slow the kernel after it).
constexpr unsigned kTimingEvent = hipEventDisableSystemFence;
// start/stop events around a ring-GEMM section when profiling
struct GemmSpan {
  Phase1Timer *t;
  hipStream_t st;
  hipEvent_t e1 = nullptr;
  hipError_t begin(double macs) {
    if (!t || !t->on) return hipSuccess;
    hipEvent_t e0;
    hipError_t r = hipEventCreateWithFlags(&e0, kTimingEvent);
    if (r == hipSuccess) r = hipEventCreateWithFlags(&e1, kTimingEvent);
    if (r == hipSuccess) r = hipEventRecord(e0, st);
    if (r != hipSuccess) return r;
    t->gev.push_back(e0);
    t->gmacs.push_back(macs);
    return hipSuccess;
  }
  hipError_t end() {
    if (!e1) return hipSuccess;
    t->gev.push_back(e1);
    return hipEventRecord(e1, st);
  }
};
}  // namespace

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

template <typename T>
struct DevBuf {
  T *p = nullptr;
  size_t n = 0;
  hipError_t alloc(size_t count) {
    if (count <= n) return hipSuccess;
    release();
    hipError_t e = hipMalloc((void **)&p, std::max<size_t>(count, 1) * sizeof(T));
    if (e == hipSuccess) n = count;
    return e;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  ~DevBuf() { release(); }
};

// Both parties' key bytes at absolute offset `off` live at k[p] + (off - begin).
struct KeyView {
  const uint8_t *k[2] = {nullptr, nullptr};
  size_t begin = 0;
};

// Key range of one gate and the sub-ranges that both parties hold identically
// (DCF correction and leaf words, the clear output mask): a streamed arena
// copies those once, from party 0's buffer.
struct GateKey {
  size_t begin = 0, end = 0;
  uint32_t gate = 0;   // the dealer's gate id (position in the plan + 1)
  int tr_kind = 0;     // truncation-family gates: kind and elements (0: another gate)
  size_t n = 0;
  int nsh = 0;
  size_t sh[2][2] = {{0, 0}, {0, 0}};
  void share(size_t b, size_t e) {
    sh[nsh][0] = b;
    sh[nsh][1] = e;
    nsh++;
  }
};

// Supplies the key bytes [begin, end) of the next gate (resident arena or a
// streamed slot) before the gate's kernels are enqueued.
struct KeySource {
  virtual hipError_t acquire(size_t begin, size_t end, KeyView *kv) = 0;
  virtual ~KeySource() = default;
};

// Exchange buffers shared by the gates: both parties' messages (the
// truncation-family gates exchange through LDS inside their one launch).
// In party mode (one process per party) m0 holds this party's message and m1
// the peer's, and b0 / b1 the two parties' DCF output-bit planes.
template <typename T>
struct Workspace {
  DevBuf<T> m0, m1;
  DevBuf<uint64_t> b0, b1;
  size_t cap = 0;
  hipError_t ensure(size_t n) {
    if (n <= cap) return hipSuccess;
    TRY(m0.alloc(n));
    TRY(m1.alloc(n));
    cap = n;
    return hipSuccess;
  }
  hipError_t ensure_bits(size_t words) {
    TRY(b0.alloc(words));
    return b1.alloc(words);
  }
};

// ---------------------------------------------------------------------------
// online evaluation of gates at a cursor
// ---------------------------------------------------------------------------
template <typename T>
struct Runner {
  const Launch &L;
  int bw, s;
  Workspace<T> &ws;
  Counters &ctr;
  Phase1Timer *timer;
  KeySource &src;
  KeyView kv;
  Cursor c;
  // Party mode (L.party = 0 or 1): only this party's kernels run; its key is
  // kv.k[L.party] and each exchange goes through the peer.
  Peer *peer = nullptr;
  // Gates of at most pair_max elements share a launch with the next gate of
  // their truncation (tr2: keys resident, both parties here), and max-pool
  // levels of at most pool_max pairs run as one launch (pool_level); with
  // pool_tail, the levels from the third on run in one launch together.
  size_t pair_max = 0, pool_max = 0;
  bool pool_tail_on = false;

  Runner(const Launch &L_, int bw_, int s_, Workspace<T> &ws_, Counters &ctr_, Phase1Timer *t, KeySource &src_,
         Peer *peer_ = nullptr)
      : L(L_), bw(bw_), s(s_), ws(ws_), ctr(ctr_), timer(t), src(src_), peer(peer_) {}

  bool party_mode() const { return L.party >= 0; }
  // [a, a + na) and [b, b + nb) (elements) share no byte: the one-launch reveal
  // and Beaver evaluations write their output while other threads still read
  // their inputs
  static bool disjoint(const T *a, size_t na, const T *b, size_t nb) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 + na * sizeof(T) <= b0 || b0 + nb * sizeof(T) <= a0;
  }
  const uint8_t *own_key() const { return kv.k[L.party]; }
  // party mode: send this party's message (ws.m0), receive the peer's (ws.m1),
  // and reconstruct out = m0 + m1
  hipError_t exchange_reconstruct(size_t n, T *out) {
    const Peer::Seg seg{ws.m0.p, ws.m1.p, n * sizeof(T)};
    TRY(peer->exchange(L.stream, &seg, 1));
    return launch_reconstruct<T>(L, n, ws.m0.p, ws.m1.p, out);
  }
  // the same for a message known modulo 2^m: on the wire at m bits per element
  // (packed into the bit-plane buffers, free once the gate's planes are used),
  // out = (m0 + m1) mod 2^m
  hipError_t exchange_reconstruct_bits(size_t n, int m, T *out) {
    if (m >= bw) return exchange_reconstruct(n, out);
    const size_t nw = packed_words(n, m);
    TRY(ws.ensure_bits(nw));
    TRY(launch_pack_bits<T>(L, n, m, ws.m0.p, ws.b0.p));
    const Peer::Seg seg{ws.b0.p, ws.b1.p, nw * 8};
    TRY(peer->exchange(L.stream, &seg, 1));
    return launch_unpack_reconstruct<T>(L, n, m, ws.m0.p, ws.b1.p, out);
  }

  // Make the gate [c.off, end) available; returns the base of the gate
  // relative to the key view.
  hipError_t enter(size_t end, size_t *rel) {
    TRY(src.acquire(c.off, end, &kv));
    *rel = c.off - kv.begin;
    return hipSuccess;
  }
  void leave(size_t end) {
    c.off = end;
    c.gate++;
  }

  hipError_t reveal(size_t n, const T *v0, const T *v1, int rowlen, T *out) {
    const size_t end = reveal_layout(bw, n, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    RevealLayout lay = reveal_layout(bw, n, b);
    ctr.msg(n, bw);
    if (party_mode()) {  // this party's share only (v0 or v1 by party)
      const T *v = L.party ? v1 : v0;
      TRY(launch_reveal_eval<T>(L, lay, own_key(), own_key(), v, v, rowlen, ws.m0.p, ws.m0.p));
      TRY(exchange_reconstruct(n, out));
    } else if (disjoint(out, n, v0, rowlen > 0 ? n * rowlen : n) && disjoint(out, n, v1, rowlen > 0 ? n * rowlen : n)) {
      TRY(launch_reveal_sum<T>(L, lay, kv.k[0], kv.k[1], v0, v1, rowlen, out));
    } else {  // out overlaps a share: messages first
      TRY(launch_reveal_eval<T>(L, lay, kv.k[0], kv.k[1], v0, v1, rowlen, ws.m0.p, ws.m1.p));
      TRY(launch_reconstruct<T>(L, n, ws.m0.p, ws.m1.p, out));
    }
    leave(end);
    return hipSuccess;
  }

  // party mode: the truncation-family gate in two launches around the two
  // exchanges (bit planes, then messages)
  hipError_t tr_party(const TrLayout &lay, size_t n, const T *x, const T *bias, int ncol, T *out) {
    const size_t W = (n + 63) / 64;
    TRY(ws.ensure_bits(2 * W));
    TRY(launch_tr_party_bits<T>(L, lay, own_key(), x, bias, ncol, ws.b0.p));
    // each plane goes on the wire as ceil(n/32) 32-bit words
    const size_t pb = ((n + 31) / 32) * 4;
    Peer::Seg seg[2];
    int ns = 0;
    if (lay.use_a) seg[ns++] = Peer::Seg{ws.b0.p, ws.b1.p, pb};
    if (lay.use_b) seg[ns++] = Peer::Seg{ws.b0.p + W, ws.b1.p + W, pb};
    TRY(peer->exchange(L.stream, seg, ns));
    if (lay.kind == G_DRELU)  // the output bit is public now
      return launch_tr_party_msg<T>(L, lay, own_key(), x, bias, ncol, ws.b0.p, ws.b1.p, out);
    TRY(launch_tr_party_msg<T>(L, lay, own_key(), x, bias, ncol, ws.b0.p, ws.b1.p, ws.m0.p));
    return exchange_reconstruct_bits(n, tr_out_bits(lay.kind, bw, s), out);
  }

  // AES calls per element and party of a gate's DCF walks
  static int tr_levels(const TrLayout &lay) {
    return (lay.use_a ? lay.a.L + 1 : 0) + (lay.use_b ? lay.b.L + 1 : 0);
  }
  // Algorithmic key bytes per element of a gate evaluated by both parties in one
  // launch: per DCF the correction words and the leaf once (both parties'
  // threads of a workgroup read party 0's copy) and each party's root (16 B) and
  // mask bit; each party's G word of the element's case and kappa (the bias
  // vector is ncol words, cache resident; the exchanges stay in LDS).
  static double tr_key_bytes(const TrLayout &lay) {
    const double tb = double(sizeof(T));
    double per = (lay.ncase > 0 ? 2.0 * tb : 0.0) + (lay.relu ? 2.0 * tb : 0.0);
    if (lay.use_a) per += 16.0 * (lay.a.L + 1) + 2.0 * (16.0 + 0.125);
    if (lay.use_b) per += 16.0 * (lay.b.L + 1) + 2.0 * (16.0 + 0.125);
    return per;
  }
  // profiled forward: events around one gate launch and its algorithmic work
  // (AES calls per element and party, bytes per element: the masked input and the
  // revealed output once, plus the keys)
  hipError_t time_begin(hipEvent_t *e0, hipEvent_t *e1, Launch *L1) {
    if (!timer || !timer->on) return hipSuccess;
    TRY(hipEventCreateWithFlags(e0, kTimingEvent));
    TRY(hipEventCreateWithFlags(e1, kTimingEvent));
    TRY(hipEventRecord(*e0, L.stream));
    L1->profiled = true;
    return hipSuccess;
  }
  hipError_t time_end(hipEvent_t e0, hipEvent_t e1, size_t n, int levels, double key_bytes) {
    if (!timer || !timer->on) return hipSuccess;
    TRY(hipEventRecord(e1, L.stream));
    timer->ev.push_back(e0);
    timer->ev.push_back(e1);
    timer->elems.push_back(n);
    timer->levels.push_back(levels);
    timer->bytes.push_back((2.0 * double(sizeof(T)) + key_bytes) * double(n));
    return hipSuccess;
  }

  hipError_t tr(int kind, size_t n, const T *x, const T *bias, int ncol, T *out) {
    const size_t end = tr_layout(kind, bw, s, n, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    TrLayout lay = tr_layout(kind, bw, s, n, b);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    Launch L1 = L;
    TRY(time_begin(&e0, &e1, &L1));
    if (party_mode())
      TRY(tr_party(lay, n, x, bias, ncol, out));
    else
      TRY(launch_tr_eval<T>(L1, lay, kv.k[0], kv.k[1], x, bias, ncol, out));
    TRY(time_end(e0, e1, n, tr_levels(lay), tr_key_bytes(lay)));
    ctr.bitplanes(n, int(lay.use_a) + int(lay.use_b));
    if (kind != G_DRELU) ctr.msg_bits(n, tr_out_bits(kind, bw, s), bw);  // DRELU: the output bit is already public
    leave(end);
    return hipSuccess;
  }

  // Gate kind on x (with the bias), then gate kind2 on its revealed output, in
  // one launch (both parties here, resident keys: both gates' keys in one view);
  // the same keys, exchanges and counted bytes as tr(kind) then tr(kind2), and x
  // is left as it was.
  hipError_t tr2(int kind, int kind2, size_t n, const T *x, const T *bias, int ncol, T *out) {
    const size_t end1 = tr_layout(kind, bw, s, n, c.off).end;
    size_t b1, b2;
    TRY(enter(end1, &b1));
    const TrLayout lay = tr_layout(kind, bw, s, n, b1);
    leave(end1);
    const size_t end2 = tr_layout(kind2, bw, s, n, c.off).end;
    TRY(enter(end2, &b2));
    const TrLayout lay2 = tr_layout(kind2, bw, s, n, b2);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    Launch L1 = L;
    TRY(time_begin(&e0, &e1, &L1));
    TRY(launch_tr_eval2<T>(L1, lay, lay2, kv.k[0], kv.k[1], x, bias, ncol, out));
    TRY(time_end(e0, e1, n, tr_levels(lay) + tr_levels(lay2), tr_key_bytes(lay) + tr_key_bytes(lay2)));
    for (const TrLayout *l : {&lay, &lay2}) {
      ctr.bitplanes(n, int(l->use_a) + int(l->use_b));
      ctr.msg_bits(n, tr_out_bits(l->kind, bw, s), bw);
    }
    leave(end2);
    return hipSuccess;
  }

  // One level of the max-pool tree over B blocks of R rows of C words, V -> Vn
  // (max(a, b) = a + ReLU(b - a) over the row pairs, an odd last row carried).
  // A level of at most pool_max pairs with both parties here is one gate launch
  // that forms the pair differences and writes the next level itself;
  // otherwise the differences (into D), the gate (into Y) and the combination
  // run apart (in party mode around the gate's exchanges; the large levels of
  // lanes of many samples measured no faster in one launch).
  hipError_t pool_level(int kind, int B, int R, int C, const T *V, T *D, T *Y, T *Vn) {
    const size_t n = size_t(B) * (R / 2) * C;
    if (party_mode() || n > pool_max || size_t(B) * R * C >= (size_t(1) << 32)) {
      TRY(launch_pool_diff<T>(L, B, R, C, V, D));
      TRY(tr(kind, n, D, nullptr, 1, Y));
      return launch_pool_combine<T>(L, B, R, C, V, Y, nullptr, Vn);
    }
    const size_t end = tr_layout(kind, bw, s, n, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    TrLayout lay = tr_layout(kind, bw, s, n, b);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    Launch L1 = L;
    TRY(time_begin(&e0, &e1, &L1));
    TRY(launch_tr_eval_pool<T>(L1, lay, kv.k[0], kv.k[1], B, R, C, V, Vn));
    TRY(time_end(e0, e1, n, tr_levels(lay), tr_key_bytes(lay)));
    ctr.bitplanes(n, int(lay.use_a) + int(lay.use_b));
    ctr.msg(n, bw);
    leave(end);
    return hipSuccess;
  }

  // The last nlev levels of the max-pool tree (pairs[l] pairs per block at
  // level l, R0 rows at the first) in one launch: every workgroup takes whole
  // columns through all of them (resident keys, both parties here); the same
  // keys, exchanges and counted bytes as nlev pool_level calls.
  hipError_t pool_tail(int kind, int B, int R0, int C, const T *V, int nlev, const int *pairs, T *out) {
    if (nlev < 1 || nlev > 8) return hipErrorInvalidValue;
    TrLayout lay[8];
    KeyView kv0;
    size_t n_all = 0;
    for (int l = 0; l < nlev; l++) {
      const size_t n = size_t(B) * pairs[l] * C;
      const size_t end = tr_layout(kind, bw, s, n, c.off).end;
      size_t b;
      TRY(enter(end, &b));
      if (l == 0)
        kv0 = kv;
      else if (kv.k[0] != kv0.k[0] || kv.k[1] != kv0.k[1] || kv.begin != kv0.begin)
        return hipErrorInvalidValue;  // the levels' keys must sit in one view
      lay[l] = tr_layout(kind, bw, s, n, b);
      leave(end);
      n_all += n;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    Launch L1 = L;
    TRY(time_begin(&e0, &e1, &L1));
    TRY(launch_tr_eval_pool_tail<T>(L1, lay, nlev, kv0.k[0], kv0.k[1], B, R0, C, V, out));
    TRY(time_end(e0, e1, n_all, tr_levels(lay[0]), tr_key_bytes(lay[0])));
    for (int l = 0; l < nlev; l++) {
      ctr.bitplanes(lay[l].N, int(lay[l].use_a) + int(lay[l].use_b));
      ctr.msg(lay[l].N, bw);
    }
    return hipSuccess;
  }

  hipError_t mul(size_t nx, size_t ny, size_t nz, const MulMap &map, const T *x, const T *y, T *out) {
    const size_t end = mul_layout(bw, nx, ny, nz, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    MulLayout lay = mul_layout(bw, nx, ny, nz, b);
    ctr.msg(nz, bw);
    if (party_mode()) {
      TRY(launch_mul_eval<T>(L, lay, own_key(), own_key(), map, x, y, ws.m0.p, ws.m0.p));
      TRY(exchange_reconstruct(nz, out));
    } else if (disjoint(out, nz, x, nx) && disjoint(out, nz, y, ny)) {
      TRY(launch_mul_eval_sum<T>(L, lay, kv.k[0], kv.k[1], map, x, y, out));
    } else {  // out overlaps an operand, which other threads gather: messages first
      TRY(launch_mul_eval<T>(L, lay, kv.k[0], kv.k[1], map, x, y, ws.m0.p, ws.m1.p));
      TRY(launch_reconstruct<T>(L, nz, ws.m0.p, ws.m1.p, out));
    }
    leave(end);
    return hipSuccess;
  }

  // vh: n-element scratch for the revealed intermediate
  hipError_t lut8(size_t n, const T *table, const T *x, T *vh, T *out) {
    const size_t end = lut8_layout(bw, n, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    Lut8Layout lay = lut8_layout(bw, n, b);
    if (party_mode()) {
      ctr.msg(n, bw);
      ctr.msg(n, bw);
      TRY(launch_lut8_phase1<T>(L, lay, own_key(), own_key(), table, x, ws.m0.p, ws.m0.p));
      TRY(exchange_reconstruct(n, vh));
      TRY(launch_lut8_phase2<T>(L, lay, own_key(), own_key(), vh, ws.m0.p, ws.m0.p));
      TRY(exchange_reconstruct(n, out));
      leave(end);
      return hipSuccess;
    }
    TRY(launch_lut8_phase1<T>(L, lay, kv.k[0], kv.k[1], table, x, ws.m0.p, ws.m1.p));
    ctr.msg(n, bw);
    TRY(launch_reconstruct<T>(L, n, ws.m0.p, ws.m1.p, vh));
    TRY(launch_lut8_phase2<T>(L, lay, kv.k[0], kv.k[1], vh, ws.m0.p, ws.m1.p));
    ctr.msg(n, bw);
    TRY(launch_reconstruct<T>(L, n, ws.m0.p, ws.m1.p, out));
    leave(end);
    return hipSuccess;
  }

  // batched C_b = A_b (M x K) . B_b (K x N), Beaver
  hipError_t sxs(int nb, int M, int K, int N, const T *A, const T *Bm, T *out) {
    const size_t end = sxs_layout(bw, nb, M, K, N, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    SxsLayout lay = sxs_layout(bw, nb, M, K, N, b);
    const uint8_t *K0 = kv.k[0], *K1 = kv.k[1];
    GemmSpan span{timer, L.stream};
    TRY(span.begin(3.0 * nb * double(M) * K * N));
    GemmArgs<T> g;
    g.M = M;
    g.K = K;
    g.N = N;
    g.batch = nb;
    g.sA = size_t(M) * K;
    g.sB = size_t(K) * N;
    g.sC = size_t(M) * N;
    // party 0: (A^ - RA0)(B^ - RB0) + C0
    g.A1 = A;
    g.A2 = reinterpret_cast<const T *>(K0 + lay.off_ra);
    g.B1 = Bm;
    g.B2 = reinterpret_cast<const T *>(K0 + lay.off_rb);
    g.Cin = reinterpret_cast<const T *>(K0 + lay.off_c);
    g.C = ws.m0.p;
    // party 1: C1 - (A^ RB1 + RA1 B^) = C1 - [A^ RA1] [RB1; B^]
    GemmArgs<T> h = g;
    h.A2 = nullptr;
    h.B2 = nullptr;
    h.B1 = reinterpret_cast<const T *>(K1 + lay.off_rb);
    h.A1b = reinterpret_cast<const T *>(K1 + lay.off_ra);
    h.B1b = Bm;
    h.Cin = reinterpret_cast<const T *>(K1 + lay.off_c);
    h.C = ws.m1.p;
    h.sign = -1;
    const size_t nc = size_t(nb) * M * N;
    ctr.msg(nc, bw);
    if (party_mode()) {  // this party's product only, into m0
      GemmArgs<T> &mine = L.party ? h : g;
      mine.C = ws.m0.p;
      TRY(launch_gemm<T>(L, mine));
      TRY(span.end());
      TRY(exchange_reconstruct(nc, out));
      leave(end);
      return hipSuccess;
    }
    // both parties' products and the reconstruction of the exchanged shares
    TRY(launch_gemm_pair_sum<T>(L, g, h, out));
    TRY(span.end());
    leave(end);
    return hipSuccess;
  }

  // last layer: unmask with the clear output mask, floor shift, bias
  hipError_t output(int B, size_t n, const T *z, int64_t bias, int64_t *out) {
    const size_t end = reveal_layout(bw, n, c.off).end;
    size_t b;
    TRY(enter(end, &b));
    RevealLayout lay = reveal_layout(bw, n, b);
    TRY(launch_output<T>(L, B, bw, s, z, reinterpret_cast<const T *>(kv.k[0] + lay.off_r), bias, out));
    leave(end);
    return hipSuccess;
  }
};

// ---------------------------------------------------------------------------
// dealer: keys of gates at a cursor, written into resident arenas
// ---------------------------------------------------------------------------
template <typename T>
struct Dealer {
  const Launch &L;
  int bw, s;
  uint64_t seed;
  uint8_t *K0, *K1;
  Cursor c;

  hipError_t reveal(size_t n, T *mask) {
    RevealLayout lay = reveal_layout(bw, n, c.off);
    TRY(launch_reveal_keygen<T>(L, lay, seed, c.gate, mask, K0, K1));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
  hipError_t tr(int kind, size_t n, const T *in, T *out) {
    TrLayout lay = tr_layout(kind, bw, s, n, c.off);
    TRY(launch_tr_keygen<T>(L, lay, seed, c.gate, in, out, K0, K1));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
  hipError_t mul(size_t nx, size_t ny, size_t nz, const MulMap &map, const T *rx, const T *ry, T *rz) {
    MulLayout lay = mul_layout(bw, nx, ny, nz, c.off);
    TRY(launch_mul_keygen<T>(L, lay, seed, c.gate, map, rx, ry, rz, K0, K1));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
  hipError_t lut8(size_t n, const T *in, T *out) {
    Lut8Layout lay = lut8_layout(bw, n, c.off);
    TRY(launch_lut8_keygen<T>(L, lay, seed, c.gate, in, out, K0, K1));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
  // SxS: C = rA.rB - RA0.RB0 + rC; tmp: nb*M*N scratch
  hipError_t sxs(int nb, int M, int K, int N, const T *rA, const T *rB, T *rC, T *tmp) {
    SxsLayout lay = sxs_layout(bw, nb, M, K, N, c.off);
    T *RA0 = reinterpret_cast<T *>(K0 + lay.off_ra), *RA1 = reinterpret_cast<T *>(K1 + lay.off_ra);
    T *RB0 = reinterpret_cast<T *>(K0 + lay.off_rb), *RB1 = reinterpret_cast<T *>(K1 + lay.off_rb);
    const size_t na = size_t(nb) * M * K, nbb = size_t(nb) * K * N, nc = size_t(nb) * M * N;
    TRY(launch_split<T>(L, seed, c.gate, F_SPLIT + 0, na, rA, RA0, RA1, nullptr));
    TRY(launch_split<T>(L, seed, c.gate, F_SPLIT + 1, nbb, rB, RB0, RB1, nullptr));
    TRY(launch_prf_ring<T>(L, seed, c.gate, F_ROUT, nc, rC));  // output mask
    GemmArgs<T> g;
    g.M = M;
    g.K = K;
    g.N = N;
    g.batch = nb;
    g.sA = size_t(M) * K;
    g.sB = size_t(K) * N;
    g.sC = size_t(M) * N;
    g.A1 = rA;
    g.B1 = rB;
    g.Cin = rC;
    g.C = tmp;
    TRY(launch_gemm<T>(L, g));  // rA.rB + rC
    g.A1 = RA0;
    g.B1 = RB0;
    g.Cin = tmp;
    g.C = tmp;
    g.sign = -1;
    TRY(launch_gemm<T>(L, g));  // - RA0.RB0
    TRY(launch_split<T>(L, seed, c.gate, F_SPLIT + 2, nc, tmp, reinterpret_cast<T *>(K0 + lay.off_c),
                        reinterpret_cast<T *>(K1 + lay.off_c), nullptr));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
  // output mask in the clear for both evaluators
  hipError_t output(size_t n, const T *mask) {
    RevealLayout lay = reveal_layout(bw, n, c.off);
    TRY(hipMemcpyAsync(K0 + lay.off_r, mask, n * sizeof(T), hipMemcpyDeviceToDevice, L.stream));
    TRY(hipMemcpyAsync(K1 + lay.off_r, mask, n * sizeof(T), hipMemcpyDeviceToDevice, L.stream));
    c.off = lay.end;
    c.gate++;
    return hipSuccess;
  }
};

// ---------------------------------------------------------------------------
// secure adjacency normalisation block (secure_adj_norm.h:203-374, 393-659):
// reveal A; reveal the degrees (row sums of the A shares); LUT8 -> T[d];
// MUL T[d_i] T[d_j] over the upper triangle; TRSLACK; MUL A (.) W.
// ---------------------------------------------------------------------------
template <typename T>
struct AdjNorm {
  int B = -1, N = -1, s = 0, nmax = 0;
  DevBuf<T> table;                  // T[k] = llround(2^s / sqrt(k)), 1 <= k <= nmax
  DevBuf<T> t0, t1, p0, p1;         // scratch: 2 x BN, 2 x BP

  static size_t layout_end(int bw, int s, int B, int N, size_t o) {
    const size_t BN = size_t(B) * N, BNN = BN * N, BP = size_t(B) * pairs_of(N);
    o = reveal_layout(bw, BNN, o).end;
    o = reveal_layout(bw, BN, o).end;
    o = lut8_layout(bw, BN, o).end;
    o = mul_layout(bw, BN, BN, BP, o).end;
    o = tr_layout(G_TRSLACK, bw, s, BP, o).end;
    o = mul_layout(bw, BNN, BP, BNN, o).end;
    return o;
  }

  hipError_t prepare(int B_, int N_, int s_, int nmax_) {
    if (B_ == B && N_ == N && s_ == s && nmax_ == nmax) return hipSuccess;
    const size_t P = pairs_of(N_), BN = size_t(B_) * N_, BNN = BN * N_;
    // the Beaver products index their operands with 32-bit element indices
    if (BNN >= (size_t(1) << 32)) return hipErrorInvalidValue;
    std::vector<T> tab(256, T(0));
    const double q = std::ldexp(1.0, s_);
    for (int k = 1; k <= nmax_ && k < 256; k++) tab[k] = T(std::llround(q / std::sqrt(double(k))));
    TRY(table.alloc(256));
    TRY(hipMemcpy(table.p, tab.data(), 256 * sizeof(T), hipMemcpyHostToDevice));
    TRY(t0.alloc(BN));
    TRY(t1.alloc(BN));
    TRY(p0.alloc(size_t(B_) * P));
    TRY(p1.alloc(size_t(B_) * P));
    B = B_;
    N = N_;
    s = s_;
    nmax = nmax_;
    return hipSuccess;
  }

  // rA: mask of the revealed A (BNN); rN: mask of A_norm (BNN)
  hipError_t keygen(Dealer<T> &d, T *rA, T *rN) {
    const size_t BN = size_t(B) * N, BNN = BN * N, BP = size_t(B) * pairs_of(N);
    TRY(d.reveal(BNN, rA));
    TRY(d.reveal(BN, t0.p));                                // degree mask
    TRY(d.lut8(BN, t0.p, t1.p));                            // mask of T[d]
    TRY(d.mul(BN, BN, BP, MulMap::of(MulMap::OUTER_TRI, N), t1.p, t1.p, p0.p));  // mask of the outer product
    TRY(d.tr(G_TRSLACK, BP, p0.p, p1.p));                    // mask of W
    TRY(d.mul(BNN, BP, BNN, MulMap::of(MulMap::SYM_HADAMARD, N), rA, p1.p, rN));  // mask of A_norm
    return hipSuccess;
  }

  // a0, a1: A shares (BNN); Ah: revealed A (BNN); An: masked A_norm (BNN)
  // pre_done (optional): recorded on the runner's stream once the memory-bound
  // gates before the truncation are enqueued (a pipelined next group waits on it)
  hipError_t eval(Runner<T> &r, const T *a0, const T *a1, T *Ah, T *An, hipEvent_t pre_done = nullptr) {
    const size_t BN = size_t(B) * N, BNN = BN * N, BP = size_t(B) * pairs_of(N);
    TRY(r.reveal(BNN, a0, a1, 0, Ah));
    TRY(r.reveal(BN, a0, a1, N, t0.p));  // degree = row sums of the A shares
    TRY(r.lut8(BN, table.p, t0.p, t1.p, t0.p));
    TRY(r.mul(BN, BN, BP, MulMap::of(MulMap::OUTER_TRI, N), t0.p, t0.p, p0.p));
    if (pre_done) TRY(hipEventRecord(pre_done, r.L.stream));
    TRY(r.tr(G_TRSLACK, BP, p0.p, nullptr, 1, p1.p));
    TRY(r.mul(BNN, BP, BNN, MulMap::of(MulMap::SYM_HADAMARD, N), Ah, p1.p, An));
    return hipSuccess;
  }
};

// Keys in one device allocation per party, addressed directly.
struct ArenaSource final : KeySource {
  const uint8_t *k[2] = {nullptr, nullptr};
  size_t bytes = 0;
  hipError_t acquire(size_t begin, size_t end, KeyView *kv) override {
    if (end > bytes || begin > end) return hipErrorInvalidValue;
    kv->k[0] = k[0];
    kv->k[1] = k[1];
    kv->begin = 0;
    return hipSuccess;
  }
};

}  // namespace

// ===========================================================================
// the model
// ===========================================================================
template <typename T>
class Model final : public ModelBase, KeySource {
 public:
  Model(int bw, int s, const ModelDims &d, const Launch &L) : bw_(bw), s_(s), d_(d), L_(L), quad_base_(L.quad_per_cu) {}
  ~Model() override {
    drop_graph();
    stop_io();
    if (cs_) (void)hipStreamSynchronize(cs_);
    free_arena();
    free_stream();
    timer.reset();
  }

  // slack 3: every layer truncation is LocalARS (the reference's default,
  // gpu_mpc/ddg_orca_batched.h:180-199): a local shift, then a RELU gate where the
  // layer has a ReLU
  bool local_trunc() const { return d_.slack == 3; }
  // the GCN products H.W^T: (slack 1, 2) TRSLACK, exact for |x| < 2^(bw-2), else
  // the layer truncation
  bool xw_slack() const { return d_.slack == 1 || d_.slack == 2; }
  // the GCN aggregation A.XW + bias, then ReLU: the layer truncation with ReLU, or
  // (slack 2) TRSLACK with the bias followed by RELUSLACK on the truncated value
  bool agg_split() const { return d_.slack == 2; }
  // The max-pool's sentinel and ReLU gate.  Exact and slack layer truncations
  // leave the GCN activations in [0, 2^(bw-s-1)) (EXTRELU outputs; RELUSLACK's
  // are smaller), so with the sentinel -2^(bw-s-1) on padding rows every pool
  // value lies in [-2^(bw-s-1), 2^(bw-s-1)), every pair difference below 2^(bw-s)
  // in magnitude, and its ReLU takes a (bw-s)-bit DCF (RELUPOOL, 14 AES at bw=32)
  // instead of a (bw-1)-bit one (25).  The maximum over a sample with a real atom
  // is the one the reference's sentinel -2^(bw-2) gives (fixed_forward.py:33-36,
  // 76-80).  Local truncation leaves activations anywhere in [0, 2^(bw-1)), and
  // a mask scale above bw-s-1 does not fit the smaller sentinel: there the
  // reference's sentinel and a full RELU gate.
  bool pool_narrow() const { return !local_trunc() && d_.mask_scale <= bw_ - s_ - 1; }
  int pool_kind() const { return pool_narrow() ? G_RELUPOOL : G_RELU; }
  int pool_sentinel_bit() const { return pool_narrow() ? bw_ - s_ - 1 : bw_ - 2; }

  // A layer truncation by s (+ bias) and, for relu, the ReLU.  Exact: the
  // truncate-reduce TRMOD (one s-bit DCF; its output is exact modulo 2^(bw-s)),
  // revealed, then EXT or EXTRELU (one (bw-s-1)-bit DCF gives the sign and the
  // wrap) -- the reference's TrFloor as truncate-reduce plus sign extension
  // (gpu_mpc/dpf_dcf_adapter.h:274-303) with the ReLU fused into the extension as
  // in gpuReluExtend (:225-234): 6 + 13 AES per element and party at bw=32
  // instead of 31 for one fused gate over the full width.  With local
  // truncation: the local shift (no key) followed, for relu, by a RELU gate.
  // Eval may overwrite x; keygen may overwrite the mask rin.
  hipError_t trunc_eval(Runner<T> &r, bool relu, size_t n, T *x, const T *bias, int ncol, T *y) {
    if (!local_trunc()) {
      if (n <= r.pair_max) return r.tr2(G_TRMOD, relu ? G_EXTRELU : G_EXT, n, x, bias, ncol, y);
      TRY(r.tr(G_TRMOD, n, x, bias, ncol, x));
      return r.tr(relu ? G_EXTRELU : G_EXT, n, x, nullptr, 1, y);
    }
    TRY(launch_local_ars<T>(L_, n, s_, x, bias, ncol, relu ? x : y));
    return relu ? r.tr(G_RELU, n, x, nullptr, 1, y) : hipSuccess;
  }
  hipError_t trunc_keygen(Dealer<T> &d, bool relu, size_t n, T *rin, T *rout) {
    if (!local_trunc()) {
      TRY(d.tr(G_TRMOD, n, rin, rin));
      return d.tr(relu ? G_EXTRELU : G_EXT, n, rin, rout);
    }
    TRY(launch_local_ars<T>(L_, n, s_, rin, nullptr, 1, relu ? rin : rout));
    return relu ? d.tr(G_RELU, n, rin, rout) : hipSuccess;
  }

  // ---------------- weights ----------------
  int nlayers() const { return 5 + d_.nfus; }
  // The fully connected products' outputs (layers l >= 3) each have their own
  // range of fc_, cleared by one launch per forward, so that their split-K
  // slices add into zeros without a clearing launch per product.
  size_t fc_off(int B, int l) const {
    size_t o = 0;
    for (int j = 3; j < l; j++) {
      int in, out;
      layer_io(j, &in, &out);
      o += size_t(B) * out;
    }
    return o;
  }
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
    return hipSuccess;
  }

  // ---------------- gate plan ----------------
  // Key range of every gate of a batch of B, in forward order.
  std::vector<GateKey> plan(int B) const {
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N;
    std::vector<GateKey> g;
    size_t o = 0;
    auto push = [&](size_t end) -> GateKey & {
      GateKey k;
      k.begin = o;
      k.end = end;
      k.gate = uint32_t(g.size() + 1);
      g.push_back(k);
      o = end;
      return g.back();
    };
    auto dcf_shared = [](GateKey &k, const DcfLayout &d) { k.share(d.off_cw, d.off_leaf + d.N * 16); };
    auto tr = [&](int kind, size_t n) {
      TrLayout lay = tr_layout(kind, bw_, s_, n, o);
      GateKey &k = push(lay.end);
      k.tr_kind = kind;
      k.n = n;
      if (lay.use_a) dcf_shared(k, lay.a);
      if (lay.use_b) dcf_shared(k, lay.b);
    };
    push(reveal_layout(bw_, BN * d_.feat, o).end);
    push(reveal_layout(bw_, BN, o).end);
    {  // adjacency block: six gates
      const size_t BNN = BN * N, BP = size_t(B) * pairs_of(N);
      push(reveal_layout(bw_, BNN, o).end);
      push(reveal_layout(bw_, BN, o).end);
      Lut8Layout lut = lut8_layout(bw_, BN, o);
      dcf_shared(push(lut.end), lut.dpf);
      push(mul_layout(bw_, BN, BN, BP, o).end);
      tr(G_TRSLACK, BP);
      push(mul_layout(bw_, BNN, BP, BNN, o).end);
    }
    // the gates of trunc_keygen / trunc_eval
    auto trunc = [&](bool relu, size_t n) {
      if (local_trunc()) {
        if (relu) tr(G_RELU, n);
        return;
      }
      tr(G_TRMOD, n);
      tr(relu ? G_EXTRELU : G_EXT, n);
    };
    for (int l = 0; l < 3; l++) {
      size_t E = BN * d_.gcn[l];
      if (xw_slack())
        tr(G_TRSLACK, E);
      else
        trunc(false, E);
      push(sxs_layout(bw_, B, N, N, d_.gcn[l], o).end);
      if (agg_split()) {
        tr(G_TRSLACK, E);
        tr(G_RELUSLACK, E);
      } else {
        trunc(true, E);
      }
    }
    int pairs[32];
    int Lv = pool_levels(N, pairs);
    for (int l = 0; l < Lv; l++) tr(pool_kind(), size_t(B) * pairs[l] * d_.gcn[2]);
    trunc(true, size_t(B) * d_.dfc[0]);
    trunc(false, size_t(B) * d_.dfc[1]);
    for (int k = 0; k < d_.nfus - 1; k++) trunc(true, size_t(B) * d_.fus[k]);
    {  // output: the clear output mask, the same for both parties
      RevealLayout lay = reveal_layout(bw_, size_t(B) * d_.fus[d_.nfus - 1], o);
      push(lay.end).share(lay.off_r, lay.end);
    }
    return g;
  }

  size_t key_bytes(int B) const override { return plan(B).back().end; }

  uint8_t *arena(int party) override { return arena_[party]; }

  void free_arena() {
    drop_graph();
    for (int p = 0; p < 2; p++) {
      if (arena_[p]) (void)hipFree(arena_[p]);
      arena_[p] = nullptr;
    }
    arena_bytes_ = 0;
  }
  hipError_t release_arena() override {
    TRY(hipStreamSynchronize(L_.stream));
    free_arena();
    if (!streaming_) keyed_B_ = -1;
    return hipSuccess;
  }

  hipError_t ensure_arena(int B) {
    size_t need = key_bytes(B);
    if (need <= arena_bytes_) return hipSuccess;
    free_arena();
    for (int p = 0; p < 2; p++)  // party mode: this party's key only
      if (party_ < 0 || p == party_) TRY(hipMalloc((void **)&arena_[p], need));
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
    TRY(hipStreamSynchronize(L_.stream));  // buffers may be reallocated under earlier work
    drop_graph();
    const int N = d_.n_nodes;
    const size_t E = emax(B), BN = size_t(B) * N, BNN = BN * N;
    for (auto *b : {&bA_, &bB_, &bC_}) TRY(b->alloc(E));
    TRY(ws_.ensure(E));
    TRY(Ah_.alloc(BNN));
    TRY(An_.alloc(BNN));
    TRY(mh_.alloc(BN));
    TRY(V0_.alloc(BN * d_.gcn[2]));
    TRY(V1_.alloc(BN * d_.gcn[2]));
    TRY(fc_.alloc(fc_off(B, 5 + d_.nfus)));
    TRY(out_.alloc(B));
    TRY(adj_.prepare(B, N, s_, d_.lut_nmax));
    work_B_ = B;
    return hipSuccess;
  }

  // ---------------- dealer ----------------
  // back from streamed keys to a resident arena (keygen or import after attach)
  hipError_t leave_stream() {
    if (!streaming_) return hipSuccess;
    stop_io();
    TRY(hipStreamSynchronize(L_.stream));
    if (cs_) TRY(hipStreamSynchronize(cs_));
    free_stream();
    keyed_B_ = -1;
    return hipSuccess;
  }

  hipError_t keygen(int B, uint64_t seed) override {
    if (party_ >= 0) return hipErrorNotSupported;  // the dealer holds both parties' keys
    TRY(leave_stream());
    keyed_B_ = -1;  // until the new keys are complete
    TRY(hipStreamSynchronize(L_.stream));  // a running forward may still read the arena
    drop_graph();
    TRY(ensure_arena(B));
    TRY(ensure_work(B));
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N, BNN = BN * N;
    const size_t E = emax(B);
    DevBuf<T> rX, t1, t2, rA, rN, rm, gt;
    TRY(rX.alloc(E));
    TRY(t1.alloc(E));
    TRY(t2.alloc(E));
    TRY(rA.alloc(BNN));
    TRY(rN.alloc(BNN));
    TRY(rm.alloc(BN));
    TRY(gt.alloc(E));
    Dealer<T> d{L_, bw_, s_, seed, arena_[0], arena_[1], Cursor{}};
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

    TRY(d.reveal(BN * d_.feat, rX.p));
    TRY(d.reveal(BN, rm.p));
    TRY(adj_.keygen(d, rA.p, rN.p));
    // GCN stack; rX holds the running activation mask
    for (int l = 0; l < 3; l++) {
      const int fo = d_.gcn[l];
      const size_t En = BN * fo;
      TRY(pub_gemm(rX.p, l, BN, t1.p));
      if (xw_slack())
        TRY(d.tr(G_TRSLACK, En, t1.p, t2.p));
      else
        TRY(trunc_keygen(d, false, En, t1.p, t2.p));
      TRY(d.sxs(B, N, N, fo, rN.p, t2.p, t1.p, gt.p));
      if (agg_split()) {
        TRY(d.tr(G_TRSLACK, En, t1.p, t2.p));
        TRY(d.tr(G_RELUSLACK, En, t2.p, rX.p));
      } else {
        TRY(trunc_keygen(d, true, En, t1.p, rX.p));
      }
    }
    // pool
    const int C = d_.gcn[2];
    const T Sm = T(1) << (pool_sentinel_bit() - d_.mask_scale);
    TRY(launch_pool_prep<T>(L_, BN, C, rX.p, rm.p, Sm, T(0), t2.p));  // rV in t2
    T *cur = t2.p, *nxt = rX.p;
    int pairs[32];
    const int Lv = pool_levels(N, pairs);
    int R = N;
    for (int l = 0; l < Lv; l++) {
      const int pr = pairs[l];
      const size_t En = size_t(B) * pr * C;
      TRY(launch_pool_diff<T>(L_, B, R, C, cur, t1.p));
      TRY(d.tr(pool_kind(), En, t1.p, gt.p));
      TRY(launch_pool_combine<T>(L_, B, R, C, cur, gt.p, nullptr, nxt));
      std::swap(cur, nxt);
      R = pr + (R & 1);
    }
    // drug FCs
    TRY(pub_gemm(cur, 3, B, t1.p));
    TRY(trunc_keygen(d, true, size_t(B) * d_.dfc[0], t1.p, gt.p));
    TRY(pub_gemm(gt.p, 4, B, t1.p));
    TRY(trunc_keygen(d, false, size_t(B) * d_.dfc[1], t1.p, gt.p));
    TRY(launch_concat<T>(L_, B, d_.dfc[1], d_.prot, gt.p, nullptr, nxt));
    T *h = nxt, *h2 = cur;
    for (int k = 0; k < d_.nfus; k++) {
      TRY(pub_gemm(h, 5 + k, B, t1.p));
      if (k < d_.nfus - 1) {
        TRY(trunc_keygen(d, true, size_t(B) * d_.fus[k], t1.p, h2));
        std::swap(h, h2);
      } else {
        TRY(d.output(size_t(B) * d_.fus[k], t1.p));
      }
    }
    // plan and dealer disagree (offsets, or gate ids of the seeded-plane expansion)
    if (d.c.off != key_bytes(B) || d.c.gate != uint32_t(plan(B).size()) + 1) return hipErrorUnknown;
    TRY(hipStreamSynchronize(L_.stream));
    for (int p = 0; p < 2; p++) party_key_bytes(L_, seed, p, pk_[p]);
    have_pk_ = true;
    keyed_B_ = B;
    return hipSuccess;
  }

  hipError_t import_keys(int B, const void *k0, const void *k1, size_t bytes) override {
    if (party_ >= 0) return hipErrorNotSupported;
    if (bytes != key_bytes(B)) return hipErrorInvalidValue;
    TRY(leave_stream());
    TRY(hipStreamSynchronize(L_.stream));  // a running forward may still read the arena
    keyed_B_ = -1;  // until the new keys are complete
    drop_graph();
    TRY(ensure_arena(B));
    TRY(hipMemcpy(arena_[0], k0, bytes, hipMemcpyHostToDevice));
    TRY(hipMemcpy(arena_[1], k1, bytes, hipMemcpyHostToDevice));
    have_pk_ = false;  // imported keys: the parties' PRF keys are not known here
    keyed_B_ = B;
    return hipSuccess;
  }
  hipError_t export_keys(int party, void *dst, size_t bytes) override {
    if (!arena_[party] || bytes > arena_bytes_) return hipErrorInvalidValue;
    TRY(hipStreamSynchronize(L_.stream));
    return hipMemcpy(dst, arena_[party], bytes, hipMemcpyDeviceToHost);
  }

  // ---------------- streaming ----------------
  // The bytes of party p's key a streamed copy moves, as runs that each lie
  // inside one gate (hence one chunk): party 1 skips the planes it reads from
  // party 0's copy (shared); a packed key also leaves out the planes that the
  // dealer drew from the party's own PRF key (seeded: regenerated in the device
  // slot after the copy).  src: offset in the party's host buffer, after the
  // packed format's header (the party's PRF key), or the arena offset.
  static constexpr size_t kPackedHeader = 256;
  struct Run {
    size_t b, e, src;
  };
  // planes of a truncation-family gate drawn from party p's own PRF key
  void seeded_planes(const GateKey &g, int p, std::vector<std::pair<size_t, size_t>> &out) const {
    if (!g.tr_kind) return;
    const TrLayout lay = tr_layout(g.tr_kind, bw_, s_, g.n, g.begin);
    const size_t tb = size_t(bw_ / 8);
    for (const DcfLayout *dl : {lay.use_a ? &lay.a : nullptr, lay.use_b ? &lay.b : nullptr}) {
      if (!dl) continue;
      out.emplace_back(dl->off_root, dl->off_root + g.n * 16);
      out.emplace_back(dl->off_z, dl->off_z + zwords(g.n) * 4);
    }
    if (p == 0) {
      if (lay.relu) out.emplace_back(lay.off_kappa, lay.off_kappa + g.n * tb);
      if (lay.ncase > 0) out.emplace_back(lay.off_g, lay.off_g + size_t(lay.ncase) * g.n * tb);
    }
  }
  std::vector<Run> party_runs(int B, int party, bool packed) const {
    std::vector<Run> r;
    size_t acc = kPackedHeader;
    std::vector<std::pair<size_t, size_t>> om;
    for (const GateKey &g : plan(B)) {
      om.clear();
      if (party == 1)
        for (int j = 0; j < g.nsh; j++) om.emplace_back(g.sh[j][0], g.sh[j][1]);
      if (packed) seeded_planes(g, party, om);
      std::sort(om.begin(), om.end());
      size_t cur = g.begin;
      auto add = [&](size_t b, size_t e) {
        if (e <= b) return;
        r.push_back(Run{b, e, packed ? acc : b});
        acc += e - b;
      };
      for (const auto &x : om) {
        add(cur, x.first);
        cur = std::max(cur, x.second);
      }
      add(cur, g.end);
    }
    return r;
  }
  // packed key of party p: the header (its PRF key) and its runs
  size_t unique_key_bytes(int B, int party) const override {
    size_t n = kPackedHeader;
    for (const Run &u : party_runs(B, party, true)) n += u.e - u.b;
    return n;
  }
  hipError_t export_unique_keys(int party, void *dst, size_t bytes) override {
    if (party < 0 || party > 1 || !arena_[party] || keyed_B_ < 1 || bytes != unique_key_bytes(keyed_B_, party))
      return hipErrorInvalidValue;
    if (!have_pk_) return hipErrorNotSupported;  // imported keys: no PRF key to expand from
    TRY(hipStreamSynchronize(L_.stream));
    uint8_t *d = static_cast<uint8_t *>(dst);
    std::memset(d, 0, kPackedHeader);
    std::memcpy(d, pk_[party], 16);
    for (const Run &u : party_runs(keyed_B_, party, true))
      TRY(hipMemcpy(d + u.src, arena_[party] + u.b, u.e - u.b, hipMemcpyDeviceToHost));
    return hipSuccess;
  }

  void free_stream() {
    for (int k = 0; k < 2; k++) {
      for (int p = 0; p < 2; p++) {
        if (slot_[k][p]) (void)hipFree(slot_[k][p]);
        slot_[k][p] = nullptr;
      }
      if (ready_[k]) (void)hipEventDestroy(ready_[k]);
      if (free_[k]) (void)hipEventDestroy(free_[k]);
      ready_[k] = free_[k] = nullptr;
    }
    if (cs_) (void)hipStreamDestroy(cs_);
    cs_ = nullptr;
    for (int p = 0; p < 2; p++)
      for (int k = 0; k < 2; k++) {
        if (stg_[p][k]) (void)hipHostFree(stg_[p][k]);
        stg_[p][k] = nullptr;
      }
    files_ = false;
    streaming_ = false;
  }

  // plan, chunks, device slots and events of the streamed arena
  hipError_t setup_stream(int B, const bool packed[2], size_t slot_bytes) {
    keyed_B_ = -1;  // the resident keys go away below; set again once the slots exist
    stop_io();
    TRY(hipStreamSynchronize(L_.stream));
    if (cs_) TRY(hipStreamSynchronize(cs_));
    free_stream();
    free_arena();  // the two slots replace the resident arena
    gates_ = plan(B);
    // chunks: maximal runs of consecutive gates that fit in one slot
    chunks_.clear();
    chunk_of_.assign(gates_.size(), 0);
    for (size_t i = 0; i < gates_.size(); i++) {
      const size_t gb = gates_[i].begin, ge = gates_[i].end;
      if (ge - gb > slot_bytes) return hipErrorInvalidValue;  // a gate larger than a slot
      if (chunks_.empty() || ge - chunks_.back().first > slot_bytes) chunks_.emplace_back(gb, ge);
      chunks_.back().second = ge;
      chunk_of_[i] = int(chunks_.size()) - 1;
    }
    chunk_max_ = 0;
    for (auto &c : chunks_) chunk_max_ = std::max(chunk_max_, c.second - c.first);
    for (int k = 0; k < 2; k++) {
      for (int p = 0; p < 2; p++) TRY(hipMalloc((void **)&slot_[k][p], chunk_max_));
      TRY(hipEventCreateWithFlags(&ready_[k], hipEventDisableTiming));
      TRY(hipEventCreateWithFlags(&free_[k], hipEventDisableTiming));
    }
    TRY(hipStreamCreateWithFlags(&cs_, hipStreamNonBlocking));
    for (int p = 0; p < 2; p++) {
      packed_[p] = packed[p];
      runs_[p] = party_runs(B, p, packed[p]);
    }
    return hipSuccess;
  }

  // a party's host key: its arena (key_bytes) or its packed key (unique_key_bytes)
  bool packed_size(int B, int party, size_t bytes, bool *packed) const {
    if (bytes == key_bytes(B)) {
      *packed = false;
      return true;
    }
    *packed = bytes == unique_key_bytes(B, party);
    return *packed;
  }

  hipError_t attach_host_keys(int B, const void *h0, size_t bytes0, const void *h1, size_t bytes1,
                              size_t slot_bytes) override {
    bool packed[2];
    if (!h0 || !h1 || slot_bytes == 0 || !packed_size(B, 0, bytes0, &packed[0]) ||
        !packed_size(B, 1, bytes1, &packed[1]))
      return hipErrorInvalidValue;
    TRY(setup_stream(B, packed, slot_bytes));
    host_[0] = static_cast<const uint8_t *>(h0);
    host_[1] = static_cast<const uint8_t *>(h1);
    for (int p = 0; p < 2; p++)
      if (packed[p]) std::memcpy(spk_[p], host_[p], 16);
    streaming_ = true;
    keyed_B_ = B;
    return hipSuccess;
  }

  // ---------------- file-backed keys ----------------
  // Key sets in two files, read chunk by chunk by an I/O thread into two pinned
  // staging buffers per party, then copied into the device slots.
  hipError_t attach_key_files(int B, const KeyFile &f0, const KeyFile &f1, bool packed0, bool packed1,
                              size_t slot_bytes) override {
    if (f0.fd < 0 || f1.fd < 0 || f0.nsets == 0 || slot_bytes == 0) return hipErrorInvalidValue;
    const bool packed[2] = {packed0, packed1};
    TRY(setup_stream(B, packed, slot_bytes));
    for (int p = 0; p < 2; p++)
      for (int k = 0; k < 2; k++) TRY(hipHostMalloc((void **)&stg_[p][k], chunk_max_, hipHostMallocDefault));
    kf_[0] = f0;
    kf_[1] = f1;
    set_ = 0;
    files_ = true;
    streaming_ = true;
    keyed_B_ = B;
    return hipSuccess;
  }

  static bool pread_all(int fd, uint8_t *dst, size_t n, uint64_t off) {
    while (n > 0) {
      const ssize_t r = ::pread(fd, dst, n, off_t(off));
      if (r <= 0) return false;
      dst += r;
      n -= size_t(r);
      off += uint64_t(r);
    }
    return true;
  }

  // I/O thread of one forward over key set `set`: chunk k goes to staging k % 2
  // once the copies of chunk k - 2 out of that buffer have completed.
  void io_loop(uint64_t set) {
    try {
      io_chunks(set);
    } catch (...) {  // allocation failure: report it to the waiting host thread
      {
        std::lock_guard<std::mutex> lk(mu_);
        io_err_ = hipErrorOutOfMemory;
      }
      cv_.notify_all();
    }
  }
  void io_chunks(uint64_t set) {
    for (int k = 0; k < int(chunks_.size()); k++) {
      const int sl = k & 1;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return abort_ || issued_ >= k - 2; });
        if (abort_) return;
      }
      // the last copies out of this buffer (this forward's chunk k - 2, or the
      // previous forward's) were recorded before ready_[sl]
      hipError_t e = hipEventSynchronize(ready_[sl]);
      const size_t b = chunks_[k].first, en = chunks_[k].second;
      // the chunk's file ranges, cut into pieces of at most kPiece bytes and
      // read by up to 16 threads (one page-cache reader moves ~19 GB/s, 16 ~41)
      struct Piece {
        int fd;
        uint8_t *dst;
        size_t n;
        uint64_t off;
      };
      constexpr size_t kPiece = size_t(64) << 20;
      const int kReaders = int(std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
      std::vector<Piece> pieces;
      auto add = [&](int fd, uint8_t *dst, size_t n, uint64_t off) {
        for (size_t o = 0; o < n; o += kPiece) pieces.push_back(Piece{fd, dst + o, std::min(kPiece, n - o), off + o});
      };
      for (int p = 0; p < 2; p++) {
        const uint64_t set_base = kf_[p].base + set * kf_[p].stride;
        if (!packed_[p] && p == 0) {  // party 0's arena: the chunk in one piece
          add(kf_[0].fd, stg_[0][sl], en - b, set_base + b);
          continue;
        }
        for (const Run &u : runs_[p])
          if (u.b >= b && u.b < en) add(kf_[p].fd, stg_[p][sl] + (u.b - b), u.e - u.b, set_base + u.src);
      }
      bool ok = e == hipSuccess;
      if (ok && k == 0)  // the set's header: the packed parties' PRF keys
        for (int p = 0; p < 2; p++)
          if (packed_[p]) ok = ok && pread_all(kf_[p].fd, spk_[p], 16, kf_[p].base + set * kf_[p].stride);
      if (ok) {
        std::vector<char> good(kReaders, 1);
        std::vector<std::thread> rd;
        try {
          for (int t = 0; t < kReaders; t++)
            rd.emplace_back([&, t] {
              for (size_t i = size_t(t); i < pieces.size(); i += kReaders)
                if (!pread_all(pieces[i].fd, pieces[i].dst, pieces[i].n, pieces[i].off)) good[t] = 0;
            });
        } catch (...) {  // joinable threads must not be destroyed
          for (auto &th : rd) th.join();
          throw;
        }
        for (auto &th : rd) th.join();
        for (char g : good) ok = ok && g;
      }
      {
        std::lock_guard<std::mutex> lk(mu_);
        if (!ok) {
          io_err_ = e != hipSuccess ? e : hipErrorFileNotFound;
        } else {
          loaded_ = k;
        }
      }
      cv_.notify_all();
      if (!ok) return;
    }
  }

  void stop_io() {
    if (!io_.joinable()) return;
    {
      std::lock_guard<std::mutex> lk(mu_);
      abort_ = true;
    }
    cv_.notify_all();
    io_.join();
  }

  // Appends this lane's key set (party 0's arena; party 1's arena or packed
  // unique planes) to fd through a pinned bounce buffer.
  hipError_t write_keys(int party, bool packed, int fd) override {
    if (!arena_[party] || keyed_B_ < 1) return hipErrorInvalidValue;
    TRY(hipStreamSynchronize(L_.stream));
    if (packed && !have_pk_) return hipErrorNotSupported;  // imported keys: no PRF key
    std::vector<Run> runs;
    if (packed)
      runs = party_runs(keyed_B_, party, true);
    else
      runs.push_back(Run{0, key_bytes(keyed_B_), 0});
    constexpr size_t kBounce = size_t(64) << 20;
    uint8_t *h = nullptr;
    TRY(hipHostMalloc((void **)&h, kBounce, hipHostMallocDefault));
    hipError_t err = hipSuccess;
    if (packed) {  // header: the party's PRF key
      uint8_t hdr[kPackedHeader] = {};
      std::memcpy(hdr, pk_[party], 16);
      for (size_t w = 0; w < kPackedHeader;) {
        const ssize_t r = ::write(fd, hdr + w, kPackedHeader - w);
        if (r <= 0) {
          (void)hipHostFree(h);
          return hipErrorFileNotFound;
        }
        w += size_t(r);
      }
    }
    for (const Run &u : runs) {
      for (size_t o = u.b; o < u.e && err == hipSuccess; o += kBounce) {
        const size_t n = std::min(kBounce, u.e - o);
        err = hipMemcpy(h, arena_[party] + o, n, hipMemcpyDeviceToHost);
        for (size_t w = 0; err == hipSuccess && w < n;) {
          const ssize_t r = ::write(fd, h + w, n - w);
          if (r <= 0) err = hipErrorFileNotFound;
          else w += size_t(r);
        }
      }
      if (err != hipSuccess) break;
    }
    (void)hipHostFree(h);
    return err;
  }

  // copy chunk k into slot k % 2 once the slot's previous chunk has been consumed;
  // party 1's copy skips the planes both parties share (read from party 0's)
  hipError_t issue_copy(int k) {
    const int sl = k & 1;
    const size_t b = chunks_[k].first, e = chunks_[k].second;
    if (files_) {  // wait for the I/O thread to stage chunk k
      std::unique_lock<std::mutex> lk(mu_);
      cv_.wait(lk, [&] { return loaded_ >= k || io_err_ != hipSuccess; });
      if (io_err_ != hipSuccess) return io_err_;
    }
    TRY(hipStreamWaitEvent(cs_, free_[sl], 0));
    for (int p = 0; p < 2; p++) {
      if (p == 0 && !packed_[0]) {  // party 0's arena: the chunk in one copy
        const uint8_t *src0 = files_ ? stg_[0][sl] : host_[0] + b;
        TRY(hipMemcpyAsync(slot_[sl][0], src0, e - b, hipMemcpyHostToDevice, cs_));
        stream_stats.bytes_h2d += e - b;
        continue;
      }
      // runs adjacent in the slot and in the source move as one copy
      size_t cb = 0, ce = 0;
      const uint8_t *csrc = nullptr;
      auto flush = [&]() -> hipError_t {
        if (ce > cb) {
          TRY(hipMemcpyAsync(slot_[sl][p] + (cb - b), csrc, ce - cb, hipMemcpyHostToDevice, cs_));
          stream_stats.bytes_h2d += ce - cb;
        }
        return hipSuccess;
      };
      for (const Run &u : runs_[p]) {
        if (u.b < b || u.b >= e) continue;
        const uint8_t *src = files_ ? stg_[p][sl] + (u.b - b) : host_[p] + u.src;
        if (ce == u.b && csrc + (ce - cb) == src) {
          ce = u.e;
          continue;
        }
        TRY(flush());
        cb = u.b;
        ce = u.e;
        csrc = src;
      }
      TRY(flush());
      if (!packed_[p]) continue;
      // the planes the party expands from its PRF key, on the copy stream
      Launch Lc = L_;
      Lc.stream = cs_;
      for (size_t i = 0; i < gates_.size(); i++) {
        const GateKey &g = gates_[i];
        if (chunk_of_[i] != k || !g.tr_kind) continue;
        const TrLayout lay = tr_layout(g.tr_kind, bw_, s_, g.n, g.begin - b);
        TRY(launch_tr_expand<T>(Lc, lay, spk_[p], g.gate, p, slot_[sl][p]));
      }
    }
    TRY(hipEventRecord(ready_[sl], cs_));
    if (files_) {
      {
        std::lock_guard<std::mutex> lk(mu_);
        issued_ = k;
      }
      cv_.notify_all();
    }
    return hipSuccess;
  }

  hipError_t acquire(size_t begin, size_t end, KeyView *kv) override {
    if (gi_ >= gates_.size() || gates_[gi_].begin != begin || gates_[gi_].end != end)
      return hipErrorUnknown;  // forward walked off the plan
    const int k = chunk_of_[gi_++];
    if (party_ >= 0) {  // this party's key in both slots
      kv->k[0] = kv->k[1] = arena_[party_];
      kv->begin = 0;
      return hipSuccess;
    }
    if (!streaming_) {
      kv->k[0] = arena_[0];
      kv->k[1] = arena_[1];
      kv->begin = 0;
      return hipSuccess;
    }
    if (k != cur_chunk_) {
      if (k > 0) {  // chunk k-1's kernels are all enqueued: its slot takes chunk k+1
        TRY(hipEventRecord(free_[(k - 1) & 1], L_.stream));
        if (k + 1 < int(chunks_.size())) TRY(issue_copy(k + 1));
      }
      TRY(hipStreamWaitEvent(L_.stream, ready_[k & 1], 0));
      kv->k[0] = slot_[k & 1][0];
      kv->k[1] = slot_[k & 1][1];
      kv->begin = chunks_[k].first;
      cur_chunk_ = k;
      stream_stats.chunks++;
    }
    return hipSuccess;
  }

  // ---------------- party mode ----------------
  // One party per process (or thread): only this party's key, shares and kernels,
  // every exchange through the peer.  party = -1 returns to both parties in one
  // process.  Drops keys and inputs.
  hipError_t set_party(int party, Peer *peer) override {
    if (party < -1 || party > 1 || (party >= 0 && !peer)) return hipErrorInvalidValue;
    if (files_ || streaming_) {
      stop_io();
      TRY(leave_stream());
    }
    TRY(hipStreamSynchronize(L_.stream));
    drop_graph();
    free_arena();
    keyed_B_ = input_B_ = -1;
    have_pk_ = false;
    party_ = party;
    peer_ = party >= 0 ? peer : nullptr;
    L_.party = party;
    return hipSuccess;
  }
  int party() const override { return party_; }
  hipError_t import_party_key(int B, const void *key, size_t bytes) override {
    if (party_ < 0) return hipErrorNotSupported;
    if (bytes != key_bytes(B)) return hipErrorInvalidValue;
    TRY(hipStreamSynchronize(L_.stream));
    keyed_B_ = -1;
    TRY(ensure_arena(B));
    TRY(hipMemcpy(arena_[party_], key, bytes, hipMemcpyHostToDevice));
    keyed_B_ = B;
    return hipSuccess;
  }
  // This party's shares of x, A and the atom mask; prot: the protein embedding
  // (the party that owns it, party 1 in the reference's deployment) or null
  // (zeros: the other party's share of it).
  hipError_t set_party_inputs(int B, const void *x, const void *a, const void *m, const int64_t *prot) override {
    if (party_ < 0) return hipErrorNotSupported;
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N, nx = BN * d_.feat, na = BN * N;
    TRY(hipStreamSynchronize(L_.stream));
    DevBuf<T> &xb = party_ ? x1_ : x0_, &ab = party_ ? a1_ : a0_, &mb = party_ ? m1_ : m0_;
    TRY(xb.alloc(nx));
    TRY(ab.alloc(na));
    TRY(mb.alloc(BN));
    TRY(prot_.alloc(size_t(B) * d_.prot));
    TRY(hipMemcpy(xb.p, x, nx * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(ab.p, a, na * sizeof(T), hipMemcpyHostToDevice));
    TRY(hipMemcpy(mb.p, m, BN * sizeof(T), hipMemcpyHostToDevice));
    std::vector<T> pr(size_t(B) * d_.prot, T(0));
    if (prot)
      for (size_t i = 0; i < pr.size(); i++) pr[i] = T(uint64_t(prot[i]));
    TRY(hipMemcpy(prot_.p, pr.data(), pr.size() * sizeof(T), hipMemcpyHostToDevice));
    input_B_ = B;
    return hipSuccess;
  }

  // ---------------- inputs ----------------
  hipError_t set_inputs(int B, const void *x0, const void *x1, const void *a0, const void *a1, const void *m0,
                        const void *m1, const int64_t *prot) override {
    if (party_ >= 0) return hipErrorNotSupported;
    const int N = d_.n_nodes;
    const size_t BN = size_t(B) * N, nx = BN * d_.feat, na = BN * N;
    TRY(hipStreamSynchronize(L_.stream));  // earlier forwards read these buffers
    if (B != input_B_) drop_graph();       // buffers may move
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
  // ---------------- graph capture ----------------
  void set_alone(bool a) override {
    if (a != alone_) drop_graph();  // the captured forward's launches depend on it
    alone_ = a;
  }
  void drop_graph() {
    if (gexec_) (void)hipGraphExecDestroy(gexec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    gexec_ = nullptr;
    graph_ = nullptr;
    graph_B_ = -1;
  }

  // Resident keys: the forward's kernels are captured once per batch size and
  // the graph is replayed (the buffers it reads are fixed until keys, inputs of
  // another size or work buffers are reallocated, which drop it).  The host-side
  // exchange counters of the captured forward are replayed with it.
  hipError_t forward_graph(int B) {
    if (keyed_B_ != B || input_B_ != B) return hipErrorInvalidValue;
    TRY(ensure_work(B));  // may synchronize: outside the capture
    if (graph_B_ != B) {
      drop_graph();
      const Counters before = counters;
      counters = Counters();
      TRY(hipStreamBeginCapture(L_.stream, hipStreamCaptureModeThreadLocal));
      const hipError_t e = forward_body(B);
      hipGraph_t g = nullptr;
      const hipError_t e2 = hipStreamEndCapture(L_.stream, &g);
      if (e != hipSuccess || e2 != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        counters = before;
        return e != hipSuccess ? e : e2;
      }
      const hipError_t e3 = hipGraphInstantiate(&gexec_, g, nullptr, nullptr, 0);
      if (e3 != hipSuccess) {
        (void)hipGraphDestroy(g);
        gexec_ = nullptr;
        counters = before;
        return e3;
      }
      graph_ = g;
      graph_B_ = B;
      graph_ctr_ = counters;
      counters = before;
    }
    TRY(hipGraphLaunch(gexec_, L_.stream));
    counters.bytes += graph_ctr_.bytes;
    counters.rounds += graph_ctr_.rounds;
    return hipSuccess;
  }

  hipError_t forward(int B) override {
    if (party_ >= 0) return forward_body(B);  // host-driven exchanges: no graph
    if (!files_ && !streaming_ && !timer.on && L_.graph) return forward_graph(B);
    if (!files_) return forward_body(B);
    if (keyed_B_ != B || input_B_ != B) return hipErrorInvalidValue;
    {
      std::lock_guard<std::mutex> lk(mu_);
      loaded_ = -1;
      issued_ = -1;
      abort_ = false;
      io_err_ = hipSuccess;
    }
    const uint64_t set = set_;
    try {
      io_ = std::thread([this, set] { io_loop(set); });
    } catch (...) {
      return hipErrorOutOfMemory;
    }
    const hipError_t e = forward_body(B);
    stop_io();
    if (e == hipSuccess) set_ = (set_ + 1) % kf_[0].nsets;
    return e;
  }

  hipError_t forward_body(int B) {
    if (keyed_B_ != B || input_B_ != B) return hipErrorInvalidValue;
    TRY(ensure_work(B));
    // A lane of a few samples is latency-bound: its small gates spread over the
    // CUs, each truncation's two gates run in one launch and so does each
    // max-pool level.  Lanes of more keep the GPU busy between them, where a
    // spread gate's workgroups take LDS from the other lanes' gates; they pair
    // only the gates of at most kFuseSmallN elements, the latency-bound end of
    // a forward (all gates paired: B = 64 in 3 lanes 0.7% and 1.5% slower; B = 1
    // 4.7% and 3.4% lower latency; up to 65536 elements: B = 32 +1.6%, B = 64
    // and bw = 64 unchanged, against none).
    const bool few = B <= kFewLaneB;
    L_.spread_small = few;
    L_.quad_per_cu = alone_ ? std::max(quad_base_, L_.quad_alone) : quad_base_;
    const int N = d_.n_nodes, bw = bw_;
    const size_t BN = size_t(B) * N;
    if (!streaming_) {
      gates_ = plan(B);
      chunk_of_.assign(gates_.size(), 0);
    }
    gi_ = 0;
    cur_chunk_ = -1;
    stream_stats = StreamStats();
    if (streaming_) {
      TRY(issue_copy(0));
      if (chunks_.size() > 1) TRY(issue_copy(1));
    }
    Runner<T> r(L_, bw_, s_, ws_, counters, &timer, *this, peer_);
    const size_t small = few ? SIZE_MAX : kFuseSmallN;
    r.pair_max = !streaming_ && party_ < 0 ? small : 0;
    r.pool_max = small;
    r.pool_tail_on = few && !streaming_ && party_ < 0 && L_.pool_tail >= 0;
    auto pub_gemm = [&](const T *x, int l, size_t rows, T *y) -> hipError_t {
      int in, out;
      layer_io(l, &in, &out);
      GemmSpan span{&timer, L_.stream};
      TRY(span.begin(double(rows) * in * out));
      GemmArgs<T> g;
      g.M = int(rows);
      g.K = in;
      g.N = out;
      g.A1 = x;
      g.B1 = wt_[l].p;
      g.C = y;
      g.c_zero = l >= 3;  // y is the layer's range of fc_
      TRY(launch_gemm<T>(L_, g));
      return span.end();
    };
    auto fc = [&](int l) { return fc_.p + fc_off(B, l); };
    T *H = bA_.p, *Z = bB_.p, *XW = bC_.p;

    TRY(r.reveal(BN * d_.feat, x0_.p, x1_.p, 0, H));
    TRY(r.reveal(BN, m0_.p, m1_.p, 0, mh_.p));
    TRY(adj_.eval(r, a0_.p, a1_.p, Ah_.p, An_.p));
    for (int l = 0; l < 3; l++) {
      const int fo = d_.gcn[l];
      const size_t En = BN * fo;
      TRY(pub_gemm(H, l, BN, Z));
      if (xw_slack())
        TRY(r.tr(G_TRSLACK, En, Z, nullptr, 1, XW));
      else
        TRY(trunc_eval(r, false, En, Z, nullptr, 1, XW));
      TRY(r.sxs(B, N, N, fo, An_.p, XW, Z));
      if (agg_split()) {  // truncate with the bias, reveal, then ReLU of the small value
        TRY(r.tr(G_TRSLACK, En, Z, bias_[l].p, fo, XW));
        TRY(r.tr(G_RELUSLACK, En, XW, nullptr, 1, H));
      } else {
        TRY(trunc_eval(r, true, En, Z, bias_[l].p, fo, H));
      }
    }
    // masked max-pool: V = H + 2^(q-ms) m^ - 2^q (the sentinel -2^q on padding rows
    // for a mask of 0 or 2^ms, q = pool_sentinel_bit()), then a tree of
    // max(a,b) = a + ReLU(b-a)
    const int C = d_.gcn[2];
    const T S = T(1) << pool_sentinel_bit(), Sm = T(1) << (pool_sentinel_bit() - d_.mask_scale);
    TRY(launch_pool_prep<T>(L_, BN, C, H, mh_.p, Sm, T(0) - S, V0_.p));
    T *cur = V0_.p, *nxt = V1_.p;
    int pairs[32];
    const int Lv = pool_levels(N, pairs);
    int R = N;
    for (int l = 0; l < Lv; l++) {
      const int pr = pairs[l];
      if (r.pool_tail_on && l == L_.pool_tail && Lv - l >= 2) {  // the latency-bound levels: one launch
        TRY(r.pool_tail(pool_kind(), B, R, C, cur, Lv - l, pairs + l, nxt));
        std::swap(cur, nxt);
        R = 1;
        break;
      }
      TRY(r.pool_level(pool_kind(), B, R, C, cur, Z, XW, nxt));
      std::swap(cur, nxt);
      R = pr + (R & 1);
    }
    // drug FCs (one clearing launch for every fully connected product's output)
    TRY(launch_axpby<T>(L_, fc_off(B, 5 + d_.nfus), T(0), nullptr, T(0), nullptr, T(0), fc_.p));
    TRY(pub_gemm(cur, 3, B, fc(3)));
    TRY(trunc_eval(r, true, size_t(B) * d_.dfc[0], fc(3), bias_[3].p, d_.dfc[0], XW));
    TRY(pub_gemm(XW, 4, B, fc(4)));
    TRY(trunc_eval(r, false, size_t(B) * d_.dfc[1], fc(4), bias_[4].p, d_.dfc[1], XW));
    // concat [drug, protein]; the protein embedding owner reveals it (one message
    // each way: the other party's share is zero, revealPublicLeaf,
    // ddg_orca_base.h:84-89)
    counters.msg(size_t(B) * d_.prot, bw);
    const T *prot_pub = prot_.p;
    if (party_ >= 0) {
      const size_t np = size_t(B) * d_.prot;
      TRY(hipMemcpyAsync(ws_.m0.p, prot_.p, np * sizeof(T), hipMemcpyDeviceToDevice, L_.stream));
      TRY(r.exchange_reconstruct(np, Z));
      prot_pub = Z;
    }
    TRY(launch_concat<T>(L_, B, d_.dfc[1], d_.prot, XW, prot_pub, H));
    T *h = H, *h2 = XW;
    for (int k = 0; k < d_.nfus; k++) {
      T *z = fc(5 + k);
      TRY(pub_gemm(h, 5 + k, B, z));
      if (k < d_.nfus - 1) {
        TRY(trunc_eval(r, true, size_t(B) * d_.fus[k], z, bias_[5 + k].p, d_.fus[k], h2));
        std::swap(h, h2);
      } else {
        TRY(r.output(B, size_t(B) * d_.fus[k], z, hbias_[5 + k][0], out_.p));
      }
    }
    if (gi_ != gates_.size()) return hipErrorUnknown;
    if (streaming_)  // both slots are free once this forward's kernels have run
      for (int k = 0; k < 2; k++) TRY(hipEventRecord(free_[k], L_.stream));
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
  int quad_base_ = 64;  // L_.quad_per_cu as created (the lane beside others)
  bool alone_ = false;
  int party_ = -1;       // party mode: this process's party
  Peer *peer_ = nullptr;  // party mode: the channel to the other party
  std::vector<DevBuf<T>> wt_, bias_;
  std::vector<std::vector<int64_t>> hbias_;
  uint8_t *arena_[2] = {nullptr, nullptr};
  size_t arena_bytes_ = 0;
  int keyed_B_ = -1, input_B_ = -1, work_B_ = -1;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t gexec_ = nullptr;
  int graph_B_ = -1;
  Counters graph_ctr_;
  DevBuf<T> x0_, x1_, a0_, a1_, m0_, m1_, prot_;
  DevBuf<T> bA_, bB_, bC_, Ah_, An_, mh_, V0_, V1_, fc_;
  DevBuf<int64_t> out_;
  Workspace<T> ws_;
  AdjNorm<T> adj_;
  // gate plan and streaming state
  std::vector<GateKey> gates_;
  std::vector<std::pair<size_t, size_t>> chunks_;
  std::vector<int> chunk_of_;
  size_t gi_ = 0;
  int cur_chunk_ = -1;
  bool streaming_ = false;
  const uint8_t *host_[2] = {nullptr, nullptr};
  size_t chunk_max_ = 0;
  // file-backed keys: files, pinned staging buffers [party][k % 2], I/O thread
  bool files_ = false;
  KeyFile kf_[2];
  uint8_t *stg_[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
  uint64_t set_ = 0;
  std::thread io_;
  std::mutex mu_;
  std::condition_variable cv_;
  int loaded_ = -1, issued_ = -1;
  bool abort_ = false;
  hipError_t io_err_ = hipSuccess;
  std::vector<Run> runs_[2];       // what a chunk copy moves per party
  bool packed_[2] = {false, false};  // streamed party p's key is packed (seeded planes expanded)
  uint8_t spk_[2][16] = {};          // the streamed packed parties' PRF keys
  uint8_t pk_[2][16] = {};           // the resident keys' PRF keys (from keygen)
  bool have_pk_ = false;
  uint8_t *slot_[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
  hipEvent_t ready_[2] = {nullptr, nullptr}, free_[2] = {nullptr, nullptr};
  hipStream_t cs_ = nullptr;
};

template <typename T>
static ModelBase *make_model_t(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L,
                               std::string *err) {
  auto *mm = new Model<T>(bw, s, d, L);
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
  return mm;
}

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
  bool widths_ok = d.feat >= 1 && d.prot >= 0 && d.lut_nmax >= 0 && d.lut_nmax <= 255;
  for (int i = 0; i < 3; i++) widths_ok = widths_ok && d.gcn[i] >= 1;
  for (int i = 0; i < 2; i++) widths_ok = widths_ok && d.dfc[i] >= 1;
  for (int i = 0; i < d.nfus; i++) widths_ok = widths_ok && d.fus[i] >= 1;
  if (!widths_ok) {
    *err = "layer widths must be >= 1 (protein width >= 0, lut_nmax in [0, 255])";
    return nullptr;
  }
  if (d.slack < 0 || d.slack > 3) {
    *err = "slack must be 0, 1, 2 or 3";
    return nullptr;
  }
  if (d.mask_scale < 0 || d.mask_scale > bw - 2 - 1) {
    *err = "mask_scale must be in [0, bw - 3]";
    return nullptr;
  }
  if (bw == 32) return make_model_t<uint32_t>(bw, s, d, W, nW, L, err);
  if (bw == 64) return make_model_t<uint64_t>(bw, s, d, W, nW, L, err);
  *err = "bw must be 32 or 64";
  return nullptr;
}

// ===========================================================================
// lanes: concurrent sub-batches
// ===========================================================================
LaneSet::LaneSet(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L)
    : bw_(bw), s_(s), d_(d), W_(W, W + nW), L_(L) {}

LaneSet::~LaneSet() {
  for (size_t i = 0; i < lane_.size(); i++) {
    if (i > 0 && st_[i]) (void)hipStreamSynchronize(st_[i]);
    delete lane_[i];
  }
  close_files();
  for (size_t i = 1; i < st_.size(); i++)
    if (st_[i]) (void)hipStreamDestroy(st_[i]);
  for (auto e : done_)
    if (e) (void)hipEventDestroy(e);
}

hipError_t LaneSet::set_lanes(int n, std::string *e) {
  if (n < 1 || n > 16) {
    *e = "lanes must be in [1, 16]";
    return hipErrorInvalidValue;
  }
  if (L_.stream) TRY(hipStreamSynchronize(L_.stream));
  for (size_t i = 0; i < lane_.size(); i++) {
    if (i > 0) TRY(hipStreamSynchronize(st_[i]));
    delete lane_[i];
  }
  lane_.clear();
  close_files();
  for (size_t i = 1; i < st_.size(); i++) (void)hipStreamDestroy(st_[i]);
  st_.clear();
  for (auto ev : done_) (void)hipEventDestroy(ev);
  done_.clear();
  keyed_B_ = -1;
  for (int i = 0; i < n; i++) {
    Launch Li = L_;
    if (i > 0) TRY(hipStreamCreateWithFlags(&Li.stream, hipStreamNonBlocking));
    // concurrent lanes keep the GPU busy beside each other's gates: the
    // both-party form pays for longer gates there
    if (n > 1 && Li.both_aes > 0) {
      Li.both_aes = std::max(Li.both_aes, kBothAesLanes);
      Li.both_min = kBothMinLanes;
    }
    st_.push_back(Li.stream);
    hipEvent_t ev;
    TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    done_.push_back(ev);
    ModelBase *m = make_model(bw_, s_, d_, W_.data(), W_.size(), Li, e);
    if (!m) return hipErrorInvalidValue;
    lane_.push_back(m);
  }
  return hipSuccess;
}

int LaneSet::lane_B(int B, int i) const {
  const int n = lanes();
  return B / n + (i < B % n ? 1 : 0);
}
int LaneSet::active(int B) const { return std::min(lanes(), std::max(B, 0)); }

// fn(i, Bi, sample offset) for every lane with samples
template <class Fn>
hipError_t LaneSet::each(int B, Fn &&fn) {
  int off = 0;
  for (int i = 0; i < active(B); i++) {
    const int Bi = lane_B(B, i);
    TRY(fn(i, Bi, off));
    off += Bi;
  }
  return hipSuccess;
}

size_t LaneSet::key_bytes(int B) const {
  size_t n = 0;
  for (int i = 0; i < active(B); i++) n += lane_[i]->key_bytes(lane_B(B, i));
  return n;
}
size_t LaneSet::unique_key_bytes(int B, int party) const {
  size_t n = 0;
  for (int i = 0; i < active(B); i++) n += lane_[i]->unique_key_bytes(lane_B(B, i), party);
  return n;
}

hipError_t LaneSet::keygen(int B, uint64_t seed) {
  keyed_B_ = -1;
  TRY(each(B, [&](int i, int Bi, int) { return lane_[i]->keygen(Bi, lane_seed(seed, i)); }));
  keyed_B_ = B;
  return hipSuccess;
}

hipError_t LaneSet::import_keys(int B, const void *k0, const void *k1, size_t bytes) {
  if (bytes != key_bytes(B)) return hipErrorInvalidValue;
  keyed_B_ = -1;
  size_t o = 0;
  TRY(each(B, [&](int i, int Bi, int) {
    const size_t n = lane_[i]->key_bytes(Bi);
    hipError_t r = lane_[i]->import_keys(Bi, static_cast<const uint8_t *>(k0) + o,
                                         static_cast<const uint8_t *>(k1) + o, n);
    o += n;
    return r;
  }));
  keyed_B_ = B;
  return hipSuccess;
}

hipError_t LaneSet::export_keys(int party, void *dst, size_t bytes) {
  if (lanes() == 1) return lane_[0]->export_keys(party, dst, bytes);
  if (keyed_B_ < 1 || bytes != key_bytes(keyed_B_)) return hipErrorInvalidValue;
  size_t o = 0;
  return each(keyed_B_, [&](int i, int Bi, int) {
    const size_t n = lane_[i]->key_bytes(Bi);
    hipError_t r = lane_[i]->export_keys(party, static_cast<uint8_t *>(dst) + o, n);
    o += n;
    return r;
  });
}

hipError_t LaneSet::export_unique_keys(int party, void *dst, size_t bytes) {
  if (keyed_B_ < 1 || bytes != unique_key_bytes(keyed_B_, party)) return hipErrorInvalidValue;
  size_t o = 0;
  return each(keyed_B_, [&](int i, int Bi, int) {
    const size_t n = lane_[i]->unique_key_bytes(Bi, party);
    hipError_t r = lane_[i]->export_unique_keys(party, static_cast<uint8_t *>(dst) + o, n);
    o += n;
    return r;
  });
}

hipError_t LaneSet::release_arena() {
  for (auto *m : lane_) TRY(m->release_arena());
  return hipSuccess;
}

hipError_t LaneSet::attach_host_keys(int B, const void *h0, size_t bytes0, const void *h1, size_t bytes1,
                                     size_t slot_bytes) {
  // each party's buffer: the lanes' arenas back to back, or their packed keys
  bool packed[2];
  const size_t bytes[2] = {bytes0, bytes1};
  for (int p = 0; p < 2; p++) {
    if (bytes[p] == key_bytes(B))
      packed[p] = false;
    else if (bytes[p] == unique_key_bytes(B, p))
      packed[p] = true;
    else
      return hipErrorInvalidValue;
  }
  keyed_B_ = -1;
  size_t o0 = 0, o1 = 0;
  TRY(each(B, [&](int i, int Bi, int) {
    const size_t n0 = packed[0] ? lane_[i]->unique_key_bytes(Bi, 0) : lane_[i]->key_bytes(Bi);
    const size_t n1 = packed[1] ? lane_[i]->unique_key_bytes(Bi, 1) : lane_[i]->key_bytes(Bi);
    hipError_t r = lane_[i]->attach_host_keys(Bi, static_cast<const uint8_t *>(h0) + o0, n0,
                                              static_cast<const uint8_t *>(h1) + o1, n1, slot_bytes);
    o0 += n0;
    o1 += n1;
    return r;
  }));
  keyed_B_ = B;
  return hipSuccess;
}

void LaneSet::close_files() {
  for (int p = 0; p < 2; p++) {
    if (fd_[p] >= 0) ::close(fd_[p]);
    fd_[p] = -1;
  }
}

hipError_t LaneSet::attach_key_files(int B, const char *path0, const char *path1, size_t slot_bytes) {
  const size_t full = key_bytes(B);
  if (!path0 || !path1 || full == 0 || slot_bytes == 0) return hipErrorInvalidValue;
  int fd[2] = {::open(path0, O_RDONLY), ::open(path1, O_RDONLY)};
  auto fail = [&](hipError_t e) {
    for (int p = 0; p < 2; p++)
      if (fd[p] >= 0) ::close(fd[p]);
    return e;
  };
  if (fd[0] < 0 || fd[1] < 0) return fail(hipErrorFileNotFound);
  // each file holds whole key sets of one format: arenas or packed keys (the
  // lanes' back to back), told apart by the file size; both files the same count
  bool packed[2];
  uint64_t set[2], nsets = 0;
  for (int p = 0; p < 2; p++) {
    const off_t size = ::lseek(fd[p], 0, SEEK_END);
    const size_t pk = unique_key_bytes(B, p);
    if (size > 0 && uint64_t(size) % full == 0)
      packed[p] = false, set[p] = full;
    else if (size > 0 && uint64_t(size) % pk == 0)
      packed[p] = true, set[p] = pk;
    else
      return fail(hipErrorFileNotFound);
    const uint64_t n = uint64_t(size) / set[p];
    if (p == 1 && n != nsets) {  // a size that divides both ways: take the matching count
      if (!packed[1] && uint64_t(size) % pk == 0 && uint64_t(size) / pk == nsets)
        packed[1] = true, set[1] = pk;
      else
        return fail(hipErrorFileNotFound);
    }
    if (p == 0) nsets = n;
  }
  keyed_B_ = -1;
  uint64_t o[2] = {0, 0};
  hipError_t e = each(B, [&](int i, int Bi, int) {
    KeyFile f[2];
    for (int p = 0; p < 2; p++) {
      f[p].fd = fd[p];
      f[p].base = o[p];
      f[p].stride = set[p];
      f[p].nsets = nsets;
      o[p] += packed[p] ? lane_[i]->unique_key_bytes(Bi, p) : lane_[i]->key_bytes(Bi);
    }
    return lane_[i]->attach_key_files(Bi, f[0], f[1], packed[0], packed[1], slot_bytes);
  });
  if (e != hipSuccess) return fail(e);
  close_files();  // the lanes no longer read earlier files
  fd_[0] = fd[0];
  fd_[1] = fd[1];
  keyed_B_ = B;
  return hipSuccess;
}

hipError_t LaneSet::write_keys(int party, bool packed, const char *path, bool append) {
  if (!path || keyed_B_ < 1 || party < 0 || party > 1) return hipErrorInvalidValue;
  const int fd = ::open(path, O_WRONLY | O_CREAT | (append ? O_APPEND : O_TRUNC), 0644);
  if (fd < 0) return hipErrorFileNotFound;
  hipError_t e = each(keyed_B_, [&](int i, int, int) { return lane_[i]->write_keys(party, packed, fd); });
  if (::close(fd) != 0 && e == hipSuccess) e = hipErrorFileNotFound;
  return e;
}

hipError_t LaneSet::set_inputs(int B, const void *x0, const void *x1, const void *a0, const void *a1,
                               const void *m0, const void *m1, const int64_t *prot) {
  const size_t es = size_t(bw_ / 8), N = size_t(d_.n_nodes);
  const size_t px = N * d_.feat * es, pa = N * N * es, pm = N * es;  // bytes per sample
  auto at = [](const void *p, size_t o) { return static_cast<const uint8_t *>(p) + o; };
  return each(B, [&](int i, int Bi, int off) {
    const size_t o = size_t(off);
    return lane_[i]->set_inputs(Bi, at(x0, o * px), at(x1, o * px), at(a0, o * pa), at(a1, o * pa), at(m0, o * pm),
                                at(m1, o * pm), prot + o * d_.prot);
  });
}

hipError_t LaneSet::forward(int B) {
  const int n = active(B);
  counters = Counters();
  stream_stats = StreamStats();
  for (int i = 0; i < n; i++) {
    // Lanes past the first do not wait for the caller's stream: the forward
    // reads only the model's own buffers (written by synchronous uploads), so a
    // lane may start its next forward while the others finish this one; the
    // join below makes the caller's stream wait for every lane.  A profiled
    // forward runs lane i after lane i-1 so that launches do not overlap.
    if (i > 0 && serial_) TRY(hipStreamWaitEvent(st_[i], done_[i - 1], 0));
    lane_[i]->counters = Counters();
    lane_[i]->set_alone(n == 1);
    hipError_t r = lane_[i]->forward(lane_B(B, i));
    if (r != hipSuccess) {  // the caller's stream still waits for the lanes already enqueued
      for (int j = 1; j < i; j++) (void)hipStreamWaitEvent(st_[0], done_[j], 0);
      err = lane_[i]->err;
      return r;
    }
    if (n > 1) TRY(hipEventRecord(done_[i], st_[i]));
    counters.bytes += lane_[i]->counters.bytes;
    counters.rounds = std::max(counters.rounds, lane_[i]->counters.rounds);
    stream_stats.chunks += lane_[i]->stream_stats.chunks;
    stream_stats.bytes_h2d += lane_[i]->stream_stats.bytes_h2d;
  }
  for (int i = 1; i < n; i++) TRY(hipStreamWaitEvent(st_[0], done_[i], 0));
  return hipSuccess;
}

hipError_t LaneSet::set_party(int party, Peer *peer) {
  if (party >= 0 && lane_.size() != 1) {
    err = "party mode runs one lane";
    return hipErrorInvalidValue;
  }
  keyed_B_ = -1;
  close_files();
  return lane_[0]->set_party(party, peer);
}

hipError_t LaneSet::import_party_key(int B, const void *key, size_t bytes) {
  if (party() < 0) return hipErrorNotSupported;
  TRY(lane_[0]->import_party_key(B, key, bytes));
  keyed_B_ = B;
  return hipSuccess;
}

hipError_t LaneSet::set_party_inputs(int B, const void *x, const void *a, const void *m, const int64_t *prot) {
  if (party() < 0) return hipErrorNotSupported;
  return lane_[0]->set_party_inputs(B, x, a, m, prot);
}

hipError_t LaneSet::output(int64_t *h_out, int B) {
  return each(B, [&](int i, int Bi, int off) { return lane_[i]->output(h_out + off, Bi); });
}

void LaneSet::profile(bool on) {
  for (auto *m : lane_) {
    m->timer.reset();
    m->timer.on = on;
  }
  serial_ = on;
}

hipError_t LaneSet::profile_read(int *launches, double *ms, double *elements, double *aes, double *hbm_bytes) {
  double tot = 0, el = 0, ae = 0, by = 0;
  int nl = 0;
  for (size_t i = 0; i < lane_.size(); i++) {
    TRY(hipStreamSynchronize(st_[i]));
    const Phase1Timer &t = lane_[i]->timer;
    for (size_t k = 0; k + 1 < t.ev.size(); k += 2) {
      float f = 0;
      TRY(hipEventElapsedTime(&f, t.ev[k], t.ev[k + 1]));
      tot += f;
      el += 2.0 * double(t.elems[k / 2]);
      ae += 2.0 * double(t.elems[k / 2]) * double(t.levels[k / 2]);
      by += t.bytes[k / 2];
      nl++;
    }
  }
  if (launches) *launches = nl;
  if (ms) *ms = tot;
  if (elements) *elements = el;
  if (aes) *aes = ae;
  if (hbm_bytes) *hbm_bytes = by;
  return hipSuccess;
}

hipError_t LaneSet::profile_gemm(int *launches, double *ms, double *macs) {
  double tot = 0, mc = 0;
  int nl = 0;
  for (size_t i = 0; i < lane_.size(); i++) {
    TRY(hipStreamSynchronize(st_[i]));
    const Phase1Timer &t = lane_[i]->timer;
    for (size_t k = 0; k + 1 < t.gev.size(); k += 2) {
      float f = 0;
      TRY(hipEventElapsedTime(&f, t.gev[k], t.gev[k + 1]));
      tot += f;
      mc += t.gmacs[k / 2];
      nl++;
    }
  }
  if (launches) *launches = nl;
  if (ms) *ms = tot;
  if (macs) *macs = mc;
  return hipSuccess;
}

LaneSet *make_lane_set(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L,
                       std::string *err) {
  auto *ls = new LaneSet(bw, s, d, W, nW, L);
  if (ls->set_lanes(1, err) != hipSuccess) {
    if (err->empty()) *err = "model allocation failed";
    delete ls;
    return nullptr;
  }
  return ls;
}

// ===========================================================================
// standalone secure adjacency normalisation
// ===========================================================================
// With L lanes the B graphs are split into L groups of consecutive graphs (B/L
// each, the first B % L one larger, as the model's lanes); group i's key set is
// the one-lane key set of its graphs under the lane seed, the sets back to back.
namespace {
int adj_lanes(int B, int lanes) { return std::max(1, std::min(lanes, B)); }
int adj_lane_B(int B, int L, int i) { return B / L + (i < B % L ? 1 : 0); }
int adj_lane_off(int B, int L, int i) { return i * (B / L) + std::min(i, B % L); }
}  // namespace

size_t adjnorm_key_bytes(int bw, int s, int B, int N, int lanes) {
  const int L = adj_lanes(B, lanes);
  size_t o = 0;
  for (int i = 0; i < L; i++) o = AdjNorm<uint32_t>::layout_end(bw, s, adj_lane_B(B, L, i), N, o);
  return o;
}

template <typename T>
static hipError_t adjnorm_keygen_t(int bw, int s, int B, int N, uint64_t seed, int lanes, const Launch &L,
                                   void *out_mask, uint8_t *k0, uint8_t *k1) {
  const int nl = adj_lanes(B, lanes);
  size_t o = 0;
  for (int i = 0; i < nl; i++) {
    const int Bi = adj_lane_B(B, nl, i);
    AdjNorm<T> adj;
    TRY(adj.prepare(Bi, N, s, 0));
    DevBuf<T> rA;
    TRY(rA.alloc(size_t(Bi) * N * N));
    Dealer<T> d{L, bw, s, LaneSet::lane_seed(seed, i), k0 + o, k1 + o, Cursor{}};
    TRY(adj.keygen(d, rA.p, static_cast<T *>(out_mask) + size_t(adj_lane_off(B, nl, i)) * N * N));
    TRY(hipStreamSynchronize(L.stream));  // rA and the lane's scratch are freed below
    o = AdjNorm<T>::layout_end(bw, s, Bi, N, o);
  }
  return hipSuccess;
}

hipError_t adjnorm_keygen(int bw, int s, int B, int N, uint64_t seed, int lanes, const Launch &L, void *out_mask,
                          uint8_t *k0, uint8_t *k1) {
  return bw == 32 ? adjnorm_keygen_t<uint32_t>(bw, s, B, N, seed, lanes, L, out_mask, k0, k1)
                  : adjnorm_keygen_t<uint64_t>(bw, s, B, N, seed, lanes, L, out_mask, k0, k1);
}

struct AdjNormCache {
  int bw = 0;
  virtual ~AdjNormCache() = default;
};

void adjnorm_cache_free(AdjNormCache *cache) { delete cache; }

namespace {
// per lane: the prepared block (index maps, table, scratch), its workspace and,
// past lane 0, its own stream and the events that join it to the caller's stream
template <typename T>
struct AdjLane {
  AdjNorm<T> adj;
  DevBuf<T> Ah;
  Workspace<T> ws;
  hipStream_t st = nullptr;
  hipEvent_t pre = nullptr, done = nullptr;
  ~AdjLane() {
    if (st) {
      (void)hipStreamSynchronize(st);
      (void)hipStreamDestroy(st);
    }
    if (pre) (void)hipEventDestroy(pre);
    if (done) (void)hipEventDestroy(done);
  }
};
template <typename T>
struct AdjNormCacheT final : AdjNormCache {
  std::vector<std::unique_ptr<AdjLane<T>>> lanes;
};
}  // namespace

template <typename T>
static hipError_t adjnorm_eval_t(int bw, int s, int B, int N, int nmax, int lanes, const Launch &L,
                                 const uint8_t *k0, const uint8_t *k1, const void *a0, const void *a1, void *out,
                                 Counters *ctr, AdjNormCache **cache) {
  if (*cache && (*cache)->bw != bw) {
    TRY(hipStreamSynchronize(L.stream));
    delete *cache;
    *cache = nullptr;
  }
  if (!*cache) {
    auto *c = new AdjNormCacheT<T>();
    c->bw = bw;
    *cache = c;
  }
  auto *st = static_cast<AdjNormCacheT<T> *>(*cache);
  const int nl = adj_lanes(B, lanes);
  while (int(st->lanes.size()) < nl) {
    auto ln = std::make_unique<AdjLane<T>>();
    TRY(hipEventCreateWithFlags(&ln->pre, hipEventDisableTiming));
    if (!st->lanes.empty()) {  // lane 0 runs on the caller's stream
      TRY(hipStreamCreateWithFlags(&ln->st, hipStreamNonBlocking));
      TRY(hipEventCreateWithFlags(&ln->done, hipEventDisableTiming));
    }
    st->lanes.push_back(std::move(ln));
  }
  Counters local;
  Counters &cnt = ctr ? *ctr : local;
  const size_t es = sizeof(T), NN = size_t(N) * N;
  size_t o = 0;
  for (int i = 0; i < nl; i++) {
    AdjLane<T> &ln = *st->lanes[size_t(i)];
    const int Bi = adj_lane_B(B, nl, i);
    const size_t g0 = size_t(adj_lane_off(B, nl, i));
    Launch Li = L;
    if (i > 0) {
      // Group i starts once group i-1 has enqueued its memory-bound gates before
      // the truncation (which also orders it after the caller's stream): its
      // reveals and products then run beside group i-1's DCF work instead of
      // in step with them.
      Li.stream = ln.st;
      TRY(hipStreamWaitEvent(ln.st, st->lanes[size_t(i - 1)]->pre, 0));
    }
    TRY(ln.adj.prepare(Bi, N, s, nmax));
    const size_t BNN = size_t(Bi) * NN;
    TRY(ln.Ah.alloc(BNN));
    TRY(ln.ws.ensure(std::max(BNN, size_t(Bi) * pairs_of(N))));
    ArenaSource src;
    src.k[0] = k0 + o;
    src.k[1] = k1 + o;
    src.bytes = AdjNorm<T>::layout_end(bw, s, Bi, N, 0);
    Runner<T> r(Li, bw, s, ln.ws, cnt, nullptr, src);
    auto at = [&](const void *p) { return reinterpret_cast<const T *>(static_cast<const uint8_t *>(p) + g0 * NN * es); };
    TRY(ln.adj.eval(r, at(a0), at(a1), ln.Ah.p,
                    reinterpret_cast<T *>(static_cast<uint8_t *>(out) + g0 * NN * es), nl > 1 ? ln.pre : nullptr));
    if (i > 0) TRY(hipEventRecord(ln.done, ln.st));
    o = AdjNorm<T>::layout_end(bw, s, Bi, N, o);
  }
  for (int i = 1; i < nl; i++) TRY(hipStreamWaitEvent(L.stream, st->lanes[size_t(i)]->done, 0));
  return hipStreamSynchronize(L.stream);
}

hipError_t adjnorm_eval(int bw, int s, int B, int N, int nmax, int lanes, const Launch &L, const uint8_t *k0,
                        const uint8_t *k1, const void *a0, const void *a1, void *out, Counters *ctr,
                        AdjNormCache **cache) {
  return bw == 32 ? adjnorm_eval_t<uint32_t>(bw, s, B, N, nmax, lanes, L, k0, k1, a0, a1, out, ctr, cache)
                  : adjnorm_eval_t<uint64_t>(bw, s, B, N, nmax, lanes, L, k0, k1, a0, a1, out, ctr, cache);
}

// ---------------------------------------------------------------------------
// standalone gates in party mode (one party per process or thread)
// ---------------------------------------------------------------------------
struct PartyWork {
  Workspace<uint32_t> w32;
  Workspace<uint64_t> w64;
  DevBuf<uint32_t> v32;  // the LUT's revealed intermediate
  DevBuf<uint64_t> v64;
};
void party_work_free(PartyWork *w) { delete w; }

namespace {
template <typename T>
Workspace<T> &party_ws(PartyWork &w);
template <>
Workspace<uint32_t> &party_ws<uint32_t>(PartyWork &w) {
  return w.w32;
}
template <>
Workspace<uint64_t> &party_ws<uint64_t>(PartyWork &w) {
  return w.w64;
}
template <typename T>
DevBuf<T> &party_tmp(PartyWork &w);
template <>
DevBuf<uint32_t> &party_tmp<uint32_t>(PartyWork &w) {
  return w.v32;
}
template <>
DevBuf<uint64_t> &party_tmp<uint64_t>(PartyWork &w) {
  return w.v64;
}

// One gate of party L.party over its key (laid out from offset 0), messages of
// nmsg elements; synchronises the stream at the end unless L.party_sync is 0
// (the output is then ready in the stream's order).
template <typename T, class Fn>
hipError_t party_gate(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, const uint8_t *key,
                      size_t key_bytes, size_t nmsg, Fn &&fn) {
  if (L.party < 0 || L.party > 1 || !peer) return hipErrorInvalidValue;
  if (!*w) *w = new PartyWork();
  Workspace<T> &ws = party_ws<T>(**w);
  TRY(ws.ensure(nmsg));
  ArenaSource src;
  src.k[0] = src.k[1] = key;
  src.bytes = key_bytes;
  Runner<T> r(L, bw, s, ws, *ctr, nullptr, src, peer);
  TRY(fn(r, **w));
  return L.party_sync ? hipStreamSynchronize(L.stream) : hipSuccess;
}
template <typename T>
const T *cp(const void *p) {
  return static_cast<const T *>(p);
}
template <typename T>
T *mp(void *p) {
  return static_cast<T *>(p);
}
}  // namespace

#define PARTY_DISPATCH(bw, CALL) ((bw) == 32 ? CALL(uint32_t) : CALL(uint64_t))

hipError_t party_tr_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, int kind,
                         size_t n, const uint8_t *key, const void *x, const void *bias, int ncol, void *y) {
  const size_t kb = tr_layout(kind, bw, s, n, 0).end;
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, key, kb, n, [&](Runner<T> &r, PartyWork &) {                  \
    return r.tr(kind, n, cp<T>(x), cp<T>(bias), ncol, mp<T>(y));                                        \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}

hipError_t party_mul_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t nx,
                          size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib, const uint8_t *key,
                          const void *x, const void *y, void *z) {
  const size_t kb = mul_layout(bw, nx, ny, nz, 0).end;
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, key, kb, nz, [&](Runner<T> &r, PartyWork &) {                 \
    return r.mul(nx, ny, nz, MulMap::explicit_maps(ia, ib), cp<T>(x), cp<T>(y), mp<T>(z));              \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}

hipError_t party_lut8_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                           const uint8_t *key, const void *table, const void *x, void *y) {
  const size_t kb = lut8_layout(bw, n, 0).end;
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, key, kb, n, [&](Runner<T> &r, PartyWork &pw) -> hipError_t {  \
    DevBuf<T> &vh = party_tmp<T>(pw);                                                                   \
    TRY(vh.alloc(n));                                                                                   \
    return r.lut8(n, cp<T>(table), cp<T>(x), vh.p, mp<T>(y));                                           \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}

hipError_t party_sxs_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, int nb, int M,
                          int K, int N, const uint8_t *key, const void *a, const void *b, void *c) {
  const size_t kb = sxs_layout(bw, nb, M, K, N, 0).end;
  const size_t nc = size_t(nb) * M * N;
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, key, kb, nc, [&](Runner<T> &r, PartyWork &) {                 \
    return r.sxs(nb, M, K, N, cp<T>(a), cp<T>(b), mp<T>(c));                                            \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}

hipError_t party_reveal_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                             const uint8_t *key, const void *v, void *vhat) {
  const size_t kb = reveal_layout(bw, n, 0).end;
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, key, kb, n, [&](Runner<T> &r, PartyWork &) {                  \
    return r.reveal(n, cp<T>(v), cp<T>(v), 0, mp<T>(vhat));                                             \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}

hipError_t party_reconstruct(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                             void *d) {
#define CALL(T)                                                                                       \
  party_gate<T>(w, L, peer, ctr, bw, s, nullptr, 0, n, [&](Runner<T> &r, PartyWork &) -> hipError_t {  \
    TRY(hipMemcpyAsync(r.ws.m0.p, d, n * sizeof(T), hipMemcpyDeviceToDevice, L.stream));               \
    ctr->msg(n, bw);                                                                                    \
    return r.exchange_reconstruct(n, mp<T>(d));                                                         \
  })
  return PARTY_DISPATCH(bw, CALL);
#undef CALL
}
#undef PARTY_DISPATCH

}  // namespace mpcx
