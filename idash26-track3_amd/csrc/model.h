// model.h -- the DeepDTAGen affinity branch as a sequence of two-party gates
// (dealer keygen and online forward), both parties on one GPU.
//
// Mirrors DeepDTAGenAffinity<T>::_forward (gpu_mpc/deepdtagen.h:183-222) with
// the op order of reference/fixed_forward.py:63-95:
//   reveal X and the atom mask
//   secure adjacency normalisation (secure_adj_norm.h:393-659)
//   3 x GCN:  Z = H.W^T (public weights, no exchange) -> TR -> A_norm.(XW) (SxS)
//             -> TRRELU(+bias)
//   masked max-pool tree (masked_maxpool_layer.h:47-165), sentinel form
//   drug FC (TRRELU), drug FC (TR), concat [drug, protein] (deepdtagen.h:45-101)
//   fusion FCs (TRRELU ...), output layer unmasked with the clear output mask
//   (ddg_orca_base.h:296-302) and truncated locally.
//
// Keys are read either from a resident arena in HBM (initGPUKeyArena,
// patches/EzPC-GPU-MPC.track3.patch:632-661) or streamed from pinned host
// memory through two device slots on a copy stream (the chunked pipeline of
// gpu_mpc/deepdtagen_inference.cu:608-859).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "gemm.h"
#include "kernels.h"
#include "mpcx_core.h"

namespace mpcx {

class Peer;

struct ModelDims {
  int n_nodes = 140, feat = 78;
  int gcn[3] = {78, 156, 312};
  int dfc[2] = {1024, 128};
  int prot = 128;
  int nfus = 3;
  int fus[4] = {1024, 512, 1, 0};
  int lut_nmax = 138;
  int mask_scale = 0;  // atom mask values are 0 or 2^mask_scale
  int slack = 0;  // 0 exact; 1 H.W^T truncated with TRSLACK; 2 also A.XW + b: TRSLACK + RELUSLACK
};

struct Counters {
  uint64_t bytes = 0;   // bytes exchanged, both directions
  uint64_t rounds = 0;  // exchange rounds
  void msg(size_t n_elems, int bw) {
    bytes += 2ull * n_elems * uint64_t(bw / 8);
    rounds++;
  }
  // a message known modulo 2^m, m < bw: packed at m bits into 64-bit words
  void msg_bits(size_t n_elems, int m, int bw) {
    if (m >= bw) return msg(n_elems, bw);
    bytes += 2ull * 8ull * packed_words(n_elems, m);
    rounds++;
  }
  void bitplanes(size_t n, int planes) {
    bytes += 2ull * uint64_t(planes) * (((n + 31) / 32) * 4);
    rounds++;
  }
};

// Per-kernel timing of the DCF gate launches (k_tr_eval), HIP events on the
// launch stream.
struct Phase1Timer {
  bool on = false;
  std::vector<hipEvent_t> ev;  // start/stop pairs
  std::vector<size_t> elems;   // elements per launch
  std::vector<int> levels;     // AES calls per element per party
  std::vector<double> bytes;   // algorithmic HBM bytes per launch (both parties)
  // ring GEMMs: start/stop pairs around each GEMM (an SxS gate's three Beaver
  // products as one pair) and the ring multiply-adds inside
  std::vector<hipEvent_t> gev;
  std::vector<double> gmacs;
  void reset();
};

// Streaming statistics of the last forward (host-key mode).
struct StreamStats {
  int chunks = 0;
  uint64_t bytes_h2d = 0;  // key bytes copied host -> device, both parties
};

// A stream of key sets in a file: set k of this lane's keys starts at
// base + k * stride (stride = bytes of a whole batch's set, all lanes).
struct KeyFile {
  int fd = -1;
  uint64_t base = 0, stride = 0, nsets = 0;
};

class ModelBase {
 public:
  virtual ~ModelBase() = default;
  virtual size_t key_bytes(int B) const = 0;
  virtual hipError_t keygen(int B, uint64_t seed) = 0;
  virtual hipError_t import_keys(int B, const void *k0, const void *k1, size_t bytes) = 0;
  virtual hipError_t export_keys(int party, void *dst, size_t bytes) = 0;
  virtual hipError_t release_arena() = 0;
  // Bytes of party p's packed key: a 256-byte header holding the party's own PRF
  // key, then its planes in arena order without those the party reads from
  // party 0's copy (party 1: the shared DCF planes) and without those the dealer
  // drew from the party's PRF key (expanded again on the device).
  virtual size_t unique_key_bytes(int B, int party) const = 0;
  // Party p's packed key (keys from keygen only: imported keys carry no PRF key).
  virtual hipError_t export_unique_keys(int party, void *dst, size_t bytes) = 0;
  // Host-key (streaming) mode: keys of a batch of B in host memory (pinned for
  // asynchronous copies), copied per chunk of consecutive gates into one of two
  // device slots of slot_bytes per party while the previous chunk computes.
  // Each party: its arena (bytes = key_bytes) or its packed key (unique_key_bytes).
  virtual hipError_t attach_host_keys(int B, const void *h_k0, size_t bytes0, const void *h_k1, size_t bytes1,
                                      size_t slot_bytes) = 0;
  // File-backed keys: each forward reads the next key set (cycling) chunk by
  // chunk through pinned staging buffers filled by an I/O thread.
  virtual hipError_t attach_key_files(int B, const KeyFile &f0, const KeyFile &f1, bool packed0, bool packed1,
                                      size_t slot_bytes) = 0;
  // Appends the resident key set of one party (arena or packed key) to fd.
  virtual hipError_t write_keys(int party, bool packed, int fd) = 0;
  virtual hipError_t set_inputs(int B, const void *x0, const void *x1, const void *a0, const void *a1,
                                const void *m0, const void *m1, const int64_t *prot) = 0;
  // The lane runs alone (no other lane's forward beside it): its mid-size gates
  // may take the quad-lane form (Launch::quad_alone) without keeping another
  // lane's workgroups off the CUs.
  virtual void set_alone(bool) {}
  virtual hipError_t forward(int B) = 0;
  virtual hipError_t output(int64_t *h_out, int B) = 0;
  virtual uint8_t *arena(int party) = 0;
  // Party mode (one party per process or thread; party -1: both parties here).
  virtual hipError_t set_party(int party, Peer *peer) = 0;
  virtual int party() const = 0;
  virtual hipError_t import_party_key(int B, const void *key, size_t bytes) = 0;
  virtual hipError_t set_party_inputs(int B, const void *x, const void *a, const void *m, const int64_t *prot) = 0;
  Counters counters;
  Phase1Timer timer;
  StreamStats stream_stats;
  std::string err;
};

ModelBase *make_model(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L,
                      std::string *err);

// The model as the library exposes it: a batch of B split into `lanes`
// sub-batches of consecutive samples (B/lanes, the first B%lanes one larger),
// each a complete ModelBase on its own stream.  Lane 0 runs on the caller's
// stream, which waits for the other lanes at the end of every forward; the
// gates of one lane that leave the GPU partly idle (small latency-bound DCF
// launches, GEMMs, the memory-bound exchange kernels) overlap another lane's
// DCF evaluation.
// The keys of a batch are the lanes' key sets back to back; lane i's key set is
// the one-lane key set of its samples under the seed lane_seed(seed, i).
class LaneSet {
 public:
  LaneSet(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L);
  ~LaneSet();
  hipError_t set_lanes(int n, std::string *err);  // drops keys and inputs
  int lanes() const { return int(lane_.size()); }
  static uint64_t lane_seed(uint64_t seed, int i) { return seed + uint64_t(i) * 0x9E3779B97F4A7C15ull; }

  size_t key_bytes(int B) const;
  size_t unique_key_bytes(int B, int party) const;
  hipError_t keygen(int B, uint64_t seed);
  hipError_t import_keys(int B, const void *k0, const void *k1, size_t bytes);
  hipError_t export_keys(int party, void *dst, size_t bytes);
  hipError_t export_unique_keys(int party, void *dst, size_t bytes);
  hipError_t release_arena();
  hipError_t attach_host_keys(int B, const void *h_k0, size_t bytes0, const void *h_k1, size_t bytes1,
                              size_t slot_bytes);
  // Key files of whole-batch key sets back to back (per party: key_bytes(B) or
  // unique_key_bytes(B, p) per set).  Returns
  // hipErrorFileNotFound for files that cannot be opened or do not hold whole sets.
  hipError_t attach_key_files(int B, const char *path0, const char *path1, size_t slot_bytes);
  hipError_t write_keys(int party, bool packed, const char *path, bool append);
  hipError_t set_inputs(int B, const void *x0, const void *x1, const void *a0, const void *a1, const void *m0,
                        const void *m1, const int64_t *prot);
  hipError_t forward(int B);
  hipError_t output(int64_t *h_out, int B);
  // Party mode: one lane only.
  hipError_t set_party(int party, Peer *peer);
  int party() const { return lane_.empty() ? -1 : lane_[0]->party(); }
  hipError_t import_party_key(int B, const void *key, size_t bytes);
  hipError_t set_party_inputs(int B, const void *x, const void *a, const void *m, const int64_t *prot);
  // Per-launch timing of the DCF-evaluation kernels.  A profiled forward runs
  // the lanes one after another, so every launch is timed alone.
  void profile(bool on);
  hipError_t profile_read(int *launches, double *ms, double *elements, double *aes, double *hbm_bytes);
  hipError_t profile_gemm(int *launches, double *ms, double *macs);

  Counters counters;         // last forward: bytes summed over lanes, rounds of one lane
  StreamStats stream_stats;  // last forward, summed over lanes
  std::string err;

 private:
  // samples of lane i for a batch of B (0 for lanes beyond B)
  int lane_B(int B, int i) const;
  int active(int B) const;
  template <class Fn>
  hipError_t each(int B, Fn &&fn);

  int bw_, s_;
  ModelDims d_;
  std::vector<int64_t> W_;
  Launch L_;
  std::vector<ModelBase *> lane_;
  std::vector<hipStream_t> st_;  // st_[i]: lane i's stream (st_[0] = the caller's)
  std::vector<hipEvent_t> done_;
  bool serial_ = false;
  int keyed_B_ = -1;
  int fd_[2] = {-1, -1};  // attached key files
  void close_files();
};

LaneSet *make_lane_set(int bw, int s, const ModelDims &d, const int64_t *W, size_t nW, const Launch &L,
                       std::string *err);

// ---------------- standalone secure adjacency normalisation ----------------
// ddgSecureAdjNormKeygen / ddgSecureAdjNormEval (gpu_mpc/secure_adj_norm.h:203-374,
// 393-659): A (B x N x N, 0/1 with self loops) as additive shares -> masked
// A_norm = A (.) floor(T[d_i] T[d_j] / 2^s) + out_mask.
size_t adjnorm_key_bytes(int bw, int s, int B, int N, int lanes);
hipError_t adjnorm_keygen(int bw, int s, int B, int N, uint64_t seed, int lanes, const Launch &L, void *out_mask,
                          uint8_t *k0, uint8_t *k1);
// *cache keeps, per lane, the index maps, D^-1/2 table, scratch and stream of
// the last (bw, B, N, nmax) between calls (created on first use; free with
// adjnorm_cache_free).
struct AdjNormCache;
void adjnorm_cache_free(AdjNormCache *cache);
hipError_t adjnorm_eval(int bw, int s, int B, int N, int nmax, int lanes, const Launch &L, const uint8_t *k0,
                        const uint8_t *k1, const void *a0, const void *a1, void *out_masked, Counters *ctr,
                        AdjNormCache **cache);

// ---------------- standalone gates in party mode ----------------
// One party's evaluation of one gate (L.party = 0 or 1) with the exchanges
// through `peer`: the party's key of the gate (laid out from offset 0), its
// share or the masked public input, the reconstructed masked output (the same
// on both parties).  *w keeps the device workspace between calls (created on
// first use; free with party_work_free).  Each call synchronises L.stream.
struct PartyWork;
void party_work_free(PartyWork *w);
hipError_t party_tr_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, int kind,
                         size_t n, const uint8_t *key, const void *x, const void *bias, int ncol, void *y);
hipError_t party_mul_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t nx,
                          size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib, const uint8_t *key,
                          const void *x, const void *y, void *z);
hipError_t party_lut8_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                           const uint8_t *key, const void *table, const void *x, void *y);
hipError_t party_sxs_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, int nb, int M,
                          int K, int N, const uint8_t *key, const void *a, const void *b, void *c);
// v: this party's additive share; vhat = v0 + v1 + mask
hipError_t party_reveal_eval(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                             const uint8_t *key, const void *v, void *vhat);
// d: this party's additive share in, the sum of both parties' shares out
hipError_t party_reconstruct(PartyWork **w, const Launch &L, Peer *peer, Counters *ctr, int bw, int s, size_t n,
                             void *d);

}  // namespace mpcx
