// mpcx_infer -- command-line driver of the secure affinity forward over the
// libmpcx C ABI (include/mpcx.h), in the role of the reference's
// gpu_mpc/deepdtagen_inference.cu (main, :183-607): it reads the reference's
// weights.bin (+ .json manifest) and batch directory (x/adj/mask share files,
// protein_emb.dat, batch_manifest.json), runs the dealer and/or the online
// two-party forward, and prints the affinities in the reference's format.
//
//   mpcx_infer <bw> <scale> <role> <keyDir> <shareDir> [batch] [reps]
//     role 0  dealer: GPU keygen, writes <keyDir>/DeepDTAGen_<bw>_<scale>_party{0,1}
//     role 1  evaluator: reads those key files and the shares of <shareDir>,
//             runs the online forward (both parties in this process)
//     role 2  dealer and evaluator in one run (keys stay resident in HBM)
//     role 3  one party's evaluator (the reference's deployment: two such
//             processes, gpu_mpc/run_local_2pc.sh:196-233): reads its own key
//             file and share files, exchanges with the other party's process over
//             the Unix socket MPCX_PEER (party 0 listens, party 1 connects);
//             party MPCX_PARTY (0 or 1); party 1 reads protein_emb.dat
//   environment: MPCX_WEIGHTS_BIN (default ./weights.bin), MPCX_DEALER_KEY (a
//   file of the dealer's 16 secret key bytes: roles 0 and 2 derive every key
//   set from them; without it the keys rest on the seed alone, which is said on
//   stderr), MPCX_SEED (dealer seed, names the key set, default 12345),
//   MPCX_LANES (concurrent sub-batches, default 1),
//   MPCX_LUT_NMAX (largest degree with a D^-1/2 table entry, default 138),
//   MPCX_SLACK (slack truncations of the GCN, 0 / 1 / 2, default 0: exact).
//
// Differences from the reference driver: roles 1 and 2 evaluate both parties in
// one process (no peer address), and "Comm (B)" is the bytes both parties
// exchange per forward (both directions), as it is for role 3, which also prints
// the bytes that crossed its socket ("Peer (B)"); the dealer's keys are this
// library's format.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <regex>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/mpcx.h"

namespace {

[[noreturn]] void die(const std::string &msg) {
  std::fprintf(stderr, "mpcx_infer: %s\n", msg.c_str());
  std::exit(1);
}

std::string read_text(const std::string &path) {
  std::ifstream f(path);
  if (!f) die("cannot open " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

template <typename T>
std::vector<T> read_array(const std::string &path, size_t count) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) die("cannot open " + path);
  const std::streamoff size = f.tellg();
  if (size < 0 || size_t(size) != count * sizeof(T))
    die(path + ": " + std::to_string(size) + " bytes, expected " + std::to_string(count * sizeof(T)));
  std::vector<T> v(count);
  f.seekg(0);
  if (!f.read(reinterpret_cast<char *>(v.data()), std::streamsize(count * sizeof(T)))) die("cannot read " + path);
  return v;
}

std::vector<uint8_t> read_bytes(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) die("cannot open " + path);
  return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

// The dealer's secret key: 16 bytes from the file MPCX_DEALER_KEY, if set.
bool dealer_key(uint8_t key[16]) {
  const char *p = std::getenv("MPCX_DEALER_KEY");
  if (!p || !*p) return false;
  const std::vector<uint8_t> k = read_bytes(p);
  if (k.size() != 16) die(std::string("MPCX_DEALER_KEY (") + p + ") must hold exactly 16 bytes");
  std::memcpy(key, k.data(), 16);
  return true;
}

// "key": integer, from a flat manifest
long json_int(const std::string &js, const std::string &key) {
  std::smatch m;
  if (!std::regex_search(js, m, std::regex("\"" + key + "\"\\s*:\\s*(-?[0-9]+)"))) die("manifest has no " + key);
  return std::stol(m[1].str());
}
bool json_bool(const std::string &js, const std::string &key, bool dflt) {
  std::smatch m;
  if (!std::regex_search(js, m, std::regex("\"" + key + "\"\\s*:\\s*(true|false)"))) return dflt;
  return m[1].str() == "true";
}
std::vector<long> json_pair(const std::string &js, const std::string &key) {
  std::smatch m;
  if (!std::regex_search(js, m, std::regex("\"" + key + "\"\\s*:\\s*\\[\\s*([0-9]+)\\s*,\\s*([0-9]+)\\s*\\]")))
    die("manifest has no " + key);
  return {std::stol(m[1].str()), std::stol(m[2].str())};
}
// every "W_shape": [in, out] in order (weights.bin.json, reference/export_weights.py:38-75)
std::vector<std::pair<long, long>> json_layers(const std::string &js) {
  std::vector<std::pair<long, long>> out;
  const std::regex re("\"W_shape\"\\s*:\\s*\\[\\s*([0-9]+)\\s*,\\s*([0-9]+)\\s*\\]");
  for (auto it = std::sregex_iterator(js.begin(), js.end(), re); it != std::sregex_iterator(); ++it)
    out.emplace_back(std::stol((*it)[1].str()), std::stol((*it)[2].str()));
  return out;
}

int env_int(const char *name, int dflt) {
  const char *v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

void check(mpcx_ctx *c, mpcx_status st, const char *what) {
  if (st != MPCX_OK) die(std::string(what) + ": " + mpcx_last_error(c));
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 6) {
    std::fprintf(stderr, "usage: %s <bw> <scale> <role 0|1|2> <keyDir> <shareDir> [batch] [reps]\n", argv[0]);
    return 2;
  }
  const int bw = std::atoi(argv[1]), scale = std::atoi(argv[2]), role = std::atoi(argv[3]);
  std::string keyDir = argv[4], shareDir = argv[5];
  if (!keyDir.empty() && keyDir.back() != '/') keyDir += '/';
  if (!shareDir.empty() && shareDir.back() != '/') shareDir += '/';
  const int reps = argc > 7 ? std::max(1, std::atoi(argv[7])) : 1;
  if ((bw != 32 && bw != 64) || role < 0 || role > 3) die("bw must be 32 or 64, role 0, 1, 2 or 3");
  const int party = env_int("MPCX_PARTY", -1);
  if (role == 3 && party != 0 && party != 1) die("role 3 needs MPCX_PARTY=0 or 1");

  // weights and the layer shapes of their manifest
  const char *wenv = std::getenv("MPCX_WEIGHTS_BIN");
  const std::string wpath = wenv && *wenv ? wenv : "./weights.bin";
  const auto layers = json_layers(read_text(wpath + ".json"));
  if (layers.size() < 7 || layers.size() > 9) die(wpath + ".json: expected 3 GCN, 2 drug FC and 2..4 fusion layers");
  size_t nW = 0;
  for (auto &l : layers) nW += size_t(l.first) * size_t(l.second) + size_t(l.second);
  const std::vector<int64_t> W = read_array<int64_t>(wpath, nW);

  // batch manifest (reference/scripts/dev_tools/prepare_batch_samples.py:154-177)
  const std::string man = read_text(shareDir + "batch_manifest.json");
  const int B = argc > 6 && std::atoi(argv[6]) > 0 ? std::atoi(argv[6]) : int(json_int(man, "batch_size"));
  if (json_int(man, "bw") != bw || json_int(man, "scale") != scale) die("batch manifest bw/scale differ from the arguments");
  if (!json_bool(man, "raw_adj", false)) die("only the raw-adjacency layout (adj at scale 0) is supported");
  const int N = int(json_int(man, "nmax")), feat = int(json_int(man, "feat_dim")), pool = int(json_int(man, "pool_dim"));
  const long prot = json_pair(man, "protein_emb")[1];

  mpcx_model_dims d{};
  d.n_nodes = N;
  d.feat = int(layers[0].first);
  for (int i = 0; i < 3; i++) d.gcn[i] = int(layers[size_t(i)].second);
  for (int i = 0; i < 2; i++) d.dfc[i] = int(layers[size_t(3 + i)].second);
  d.prot = int(layers[5].first) - d.dfc[1];
  d.nfus = int(layers.size()) - 5;
  for (int i = 0; i < d.nfus; i++) d.fus[i] = int(layers[size_t(5 + i)].second);
  d.lut_nmax = env_int("MPCX_LUT_NMAX", 138);
  d.mask_scale = scale;  // the mask files hold 2^s for a real atom (reference/share_data.py:135-159)
  d.slack = env_int("MPCX_SLACK", 0);
  if (d.feat != feat || d.prot != prot) die("weights and batch manifest disagree on feature or protein width");

  mpcx_ctx *ctx = nullptr;
  if (mpcx_create(bw, scale, 0, &ctx) != MPCX_OK) die("mpcx_create failed (no GPU?)");
  if (role == 0 || role == 2) {  // the dealer: its secret key, read by models created afterwards
    uint8_t dk[16];
    if (dealer_key(dk)) {
      check(ctx, mpcx_set_dealer_key(ctx, dk), "set_dealer_key");
      volatile uint8_t *v = dk;
      for (int i = 0; i < 16; i++) v[i] = 0;
    } else {
      std::fprintf(stderr,
                   "mpcx_infer: warning: no MPCX_DEALER_KEY: the key sets derive from the seed MPCX_SEED alone, "
                   "so anyone who knows the seed can regenerate every mask\n");
    }
  }
  mpcx_model *m = nullptr;
  check(ctx, mpcx_model_create(ctx, &d, W.data(), W.size(), &m), "model_create");
  check(ctx, mpcx_model_set_lanes(m, env_int("MPCX_LANES", 1)), "model_set_lanes");
  const std::string expName = "DeepDTAGen_" + std::to_string(bw) + "_" + std::to_string(scale);
  const std::string kf[2] = {keyDir + expName + "_party0", keyDir + expName + "_party1"};
  const size_t kbytes = mpcx_model_key_bytes(m, B);

  if (role == 0 || role == 2) {
    const auto t0 = std::chrono::steady_clock::now();
    check(ctx, mpcx_model_keygen(m, B, uint64_t(env_int("MPCX_SEED", 12345))), "model_keygen");
    if (role == 0)
      for (int p = 0; p < 2; p++) check(ctx, mpcx_model_write_keys(m, p, 0, kf[p].c_str(), 0), "model_write_keys");
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    std::printf("Dealer: %zu key bytes per party for B=%d in %.1f ms\n", kbytes, B, ms);
  }
  if (role == 1) {
    const std::vector<uint8_t> k0 = read_bytes(kf[0]), k1 = read_bytes(kf[1]);
    if (k0.size() != kbytes || k1.size() != kbytes) die("key files do not hold one key set of this batch");
    check(ctx, mpcx_model_import_keys(m, B, k0.data(), k1.data(), kbytes), "model_import_keys");
  }
  mpcx_peer *peer = nullptr;
  if (role == 3) {
    const char *penv = std::getenv("MPCX_PEER");
    const std::string path = penv && *penv ? penv : "/tmp/mpcx_" + std::to_string(bw) + ".sock";
    if (mpcx_peer_connect(party, path.c_str(), 60000, &peer) != MPCX_OK) die("no connection to the other party");
    check(ctx, mpcx_model_set_party(m, peer), "model_set_party");
    const std::vector<uint8_t> k = read_bytes(kf[party]);
    if (k.size() != kbytes) die("key file does not hold one key set of this batch");
    check(ctx, mpcx_model_import_party_key(m, B, k.data(), kbytes), "model_import_party_key");
  }
  if (role >= 1) {
    // share files (read by the reference at deepdtagen_inference.cu:426-432)
    const size_t es = size_t(bw / 8), BN = size_t(B) * size_t(N);
    std::vector<uint8_t> x[2], a[2], mk[2];
    for (int p = 0; p < 2; p++) {
      if (role == 3 && p != party) continue;  // the other party's shares stay with it
      const std::string sfx = "_share" + std::to_string(p) + ".dat";
      x[p] = read_array<uint8_t>(shareDir + "x" + sfx, BN * size_t(feat) * es);
      a[p] = read_array<uint8_t>(shareDir + "adj" + sfx, BN * size_t(N) * es);
      const std::vector<uint8_t> tiled = read_array<uint8_t>(shareDir + "mask" + sfx, BN * size_t(pool) * es);
      mk[p].resize(BN * es);
      for (size_t r = 0; r < BN; r++) std::memcpy(&mk[p][r * es], &tiled[r * size_t(pool) * es], es);  // column 0
    }
    // the protein embedding: public to the evaluator of both parties, party 1's
    // alone in the two-process deployment (revealed inside the forward)
    const bool has_prot = role != 3 || party == 1;
    const std::vector<uint8_t> pr =
        has_prot ? read_array<uint8_t>(shareDir + "protein_emb.dat", size_t(B) * size_t(prot) * es)
                 : std::vector<uint8_t>(size_t(B) * size_t(prot) * es, 0);
    std::vector<int64_t> protv(size_t(B) * size_t(prot));
    for (size_t i = 0; i < protv.size(); i++) {
      if (bw == 32) {
        int32_t v;
        std::memcpy(&v, &pr[i * 4], 4);
        protv[i] = v;
      } else {
        std::memcpy(&protv[i], &pr[i * 8], 8);
      }
    }
    if (role == 3)
      check(ctx, mpcx_model_set_party_inputs(m, B, x[party].data(), a[party].data(), mk[party].data(),
                                             has_prot ? protv.data() : nullptr),
            "model_set_party_inputs");
    else
      check(ctx, mpcx_model_set_inputs(m, B, x[0].data(), x[1].data(), a[0].data(), a[1].data(), mk[0].data(),
                                       mk[1].data(), protv.data()),
            "model_set_inputs");
    std::vector<int64_t> out(static_cast<size_t>(B));
    double total_us = 0;
    uint64_t comm = 0, wire = 0;
    for (int r = 0; r < reps; r++) {
      mpcx_reset_counters(ctx);
      const uint64_t w0 = peer ? mpcx_peer_bytes(peer) : 0;
      const auto t0 = std::chrono::steady_clock::now();
      check(ctx, mpcx_model_forward(m, B), "model_forward");
      check(ctx, mpcx_model_output(m, B, out.data()), "model_output");
      total_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
      comm = mpcx_bytes_exchanged(ctx);
      wire = peer ? mpcx_peer_bytes(peer) - w0 : 0;
    }
    std::printf("Average time taken (microseconds)=%f\n", total_us / reps);
    std::printf("Comm (B)=%llu\n", static_cast<unsigned long long>(comm));
    if (peer) {
    std::printf("Peer (B)=%llu\n", static_cast<unsigned long long>(wire));
    const int tr = mpcx_peer_transport(peer);
    std::printf("Peer transport=%s\n", tr == 1 ? "ipc" : tr == 2 ? "local" : tr == 0 ? "socket" : "none");
  }
    for (int j = 0; j < B; j++) {
      const double aff = double(out[size_t(j)]) / std::ldexp(1.0, scale);
      if (B == 1)
        std::printf("AFFINITY=%.6f\n", aff);
      else
        std::printf("AFFINITY[%d]=%.6f\n", j, aff);
    }
  }
  mpcx_model_destroy(m);
  mpcx_peer_close(peer);
  mpcx_destroy(ctx);
  return 0;
}
