// mpcx_ezpc.hpp -- the EzPC GPU-MPC primitive entry points that the reference's
// secure-inference code calls, implemented over the libmpcx C ABI (mpcx.h).
//
// The reference's online path (gpu_mpc/ddg_orca*.h, secure_adj_norm.h,
// dpf_dcf_adapter.h) calls EzPC GPU-MPC by these names (signatures taken from
// those call sites; EzPC itself is not vendored).  A caller written against
// them compiles against this header with hipcc instead, one process (or thread)
// per party, unchanged in its conventions:
//   - key material goes through a host `u8 **` cursor: each keygen function
//     appends the calling party's key at the cursor and returns the output mask
//     (a device buffer from gpuMalloc); the matching read function consumes the
//     same bytes in the same order and returns the key;
//   - eval functions take the party, the peer, the key and device inputs and
//     return a newly gpuMalloc'd device output that the caller frees with gpuFree;
//   - errors abort with a message (checkCudaErrors' convention);
//   - AESGlobalContext / Stats are passed along; the peer is a SigmaPeer /
//     GpuPeer (GpuPeer(compress) + connect(party, addr), reconstructInPlace).
// Differences, by design:
//   - the two keygen runs (one per party) draw the dealer's randomness from the
//     same secret key and seed (the 16-byte file MPCX_DEALER_KEY and
//     MPCX_DEALER_SEED, default 0x5EED, read by initGPURandomness), so both
//     write consistent keys, as the reference's seeded GPU RNG does; without a
//     key file the seed alone determines the keys (a warning on stderr);
//   - the key bytes are libmpcx's format: a 256-byte record header (type and
//     sizes) before each key, checked by the read functions; writeShares writes
//     raw ring elements, as the reference's readers expect;
//   - the ring width is the element type's: bw must be 8 * sizeof(T);
//   - connect() takes a Unix socket path ("/..."), or a name that maps to
//     /tmp/mpcx_peer_<name>.sock, instead of an IP address;
//   - gpuMatmul with public weights (wIsOnGpu = false) runs the reference's
//     Beaver product with a zero weight mask (one exchange), since keygen does
//     not see the weights; the Backend<T> of mpcx_sytorch.hpp, whose keygen does,
//     uses the exchange-free product instead.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "mpcx.h"

#ifndef MPCX_EZPC_HAVE_INT_TYPES
typedef uint8_t u8;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int64_t i64;
#endif

// Server ids of the reference (SERVER0 = party 0, SERVER1 = party 1).
#ifndef SERVER0
#define SERVER0 0
#define SERVER1 1
#endif

// TruncateType of the reference's call sites (gpu_mpc/ddg_orca*.h, secure_adj_norm.h).
enum class TruncateType { None = 0, LocalLRS = 1, LocalARS = 2, TrWithSlack = 3, TrFloor = 4 };
// gpuLocalTr's shift kind (ddg_orca_base.h:300 passes ars).
enum LocalTrKind { lrs = 0, ars = 1 };
// gpuDcf's prologue / epilogue tags (dpf_dcf_adapter.h:266, 293).
struct idPrologue {};
struct maskEpilogue {};

struct Stats {
  u64 comm_time = 0, transfer_time = 0, compute_time = 0;
  u64 matmul_time = 0, matmul_comm_time = 0, conv_time = 0, conv_comm_time = 0;
  u64 relu_time = 0, reluext_time = 0, truncate_time = 0, signext_time = 0, maxpool_time = 0;
  u64 linear_comm_bytes = 0;
};

// The reference's AES context; here it names the GPU the contexts run on.
struct AESGlobalContext {
  int device = 0;
};

namespace mpcx_ezpc {

[[noreturn]] inline void die(const std::string &what) {
  std::fprintf(stderr, "mpcx_ezpc: %s\n", what.c_str());
  std::abort();
}
inline void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) die(std::string(what) + ": " + hipGetErrorString(e));
}

// The scale of the context that serves a gate which does not read it (the
// full-width DReLU and ReLU): any valid one; 12 is the reference's.
constexpr int kFullWidthScale = 12;

// Process-wide state: the dealer's seed and gate counter, identity index maps,
// the registered device key arena.
struct Runtime {
  std::mutex mu;
  int device = 0;
  uint64_t seed = 0x5EED;
  uint32_t gate = 1;
  // the dealer's secret key (initGPURandomness, from the file MPCX_DEALER_KEY);
  // key_epoch counts its changes so that every thread's contexts take it up
  uint8_t dealer_key[16] = {};
  bool has_key = false;
  uint32_t key_epoch = 0;
  std::map<size_t, uint32_t *> iota;
  const u8 *host_base = nullptr;  // initGPUKeyArena: [host_base, +arena_bytes) mirrored at arena
  u8 *arena = nullptr;
  size_t arena_bytes = 0;
  static Runtime &get() {
    static Runtime r;
    return r;
  }
};

// Contexts by (bw, scale), one set per thread (a context's stream and
// workspaces serve one caller at a time; two parties may run as two threads),
// destroyed when the thread ends.
// Each context runs on a stream of its own, a blocking one (default flags and
// priority): the legacy null stream, on which the callers' copies run
// (hipMemcpy, hipMemcpy2D, whose device-to-device and pageable forms may return
// before the copy is done) and the shim's own key and weight copies, orders
// with it both ways, as the reference's code, all on the default stream,
// expects.  So no shim call has to wait for its kernels: a later copy or
// gpuFree of the caller waits for them, and the party-mode exchanges wait for
// what they send.
// A thread's contexts share its one stream, so that all of the thread's GPU
// work (that stream and the null stream) is ordered, which the thread's block
// cache (dmalloc) relies on.
struct ThreadContexts {
  struct Entry {
    mpcx_ctx *c = nullptr;
    uint32_t key_epoch = 0;  // the dealer key this context holds (Runtime::key_epoch)
  };
  std::map<std::pair<int, int>, Entry> ctx;
  hipStream_t stream = nullptr;
  ~ThreadContexts() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto &kv : ctx) mpcx_destroy(kv.second.c);
    if (stream) (void)hipStreamDestroy(stream);
  }
};
inline mpcx_ctx *ctx(int bw, int scale = 12) {
  thread_local ThreadContexts tc;
  Runtime &R = Runtime::get();
  auto it = tc.ctx.find({bw, scale});
  if (it == tc.ctx.end()) {
    ThreadContexts::Entry e;
    if (mpcx_create(bw, scale, R.device, &e.c) != MPCX_OK)
      die("mpcx_create(bw " + std::to_string(bw) + ", scale " + std::to_string(scale) + ") failed");
    if (!tc.stream) hip_check(hipStreamCreateWithFlags(&tc.stream, hipStreamDefault), "context stream");
    if (mpcx_set_stream(e.c, tc.stream) != MPCX_OK) die("mpcx_set_stream failed");
    // the stream is blocking: the caller's null-stream copies and frees wait
    // for the party calls' work, so those calls need not synchronise it
    if (mpcx_set_party_sync(e.c, 0) != MPCX_OK) die("mpcx_set_party_sync failed");
    it = tc.ctx.emplace(std::make_pair(bw, scale), e).first;
  }
  std::lock_guard<std::mutex> lk(R.mu);
  if (it->second.key_epoch != R.key_epoch) {  // a new dealer key (or none) since this context last dealt
    if (mpcx_set_dealer_key(it->second.c, R.has_key ? R.dealer_key : nullptr) != MPCX_OK)
      die("mpcx_set_dealer_key failed");
    it->second.key_epoch = R.key_epoch;
  }
  return it->second.c;
}
// A library call's status (its kernels run on; see ctx()).
inline void check(mpcx_ctx *c, mpcx_status st, const char *what) {
  if (st != MPCX_OK) die(std::string(what) + ": " + (c ? mpcx_last_error(c) : "status " + std::to_string(st)));
}
template <typename T>
inline int bw_of(int bw) {
  if (bw != int(8 * sizeof(T))) die("ring width " + std::to_string(bw) + " differs from the element type's");
  return bw;
}
inline uint32_t next_gate() {
  Runtime &R = Runtime::get();
  std::lock_guard<std::mutex> lk(R.mu);
  return R.gate++;
}
inline uint64_t seed() { return Runtime::get().seed; }

// Device memory of the shim: the device's stream-ordered pool on the null
// stream, its release threshold at the maximum so that freed blocks stay
// cached (the reference's initGPUMemPool with cudaMallocAsync / cudaFreeAsync):
// no allocation or free waits for the device, as a hipFree would.  A free is
// ordered after the kernels that use the block because the contexts' streams
// are blocking streams (ctx()); pointers from elsewhere go to hipFree.
// Blocks come in size classes (four per power of two from 256 bytes); a block
// freed by the thread that allocated it stays on that thread's free list and
// is handed out again with no HIP call: the thread's GPU work is ordered (its
// contexts' one blocking stream and the null stream), so the block's next work
// follows its last.  A block freed by another thread goes back to the pool in
// null-stream order.
struct Pool {
  struct Blk {
    size_t cls;
    std::thread::id owner;
  };
  std::mutex mu;
  std::unordered_map<void *, Blk> live;
  bool ready = false;
  static Pool &get() {
    static Pool p;
    return p;
  }
};
inline size_t size_class(size_t b) {
  if (b <= 256) return 256;
  size_t p = 256;
  while (p * 2 <= b) p *= 2;  // p <= b < 2p
  const size_t step = p / 4;
  return (b + step - 1) / step * step;
}
struct ThreadBlocks {
  std::unordered_map<size_t, std::vector<void *>> free;  // size class -> blocks
  ~ThreadBlocks() {
    Pool &P = Pool::get();
    for (auto &kv : free)
      for (void *p : kv.second) {
        {
          std::lock_guard<std::mutex> lk(P.mu);
          P.live.erase(p);
        }
        (void)hipFreeAsync(p, nullptr);
      }
  }
};
inline ThreadBlocks &thread_blocks() {
  thread_local ThreadBlocks t;
  return t;
}
inline void *dmalloc(size_t bytes) {
  const size_t cls = size_class(bytes);
  auto &fl = thread_blocks().free[cls];
  if (!fl.empty()) {
    void *p = fl.back();
    fl.pop_back();
    return p;
  }
  Pool &P = Pool::get();
  {
    std::lock_guard<std::mutex> lk(P.mu);
    if (!P.ready) {
      int dev = 0;
      hipMemPool_t pool;
      hip_check(hipGetDevice(&dev), "memory pool");
      hip_check(hipDeviceGetDefaultMemPool(&pool, dev), "memory pool");
      uint64_t keep = ~uint64_t(0);
      hip_check(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep), "memory pool");
      P.ready = true;
    }
  }
  void *p = nullptr;
  hip_check(hipMallocAsync(&p, cls, nullptr), "gpuMalloc");
  std::lock_guard<std::mutex> lk(P.mu);
  P.live[p] = Pool::Blk{cls, std::this_thread::get_id()};
  return p;
}
inline void dfree(void *p) {
  if (!p) return;
  Pool &P = Pool::get();
  bool pooled = false, mine = false;
  size_t cls = 0;
  {
    std::lock_guard<std::mutex> lk(P.mu);
    auto it = P.live.find(p);
    if (it != P.live.end()) {
      pooled = true;
      cls = it->second.cls;
      mine = it->second.owner == std::this_thread::get_id();
      if (!mine) P.live.erase(it);
    }
  }
  if (mine)
    thread_blocks().free[cls].push_back(p);
  else if (pooled)
    hip_check(hipFreeAsync(p, nullptr), "gpuFree");
  else
    (void)hipFree(p);
}
// Identity index map 0..n-1 (element-wise Beaver products).
inline const uint32_t *iota(size_t n) {
  Runtime &R = Runtime::get();
  std::lock_guard<std::mutex> lk(R.mu);
  auto it = R.iota.find(n);
  if (it != R.iota.end()) return it->second;
  std::vector<uint32_t> h(n);
  for (size_t i = 0; i < n; i++) h[i] = uint32_t(i);
  auto *d = static_cast<uint32_t *>(dmalloc(n * 4));
  hip_check(hipMemcpy(d, h.data(), n * 4, hipMemcpyHostToDevice), "iota");
  R.iota[n] = d;
  return d;
}
inline bool in_arena(const void *d) {
  Runtime &R = Runtime::get();
  return R.arena && d >= R.arena && d < R.arena + R.arena_bytes;
}

// ---------------- key records in the u8** cursor ----------------
enum RecType : uint32_t { R_DCF = 1, R_DRELU, R_RELU, R_RELUEXT, R_LUT, R_MUL, R_TRUNC, R_SIGNEXT, R_SXS, R_SXP };
constexpr uint32_t kMagic = 0x5843504Du;  // "MPCX"
constexpr size_t kHdr = 256;
struct Hdr {
  uint32_t magic, type;
  uint64_t payload;  // bytes after the header (a multiple of 256)
  int64_t p[8];      // record parameters
};
inline size_t pad256(size_t n) { return (n + 255) & ~size_t(255); }

// Appends a record: header, then the device payload parts (each padded to 256).
struct Part {
  const void *d;
  size_t bytes;
};
inline void append(u8 **kb, uint32_t type, const std::vector<int64_t> &params, const std::vector<Part> &parts) {
  Hdr h{};
  h.magic = kMagic;
  h.type = type;
  for (size_t i = 0; i < params.size() && i < 8; i++) h.p[i] = params[i];
  size_t total = 0;
  for (auto &q : parts) total += pad256(q.bytes);
  h.payload = total;
  std::memset(*kb, 0, kHdr);
  std::memcpy(*kb, &h, sizeof h);
  u8 *o = *kb + kHdr;
  for (auto &q : parts) {
    if (q.bytes) hip_check(hipMemcpy(o, q.d, q.bytes, hipMemcpyDeviceToHost), "key to host");
    std::memset(o + q.bytes, 0, pad256(q.bytes) - q.bytes);
    o += pad256(q.bytes);
  }
  *kb = o;
}
struct Rec {
  Hdr h;
  u8 *payload;  // host (or arena) address of the payload in the key buffer
};
inline Rec take(u8 **kb, uint32_t type, const char *what) {
  Rec r;
  std::memcpy(&r.h, *kb, sizeof r.h);
  if (r.h.magic != kMagic || r.h.type != type)
    die(std::string(what) + ": the key cursor is not at a key of this kind (keygen and eval out of step)");
  r.payload = *kb + kHdr;
  *kb += kHdr + r.h.payload;
  return r;
}
// Device copy of `bytes` key bytes at host address h (or the arena mirror of
// h when the key buffer was moved to HBM with initGPUKeyArena and the address
// is 256-byte aligned there); release with key_release.
struct DevKey {
  u8 *d = nullptr;
  bool owned = false;
};
inline DevKey key_on_device(const u8 *h, size_t bytes) {
  Runtime &R = Runtime::get();
  DevKey k;
  if (!h || bytes == 0) return k;  // nothing to stage: a null device pointer
  if (R.arena && h >= R.host_base && h + bytes <= R.host_base + R.arena_bytes) {
    u8 *d = R.arena + (h - R.host_base);
    if ((reinterpret_cast<uintptr_t>(d) & 255u) == 0) {
      k.d = d;
      return k;
    }
  }
  k.d = static_cast<u8 *>(dmalloc(bytes));
  k.owned = true;
  hip_check(hipMemcpy(k.d, h, bytes, hipMemcpyHostToDevice), "key to device");
  return k;
}
// Device view of a host or device buffer (copied when it is host memory).
inline DevKey on_device(const void *p, size_t bytes) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) == hipSuccess && a.type == hipMemoryTypeDevice) {
    DevKey k;
    k.d = static_cast<u8 *>(const_cast<void *>(p));
    return k;
  }
  (void)hipGetLastError();  // a plain host pointer is not an error here
  return key_on_device(static_cast<const u8 *>(p), bytes);
}
inline void key_release(DevKey &k) {
  if (k.owned && k.d) dfree(k.d);
  k.d = nullptr;
}

// Shares of a dealer value: share 0 from the dealer's PRF, share 1 = v - share 0.
template <typename T>
inline void split(mpcx_ctx *c, size_t n, const T *d_v, T *d_s0, T *d_s1) {
  const size_t blocks = (n * sizeof(T) + 15) / 16;
  void *tmp = dmalloc(blocks * 16);
  check(c, mpcx_prf(c, seed(), next_gate(), 0x51u, blocks, tmp), "share PRF");
  hip_check(hipMemcpy(d_s0, tmp, n * sizeof(T), hipMemcpyDeviceToDevice), "share");
  dfree(tmp);
  check(c, mpcx_ring_lincomb(c, n, 1, 1, d_v, uint64_t(0) - 1, d_s0, nullptr, 0, d_s1), "share");
}

}  // namespace mpcx_ezpc

// ===========================================================================
// memory (extern "C" in the reference: gpuMalloc, gpuFree, moveToGPU,
// moveIntoCPUMem, initGPUKeyArena, freeGPUKeyArena; patch:632-768)
// ===========================================================================
inline void initGPUMemPool() { mpcx_ezpc::dfree(mpcx_ezpc::dmalloc(1)); }
inline u8 *gpuMalloc(size_t bytes) { return static_cast<u8 *>(mpcx_ezpc::dmalloc(bytes)); }
// No-op for addresses inside the key arena (patch:692-697).
inline void gpuFree(void *d) {
  if (d && !mpcx_ezpc::in_arena(d)) mpcx_ezpc::dfree(d);
}
inline u8 *cpuMalloc(size_t bytes, bool pin = true) {
  void *p = nullptr;
  if (pin) {
    mpcx_ezpc::hip_check(hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault), "cpuMalloc");
  } else {
    p = std::malloc(bytes ? bytes : 1);
    if (!p) mpcx_ezpc::die("cpuMalloc");
  }
  return static_cast<u8 *>(p);
}
inline void cpuFree(void *h, bool pinned = true) {
  if (!h) return;
  if (pinned)
    (void)hipHostFree(h);
  else
    std::free(h);
}
inline void getAlignedBuf(u8 **buf, size_t bytes, bool pin = true) { *buf = cpuMalloc(bytes, pin); }
// Host -> device copy of a key or mask region; inside the key arena, the
// arena's mirror of it (translation, patch:721-731).
inline u8 *moveToGPU(u8 *h, size_t bytes, Stats *) {
  mpcx_ezpc::Runtime &R = mpcx_ezpc::Runtime::get();
  if (R.arena && h >= R.host_base && h + bytes <= R.host_base + R.arena_bytes) return R.arena + (h - R.host_base);
  u8 *d = gpuMalloc(bytes);
  mpcx_ezpc::hip_check(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice), "moveToGPU");
  return d;
}
inline void moveIntoCPUMem(u8 *h, u8 *d, size_t bytes, Stats *) {
  mpcx_ezpc::hip_check(hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost), "moveIntoCPUMem");
}
// The whole host key buffer [h, h + bytes) copied to HBM once; later key
// reads in that range use the device copy (initGPUKeyArena, patch:632-661).
inline void initGPUKeyArena(u8 *h, size_t bytes) {
  mpcx_ezpc::Runtime &R = mpcx_ezpc::Runtime::get();
  if (R.arena) mpcx_ezpc::dfree(R.arena);
  R.arena = static_cast<u8 *>(mpcx_ezpc::dmalloc(bytes));
  mpcx_ezpc::hip_check(hipMemcpy(R.arena, h, bytes, hipMemcpyHostToDevice), "initGPUKeyArena");
  R.host_base = h;
  R.arena_bytes = bytes;
}
inline void freeGPUKeyArena() {
  mpcx_ezpc::Runtime &R = mpcx_ezpc::Runtime::get();
  if (R.arena) mpcx_ezpc::dfree(R.arena);
  R.arena = nullptr;
  R.host_base = nullptr;
  R.arena_bytes = 0;
}

// ===========================================================================
// randomness and AES context
// ===========================================================================
inline void initAESContext(AESGlobalContext *g) {
  const char *d = std::getenv("MPCX_DEVICE");
  mpcx_ezpc::Runtime::get().device = d && *d ? std::atoi(d) : 0;
  if (g) g->device = mpcx_ezpc::Runtime::get().device;
}
// Resets the dealer's randomness: both parties' keygen runs then draw the same
// sequence and write consistent keys.  The dealer's secret key comes from the
// file named by MPCX_DEALER_KEY (16 bytes), and the seed (MPCX_DEALER_SEED)
// then only names the key set; without a key file the keys rest on the seed
// alone, which is said once on stderr.
inline void initGPURandomness() {
  mpcx_ezpc::Runtime &R = mpcx_ezpc::Runtime::get();
  const char *s = std::getenv("MPCX_DEALER_SEED");
  const char *kf = std::getenv("MPCX_DEALER_KEY");
  uint8_t key[16] = {};
  bool has = false;
  if (kf && *kf) {
    FILE *f = std::fopen(kf, "rb");
    if (!f) mpcx_ezpc::die(std::string("cannot open MPCX_DEALER_KEY file ") + kf);
    const size_t got = std::fread(key, 1, 16, f);
    const int extra = std::fgetc(f);
    std::fclose(f);
    if (got != 16 || extra != EOF) mpcx_ezpc::die(std::string("MPCX_DEALER_KEY (") + kf + ") must hold exactly 16 bytes");
    has = true;
  }
  std::lock_guard<std::mutex> lk(R.mu);
  R.seed = s && *s ? std::strtoull(s, nullptr, 0) : 0x5EEDull;
  R.gate = 1;
  if (has != R.has_key || std::memcmp(key, R.dealer_key, 16) != 0) {
    std::memcpy(R.dealer_key, key, 16);
    R.has_key = has;
    R.key_epoch++;
  }
  static bool warned = false;
  if (!has && !warned) {
    warned = true;
    std::fprintf(stderr, "mpcx_ezpc: warning: no MPCX_DEALER_KEY: the dealer's keys derive from the seed "
                         "MPCX_DEALER_SEED alone, so anyone who knows the seed can regenerate every mask\n");
  }
}
inline void destroyGPURandomness() {}
inline void initCPURandomness() {}
inline void destroyCPURandomness() {}

// Dealer randomness on the device: N uniform ring elements (randomGEOnGpu).
template <typename T>
inline T *randomGEOnGpu(u64 N, int bw) {
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  const size_t blocks = (N * sizeof(T) + 15) / 16;
  T *d = reinterpret_cast<T *>(gpuMalloc(blocks * 16));
  mpcx_ezpc::check(c, mpcx_prf(c, mpcx_ezpc::seed(), mpcx_ezpc::next_gate(), 0x52u, blocks, d), "randomGEOnGpu");
  if (bw < int(8 * sizeof(T)))  // reduce mod 2^bw: x - (x >> bw << bw) is not a ring op; mask on the host
  {
    std::vector<T> h(N);
    mpcx_ezpc::hip_check(hipMemcpy(h.data(), d, N * sizeof(T), hipMemcpyDeviceToHost), "randomGEOnGpu");
    for (auto &v : h) v &= T((T(1) << bw) - 1);
    mpcx_ezpc::hip_check(hipMemcpy(d, h.data(), N * sizeof(T), hipMemcpyHostToDevice), "randomGEOnGpu");
  }
  return d;
}

// ===========================================================================
// linear ops (gpuLinearComb / gpuAdd behind add, sub, scalarmul:
// ddg_orca_base.h:304-314, ddg_orca.h:65-81)
// ===========================================================================
template <typename T>
inline void gpuLinearComb(int bw, u64 N, T *d_out, T a, const T *d_x) {
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw));
  mpcx_ezpc::check(c, mpcx_ring_lincomb(c, N, 1, uint64_t(a), d_x, 0, nullptr, nullptr, 0, d_out), "gpuLinearComb");
}
template <typename T>
inline void gpuLinearComb(int bw, u64 N, T *d_out, T a, const T *d_x, T b, const T *d_y) {
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw));
  mpcx_ezpc::check(c, mpcx_ring_lincomb(c, N, 1, uint64_t(a), d_x, uint64_t(b), d_y, nullptr, 0, d_out),
                   "gpuLinearComb");
}
template <typename T>
inline T *gpuAdd(int bw, u64 N, const std::vector<T *> &in) {
  T *out = reinterpret_cast<T *>(gpuMalloc(N * sizeof(T)));
  mpcx_ezpc::hip_check(hipMemcpy(out, in.at(0), N * sizeof(T), hipMemcpyDeviceToDevice), "gpuAdd");
  for (size_t i = 1; i < in.size(); i++) gpuLinearComb<T>(bw, N, out, T(1), out, T(1), in[i]);
  return out;
}
// Party p's share of the dealer's d_A, raw at the cursor (writeShares).
template <typename T, typename U>
inline void writeShares(u8 **kb, int party, u64 N, T *d_A, int bw) {
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw));
  T *s0 = reinterpret_cast<T *>(gpuMalloc(N * sizeof(T)));
  T *s1 = reinterpret_cast<T *>(gpuMalloc(N * sizeof(T)));
  mpcx_ezpc::split<T>(c, N, d_A, s0, s1);
  moveIntoCPUMem(*kb, reinterpret_cast<u8 *>(party == SERVER0 ? s0 : s1), N * sizeof(T), nullptr);
  *kb += N * sizeof(T);
  gpuFree(s0);
  gpuFree(s1);
}
// d_A -= the clear mask at h_mask (the output unmasking of DDGOrcaBase::output).
template <typename T>
inline void unmaskValues(int bw, u64 N, T *d_A, T *h_mask, Stats *s) {
  T *d_m = reinterpret_cast<T *>(moveToGPU(reinterpret_cast<u8 *>(h_mask), N * sizeof(T), s));
  gpuLinearComb<T>(bw, N, d_A, T(1), d_A, T(0) - T(1), d_m);
  gpuFree(d_m);
}
// Local shift of masked values (gpuLocalTr<T, T, ars>).
template <typename T, typename U, LocalTrKind K>
inline T *gpuLocalTr(int party, int bin, int shift, u64 N, T *d_I, bool inPlace) {
  static_assert(K == ars, "only the arithmetic local shift is provided");
  (void)party;
  mpcx_ctx *c = mpcx_ezpc::ctx(int(8 * sizeof(T)), shift);
  T *out = inPlace ? d_I : reinterpret_cast<T *>(gpuMalloc(N * sizeof(T)));
  (void)bin;
  mpcx_ezpc::check(c, mpcx_tr_eval(c, MPCX_LOCALARS, N, nullptr, nullptr, d_I, nullptr, 0, out), "gpuLocalTr");
  return out;
}

// ===========================================================================
// the peer (GpuPeer / SigmaPeer, gpu_mpc/utils/gpu_comms.h:94-397,
// gpu_mpc/utils/sigma_comms.cpp:36-150)
// ===========================================================================
class SigmaPeer {
 public:
  mpcx_peer *h = nullptr;
  int party = -1;
  explicit SigmaPeer(bool compress = true) { (void)compress; }
  virtual ~SigmaPeer() { close(); }
  // Party 0 listens, party 1 connects, on a Unix socket: addr is its path, or a
  // name for /tmp/mpcx_peer_<name>.sock.
  void connect(int p, const std::string &addr) {
    const std::string path = !addr.empty() && addr[0] == '/' ? addr : "/tmp/mpcx_peer_" + addr + ".sock";
    if (mpcx_peer_connect(p, path.c_str(), 60000, &h) != MPCX_OK) mpcx_ezpc::die("connect to the peer failed");
    party = p;
  }
  // Both parties in one process (two threads): an end of mpcx_peer_pair.
  void attach(mpcx_peer *end) {
    h = end;
    party = mpcx_peer_party(end);
  }
  void close() {
    if (h) mpcx_peer_close(h);
    h = nullptr;
  }
  u64 bytesSent() const { return h ? mpcx_peer_bytes(h) / 2 : 0; }
  u64 bytesReceived() const { return h ? mpcx_peer_bytes(h) / 2 : 0; }
  // d_A: this party's additive share in, the sum of both parties' shares out.
  template <typename T>
  void reconstructInPlace(T *d_A, int bw, u64 N, Stats *) {
    mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw));
    mpcx_ezpc::check(c, mpcx_party_reconstruct(c, h, N, d_A), "reconstructInPlace");
  }
};
class GpuPeer : public SigmaPeer {
 public:
  explicit GpuPeer(bool compress = true) : SigmaPeer(compress) {}
};

namespace mpcx_ezpc {
inline mpcx_peer *peer_of(SigmaPeer *p, int party) {
  if (!p || !p->h) die("no peer");
  if (p->party != party) die("the party argument differs from the peer's party");
  return p->h;
}
// Key of a gate record: device copy of its payload, released at scope end.
struct ScopedKey {
  DevKey k;
  ScopedKey(const u8 *h, size_t bytes) : k(key_on_device(h, bytes)) {}
  ~ScopedKey() { key_release(k); }
  const u8 *get() const { return k.d; }
};
// Both parties' keys of one gate from the dealer (keygen writes both; the
// calling party keeps its own).
struct KeyPair {
  void *k[2] = {nullptr, nullptr};
  size_t bytes = 0;
  explicit KeyPair(size_t n) : bytes(n) {
    k[0] = dmalloc(n);
    k[1] = dmalloc(n);
  }
  ~KeyPair() {
    dfree(k[0]);
    dfree(k[1]);
  }
};
// The ReLU gate for inputs of bin significant bits: the full-width RELU at
// bin = bw; for bin < bw (the reference's mode-3 ReLU, bin = bw - scale,
// gpu_mpc/ddg_orca.h:229-233) the narrow RELUPOOL gate, exact for a full-width
// input with |x| < 2^bin, i.e. at the context scale bw - bin, which a context
// supports for 1 <= bw - bin <= bw/2 - 2.  Other widths cannot be served.
inline int relu_scale(int bw, int bin, int bout) {
  if (bout != bin && bout != bw) die("gpuGenReluKey: bout must be bin or the ring width");
  if (bin == bw) return kFullWidthScale;
  if (bw - bin < 1 || bw - bin > bw / 2 - 2)
    die("gpuGenReluKey: no ReLU gate for " + std::to_string(bin) + "-bit inputs in a " + std::to_string(bw) +
        "-bit ring (bin must be bw, or bw - scale with 1 <= scale <= bw/2 - 2)");
  return bw - bin;
}
}  // namespace mpcx_ezpc

// ===========================================================================
// DCF (gpuKeyGenDCF / readGPUDcfKey / gpuDcf, dpf_dcf_adapter.h:100, 266, 372)
// ===========================================================================
struct GPUDPFKey {
  int bin = 0, M = 0;
  u8 *key = nullptr;  // this party's key bytes in the key buffer
  size_t bytes = 0;
};
// DCF of [x < rin] over bin-bit inputs, XOR-shared output bits.
template <typename T>
inline void gpuKeyGenDCF(u8 **kb, int party, int bin, int N, T *d_rin, AESGlobalContext *) {
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  std::vector<T> h(static_cast<size_t>(N));
  std::vector<uint64_t> a(static_cast<size_t>(N));
  mpcx_ezpc::hip_check(hipMemcpy(h.data(), d_rin, N * sizeof(T), hipMemcpyDeviceToHost), "gpuKeyGenDCF");
  const uint64_t lim = bin >= 64 ? ~uint64_t(0) : (uint64_t(1) << bin) - 1;
  for (int i = 0; i < N; i++) a[size_t(i)] = uint64_t(h[size_t(i)]) & lim;
  auto *d_a = reinterpret_cast<uint64_t *>(gpuMalloc(size_t(N) * 8));
  mpcx_ezpc::hip_check(hipMemcpy(d_a, a.data(), size_t(N) * 8, hipMemcpyHostToDevice), "gpuKeyGenDCF");
  mpcx_ezpc::KeyPair kp(mpcx_dcf_key_bytes(bin, size_t(N)));
  mpcx_ezpc::check(c, mpcx_dcf_keygen(c, bin, size_t(N), d_a, nullptr, mpcx_ezpc::seed(), mpcx_ezpc::next_gate(),
                                      kp.k[0], kp.k[1]),
                   "gpuKeyGenDCF");
  gpuFree(d_a);
  mpcx_ezpc::append(kb, mpcx_ezpc::R_DCF, {bin, N}, {{kp.k[party], kp.bytes}});
}
inline GPUDPFKey readGPUDcfKey(u8 **kb) {
  auto r = mpcx_ezpc::take(kb, mpcx_ezpc::R_DCF, "readGPUDcfKey");
  GPUDPFKey k;
  k.bin = int(r.h.p[0]);
  k.M = int(r.h.p[1]);
  k.key = r.payload;
  k.bytes = mpcx_dcf_key_bytes(k.bin, size_t(k.M));
  return k;
}
// Party p's share of the packed output bits (32 per u32 word), XORed with
// (*h_mask)[0] when given (maskEpilogue: the masked DCF of DReLU / truncation).
// The inputs stay on the device (read modulo 2^bin by the kernel) and the mask
// words go to the device with the key (the arena's copy when the key buffer is
// resident), so nothing returns to the host.
template <typename T, int E, typename Pro, typename Epi>
inline u32 *gpuDcf(GPUDPFKey k, int party, T *d_in, AESGlobalContext *, Stats *, std::vector<u32 *> *h_mask = nullptr) {
  static_assert(E == 1, "one output bit per element");
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  const size_t N = size_t(k.M), words = (N + 63) / 64;
  auto *d_out = reinterpret_cast<uint64_t *>(gpuMalloc(words * 8));
  mpcx_ezpc::ScopedKey key(k.key, k.bytes);
  const bool masked = h_mask && !h_mask->empty() && (*h_mask)[0];
  mpcx_ezpc::ScopedKey mask(masked ? reinterpret_cast<const u8 *>((*h_mask)[0]) : nullptr,
                            masked ? ((N + 31) / 32) * 4 : 0);
  mpcx_ezpc::check(c,
                   mpcx_dcf_eval_ring(c, party, k.bin, N, key.get(), d_in,
                                      reinterpret_cast<const uint32_t *>(mask.get()), d_out),
                   "gpuDcf");
  return reinterpret_cast<u32 *>(d_out);
}

// ===========================================================================
// DReLU and ReLU (gpuKeyGenDRelu, dpf_dcf_adapter.h:330; gpuGenReluKey /
// readReluKey / gpuRelu, ddg_orca.h:103-104, 233; gpuKeygenReluExtend /
// gpuReluExtend, ddg_orca.h:90, 222, dpf_dcf_adapter.h:225-234)
// ===========================================================================
template <typename T>
struct GPUReluKey {
  int bin = 0, bout = 0, N = 0, kind = 0, scale = 0;
  u8 *key = nullptr;
  size_t bytes = 0;
};
using GPUDReluKey = GPUReluKey<u64>;

namespace mpcx_ezpc {
// keygen of one truncation-family gate over N inputs with mask d_in; returns
// the output mask; appends the party's key as record `type`.
template <typename T>
inline T *tr_keygen(u8 **kb, int party, uint32_t type, int kind, int scale, int bin, int bout, int N,
                    const T *d_in) {
  mpcx_ctx *c = ctx(8 * int(sizeof(T)), scale);
  T *out = reinterpret_cast<T *>(gpuMalloc(size_t(N) * sizeof(T)));
  if (kind == MPCX_LOCALARS) {
    check(c, mpcx_tr_keygen(c, kind, size_t(N), d_in, out, seed(), next_gate(), nullptr, nullptr), "keygen");
    append(kb, type, {bin, bout, N, kind, scale}, {});
    return out;
  }
  KeyPair kp(mpcx_tr_key_bytes(c, kind, size_t(N)));
  check(c, mpcx_tr_keygen(c, kind, size_t(N), d_in, out, seed(), next_gate(), kp.k[0], kp.k[1]), "keygen");
  append(kb, type, {bin, bout, N, kind, scale}, {{kp.k[party], kp.bytes}});
  return out;
}
template <typename T>
inline GPUReluKey<T> tr_read(u8 **kb, uint32_t type, const char *what) {
  auto r = take(kb, type, what);
  GPUReluKey<T> k;
  k.bin = int(r.h.p[0]);
  k.bout = int(r.h.p[1]);
  k.N = int(r.h.p[2]);
  k.kind = int(r.h.p[3]);
  k.scale = int(r.h.p[4]);
  k.key = r.payload;
  k.bytes = k.kind == MPCX_LOCALARS ? 0 : mpcx_tr_key_bytes(ctx(8 * int(sizeof(T)), k.scale), k.kind, size_t(k.N));
  return k;
}
// AES calls of this thread's gate evaluations (one thread per party), for the
// caller's accounting of the DCF work.
inline uint64_t &aes_calls() {
  thread_local uint64_t n = 0;
  return n;
}
template <typename T>
inline T *tr_eval(SigmaPeer *peer, int party, const GPUReluKey<T> &k, const T *d_in, const T *d_bias = nullptr,
                  int ncol = 0) {
  mpcx_ctx *c = ctx(8 * int(sizeof(T)), k.scale);
  aes_calls() += uint64_t(k.N) * uint64_t(std::max(0, mpcx_tr_aes_calls(c, k.kind)));
  T *out = reinterpret_cast<T *>(gpuMalloc(size_t(k.N) * sizeof(T)));
  if (k.kind == MPCX_LOCALARS) {
    check(c, mpcx_tr_eval(c, k.kind, size_t(k.N), nullptr, nullptr, d_in, d_bias, ncol, out), "eval");
    return out;
  }
  ScopedKey key(k.key, k.bytes);
  check(c, mpcx_party_tr_eval(c, peer_of(peer, party), k.kind, size_t(k.N), key.get(), d_in, d_bias, ncol, out),
        "eval");
  return out;
}
}  // namespace mpcx_ezpc

// DReLU of inputs masked by d_mask: returns the mask bit (a 0/1 ring element);
// gpuDRelu gives the masked public bit, [x >= 0] = bit XOR mask.
template <typename T>
inline T *gpuKeyGenDRelu(u8 **kb, int party, int bin, int N, T *d_mask, AESGlobalContext *) {
  if (bin != 8 * int(sizeof(T))) mpcx_ezpc::die("gpuKeyGenDRelu: only full-width inputs (bin = the ring width)");
  return mpcx_ezpc::tr_keygen<T>(kb, party, mpcx_ezpc::R_DRELU, MPCX_DRELU, mpcx_ezpc::kFullWidthScale, bin, 1, N,
                                 d_mask);
}
inline GPUDReluKey readGPUDReluKey(u8 **kb) {
  return mpcx_ezpc::tr_read<u64>(kb, mpcx_ezpc::R_DRELU, "readGPUDReluKey");
}
template <typename T>
inline T *gpuDRelu(SigmaPeer *peer, int party, GPUDReluKey k, T *d_in, AESGlobalContext *, Stats *) {
  GPUReluKey<T> kk{k.bin, k.bout, k.N, k.kind, k.scale, k.key, k.bytes};
  return mpcx_ezpc::tr_eval<T>(peer, party, kk, d_in);
}

template <typename TIn, typename TOut, int E1, int E2, bool B>
inline TOut *gpuGenReluKey(u8 **kb, int party, int bin, int bout, int N, TIn *d_inMask, AESGlobalContext *) {
  static_assert(std::is_same<TIn, TOut>::value, "one ring type in and out");
  const int bw = 8 * int(sizeof(TIn));
  // an input known to fit bin < bw bits (the reference's mode-3 ReLU) takes the narrow gate
  const int sc = mpcx_ezpc::relu_scale(bw, bin, bout);
  return mpcx_ezpc::tr_keygen<TIn>(kb, party, mpcx_ezpc::R_RELU, bin == bw ? MPCX_RELU : MPCX_RELUPOOL, sc, bin, bout,
                                   N, d_inMask);
}
template <typename T>
inline GPUReluKey<T> readReluKey(u8 **kb) {
  return mpcx_ezpc::tr_read<T>(kb, mpcx_ezpc::R_RELU, "readReluKey");
}
template <typename TIn, typename TOut, int E1, int E2, bool B>
inline TOut *gpuRelu(SigmaPeer *peer, int party, GPUReluKey<TIn> k, TIn *d_in, AESGlobalContext *, Stats *) {
  return mpcx_ezpc::tr_eval<TIn>(peer, party, k, d_in);
}

// ReLU of a value held in its low bin bits (a truncate-reduce output), extended
// to bout = bw bits: keygen returns (nullptr, output mask).
template <typename T>
inline std::pair<u8 *, T *> gpuKeygenReluExtend(u8 **kb, int party, int bin, int bout, int N, T *d_inMask,
                                                AESGlobalContext *) {
  const int bw = 8 * int(sizeof(T));
  if (bout != bw) mpcx_ezpc::die("gpuKeygenReluExtend: bout must be the ring width");
  return {nullptr,
          mpcx_ezpc::tr_keygen<T>(kb, party, mpcx_ezpc::R_RELUEXT, MPCX_EXTRELU, bw - bin, bin, bout, N, d_inMask)};
}
template <typename T>
inline GPUReluKey<T> readGPUReluExtendKey(u8 **kb) {
  return mpcx_ezpc::tr_read<T>(kb, mpcx_ezpc::R_RELUEXT, "readGPUReluExtendKey");
}
template <typename T>
inline std::pair<u32 *, T *> gpuReluExtend(SigmaPeer *peer, int party, GPUReluKey<T> k, T *d_I, AESGlobalContext *,
                                          Stats *) {
  return {nullptr, mpcx_ezpc::tr_eval<T>(peer, party, k, d_I)};
}
namespace dpf_dcf {
using ::gpuKeygenReluExtend;
using ::gpuReluExtend;
using ::readGPUReluExtendKey;
}  // namespace dpf_dcf

// ===========================================================================
// truncation (genGPUTruncateKey / readGPUTruncateKey / gpuTruncate,
// ddg_orca.h:116-118, 240-241; sign extension genGPUSignExtendKey /
// gpuSignExtend, ddg_orca.h:125-138, 258-263)
// ===========================================================================
template <typename T>
struct GPUTruncateKey {
  TruncateType t = TruncateType::None;
  GPUReluKey<T> a, b;  // TrFloor: truncate-reduce then sign extension; else a alone
};
template <typename T>
using GPUSignExtendKey = GPUReluKey<T>;

namespace mpcx_ezpc {
template <typename T>
inline T *trunc_keygen(u8 **kb, int party, TruncateType t, int shift, int N, const T *d_in) {
  const int bw = 8 * int(sizeof(T));
  switch (t) {
    case TruncateType::TrFloor: {
      T *r1 = tr_keygen<T>(kb, party, R_TRUNC, MPCX_TRMOD, shift, bw, bw - shift, N, d_in);
      T *r2 = tr_keygen<T>(kb, party, R_TRUNC, MPCX_EXT, shift, bw - shift, bw, N, r1);
      gpuFree(r1);
      return r2;
    }
    case TruncateType::TrWithSlack:
      return tr_keygen<T>(kb, party, R_TRUNC, MPCX_TRSLACK, shift, bw, bw, N, d_in);
    case TruncateType::LocalARS:
      return tr_keygen<T>(kb, party, R_TRUNC, MPCX_LOCALARS, shift, bw, bw, N, d_in);
    default:
      die("truncation type not provided");
  }
}
template <typename T>
inline GPUTruncateKey<T> trunc_read(TruncateType t, u8 **kb) {
  GPUTruncateKey<T> k;
  k.t = t;
  k.a = tr_read<T>(kb, R_TRUNC, "readGPUTruncateKey");
  if (t == TruncateType::TrFloor) k.b = tr_read<T>(kb, R_TRUNC, "readGPUTruncateKey");
  return k;
}
template <typename T>
inline T *trunc_eval(SigmaPeer *peer, int party, const GPUTruncateKey<T> &k, const T *d_in, const T *d_bias = nullptr,
                     int ncol = 0) {
  T *y = tr_eval<T>(peer, party, k.a, d_in, d_bias, ncol);
  if (k.t != TruncateType::TrFloor) return y;
  T *z = tr_eval<T>(peer, party, k.b, y);
  gpuFree(y);
  return z;
}
}  // namespace mpcx_ezpc

template <typename T, typename U>
inline T *genGPUTruncateKey(u8 **kb, int party, TruncateType t, int bin, int bout, int shift, int N, T *d_inMask,
                            AESGlobalContext *) {
  const int bw = 8 * int(sizeof(T));
  if (bin != bw || bout != bw) mpcx_ezpc::die("genGPUTruncateKey: bin and bout must be the ring width");
  return mpcx_ezpc::trunc_keygen<T>(kb, party, t, shift, N, d_inMask);
}
template <typename T>
inline GPUTruncateKey<T> readGPUTruncateKey(TruncateType t, u8 **kb) {
  return mpcx_ezpc::trunc_read<T>(t, kb);
}
template <typename T, typename U>
inline T *gpuTruncate(int bin, int bout, TruncateType t, GPUTruncateKey<T> k, int shift, SigmaPeer *peer, int party,
                      int N, T *d_I, AESGlobalContext *, Stats *) {
  if (k.t != t || k.a.N != N || k.a.scale != shift) mpcx_ezpc::die("gpuTruncate: key of another truncation");
  (void)bin;
  (void)bout;
  return mpcx_ezpc::trunc_eval<T>(peer, party, k, d_I);
}
// Sign extension of a value held in its low bin bits (a truncate-reduce output).
template <typename T, typename U>
inline T *genGPUSignExtendKey(u8 **kb, int party, int bin, int bout, int N, T *d_inMask, AESGlobalContext *) {
  const int bw = 8 * int(sizeof(T));
  if (bout != bw) mpcx_ezpc::die("genGPUSignExtendKey: bout must be the ring width");
  return mpcx_ezpc::tr_keygen<T>(kb, party, mpcx_ezpc::R_SIGNEXT, MPCX_EXT, bw - bin, bin, bout, N, d_inMask);
}
template <typename T>
inline GPUSignExtendKey<T> readGPUSignExtendKey(u8 **kb) {
  return mpcx_ezpc::tr_read<T>(kb, mpcx_ezpc::R_SIGNEXT, "readGPUSignExtendKey");
}
template <typename T, typename U>
inline T *gpuSignExtend(int party, SigmaPeer *peer, int bin, int bout, int N, GPUSignExtendKey<T> k, T *d_I,
                        AESGlobalContext *, Stats *) {
  (void)bin;
  (void)bout;
  (void)N;
  return mpcx_ezpc::tr_eval<T>(peer, party, k, d_I);
}

// ===========================================================================
// 8-bit DPF lookup table (gpuKeyGenLUT / readGPULUTKey / gpuDpfLUT,
// secure_adj_norm.h:270-279, 498-520)
// ===========================================================================
template <typename T>
struct GPULUTKey {
  int bin = 0, bout = 0, N = 0;
  u8 *key = nullptr;
  size_t bytes = 0;
};
template <typename T, typename U>
inline T *gpuKeyGenLUT(u8 **kb, int party, int bin, int bout, int N, T *d_inMask, AESGlobalContext *) {
  if (bin != 8) mpcx_ezpc::die("gpuKeyGenLUT: an 8-bit input domain only");
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bout));
  T *out = reinterpret_cast<T *>(gpuMalloc(size_t(N) * sizeof(T)));
  mpcx_ezpc::KeyPair kp(mpcx_lut8_key_bytes(c, size_t(N)));
  mpcx_ezpc::check(c, mpcx_lut8_keygen(c, size_t(N), d_inMask, out, mpcx_ezpc::seed(), mpcx_ezpc::next_gate(),
                                       kp.k[0], kp.k[1]),
                   "gpuKeyGenLUT");
  mpcx_ezpc::append(kb, mpcx_ezpc::R_LUT, {bin, bout, N}, {{kp.k[party], kp.bytes}});
  return out;
}
template <typename T>
inline GPULUTKey<T> readGPULUTKey(u8 **kb) {
  auto r = mpcx_ezpc::take(kb, mpcx_ezpc::R_LUT, "readGPULUTKey");
  GPULUTKey<T> k;
  k.bin = int(r.h.p[0]);
  k.bout = int(r.h.p[1]);
  k.N = int(r.h.p[2]);
  k.key = r.payload;
  k.bytes = mpcx_lut8_key_bytes(mpcx_ezpc::ctx(8 * int(sizeof(T))), size_t(k.N));
  return k;
}
// d_x: masked public inputs; d_table: 256 ring elements; returns T[x] masked.
template <typename T, typename U>
inline T *gpuDpfLUT(GPULUTKey<T> k, SigmaPeer *peer, int party, T *d_x, T *d_table, AESGlobalContext *, Stats *,
                    bool opMasked = true) {
  if (!opMasked) mpcx_ezpc::die("gpuDpfLUT: masked outputs only");
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  T *out = reinterpret_cast<T *>(gpuMalloc(size_t(k.N) * sizeof(T)));
  mpcx_ezpc::ScopedKey key(k.key, k.bytes);
  mpcx_ezpc::check(c, mpcx_party_lut8_eval(c, mpcx_ezpc::peer_of(peer, party), size_t(k.N), key.get(), d_table, d_x,
                                           out),
                   "gpuDpfLUT");
  return out;
}

// ===========================================================================
// Beaver element-wise product (gpuKeygenMul / readGPUMulKey / gpuMul,
// secure_adj_norm.h:326-365, 569-651; ddg_orca.h:43-63)
// ===========================================================================
template <typename T>
struct GPUMulKey {
  u64 szA = 0, szB = 0, szC = 0;
  T *a = nullptr, *b = nullptr, *c = nullptr;  // this party's shares of the masks of A and B, its C term
  u8 *key = nullptr;
  size_t bytes = 0;
  GPUTruncateKey<T> tr;  // the truncation after the product
};
template <typename T>
inline T *gpuKeygenMul(u8 **kb, int party, int bw, int scale, int N, T *d_maskA, T *d_maskB, TruncateType t,
                       AESGlobalContext *) {
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw), scale);
  const size_t n = size_t(N);
  const uint32_t *id = mpcx_ezpc::iota(n);
  T *rz = reinterpret_cast<T *>(gpuMalloc(n * sizeof(T)));
  mpcx_ezpc::KeyPair kp(mpcx_mul_key_bytes(c, n, n, n));
  mpcx_ezpc::check(c, mpcx_mul_keygen(c, n, n, n, id, id, d_maskA, d_maskB, rz, mpcx_ezpc::seed(),
                                      mpcx_ezpc::next_gate(), kp.k[0], kp.k[1]),
                   "gpuKeygenMul");
  mpcx_ezpc::append(kb, mpcx_ezpc::R_MUL, {N, int(t), scale}, {{kp.k[party], kp.bytes}});
  if (t == TruncateType::None) return rz;
  T *out = mpcx_ezpc::trunc_keygen<T>(kb, party, t, scale, N, rz);
  gpuFree(rz);
  return out;
}
template <typename T>
inline GPUMulKey<T> readGPUMulKey(u8 **kb, u64 szA, u64 szB, u64 szC, TruncateType t) {
  auto r = mpcx_ezpc::take(kb, mpcx_ezpc::R_MUL, "readGPUMulKey");
  GPUMulKey<T> k;
  k.szA = szA;
  k.szB = szB;
  k.szC = szC;
  if (szA != szC || szB != szC || u64(r.h.p[0]) != szC || int(r.h.p[1]) != int(t))
    mpcx_ezpc::die("readGPUMulKey: key of another product");
  mpcx_ctx *c = mpcx_ezpc::ctx(8 * int(sizeof(T)));
  size_t off[3];
  mpcx_ezpc::check(c, mpcx_mul_key_layout(c, szA, szB, szC, off), "readGPUMulKey");
  k.key = r.payload;
  k.bytes = mpcx_mul_key_bytes(c, szA, szB, szC);
  k.a = reinterpret_cast<T *>(k.key + off[0]);
  k.b = reinterpret_cast<T *>(k.key + off[1]);
  k.c = reinterpret_cast<T *>(k.key + off[2]);
  if (t != TruncateType::None) k.tr = mpcx_ezpc::trunc_read<T>(t, kb);
  k.tr.t = t;
  return k;
}
// d_A, d_B: masked public operands; returns the masked product (truncated by t).
template <typename T>
inline T *gpuMul(SigmaPeer *peer, int party, int bw, int scale, int N, GPUMulKey<T> k, T *d_A, T *d_B, TruncateType t,
                 AESGlobalContext *, Stats *) {
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(bw), scale);
  const size_t n = size_t(N);
  const uint32_t *id = mpcx_ezpc::iota(n);
  T *z = reinterpret_cast<T *>(gpuMalloc(n * sizeof(T)));
  {
    mpcx_ezpc::ScopedKey key(k.key, k.bytes);
    mpcx_ezpc::check(c, mpcx_party_mul_eval(c, mpcx_ezpc::peer_of(peer, party), n, n, n, id, id, key.get(), d_A, d_B,
                                            z),
                     "gpuMul");
  }
  if (t == TruncateType::None) return z;
  T *y = mpcx_ezpc::trunc_eval<T>(peer, party, k.tr, z);
  gpuFree(z);
  return y;
}

// ===========================================================================
// ring GEMMs (stdInit / gpuKeygenMatmul / readGPUMatmulKey / gpuMatmul,
// ddg_orca_base.h:175-198, 248-263, 394-465)
// ===========================================================================
struct MatmulParams {
  int bw = 0, shift = 0;
  int M = 0, K = 0, N = 0, batchSz = 1;
  u64 size_A = 0, size_B = 0, size_C = 0;
};
inline void stdInit(MatmulParams &p, int bw, int shift) {
  p.bw = bw;
  p.shift = shift;
  p.size_A = u64(p.batchSz) * p.M * p.K;
  p.size_B = u64(p.batchSz) * p.K * p.N;
  p.size_C = u64(p.batchSz) * p.M * p.N;
}
template <typename T>
struct GPUMatmulKey {
  MatmulParams p;
  bool sxs = false;
  T *A = nullptr, *B = nullptr, *C = nullptr;  // this party's shares of the masks of A and B, its C / output-mask share
  u64 mem_size_A = 0, mem_size_B = 0, mem_size_C = 0;
  u8 *key = nullptr;
  size_t bytes = 0;
};
// wIsOnGpu: B is secret with the device mask maskB (Beaver, SxS); otherwise B is
// public with mask zero (maskB ignored) and the product is the Beaver product
// with that zero mask (one exchange; output mask fresh).
template <typename T>
inline T *gpuKeygenMatmul(u8 **kb, int party, MatmulParams p, T *d_maskA, T *maskB, T *bias, TruncateType t,
                          AESGlobalContext *, bool wIsOnGpu) {
  if (t != TruncateType::None) mpcx_ezpc::die("gpuKeygenMatmul: truncation is a separate gate");
  (void)bias;
  const int bw = mpcx_ezpc::bw_of<T>(p.bw);
  mpcx_ctx *c = mpcx_ezpc::ctx(bw);
  T *out = reinterpret_cast<T *>(gpuMalloc(p.size_C * sizeof(T)));
  if (wIsOnGpu) {
    mpcx_ezpc::KeyPair kp(mpcx_sxs_key_bytes(c, p.batchSz, p.M, p.K, p.N));
    mpcx_ezpc::check(c, mpcx_sxs_keygen(c, p.batchSz, p.M, p.K, p.N, d_maskA, maskB, out, mpcx_ezpc::seed(),
                                        mpcx_ezpc::next_gate(), kp.k[0], kp.k[1]),
                     "gpuKeygenMatmul");
    mpcx_ezpc::append(kb, mpcx_ezpc::R_SXS, {p.batchSz, p.M, p.K, p.N}, {{kp.k[party], kp.bytes}});
    return out;
  }
  // public B: shares of r_A and of the fresh output mask
  T *ra[2], *rz[2];
  for (int q = 0; q < 2; q++) {
    ra[q] = reinterpret_cast<T *>(gpuMalloc(p.size_A * sizeof(T)));
    rz[q] = reinterpret_cast<T *>(gpuMalloc(p.size_C * sizeof(T)));
  }
  T *r = randomGEOnGpu<T>(p.size_C, bw);
  mpcx_ezpc::hip_check(hipMemcpy(out, r, p.size_C * sizeof(T), hipMemcpyDeviceToDevice), "gpuKeygenMatmul");
  gpuFree(r);
  mpcx_ezpc::split<T>(c, p.size_A, d_maskA, ra[0], ra[1]);
  mpcx_ezpc::split<T>(c, p.size_C, out, rz[0], rz[1]);
  mpcx_ezpc::append(kb, mpcx_ezpc::R_SXP, {p.batchSz, p.M, p.K, p.N},
                    {{ra[party], p.size_A * sizeof(T)}, {rz[party], p.size_C * sizeof(T)}});
  for (int q = 0; q < 2; q++) {
    gpuFree(ra[q]);
    gpuFree(rz[q]);
  }
  return out;
}
template <typename T>
inline GPUMatmulKey<T> readGPUMatmulKey(MatmulParams p, TruncateType t, u8 **kb) {
  if (t != TruncateType::None) mpcx_ezpc::die("readGPUMatmulKey: truncation is a separate gate");
  mpcx_ezpc::Hdr h;
  std::memcpy(&h, *kb, sizeof h);
  const bool sxs = h.type == mpcx_ezpc::R_SXS;
  auto r = mpcx_ezpc::take(kb, sxs ? mpcx_ezpc::R_SXS : mpcx_ezpc::R_SXP, "readGPUMatmulKey");
  if (r.h.p[0] != p.batchSz || r.h.p[1] != p.M || r.h.p[2] != p.K || r.h.p[3] != p.N)
    mpcx_ezpc::die("readGPUMatmulKey: key of another product");
  GPUMatmulKey<T> k;
  k.p = p;
  k.sxs = sxs;
  k.key = r.payload;
  k.mem_size_A = p.size_A * sizeof(T);
  k.mem_size_B = p.size_B * sizeof(T);
  k.mem_size_C = p.size_C * sizeof(T);
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(p.bw));
  if (sxs) {
    size_t off[3];
    mpcx_ezpc::check(c, mpcx_sxs_key_layout(c, p.batchSz, p.M, p.K, p.N, off), "readGPUMatmulKey");
    k.bytes = mpcx_sxs_key_bytes(c, p.batchSz, p.M, p.K, p.N);
    k.A = reinterpret_cast<T *>(k.key + off[0]);
    k.B = reinterpret_cast<T *>(k.key + off[1]);
    k.C = reinterpret_cast<T *>(k.key + off[2]);
  } else {
    k.bytes = r.h.payload;
    k.A = reinterpret_cast<T *>(k.key);
    k.C = reinterpret_cast<T *>(k.key + mpcx_ezpc::pad256(k.mem_size_A));
  }
  return k;
}
// d_A: masked public A; B: the masked public B (device, wIsOnGpu) or the public
// weights (host or device); bias (N, at the product's scale) added once.
template <typename T>
inline T *gpuMatmul(SigmaPeer *peer, int party, MatmulParams p, GPUMatmulKey<T> k, T *d_A, T *B, T *bias,
                    TruncateType t, AESGlobalContext *, Stats *s, bool wIsOnGpu, T *d_maskA) {
  (void)d_maskA;
  if (t != TruncateType::None) mpcx_ezpc::die("gpuMatmul: truncation is a separate gate");
  mpcx_ctx *c = mpcx_ezpc::ctx(mpcx_ezpc::bw_of<T>(p.bw));
  mpcx_peer *pe = mpcx_ezpc::peer_of(peer, party);
  T *out = reinterpret_cast<T *>(gpuMalloc(p.size_C * sizeof(T)));
  if (k.sxs) {
    if (!wIsOnGpu) mpcx_ezpc::die("gpuMatmul: a secret-secret key needs B on the device");
    mpcx_ezpc::ScopedKey key(k.key, k.bytes);
    mpcx_ezpc::check(c, mpcx_party_sxs_eval(c, pe, p.batchSz, p.M, p.K, p.N, key.get(), d_A, B, out), "gpuMatmul");
  } else {
    if (p.batchSz != 1) mpcx_ezpc::die("gpuMatmul: public weights with one batch");
    // party p's share of A.W + r_Z: ([p = 0] A^ - RA_p) . W + RZ_p (+ bias on party 0)
    mpcx_ezpc::DevKey W = mpcx_ezpc::on_device(B, k.mem_size_B);
    const T *dW = reinterpret_cast<const T *>(W.d);
    mpcx_ezpc::ScopedKey key(k.key, k.bytes);
    const T *RA = reinterpret_cast<const T *>(key.get());
    const T *RZ = reinterpret_cast<const T *>(key.get() + mpcx_ezpc::pad256(k.mem_size_A));
    T *D = reinterpret_cast<T *>(gpuMalloc(k.mem_size_A));
    mpcx_ezpc::check(c, mpcx_ring_lincomb(c, p.size_A, 1, party == SERVER0 ? 1 : 0, d_A, uint64_t(0) - 1, RA,
                                          nullptr, 0, D),
                     "gpuMatmul");
    mpcx_ezpc::check(c, mpcx_ring_gemm(c, p.M, p.K, p.N, D, dW, out), "gpuMatmul");
    mpcx_ezpc::check(c, mpcx_ring_lincomb(c, size_t(p.M), size_t(p.N), 1, out, 1, RZ,
                                          party == SERVER0 ? bias : nullptr, 0, out),
                     "gpuMatmul");
    mpcx_ezpc::check(c, mpcx_party_reconstruct(c, pe, p.size_C, out), "gpuMatmul");
    gpuFree(D);
    mpcx_ezpc::key_release(W);
  }
  return out;
}
