// capi.hip -- extern "C" entry points of libmpcx (declared in include/mpcx.h).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "../../include/mpcx.h"
#include "gemm.h"
#include "kernels.h"
#include "model.h"
#include "mpcx_core.h"
#include "peer.h"

// ---------------------------------------------------------------------------
// dealer and party keys (the S-box and key schedule are mpcx_core.h's)
// ---------------------------------------------------------------------------
namespace mpcx {

// FIPS-197 encryption of one block on the host (columns as little-endian words,
// the device code's state layout); used only to derive the parties' PRF keys.
static void aes_encrypt_host(const AesRK &rk, const uint32_t in[4], uint32_t out[4]) {
  auto xt = [](uint8_t a) { return uint8_t((a << 1) ^ ((a & 0x80) ? 0x1b : 0)); };
  uint8_t st[16];
  for (int j = 0; j < 4; j++)
    for (int b = 0; b < 4; b++) st[4 * j + b] = uint8_t((in[j] ^ rk.w[j]) >> (8 * b));
  for (int r = 1; r <= 10; r++) {
    uint8_t u[16];
    for (int j = 0; j < 4; j++)  // SubBytes + ShiftRows: row b of column j from column j + b
      for (int b = 0; b < 4; b++) u[4 * j + b] = kSboxC[st[4 * ((j + b) & 3) + b]];
    if (r < 10)
      for (int j = 0; j < 4; j++) {  // MixColumns
        const uint8_t a0 = u[4 * j], a1 = u[4 * j + 1], a2 = u[4 * j + 2], a3 = u[4 * j + 3];
        u[4 * j + 0] = uint8_t(xt(a0) ^ xt(a1) ^ a1 ^ a2 ^ a3);
        u[4 * j + 1] = uint8_t(a0 ^ xt(a1) ^ xt(a2) ^ a2 ^ a3);
        u[4 * j + 2] = uint8_t(a0 ^ a1 ^ xt(a2) ^ xt(a3) ^ a3);
        u[4 * j + 3] = uint8_t(xt(a0) ^ a0 ^ a1 ^ a2 ^ xt(a3));
      }
    for (int j = 0; j < 4; j++)
      for (int b = 0; b < 4; b++) st[4 * j + b] = uint8_t(u[4 * j + b] ^ (rk.w[4 * r + j] >> (8 * b)));
  }
  for (int j = 0; j < 4; j++)
    out[j] = uint32_t(st[4 * j]) | (uint32_t(st[4 * j + 1]) << 8) | (uint32_t(st[4 * j + 2]) << 16) |
             (uint32_t(st[4 * j + 3]) << 24);
}

static void words_to_bytes(const uint32_t w[4], uint8_t out[16]) {
  for (int j = 0; j < 4; j++)
    for (int b = 0; b < 4; b++) out[4 * j + b] = uint8_t(w[j] >> (8 * b));
}

AesRK dealer_key(const Launch &L, uint64_t seed) {
  uint8_t k[16];
  if (L.has_dealer_key) {
    const uint32_t in[4] = {uint32_t(seed), uint32_t(seed >> 32), 0x4D415354u, 0xFFFFFFFEu};
    uint32_t w[4];
    aes_encrypt_host(aes_expand(L.dealer_key), in, w);
    words_to_bytes(w, k);
  } else {
    const uint64_t a = seed, b = seed ^ 0x9E3779B97F4A7C15ull;
    for (int i = 0; i < 8; i++) {
      k[i] = uint8_t(a >> (8 * i));
      k[8 + i] = uint8_t(b >> (8 * i));
    }
  }
  return aes_expand(k);
}

void party_key_bytes(const Launch &L, uint64_t seed, int party, uint8_t out[16]) {
  const AesRK kd = dealer_key(L, seed);
  const uint32_t in[4] = {uint32_t(party), 0u, uint32_t(F_PARTY), 0xFFFFFFFFu};
  uint32_t w[4];
  aes_encrypt_host(kd, in, w);
  words_to_bytes(w, out);
}

AesRK party_key(const Launch &L, uint64_t seed, int party) {
  uint8_t k[16];
  party_key_bytes(L, seed, party, k);
  return aes_expand(k);
}

}  // namespace mpcx

using namespace mpcx;

struct mpcx_ctx {
  int bw = 32, s = 12, device = 0;
  hipStream_t own = nullptr;
  Launch L;
  Counters counters;
  std::string err;
  // Device workspace of the standalone gate evaluations, grown on demand and
  // kept until the context is destroyed (every such call synchronizes its
  // stream before returning, so the next call may reuse it).
  void *work = nullptr;
  size_t work_bytes = 0;
  // this device's copy of the static scratch array (mpcx_maxpool_eval_noalloc)
  void *noalloc_scratch = nullptr;
  hipError_t noalloc_err = hipSuccess;
  hipEvent_t noalloc_done = nullptr;  // recorded after each of this context's calls on the array
  PartyWork *party = nullptr;   // workspace of the party-mode gate calls
  AdjNormCache *adj = nullptr;  // prepared state of mpcx_adjnorm_eval
  int adj_lanes = 1;            // concurrent graph groups of the adjacency normalisation
};

struct mpcx_model {
  mpcx_ctx *ctx = nullptr;
  LaneSet *impl = nullptr;
};

struct mpcx_peer {
  Peer *impl = nullptr;
};

static mpcx_status fail(mpcx_ctx *c, mpcx_status st, const std::string &msg) {
  if (c) c->err = msg;
  return st;
}
static mpcx_status hip_status(mpcx_ctx *c, hipError_t e, const char *what) {
  if (e == hipSuccess) return MPCX_OK;
  std::string m = std::string(what) + ": " + hipGetErrorString(e);
  if (e == hipErrorOutOfMemory) return fail(c, MPCX_ENOMEM, m);
  if (e == hipErrorInvalidValue) return fail(c, MPCX_EINVAL, m);
  return fail(c, MPCX_EHIP, m);
}
#define CHECK_CTX(c)                  \
  do {                                \
    if (!(c)) return MPCX_EINVAL;     \
  } while (0)
#define HIPC(c, x, what)                                   \
  do {                                                     \
    hipError_t e_ = (x);                                   \
    if (e_ != hipSuccess) return hip_status(c, e_, what);  \
  } while (0)

// C++ exceptions (allocation failures of host-side plans and threads) must not
// cross the C ABI: model calls run through these guards.
template <class F>
static hipError_t guard(F &&f) noexcept {
  try {
    return f();
  } catch (const std::bad_alloc &) {
    return hipErrorOutOfMemory;
  } catch (...) {
    return hipErrorUnknown;
  }
}
template <class F>
static size_t guard_size(F &&f) noexcept {
  try {
    return f();
  } catch (...) {
    return 0;
  }
}

// ---------------- allocation-free max-pool ----------------
// mpcx_maxpool_eval_noalloc runs the same kernels as mpcx_maxpool_eval on a
// workspace that is never allocated at call time: the file-scope device array
// `scratch` below, one copy per GPU, loaded with the library's code object and
// held until the process ends.  Its per-device address is looked up once per
// device by mpcx_create (noalloc_scratch_resolve) and kept in g_scratch_addr;
// host code uses only that address, never the array's name (which names a
// host-side stand-in).  Every level plane is written before it is read, so
// nothing in the array has to start at zero.  The array's last user on each
// device (its stream and the event its context recorded after the call) is
// kept in g_scratch_stream / g_scratch_event: a call from another stream while
// that event is pending is refused (MPCX_EBUSY) instead of racing on the array.
static __device__ __align__(256) unsigned char scratch[MPCX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_addr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
bool g_scratch_done[kMaxDevices];
hipStream_t g_scratch_stream[kMaxDevices];
hipEvent_t g_scratch_event[kMaxDevices];  // the owner context's noalloc_done (null: none)

// With `device` current: look up the device's copy of `scratch` (once per device).
hipError_t noalloc_scratch_resolve(int device, void **out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_done[device]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_err[device] = e;
    g_scratch_addr[device] = e == hipSuccess ? ptr : nullptr;
    g_scratch_done[device] = true;
  }
  *out = g_scratch_addr[device];
  return g_scratch_err[device];
}
}  // namespace

// All entry points below were declared extern "C" in mpcx.h and keep C linkage.

mpcx_status mpcx_create(int bw, int scale, int device, mpcx_ctx **out) {
  if (!out || (bw != 32 && bw != 64) || scale < 1 || scale > bw / 2 - 2) return MPCX_EINVAL;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return MPCX_EHIP;
  if (device < 0 || device >= ndev) return MPCX_EINVAL;
  if (hipSetDevice(device) != hipSuccess) return MPCX_EHIP;
  auto *c = new mpcx_ctx();
  c->bw = bw;
  c->s = scale;
  c->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->L.num_cu = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return MPCX_EHIP;
  }
  c->L.stream = c->own;
  c->noalloc_err = noalloc_scratch_resolve(device, &c->noalloc_scratch);
  if (hipEventCreateWithFlags(&c->noalloc_done, hipEventDisableTiming) != hipSuccess) {
    (void)hipStreamDestroy(c->own);
    delete c;
    return MPCX_EHIP;
  }
  // The environment overrides take the same checks as mpcx_set_aes_variant: a
  // bad value is ignored with a warning (a block that is not a whole number of
  // wave pairs would misplace the DCF kernels' ballot words).
  {
    int variant = 0, block = 0;
    if (const char *v = std::getenv("MPCX_AES_VARIANT")) variant = std::atoi(v);
    if (const char *v = std::getenv("MPCX_AES_BLOCK")) block = std::atoi(v);
    if (mpcx_set_aes_variant(c, variant, block) != MPCX_OK) {
      std::fprintf(stderr, "libmpcx: ignoring MPCX_AES_VARIANT=%d / MPCX_AES_BLOCK=%d: %s\n", variant, block,
                   c->err.c_str());
      c->err.clear();
      c->L.aes_variant = 0;
      c->L.aes_block = 0;
    }
  }
  if (const char *v = std::getenv("MPCX_GEMM")) {
    if (std::strcmp(v, "valu") == 0) c->L.gemm = 1;
    else if (std::strcmp(v, "tiled") == 0) c->L.gemm = 2;
    else if (std::strcmp(v, "wide") == 0) c->L.gemm = 3;
    else if (std::strcmp(v, "auto") == 0 || !*v) c->L.gemm = 0;
    else std::fprintf(stderr, "libmpcx: ignoring MPCX_GEMM=%s (auto, wide, tiled or valu)\n", v);
  }
  if (const char *v = std::getenv("MPCX_GRAPH")) c->L.graph = std::atoi(v) != 0 ? 1 : 0;
  if (const char *v = std::getenv("MPCX_POOL_TAIL")) c->L.pool_tail = std::max(-1, std::atoi(v));
  if (const char *v = std::getenv("MPCX_PANEL_PF")) c->L.panel_pf = std::atoi(v) != 0 ? 1 : 0;
  if (const char *v = std::getenv("MPCX_QUAD_PER_CU")) c->L.quad_per_cu = std::max(64, std::min(256, std::atoi(v)));
  if (const char *v = std::getenv("MPCX_QUAD_ALONE")) c->L.quad_alone = std::max(64, std::min(256, std::atoi(v)));
  if (const char *v = std::getenv("MPCX_PANEL_NT")) c->L.panel_nt = std::max(0, std::min(3, std::atoi(v)));
  if (const char *v = std::getenv("MPCX_SXS_STAGED")) c->L.sxs_staged = std::atoi(v) != 0 ? 1 : 0;
  *out = c;
  return MPCX_OK;
}

void mpcx_destroy(mpcx_ctx *c) {
  if (!c) return;
  if (c->noalloc_done) {  // no longer the scratch array's owner once its last call is done
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    (void)hipEventSynchronize(c->noalloc_done);
    if (c->device >= 0 && c->device < kMaxDevices && g_scratch_event[c->device] == c->noalloc_done) {
      g_scratch_event[c->device] = nullptr;
      g_scratch_stream[c->device] = nullptr;
    }
    (void)hipEventDestroy(c->noalloc_done);
  }
  if (c->own) {
    (void)hipStreamSynchronize(c->own);
    (void)hipStreamDestroy(c->own);
  }
  if (c->work) (void)hipFree(c->work);
  party_work_free(c->party);
  adjnorm_cache_free(c->adj);
  delete c;
}

const char *mpcx_last_error(const mpcx_ctx *c) { return c ? c->err.c_str() : "null context"; }
int mpcx_bw(const mpcx_ctx *c) { return c ? c->bw : 0; }
int mpcx_scale(const mpcx_ctx *c) { return c ? c->s : 0; }

mpcx_status mpcx_set_stream(mpcx_ctx *c, void *s) {
  CHECK_CTX(c);
  c->L.stream = s ? static_cast<hipStream_t>(s) : c->own;
  return MPCX_OK;
}

mpcx_status mpcx_set_party_sync(mpcx_ctx *c, int sync) {
  CHECK_CTX(c);
  c->L.party_sync = sync != 0 ? 1 : 0;
  return MPCX_OK;
}

mpcx_status mpcx_synchronize(mpcx_ctx *c) {
  CHECK_CTX(c);
  HIPC(c, hipStreamSynchronize(c->L.stream), "hipStreamSynchronize");
  return MPCX_OK;
}

int mpcx_aes_variant_count(void) {
  int n;
  aes_variants(&n);
  return n;
}
const char *mpcx_aes_variant_name(int i) {
  int n;
  const AesVariant *v = aes_variants(&n);
  return (i >= 0 && i < n) ? v[i].name : "";
}
int mpcx_aes_variant(const mpcx_ctx *c) { return c ? c->L.aes_variant : -1; }

mpcx_status mpcx_set_aes_variant(mpcx_ctx *c, int variant, int block) {
  CHECK_CTX(c);
  if (variant < 0 || variant >= mpcx_aes_variant_count()) return fail(c, MPCX_EINVAL, "bad AES variant");
  // the gate kernel splits a workgroup into two parties' halves of whole waves
  if (block != 0 && (block < 128 || block > 1024 || (block % 128) != 0))
    return fail(c, MPCX_EINVAL, "block must be a multiple of 128 in [128, 1024]");
  c->L.aes_variant = variant;
  c->L.aes_block = block;
  return MPCX_OK;
}

mpcx_status mpcx_set_both_party_aes(mpcx_ctx *c, int max_aes) {
  CHECK_CTX(c);
  if (max_aes < 0 || max_aes > 64) return fail(c, MPCX_EINVAL, "max_aes must be in [0, 64]");
  c->L.both_aes = max_aes;
  return MPCX_OK;
}

mpcx_status mpcx_set_dealer_key(mpcx_ctx *c, const uint8_t *key) {
  CHECK_CTX(c);
  c->L.has_dealer_key = key != nullptr;
  for (int i = 0; i < 16; i++) c->L.dealer_key[i] = key ? key[i] : 0;
  return MPCX_OK;
}

uint64_t mpcx_bytes_exchanged(const mpcx_ctx *c) { return c ? c->counters.bytes : 0; }
uint64_t mpcx_rounds(const mpcx_ctx *c) { return c ? c->counters.rounds : 0; }
void mpcx_reset_counters(mpcx_ctx *c) {
  if (c) c->counters = Counters();
}

// ---------------- PRG ----------------
mpcx_status mpcx_prg_hash(mpcx_ctx *c, int leaf, size_t n, const void *in, void *out) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!in || !out) return fail(c, MPCX_EINVAL, "null pointer");
  HIPC(c, launch_hash(c->L, leaf, n, static_cast<const uint4 *>(in), static_cast<uint4 *>(out)), "prg_hash");
  return MPCX_OK;
}
mpcx_status mpcx_prf(mpcx_ctx *c, uint64_t seed, uint32_t gate, uint32_t field, size_t n, void *out) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!out) return fail(c, MPCX_EINVAL, "null pointer");
  HIPC(c, launch_prf(c->L, seed, gate, field, n, static_cast<uint4 *>(out)), "prf");
  return MPCX_OK;
}

// ---------------- DCF ----------------
size_t mpcx_dcf_key_bytes(int bin, size_t n) { return dcf_layout(bin, n, 0, true).end; }

mpcx_status mpcx_dcf_keygen(mpcx_ctx *c, int bin, size_t n, const uint64_t *alpha, const uint8_t *rbit,
                            uint64_t seed, uint32_t gate, void *k0, void *k1) {
  CHECK_CTX(c);
  if (bin < 1 || bin > 64) return fail(c, MPCX_EINVAL, "dcf_keygen: bad argument");
  if (n == 0) return MPCX_OK;
  if (!alpha || !k0 || !k1) return fail(c, MPCX_EINVAL, "dcf_keygen: null pointer");
  HIPC(c,
       launch_dcf_keygen(c->L, seed, gate, F_DCFA, bin, n, alpha, rbit, static_cast<uint8_t *>(k0),
                         static_cast<uint8_t *>(k1), 0),
       "dcf_keygen");
  return MPCX_OK;
}

mpcx_status mpcx_dcf_eval(mpcx_ctx *c, int party, int bin, size_t n, const void *key, const uint64_t *x,
                          uint64_t *out) {
  CHECK_CTX(c);
  if (bin < 1 || bin > 64 || (party != 0 && party != 1)) return fail(c, MPCX_EINVAL, "dcf_eval: bad argument");
  if (n == 0) return MPCX_OK;
  if (!key || !x || !out) return fail(c, MPCX_EINVAL, "dcf_eval: null pointer");
  HIPC(c, launch_dcf_eval(c->L, party, bin, n, static_cast<const uint8_t *>(key), 0, x, out), "dcf_eval");
  return MPCX_OK;
}

mpcx_status mpcx_dcf_eval_ring(mpcx_ctx *c, int party, int bin, size_t n, const void *key, const void *x,
                               const uint32_t *mask, uint64_t *out) {
  CHECK_CTX(c);
  if (bin < 1 || bin > c->bw || (party != 0 && party != 1)) return fail(c, MPCX_EINVAL, "dcf_eval_ring: bad argument");
  if (n == 0) return MPCX_OK;
  if (!key || !x || !out) return fail(c, MPCX_EINVAL, "dcf_eval_ring: null pointer");
  const uint8_t *k = static_cast<const uint8_t *>(key);
  HIPC(c,
       c->bw == 32 ? launch_dcf_eval_ring<uint32_t>(c->L, bin, n, k, static_cast<const uint32_t *>(x), mask, out)
                   : launch_dcf_eval_ring<uint64_t>(c->L, bin, n, k, static_cast<const uint64_t *>(x), mask, out),
       "dcf_eval_ring");
  return MPCX_OK;
}

// ---------------- workspace for standalone gate evaluation ----------------
namespace {
hipError_t ctx_work(mpcx_ctx *c, size_t bytes, void **p) {
  if (bytes > c->work_bytes) {
    if (c->work) {
      hipError_t e = hipDeviceSynchronize();
      if (e != hipSuccess) return e;
      (void)hipFree(c->work);
      c->work = nullptr;
      c->work_bytes = 0;
    }
    hipError_t e = hipMalloc(&c->work, bytes);
    if (e != hipSuccess) return e;
    c->work_bytes = bytes;
  }
  *p = c->work;
  return hipSuccess;
}
static_assert(MPCX_TR == G_TR && MPCX_TRRELU == G_TRRELU && MPCX_RELU == G_RELU && MPCX_TRSLACK == G_TRSLACK &&
                  MPCX_RELUSLACK == G_RELUSLACK && MPCX_LOCALARS == G_LOCALARS && MPCX_DRELU == G_DRELU &&
                  MPCX_TRMOD == G_TRMOD && MPCX_EXT == G_EXT && MPCX_EXTRELU == G_EXTRELU &&
                  MPCX_RELUPOOL == G_RELUPOOL,
              "the C API's gate kinds are the library's");
bool valid_kind(int k) {
  return k == MPCX_TR || k == MPCX_TRRELU || k == MPCX_RELU || k == MPCX_TRSLACK || k == MPCX_RELUSLACK ||
         k == MPCX_LOCALARS || k == MPCX_DRELU || k == MPCX_TRMOD || k == MPCX_EXT || k == MPCX_EXTRELU ||
         k == MPCX_RELUPOOL;
}
}  // namespace

size_t mpcx_tr_key_bytes(mpcx_ctx *c, int kind, size_t n) {
  if (!c || !valid_kind(kind)) return 0;
  return tr_layout(kind, c->bw, c->s, n, 0).end;
}

int mpcx_tr_eval_form(const mpcx_ctx *c, int kind, size_t n) {
  if (!c || !valid_kind(kind) || kind == MPCX_LOCALARS) return -1;
  static_assert(MPCX_FORM_ONE_LANE == kFormOneLane && MPCX_FORM_BOTH == kFormBoth && MPCX_FORM_QUAD == kFormQuad,
                "form codes");
  return tr_eval_form(c->L, tr_layout(kind, c->bw, c->s, n, 0));
}

int mpcx_tr_aes_calls(const mpcx_ctx *c, int kind) {
  if (!c || !valid_kind(kind)) return -1;
  const TrLayout lay = tr_layout(kind, c->bw, c->s, 1, 0);
  return (lay.use_a ? lay.a.L + 1 : 0) + (lay.use_b ? lay.b.L + 1 : 0);
}

template <typename T>
static mpcx_status tr_keygen_t(mpcx_ctx *c, int kind, size_t n, const void *in, void *out, uint64_t seed,
                               uint32_t gate, void *k0, void *k1) {
  if (kind == MPCX_LOCALARS) {  // no key: the output mask is the shifted input mask
    HIPC(c, launch_local_ars<T>(c->L, n, c->s, static_cast<const T *>(in), nullptr, 1, static_cast<T *>(out)),
         "tr_keygen");
    HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
    return MPCX_OK;
  }
  TrLayout lay = tr_layout(kind, c->bw, c->s, n, 0);
  HIPC(c,
       launch_tr_keygen<T>(c->L, lay, seed, gate, static_cast<const T *>(in), static_cast<T *>(out),
                           static_cast<uint8_t *>(k0), static_cast<uint8_t *>(k1)),
       "tr_keygen");
  return MPCX_OK;
}

mpcx_status mpcx_tr_keygen(mpcx_ctx *c, int kind, size_t n, const void *in, void *out, uint64_t seed, uint32_t gate,
                           void *k0, void *k1) {
  CHECK_CTX(c);
  if (!valid_kind(kind)) return fail(c, MPCX_EINVAL, "tr_keygen: bad gate kind");
  if (n == 0) return MPCX_OK;
  if (!in || !out || (kind != MPCX_LOCALARS && (!k0 || !k1))) return fail(c, MPCX_EINVAL, "tr_keygen: null pointer");
  return c->bw == 32 ? tr_keygen_t<uint32_t>(c, kind, n, in, out, seed, gate, k0, k1)
                     : tr_keygen_t<uint64_t>(c, kind, n, in, out, seed, gate, k0, k1);
}

// One TR-family gate evaluation of both parties into y (no synchronisation).
template <typename T>
static hipError_t tr_eval_run(mpcx_ctx *c, const TrLayout &lay, size_t n, const uint8_t *K0, const uint8_t *K1,
                              const T *X, const T *Bi, int ncol, T *y) {
  hipError_t e = launch_tr_eval<T>(c->L, lay, K0, K1, X, Bi, ncol, y);
  if (e != hipSuccess) return e;
  c->counters.bitplanes(n, int(lay.use_a) + int(lay.use_b));
  if (lay.kind != MPCX_DRELU)  // DRELU: the output bit is already public
    c->counters.msg_bits(n, tr_out_bits(lay.kind, c->bw, c->s), c->bw);
  return hipSuccess;
}

template <typename T>
static mpcx_status tr_eval_t(mpcx_ctx *c, int kind, size_t n, const void *k0, const void *k1, const void *x,
                             const void *bias, int ncol, void *y) {
  if (kind == MPCX_LOCALARS) {  // local: no key, no exchange
    HIPC(c,
         launch_local_ars<T>(c->L, n, c->s, static_cast<const T *>(x), static_cast<const T *>(bias), ncol,
                             static_cast<T *>(y)),
         "tr_eval");
    HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
    return MPCX_OK;
  }
  TrLayout lay = tr_layout(kind, c->bw, c->s, n, 0);
  HIPC(c,
       tr_eval_run<T>(c, lay, n, static_cast<const uint8_t *>(k0), static_cast<const uint8_t *>(k1),
                      static_cast<const T *>(x), static_cast<const T *>(bias), ncol, static_cast<T *>(y)),
       "tr_eval");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}

mpcx_status mpcx_tr_eval(mpcx_ctx *c, int kind, size_t n, const void *k0, const void *k1, const void *x,
                         const void *bias, int ncol, void *y) {
  CHECK_CTX(c);
  if (!valid_kind(kind) || (bias && ncol < 1)) return fail(c, MPCX_EINVAL, "tr_eval: bad argument");
  if (n == 0) return MPCX_OK;
  if ((kind != MPCX_LOCALARS && (!k0 || !k1)) || !x || !y) return fail(c, MPCX_EINVAL, "tr_eval: null pointer");
  return c->bw == 32 ? tr_eval_t<uint32_t>(c, kind, n, k0, k1, x, bias, ncol, y)
                     : tr_eval_t<uint64_t>(c, kind, n, k0, k1, x, bias, ncol, y);
}

// ---------------- masked max-pool ----------------
namespace {
constexpr int kMaxPoolLevels = 32;
bool maxpool_dims_ok(int B, int N, int C) { return B >= 1 && N >= 1 && C >= 1; }
// the key of level l: a RELU gate over B * pairs[l] * C differences, back to back
int maxpool_plan(const mpcx_ctx *c, int B, int N, int C, TrLayout *lay, int *pairs) {
  const int Lv = pool_levels(N, pairs);
  size_t o = 0;
  for (int l = 0; l < Lv; l++) {
    lay[l] = tr_layout(MPCX_RELU, c->bw, c->s, size_t(B) * pairs[l] * C, o);
    o = lay[l].end;
  }
  return Lv;
}
}  // namespace

int mpcx_maxpool_levels(int N) {
  int pairs[kMaxPoolLevels];
  return N >= 1 ? pool_levels(N, pairs) : 0;
}

size_t mpcx_maxpool_key_bytes(mpcx_ctx *c, int B, int N, int C) {
  if (!c || !maxpool_dims_ok(B, N, C)) return 0;
  TrLayout lay[kMaxPoolLevels];
  int pairs[kMaxPoolLevels];
  const int Lv = maxpool_plan(c, B, N, C, lay, pairs);
  return Lv ? lay[Lv - 1].end : 0;
}

// The dealer runs the evaluator's linear steps on the masks: the difference of a
// pair has mask r_odd - r_even, the ReLU gate returns a fresh output mask r_y,
// and the pair's maximum has mask r_even + r_y.
template <typename T>
static mpcx_status maxpool_keygen_t(mpcx_ctx *c, int B, int N, int C, const void *in_mask, void *out_mask,
                                    uint64_t seed, uint32_t gate, void *k0, void *k1) {
  TrLayout lay[kMaxPoolLevels];
  int pairs[kMaxPoolLevels];
  const int Lv = maxpool_plan(c, B, N, C, lay, pairs);
  const size_t rows = size_t(B) * N * C, P0 = Lv ? size_t(B) * pairs[0] * C : 0;
  void *sp = nullptr;
  HIPC(c, ctx_work(c, (2 * rows + 2 * P0) * sizeof(T), &sp), "hipMalloc");
  T *va = static_cast<T *>(sp), *vb = va + rows, *dm = vb + rows, *ym = dm + P0;
  const T *cur = static_cast<const T *>(in_mask);
  T *nxt = va;
  uint8_t *K0 = static_cast<uint8_t *>(k0), *K1 = static_cast<uint8_t *>(k1);
  int R = N;
  for (int l = 0; l < Lv; l++) {
    HIPC(c, launch_pool_diff<T>(c->L, B, R, C, cur, dm), "maxpool_keygen");
    HIPC(c, launch_tr_keygen<T>(c->L, lay[l], seed, gate + uint32_t(l), dm, ym, K0, K1), "maxpool_keygen");
    HIPC(c, launch_pool_combine<T>(c->L, B, R, C, cur, ym, nullptr, nxt), "maxpool_keygen");
    cur = nxt;
    nxt = nxt == va ? vb : va;
    R = pairs[l] + (R & 1);
  }
  HIPC(c, hipMemcpyAsync(out_mask, cur, size_t(B) * C * sizeof(T), hipMemcpyDeviceToDevice, c->L.stream),
       "maxpool_keygen");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}

mpcx_status mpcx_maxpool_keygen(mpcx_ctx *c, int B, int N, int C, const void *in_mask, void *out_mask, uint64_t seed,
                                uint32_t gate, void *k0, void *k1) {
  CHECK_CTX(c);
  if (!maxpool_dims_ok(B, N, C) || !in_mask || !out_mask || (N > 1 && (!k0 || !k1)))
    return fail(c, MPCX_EINVAL, "maxpool_keygen: bad argument");
  return c->bw == 32 ? maxpool_keygen_t<uint32_t>(c, B, N, C, in_mask, out_mask, seed, gate, k0, k1)
                     : maxpool_keygen_t<uint64_t>(c, B, N, C, in_mask, out_mask, seed, gate, k0, k1);
}

// Per level: the pair differences (local), one RELU gate (two exchange rounds),
// and max(a, b) = a + ReLU(b - a) (local), on planes (B, R, C) that shrink to
// (B, 1, C); with both parties here one gate launch per level does all three.
template <typename T>
static hipError_t maxpool_eval_run(mpcx_ctx *c, int B, int N, int C, const void *k0, const void *k1, const void *in,
                                   void *out, void *work) {
  TrLayout lay[kMaxPoolLevels];
  int pairs[kMaxPoolLevels];
  const int Lv = maxpool_plan(c, B, N, C, lay, pairs);
  const size_t rows = size_t(B) * N * C, P0 = Lv ? size_t(B) * pairs[0] * C : 0;
  T *va = static_cast<T *>(work), *vb = va + rows, *d = vb + rows, *y = d + P0;
  const T *cur = static_cast<const T *>(in);
  T *nxt = va;
  const uint8_t *K0 = static_cast<const uint8_t *>(k0), *K1 = static_cast<const uint8_t *>(k1);
  int R = N;
  for (int l = 0; l < Lv; l++) {
    const size_t n = size_t(B) * pairs[l] * C;
    hipError_t e;
    if (c->L.party < 0 && rows < (size_t(1) << 32)) {
      e = launch_tr_eval_pool<T>(c->L, lay[l], K0, K1, B, R, C, cur, nxt);
      if (e == hipSuccess) {
        c->counters.bitplanes(n, int(lay[l].use_a) + int(lay[l].use_b));
        c->counters.msg(n, c->bw);
      }
    } else {
      e = launch_pool_diff<T>(c->L, B, R, C, cur, d);
      if (e == hipSuccess) e = tr_eval_run<T>(c, lay[l], n, K0, K1, d, nullptr, 1, y);
      if (e == hipSuccess) e = launch_pool_combine<T>(c->L, B, R, C, cur, y, nullptr, nxt);
    }
    if (e != hipSuccess) return e;
    cur = nxt;
    nxt = nxt == va ? vb : va;
    R = pairs[l] + (R & 1);
  }
  return hipMemcpyAsync(out, cur, size_t(B) * C * sizeof(T), hipMemcpyDeviceToDevice, c->L.stream);
}

// Device workspace of a max-pool evaluation: the level planes (two of B x N x C,
// ping-pong) and the first level's pair differences and ReLU outputs.
static size_t maxpool_work_bytes(const mpcx_ctx *c, int B, int N, int C) {
  int pairs[kMaxPoolLevels];
  const int Lv = pool_levels(N, pairs);
  const size_t rows = size_t(B) * N * C, P0 = Lv ? size_t(B) * pairs[0] * C : 0;
  return (2 * rows + 2 * P0) * size_t(c->bw / 8);
}

template <typename T>
static mpcx_status maxpool_eval_t(mpcx_ctx *c, int B, int N, int C, const void *k0, const void *k1, const void *in,
                                  void *out) {
  void *sp = nullptr;
  HIPC(c, ctx_work(c, maxpool_work_bytes(c, B, N, C), &sp), "hipMalloc");
  HIPC(c, (maxpool_eval_run<T>(c, B, N, C, k0, k1, in, out, sp)), "maxpool_eval");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}

mpcx_status mpcx_maxpool_eval(mpcx_ctx *c, int B, int N, int C, const void *k0, const void *k1, const void *in,
                              void *out) {
  CHECK_CTX(c);
  if (!maxpool_dims_ok(B, N, C) || !in || !out || (N > 1 && (!k0 || !k1)))
    return fail(c, MPCX_EINVAL, "maxpool_eval: bad argument");
  return c->bw == 32 ? maxpool_eval_t<uint32_t>(c, B, N, C, k0, k1, in, out)
                     : maxpool_eval_t<uint64_t>(c, B, N, C, k0, k1, in, out);
}

// Allocation-free variant of mpcx_maxpool_eval on the static scratch array
// (defined with its per-device lookup above mpcx_create).
mpcx_status mpcx_maxpool_eval_noalloc(mpcx_ctx *c, int B, int N, int C, const void *k0, const void *k1,
                                      const void *in, void *out) {
  CHECK_CTX(c);
  if (!maxpool_dims_ok(B, N, C) || !in || !out || (N > 1 && (!k0 || !k1)))
    return fail(c, MPCX_EINVAL, "maxpool_eval_noalloc: bad argument");
  const size_t need = maxpool_work_bytes(c, B, N, C);
  if (need > MPCX_NOALLOC_SCRATCH_BYTES)
    return fail(c, MPCX_EINVAL,
                "maxpool_eval_noalloc: workspace of " + std::to_string(need) + " bytes exceeds the " +
                    std::to_string(size_t(MPCX_NOALLOC_SCRATCH_BYTES)) + "-byte static scratch array");
  if (!c->noalloc_scratch)
    return fail(c, MPCX_EHIP, std::string("maxpool_eval_noalloc: no scratch address on this device: ") +
                                  hipGetErrorString(c->noalloc_err));
  const int dv = c->device;
  std::lock_guard<std::mutex> lk(g_scratch_mu);  // held until this call's work and event are enqueued
  if (g_scratch_event[dv] && g_scratch_stream[dv] != c->L.stream) {
    const hipError_t q = hipEventQuery(g_scratch_event[dv]);
    if (q == hipErrorNotReady)
      return fail(c, MPCX_EBUSY,
                  "maxpool_eval_noalloc: the static scratch array is in use by a call still pending on another stream");
    HIPC(c, q, "maxpool_eval_noalloc: hipEventQuery");
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIPC(c, hipStreamIsCapturing(c->L.stream, &cs), "maxpool_eval_noalloc: hipStreamIsCapturing");
  const hipError_t e = c->bw == 32
                           ? maxpool_eval_run<uint32_t>(c, B, N, C, k0, k1, in, out, c->noalloc_scratch)
                           : maxpool_eval_run<uint64_t>(c, B, N, C, k0, k1, in, out, c->noalloc_scratch);
  HIPC(c, e, "maxpool_eval_noalloc");
  if (cs == hipStreamCaptureStatusNone) {  // captured calls run at replay: not tracked
    HIPC(c, hipEventRecord(c->noalloc_done, c->L.stream), "maxpool_eval_noalloc: hipEventRecord");
    g_scratch_stream[dv] = c->L.stream;
    g_scratch_event[dv] = c->noalloc_done;
  }
  return MPCX_OK;
}

// ---------------- MUL ----------------
size_t mpcx_mul_key_bytes(mpcx_ctx *c, size_t nx, size_t ny, size_t nz) {
  return c ? mul_layout(c->bw, nx, ny, nz, 0).end : 0;
}
template <typename T>
static mpcx_status mul_keygen_t(mpcx_ctx *c, size_t nx, size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib,
                                const void *rx, const void *ry, void *rz, uint64_t seed, uint32_t gate, void *k0,
                                void *k1) {
  MulLayout lay = mul_layout(c->bw, nx, ny, nz, 0);
  HIPC(c,
       launch_mul_keygen<T>(c->L, lay, seed, gate, MulMap::explicit_maps(ia, ib), static_cast<const T *>(rx),
                            static_cast<const T *>(ry),
                            static_cast<T *>(rz), static_cast<uint8_t *>(k0), static_cast<uint8_t *>(k1)),
       "mul_keygen");
  return MPCX_OK;
}
mpcx_status mpcx_mul_keygen(mpcx_ctx *c, size_t nx, size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib,
                            const void *rx, const void *ry, void *rz, uint64_t seed, uint32_t gate, void *k0,
                            void *k1) {
  CHECK_CTX(c);
  if (nx == 0 && ny == 0 && nz == 0) return MPCX_OK;
  if (!ia || !ib || !rx || !ry || !rz || !k0 || !k1) return fail(c, MPCX_EINVAL, "mul_keygen: null pointer");
  return c->bw == 32 ? mul_keygen_t<uint32_t>(c, nx, ny, nz, ia, ib, rx, ry, rz, seed, gate, k0, k1)
                     : mul_keygen_t<uint64_t>(c, nx, ny, nz, ia, ib, rx, ry, rz, seed, gate, k0, k1);
}
template <typename T>
static mpcx_status mul_eval_t(mpcx_ctx *c, size_t nx, size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib,
                              const void *k0, const void *k1, const void *x, const void *y, void *z) {
  MulLayout lay = mul_layout(c->bw, nx, ny, nz, 0);
  void *sp = nullptr;
  HIPC(c, ctx_work(c, 2 * nz * sizeof(T), &sp), "hipMalloc");
  T *m0 = static_cast<T *>(sp), *m1 = m0 + nz;
  HIPC(c,
       launch_mul_eval<T>(c->L, lay, static_cast<const uint8_t *>(k0), static_cast<const uint8_t *>(k1),
                          MulMap::explicit_maps(ia, ib),
                          static_cast<const T *>(x), static_cast<const T *>(y), m0, m1),
       "mul_eval");
  c->counters.msg(nz, c->bw);
  HIPC(c, launch_reconstruct<T>(c->L, nz, m0, m1, static_cast<T *>(z)), "reconstruct");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}
mpcx_status mpcx_mul_eval(mpcx_ctx *c, size_t nx, size_t ny, size_t nz, const uint32_t *ia, const uint32_t *ib,
                          const void *k0, const void *k1, const void *x, const void *y, void *z) {
  CHECK_CTX(c);
  if (nz == 0) return MPCX_OK;  // no products
  if (!ia || !ib || !k0 || !k1 || !x || !y || !z) return fail(c, MPCX_EINVAL, "mul_eval: null pointer");
  return c->bw == 32 ? mul_eval_t<uint32_t>(c, nx, ny, nz, ia, ib, k0, k1, x, y, z)
                     : mul_eval_t<uint64_t>(c, nx, ny, nz, ia, ib, k0, k1, x, y, z);
}

mpcx_status mpcx_mul_key_layout(mpcx_ctx *c, size_t nx, size_t ny, size_t nz, size_t off[3]) {
  CHECK_CTX(c);
  if (!off) return fail(c, MPCX_EINVAL, "mul_key_layout: null pointer");
  const MulLayout l = mul_layout(c->bw, nx, ny, nz, 0);
  off[0] = l.off_rx;
  off[1] = l.off_ry;
  off[2] = l.off_c;
  return MPCX_OK;
}

// ---------------- LUT8 ----------------
size_t mpcx_lut8_key_bytes(mpcx_ctx *c, size_t n) { return c ? lut8_layout(c->bw, n, 0).end : 0; }
template <typename T>
static mpcx_status lut_keygen_t(mpcx_ctx *c, size_t n, const void *in, void *out, uint64_t seed, uint32_t gate,
                                void *k0, void *k1) {
  Lut8Layout lay = lut8_layout(c->bw, n, 0);
  HIPC(c,
       launch_lut8_keygen<T>(c->L, lay, seed, gate, static_cast<const T *>(in), static_cast<T *>(out),
                             static_cast<uint8_t *>(k0), static_cast<uint8_t *>(k1)),
       "lut8_keygen");
  return MPCX_OK;
}
mpcx_status mpcx_lut8_keygen(mpcx_ctx *c, size_t n, const void *in, void *out, uint64_t seed, uint32_t gate, void *k0,
                             void *k1) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!in || !out || !k0 || !k1) return fail(c, MPCX_EINVAL, "lut8_keygen: null pointer");
  return c->bw == 32 ? lut_keygen_t<uint32_t>(c, n, in, out, seed, gate, k0, k1)
                     : lut_keygen_t<uint64_t>(c, n, in, out, seed, gate, k0, k1);
}
template <typename T>
static mpcx_status lut_eval_t(mpcx_ctx *c, size_t n, const void *k0, const void *k1, const void *table, const void *x,
                              void *y) {
  Lut8Layout lay = lut8_layout(c->bw, n, 0);
  void *sp = nullptr;
  HIPC(c, ctx_work(c, 3 * n * sizeof(T), &sp), "hipMalloc");
  T *m0 = static_cast<T *>(sp), *m1 = m0 + n, *vh = m1 + n;
  const uint8_t *K0 = static_cast<const uint8_t *>(k0), *K1 = static_cast<const uint8_t *>(k1);
  HIPC(c,
       launch_lut8_phase1<T>(c->L, lay, K0, K1, static_cast<const T *>(table), static_cast<const T *>(x), m0, m1),
       "lut8_phase1");
  c->counters.msg(n, c->bw);
  HIPC(c, launch_reconstruct<T>(c->L, n, m0, m1, vh), "reconstruct");
  HIPC(c, launch_lut8_phase2<T>(c->L, lay, K0, K1, vh, m0, m1), "lut8_phase2");
  c->counters.msg(n, c->bw);
  HIPC(c, launch_reconstruct<T>(c->L, n, m0, m1, static_cast<T *>(y)), "reconstruct");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}
mpcx_status mpcx_lut8_eval(mpcx_ctx *c, size_t n, const void *k0, const void *k1, const void *table, const void *x,
                           void *y) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!k0 || !k1 || !table || !x || !y) return fail(c, MPCX_EINVAL, "lut8_eval: null pointer");
  return c->bw == 32 ? lut_eval_t<uint32_t>(c, n, k0, k1, table, x, y)
                     : lut_eval_t<uint64_t>(c, n, k0, k1, table, x, y);
}

// ---------------- SxS ----------------
size_t mpcx_sxs_key_bytes(mpcx_ctx *c, int nb, int M, int K, int N) {
  return c ? sxs_layout(c->bw, nb, M, K, N, 0).end : 0;
}
template <typename T>
static mpcx_status sxs_keygen_t(mpcx_ctx *c, int nb, int M, int K, int N, const void *ra, const void *rb, void *rc,
                                uint64_t seed, uint32_t gate, void *k0v, void *k1v) {
  SxsLayout lay = sxs_layout(c->bw, nb, M, K, N, 0);
  uint8_t *k0 = static_cast<uint8_t *>(k0v), *k1 = static_cast<uint8_t *>(k1v);
  const size_t nc = size_t(nb) * M * N;
  T *RA0 = reinterpret_cast<T *>(k0 + lay.off_ra), *RA1 = reinterpret_cast<T *>(k1 + lay.off_ra);
  T *RB0 = reinterpret_cast<T *>(k0 + lay.off_rb), *RB1 = reinterpret_cast<T *>(k1 + lay.off_rb);
  HIPC(c, launch_split<T>(c->L, seed, gate, F_SPLIT + 0, size_t(nb) * M * K, static_cast<const T *>(ra), RA0, RA1,
                          nullptr),
       "split");
  HIPC(c, launch_split<T>(c->L, seed, gate, F_SPLIT + 1, size_t(nb) * K * N, static_cast<const T *>(rb), RB0, RB1,
                          nullptr),
       "split");
  HIPC(c, launch_prf_ring<T>(c->L, seed, gate, F_ROUT, nc, static_cast<T *>(rc)), "prf");
  void *sp = nullptr;
  HIPC(c, ctx_work(c, nc * sizeof(T), &sp), "hipMalloc");
  T *g = static_cast<T *>(sp);
  GemmArgs<T> a;
  a.M = M;
  a.K = K;
  a.N = N;
  a.batch = nb;
  a.sA = size_t(M) * K;
  a.sB = size_t(K) * N;
  a.sC = size_t(M) * N;
  a.A1 = static_cast<const T *>(ra);
  a.B1 = static_cast<const T *>(rb);
  a.Cin = static_cast<const T *>(rc);
  a.C = g;
  HIPC(c, launch_gemm<T>(c->L, a), "gemm");
  a.A1 = RA0;
  a.B1 = RB0;
  a.Cin = g;
  a.sign = -1;
  HIPC(c, launch_gemm<T>(c->L, a), "gemm");
  HIPC(c, launch_split<T>(c->L, seed, gate, F_SPLIT + 2, nc, g, reinterpret_cast<T *>(k0 + lay.off_c),
                          reinterpret_cast<T *>(k1 + lay.off_c), nullptr),
       "split");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}
mpcx_status mpcx_sxs_keygen(mpcx_ctx *c, int nb, int M, int K, int N, const void *ra, const void *rb, void *rc,
                            uint64_t seed, uint32_t gate, void *k0, void *k1) {
  CHECK_CTX(c);
  if (nb < 1 || M < 1 || K < 1 || N < 1 || !ra || !rb || !rc || !k0 || !k1)
    return fail(c, MPCX_EINVAL, "sxs_keygen: bad argument");
  return c->bw == 32 ? sxs_keygen_t<uint32_t>(c, nb, M, K, N, ra, rb, rc, seed, gate, k0, k1)
                     : sxs_keygen_t<uint64_t>(c, nb, M, K, N, ra, rb, rc, seed, gate, k0, k1);
}
template <typename T>
static mpcx_status sxs_eval_t(mpcx_ctx *c, int nb, int M, int K, int N, const void *k0v, const void *k1v,
                              const void *a, const void *b, void *out) {
  SxsLayout lay = sxs_layout(c->bw, nb, M, K, N, 0);
  const uint8_t *k0 = static_cast<const uint8_t *>(k0v), *k1 = static_cast<const uint8_t *>(k1v);
  const size_t nc = size_t(nb) * M * N;
  void *sp = nullptr;
  HIPC(c, ctx_work(c, 2 * nc * sizeof(T), &sp), "hipMalloc");
  T *m0 = static_cast<T *>(sp), *m1 = m0 + nc;
  GemmArgs<T> g;
  g.M = M;
  g.K = K;
  g.N = N;
  g.batch = nb;
  g.sA = size_t(M) * K;
  g.sB = size_t(K) * N;
  g.sC = size_t(M) * N;
  g.A1 = static_cast<const T *>(a);
  g.A2 = reinterpret_cast<const T *>(k0 + lay.off_ra);
  g.B1 = static_cast<const T *>(b);
  g.B2 = reinterpret_cast<const T *>(k0 + lay.off_rb);
  g.Cin = reinterpret_cast<const T *>(k0 + lay.off_c);
  g.C = m0;
  // party 1: C1 - [A^ RA1] [RB1; B^]
  GemmArgs<T> h = g;
  h.A2 = nullptr;
  h.B2 = nullptr;
  h.B1 = reinterpret_cast<const T *>(k1 + lay.off_rb);
  h.A1b = reinterpret_cast<const T *>(k1 + lay.off_ra);
  h.B1b = static_cast<const T *>(b);
  h.Cin = reinterpret_cast<const T *>(k1 + lay.off_c);
  h.C = m1;
  h.sign = -1;
  // both parties' products and the reconstruction of the exchanged shares
  HIPC(c, launch_gemm_pair_sum<T>(c->L, g, h, static_cast<T *>(out)), "gemm");
  c->counters.msg(nc, c->bw);
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}
mpcx_status mpcx_sxs_eval(mpcx_ctx *c, int nb, int M, int K, int N, const void *k0, const void *k1, const void *a,
                          const void *b, void *out) {
  CHECK_CTX(c);
  if (nb < 1 || M < 1 || K < 1 || N < 1 || !k0 || !k1 || !a || !b || !out)
    return fail(c, MPCX_EINVAL, "sxs_eval: bad argument");
  return c->bw == 32 ? sxs_eval_t<uint32_t>(c, nb, M, K, N, k0, k1, a, b, out)
                     : sxs_eval_t<uint64_t>(c, nb, M, K, N, k0, k1, a, b, out);
}

mpcx_status mpcx_sxs_key_layout(mpcx_ctx *c, int nb, int M, int K, int N, size_t off[3]) {
  CHECK_CTX(c);
  if (!off || nb < 1 || M < 1 || K < 1 || N < 1) return fail(c, MPCX_EINVAL, "sxs_key_layout: bad argument");
  const SxsLayout l = sxs_layout(c->bw, nb, M, K, N, 0);
  off[0] = l.off_ra;
  off[1] = l.off_rb;
  off[2] = l.off_c;
  return MPCX_OK;
}

template <typename T>
static mpcx_status gemm_t(mpcx_ctx *c, int M, int K, int N, const void *a, const void *b, void *out) {
  GemmArgs<T> g;
  g.M = M;
  g.K = K;
  g.N = N;
  g.A1 = static_cast<const T *>(a);
  g.B1 = static_cast<const T *>(b);
  g.C = static_cast<T *>(out);
  HIPC(c, launch_gemm<T>(c->L, g), "gemm");
  return MPCX_OK;
}
mpcx_status mpcx_ring_gemm(mpcx_ctx *c, int M, int K, int N, const void *a, const void *b, void *out) {
  CHECK_CTX(c);
  if (M < 1 || K < 1 || N < 1 || !a || !b || !out) return fail(c, MPCX_EINVAL, "ring_gemm: bad argument");
  return c->bw == 32 ? gemm_t<uint32_t>(c, M, K, N, a, b, out) : gemm_t<uint64_t>(c, M, K, N, a, b, out);
}

// ---------------- local linear maps ----------------
mpcx_status mpcx_ring_lincomb(mpcx_ctx *c, size_t rows, size_t cols, uint64_t a, const void *x, uint64_t b,
                              const void *y, const void *v, int shift, void *out) {
  CHECK_CTX(c);
  if (cols == 0 || shift < 0 || shift >= c->bw) return fail(c, MPCX_EINVAL, "ring_lincomb: bad argument");
  if (rows == 0) return MPCX_OK;
  if (!out) return fail(c, MPCX_EINVAL, "ring_lincomb: null pointer");
  if (c->bw == 32) {
    HIPC(c,
         launch_lincomb<uint32_t>(c->L, rows, cols, uint32_t(a), static_cast<const uint32_t *>(x), uint32_t(b),
                                  static_cast<const uint32_t *>(y), static_cast<const uint32_t *>(v), shift,
                                  static_cast<uint32_t *>(out)),
         "ring_lincomb");
  } else {
    HIPC(c,
         launch_lincomb<uint64_t>(c->L, rows, cols, a, static_cast<const uint64_t *>(x), b,
                                  static_cast<const uint64_t *>(y), static_cast<const uint64_t *>(v), shift,
                                  static_cast<uint64_t *>(out)),
         "ring_lincomb");
  }
  return MPCX_OK;
}

// ---------------- reveal ----------------
size_t mpcx_reveal_key_bytes(mpcx_ctx *c, size_t n) { return c ? reveal_layout(c->bw, n, 0).end : 0; }
template <typename T>
static mpcx_status reveal_keygen_t(mpcx_ctx *c, size_t n, void *mask, uint64_t seed, uint32_t gate, void *k0,
                                   void *k1) {
  RevealLayout lay = reveal_layout(c->bw, n, 0);
  HIPC(c,
       launch_reveal_keygen<T>(c->L, lay, seed, gate, static_cast<T *>(mask), static_cast<uint8_t *>(k0),
                               static_cast<uint8_t *>(k1)),
       "reveal_keygen");
  return MPCX_OK;
}
mpcx_status mpcx_reveal_keygen(mpcx_ctx *c, size_t n, void *mask, uint64_t seed, uint32_t gate, void *k0, void *k1) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!mask || !k0 || !k1) return fail(c, MPCX_EINVAL, "reveal_keygen: null pointer");
  return c->bw == 32 ? reveal_keygen_t<uint32_t>(c, n, mask, seed, gate, k0, k1)
                     : reveal_keygen_t<uint64_t>(c, n, mask, seed, gate, k0, k1);
}
template <typename T>
static mpcx_status reveal_eval_t(mpcx_ctx *c, size_t n, const void *k0, const void *k1, const void *v0,
                                 const void *v1, void *out) {
  RevealLayout lay = reveal_layout(c->bw, n, 0);
  void *sp = nullptr;
  HIPC(c, ctx_work(c, 2 * n * sizeof(T), &sp), "hipMalloc");
  T *m0 = static_cast<T *>(sp), *m1 = m0 + n;
  HIPC(c,
       launch_reveal_eval<T>(c->L, lay, static_cast<const uint8_t *>(k0), static_cast<const uint8_t *>(k1),
                             static_cast<const T *>(v0), static_cast<const T *>(v1), 0, m0, m1),
       "reveal_eval");
  c->counters.msg(n, c->bw);
  HIPC(c, launch_reconstruct<T>(c->L, n, m0, m1, static_cast<T *>(out)), "reconstruct");
  HIPC(c, hipStreamSynchronize(c->L.stream), "sync");
  return MPCX_OK;
}
mpcx_status mpcx_reveal_eval(mpcx_ctx *c, size_t n, const void *k0, const void *k1, const void *v0, const void *v1,
                             void *out) {
  CHECK_CTX(c);
  if (n == 0) return MPCX_OK;
  if (!k0 || !k1 || !v0 || !v1 || !out) return fail(c, MPCX_EINVAL, "reveal_eval: null pointer");
  return c->bw == 32 ? reveal_eval_t<uint32_t>(c, n, k0, k1, v0, v1, out)
                     : reveal_eval_t<uint64_t>(c, n, k0, k1, v0, v1, out);
}

// ---------------- adjacency normalisation ----------------
mpcx_status mpcx_set_adjnorm_lanes(mpcx_ctx *c, int lanes) {
  CHECK_CTX(c);
  if (lanes < 1 || lanes > 16) return fail(c, MPCX_EINVAL, "adjnorm lanes must be in [1, 16]");
  c->adj_lanes = lanes;
  return MPCX_OK;
}

size_t mpcx_adjnorm_key_bytes(mpcx_ctx *c, int B, int N) {
  return (c && B > 0 && N > 0) ? adjnorm_key_bytes(c->bw, c->s, B, N, c->adj_lanes) : 0;
}

mpcx_status mpcx_adjnorm_keygen(mpcx_ctx *c, int B, int N, uint64_t seed, void *mask, void *k0, void *k1) {
  CHECK_CTX(c);
  if (B < 1 || N < 1 || N > 255 || !mask || !k0 || !k1) return fail(c, MPCX_EINVAL, "adjnorm_keygen: bad argument");
  HIPC(c,
       adjnorm_keygen(c->bw, c->s, B, N, seed, c->adj_lanes, c->L, mask, static_cast<uint8_t *>(k0),
                      static_cast<uint8_t *>(k1)),
       "adjnorm_keygen");
  return MPCX_OK;
}

mpcx_status mpcx_adjnorm_eval(mpcx_ctx *c, int B, int N, int nmax, const void *k0, const void *k1, const void *a0,
                              const void *a1, void *out) {
  CHECK_CTX(c);
  if (B < 1 || N < 1 || N > 255 || nmax < 0 || nmax > 255 || !k0 || !k1 || !a0 || !a1 || !out)
    return fail(c, MPCX_EINVAL, "adjnorm_eval: bad argument");
  HIPC(c,
       adjnorm_eval(c->bw, c->s, B, N, nmax, c->adj_lanes, c->L, static_cast<const uint8_t *>(k0),
                    static_cast<const uint8_t *>(k1), a0, a1, out, &c->counters, &c->adj),
       "adjnorm_eval");
  return MPCX_OK;
}

// ---------------- party mode ----------------
constexpr int kPeerIoTimeoutMs = 120000;  // a silent peer fails the exchange after this

mpcx_status mpcx_peer_connect(int party, const char *path, int timeout_ms, mpcx_peer **out) {
  if (!out || !path || (party != 0 && party != 1) || timeout_ms < 0) return MPCX_EINVAL;
  *out = nullptr;
  std::string err;
  Peer *p = nullptr;
  const hipError_t e = guard([&] {
    return peer_connect(party, path, timeout_ms, std::max(timeout_ms, kPeerIoTimeoutMs), &p, &err);
  });
  if (e != hipSuccess) {
    std::fprintf(stderr, "libmpcx: mpcx_peer_connect(party %d): %s\n", party, err.c_str());
    return e == hipErrorInvalidValue ? MPCX_EINVAL : e == hipErrorOutOfMemory ? MPCX_ENOMEM : MPCX_EIO;
  }
  *out = new (std::nothrow) mpcx_peer();
  if (!*out) {
    delete p;
    return MPCX_ENOMEM;
  }
  (*out)->impl = p;
  return MPCX_OK;
}

mpcx_status mpcx_peer_pair(int timeout_ms, mpcx_peer **p0, mpcx_peer **p1) {
  if (!p0 || !p1 || timeout_ms < 0) return MPCX_EINVAL;
  *p0 = *p1 = nullptr;
  std::string err;
  Peer *a = nullptr, *b = nullptr;
  // MPCX_PEER_SOCKETPAIR=1: a socket pair, staged as between two processes
  const char *sp = std::getenv("MPCX_PEER_SOCKETPAIR");
  const bool sock = sp && std::atoi(sp) != 0;
  const hipError_t e = guard([&] { return peer_pair(timeout_ms, &a, &b, &err, sock); });
  if (e != hipSuccess) return e == hipErrorOutOfMemory ? MPCX_ENOMEM : MPCX_EIO;
  *p0 = new (std::nothrow) mpcx_peer();
  *p1 = new (std::nothrow) mpcx_peer();
  if (!*p0 || !*p1) {
    delete a;
    delete b;
    delete *p0;
    delete *p1;
    *p0 = *p1 = nullptr;
    return MPCX_ENOMEM;
  }
  (*p0)->impl = a;
  (*p1)->impl = b;
  return MPCX_OK;
}

void mpcx_peer_close(mpcx_peer *p) {
  if (!p) return;
  delete p->impl;
  delete p;
}
int mpcx_peer_party(const mpcx_peer *p) { return p ? p->impl->party() : -1; }
uint64_t mpcx_peer_bytes(const mpcx_peer *p) { return p ? p->impl->bytes_sent() + p->impl->bytes_received() : 0; }
uint64_t mpcx_peer_rounds(const mpcx_peer *p) { return p ? p->impl->rounds() : 0; }
int mpcx_peer_transport(const mpcx_peer *p) { return p ? p->impl->transport() : -1; }
const char *mpcx_peer_error(const mpcx_peer *p) { return p ? p->impl->error().c_str() : "null peer"; }

namespace {
// A party-mode call's status: channel failures are MPCX_EIO with the peer's message.
mpcx_status party_status(mpcx_ctx *c, mpcx_peer *p, hipError_t e, const char *what) {
  if (e == hipSuccess) return MPCX_OK;
  if (e == hipErrorNotReady) return fail(c, MPCX_EIO, std::string(what) + ": " + p->impl->error());
  return hip_status(c, e, what);
}
Launch party_launch(const mpcx_ctx *c, const mpcx_peer *p) {
  Launch L = c->L;
  L.party = p->impl->party();
  return L;
}
}  // namespace

mpcx_status mpcx_party_reconstruct(mpcx_ctx *c, mpcx_peer *p, size_t n, void *d) {
  CHECK_CTX(c);
  if (!p) return fail(c, MPCX_EINVAL, "party_reconstruct: null peer");
  if (n == 0) return MPCX_OK;
  if (!d) return fail(c, MPCX_EINVAL, "party_reconstruct: null pointer");
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] { return party_reconstruct(&c->party, L, p->impl, &c->counters, c->bw, c->s, n, d); }),
                      "party_reconstruct");
}

mpcx_status mpcx_party_tr_eval(mpcx_ctx *c, mpcx_peer *p, int kind, size_t n, const void *key, const void *x,
                               const void *bias, int ncol, void *y) {
  CHECK_CTX(c);
  if (!p || !valid_kind(kind) || (bias && ncol < 1)) return fail(c, MPCX_EINVAL, "party_tr_eval: bad argument");
  if (n == 0) return MPCX_OK;
  if ((kind != MPCX_LOCALARS && !key) || !x || !y) return fail(c, MPCX_EINVAL, "party_tr_eval: null pointer");
  if (kind == MPCX_LOCALARS)  // local: the same on both parties, no key, no exchange
    return mpcx_tr_eval(c, kind, n, nullptr, nullptr, x, bias, ncol, y);
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] {
                        return party_tr_eval(&c->party, L, p->impl, &c->counters, c->bw, c->s, kind, n,
                                             static_cast<const uint8_t *>(key), x, bias, ncol, y);
                      }),
                      "party_tr_eval");
}

mpcx_status mpcx_party_mul_eval(mpcx_ctx *c, mpcx_peer *p, size_t nx, size_t ny, size_t nz, const uint32_t *ia,
                                const uint32_t *ib, const void *key, const void *x, const void *y, void *z) {
  CHECK_CTX(c);
  if (!p) return fail(c, MPCX_EINVAL, "party_mul_eval: null peer");
  if (nz == 0) return MPCX_OK;
  if (!ia || !ib || !key || !x || !y || !z) return fail(c, MPCX_EINVAL, "party_mul_eval: null pointer");
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] {
                        return party_mul_eval(&c->party, L, p->impl, &c->counters, c->bw, c->s, nx, ny, nz, ia, ib,
                                              static_cast<const uint8_t *>(key), x, y, z);
                      }),
                      "party_mul_eval");
}

mpcx_status mpcx_party_lut8_eval(mpcx_ctx *c, mpcx_peer *p, size_t n, const void *key, const void *table,
                                 const void *x, void *y) {
  CHECK_CTX(c);
  if (!p) return fail(c, MPCX_EINVAL, "party_lut8_eval: null peer");
  if (n == 0) return MPCX_OK;
  if (!key || !table || !x || !y) return fail(c, MPCX_EINVAL, "party_lut8_eval: null pointer");
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] {
                        return party_lut8_eval(&c->party, L, p->impl, &c->counters, c->bw, c->s, n,
                                               static_cast<const uint8_t *>(key), table, x, y);
                      }),
                      "party_lut8_eval");
}

mpcx_status mpcx_party_sxs_eval(mpcx_ctx *c, mpcx_peer *p, int nb, int M, int K, int N, const void *key,
                                const void *a, const void *b, void *out) {
  CHECK_CTX(c);
  if (!p || nb < 1 || M < 1 || K < 1 || N < 1 || !key || !a || !b || !out)
    return fail(c, MPCX_EINVAL, "party_sxs_eval: bad argument");
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] {
                        return party_sxs_eval(&c->party, L, p->impl, &c->counters, c->bw, c->s, nb, M, K, N,
                                              static_cast<const uint8_t *>(key), a, b, out);
                      }),
                      "party_sxs_eval");
}

mpcx_status mpcx_party_reveal_eval(mpcx_ctx *c, mpcx_peer *p, size_t n, const void *key, const void *v,
                                   void *out) {
  CHECK_CTX(c);
  if (!p) return fail(c, MPCX_EINVAL, "party_reveal_eval: null peer");
  if (n == 0) return MPCX_OK;
  if (!key || !v || !out) return fail(c, MPCX_EINVAL, "party_reveal_eval: null pointer");
  const Launch L = party_launch(c, p);
  return party_status(c, p, guard([&] {
                        return party_reveal_eval(&c->party, L, p->impl, &c->counters, c->bw, c->s, n,
                                                 static_cast<const uint8_t *>(key), v, out);
                      }),
                      "party_reveal_eval");
}

// ---------------- pinned host memory ----------------
mpcx_status mpcx_host_alloc(size_t bytes, void **out) {
  if (!out || bytes == 0) return MPCX_EINVAL;
  *out = nullptr;
  hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return MPCX_ENOMEM;
  return e == hipSuccess ? MPCX_OK : MPCX_EHIP;
}

void mpcx_host_free(void *p) {
  if (p) (void)hipHostFree(p);
}

// ---------------- model ----------------
mpcx_status mpcx_model_create(mpcx_ctx *c, const mpcx_model_dims *dims, const int64_t *W, size_t nW,
                              mpcx_model **out) {
  CHECK_CTX(c);
  if (!dims || !W || !out) return fail(c, MPCX_EINVAL, "model_create: null pointer");
  ModelDims d;
  d.n_nodes = dims->n_nodes;
  d.feat = dims->feat;
  for (int i = 0; i < 3; i++) d.gcn[i] = dims->gcn[i];
  for (int i = 0; i < 2; i++) d.dfc[i] = dims->dfc[i];
  d.prot = dims->prot;
  d.nfus = dims->nfus;
  for (int i = 0; i < 4; i++) d.fus[i] = dims->fus[i];
  d.lut_nmax = dims->lut_nmax;
  d.mask_scale = dims->mask_scale;
  d.slack = dims->slack;
  std::string err;
  LaneSet *impl = nullptr;
  try {
    impl = make_lane_set(c->bw, c->s, d, W, nW, c->L, &err);
  } catch (const std::bad_alloc &) {
    return fail(c, MPCX_ENOMEM, "model_create: host allocation failed");
  }
  if (!impl) return fail(c, MPCX_EINVAL, "model_create: " + err);
  auto *m = new (std::nothrow) mpcx_model();
  if (!m) {
    delete impl;
    return fail(c, MPCX_ENOMEM, "model_create: host allocation failed");
  }
  m->ctx = c;
  m->impl = impl;
  *out = m;
  return MPCX_OK;
}

void mpcx_model_destroy(mpcx_model *m) {
  if (!m) return;
  delete m->impl;
  delete m;
}

mpcx_status mpcx_model_set_lanes(mpcx_model *m, int lanes) {
  if (!m) return MPCX_EINVAL;
  if (lanes < 1 || lanes > 16) return fail(m->ctx, MPCX_EINVAL, "model_set_lanes: lanes must be in [1, 16]");
  std::string err;
  hipError_t e = guard([&] { return m->impl->set_lanes(lanes, &err); });
  if (e == hipErrorInvalidValue) return fail(m->ctx, MPCX_EINVAL, "model_set_lanes: " + err);
  HIPC(m->ctx, e, "model_set_lanes");
  return MPCX_OK;
}

int mpcx_model_lanes(const mpcx_model *m) { return m ? m->impl->lanes() : 0; }

size_t mpcx_model_key_bytes(const mpcx_model *m, int B) {
  return (m && B > 0) ? guard_size([&] { return m->impl->key_bytes(B); }) : 0;
}

mpcx_status mpcx_model_keygen(mpcx_model *m, int B, uint64_t seed) {
  if (!m) return MPCX_EINVAL;
  if (B < 1) return fail(m->ctx, MPCX_EINVAL, "B must be >= 1");
  HIPC(m->ctx, guard([&] { return m->impl->keygen(B, seed); }), "model_keygen");
  return MPCX_OK;
}

mpcx_status mpcx_model_import_keys(mpcx_model *m, int B, const void *k0, const void *k1, size_t bytes) {
  if (!m || !k0 || !k1) return MPCX_EINVAL;
  if (bytes != mpcx_model_key_bytes(m, B)) return fail(m->ctx, MPCX_EINVAL, "key size mismatch");
  HIPC(m->ctx, guard([&] { return m->impl->import_keys(B, k0, k1, bytes); }), "model_import_keys");
  return MPCX_OK;
}

mpcx_status mpcx_model_export_keys(mpcx_model *m, int party, void *dst, size_t bytes) {
  if (!m || !dst || (party != 0 && party != 1)) return MPCX_EINVAL;
  HIPC(m->ctx, guard([&] { return m->impl->export_keys(party, dst, bytes); }), "model_export_keys");
  return MPCX_OK;
}

mpcx_status mpcx_model_release_arena(mpcx_model *m) {
  if (!m) return MPCX_EINVAL;
  HIPC(m->ctx, guard([&] { return m->impl->release_arena(); }), "model_release_arena");
  return MPCX_OK;
}

mpcx_status mpcx_model_attach_host_keys(mpcx_model *m, int B, const void *k0, size_t bytes0, const void *k1,
                                        size_t bytes1, size_t slot_bytes) {
  if (!m || !k0 || !k1) return MPCX_EINVAL;
  if (B < 1 || (bytes0 != mpcx_model_key_bytes(m, B) && bytes0 != mpcx_model_unique_key_bytes(m, B, 0)) ||
      (bytes1 != mpcx_model_key_bytes(m, B) && bytes1 != mpcx_model_unique_key_bytes(m, B, 1)))
    return fail(m->ctx, MPCX_EINVAL, "attach_host_keys: key size mismatch");
  hipError_t e = guard([&] { return m->impl->attach_host_keys(B, k0, bytes0, k1, bytes1, slot_bytes); });
  if (e == hipErrorInvalidValue)
    return fail(m->ctx, MPCX_EINVAL, "attach_host_keys: slot_bytes smaller than the largest gate key");
  HIPC(m->ctx, e, "model_attach_host_keys");
  return MPCX_OK;
}

mpcx_status mpcx_model_write_keys(mpcx_model *m, int party, int packed, const char *path, int append) {
  if (!m || !path || (party != 0 && party != 1)) return MPCX_EINVAL;
  hipError_t e = guard([&] { return m->impl->write_keys(party, packed != 0, path, append != 0); });
  if (e == hipErrorInvalidValue) return fail(m->ctx, MPCX_ESTATE, "write_keys: no resident keys");
  if (e == hipErrorNotSupported)
    return fail(m->ctx, MPCX_ESTATE, "write_keys: packed keys need keys from mpcx_model_keygen (imported keys)");
  if (e == hipErrorFileNotFound) return fail(m->ctx, MPCX_EIO, std::string("write_keys: cannot write ") + path);
  HIPC(m->ctx, e, "model_write_keys");
  return MPCX_OK;
}

mpcx_status mpcx_model_attach_key_files(mpcx_model *m, int B, const char *path0, const char *path1,
                                        size_t slot_bytes) {
  if (!m || !path0 || !path1) return MPCX_EINVAL;
  if (B < 1 || slot_bytes == 0) return fail(m->ctx, MPCX_EINVAL, "attach_key_files: bad argument");
  hipError_t e = guard([&] { return m->impl->attach_key_files(B, path0, path1, slot_bytes); });
  if (e == hipErrorFileNotFound)
    return fail(m->ctx, MPCX_EIO, "attach_key_files: key files missing or not whole key sets of this batch");
  if (e == hipErrorInvalidValue)
    return fail(m->ctx, MPCX_EINVAL, "attach_key_files: slot_bytes smaller than the largest gate key");
  HIPC(m->ctx, e, "model_attach_key_files");
  return MPCX_OK;
}

size_t mpcx_model_unique_key_bytes(const mpcx_model *m, int B, int party) {
  return (m && B > 0 && (party == 0 || party == 1)) ? guard_size([&] { return m->impl->unique_key_bytes(B, party); })
                                                   : 0;
}

mpcx_status mpcx_model_export_unique_keys(mpcx_model *m, int party, void *dst, size_t bytes) {
  if (!m || !dst || (party != 0 && party != 1)) return MPCX_EINVAL;
  hipError_t e = guard([&] { return m->impl->export_unique_keys(party, dst, bytes); });
  if (e == hipErrorNotSupported)
    return fail(m->ctx, MPCX_ESTATE, "export_unique_keys: packed keys need keys from mpcx_model_keygen");
  HIPC(m->ctx, e, "model_export_unique_keys");
  return MPCX_OK;
}

mpcx_status mpcx_model_stream_stats(const mpcx_model *m, int *chunks, uint64_t *bytes_h2d) {
  if (!m) return MPCX_EINVAL;
  if (chunks) *chunks = m->impl->stream_stats.chunks;
  if (bytes_h2d) *bytes_h2d = m->impl->stream_stats.bytes_h2d;
  return MPCX_OK;
}

mpcx_status mpcx_model_set_inputs(mpcx_model *m, int B, const void *x0, const void *x1, const void *a0, const void *a1,
                                  const void *m0, const void *m1, const int64_t *prot) {
  if (!m || !x0 || !x1 || !a0 || !a1 || !m0 || !m1 || !prot) return MPCX_EINVAL;
  if (B < 1) return fail(m->ctx, MPCX_EINVAL, "B must be >= 1");
  HIPC(m->ctx, guard([&] { return m->impl->set_inputs(B, x0, x1, a0, a1, m0, m1, prot); }), "model_set_inputs");
  return MPCX_OK;
}

mpcx_status mpcx_model_forward(mpcx_model *m, int B) {
  if (!m) return MPCX_EINVAL;
  hipError_t e = guard([&] { return m->impl->forward(B); });
  if (e == hipErrorInvalidValue) return fail(m->ctx, MPCX_ESTATE, "forward: keys or inputs not set for this B");
  if (e == hipErrorFileNotFound) return fail(m->ctx, MPCX_EIO, "forward: key file read failed");
  if (e == hipErrorNotReady) return fail(m->ctx, MPCX_EIO, "forward: the channel to the other party failed");
  HIPC(m->ctx, e, "model_forward");
  m->ctx->counters.bytes += m->impl->counters.bytes;
  m->ctx->counters.rounds += m->impl->counters.rounds;
  return MPCX_OK;
}

mpcx_status mpcx_model_output(mpcx_model *m, int B, int64_t *out) {
  if (!m || !out) return MPCX_EINVAL;
  HIPC(m->ctx, guard([&] { return m->impl->output(out, B); }), "model_output");
  return MPCX_OK;
}

mpcx_status mpcx_model_set_party(mpcx_model *m, mpcx_peer *peer) {
  if (!m) return MPCX_EINVAL;
  const hipError_t e =
      guard([&] { return m->impl->set_party(peer ? peer->impl->party() : -1, peer ? peer->impl : nullptr); });
  if (e == hipErrorInvalidValue) return fail(m->ctx, MPCX_EINVAL, "model_set_party: " + m->impl->err);
  HIPC(m->ctx, e, "model_set_party");
  return MPCX_OK;
}

mpcx_status mpcx_model_import_party_key(mpcx_model *m, int B, const void *key, size_t bytes) {
  if (!m || !key) return MPCX_EINVAL;
  if (m->impl->party() < 0) return fail(m->ctx, MPCX_ESTATE, "import_party_key: the model is not in party mode");
  if (B < 1 || bytes != mpcx_model_key_bytes(m, B)) return fail(m->ctx, MPCX_EINVAL, "import_party_key: key size mismatch");
  HIPC(m->ctx, guard([&] { return m->impl->import_party_key(B, key, bytes); }), "model_import_party_key");
  return MPCX_OK;
}

mpcx_status mpcx_model_set_party_inputs(mpcx_model *m, int B, const void *x, const void *a, const void *mask,
                                        const int64_t *prot) {
  if (!m || !x || !a || !mask) return MPCX_EINVAL;
  if (m->impl->party() < 0) return fail(m->ctx, MPCX_ESTATE, "set_party_inputs: the model is not in party mode");
  if (B < 1) return fail(m->ctx, MPCX_EINVAL, "B must be >= 1");
  HIPC(m->ctx, guard([&] { return m->impl->set_party_inputs(B, x, a, mask, prot); }), "model_set_party_inputs");
  return MPCX_OK;
}

mpcx_status mpcx_model_profile(mpcx_model *m, int enable) {
  if (!m) return MPCX_EINVAL;
  m->impl->profile(enable != 0);
  return MPCX_OK;
}

mpcx_status mpcx_model_profile_read(mpcx_model *m, int *launches, double *ms, double *elements, double *aes,
                                    double *hbm_bytes) {
  if (!m) return MPCX_EINVAL;
  HIPC(m->ctx, guard([&] { return m->impl->profile_read(launches, ms, elements, aes, hbm_bytes); }), "model_profile_read");
  return MPCX_OK;
}

mpcx_status mpcx_model_profile_gemm(mpcx_model *m, int *sections, double *ms, double *ring_macs) {
  if (!m) return MPCX_EINVAL;
  HIPC(m->ctx, guard([&] { return m->impl->profile_gemm(sections, ms, ring_macs); }), "model_profile_gemm");
  return MPCX_OK;
}
