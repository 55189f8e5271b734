// peer.hip -- socket channel between the two parties (host code only).
#include "peer.h"

#include <poll.h>
#include <sys/socket.h>
#include <sys/time.h>
#include <sys/un.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstdlib>
#include <cstring>

namespace mpcx {

// Two ends of one process: each exchange, an end posts its segments and the
// event recorded after its message on its stream, waits for the peer's post,
// makes its stream wait for the peer's event and copies the peer's segments
// into its own receive regions (device to device), then posts an event after
// those copies and makes its stream wait for the peer's: a party's send
// regions are not rewritten before the peer has read them.  Both ends pass the
// second post of a round before either starts the next, so each event is
// waited on before it is recorded again.
struct LocalLink {
  struct End {
    uint64_t ready = 0, consumed = 0;  // rounds posted
    const Peer::Seg *segs = nullptr;
    int nseg = 0;
    size_t total = 0;
    hipEvent_t ev_ready = nullptr, ev_consumed = nullptr;
    bool closed = false;
  };
  std::mutex mu;
  std::condition_variable cv;
  End end[2];
};

// (no HIP call here: the pair may be made before the process's first context;
// the events are created at the first exchange)
Peer::Peer(std::shared_ptr<LocalLink> link, int party, int io_timeout_ms)
    : party_(party), link_(std::move(link)), io_timeout_ms_(io_timeout_ms) {}

Peer::Peer(int fd, int party) : fd_(fd), party_(party) {
  // Messages sent inline must fit the socket's send buffer in both directions
  // at once: take a quarter of what the kernel grants (at most kInline).
  int want = int(4 * kInline), got = 0;
  socklen_t len = sizeof got;
  (void)setsockopt(fd_, SOL_SOCKET, SO_SNDBUF, &want, sizeof want);
  if (getsockopt(fd_, SOL_SOCKET, SO_SNDBUF, &got, &len) == 0 && got > 0)
    inline_max_ = std::min(kInline, size_t(got) / 4);
  th_ = std::thread([this] { sender_loop(); });
}

Peer::~Peer() {
  if (link_) {
    {
      std::lock_guard<std::mutex> lk(link_->mu);
      link_->end[party_].closed = true;
    }
    link_->cv.notify_all();
  }
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  if (th_.joinable()) th_.join();
  for (hipEvent_t e : lev_)
    if (e) (void)hipEventDestroy(e);
  if (read_pending_) (void)hipEventSynchronize(ipc_ev_[1]);
  if (peer_inbox_) (void)hipIpcCloseMemHandle(peer_inbox_);
  if (inbox_) (void)hipFree(inbox_);
  for (hipEvent_t e : ipc_ev_)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : ev_) (void)hipEventDestroy(e);
  if (fd_ >= 0) ::close(fd_);
  if (hs_) (void)hipHostFree(hs_);
  if (hr_) (void)hipHostFree(hr_);
}

hipError_t Peer::ensure(size_t bytes) {
  if (bytes <= cap_) return hipSuccess;
  size_t cap = cap_ ? cap_ : (size_t(1) << 20);
  while (cap < bytes) cap *= 2;
  uint8_t *s = nullptr, *r = nullptr;
  hipError_t e = hipHostMalloc((void **)&s, cap, hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void **)&r, cap, hipHostMallocDefault);
  if (e != hipSuccess) {
    if (s) (void)hipHostFree(s);
    return e;
  }
  if (hs_) (void)hipHostFree(hs_);
  if (hr_) (void)hipHostFree(hr_);
  hs_ = s;
  hr_ = r;
  cap_ = cap;
  return hipSuccess;
}

bool Peer::send_all(const uint8_t *p, size_t n) {
  while (n > 0) {
    const ssize_t k = ::send(fd_, p, n, MSG_NOSIGNAL);
    if (k < 0 && errno == EINTR) continue;
    if (k <= 0) return false;
    p += k;
    n -= size_t(k);
  }
  return true;
}

bool Peer::recv_all(uint8_t *p, size_t n) {
  while (n > 0) {
    const ssize_t k = ::recv(fd_, p, n, 0);
    if (k < 0 && errno == EINTR) continue;
    if (k <= 0) return false;  // closed, error or receive timeout
    p += k;
    n -= size_t(k);
  }
  return true;
}

// The sender thread: the chunks of the current message, each once its staging
// copy (the event recorded after it) is done.
void Peer::sender_loop() {
  std::unique_lock<std::mutex> lk(mu_);
  for (;;) {
    cv_.wait(lk, [this] { return stop_ || job_ready_; });
    if (stop_) return;
    const uint8_t *p = job_;
    const size_t n = job_n_;
    job_ready_ = false;
    lk.unlock();
    bool ok = true;
    for (size_t c = 0, lo = 0; ok && lo < n; c++, lo += kChunk)
      ok = hipEventSynchronize(ev_[c]) == hipSuccess && send_all(p + lo, std::min(kChunk, n - lo));
    lk.lock();
    job_ok_ = ok;
    job_done_ = true;
    cv_.notify_all();
  }
}

hipError_t Peer::ensure_events(size_t n) {
  while (ev_.size() < n) {
    hipEvent_t e = nullptr;
    const hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (r != hipSuccess) return r;
    ev_.push_back(e);
  }
  return hipSuccess;
}

// The parts of the segments that fall in [lo, hi) of the message (the
// segments back to back), copied device -> staging (to_host) or staging ->
// device on `stream`.
static hipError_t copy_part(hipStream_t stream, const Peer::Seg *segs, int nseg, size_t lo, size_t hi,
                            uint8_t *stage, bool to_host) {
  size_t o = 0;
  for (int k = 0; k < nseg; k++) {
    const size_t b = o, e = o + segs[k].bytes;
    o = e;
    const size_t a0 = std::max(b, lo), a1 = std::min(e, hi);
    if (a0 >= a1) continue;
    const hipError_t r =
        to_host ? hipMemcpyAsync(stage + a0, static_cast<const uint8_t *>(segs[k].send) + (a0 - b), a1 - a0,
                                 hipMemcpyDeviceToHost, stream)
                : hipMemcpyAsync(static_cast<uint8_t *>(segs[k].recv) + (a0 - b), stage + a0, a1 - a0,
                                 hipMemcpyHostToDevice, stream);
    if (r != hipSuccess) return r;
  }
  return hipSuccess;
}

// One exchange.  The message is staged to pinned memory in chunks of kChunk
// bytes, an event after each: the sender thread sends a chunk once it is
// staged, while the next ones are still being copied, and each received chunk
// goes back to the device at once, so the copies overlap the socket.  A
// message of at most inline_max_ bytes is sent from this thread (both
// directions fit the socket buffers, so neither send can block on the other).
hipError_t Peer::exchange(hipStream_t stream, const Seg *segs, int nseg) {
  if (broken_) return hipErrorNotReady;
  size_t total = 0;
  for (int k = 0; k < nseg; k++) total += segs[k].bytes;
  rounds_++;
  if (total == 0) return hipSuccess;
  if (link_) return exchange_local(stream, segs, nseg, total);
  if (cross_process_ && ipc_state_ < 0) {
    const hipError_t ne = ipc_negotiate();
    if (ne != hipSuccess) return ne;
  }
  if (ipc_state_ == 1 && total <= kIpcMax) return exchange_ipc(stream, segs, nseg, total);
  return exchange_socket(stream, segs, nseg, total);
}

hipError_t Peer::exchange_socket(hipStream_t stream, const Seg *segs, int nseg, size_t total) {
  hipError_t e = ensure(total);
  if (e != hipSuccess) return e;
  const size_t nch = (total + kChunk - 1) / kChunk;
  e = ensure_events(nch);
  if (e != hipSuccess) return e;
  for (size_t c = 0; c < nch; c++) {
    e = copy_part(stream, segs, nseg, c * kChunk, std::min(total, (c + 1) * kChunk), hs_, true);
    if (e == hipSuccess) e = hipEventRecord(ev_[c], stream);
    if (e != hipSuccess) return e;
  }
  bool rok = true, sok = true;
  if (total <= inline_max_) {
    // staged, and (stream order) the previous exchange's copies out of hr_ done
    e = hipEventSynchronize(ev_[nch - 1]);
    if (e != hipSuccess) return e;
    sok = send_all(hs_, total);
    rok = sok && recv_all(hr_, total);
    if (rok) e = copy_part(stream, segs, nseg, 0, total, hr_, false);
  } else {
    // the previous exchange's copies out of hr_ are done once chunk 0 is staged
    e = hipEventSynchronize(ev_[0]);
    if (e != hipSuccess) return e;
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = hs_;
      job_n_ = total;
      job_ready_ = true;
      job_done_ = false;
    }
    cv_.notify_all();
    for (size_t lo = 0; rok && lo < total; lo += kChunk) {
      const size_t hi = std::min(total, lo + kChunk);
      rok = recv_all(hr_ + lo, hi - lo);
      if (rok && e == hipSuccess) e = copy_part(stream, segs, nseg, lo, hi, hr_, false);
    }
    std::unique_lock<std::mutex> lk(mu_);
    if (!rok) ::shutdown(fd_, SHUT_RDWR);  // unblock a sender stuck on a full socket
    cv_.wait(lk, [this] { return job_done_; });
    sok = job_ok_;
  }
  if (!rok || !sok) {
    broken_ = true;
    err_ = !rok ? "receive from the peer failed (closed or timed out)" : "send to the peer failed";
    return hipErrorNotReady;
  }
  if (e != hipSuccess) return e;
  sent_ += total;
  recv_ += total;
  return hipSuccess;
}

hipError_t Peer::exchange_local(hipStream_t stream, const Seg *segs, int nseg, size_t total) {
  LocalLink &L = *link_;
  LocalLink::End &me = L.end[party_], &pe = L.end[1 - party_];
  const uint64_t r = rounds_;
  for (hipEvent_t &ev : lev_)
    if (!ev) {
      const hipError_t ce = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (ce != hipSuccess) return ce;
    }
  auto wait_peer = [&](std::unique_lock<std::mutex> &lk, uint64_t LocalLink::End::*field) {
    auto ok = [&] { return pe.*field >= r || pe.closed; };
    if (io_timeout_ms_ > 0) return L.cv.wait_for(lk, std::chrono::milliseconds(io_timeout_ms_), ok) && !pe.closed;
    L.cv.wait(lk, ok);
    return !pe.closed;
  };
  hipError_t e = hipEventRecord(lev_[0], stream);
  if (e != hipSuccess) return e;
  std::vector<Seg> from;
  hipEvent_t peer_ready = nullptr;
  {
    std::unique_lock<std::mutex> lk(L.mu);
    me.segs = segs;
    me.nseg = nseg;
    me.total = total;
    me.ev_ready = lev_[0];
    me.ready = r;
    L.cv.notify_all();
    // on failure this end closes, so that a late peer does not read `segs`
    if (!wait_peer(lk, &LocalLink::End::ready)) {
      broken_ = me.closed = true;
      err_ = "the peer closed or did not reach the exchange in time";
      L.cv.notify_all();
      return hipErrorNotReady;
    }
    if (pe.total != total) {
      broken_ = me.closed = true;
      err_ = "the peer's message has another length";
      L.cv.notify_all();
      return hipErrorNotReady;
    }
    from.assign(pe.segs, pe.segs + pe.nseg);  // the peer's array lives until it sees our second post
    peer_ready = pe.ev_ready;
  }
  e = hipStreamWaitEvent(stream, peer_ready, 0);
  // the peer's send regions into ours, by offset in the message (segments back to back)
  size_t i = 0, j = 0, oi = 0, oj = 0;
  while (e == hipSuccess && i < size_t(nseg) && j < from.size()) {
    const size_t n = std::min(segs[i].bytes - oi, from[j].bytes - oj);
    if (n) e = hipMemcpyAsync(static_cast<uint8_t *>(segs[i].recv) + oi,
                              static_cast<const uint8_t *>(from[j].send) + oj, n, hipMemcpyDeviceToDevice, stream);
    oi += n;
    oj += n;
    if (oi == segs[i].bytes) i++, oi = 0;
    if (oj == from[j].bytes) j++, oj = 0;
  }
  if (e == hipSuccess) e = hipEventRecord(lev_[1], stream);
  hipEvent_t peer_consumed = nullptr;
  {
    std::unique_lock<std::mutex> lk(L.mu);
    me.ev_consumed = lev_[1];
    me.consumed = r;  // posted even after a failed copy, so that the peer does not wait out its timeout
    L.cv.notify_all();
    if (!wait_peer(lk, &LocalLink::End::consumed)) {
      broken_ = me.closed = true;
      err_ = "the peer closed or did not finish the exchange in time";
      L.cv.notify_all();
      return hipErrorNotReady;
    }
    peer_consumed = pe.ev_consumed;
  }
  if (e == hipSuccess) e = hipStreamWaitEvent(stream, peer_consumed, 0);
  if (e != hipSuccess) return e;
  sent_ += total;
  recv_ += total;
  return hipSuccess;
}

// ---- two processes on one GPU ----
bool Peer::token(char t) {
  uint8_t in = 0;
  const uint8_t out = uint8_t(t);
  if (!send_all(&out, 1) || !recv_all(&in, 1) || in != out) {
    broken_ = true;
    err_ = "the peer closed, timed out or left the exchange order";
    return false;
  }
  return true;
}

// Both ends send the same hello (whether they want IPC, the process, the GPU's
// PCI bus id) and take the same decision: IPC when both want it, in two
// processes on the same GPU.
hipError_t Peer::ipc_negotiate() {
  struct Hello {
    uint32_t magic, want;
    int64_t pid;  // two ends of one process (threads): no IPC (a process cannot open its own handle)
    char bus[64];
  } h{}, q{};
  h.magic = 0x4d504358u;  // "MPCX"
  h.pid = int64_t(::getpid());
  const char *v = std::getenv("MPCX_PEER_IPC");
  h.want = v && std::atoi(v) == 0 ? 0u : 1u;
  int dev = 0;
  if (h.want && (hipGetDevice(&dev) != hipSuccess || hipDeviceGetPCIBusId(h.bus, int(sizeof h.bus), dev) != hipSuccess))
    h.want = 0;
  h.bus[sizeof h.bus - 1] = 0;
  if (!send_all(reinterpret_cast<const uint8_t *>(&h), sizeof h) || !recv_all(reinterpret_cast<uint8_t *>(&q), sizeof q)) {
    broken_ = true;
    err_ = "the peer closed or timed out before the first exchange";
    return hipErrorNotReady;
  }
  q.bus[sizeof q.bus - 1] = 0;
  ipc_state_ = h.want && q.want && q.magic == h.magic && q.pid != h.pid && std::strcmp(h.bus, q.bus) == 0 ? 1 : 0;
  if (ipc_state_ == 1) {
    for (hipEvent_t &e : ipc_ev_) {
      const hipError_t ce = hipEventCreateWithFlags(&e, hipEventDisableTiming);
      if (ce != hipSuccess) return ce;
    }
    return ipc_grow(kIpcMin);
  }
  return hipSuccess;
}

// New inboxes of at least `bytes` on both ends (both call it at the same
// exchange: the messages have one length); the old ones are released once
// both ends have closed their mappings.
hipError_t Peer::ipc_grow(size_t bytes) {
  size_t cap = kIpcMin;
  while (cap < bytes) cap *= 2;
  if (read_pending_) {
    const hipError_t se = hipEventSynchronize(ipc_ev_[1]);
    if (se != hipSuccess) return se;
    read_pending_ = false;
  }
  if (peer_inbox_) {
    (void)hipIpcCloseMemHandle(peer_inbox_);
    peer_inbox_ = nullptr;
    if (!token('C')) return hipErrorNotReady;
  }
  if (inbox_) (void)hipFree(inbox_);
  inbox_ = nullptr;
  inbox_cap_ = 0;
  hipError_t e = hipMalloc(&inbox_, cap);
  hipIpcMemHandle_t mine{}, theirs{};
  if (e == hipSuccess) e = hipIpcGetMemHandle(&mine, inbox_);
  // the handle goes across even after a failure (zeroed), so that the peer
  // does not wait out its timeout; a failure then ends IPC on both sides
  const uint8_t ok = e == hipSuccess ? 1 : 0;
  uint8_t pok = 0;
  if (!send_all(&ok, 1) || !send_all(reinterpret_cast<const uint8_t *>(&mine), sizeof mine) ||
      !recv_all(&pok, 1) || !recv_all(reinterpret_cast<uint8_t *>(&theirs), sizeof theirs)) {
    broken_ = true;
    err_ = "the peer closed or timed out while mapping the inboxes";
    return hipErrorNotReady;
  }
  if (!ok || !pok) {
    broken_ = true;
    err_ = "an inbox could not be shared with the peer process";
    return e != hipSuccess ? e : hipErrorNotReady;
  }
  e = hipIpcOpenMemHandle(&peer_inbox_, theirs, hipIpcMemLazyEnablePeerAccess);
  if (e != hipSuccess) {
    peer_inbox_ = nullptr;
    broken_ = true;
    err_ = "the peer's inbox could not be mapped";
    return e;
  }
  inbox_cap_ = cap;
  return hipSuccess;
}

// One exchange through the inboxes: this end's inbox is free (its last read
// done) -> 'R' both ways -> the message into the peer's inbox, waited for ->
// 'D' both ways -> the peer's message from this end's inbox into the receive
// regions, on the stream (waited for at the next exchange).
hipError_t Peer::exchange_ipc(hipStream_t stream, const Seg *segs, int nseg, size_t total) {
  hipError_t e = hipSuccess;
  if (total > inbox_cap_) {
    e = ipc_grow(total);
    if (e != hipSuccess) return e;
  }
  if (read_pending_) {
    e = hipEventSynchronize(ipc_ev_[1]);
    if (e != hipSuccess) return e;
    read_pending_ = false;
  }
  if (!token('R')) return hipErrorNotReady;
  size_t o = 0;
  for (int k = 0; k < nseg && e == hipSuccess; k++) {
    if (segs[k].bytes)
      e = hipMemcpyAsync(static_cast<uint8_t *>(peer_inbox_) + o, segs[k].send, segs[k].bytes,
                         hipMemcpyDeviceToDevice, stream);
    o += segs[k].bytes;
  }
  if (e == hipSuccess) e = hipEventRecord(ipc_ev_[0], stream);
  if (e == hipSuccess) e = hipEventSynchronize(ipc_ev_[0]);
  if (e != hipSuccess) return e;
  if (!token('D')) return hipErrorNotReady;
  o = 0;
  for (int k = 0; k < nseg && e == hipSuccess; k++) {
    if (segs[k].bytes)
      e = hipMemcpyAsync(segs[k].recv, static_cast<const uint8_t *>(inbox_) + o, segs[k].bytes,
                         hipMemcpyDeviceToDevice, stream);
    o += segs[k].bytes;
  }
  if (e == hipSuccess) e = hipEventRecord(ipc_ev_[1], stream);
  if (e != hipSuccess) return e;
  read_pending_ = true;
  sent_ += total;
  recv_ += total;
  return hipSuccess;
}

static void set_io_timeout(int fd, int ms) {
  if (ms <= 0) return;
  timeval tv;
  tv.tv_sec = ms / 1000;
  tv.tv_usec = (ms % 1000) * 1000;
  (void)setsockopt(fd, SOL_SOCKET, SO_RCVTIMEO, &tv, sizeof tv);
  (void)setsockopt(fd, SOL_SOCKET, SO_SNDTIMEO, &tv, sizeof tv);
}

static bool make_addr(const std::string &path, sockaddr_un *a, std::string *err) {
  std::memset(a, 0, sizeof *a);
  a->sun_family = AF_UNIX;
  if (path.empty() || path.size() >= sizeof(a->sun_path)) {
    *err = "socket path empty or too long: " + path;
    return false;
  }
  std::memcpy(a->sun_path, path.c_str(), path.size());
  return true;
}

hipError_t peer_connect(int party, const std::string &path, int timeout_ms, int io_timeout_ms, Peer **out,
                        std::string *err) {
  *out = nullptr;
  sockaddr_un a;
  if ((party != 0 && party != 1) || !make_addr(path, &a, err)) {
    if (err->empty()) *err = "party must be 0 or 1";
    return hipErrorInvalidValue;
  }
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::milliseconds(timeout_ms);
  int fd = -1;
  if (party == 0) {
    const int ls = ::socket(AF_UNIX, SOCK_STREAM, 0);
    if (ls < 0) {
      *err = std::string("socket: ") + std::strerror(errno);
      return hipErrorNotReady;
    }
    (void)::unlink(path.c_str());
    if (::bind(ls, reinterpret_cast<sockaddr *>(&a), sizeof a) != 0 || ::listen(ls, 1) != 0) {
      *err = std::string("bind/listen ") + path + ": " + std::strerror(errno);
      ::close(ls);
      return hipErrorNotReady;
    }
    pollfd pf{ls, POLLIN, 0};
    const int r = ::poll(&pf, 1, timeout_ms);
    if (r == 1) fd = ::accept(ls, nullptr, nullptr);
    ::close(ls);
    (void)::unlink(path.c_str());
    if (fd < 0) {
      *err = "no connection from party 1 on " + path;
      return hipErrorNotReady;
    }
  } else {
    for (;;) {
      fd = ::socket(AF_UNIX, SOCK_STREAM, 0);
      if (fd < 0) {
        *err = std::string("socket: ") + std::strerror(errno);
        return hipErrorNotReady;
      }
      if (::connect(fd, reinterpret_cast<sockaddr *>(&a), sizeof a) == 0) break;
      ::close(fd);
      fd = -1;
      if (std::chrono::steady_clock::now() >= deadline) {
        *err = "could not connect to party 0 on " + path;
        return hipErrorNotReady;
      }
      std::this_thread::sleep_for(std::chrono::milliseconds(20));
    }
  }
  set_io_timeout(fd, io_timeout_ms);
  try {
    *out = new Peer(fd, party);
  } catch (...) {
    ::close(fd);
    return hipErrorOutOfMemory;
  }
  (*out)->cross_process_ = true;
  return hipSuccess;
}

hipError_t peer_pair(int io_timeout_ms, Peer **p0, Peer **p1, std::string *err, bool socket) {
  *p0 = *p1 = nullptr;
  if (!socket) {
    try {
      auto link = std::make_shared<LocalLink>();
      *p0 = new Peer(link, 0, io_timeout_ms);
      *p1 = new Peer(link, 1, io_timeout_ms);
    } catch (...) {
      delete *p0;
      *p0 = nullptr;
      *err = "out of memory";
      return hipErrorOutOfMemory;
    }
    return hipSuccess;
  }
  int sv[2];
  if (::socketpair(AF_UNIX, SOCK_STREAM, 0, sv) != 0) {
    *err = std::string("socketpair: ") + std::strerror(errno);
    return hipErrorNotReady;
  }
  set_io_timeout(sv[0], io_timeout_ms);
  set_io_timeout(sv[1], io_timeout_ms);
  try {
    *p0 = new Peer(sv[0], 0);
    *p1 = new Peer(sv[1], 1);
  } catch (...) {
    delete *p0;
    *p0 = nullptr;
    ::close(sv[1]);
    return hipErrorOutOfMemory;
  }
  return hipSuccess;
}

}  // namespace mpcx
