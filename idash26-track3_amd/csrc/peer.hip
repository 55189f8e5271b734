// peer.hip -- socket channel between the two parties (host code only).
#include "peer.h"

#include <poll.h>
#include <sys/socket.h>
#include <sys/time.h>
#include <sys/un.h>
#include <unistd.h>

#include <cerrno>
#include <chrono>
#include <cstring>

namespace mpcx {

Peer::Peer(int fd, int party) : fd_(fd), party_(party) { th_ = std::thread([this] { sender_loop(); }); }

Peer::~Peer() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  if (th_.joinable()) th_.join();
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

void Peer::sender_loop() {
  std::unique_lock<std::mutex> lk(mu_);
  for (;;) {
    cv_.wait(lk, [this] { return stop_ || job_ready_; });
    if (stop_) return;
    const uint8_t *p = job_;
    const size_t n = job_n_;
    job_ready_ = false;
    lk.unlock();
    const bool ok = send_all(p, n);
    lk.lock();
    job_ok_ = ok;
    job_done_ = true;
    cv_.notify_all();
  }
}

hipError_t Peer::exchange(hipStream_t stream, const Seg *segs, int nseg) {
  if (broken_) return hipErrorNotReady;
  size_t total = 0;
  for (int k = 0; k < nseg; k++) total += segs[k].bytes;
  rounds_++;
  if (total == 0) return hipSuccess;
  hipError_t e = ensure(total);
  if (e != hipSuccess) return e;
  size_t o = 0;
  for (int k = 0; k < nseg; k++) {
    if (segs[k].bytes) {
      e = hipMemcpyAsync(hs_ + o, segs[k].send, segs[k].bytes, hipMemcpyDeviceToHost, stream);
      if (e != hipSuccess) return e;
    }
    o += segs[k].bytes;
  }
  // the messages are complete, and the previous exchange's copies out of hr_ done
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(mu_);
    job_ = hs_;
    job_n_ = total;
    job_ready_ = true;
    job_done_ = false;
  }
  cv_.notify_all();
  const bool rok = recv_all(hr_, total);
  bool sok;
  {
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
  sent_ += total;
  recv_ += total;
  o = 0;
  for (int k = 0; k < nseg; k++) {
    if (segs[k].bytes) {
      e = hipMemcpyAsync(segs[k].recv, hr_ + o, segs[k].bytes, hipMemcpyHostToDevice, stream);
      if (e != hipSuccess) return e;
    }
    o += segs[k].bytes;
  }
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
  return hipSuccess;
}

hipError_t peer_pair(int io_timeout_ms, Peer **p0, Peer **p1, std::string *err) {
  *p0 = *p1 = nullptr;
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
