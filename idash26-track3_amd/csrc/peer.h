// peer.h -- one party's end of the two-party channel (one process, or one
// thread, per party).
//
// Replaces the reference's GpuPeer / SigmaPeer (gpu_mpc/utils/gpu_comms.h:94-397,
// gpu_mpc/utils/sigma_comms.cpp:36-150): a connected stream socket between the
// two parties, a background sender so that both parties can send a large message
// at the same time, and device <-> pinned-host staging around each exchange.
// Messages are sent exactly as counted: ring elements at their width, bit planes
// packed 32 per 32-bit word (the reference's bit-packed wire format for bit
// outputs, gpu_comms.h:28-73).
#pragma once
#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace mpcx {

struct LocalLink;  // the shared state of two ends in one process (peer.hip)

class Peer {
 public:
  // One region of an exchange: `bytes` of device memory `send` go to the peer,
  // the peer's matching region lands in device memory `recv`.
  struct Seg {
    const void *send;
    void *recv;
    size_t bytes;
  };

  Peer(int fd, int party);
  // An end of an in-process pair: messages go device to device (no staging,
  // no socket), ordered by events on the two parties' streams.
  Peer(std::shared_ptr<LocalLink> link, int party, int io_timeout_ms);
  ~Peer();
  Peer(const Peer &) = delete;
  Peer &operator=(const Peer &) = delete;

  int party() const { return party_; }
  // Stages the segments (produced on `stream`) back to back, sends them while
  // receiving the peer's, and enqueues the copies of the peer's segments into
  // the recv regions on `stream`.  hipErrorNotReady: the channel failed (peer
  // gone, timeout); the peer is unusable afterwards.
  hipError_t exchange(hipStream_t stream, const Seg *segs, int nseg);
  // chunk of the pipelined staging, and the largest message sent inline (the
  // per-sample products of a GCN layer are 44-88 KB)
  static constexpr size_t kChunk = size_t(4) << 20, kInline = size_t(128) << 10;
  uint64_t bytes_sent() const { return sent_; }
  uint64_t bytes_received() const { return recv_; }
  uint64_t rounds() const { return rounds_; }
  // 2 linked in memory (in-process pair), 1 IPC inboxes, 0 staged through the
  // socket, -1 not yet decided (a cross-process channel before its first exchange)
  int transport() const { return link_ ? 2 : ipc_state_ == 1 ? 1 : (cross_process_ && ipc_state_ < 0) ? -1 : 0; }
  const std::string &error() const { return err_; }

 private:
  hipError_t ensure(size_t bytes);
  hipError_t ensure_events(size_t n);
  hipError_t exchange_local(hipStream_t stream, const Seg *segs, int nseg, size_t total);
  hipError_t exchange_socket(hipStream_t stream, const Seg *segs, int nseg, size_t total);
  hipError_t exchange_ipc(hipStream_t stream, const Seg *segs, int nseg, size_t total);
  hipError_t ipc_negotiate();
  hipError_t ipc_grow(size_t bytes);
  bool token(char t);  // sends t, receives the peer's token, checks it is t
  void sender_loop();
  bool send_all(const uint8_t *p, size_t n);
  bool recv_all(uint8_t *p, size_t n);

  int fd_ = -1, party_ = 0;
  uint8_t *hs_ = nullptr, *hr_ = nullptr;  // pinned staging (send, receive)
  std::vector<hipEvent_t> ev_;              // one per staged chunk of the current message
  size_t inline_max_ = size_t(16) << 10;    // set from the socket's send buffer
  size_t cap_ = 0;
  uint64_t sent_ = 0, recv_ = 0, rounds_ = 0;
  bool broken_ = false;
  std::string err_;
  // background sender: one job at a time
  std::thread th_;
  std::mutex mu_;
  std::condition_variable cv_;
  const uint8_t *job_ = nullptr;
  size_t job_n_ = 0;
  bool job_ready_ = false, job_done_ = true, job_ok_ = true, stop_ = false;
  // two processes on one GPU (peer_connect): device inboxes mapped into the
  // peer process (IPC), negotiated at the first exchange
 public:
  static constexpr size_t kIpcMin = size_t(16) << 20, kIpcMax = size_t(1) << 30;
  bool ipc() const { return ipc_state_ == 1; }

 private:
  bool cross_process_ = false;
  int ipc_state_ = -1;  // -1 not negotiated, 0 staged socket, 1 IPC
  void *inbox_ = nullptr, *peer_inbox_ = nullptr;
  size_t inbox_cap_ = 0;
  hipEvent_t ipc_ev_[2] = {nullptr, nullptr};  // message written into the peer's inbox; own inbox read
  bool read_pending_ = false;
  friend hipError_t peer_connect(int, const std::string &, int, int, Peer **, std::string *);
  // in-process pair
  std::shared_ptr<LocalLink> link_;
  hipEvent_t lev_[2] = {nullptr, nullptr};  // this end's message ready, the peer's message consumed
  int io_timeout_ms_ = 0;
};

// Party 0 listens on the Unix socket `path` and accepts one connection; party 1
// connects to it (retrying until timeout_ms).  Receives time out after
// io_timeout_ms of silence.  When both processes run on the same GPU (and
// neither sets MPCX_PEER_IPC=0), each exchange writes this party's message
// straight into the peer's device inbox, mapped into this process by an IPC
// memory handle, with one-byte tokens on the socket for the ordering; messages
// over kIpcMax bytes, and every exchange otherwise, are staged through pinned
// host memory and the socket.
hipError_t peer_connect(int party, const std::string &path, int timeout_ms, int io_timeout_ms, Peer **out,
                        std::string *err);
// Both ends of one channel, for two parties as two threads of one process:
// linked in memory, each exchange a pair of device-to-device copies ordered by
// events (socket = true: a socket pair, staged as between processes).
hipError_t peer_pair(int io_timeout_ms, Peer **p0, Peer **p1, std::string *err, bool socket = false);

}  // namespace mpcx
