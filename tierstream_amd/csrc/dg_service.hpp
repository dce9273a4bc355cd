// The device-gated context's service thread: it serves every token the engine opens with ss_begin. For each gated layer
// the token exports, in layer order, it waits for the layer's export flag in the mapped control area, validates the
// record, has the core serve the misses (copies, device checks, the layer's ready word), records the uses, serves the
// next layer's prediction when the export promised one, and spends the layer's write-back credit. The protocol (its
// words, records and the errors a token fails on) is the reference's device-gated service (src/dg_service.cpp:116-365);
// the structure is this library's:
//  * Poller: one wait on a mapped word with a time-based schedule - pause instructions for the first stretch of the
//    wait, then (where a wait may be long) a yield per poll - and slow checks (stop, deadline, host abort) once every
//    64 polls;
//  * a token's plan (its exported gated layers, fixed at ss_begin) and a validated layer record;
//  * the outcome of the last token, published as two words: the last sequence served in full, and a halt state once
//    the thread has ended (failed, with its first error, or stopped). ss_end reads both.
#pragma once

#include <atomic>
#include <chrono>
#include <cstdint>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "dg_core.hpp"
#include "dg_proto.hpp"

namespace tsa {

class DgService {
 public:
  using Clock = std::chrono::steady_clock;
  enum class Outcome { kPending, kServed, kFailed, kStopped };
  // dg_diag: one gated layer's row of the last token served (host times in microseconds; the counters' deltas)
  struct Row {
    double seen_us = 0, demand_us = 0, pred_wait_us = 0, prefetch_us = 0, serve_us = 0;
    uint32_t ids = 0, misses = 0, covered = 0, fetched = 0, prefetched = 0, predicted_true = 0, covered_waits = 0;
  };

  DgService(DgCore* core, const DgMappedHost& m, uint32_t max_ids, uint32_t timeout_ms, int device);
  ~DgService() { stop_join(); }
  DgService(const DgService&) = delete;
  DgService& operator=(const DgService&) = delete;

  // The transport's work on the service thread: between two polls of a mapped word (queued device checks whose copies
  // have landed are launched), and after a token's last layer, before it counts as served (every queued check
  // launched: each layer's ready word depends on one).
  struct Hooks {
    std::function<void()> while_waiting, before_served;
  };
  std::thread::id thread_id() const { return th_.get_id(); }
  void set_hooks(Hooks h) { hooks_ = std::move(h); }
  void enable_timeline();
  const std::vector<Row>& timeline() const { return rows_; }  // between tokens only (ordered by the outcome word)
  void start();
  // ss_begin: the token's exported gated layers (run[g] != 0) and its sequence, published to the thread.
  void begin(uint32_t seq, const std::vector<uint8_t>& run);
  // The outcome of token seq: kServed once the thread served it in full; kFailed / kStopped once the thread ended;
  // kPending when the deadline passed first.
  Outcome wait_outcome(uint32_t seq, Clock::time_point deadline) const;
  void stop_join();  // the thread ends (a token in service is abandoned; the device's waits end on host_abort)
  std::string error() const;

 private:
  struct Stop {};  // unwinds a token when the thread is told to stop
  class Poller;
  struct Record {  // a validated export record
    std::vector<uint32_t> ids;
    uint64_t dev_mask = 0;
    uint32_t n_pred = 0;
  };

  void thread_main(uint32_t last_seen);
  void halt(Outcome o, const std::string& why);
  void serve(uint32_t seq);
  void serve_layer(uint32_t seq, uint32_t g, uint32_t next);
  Record read_record(uint32_t seq, uint32_t g) const;
  void await_flag(const uint32_t* w, uint32_t seq, uint32_t g, const char* what, const uint32_t* last);
  void await_began(uint32_t seq);

  DgCore* core_;
  Hooks hooks_;
  DgMappedHost m_;
  uint32_t max_ids_;
  std::chrono::milliseconds timeout_;
  int device_;
  uint32_t G_;
  std::vector<uint8_t> next_run_;     // written by begin() before its sequence is published
  std::vector<uint8_t> run_;          // the token in service's exported layers (the core reads it until the boundary)
  std::vector<uint32_t> plan_;        // this token's exported gated layers, in order
  std::vector<uint32_t> flag_seen_;   // per gated layer: the sequence its export flag held after its last export
  std::vector<uint32_t> pred_;
  bool diag_ = false;
  std::vector<Row> rows_;
  Clock::time_point last_end_{};      // the origin of the next token's first seen_us
  std::atomic<uint32_t> opened_{0};   // the sequence ss_begin published
  std::atomic<uint32_t> served_{0};   // the last sequence served in full
  std::atomic<int> halted_{0};        // 0 while running, else the Outcome the thread ended with
  std::atomic<bool> stop_{false};
  mutable std::mutex err_mu_;
  std::string err_;
  std::thread th_;
};

}  // namespace tsa
