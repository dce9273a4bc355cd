// The three-tier file reads in flight (dg_disk_queue > 1): reader threads read units into host buffers in pieces (at
// most 8 MiB of one part each), so one unit's read runs on every reader at once. Each read targets one read word (a
// 32-bit word in fine-grained host memory, one per staging buffer, kept-read bank slot and landing block): when its
// last piece has landed the pool runs the unit's finisher (the host hash check with verify_hash 1) and then stores the
// read's generation into the word, which the stream that copies out of the buffer polls first. The word is stored on
// every path (a failed read records its error first), so every await of it ends. At most one read per word is in
// flight: a new read of a word waits for the previous one.
//
// Landing reads (dg_landing_blocks) wait in a second queue (reference src/dg_load.hpp:211-222, docs/design.md 3.15):
// a reader takes a queued demand piece first and a landing piece only while no demand piece is queued, fewer than
// `cap` landing pieces run and (reserve) one reader stays free of them. Pieces are the landing chunk, so a demand read
// queued behind a landing read in progress runs at its next piece boundary (a yield). A landing read that is claimed
// (its unit demanded) becomes a demand read: its queued pieces join the demand queue and it runs to its end. A dropped
// landing read (its unit expired) loses its queued pieces: never started, it is cancelled with nothing read; part-way,
// it ends when its running pieces have (aborted, never copied). A landing read's failure is kept, not reported: a
// claim then finds it Failed, and the demand reads the unit again; a claimed read's failure is reported.
//
// dg_disk_queue_adapt: pieces run at most depth() at a time, the depth chosen by a ReadDepthController fed each busy
// period (from the first piece taken while idle to no piece queued or running: its units and their bytes).
#pragma once

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <exception>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "depth_ctl.hpp"

namespace tsa {

class ReadPool {
 public:
  struct Piece {
    uint32_t part;
    uint64_t off, bytes, dst_off;  // offset inside the part, bytes, offset inside the host buffer
  };
  using PieceReader = std::function<void(uint32_t key, uint32_t part, uint64_t off, uint64_t bytes, char* dst)>;
  using Finisher = std::function<void(uint32_t key, const char* block)>;
  struct LandingRule {
    std::vector<Piece> pieces;  // a landing read's pieces (the landing chunk)
    uint32_t cap = 1;           // landing pieces running at most
    bool reserve = true;        // one reader stays free of landing pieces (false: landing pieces only while fewer
                                // than `cap` pieces of any kind run)
  };
  // Physical landing outcomes: reads dropped before they started; demand reads a part-way landing read gave its
  // readers to; bytes never read of reads dropped part-way; failed landing reads; every byte a landing read did not
  // land (cancelled, aborted, failed); claims of a read still in flight.
  struct LandingCounts {
    uint64_t cancelled = 0, yields = 0, aborted_bytes = 0, failed = 0, unread_bytes = 0, late = 0;
  };
  enum class Claim : uint8_t { Landed, Late, Failed };

  ReadPool(uint32_t threads, uint32_t words, std::vector<Piece> pieces, LandingRule landing, PieceReader read,
           Finisher finish);
  ~ReadPool() { stop(); }
  ReadPool(const ReadPool&) = delete;
  ReadPool& operator=(const ReadPool&) = delete;

  void adapt();  // dg_disk_queue_adapt from now on
  void with_controller(const std::function<void(const ReadDepthController&)>& f);  // under the lock; no-op unless adapting
  // Unclaimed landing reads are dropped, every other queued read finishes; then the readers end.
  void stop();

  // A demand read / a landing read of `key` into `dst` for word w (0 .. words - 1), finished by storing gen there.
  void submit(uint32_t w, uint32_t key, char* dst, uint32_t* word, uint32_t gen) { enqueue(w, key, dst, word, gen, false); }
  void submit_landing(uint32_t w, uint32_t key, char* dst, uint32_t* word, uint32_t gen) {
    enqueue(w, key, dst, word, gen, true);
  }
  // A demand of word w's landing read: Landed (it has landed), Late (still in flight: it is a demand read now) or
  // Failed (it failed: the caller reads the unit again).
  Claim claim(uint32_t w);
  // Word w's landing read will never be copied out (no-op when it has finished or was claimed).
  void drop(uint32_t w);
  // Waits until no read of word w is in flight; returns the ns waited.
  uint64_t wait_idle(uint32_t w);
  // Waits for every demand read (the ns waited); rethrows the first demand read failure not yet reported.
  uint64_t drain();

  uint64_t read_ns() const { return read_ns_.load(std::memory_order_relaxed); }
  uint64_t max_running();
  LandingCounts landing_counts();
  // Test observation: pieces running (all / landing), pieces queued (demand / landing).
  struct Load {
    uint32_t running = 0, landing_running = 0;
    size_t queued = 0, landing_queued = 0;
  };
  Load load();

 private:
  using Clock = std::chrono::steady_clock;
  struct Unit {
    uint32_t w = 0, key = 0, gen = 0;
    char* dst = nullptr;
    uint32_t* word = nullptr;
    uint32_t left = 0, running = 0;  // pieces queued or running; running
    bool landing = false, started = false, dropped = false, failed = false;
    bool finishing = false;  // its last piece ended: the finisher runs (no piece left to take or drop)
    std::exception_ptr err;
  };
  struct Job {
    Unit* unit;
    const Piece* piece;
  };
  void enqueue(uint32_t w, uint32_t key, char* dst, uint32_t* word, uint32_t gen, bool landing);
  bool demand_ready() const { return !q_.empty() && running_ < limit_; }
  bool landing_ready() const;
  void run();
  void finish_locked(Unit& u);  // every piece ended: the word, the counts, the unit gone (lock held)
  void drop_locked(Unit& u);
  uint64_t take_landing_pieces(Unit* u, std::deque<Job>* to);  // u's queued landing pieces out of lq_ (their bytes)
  void set_partway(Unit* u, bool on);  // u: a landing read started with pieces still queued

  std::vector<Piece> pieces_;
  LandingRule land_;
  PieceReader read_;
  Finisher finish_;
  uint64_t unit_bytes_ = 0;
  std::mutex m_;
  std::condition_variable cv_, idle_, word_cv_;
  std::deque<Job> q_, lq_;                  // demand pieces, landing pieces
  std::vector<std::unique_ptr<Unit>> at_;   // per word: its read in flight
  std::vector<uint8_t> failed_;             // per word: its last landing read failed (unclaimed)
  std::vector<Unit*> partway_;              // landing reads started with pieces still queued
  std::vector<std::thread> th_;
  uint32_t threads_ = 0, limit_ = 0;        // readers; pieces that may run at once
  uint32_t running_ = 0, landing_running_ = 0;
  uint64_t demand_inflight_ = 0, max_running_ = 0;
  std::unique_ptr<ReadDepthController> ctl_;
  bool busy_ = false;
  Clock::time_point busy_t0_{};
  uint64_t busy_units_ = 0;
  std::atomic<uint64_t> read_ns_{0};
  LandingCounts lc_;
  std::exception_ptr err_;
  bool stop_ = false;
};

}  // namespace tsa
