// Test hook over the three-tier read pool alone (include/tierstream_amd/tsa_test.h, tsa_test_read_pool): scenarios
// on a pool whose reader blocks each unit's pieces behind a gate the scenario opens, and records the order pieces
// start in and how many run at once. The rules they check are the reference's read pool's (src/dg_load.hpp:211-222,
// its tests tests/test_dg_load.cpp:463-1120): a queued demand read before every queued landing read, at most `cap`
// landing pieces running and one reader kept free of them, a claimed landing read running as a demand, a dropped one
// cancelled or cut short, a landing read's failure kept until it is claimed.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"
#include "read_pool.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {
namespace {

using namespace std::chrono_literals;
constexpr uint64_t kPiece = 4096;
constexpr uint32_t kPieces = 4, kWords = 8, kLandingKey = 1000;  // keys from 1000 on are landing reads

struct Failed : std::runtime_error {
  using std::runtime_error::runtime_error;
};
#define CHECK(c)                                                           \
  do {                                                                     \
    if (!(c)) throw Failed(std::string("line ") + std::to_string(__LINE__) + ": " #c); \
  } while (0)

// The reader: a piece of key k waits until k's gate is open (at most 10 s, then the scenario fails), optionally
// sleeps, and throws for a failing key.
struct Rig {
  std::mutex m;
  std::condition_variable cv;
  std::set<uint32_t> open_keys, fail_keys;
  bool all_open = false, timed_out = false;
  std::vector<std::pair<uint32_t, uint64_t>> starts;  // (key, piece offset) in start order
  std::vector<uint32_t> finished;                     // keys the finisher ran for
  int running = 0, running_land = 0, max_running = 0, max_land = 0;
  std::chrono::microseconds sleep{0};
  std::vector<std::vector<char>> buf = std::vector<std::vector<char>>(kWords, std::vector<char>(kPieces * kPiece));
  uint32_t word[kWords] = {};

  void read(uint32_t key, uint64_t off, uint64_t bytes, char* dst) {
    {
      std::unique_lock<std::mutex> l(m);
      starts.emplace_back(key, off);
      max_running = std::max(max_running, ++running);
      if (key >= kLandingKey) max_land = std::max(max_land, ++running_land);
      if (!cv.wait_for(l, 10s, [&] { return all_open || open_keys.count(key) > 0; })) timed_out = true;
    }
    if (sleep.count()) std::this_thread::sleep_for(sleep);
    std::memset(dst, int(key & 0xff), bytes);
    std::lock_guard<std::mutex> l(m);
    --running;
    if (key >= kLandingKey) --running_land;
    if (fail_keys.count(key)) throw std::runtime_error("injected read failure of key " + std::to_string(key));
  }
  void open(uint32_t key) {
    std::lock_guard<std::mutex> l(m);
    open_keys.insert(key);
    cv.notify_all();
  }
  void open_all() {
    std::lock_guard<std::mutex> l(m);
    all_open = true;
    cv.notify_all();
  }
  size_t started() {
    std::lock_guard<std::mutex> l(m);
    return starts.size();
  }
  std::vector<uint32_t> order() {  // keys in piece start order
    std::lock_guard<std::mutex> l(m);
    std::vector<uint32_t> v;
    for (const auto& s : starts) v.push_back(s.first);
    return v;
  }
  uint32_t load_word(uint32_t w) { return __atomic_load_n(&word[w], __ATOMIC_ACQUIRE); }
};

template <class F>
void spin_until(F f) {
  const auto t0 = std::chrono::steady_clock::now();
  while (!f()) {
    if (std::chrono::steady_clock::now() - t0 > 10s) throw Failed("a condition never came");
    std::this_thread::sleep_for(200us);
  }
}

std::vector<ReadPool::Piece> pieces(uint64_t piece) {
  std::vector<ReadPool::Piece> v;
  for (uint64_t o = 0; o < kPieces * kPiece; o += piece) v.push_back(ReadPool::Piece{0, o, piece, o});
  return v;
}

std::unique_ptr<ReadPool> make(Rig& r, uint32_t threads, uint32_t cap, bool whole = false) {
  ReadPool::LandingRule lr;
  lr.pieces = whole ? pieces(kPieces * kPiece) : pieces(kPiece);
  lr.cap = cap;
  lr.reserve = !whole;
  return std::make_unique<ReadPool>(
      threads, kWords, pieces(kPiece), std::move(lr),
      [&r](uint32_t key, uint32_t, uint64_t off, uint64_t bytes, char* dst) { r.read(key, off, bytes, dst); },
      [&r](uint32_t key, const char*) {
        std::lock_guard<std::mutex> l(r.m);
        r.finished.push_back(key);
      });
}
void demand(ReadPool& p, Rig& r, uint32_t w, uint32_t key, uint32_t gen = 1) {
  p.submit(w, key, r.buf[w].data(), &r.word[w], gen);
}
void landing(ReadPool& p, Rig& r, uint32_t w, uint32_t key, uint32_t gen = 1) {
  p.submit_landing(w, key, r.buf[w].data(), &r.word[w], gen);
}
std::vector<uint32_t> repeat(std::initializer_list<std::pair<uint32_t, uint32_t>> runs) {
  std::vector<uint32_t> v;
  for (const auto& kv : runs) v.insert(v.end(), kv.second, kv.first);
  return v;
}

// 0: one reader busy with a demand read; two landing reads, then a demand read, are queued: the demand read runs
// first, the landing reads after it in their order.
void demand_first() {
  Rig r;
  auto p = make(r, 1, 1);
  demand(*p, r, 0, 1);
  spin_until([&] { return r.started() == 1; });
  landing(*p, r, 1, kLandingKey);
  landing(*p, r, 2, kLandingKey + 1);
  demand(*p, r, 3, 2);
  r.open_all();
  p->drain();
  p->wait_idle(1);
  p->wait_idle(2);
  CHECK(r.order() == repeat({{1, 4}, {2, 4}, {kLandingKey, 4}, {kLandingKey + 1, 4}}));
  for (uint32_t w : {0u, 1u, 2u, 3u}) CHECK(r.load_word(w) == 1);
  CHECK(p->landing_counts().late == 0 && p->landing_counts().cancelled == 0);
}

// 1: four readers, cap 2: eight landing reads never run more than two pieces at once (and do run two); 2: two
// readers, cap 4: one reader stays free of landing reads (one at a time).
void cap_and_reserve(uint32_t threads, uint32_t cap, int want) {
  Rig r;
  r.sleep = 2ms;
  r.all_open = true;
  auto p = make(r, threads, cap);
  for (uint32_t w = 0; w < kWords; ++w) landing(*p, r, w, kLandingKey + w);
  for (uint32_t w = 0; w < kWords; ++w) p->wait_idle(w);
  CHECK(r.max_land == want);
  CHECK(r.started() == kWords * kPieces);
}

// 3: a queued landing read dropped is cancelled (nothing read, its word stored at once); one dropped part-way loses
// its queued pieces (aborted bytes) and ends with its running piece, its finisher never run.
void drop() {
  Rig r;
  auto p = make(r, 1, 1);
  demand(*p, r, 0, 1);
  spin_until([&] { return r.started() == 1; });
  landing(*p, r, 1, kLandingKey, 7);
  p->drop(1);
  CHECK(r.load_word(1) == 7);
  CHECK(p->wait_idle(1) == 0);
  CHECK(p->landing_counts().cancelled == 1);
  landing(*p, r, 2, kLandingKey + 1, 9);
  r.open(1);
  spin_until([&] { return r.started() == 5; });  // the landing's first piece is running
  p->drop(2);
  r.open(kLandingKey + 1);
  p->wait_idle(2);
  CHECK(r.load_word(2) == 9);
  const ReadPool::LandingCounts c = p->landing_counts();
  CHECK(c.cancelled == 1 && c.aborted_bytes == 3 * kPiece && c.unread_bytes == 7 * kPiece);
  CHECK(r.order() == repeat({{1, 4}, {kLandingKey + 1, 1}}));
  std::lock_guard<std::mutex> l(r.m);
  CHECK(r.finished == std::vector<uint32_t>{1});
}

// 4: a claimed landing read runs as a demand read: ahead of the landing reads queued before it, and drain waits
// for it; a claim after it landed finds it Landed.
void claim() {
  Rig r;
  auto p = make(r, 1, 1);
  demand(*p, r, 0, 1);
  spin_until([&] { return r.started() == 1; });
  landing(*p, r, 1, kLandingKey);
  landing(*p, r, 2, kLandingKey + 1);
  CHECK(p->claim(2) == ReadPool::Claim::Late);
  r.open_all();
  p->drain();
  CHECK(r.load_word(2) == 1);  // (drain waited for the claimed read)
  p->wait_idle(1);
  CHECK(r.order() == repeat({{1, 4}, {kLandingKey + 1, 4}, {kLandingKey, 4}}));
  CHECK(p->claim(1) == ReadPool::Claim::Landed);
  CHECK(p->landing_counts().late == 1);
}

// 5: a landing read that fails is not reported (drain passes) and a claim finds it Failed; a claimed one that then
// fails is reported by drain.
void failures() {
  Rig r;
  r.fail_keys = {kLandingKey, kLandingKey + 1};
  auto p = make(r, 2, 1);
  r.open(kLandingKey);
  landing(*p, r, 0, kLandingKey);
  p->wait_idle(0);
  p->drain();
  CHECK(r.load_word(0) == 1);
  CHECK(p->landing_counts().failed == 1 && p->landing_counts().unread_bytes == kPieces * kPiece);
  CHECK(p->claim(0) == ReadPool::Claim::Failed);
  landing(*p, r, 1, kLandingKey + 1);
  spin_until([&] { return r.started() >= 5; });
  CHECK(p->claim(1) == ReadPool::Claim::Late);
  r.open(kLandingKey + 1);
  bool threw = false;
  try {
    p->drain();
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw);
  CHECK(r.load_word(1) == 1);  // (the word is stored on failure too)
}

// 6: a landing read part-way yields to a demand read submitted meanwhile: the demand's pieces run before its
// remaining ones (one yield).
void yields() {
  Rig r;
  auto p = make(r, 1, 1);
  landing(*p, r, 0, kLandingKey);
  spin_until([&] { return r.started() == 1; });
  demand(*p, r, 1, 1);
  r.open_all();
  p->drain();
  p->wait_idle(0);
  CHECK(r.order() == repeat({{kLandingKey, 1}, {1, 4}, {kLandingKey, 3}}));
  CHECK(p->landing_counts().yields == 1);
}

// 10: no yield while idle readers take the demand read: five readers, one running a landing read's first piece, the
// four others take the demand read's four pieces at once; the landing read then runs to its end.
void no_yield_with_idle_readers() {
  Rig r;
  auto p = make(r, 5, 1);
  landing(*p, r, 0, kLandingKey);
  spin_until([&] { return r.started() == 1; });
  demand(*p, r, 1, 1);
  spin_until([&] { return r.started() == 5; });
  r.open_all();
  p->drain();
  p->wait_idle(0);
  CHECK(r.order() == repeat({{kLandingKey, 1}, {1, 4}, {kLandingKey, 3}}));
  CHECK(p->landing_counts().yields == 0);
}

// 7: whole landing reads (no chunks, no reserve): a landing read starts only while fewer than `cap` pieces of any kind
// run, in one piece.
void whole() {
  Rig r;
  auto p = make(r, 2, 1, true);
  demand(*p, r, 0, 1);
  spin_until([&] { return r.started() == 2; });  // both readers on the demand read
  landing(*p, r, 1, kLandingKey);
  std::this_thread::sleep_for(20ms);
  CHECK(r.started() == 2);
  r.open(1);
  p->drain();
  r.open(kLandingKey);
  p->wait_idle(1);
  CHECK(r.order() == repeat({{1, 4}, {kLandingKey, 1}}));
}

// 8: stop drops a landing read nobody claimed (never read) and finishes the demand reads.
void stop_drops() {
  Rig r;
  auto p = make(r, 1, 1);
  demand(*p, r, 0, 1);
  spin_until([&] { return r.started() == 1; });
  landing(*p, r, 1, kLandingKey);
  std::thread opener([&] {
    std::this_thread::sleep_for(20ms);
    r.open_all();
  });
  p->stop();
  opener.join();
  CHECK(r.order() == repeat({{1, 4}}));
  CHECK(p->landing_counts().cancelled == 1);
  CHECK(r.load_word(0) == 1 && r.load_word(1) == 1);
}

// 9: wait_idle returns only once the word's read ended; a second read of a word waits for the first.
void word_order() {
  Rig r;
  auto p = make(r, 2, 1);
  landing(*p, r, 0, kLandingKey, 1);
  spin_until([&] { return r.started() >= 1; });
  std::atomic<bool> back{false};
  std::thread t([&] {
    landing(*p, r, 0, kLandingKey + 1, 2);  // waits for the first read of word 0
    back = true;
  });
  std::this_thread::sleep_for(20ms);
  const bool early = back.load();
  r.open(kLandingKey);
  t.join();
  CHECK(!early);
  CHECK(r.load_word(0) == 1);
  r.open(kLandingKey + 1);
  p->wait_idle(0);
  CHECK(r.load_word(0) == 2);
}

}  // namespace
}  // namespace tsa

extern "C" ss_status tsa_test_read_pool(uint32_t scenario, char* msg, uint32_t cap) {
  using namespace tsa;
  if (msg && cap) msg[0] = '\0';
  try {
    switch (scenario) {
      case 0: demand_first(); break;
      case 1: cap_and_reserve(4, 2, 2); break;
      case 2: cap_and_reserve(2, 4, 1); break;
      case 3: drop(); break;
      case 4: claim(); break;
      case 5: failures(); break;
      case 6: yields(); break;
      case 7: whole(); break;
      case 8: stop_drops(); break;
      case 9: word_order(); break;
      case 10: no_yield_with_idle_readers(); break;
      default: return SS_E_INVALID;
    }
    return SS_OK;
  } catch (const std::exception& e) {
    if (msg && cap) std::snprintf(msg, cap, "%s", e.what());
    return SS_E_BACKEND;
  }
}
