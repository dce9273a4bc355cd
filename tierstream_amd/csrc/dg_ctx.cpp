#include "dg_ctx.hpp"

#include <hip/hip_runtime_api.h>
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <exception>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "dg_core.hpp"
#include "depth_ctl.hpp"
#include "dg_geometry.hpp"
#include "dg_proto.hpp"
#include "dg_service.hpp"
#include "hip_rt.hpp"
#include "hsa_copy.hpp"
#include "read_pool.hpp"
#include "score_profile.hpp"
#include "source.hpp"
#include "stats_json.hpp"
#include "tsa_device.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {
namespace {

using Clock = std::chrono::steady_clock;
// The device check's checkpoint segment (a quad of lanes per segment): 2 KiB for every unit size, 32 B of
// checkpoints per segment (1.6 % of the unit). Measured live on the Mixtral shape (336 MiB units, 64-token runs):
// 8 KiB 0.549 of the HBM peak, 4 KiB 0.562, 2 KiB 0.581, 1 KiB 0.475, 512 B 0.300; a small unit (the DeepSeek
// shape's 24.8 MB) needs segments this small for its check to fill the chip at all.
uint64_t verify_seg_bytes(uint64_t) { return 2 * 1024; }
constexpr uint64_t kScatterBelow = 8ull << 20;     // parts smaller than this land staged + scattered
constexpr uint64_t kReadPiece = 8ull << 20;        // three-tier reads in flight: the largest piece one reader reads

uint64_t align64(uint64_t v) { return (v + 63) / 64 * 64; }

// The open's geometry and refusals: dg_geometry.hpp.
using Layout = DgGeometry;

// ---- fine-grained control area layout ----
struct MappedLayout {
  uint64_t rec, prec, flag, pflag, words, total;
};
MappedLayout mapped_layout(uint32_t G) {
  MappedLayout m;
  m.rec = 0;
  m.prec = align64(m.rec + uint64_t(G) * sizeof(DgRecord));
  m.flag = align64(m.prec + uint64_t(G) * sizeof(DgPredRecord));
  m.pflag = align64(m.flag + uint64_t(G) * 4);
  m.words = align64(m.pflag + uint64_t(G) * 4);
  m.total = align64(m.words + 8 * 4);
  return m;
}

// ---- the HIP transport ----------------------------------------------------------------------------------------------
class HipTransport final : public DgTransport {
 public:
  // max_copies: the most unit copies one stream can enqueue between two boundaries (the boundary synchronizes the
  // copy streams, so a scatter job entry is never rewritten while its upload may still be pending)
  HipTransport(HipDevice* dev, const Layout& x, std::vector<void*> arena, int32_t* slot_of_dev, uint32_t* ready_dev,
               std::vector<void*> block_chunks, uint64_t blocks_per_chunk, uint32_t max_copies)
      : dev_(dev), x_(x), arena_(std::move(arena)), slot_of_(slot_of_dev), ready_(ready_dev),
        chunks_(std::move(block_chunks)), per_chunk_(blocks_per_chunk), kJobRing(max_copies + 8) {
    for (auto& s : s_) s = dev_->stream_create_dedicated();
    part_ev_.assign((size_t(x_.slots) + size_t(x_.blocks)) * x_.part_bytes.size(), nullptr);
    stage_host_ = static_cast<int32_t*>(dev_->alloc_pinned(4ull * x_.keys, "slot table upload stage"));
    bool small = false;
    for (uint64_t pb : x_.part_bytes) small = small || pb < kScatterBelow;
    scatter_ = small && x_.part_bytes.size() > 1;
    if (scatter_) {
      for (int k = 0; k < 2; ++k) {
        stage_dev_[k] = dev_->alloc_device(x_.unit_bytes, "scatter staging");
        jobs_host_[k] = static_cast<tsa_scatter_job*>(dev_->alloc_pinned(sizeof(tsa_scatter_job) * kJobRing, "jobs"));
        jobs_dev_[k] = static_cast<tsa_scatter_job*>(dev_->alloc_device(sizeof(tsa_scatter_job) * kJobRing, "jobs"));
      }
      scatter_blocks_ = tsa_scatter_blocks(x_.part_bytes.data(), uint32_t(x_.part_bytes.size()));
    }
  }
  ~HipTransport() override {
    if (hsa_) hsa_->wait_all();  // every copy out of and into the context's memory has ended
    if (pool_) pool_->stop();  // every read's word stored: no await left waiting on the streams below
    if (vs_) (void)hipStreamSynchronize(vs_);
    for (auto& s : s_) {
      (void)hipStreamSynchronize(s);
      dev_->stream_destroy(s);
    }
    dev_->free_pinned(stage_host_);
    for (int k = 0; k < 2; ++k) {
      dev_->free_device(stage_dev_[k]);
      dev_->free_pinned(jobs_host_[k]);
      dev_->free_device(jobs_dev_[k]);
    }
    dev_->free_device(digests_dev_);
    dev_->stream_destroy(vs_);
    for (hipEvent_t e : vev_) dev_->event_destroy(e);
    for (hipEvent_t e : part_ev_) dev_->event_destroy(e);
    dev_->free_pinned(vfail_host_);
    dev_->free_device(vfail_dev_);
    for (hipEvent_t e : prof_events_) dev_->event_destroy(e);
    for (char* b : stage_) dev_->free_pinned(b);
    for (void* c : land_chunks_) dev_->free_pinned(c);
    for (hipEvent_t e : land_copy_ev_) dev_->event_destroy(e);
    for (auto* v : {&dma_a_, &dma_b_, &dma_f_})
      for (hipEvent_t e : *v) dev_->event_destroy(e);
    for (hipEvent_t e : wb_end_) dev_->event_destroy(e);
    dev_->free_pinned(rword_host_);
  }

  hipStream_t stream(Stream s) const { return s_[s]; }

  // Unit copies through the HSA runtime (HsaCopier) instead of the HIP streams, possible where every part is copied
  // whole (no scatter) and no file tier reads into the blocks (its reads order the copies behind device waits).
  // Decided before the core makes its first event. Each library stream is then a lane: `tail_` holds the copies
  // (signals, one reference each) its next operation waits for - its last copy and what wait() added since - and the
  // core's events are Marks, the tail of the lane they were recorded on. A lane's value writes (slot entries, ready
  // words) and timing marks go through the host-launched queue of checks, behind the copies they follow, on one HIP
  // stream; no HIP stream carries a unit copy.
  bool enable_hsa_copies(int device) {
    if (scatter_ || reader_) return false;
    hsa_ = std::make_unique<HsaCopier>(device);
    part_sig_.assign(part_ev_.size(), 0);
    return true;
  }
  bool hsa_copies() const { return hsa_ != nullptr; }
  // blocks 0 .. blocks - 1: the pinned homes and spares (in chunks); blocks .. blocks + S - 1: the staging buffers;
  // blocks + S .. blocks + S + L - 1: the landing blocks (in chunks)
  char* block_ptr(int32_t b) const {
    if (uint32_t(b) >= x_.blocks + x_.S) {
      const uint64_t l = uint32_t(b) - x_.blocks - x_.S;
      return static_cast<char*>(land_chunks_[size_t(l / land_per_chunk_)]) + (l % land_per_chunk_) * x_.host_stride;
    }
    if (uint32_t(b) >= x_.blocks) return stage_[size_t(uint32_t(b) - x_.blocks)];
    return static_cast<char*>(chunks_[size_t(uint64_t(b) / per_chunk_)]) + (uint64_t(b) % per_chunk_) * x_.host_stride;
  }
  bool landing_block(int32_t b) const { return uint32_t(b) >= x_.blocks + x_.S; }
  // Three-tier: the staging buffers (pinned, one host stride each) and the context's readers of a key's file bytes
  // (the whole unit; a piece of a part) and its finisher; with x_.disk_queue > 1 a read pool, one word per staging
  // buffer in fine-grained host memory (then one per bank slot with dg_bank_keep, then one per landing block) and the
  // landing blocks (pinned, in chunks of at most 1 GiB).
  void enable_disk(std::function<void(uint32_t, char*)> reader, ReadPool::PieceReader piece_reader,
                   ReadPool::Finisher finisher, const DgDevWords& dw) {
    require(!hsa_, SS_E_BACKEND, "device-gated: the file tier with copies through the HSA runtime");
    reader_ = std::move(reader);
    for (uint32_t i = 0; i < x_.S; ++i)
      stage_.push_back(static_cast<char*>(dev_->alloc_pinned(x_.host_stride, "disk staging buffer")));
    if (x_.disk_queue > 1) {
      land_word0_ = x_.S + (x_.bank_keep ? 2 * x_.B : 0);
      const uint32_t words = land_word0_ + x_.L;
      rword_host_ = static_cast<uint32_t*>(dev_->alloc_mapped(4ull * words, &rword_dev_, "read words"));
      std::memset(rword_host_, 0, 4ull * words);
      rgen_.assign(words, 0);
      rpending_.assign(words, 0);
      raux_.assign(words, 0);
      dw_ = dw;
      const auto slices = [&](uint64_t piece) {  // slices of each part (4 KiB-aligned; the last one the rest)
        std::vector<ReadPool::Piece> v;
        for (uint32_t p = 0; p < x_.part_bytes.size(); ++p) {
          const uint64_t step = piece ? piece : x_.part_bytes[p];
          for (uint64_t o = 0; o < x_.part_bytes[p]; o += step)
            v.push_back(ReadPool::Piece{p, o, std::min(step, x_.part_bytes[p] - o), x_.part_offset[p] + o});
        }
        return v;
      };
      ReadPool::LandingRule lr;
      if (x_.L) {
        land_per_chunk_ = std::max<uint64_t>(1, kPinnedChunk / x_.host_stride);
        for (uint64_t left = x_.L; left > 0;) {
          const uint64_t n = std::min(land_per_chunk_, left);
          land_chunks_.push_back(dev_->alloc_pinned(n * x_.host_stride, "landing blocks"));
          left -= n;
        }
        land_copy_ev_.assign(x_.L, nullptr);
        land_key_.assign(x_.L, 0);
        lr.pieces = slices(x_.landing_chunk);
        lr.cap = x_.landing_queued;
        lr.reserve = x_.landing_chunk != 0;  // (whole reads: at most `cap` reads of any kind, as before chunks)
      }
      pool_ = std::make_unique<ReadPool>(x_.disk_queue, words, slices(kReadPiece), std::move(lr),
                                         std::move(piece_reader), std::move(finisher));
    }
  }
  // A file read into staging buffer `block`, or (dg_bank_keep) into pinned block `block` for bank slot `slot`:
  // synchronous, or queued to the pool (the copy out of the block then awaits the read's word: a staging buffer's, or
  // the bank slot's, which is reused only once the copy that awaited it last has run).
  void read_unit(uint32_t key, int32_t block, int32_t slot) override {
    const bool staged = uint32_t(block) >= x_.blocks && uint32_t(block) < x_.blocks + x_.S;
    const bool kept = !staged && x_.bank_keep && slot >= int32_t(x_.persistent_slots) &&
                      uint32_t(slot) < x_.persistent_slots + 2 * x_.B;
    require(reader_ && (staged || kept), SS_E_BACKEND,
            "device-gated: a file read into neither a staging buffer nor a kept block");
    if (!pool_) {
      const auto t0 = Clock::now();
      reader_(key, block_ptr(block));
      const uint64_t ns = uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0).count());
      read_ns_ += ns;
      read_wait_ns_ += ns;
      return;
    }
    const uint32_t i = staged ? uint32_t(block) - x_.blocks : x_.S + (uint32_t(slot) - x_.persistent_slots);
    if (++rgen_[i] == 0) rgen_[i] = 1;  // (0 is the word's initial value)
    rpending_[i] = rgen_[i];
    raux_[i] = gated_of(key);
    if (!staged) kept_word_[block] = i;
    pool_->submit(i, key, block_ptr(block), rword_host_ + i, rgen_[i]);
  }
  uint32_t gated_of(uint32_t key) const {
    return uint32_t(std::upper_bound(x_.unit_base.begin(), x_.unit_base.end(), key) - x_.unit_base.begin()) - 1;
  }
  // A landing read into landing block `block`, on the pool's landing queue. The block's previous read (a landing
  // dropped while it ran) and its last copy out (a promotion's) end first: waited for here, on the host.
  void read_landing(uint32_t key, int32_t block) override {
    require(pool_ && landing_block(block), SS_E_BACKEND, "device-gated: a landing read without landing blocks");
    const uint32_t l = uint32_t(block) - x_.blocks - x_.S, i = land_word0_ + l;
    const auto t0 = Clock::now();
    bool waited = pool_->wait_idle(i) > 0;
    if (hipEvent_t e = land_copy_ev_[l]; e && !ev_done(e)) {
      ev_sync(e);
      waited = true;
    }
    if (waited)
      land_wait_ns_ += uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0).count());
    if (++rgen_[i] == 0) rgen_[i] = 1;
    rpending_[i] = rgen_[i];
    raux_[i] = gated_of(key);
    land_key_[l] = key;
    pool_->submit_landing(i, key, block_ptr(block), rword_host_ + i, rgen_[i]);
  }
  void drop_landing(int32_t block) override {
    if (pool_ && landing_block(block)) pool_->drop(land_word0_ + (uint32_t(block) - x_.blocks - x_.S));
  }
  // dg_diag: per gated layer three timed events (before its first copy on the demand stream, after its first miss's
  // copies there, after its ready word on the stream that writes it) and the boundary's write-back end, alternating
  // between two events so that a token is compared with the boundary before it.
  void enable_diag(uint32_t G) {
    for (auto* v : {&dma_a_, &dma_b_, &dma_f_})
      for (uint32_t g = 0; g < G; ++g) v->push_back(dev_->event_create_timed());
    dma_used_.assign(G, 0);
    for (hipEvent_t& e : wb_end_) e = dev_->event_create_timed();
    diag_ = true;
  }
  void diag_mark(uint32_t g, int which) override {
    if (!diag_ || g >= dma_used_.size()) return;
    if (which == 0) {
      ev_record(dma_a_[g], s_[kDem]);
      dma_used_[g] = 1;
    } else if (which == 2) {
      dma_used_[g] = 2;
      if (!hsa_) return ev_record(dma_f_[g], s_[kDem]);
      Check c;  // (with HSA copies: once the layer's copies so far have ended)
      c.kind = Check::kMark;
      c.mark = dma_f_[g];
      hold(c.sigs, tail_[kDem]);
      checks_.push_back(std::move(c));
      poll_checks();
    } else if ((verify_ && !fused()) || hsa_) {  // after the layer's ready word, in the order of the checks
      Check c;
      c.kind = Check::kMark;
      c.mark = dma_b_[g];
      checks_.push_back(std::move(c));
      poll_checks();
    } else {
      ev_record(dma_b_[g], s_[kDem]);
    }
  }
  void diag_boundary() override {
    if (!diag_) return;
    wb_prev_ = wb_cur_;
    wb_prev_valid_ = wb_cur_valid_;
    wb_cur_ ^= 1;
    wb_cur_valid_ = false;
  }
  void diag_writebacks_issued() override {
    if (!diag_) return;
    wb_cur_valid_ = true;
    if (!hsa_) return ev_record(wb_end_[wb_cur_], s_[kD2h]);
    drop(wb_sigs_[wb_cur_]);  // (with HSA copies: recorded when a poll of the queue sees the write-backs ended)
    hold(wb_sigs_[wb_cur_], tail_[kD2h]);
    wb_seen_[wb_cur_] = false;
    poll_wb_marks();
  }
  void poll_wb_marks() {
    if (!diag_ || !hsa_) return;
    for (int i = 0; i < 2; ++i)
      if (!wb_seen_[i] && all_done(wb_sigs_[i])) {
        ev_record(wb_end_[i], s_[kD2h]);
        drop(wb_sigs_[i]);
        wb_seen_[i] = true;
      }
  }
  struct LayerDma {
    double dma_ms = -1, dma_first_ms = -1, wb_left_ms = -1;
  };
  // After the boundary: per marked layer the times between its marks, and how long the previous boundary's
  // write-backs ran past its first mark (-2: still running now). Never throws (a timing error gives -1).
  std::vector<LayerDma> diag_collect() {
    std::vector<LayerDma> out(dma_used_.size());
    if (!diag_) return out;
    int wb = 0;
    poll_wb_marks();
    if (wb_prev_valid_ && hsa_ && !wb_seen_[wb_prev_]) {
      wb = -2;
    } else if (wb_prev_valid_) {
      const hipError_t q = hipEventQuery(wb_end_[wb_prev_]);
      wb = q == hipSuccess ? 1 : q == hipErrorNotReady ? -2 : 0;
    }
    const auto elapsed = [](hipEvent_t a, hipEvent_t b) {
      float ms = 0;
      if (hipEventSynchronize(b) != hipSuccess) return -1.0;
      return hipEventElapsedTime(&ms, a, b) == hipSuccess ? double(ms) : -1.0;
    };
    for (size_t g = 0; g < dma_used_.size(); ++g) {
      if (!dma_used_[g]) continue;
      LayerDma& d = out[g];
      d.dma_ms = elapsed(dma_a_[g], dma_b_[g]);
      if (dma_used_[g] == 2) d.dma_first_ms = elapsed(dma_a_[g], dma_f_[g]);
      dma_used_[g] = 0;
      if (wb == 1) {
        const double ms = elapsed(dma_a_[g], wb_end_[wb_prev_]);
        d.wb_left_ms = ms == -1.0 ? -1.0 : ms > 0 ? ms : 0.0;
      } else if (wb == -2) {
        d.wb_left_ms = -2;
      }
    }
    return out;
  }
  void diag_forget() { std::fill(dma_used_.begin(), dma_used_.end(), uint8_t(0)); }
  // The physical side of landings: ns the service waited on a landing block's reuse, and the pool's counts.
  uint64_t landing_wait_ns() const { return land_wait_ns_; }
  ReadPool::LandingCounts landing_counts() const { return pool_ ? pool_->landing_counts() : ReadPool::LandingCounts{}; }
  // Every read submitted so far has returned; rethrows the first failed read (the token fails before the layer whose
  // copies read it is signalled ready, so its bytes never reach an engine).
  void drain_reads() {
    if (pool_) read_wait_ns_ += pool_->drain();
  }
  void adapt_reads() {
    if (pool_) pool_->adapt();
  }
  void read_controller(const std::function<void(const ReadDepthController&)>& f) const {
    if (pool_) pool_->with_controller(f);
  }
  void stop_reads() {
    if (pool_) pool_->stop();
  }
  uint64_t read_ns() const { return pool_ ? pool_->read_ns() : read_ns_; }
  uint64_t read_wait_ns() const { return read_wait_ns_; }
  uint64_t max_reads_in_flight() const { return pool_ ? pool_->max_running() : (read_ns_ ? 1 : 0); }
  char* slot_ptr(uint32_t p, int32_t slot) const {
    return static_cast<char*>(arena_[p]) + uint64_t(slot) * x_.part_bytes[p];
  }

  // A write-back's parts are separate copies (one arena per part), so each part's copy records its own events on
  // the slot it read and the block it wrote; the next copy into that slot waits part by part: part p of the new unit
  // starts once part p of the old one is out, instead of once the whole unit is.
  void wait_copy_in(Stream s, int32_t slot, int32_t block, void* slot_ev, void* block_ev) override {
    (void)s;
    wait_slot_ = slot_ev ? slot : -1;
    wait_block_ = block_ev ? block : -1;
  }
  void h2d(Stream s, int32_t slot, int32_t block, uint32_t key) override {
    h2d_unit(s, slot, block, key);
    wait_slot_ = wait_block_ = -1;
    if (landing_block(block)) {  // the block's next landing read waits for this copy
      hipEvent_t& e = land_copy_ev_[size_t(uint32_t(block) - x_.blocks - x_.S)];
      if (!e) e = dev_->event_create();
      ev_record(e, s_[s]);
    }
  }
  void part_wait(Stream s, int32_t slot, int32_t block, uint32_t p) {
    if (slot >= 0 && slot == wait_slot_) gate(s, part_ev_[part_ev_index(false, slot, p)]);
    if (block >= 0 && block == wait_block_) gate(s, part_ev_[part_ev_index(true, block, p)]);
  }
  // Waits on the library's queues. A device barrier (hipStreamWaitEvent) parked on one CU-masked queue while its event
  // is still running slows every kernel dispatched from the other CU-masked queues, the device check among them
  // (measured on one MI355X: one 336 MiB check 57 us with no such barrier, about 90 us beside two). So a wait reaches
  // the device only when it must: an event that has completed is no wait at all; on the demand stream the service
  // thread waits on the host (the stream is in order: nothing behind the copy could start earlier), launching the
  // checks whose copies land meanwhile; the D2H stream's waits are kept until its next copy (one followed by nothing
  // is dropped); anything else is a device barrier.
  void gate(Stream s, hipEvent_t ev) {
    if (!ev || ev_done(ev)) return;
    if (s == kDem && std::this_thread::get_id() == service_thread_) {
      while (!ev_done(ev)) {
        poll_checks();
        _mm_pause();
      }
      return;
    }
    if (s == kD2h) {
      d2h_waits_.push_back(ev);
      return;
    }
    stream_wait(s_[s], ev);
  }
  void d2h_ready() {  // before an operation on the D2H stream: its kept waits
    for (hipEvent_t e : d2h_waits_)
      if (!ev_done(e)) stream_wait(s_[kD2h], e);
    d2h_waits_.clear();
  }
  void set_service_thread(std::thread::id id) { service_thread_ = id; }
  void h2d_unit(Stream s, int32_t slot, int32_t block, uint32_t key) {
    const char* src = block_ptr(block);
    if (hsa_) {  // part by part on the lane, each after the same part of the write-backs named by wait_copy_in
      for (uint32_t p = 0; p < uint32_t(x_.part_bytes.size()); ++p) {
        const uint32_t ws = slot >= 0 && slot == wait_slot_ ? part_sig_[part_ev_index(false, slot, p)] : 0;
        const uint32_t wb = block >= 0 && block == wait_block_ ? part_sig_[part_ev_index(true, block, p)] : 0;
        const uint32_t sig = lane_copy(s, slot_ptr(p, slot), src + x_.part_offset[p], x_.part_bytes[p], false, ws, wb);
        prof_copy(kProfCopy, sig, x_.part_bytes[p], p == 0 ? 1 : 0);
      }
      return;
    }
    const bool landing = landing_block(block);
    if (landing) {  // a promotion: its landing read becomes a demand read if it still runs; one that failed reads again
      const uint32_t l = uint32_t(block) - x_.blocks - x_.S, i = land_word0_ + l;
      const ReadPool::Claim c = pool_->claim(i);
      if (c == ReadPool::Claim::Landed) {
        rpending_[i] = 0;  // (its word is stored: nothing to await)
      } else if (c == ReadPool::Claim::Failed) {
        if (++rgen_[i] == 0) rgen_[i] = 1;
        rpending_[i] = rgen_[i];
        pool_->submit(i, land_key_[l], block_ptr(block), rword_host_ + i, rgen_[i]);
      }
    }
    if (pool_) {  // a read into this block may still run: the stream waits for the read's word
      uint32_t i = UINT32_MAX;
      if (landing) {
        i = land_word0_ + (uint32_t(block) - x_.blocks - x_.S);
      } else if (uint32_t(block) >= x_.blocks) {
        i = uint32_t(block) - x_.blocks;
      } else if (!kept_word_.empty()) {
        const auto it = kept_word_.find(block);
        if (it != kept_word_.end()) {
          i = it->second;
          kept_word_.erase(it);
        }
      }
      if (i != UINT32_MAX && rpending_[i]) {
        const uint32_t* w = static_cast<const uint32_t*>(rword_dev_) + i;
        hip_check(hipError_t(dg_launch_await(dw_, w, rpending_[i], raux_[i], s_[s])), "await of a file read");
        rpending_[i] = 0;
      }
    }
    const uint32_t P = uint32_t(x_.part_bytes.size());
    if (!scatter_) {  // one SDMA copy per part straight into its arena slot (timed after its wait: engine busy time)
      for (uint32_t p = 0; p < P; ++p) {
        part_wait(s, slot, block, p);
        Timed t = prof_start(kProfCopy, x_.part_bytes[p], p == 0 ? 1 : 0, s_[s]);
        copy_h2d(slot_ptr(p, slot), src + x_.part_offset[p], x_.part_bytes[p], s_[s]);
        prof_end(t, s_[s]);
      }
      return;
    }
    // small parts: the whole unit in one SDMA copy to the stream's HBM staging, then one kernel writes every part
    const int k = s == kPf ? 1 : 0;
    for (uint32_t p = 0; p < P; ++p) part_wait(s, -1, block, p);  // the staging copy reads every part of the block
    Timed t = prof_start(kProfCopy, x_.unit_bytes, 1, s_[s]);
    copy_h2d(stage_dev_[k], src, x_.unit_bytes, s_[s]);
    for (uint32_t p = 0; p < P; ++p) part_wait(s, slot, -1, p);   // the scatter writes every part of the slot
    if (fused()) {  // with device verify, the scatter is the check: the staged bytes cross HBM once each way
      scatter_check(s, k, slot, key);
      prof_end(t, s_[s]);
      return;
    }
    const uint32_t j = job_next_[k]++ % kJobRing;
    tsa_scatter_job& job = jobs_host_[k][j];
    std::memset(&job, 0, sizeof job);
    job.src = stage_dev_[k];
    for (uint32_t p = 0; p < x_.part_bytes.size(); ++p) {
      job.dst[p] = slot_ptr(p, slot);
      job.bytes[p] = x_.part_bytes[p];
    }
    job.n_parts = uint32_t(x_.part_bytes.size());
    job.block_first = 0;
    copy_h2d(jobs_dev_[k] + j, &job, sizeof job, s_[s]);
    hip_check(hipError_t(launch_scatter(jobs_dev_[k] + j, 1, scatter_blocks_, s_[s])), "scatter launch");
    prof_end(t, s_[s]);
  }
  // The staged unit in staging buffer k into `slot`, hashed on the way against its checkpoints and digest, on the
  // copy's stream: a mismatch raises the token's abort; a one-wave kernel behind it publishes the unit's slot entry.
  void scatter_check(Stream s, int k, int32_t slot, uint32_t key) {
    require(vused_ + 1 <= vcap_, SS_E_BACKEND, "device verify: more landed units in a token than the table holds");
    DgVerifyLaunch a = vlaunch_;  // (the shape, checkpoints, digests and abort words)
    a.n = 1;
    a.keys[0] = key;
    a.slots[0] = slot;
    a.fail = vfail_dev_ + vused_;
    a.aux = gated_of(key);
    a.ready = nullptr;
    Timed t = prof_take(kProfVerify, x_.unit_bytes, 1);
    hip_check(hipError_t(launch_dg_scatter_verify(a, stage_dev_[k], s_[s], t.a, t.b)), "scatter check launch");
    prof_put(t);
    vkeys_.push_back(key);
    ++vused_;
  }
  // Device verify of staged units happens in their scatter (no launch on the verify stream).
  bool fused() const { return scatter_ && verify_; }
  void d2h(int32_t slot, int32_t block) override {
    if (hsa_) {
      for (uint32_t p = 0; p < parts(); ++p) hsa_d2h_part(kD2h, slot, block, p, p == 0 ? 1 : 0);
      return;
    }
    d2h_ready();
    Timed t = prof_start(kProfWb, x_.unit_bytes, 1, s_[kD2h]);
    char* dst = block_ptr(block);
    for (uint32_t p = 0; p < x_.part_bytes.size(); ++p) {
      copy_d2h(dst + x_.part_offset[p], slot_ptr(p, slot), x_.part_bytes[p], s_[kD2h]);
      mark_part(kD2h, slot, block, p);
    }
    prof_end(t, s_[kD2h]);
  }
  // Deferred write-backs are copied at the boundary that chose them (prestage), in the core's order, on the D2H
  // stream: the copy engine of that direction is otherwise idle, and PCIe is full duplex, so a miss copy later into
  // the slot finds its write-back done instead of queued behind the token's other write-backs. The core still submits
  // each one part by part when its credit or a needed slot says so (its bookkeeping, hence placement, is unchanged);
  // those submissions find the part copied and only the part's events matter (recorded at the copy).
  void prestage(int32_t slot, int32_t block) override {
    const uint32_t P = uint32_t(x_.part_bytes.size());
    if (hsa_) {
      for (uint32_t p = 0; p < P; ++p) hsa_d2h_part(kD2h, slot, block, p, 1);
    } else {
      d2h_ready();
      for (uint32_t p = 0; p < P; ++p) {
        Timed t = prof_start(kProfWb, x_.part_bytes[p], 1, s_[kD2h]);
        copy_d2h(block_ptr(block) + x_.part_offset[p], slot_ptr(p, slot), x_.part_bytes[p], s_[kD2h]);
        mark_part(kD2h, slot, block, p);
        prof_end(t, s_[kD2h]);
      }
    }
    prestaged_[slot] = {block, (1u << P) - 1u};
  }
  void unqueue(int32_t slot, int32_t block) override {  // (its copies, if any, stay in the stream's order)
    const auto it = prestaged_.find(slot);
    if (it != prestaged_.end() && it->second.block == block) prestaged_.erase(it);
  }
  // One part of a write-back on lane s (HSA copies): the part's signal becomes the slot's and the block's.
  void hsa_d2h_part(Stream s, int32_t slot, int32_t block, uint32_t p, uint32_t count) {
    const uint32_t sig = lane_copy(s, block_ptr(block) + x_.part_offset[p], slot_ptr(p, slot), x_.part_bytes[p], true);
    for (size_t i : {part_ev_index(false, slot, p), part_ev_index(true, block, p)}) {
      hsa_->ref(sig);
      hsa_->unref(part_sig_[i]);
      part_sig_[i] = sig;
    }
    prof_copy(kProfWb, sig, x_.part_bytes[p], count);
  }
  void d2h_part(Stream s, int32_t slot, int32_t block, uint32_t p) override {
    auto it = prestaged_.find(slot);
    if (it != prestaged_.end() && it->second.block == block && (it->second.parts >> p & 1u)) {
      it->second.parts &= ~(1u << p);
      if (!it->second.parts) prestaged_.erase(it);
      return;
    }
    if (hsa_) return hsa_d2h_part(s, slot, block, p, 1);
    if (s == kD2h) d2h_ready();
    Timed t = prof_start(kProfWb, x_.part_bytes[p], 1, s_[s]);
    copy_d2h(block_ptr(block) + x_.part_offset[p], slot_ptr(p, slot), x_.part_bytes[p], s_[s]);
    mark_part(s, slot, block, p);
    prof_end(t, s_[s]);
  }
  // events of the last write-back copy of (slot, part) and into (block, part)
  size_t part_ev_index(bool block, int32_t i, uint32_t p) const {
    const size_t P = x_.part_bytes.size();
    return (block ? size_t(x_.slots) * P : 0) + size_t(i) * P + p;
  }
  void mark_part(Stream s, int32_t slot, int32_t block, uint32_t p) {
    for (size_t i : {part_ev_index(false, slot, p), part_ev_index(true, block, p)}) {
      if (!part_ev_[i]) part_ev_[i] = dev_->event_create();
      ev_record(part_ev_[i], s_[s]);
    }
  }
  uint32_t parts() const override { return uint32_t(x_.part_bytes.size()); }
  uint64_t part_bytes(uint32_t p) const override { return x_.part_bytes[p]; }
  void write_entry(Stream s, uint32_t key, int32_t v) override {
    if (hsa_) {  // behind the lane's copies (a fetched unit's entry after its bytes), in the queue's order
      Check c;
      c.kind = Check::kEntry;
      hold(c.sigs, tail_[s]);
      c.key = key;
      c.v = v;
      checks_.push_back(std::move(c));
      poll_checks();
      return;
    }
    hip_check(hipStreamWriteValue32(s_[s], slot_of_ + key, uint32_t(v), 0), "hipStreamWriteValue32 (slot entry)");
  }
  // ready[g] = seq after the layer's demand copies (and cover waits) on kDem; with device verify on the verify stream,
  // behind the checks of every unit landed so far in the token (its stream order).
  void signal_ready(uint32_t g, uint32_t seq) override {
    drain_reads();
    // (fused checks: every check of the layer ran on the demand stream before this, or on the prefetch stream before
    // an event the demand stream waited for)
    if ((!verify_ || fused()) && !hsa_) {
      hip_check(hipStreamWriteValue32(s_[kDem], ready_ + g, seq, 0), "hipStreamWriteValue32 (ready)");
      return;
    }
    if (hsa_) {  // the layer's cover waits and copies, all on kDem's lane
      hold(vsigs_, tail_[kDem]);
    } else {
      hipEvent_t ev = next_vev();
      ev_record(ev, s_[kDem]);
      vafter_.push_back(ev);
    }
    if (vpending_) {  // the layer's last check writes the ready word when it has published its units
      vlaunch_.ready = ready_;
      vlaunch_.ready_g = g;
      vlaunch_.seq = seq;
      flush_verify();
      vlaunch_.ready = nullptr;
    } else {
      Check c;
      c.kind = Check::kReady;
      c.after.swap(vafter_);
      c.sigs.swap(vsigs_);
      c.g = g;
      c.seq = seq;
      checks_.push_back(std::move(c));
      poll_checks();
    }
  }
  struct Mark {
    std::vector<uint32_t> sigs;
  };
  void* event_create() override { return hsa_ ? static_cast<void*>(new Mark) : dev_->event_create(); }
  void event_destroy(void* ev) override {
    if (!hsa_) return dev_->event_destroy(static_cast<hipEvent_t>(ev));
    if (Mark* m = static_cast<Mark*>(ev)) {
      drop(m->sigs);
      delete m;
    }
  }
  void record(void* ev, Stream s) override {
    if (hsa_) {
      Mark* m = static_cast<Mark*>(ev);
      drop(m->sigs);
      hold(m->sigs, tail_[s]);
      return;
    }
    if (s == kD2h) d2h_ready();
    ev_record(static_cast<hipEvent_t>(ev), s_[s]);
  }
  void wait(Stream s, void* ev) override {
    if (hsa_) return hold(tail_[s], static_cast<Mark*>(ev)->sigs);
    gate(s, static_cast<hipEvent_t>(ev));
  }
  bool done(void* ev) override {  // the canonical schedule: a completion query waits for the completion
    event_sync(ev);
    return true;
  }
  bool query(void* ev) override {
    return hsa_ ? all_done(static_cast<Mark*>(ev)->sigs) : ev_done(static_cast<hipEvent_t>(ev));
  }
  void event_sync(void* ev) override {
    if (hsa_) return host_wait(static_cast<Mark*>(ev)->sigs);
    ev_sync(static_cast<hipEvent_t>(ev));
  }
  void sync(Stream s) override {
    if (hsa_) {  // the lane's copies, then (a copy-in lane) the queued value writes behind them
      host_wait(tail_[s]);
      if (s != kD2h) {
        drain_checks();
        stream_sync(queue_stream());
      }
      return;
    }
    if (s == kD2h) d2h_ready();
    stream_sync(s_[s]);
  }
  // ---- lanes (HSA copies) ----
  // Adds the signals of `sigs` still running to `into`, with a reference each.
  void hold(std::vector<uint32_t>& into, const std::vector<uint32_t>& sigs) {
    for (uint32_t g : sigs)
      if (!hsa_->done(g)) {
        hsa_->ref(g);
        into.push_back(g);
      }
  }
  void drop(std::vector<uint32_t>& sigs) {
    for (uint32_t g : sigs) hsa_->unref(g);
    sigs.clear();
  }
  bool all_done(const std::vector<uint32_t>& sigs) const {
    for (uint32_t g : sigs)
      if (!hsa_->done(g)) return false;
    return true;
  }
  // One copy on lane s after the lane's tail and up to two more signals; it becomes the lane's tail.
  uint32_t lane_copy(Stream s, void* dst, const void* src, uint64_t bytes, bool to_host, uint32_t also = 0,
                     uint32_t also2 = 0) {
    std::vector<uint32_t>& t = tail_[s];
    deps_.assign(t.begin(), t.end());
    if (also) deps_.push_back(also);
    if (also2) deps_.push_back(also2);
    const uint32_t sig = hsa_->copy(dst, src, bytes, to_host, deps_.data(), uint32_t(deps_.size()));
    drop(t);
    t.push_back(sig);  // (the copy's own reference)
    return sig;
  }
  // On the host until every signal has ended; the service thread launches the checks whose copies land meanwhile.
  void host_wait(const std::vector<uint32_t>& sigs) {
    const bool svc = std::this_thread::get_id() == service_thread_;
    for (uint32_t spins = 0; !all_done(sigs); ++spins) {
      if (svc) poll_checks();
      if (svc || spins < 4096) _mm_pause();
      else std::this_thread::yield();
    }
  }
  // The HIP stream of the queue's value writes and launches: the verify stream, else (HSA copies without device
  // verify) the demand stream's, which then carries no copy.
  hipStream_t queue_stream() const { return vs_ ? vs_ : s_[kDem]; }
  void upload_table(const int32_t* table, uint32_t n) override {
    if (hsa_) {  // no queued entry write may land after the table
      drain_checks();
      stream_sync(queue_stream());
    }
    std::memcpy(stage_host_, table, 4ull * n);
    copy_h2d(slot_of_, stage_host_, 4ull * n, s_[kDem]);
    stream_sync(s_[kDem]);
  }

  // ---- device verify of landed units (verify_hash = 2) ----
  // Every landed unit is re-hashed in HBM on the verify stream once its copies are done, and the layer's ready word
  // is written behind those checks on the same stream: an engine reads a landed unit only after its bytes reproduced
  // the descriptor hash. A mismatch raises the token's sticky abort (kDgHash) before the ready word, so every later
  // ss_dg_slot of the token gives the guard slot and the token fails.
  void enable_verify(const std::vector<uint64_t>& digests, uint64_t* ckpt_dev, uint64_t n_ckpt, uint32_t max_per_token,
                     const DgDevWords& dw) {
    verify_ = true;
    vcap_ = max_per_token;
    digests_dev_ = static_cast<uint64_t*>(dev_->alloc_device(8ull * digests.size(), "verify digests"));
    hip_check(hipMemcpy(digests_dev_, digests.data(), 8ull * digests.size(), hipMemcpyHostToDevice),
              "hipMemcpy (digests)");
    vfail_host_ = static_cast<uint32_t*>(dev_->alloc_pinned(4ull * vcap_, "verify results"));
    vfail_dev_ = static_cast<uint32_t*>(dev_->alloc_device(4ull * vcap_, "verify results"));
    hip_check(hipMemset(vfail_dev_, 0, 4ull * vcap_), "hipMemset");
    vs_ = dev_->stream_create_dedicated();
    DgVerifyLaunch& a = vlaunch_;
    require(set_dg_verify_shape(a, arena_.data(), x_.part_bytes.data(), uint32_t(x_.part_bytes.size()),
                                verify_seg_bytes(x_.unit_bytes)) &&
                a.unit_segs == n_ckpt && a.unit_bytes == x_.unit_bytes,
            SS_E_BACKEND, "device verify: the parts' segments disagree with the checkpoint count");
    a.ckpt = ckpt_dev;
    a.digests = digests_dev_;
    a.abort = dw.abort;
    a.err_code = dw.err_code;
    a.err_aux = dw.err_aux;
    a.err = kDgHash;
    a.publish = 1;
    a.slot_of = slot_of_;
  }
  bool publishes_landed() const override { return verify_; }
  hipEvent_t next_vev() {
    if (vev_used_ == vev_.size()) vev_.push_back(dev_->event_create());
    return vev_[vev_used_++];
  }
  // A landed unit's check is launched once the next landed() or the layer's signal_ready() comes (the service issues
  // them back to back), so the layer's last check can carry the ready word; each waits for its own unit's copies.
  void landed(Stream s, uint32_t g, const uint32_t* keys, const int32_t* slots, uint32_t n) override {
    if (!verify_ || n == 0 || fused()) return;  // (fused: checked and published by the unit's scatter)
    require(vused_ + n <= vcap_, SS_E_BACKEND, "device verify: more landed units in a token than the table holds");
    flush_verify();
    if (hsa_) {
      hold(vsigs_, tail_[s]);
    } else {
      hipEvent_t landed_ev = next_vev();
      ev_record(landed_ev, s_[s]);
      vafter_.push_back(landed_ev);
    }
    for (uint32_t i0 = 0; i0 < n; i0 += kDgVerifyMax) {
      if (i0) flush_verify();
      DgVerifyLaunch& a = vlaunch_;
      a.n = std::min(kDgVerifyMax, n - i0);
      a.fail = vfail_dev_ + vused_;
      a.aux = g;
      a.ready = nullptr;
      for (uint32_t i = 0; i < a.n; ++i) {
        a.keys[i] = keys[i0 + i];
        a.slots[i] = slots[i0 + i];
        vkeys_.push_back(keys[i0 + i]);
      }
      vused_ += a.n;
      vpending_ = true;
    }
    if (s != kDem) flush_verify();  // a prefetch's check carries no ready word
  }
  // The check of the units gathered in vlaunch_ joins the queue of checks, behind the events of their copies.
  void flush_verify() {
    if (!vpending_) return;
    vpending_ = false;
    Check c;
    c.after.swap(vafter_);
    c.sigs.swap(vsigs_);
    c.launch = vlaunch_;
    checks_.push_back(std::move(c));
    poll_checks();
  }
  // The queue of checks, launched in order from the host: the head goes once every event and copy signal it waits for
  // has completed, so its stream never holds a device barrier. A ready word without a check of its own is a value
  // write in the same order, as is (HSA copies) a slot entry; a timing mark is an event record. Called by the service
  // thread (while it waits, and before a token is marked served) and at the boundary.
  struct Check {
    enum Kind { kLaunch, kReady, kMark, kEntry } kind = kLaunch;
    std::vector<hipEvent_t> after;
    std::vector<uint32_t> sigs;  // (HSA copies) with a reference each
    DgVerifyLaunch launch;
    uint32_t g = 0, seq = 0;
    hipEvent_t mark = nullptr;
    uint32_t key = 0;
    int32_t v = 0;
  };
  bool poll_checks() {
    poll_wb_marks();
    while (!checks_.empty()) {
      Check& c = checks_.front();
      while (!c.after.empty() && ev_done(c.after.back())) c.after.pop_back();
      if (!c.after.empty()) return false;
      while (!c.sigs.empty() && hsa_->done(c.sigs.back())) {
        hsa_->unref(c.sigs.back());
        c.sigs.pop_back();
      }
      if (!c.sigs.empty()) return false;
      const hipStream_t q = queue_stream();
      if (c.kind == Check::kLaunch) {
        // timed by the launch's own start / stop events (the kernel's begin and end, not the queue around it)
        Timed t = prof_take(kProfVerify, uint64_t(c.launch.n) * x_.unit_bytes, c.launch.n);
        hip_check(hipError_t(launch_dg_verify(c.launch, vs_, t.a, t.b)), "device verify launch");
        prof_put(t);
      } else if (c.kind == Check::kReady) {
        hip_check(hipStreamWriteValue32(q, ready_ + c.g, c.seq, 0), "hipStreamWriteValue32 (ready)");
      } else if (c.kind == Check::kEntry) {
        hip_check(hipStreamWriteValue32(q, slot_of_ + c.key, uint32_t(c.v), 0), "hipStreamWriteValue32 (slot entry)");
      } else {
        ev_record(c.mark, q);
      }
      checks_.pop_front();
    }
    return true;
  }
  void drain_checks() {
    while (!poll_checks()) _mm_pause();
  }
  // A small device-to-host read on the demand stream (between tokens), not on the null stream.
  void read_device(void* dst, const void* src, uint64_t bytes) {
    copy_d2h(dst, src, bytes, s_[kDem]);
    stream_sync(s_[kDem]);
  }
  // Before the boundary may reuse a slot: every check of this token has read its bytes.
  void verify_sync() {
    flush_verify();  // (every demand landing is followed by its layer's signal_ready: nothing should be pending)
    drain_checks();
    if (vs_) stream_sync(vs_);
    if (fused()) {  // the checks ran on the copy streams
      stream_sync(s_[kDem]);
      stream_sync(s_[kPf]);
    }
  }
  // At the boundary: the keys whose landed bytes differ from their descriptor hash.
  std::vector<uint32_t> collect_verify() {
    std::vector<uint32_t> bad;
    verify_sync();
    vev_used_ = 0;
    if (!verify_ || vused_ == 0) return bad;
    // on the verify stream, never the null stream: the library's streams (CU-masked, hence blocking) would all be
    // waited for, the write-backs on the D2H stream included
    copy_d2h(vfail_host_, vfail_dev_, 4ull * vused_, vs_);
    stream_sync(vs_);
    for (uint32_t i = 0; i < vused_; ++i)
      if (vfail_host_[i]) bad.push_back(vkeys_[i]);
    hip_check(hipMemsetAsync(vfail_dev_, 0, 4ull * vused_, vs_), "hipMemsetAsync");
    verified_ += vused_;
    vused_ = 0;
    vkeys_.clear();
    return bad;
  }
  uint64_t verified() const { return verified_; }

  // ---- timing (a test hook): timed events around unit copies, write-backs and verify launches ----
  void profile_enable(int on) {
    std::lock_guard<std::mutex> lk(prof_mu_);
    drain_locked(true);
    prof_mask_ = on == 1 ? (TSA_TEST_PROF_COPY | TSA_TEST_PROF_WRITEBACK | TSA_TEST_PROF_VERIFY) : uint32_t(on);
    prof_tot_ = tsa_test_profile{};
    // HSA copies are timed by the copy engine's own timestamps (start to end of each part)
    if (hsa_) hsa_->profiling((prof_mask_ & (TSA_TEST_PROF_COPY | TSA_TEST_PROF_WRITEBACK)) != 0);
  }
  tsa_test_profile profile_read(bool wait) {
    std::lock_guard<std::mutex> lk(prof_mu_);
    drain_locked(wait);
    tsa_test_profile out = prof_tot_;
    out.pending = pending_.size();
    return out;
  }
  void profile_collect() {  // completed brackets only; recycles their events
    std::lock_guard<std::mutex> lk(prof_mu_);
    drain_locked(false);
  }

 private:
  enum ProfKind : uint32_t { kProfCopy, kProfWb, kProfVerify };
  struct Timed {
    hipEvent_t a = nullptr, b = nullptr;
    uint32_t sig = 0;  // (HSA copies) the copy's signal, referenced, instead of the events
    ProfKind kind = kProfCopy;
    uint64_t bytes = 0;
    uint32_t units = 0;
  };
  void prof_copy(ProfKind k, uint32_t sig, uint64_t bytes, uint32_t units) {
    std::lock_guard<std::mutex> lk(prof_mu_);
    if (!(prof_mask_ & prof_bit(k))) return;
    Timed t;
    t.sig = sig;
    t.kind = k;
    t.bytes = bytes;
    t.units = units;
    hsa_->ref(sig);
    pending_.push_back(t);
  }
  hipEvent_t take_event_locked() {
    if (prof_free_.empty()) {
      prof_events_.push_back(dev_->event_create_timed());
      return prof_events_.back();
    }
    hipEvent_t e = prof_free_.back();
    prof_free_.pop_back();
    return e;
  }
  static uint32_t prof_bit(ProfKind k) {
    return k == kProfCopy ? TSA_TEST_PROF_COPY : k == kProfWb ? TSA_TEST_PROF_WRITEBACK : TSA_TEST_PROF_VERIFY;
  }
  Timed prof_start(ProfKind k, uint64_t bytes, uint32_t units, hipStream_t s) {
    Timed t;
    std::lock_guard<std::mutex> lk(prof_mu_);
    if (!(prof_mask_ & prof_bit(k))) return t;
    t.a = take_event_locked();
    t.b = take_event_locked();
    t.kind = k;
    t.bytes = bytes;
    t.units = units;
    ev_record(t.a, s);
    return t;
  }
  void prof_end(const Timed& t, hipStream_t s) {
    if (!t.a) return;
    std::lock_guard<std::mutex> lk(prof_mu_);
    ev_record(t.b, s);
    pending_.push_back(t);
  }
  // A pair of timing events for a launch that records them itself (prof_take, launch with them, prof_put).
  Timed prof_take(ProfKind k, uint64_t bytes, uint32_t units) {
    Timed t;
    std::lock_guard<std::mutex> lk(prof_mu_);
    if (!(prof_mask_ & prof_bit(k))) return t;
    t.a = take_event_locked();
    t.b = take_event_locked();
    t.kind = k;
    t.bytes = bytes;
    t.units = units;
    return t;
  }
  void prof_put(const Timed& t) {
    if (!t.a) return;
    std::lock_guard<std::mutex> lk(prof_mu_);
    pending_.push_back(t);
  }
  void drain_locked(bool wait) {
    size_t keep = 0;
    for (const Timed& t : pending_) {
      uint64_t ns = 0;
      if (t.sig) {
        if (!wait && !hsa_->done(t.sig)) {
          pending_[keep++] = t;
          continue;
        }
        while (!hsa_->done(t.sig)) std::this_thread::yield();
        (void)hsa_->copy_ns(t.sig, &ns);
        hsa_->unref(t.sig);
      } else {
        if (wait) ev_sync(t.b);
        else if (!ev_done(t.b)) {
          pending_[keep++] = t;
          continue;
        }
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, t.a, t.b), "hipEventElapsedTime");
        ns = uint64_t(double(ms) * 1e6 + 0.5);
      }
      switch (t.kind) {
        case kProfCopy:
          prof_tot_.copies += t.units;  // a unit's first part counts the unit
          prof_tot_.copy_bytes += t.bytes;
          prof_tot_.copy_ns += ns;
          break;
        case kProfWb:
          prof_tot_.writebacks += t.units;  // (a unit copied out whole counts once, at its first part)
          prof_tot_.writeback_bytes += t.bytes;
          prof_tot_.writeback_ns += ns;
          break;
        case kProfVerify:
          ++prof_tot_.verifies;
          prof_tot_.verify_units += t.units;
          prof_tot_.verify_bytes += t.bytes;
          prof_tot_.verify_ns += ns;
          break;
      }
      if (t.a) {
        prof_free_.push_back(t.a);
        prof_free_.push_back(t.b);
      }
    }
    pending_.resize(keep);
  }

  std::mutex prof_mu_;  // the service thread brackets demand copies, the engine thread reads and the boundary's copies
  uint32_t prof_mask_ = 0;  // TSA_TEST_PROF_* kinds bracketed
  tsa_test_profile prof_tot_{};
  std::vector<Timed> pending_;
  std::vector<hipEvent_t> prof_events_, prof_free_;

  HipDevice* dev_;
  const Layout& x_;
  std::vector<void*> arena_;
  int32_t* slot_of_;
  uint32_t* ready_;
  std::vector<void*> chunks_;
  uint64_t per_chunk_;
  uint32_t kJobRing;
  hipStream_t s_[3] = {nullptr, nullptr, nullptr};
  int32_t* stage_host_ = nullptr;
  bool scatter_ = false;
  void* stage_dev_[2] = {nullptr, nullptr};
  tsa_scatter_job* jobs_host_[2] = {nullptr, nullptr};
  tsa_scatter_job* jobs_dev_[2] = {nullptr, nullptr};
  uint32_t job_next_[2] = {0, 0};
  uint64_t scatter_blocks_ = 0;
  bool verify_ = false;
  DgVerifyLaunch vlaunch_;            // the next launch (arena, shape, checkpoints, gate and publication words fixed)
  bool vpending_ = false;             // vlaunch_ holds units whose check is not launched yet
  std::vector<hipEvent_t> vafter_;    // the copies the next queued check (or ready word) waits for
  std::deque<Check> checks_;          // queued checks, ready words and marks, in verify-stream order
  std::vector<hipEvent_t> d2h_waits_; // waits of the D2H stream kept until its next operation
  std::unique_ptr<HsaCopier> hsa_;    // unit copies through the HSA runtime (null: on the HIP streams)
  std::vector<uint32_t> tail_[3];     // (HSA copies) per lane: what its next operation waits for
  std::vector<uint32_t> deps_;        // (HSA copies) a copy's dependencies, reused
  std::vector<uint32_t> vsigs_;       // (HSA copies) the copies the next queued check (or ready word) waits for
  std::vector<uint32_t> part_sig_;    // (HSA copies) as part_ev_: the last write-back copy of each part (0: none)
  std::vector<uint32_t> wb_sigs_[2];  // (HSA copies, dg_diag) the boundary's write-backs, until seen ended
  bool wb_seen_[2] = {true, true};
  std::thread::id service_thread_;
  uint64_t* digests_dev_ = nullptr;   // [keys]: the descriptor hashes
  uint32_t vcap_ = 0, vused_ = 0;
  uint32_t* vfail_host_ = nullptr;
  uint32_t* vfail_dev_ = nullptr;
  std::vector<uint32_t> vkeys_;
  uint64_t verified_ = 0;
  std::vector<hipEvent_t> part_ev_;  // [slots + blocks][parts]: the last write-back copy of each part (lazily made)
  int32_t wait_slot_ = -1, wait_block_ = -1;  // the next h2d waits per part on these (wait_copy_in)
  struct Prestaged {
    int32_t block;
    uint32_t parts;  // the parts copied at the boundary whose submission has not come yet
  };
  std::unordered_map<int32_t, Prestaged> prestaged_;  // by slot
  std::vector<char*> stage_;                          // three-tier staging buffers
  std::unique_ptr<ReadPool> pool_;                    // reads in flight (dg_disk_queue > 1)
  uint32_t* rword_host_ = nullptr;                    // per staging buffer: the generation of its last finished read
  void* rword_dev_ = nullptr;
  std::vector<uint32_t> rgen_, rpending_, raux_;      // per read word: last generation, one to await, its layer
  std::unordered_map<int32_t, uint32_t> kept_word_;   // dg_bank_keep: a pinned block read into -> its read's word
  std::vector<void*> land_chunks_;                    // the landing blocks (pinned chunks)
  uint64_t land_per_chunk_ = 1;
  uint32_t land_word0_ = 0;                           // the first landing block's read word
  std::vector<hipEvent_t> land_copy_ev_;              // per landing block: its last copy out (lazily made)
  std::vector<uint32_t> land_key_;                    // per landing block: the key of its last landing read
  uint64_t land_wait_ns_ = 0;
  bool diag_ = false;                                 // dg_diag: the timeline's device marks
  std::vector<hipEvent_t> dma_a_, dma_b_, dma_f_;
  std::vector<uint8_t> dma_used_;                     // per layer: 0 unmarked, 1 marked, 2 with its first miss
  hipEvent_t wb_end_[2] = {nullptr, nullptr};
  int wb_cur_ = 0, wb_prev_ = 1;
  bool wb_cur_valid_ = false, wb_prev_valid_ = false;
  DgDevWords dw_;                                     // the await kernel's abort words and deadline
  uint64_t read_ns_ = 0, read_wait_ns_ = 0;
  std::function<void(uint32_t, char*)> reader_;       // three-tier: a key's bytes from its file, host block layout
  hipStream_t vs_ = nullptr;        // the verify stream (a hardware queue of its own)
  std::vector<hipEvent_t> vev_;     // per landed batch and ready write of the token: the copies before it
  size_t vev_used_ = 0;
};

// ---- the context ------------------------------------------------------------------------------------------------------
class HipDgCtx final : public DgCtx {
 public:
  HipDgCtx(const Desc& d, const Plan& p, const ss_options& o) : d_(d), o_(o), x_(dg_geometry(d, p, o)) {
    try {
      init();
    } catch (...) {
      release();
      throw;
    }
  }
  ~HipDgCtx() override { release(); }

  bool poisoned() const override { return poisoned_; }
  void poison() override { poisoned_ = true; }
  int n_sources() const override { return int(files_.size()); }
  bool source_direct(int i) const override { return files_[size_t(i)]->direct(); }

  // The device's words after the last token, as ss_begin and ss_end need them.
  struct SeqWords {
    uint32_t done = 0, began = 0;
    bool flags_behind = true;  // no export or prediction flag is past the last token
  };
  SeqWords seq_words() const {
    SeqWords w;
    w.done = load_acquire(m_.done);
    w.began = load_acquire(m_.began);
    for (size_t g = 0; g < x_.gated.size() && w.flags_behind; ++g)
      w.flags_behind = int32_t(load_acquire(m_.flag + g) - seq_) <= 0 && int32_t(load_acquire(m_.pflag + g) - seq_) <= 0;
    return w;
  }
  // A token that cannot be trusted ends the context: the device's waits end on host_abort, the service stops, and
  // every later call but close and stats is refused.
  [[noreturn]] void fail_closed(const std::string& why) {
    const std::string dev = device_error();
    store_release(m_.host_abort, 1);
    svc_->stop_join();
    poisoned_ = true;
    fail(SS_E_BACKEND, token_failure(dev, why));
  }

  // ss_begin: a new token may open only where the last one closed - the device's done and began words hold its
  // sequence and no flag is ahead of it (anything else is a step that ran outside ss_begin / ss_end).
  void begin(const uint32_t* rows, int n_layers) override {
    require(!in_token_, SS_E_INVALID, "ss_begin: a gated token is already open (call ss_end)");
    require(!rows || n_layers == int(d_.layers.size()), SS_E_INVALID, "ss_begin: rows_per_layer must cover every layer");
    const SeqWords w = seq_words();
    if (w.done != seq_ || w.began != seq_ || !w.flags_behind) {
      store_release(m_.host_abort, 1);
      svc_->stop_join();
      poisoned_ = true;
      fail(SS_E_BACKEND, "device-gated: ss_begin found a step that ran outside ss_begin / ss_end (device done " +
                             std::to_string(w.done) + ", began " + std::to_string(w.began) + ", last token " +
                             std::to_string(seq_) + (w.flags_behind ? "" : ", a flag ahead of it") +
                             "); the context is poisoned");
    }
    for (size_t g = 0; g < x_.gated.size(); ++g) run_[g] = !rows || rows[size_t(x_.gated[g])] != 0;
    ++seq_;
    in_token_ = true;
    store_release(m_.host_seq, seq_);  // the begin kernel authorizes exactly this sequence
    svc_->begin(seq_, run_);
  }

  // Waits for the device's done word to reach this token (the end kernel ran after every reader of the token); the
  // reason it cannot be trusted, or empty.
  std::string completion_problem(Clock::time_point deadline) const {
    for (uint32_t polls = 0;; ++polls) {
      const uint32_t v = load_acquire(m_.done);
      if (v == seq_) break;
      if (int32_t(v - seq_) > 0) return "sequence desync at ss_end: the device finished token " + std::to_string(v);
      if ((polls & 1023u) == 0 && Clock::now() > deadline) return "the device did not finish it (no end kernel)";
      if (polls < 100000) _mm_pause();
      else std::this_thread::yield();
    }
    return load_acquire(m_.began) == seq_ ? std::string() : "sequence desync at ss_end: another gated step ran in it";
  }

  // ss_end: the token must be complete on the device and served in full; then the boundary runs and the device checks
  // of the token's landed units report. A device error or a failed check poisons the context.
  void end(uint32_t rows) override {
    require(rows > 0, SS_E_INVALID, "ss_dg_end_rows: rows must be positive");
    require(in_token_, SS_E_INVALID, "ss_end: no gated token is open");
    in_token_ = false;
    struct FailedRows {  // dg_diag: a failed token's host rows stay readable, its device measurements -1
      HipDgCtx* c;
      bool ok = false;
      ~FailedRows() {
        if (!ok) c->failed_timeline();
      }
    } rows_guard{this};
    const auto deadline = Clock::now() + std::chrono::milliseconds(uint64_t(o_.dg_wait_timeout_ms) + 5000);
    if (const std::string why = completion_problem(deadline); !why.empty()) fail_closed(why);
    if (svc_->wait_outcome(seq_, deadline) != DgService::Outcome::kServed) {
      const std::string why = svc_->error();
      fail_closed("the service: " + (why.empty() ? std::string("it did not finish") : why));
    }
    const std::string dev = device_error();
    const bool hash_abort = load_acquire(m_.err_code) == kDgHash;  // a failed device check: named with its units below
    if (!dev.empty() && !hash_abort) {
      poisoned_ = true;
      fail(SS_E_BACKEND, token_failure(dev, ""));
    }
    // the boundary: every check of the token has ended (it may hand a landed slot to a write-back or a new copy) and
    // every read has returned (a prefetch's read may still use a staging buffer the boundary reuses)
    tr_->verify_sync();
    try {
      tr_->drain_reads();
    } catch (...) {
      poisoned_ = true;
      throw;
    }
    core_->close_token(rows, all_kept());
    const std::vector<uint32_t> bad = tr_->collect_verify();  // (a prefetch's check may end after the end kernel)
    tr_->profile_collect();
    if (!bad.empty()) {
      verify_failures_ += bad.size();
      poisoned_ = true;
      const uint32_t g = core_->gated_of(bad[0]);
      fail(SS_E_HASH, token_failure(dev, std::to_string(bad.size()) + " landed unit(s) differ from the descriptor hash "
                                         "in HBM, first gated (" + std::to_string(g) + ", " +
                                         std::to_string(bad[0] - core_->unit_base()[g]) + ")"));
    }
    if (hash_abort) {
      poisoned_ = true;
      fail(SS_E_BACKEND, token_failure(dev, "no device check result names the unit"));
    }
    if (o_.dg_diag) collect_timeline();
    rows_guard.ok = true;
    fold(true);
  }

  // dg_diag, after a successful boundary: the device side of each exported layer's row - the transport's marks and the
  // device stamps (export end, wait entry, ready seen; 100 ticks per microsecond).
  void collect_timeline() {
    const std::vector<HipTransport::LayerDma> dma = tr_->diag_collect();
    std::vector<uint64_t> st(4 * x_.gated.size(), 0);
    tr_->read_device(st.data(), dw_.stamps, 8 * st.size());
    for (size_t g = 0; g < diag_rows_.size(); ++g) {
      LayerDiag& d = diag_rows_[g];
      d = LayerDiag{};
      if (!run_[g]) continue;  // (its stamps are an older token's)
      d.dma_ms = dma[g].dma_ms;
      d.dma_first_ms = dma[g].dma_first_ms;
      d.wb_left_ms = dma[g].wb_left_ms;
      const uint64_t ex = st[4 * g], in = st[4 * g + 1], rd = st[4 * g + 2];
      if (ex && in && rd && rd >= in && rd >= ex) {
        d.gpu_wait_us = double(rd - in) / 100.0;
        d.gpu_export_ready_us = double(rd - ex) / 100.0;
      }
    }
    timeline_valid_ = true;
  }
  void failed_timeline() noexcept {
    if (!o_.dg_diag) return;
    std::fill(diag_rows_.begin(), diag_rows_.end(), LayerDiag{});
    tr_->diag_forget();
    timeline_valid_ = true;
  }
  void timeline(int g, ss_dg_layer_timeline* out) const override {
    require(!in_token_, SS_E_INVALID, "ss_dg_timeline: between tokens only");
    require(o_.dg_diag != 0, SS_E_INVALID, "ss_dg_timeline: open the context with dg_diag = 1");
    check_g(g, "ss_dg_timeline");
    require(timeline_valid_, SS_E_INVALID, "ss_dg_timeline: no token has completed");
    const DgService::Row& t = svc_->timeline()[size_t(g)];
    const LayerDiag& d = diag_rows_[size_t(g)];
    std::memset(out, 0, sizeof *out);
    out->struct_size = uint32_t(sizeof *out);
    out->layer = uint32_t(x_.gated[size_t(g)]);
    out->seen_us = t.seen_us;
    out->demand_us = t.demand_us;
    out->pred_wait_us = t.pred_wait_us;
    out->prefetch_us = t.prefetch_us;
    out->serve_us = t.serve_us;
    out->ids = t.ids;
    out->misses = t.misses;
    out->covered = t.covered;
    out->fetched = t.fetched;
    out->prefetched = t.prefetched;
    out->predicted_true = t.predicted_true;
    out->covered_waits = t.covered_waits;
    out->dma_ms = d.dma_ms;
    out->dma_first_ms = d.dma_first_ms;
    out->wb_left_ms = d.wb_left_ms;
    out->gpu_wait_us = d.gpu_wait_us;
    out->gpu_export_ready_us = d.gpu_export_ready_us;
  }
  void boundary_timeline(ss_dg_boundary_timeline* out) const override {
    require(!in_token_, SS_E_INVALID, "ss_dg_boundary_timeline: between tokens only");
    require(o_.dg_diag != 0, SS_E_INVALID, "ss_dg_boundary_timeline: open the context with dg_diag = 1");
    const DgBoundaryTimes& b = core_->boundary_times();
    require(b.boundaries > 0, SS_E_INVALID, "ss_dg_boundary_timeline: no token has completed");
    std::memset(out, 0, sizeof *out);
    out->struct_size = uint32_t(sizeof *out);
    out->writebacks = b.writebacks;
    out->sync_us = b.sync_us;
    out->select_us = b.select_us;
    out->upload_us = b.upload_us;
    out->issue_us = b.issue_us;
  }

  ss_dg_device_view device_view() const override {
    ss_dg_device_view v{};
    v.struct_size = uint32_t(sizeof v);
    v.protocol = SS_DG_PROTOCOL;
    v.n_gated = uint32_t(x_.gated.size());
    v.n_parts = uint32_t(x_.part_bytes.size());
    v.guard_slot = x_.guard_slot;
    v.slots = x_.slots;
    v.slot_of = dw_.slot_of;
    v.unit_base = dw_.unit_base;
    v.abort = dw_.abort;
    for (size_t p = 0; p < x_.part_bytes.size(); ++p) v.parts[p] = {arena_[p], x_.part_bytes[p], x_.part_bytes[p]};
    v.absent_err = dw_.absent_err;
    return v;
  }
  int gated_index(int layer) const override {
    return layer < 0 || size_t(layer) >= x_.ordinal.size() ? -1 : x_.ordinal[size_t(layer)];
  }
  void check_g(int g, const char* fn) const {
    require(g >= 0 && size_t(g) < x_.gated.size(), SS_E_INVALID, std::string(fn) + ": gated layer out of range");
  }
  // Any engine stream but the legacy null stream. The library's streams are CU-masked (a hardware queue each), which
  // the HIP runtime creates as blocking streams: work on the legacy null stream and theirs wait for each other, so a
  // layer's wait kernel there would hold the checks and ready words it waits for until dg_wait_timeout_ms.
  static void check_engine_stream(void* stream, const char* fn) {
    require(stream != nullptr && stream != static_cast<void*>(hipStreamLegacy), SS_E_INVALID,
            std::string(fn) + ": the engine stream cannot be the legacy null stream (the library's streams wait for "
                              "it); use a stream created with hipStreamNonBlocking");
  }
  void enqueue_begin(void* stream) override {
    check_engine_stream(stream, "ss_dg_enqueue_begin");
    launch_ck(dg_launch_begin(dw_, stream), "ss_dg_enqueue_begin");
  }
  void enqueue_export(int g, const int32_t* ids_dev, int n, int n_pred, void* stream) override {
    check_engine_stream(stream, "ss_dg_enqueue_export");
    check_g(g, "ss_dg_enqueue_export");
    require(ids_dev && n >= 1 && uint32_t(n) <= x_.B, SS_E_INVALID, "ss_dg_enqueue_export: 1..dg_max_ids ids");
    require(n_pred >= 0 && n_pred <= int(kDgMaxIds), SS_E_INVALID, "ss_dg_enqueue_export: n_pred 0..64");
    launch_ck(dg_launch_export(dw_, uint32_t(g), ids_dev, uint32_t(n), uint32_t(n_pred), stream),
              "ss_dg_enqueue_export");
  }
  void enqueue_predict(int g, const int32_t* ids_dev, int n, void* stream) override {
    check_engine_stream(stream, "ss_dg_enqueue_predict");
    check_g(g, "ss_dg_enqueue_predict");
    require(ids_dev && n >= 1 && n <= int(kDgMaxIds), SS_E_INVALID, "ss_dg_enqueue_predict: 1..64 ids");
    launch_ck(dg_launch_predict(dw_, uint32_t(g), ids_dev, uint32_t(n), stream), "ss_dg_enqueue_predict");
  }
  void enqueue_wait(int g, void* stream) override {
    check_engine_stream(stream, "ss_dg_enqueue_wait");
    check_g(g, "ss_dg_enqueue_wait");
    launch_ck(dg_launch_wait(dw_, uint32_t(g), stream), "ss_dg_enqueue_wait");
  }
  void enqueue_end(void* stream) override {
    check_engine_stream(stream, "ss_dg_enqueue_end");
    launch_ck(dg_launch_end(dw_, stream), "ss_dg_enqueue_end");
  }

  uint32_t residency(ss_dg_unit* out, uint32_t cap) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_residency: between tokens only");
    const std::vector<uint32_t> r = core_->device_order();
    for (uint32_t i = 0; i < cap && i < r.size(); ++i) {
      const uint32_t g = core_->gated_of(r[i]);
      out[i] = {int32_t(g), int32_t(r[i] - core_->unit_base()[g])};
    }
    return uint32_t(r.size());
  }
  void set_budgets(uint32_t spare_target, uint32_t per_layer, uint32_t per_token) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_set_budgets: between tokens only");
    require(spare_target <= x_.D, SS_E_INVALID, "ss_dg_set_budgets: spare target above the billed spares");
    core_->set_spare_target(spare_target);
    core_->set_prefetch_budget(per_layer, per_token);
  }

  // ss_dg_keep (reference include/strix_stream/ss.h:683-688): a plain keep set of gated layer g, replacing the last
  // one; the next boundaries never choose a kept unit as a victim.
  void keep(int g, const int32_t* ids, int n) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_keep: between tokens only");
    check_g(g, "ss_dg_keep");
    require(n >= 0 && (n == 0 || ids), SS_E_INVALID, "ss_dg_keep: bad arguments");
    std::vector<uint32_t> keys(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) {
      require(ids[i] >= 0 && uint32_t(ids[i]) < core_->units(uint32_t(g)), SS_E_INVALID, "ss_dg_keep: id out of range");
      keys[size_t(i)] = core_->key(uint32_t(g), uint32_t(ids[i]));
    }
    kept_[size_t(g)] = std::move(keys);
  }
  // ss_dg_set_sched (reference include/strix_stream/ss.h:693-699). dg_flush_ready is accepted and kept: HIP submits
  // every copy and value-write when it is enqueued, so there is no batched submission to flush.
  void set_sched(uint32_t wb_defer, uint32_t flush_ready) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_set_sched: between tokens only");
    require(wb_defer <= 1 && flush_ready <= 1, SS_E_INVALID, "ss_dg_set_sched: flags are 0 or 1");
    core_->defer_writebacks(wb_defer != 0);
    o_.dg_wb_defer = wb_defer;
    o_.dg_flush_ready = flush_ready;
  }
  // ss_dg_set_clean_evict (reference include/strix_stream/ss.h:1756-1760): from the next boundary's victims on.
  void set_clean_evict(uint32_t on) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_set_clean_evict: between tokens only");
    require(!poisoned_, SS_E_BACKEND, "ss_dg_set_clean_evict: poisoned context");
    require(on <= 1, SS_E_INVALID, "ss_dg_set_clean_evict: on is 0 or 1");
    core_->set_clean_evict(on != 0);
    o_.dg_clean_evict = on;
  }
  // Test hooks under the reference's names (its include/strix_stream/ss_test.h:19, :30), for a context opened with
  // dg_test_hooks = 1.
  void test_hooks_on(const char* what) const {
    require(o_.dg_test_hooks != 0, SS_E_INVALID, std::string(what) + ": open the context with dg_test_hooks = 1");
  }
  void test_check() override {
    test_hooks_on("ss_test_dg_check");
    require(!in_token_, SS_E_INVALID, "ss_test_dg_check: between tokens only");
    core_->audit();
  }
  void test_stop_service() override {
    test_hooks_on("ss_test_dg_stop_service");
    svc_->stop_join();
  }
  std::vector<uint32_t> all_kept() const {
    std::vector<uint32_t> v;
    for (const auto& k : kept_) v.insert(v.end(), k.begin(), k.end());
    return v;
  }

  // Between tokens, with the device and the service done with the last one (reference src/dg_ctx.cpp:619-629).
  void set_policy(ss_policy policy) override {
    require(!in_token_, SS_E_INVALID, "ss_dg_set_policy: between tokens only");
    require(!poisoned_, SS_E_BACKEND, "ss_dg_set_policy: poisoned context");
    require(load_acquire(m_.done) == seq_ && load_acquire(m_.began) == seq_, SS_E_BACKEND,
            "ss_dg_set_policy: device sequence desync");
    require(!seq_ || svc_->wait_outcome(seq_, Clock::now()) == DgService::Outcome::kServed, SS_E_BACKEND,
            "ss_dg_set_policy: the service does not hold the last token's terminal state");
    core_->set_policy(uint32_t(policy));
    fold(false);  // the drain's write-backs in the counters; no token for the hook
  }

  // Counters as folded at the last successful boundary (and at open): a token whose ss_end failed never shows, and a
  // call between tokens never reads the service's live counters (reference src/dg_ctx.cpp:1547-1577).
  ss_dg_stats stats() const override {
    const DgCounts& a = fold_;
    const DgCounts& b = base_;
    ss_dg_stats s{};
    s.struct_size = uint32_t(sizeof s);
#define TSA_D(f) s.f = a.f - b.f
    TSA_D(tokens);
    TSA_D(lookups);
    TSA_D(misses);
    TSA_D(covered);
    TSA_D(fetched);
    TSA_D(prefetched);
    TSA_D(prefetch_used);
    TSA_D(pred_invalid);
    TSA_D(resurrected);
    TSA_D(bank_serves);
    TSA_D(collected_mid);
    TSA_D(evicted);
    TSA_D(evict_short);
    TSA_D(writebacks_done);
    TSA_D(stalled);
    TSA_D(predicted);
    TSA_D(predicted_true);
    TSA_D(miss_layers);
    TSA_D(covered_waits);
    TSA_D(wb_deferred);
    TSA_D(wb_cancelled);
    TSA_D(wb_forced);
    TSA_D(wb_boundary_flushed);
    TSA_D(wb_issued_bytes);
    TSA_D(wb_completed_bytes);
    TSA_D(wb_cancelled_bytes);
    TSA_D(wb_boundary_flushed_bytes);
    TSA_D(wb_forced_wait_ns);
    TSA_D(inclusive_kept);
    TSA_D(inclusive_drops);
    TSA_D(disk_reads);
    TSA_D(disk_read_bytes);
    TSA_D(disk_stage_waits);
    TSA_D(disk_drops);
    TSA_D(disk_discards);
    TSA_D(clean_drops);
    TSA_D(clean_drop_bytes);
    TSA_D(bank_kept);
    TSA_D(landing_issued);
    TSA_D(landing_promoted);
    TSA_D(landing_late);
    TSA_D(landing_wait_ns);
    TSA_D(landing_expired);
    TSA_D(landing_dropped_full);
    TSA_D(landing_read_bytes);
    TSA_D(landing_cancelled);
    TSA_D(landing_expired_layer);
    TSA_D(landing_skipped_passed);
    TSA_D(landing_yields);
    TSA_D(landing_aborted_bytes);
    TSA_D(score_fallbacks);
    TSA_D(scored_victims);
    TSA_D(score_layers);
    TSA_D(score_candidates);
    TSA_D(score_saturated);
    TSA_D(score_ns);
#undef TSA_D
    s.disk_units = fold_file_units_;
    s.disk_queue_resolved = x_.disk_tier ? x_.disk_queue : 0;
    s.disk_depth_adapt = adapt_;
    s.disk_depth_active = x_.disk_tier ? x_.disk_queue : 0;
    if (adapt_ == 1)
      tr_->read_controller([&](const ReadDepthController& c) {
        s.disk_depth_active = c.depth();
        s.disk_depth_changes = c.changes;
        s.disk_depth_calibrations = c.calibrations;
      });
    s.disk_locations = x_.disk_tier ? 1 : 0;
    s.disk_read_ns = fold_read_ns_ - base_read_ns_;
    s.disk_wait_ns = fold_wait_ns_ - base_wait_ns_;
    s.disk_max_in_flight = fold_max_in_flight_;
    s.free_slots = fold_free_slots_;
    s.blocks = x_.blocks;
    s.slots = x_.slots;
    s.device_timeouts = load_acquire(m_.err_count);
    s.wb_outstanding_bytes = fold_outstanding_;
    s.backed_units = fold_backed_;
    return s;
  }
  ss_layer_stats layer_stats(int layer) const override {
    require(layer >= 0 && size_t(layer) < d_.layers.size(), SS_E_INVALID, "ss_stats_layer: layer out of range");
    const int g = x_.ordinal[size_t(layer)];
    if (g < 0) return ss_layer_stats{};
    return to_layer(fold_l_[size_t(g)], base_l_[size_t(g)]);
  }
  ss_layer_stats total_stats() const override {
    ss_layer_stats t{};
    for (size_t g = 0; g < x_.gated.size(); ++g) {
      const ss_layer_stats l = to_layer(fold_l_[g], base_l_[g]);
      t.routed += l.routed;
      t.hits += l.hits;
      t.admitted += l.admitted;
      t.transient += l.transient;
      t.evicted += l.evicted;
      t.spec_issued += l.spec_issued;
      t.spec_used += l.spec_used;
      t.spec_dropped += l.spec_dropped;
      t.bytes_pinned += l.bytes_pinned;
    }
    return t;
  }
  // Since open, never reset (reference src/dg_ctx.cpp:1081-1091): evictions that copied (not cancelled, not dropped
  // as a clean copy, not discarded to their file), the bytes copied, the copies into persistent slots.
  ss_exclusive_stats exclusive_stats() const override {
    const DgCounts& a = fold_;
    ss_exclusive_stats x{};
    x.struct_size = uint32_t(sizeof x);
    x.writebacks = a.evicted - a.wb_cancelled - a.inclusive_drops - a.disk_discards;
    x.writeback_bytes = a.wb_issued_bytes;
    x.deferred = a.evict_short;
    x.promoted = a.fetched - a.bank_serves + a.prefetched;
    x.free_blocks = fold_free_blocks_;
    x.min_free_blocks = min_free_blocks_;
    return x;
  }
  void stats_reset() override {
    if (in_token_) return;  // (nothing changes inside a gated token)
    base_ = fold_;
    base_l_ = fold_l_;
    base_read_ns_ = fold_read_ns_;
    base_wait_ns_ = fold_wait_ns_;
    publish();
  }
  void set_hook(ss_stats_hook h, void* user) override {
    hook_ = h;
    hook_user_ = user;
  }
  Json stats_json() const override {
    return format_stats(stats(), exclusive_stats(), layers_now(), core_->policy(), extras());
  }
  bool snapshot(ss_layer_stats* total, ss_snapshot_info* info) const override {
    snap_armed_.store(true, std::memory_order_relaxed);
    std::lock_guard<std::mutex> lk(snap_mu_);
    if (snap_.seq == 0) return false;
    ss_layer_stats t{};
    for (const ss_layer_stats& l : snap_.layers) add_stats(t, l);
    if (total) *total = t;
    if (info) {
      *info = ss_snapshot_info{};
      info->struct_size = uint32_t(sizeof *info);
      info->flags = SS_SNAPSHOT_EXCLUSIVE;
      info->sequence = snap_.seq;
      info->forwards = snap_.s.tokens;
      info->exclusive_writebacks = snap_.x.writebacks;
      info->exclusive_writeback_bytes = snap_.x.writeback_bytes;
      info->exclusive_deferred = snap_.x.deferred;
      info->exclusive_promoted = snap_.x.promoted;
      info->exclusive_free_blocks = snap_.x.free_blocks;
      info->exclusive_min_free_blocks = snap_.x.min_free_blocks;
      info->exclusive_blocks = x_.blocks;
    }
    return true;
  }
  bool snapshot_json(Json* out) const override {
    snap_armed_.store(true, std::memory_order_relaxed);
    Published p;
    {
      std::lock_guard<std::mutex> lk(snap_mu_);
      if (snap_.seq == 0) return false;
      p = snap_;
    }
    *out = format_stats(p.s, p.x, p.layers, p.policy, p.extra);
    return true;
  }
  // After a successful boundary (and at open): the core's counters as the stats show them, the hook with this
  // token's per-layer numbers, the snapshot when armed (reference src/dg_ctx.cpp:1547-1577).
  void fold(bool call_hook) {
    prev_l_ = fold_l_;
    fold_ = core_->counts();
    if (x_.L) {  // the landings' physical side; the bytes landed are the reads issued less those never read
      const ReadPool::LandingCounts lc = tr_->landing_counts();
      fold_.landing_late = lc.late;
      fold_.landing_wait_ns = tr_->landing_wait_ns();
      fold_.landing_cancelled = lc.cancelled;
      fold_.landing_yields = lc.yields;
      fold_.landing_aborted_bytes = lc.aborted_bytes;
      fold_.landing_failed = lc.failed;
      fold_.landing_read_bytes -= std::min(fold_.landing_read_bytes, lc.unread_bytes);
    }
    fold_l_ = core_->layer_counts();
    fold_free_slots_ = core_->free_slots();
    fold_free_blocks_ = core_->free_blocks();
    fold_outstanding_ = core_->outstanding_bytes();
    fold_backed_ = core_->clean_copies();
    fold_file_units_ = core_->file_units();
    fold_read_ns_ = tr_->read_ns();
    fold_wait_ns_ = tr_->read_wait_ns();
    fold_max_in_flight_ = tr_->max_reads_in_flight();
    min_free_blocks_ = std::min(min_free_blocks_, fold_free_blocks_);
    if (hook_ && call_hook) {
      std::vector<ss_layer_stats> fwd(d_.layers.size());
      ss_layer_stats tot{};
      for (size_t g = 0; g < fold_l_.size(); ++g) {
        fwd[size_t(x_.gated[g])] = to_layer(fold_l_[g], prev_l_[g]);
        add_stats(tot, fwd[size_t(x_.gated[g])]);
      }
      hook_(hook_user_, &tot, fwd.data(), int(fwd.size()));
    }
    publish();
  }
  uint32_t host_table(int32_t* out, uint32_t cap) const override {
    const std::vector<int32_t>& t = core_->table();
    for (uint32_t i = 0; i < cap && i < t.size(); ++i) out[i] = t[i];
    return uint32_t(t.size());
  }
  uint64_t verify_failures() const override { return verify_failures_; }
  bool hsa_copies() const override { return tr_ && tr_->hsa_copies(); }

  void profile_enable(int on) override {
    require(!in_token_, SS_E_INVALID, "tsa_test_profile_enable: between tokens only");
    tr_->profile_enable(on);
  }
  tsa_test_profile profile_read(bool wait) override {
    require(!in_token_, SS_E_INVALID, "tsa_test_profile_read: between tokens only");
    return tr_->profile_read(wait);
  }
  uint32_t stamps(uint64_t* out, uint32_t cap) const override {
    require(!in_token_, SS_E_INVALID, "tsa_test_dg_stamps: between tokens only");
    const uint32_t n = 4u * uint32_t(x_.gated.size());
    if (out && cap)
      tr_->read_device(out, dw_.stamps, 8ull * std::min(n, cap));
    return n;
  }

  void corrupt_block(int g, int unit, uint64_t offset) override {
    require(!in_token_, SS_E_INVALID, "tsa_test_dg_corrupt_block: between tokens only");
    check_g(g, "tsa_test_dg_corrupt_block");
    require(unit >= 0 && uint32_t(unit) < core_->units(uint32_t(g)), SS_E_INVALID,
            "tsa_test_dg_corrupt_block: unit out of range");
    const uint32_t k = core_->key(uint32_t(g), uint32_t(unit));
    require(core_->where(k) == DgCore::Where::Pinned && core_->block_of(k) >= 0, SS_E_INVALID,
            "tsa_test_dg_corrupt_block: the unit is not in its pinned block");
    require(offset < x_.unit_bytes, SS_E_INVALID, "tsa_test_dg_corrupt_block: offset past the unit");
    tr_->block_ptr(core_->block_of(k))[offset] ^= char(0xff);
  }

 private:
  static void launch_ck(int e, const char* what) { hip_check(hipError_t(e), what); }
  ss_layer_stats to_layer(const DgLayerCounts& a, const DgLayerCounts& b) const {
    ss_layer_stats l{};
    l.routed = a.lookups - b.lookups;
    l.hits = l.routed - (a.misses - b.misses);
    l.transient = a.bank_serves - b.bank_serves;
    l.admitted = (a.fetched - b.fetched) - l.transient;
    l.evicted = a.evicted - b.evicted;
    l.spec_issued = a.prefetched - b.prefetched;
    l.spec_used = a.prefetch_used - b.prefetch_used;
    l.spec_dropped = l.spec_issued >= l.spec_used ? l.spec_issued - l.spec_used : 0;
    l.bytes_pinned = ((a.fetched - b.fetched) + (a.prefetched - b.prefetched)) * x_.unit_bytes;
    return l;
  }
  std::string device_error() const {
    const uint32_t code = load_acquire(m_.err_code), aux = load_acquire(m_.err_aux);
    if (code == kDgOk) return std::string();
    const char* what = code == kDgTimeout ? "a wait timed out" : code == kDgBadId ? "an exported id was out of range"
                       : code == kDgHostAbort ? "the host aborted the token"
                       : code == kDgDesync ? "a step the host did not authorize"
                       : code == kDgAbsent ? "a slot lookup met an absent entry"
                       : code == kDgHash ? "a landed unit differs from its descriptor hash" : "unknown device error";
    return std::string(what) + (code == kDgDesync ? " (seq " : code == kDgAbsent ? "" : " (gated layer ") +
           (code == kDgAbsent ? std::string() : std::to_string(aux) + ")");
  }
  std::string token_failure(const std::string& device, const std::string& host) const {
    std::string m = "device-gated: token " + std::to_string(seq_) + ": ";
    if (!device.empty()) m += "the device: " + device + (host.empty() ? "" : "; ");
    return m + host + " (the context is poisoned, the token's outputs must be discarded)";
  }

  void init();
  void fill();
  void release() noexcept;
  // Every part of key k from its source file into dst, laid out as a host block (part p at part_offset[p]).
  void read_key(uint32_t k, char* dst) const;
  // Bytes off .. off + bytes - 1 of part p of key k from its source file into dst.
  void read_part(uint32_t k, uint32_t p, uint64_t off, uint64_t bytes, char* dst) const;
  // The XXH64 of key k's bytes at dst against its descriptor hash (SS_E_HASH on a mismatch).
  void check_key(uint32_t k, const char* dst) const;

  Desc d_;
  ss_options o_;
  Layout x_;
  std::unique_ptr<HipDevice> dev_;
  std::vector<std::unique_ptr<SourceFile>> files_;
  std::vector<void*> arena_;
  int32_t* slot_of_dev_ = nullptr;
  char* ctl_dev_ = nullptr;
  void* mapped_host_ = nullptr;
  void* mapped_dev_ = nullptr;
  std::vector<void*> block_chunks_;
  uint64_t per_chunk_ = 1;
  uint64_t* ckpt_dev_ = nullptr;
  DgDevWords dw_;
  DgMappedHost m_;
  std::unique_ptr<HipTransport> tr_;
  std::unique_ptr<DgCore> core_;
  std::unique_ptr<DgService> svc_;
  std::vector<uint8_t> run_;
  std::vector<std::vector<uint32_t>> kept_;  // per gated layer: its ss_dg_keep set (keys)
  uint32_t seq_ = 0;
  bool in_token_ = false, poisoned_ = false;
  DgCounts base_, fold_;
  std::vector<DgLayerCounts> base_l_, fold_l_, prev_l_;
  uint32_t fold_free_slots_ = 0, fold_free_blocks_ = 0, min_free_blocks_ = UINT32_MAX;
  uint64_t fold_outstanding_ = 0, fold_backed_ = 0, fold_file_units_ = 0;
  uint64_t fold_read_ns_ = 0, fold_wait_ns_ = 0, fold_max_in_flight_ = 0, base_read_ns_ = 0, base_wait_ns_ = 0;
  ss_stats_hook hook_ = nullptr;
  void* hook_user_ = nullptr;
  struct Extras {  // counters the stats document shows outside ss_dg_stats (since the last reset)
    uint64_t keep_drops = 0, keep_rereads = 0, landing_failed = 0;
  };
  Extras extras() const {
    return Extras{fold_.bank_keep_drops - base_.bank_keep_drops, fold_.bank_keep_rereads - base_.bank_keep_rereads,
                  fold_.landing_failed - base_.landing_failed};
  }
  struct Published {
    uint64_t seq = 0;
    ss_dg_stats s{};
    ss_exclusive_stats x{};
    std::vector<ss_layer_stats> layers;
    uint32_t policy = 0;
    Extras extra;
  };
  mutable std::atomic<bool> snap_armed_{false};
  mutable std::mutex snap_mu_;
  Published snap_;
  uint64_t verify_failures_ = 0;
  std::string score_prov_;  // the score profile's provenance (reported in the stats document)
  uint32_t adapt_ = 0;      // dg_disk_queue_adapt: 0 off, 1 adapting, 2 declined (adapt_why_)
  struct LayerDiag {        // dg_diag: a layer's device measurements of the last token (-1: none)
    double dma_ms = -1, dma_first_ms = -1, wb_left_ms = -1, gpu_wait_us = -1, gpu_export_ready_us = -1;
  };
  std::vector<LayerDiag> diag_rows_;
  bool timeline_valid_ = false;
  std::string adapt_why_;

  static void add_stats(ss_layer_stats& a, const ss_layer_stats& b) {
    a.routed += b.routed;
    a.hits += b.hits;
    a.admitted += b.admitted;
    a.transient += b.transient;
    a.evicted += b.evicted;
    a.prefetched += b.prefetched;
    a.spec_issued += b.spec_issued;
    a.spec_used += b.spec_used;
    a.spec_dropped += b.spec_dropped;
    a.bytes_pinned += b.bytes_pinned;
    a.bytes_disk += b.bytes_disk;
    a.wait_ns += b.wait_ns;
  }
  // per descriptor layer (0 for a layer with no gated units)
  std::vector<ss_layer_stats> layers_now() const {
    std::vector<ss_layer_stats> v(d_.layers.size());
    for (size_t L = 0; L < v.size(); ++L) v[L] = layer_stats(int(L));
    return v;
  }
  // A poisoned context publishes no more: the last successful publication stays.
  void publish() {
    if (!snap_armed_.load(std::memory_order_relaxed) || poisoned_) return;
    Published p;
    p.s = stats();
    p.x = exclusive_stats();
    p.layers = layers_now();
    p.policy = core_->policy();  // (the engine thread's: a reader on another thread formats this copy)
    p.extra = extras();
    std::lock_guard<std::mutex> lk(snap_mu_);
    p.seq = snap_.seq + 1;
    std::swap(snap_, p);
  }
  Json format_stats(const ss_dg_stats& s, const ss_exclusive_stats& x, const std::vector<ss_layer_stats>& layers,
                    uint32_t policy, const Extras& extra) const;
};

void HipDgCtx::init() {
  dev_ = std::make_unique<HipDevice>(o_.device);
  for (const auto& s : d_.sources) files_.push_back(std::make_unique<SourceFile>(s.path, o_.direct_io != 0));
  const uint32_t G = uint32_t(x_.gated.size());
  // the arena: one HBM array per part, the guard slot zeroed
  for (uint64_t pb : x_.part_bytes) {
    arena_.push_back(dev_->alloc_device(uint64_t(x_.slots) * pb, "device-gated arena"));
    hip_check(hipMemset(static_cast<char*>(arena_.back()) + uint64_t(x_.guard_slot) * pb, 0, pb), "hipMemset (guard)");
  }
  slot_of_dev_ = static_cast<int32_t*>(dev_->alloc_device(4ull * x_.keys, "slot table"));
  // HBM control words: seq, abort, err_count, err_code, err_aux, absent_err | any_miss[G] | ready[G] | unit_base[G+1]
  // | stamps[4G]
  const uint64_t o_any = 64, o_ready = align64(o_any + 4ull * G), o_base = align64(o_ready + 4ull * G),
                 o_stamps = align64(o_base + 4ull * (G + 1)), ctl_bytes = align64(o_stamps + 32ull * G);
  ctl_dev_ = static_cast<char*>(dev_->alloc_device(ctl_bytes, "device-gated control words"));
  hip_check(hipMemset(ctl_dev_, 0, ctl_bytes), "hipMemset (control words)");
  hip_check(hipMemcpy(ctl_dev_ + o_base, x_.unit_base.data(), 4ull * (G + 1), hipMemcpyHostToDevice),
            "hipMemcpy (unit_base)");
  uint32_t* w = reinterpret_cast<uint32_t*>(ctl_dev_);
  dw_.seq = w + 0;
  dw_.abort = w + 1;
  dw_.err_count = w + 2;
  dw_.err_code = w + 3;
  dw_.err_aux = w + 4;
  dw_.absent_err = w + 5;
  dw_.any_miss = reinterpret_cast<uint32_t*>(ctl_dev_ + o_any);
  dw_.ready = reinterpret_cast<uint32_t*>(ctl_dev_ + o_ready);
  dw_.unit_base = reinterpret_cast<const uint32_t*>(ctl_dev_ + o_base);
  dw_.stamps = reinterpret_cast<uint64_t*>(ctl_dev_ + o_stamps);
  dw_.slot_of = slot_of_dev_;
  dw_.timeout_ticks = uint64_t(o_.dg_wait_timeout_ms) * 100000ull;  // wall clock: 100 MHz
  // the fine-grained control area (device writes, host polls; host writes, device reads)
  const MappedLayout ml = mapped_layout(G);
  mapped_host_ = dev_->alloc_mapped(ml.total, &mapped_dev_, "device-gated control area");
  char* h = static_cast<char*>(mapped_host_);
  char* dv = static_cast<char*>(mapped_dev_);
  m_.rec = reinterpret_cast<DgRecord*>(h + ml.rec);
  m_.prec = reinterpret_cast<DgPredRecord*>(h + ml.prec);
  m_.flag = reinterpret_cast<uint32_t*>(h + ml.flag);
  m_.pflag = reinterpret_cast<uint32_t*>(h + ml.pflag);
  uint32_t* hw = reinterpret_cast<uint32_t*>(h + ml.words);
  m_.done = hw + 0;
  m_.err_code = hw + 1;
  m_.err_aux = hw + 2;
  m_.err_count = hw + 3;
  m_.host_abort = hw + 4;
  m_.host_seq = hw + 5;
  m_.began = hw + 6;
  dw_.rec = reinterpret_cast<DgRecord*>(dv + ml.rec);
  dw_.prec = reinterpret_cast<DgPredRecord*>(dv + ml.prec);
  dw_.flag = reinterpret_cast<uint32_t*>(dv + ml.flag);
  dw_.pflag = reinterpret_cast<uint32_t*>(dv + ml.pflag);
  uint32_t* dvw = reinterpret_cast<uint32_t*>(dv + ml.words);
  dw_.done = dvw + 0;
  dw_.m_err_code = dvw + 1;
  dw_.m_err_aux = dvw + 2;
  dw_.m_err_count = dvw + 3;
  dw_.host_abort = dvw + 4;
  dw_.host_seq = dvw + 5;
  dw_.began = dvw + 6;
  // pinned blocks: P + Q of one host stride each, in chunks of at most 1 GiB (a larger block alone)
  per_chunk_ = std::max<uint64_t>(1, kPinnedChunk / x_.host_stride);
  for (uint64_t left = x_.blocks; left > 0;) {
    const uint64_t n = std::min(per_chunk_, left);
    block_chunks_.push_back(dev_->alloc_pinned(n * x_.host_stride, "pinned blocks"));
    left -= n;
  }
  tr_ = std::make_unique<HipTransport>(dev_.get(), x_, arena_, slot_of_dev_, dw_.ready, block_chunks_, per_chunk_,
                                       G * x_.B + o_.dg_prefetch_per_token + x_.D);
  // unit copies through the HSA runtime, except with the file tier or small parts (staged and scattered) and unless
  // TSA_DG_COPIES=hip asks for the HIP streams' copies
  const char* copies = std::getenv("TSA_DG_COPIES");
  if (!x_.disk_tier && !(copies && std::strcmp(copies, "hip") == 0)) tr_->enable_hsa_copies(o_.device);
  DgConfig c;
  for (int L : x_.gated) c.n_units.push_back(uint32_t(d_.layers[size_t(L)].n_units));
  c.persistent_slots = x_.persistent_slots;
  c.bank_slots = x_.B;
  c.blocks = x_.blocks;
  const uint32_t T = o_.dg_spare_target == 0xFFFFFFFFu ? x_.D : o_.dg_spare_target;
  require(T <= x_.D, SS_E_INVALID,
          "device-gated: dg_spare_target " + std::to_string(T) + " above the billed spares (" + std::to_string(x_.D) + ")");
  c.spare_target = T;
  c.prefetch_reserve_auto = o_.dg_prefetch_reserve == 0xFFFFFFFFu;
  c.prefetch_reserve = c.prefetch_reserve_auto ? std::min<uint32_t>(24, T / 4) : o_.dg_prefetch_reserve;
  c.prefetch_per_layer = o_.dg_prefetch_per_layer;
  c.prefetch_per_token = o_.dg_prefetch_per_token;
  c.wb_defer = o_.dg_wb_defer != 0;
  c.wb_on_d2h = o_.dg_wb_stream == 1;
  c.wb_layer_bytes = o_.dg_wb_layer_bytes;
  c.wb_max_outstanding = o_.dg_wb_max_outstanding;
  c.inclusive = x_.I;
  c.disk_tier = x_.disk_tier;
  c.disk_prefetch = x_.disk_prefetch;
  c.home_blocks = x_.disk_tier ? x_.P : 0;
  c.disk_staging = x_.S;
  c.clean_evict = o_.dg_clean_evict != 0;
  c.bank_keep = x_.bank_keep;
  c.landing_blocks = x_.L;
  c.landing_ttl = x_.landing_ttl;
  c.scored = x_.scored;
  c.scored_auto = o_.policy == SS_POLICY_SCORED_AUTO;
  c.w_trans = x_.w_trans;
  c.w_freq = x_.w_freq;
  c.w_rec = x_.w_rec;
  c.max_ids = x_.B;
  core_ = std::make_unique<DgCore>(c, tr_.get());
  if (x_.disk_tier)
    tr_->enable_disk(
        [this](uint32_t k, char* dst) {
          read_key(k, dst);
          if (o_.verify_hash == 1) check_key(k, dst);  // (verify_hash 2: the device checks the landed bytes)
        },
        [this](uint32_t k, uint32_t p, uint64_t off, uint64_t bytes, char* dst) {  // (reader threads: the sources'
          read_part(k, p, off, bytes, dst);                                         // positional reads are thread-safe)
        },
        [this](uint32_t k, const char* block) {
          if (o_.verify_hash == 1) check_key(k, block);
        },
        dw_);
  // dg_disk_queue_adapt (the open accepted it only with the file tier at SS_DG_DISK_QUEUE_AUTO): the pool's depth
  // from its measured throughput, unless one reader or file prefetches make it moot (reference src/dg_ctx.cpp:1897)
  if (o_.dg_disk_queue_adapt) {
    adapt_ = 2;
    if (x_.disk_queue <= 1) adapt_why_ = "one reader";
    else if (x_.disk_prefetch) adapt_why_ = "file prefetches";
    else adapt_ = 1, tr_->adapt_reads();
  }
  // priority: the seed (validated), the plan's residents, then key order
  std::vector<uint32_t> order;
  for (uint32_t i = 0; i < o_.dg_seed_n; ++i) {
    require(o_.dg_seed != nullptr, SS_E_INVALID, "device-gated: dg_seed_n > 0 with a null dg_seed");
    const ss_dg_unit& e = o_.dg_seed[i];
    require(e.gated >= 0 && uint32_t(e.gated) < G && e.unit >= 0 &&
                uint32_t(e.unit) < core_->units(uint32_t(e.gated)),
            SS_E_INVALID, "device-gated: dg_seed entry " + std::to_string(i) + " is out of range");
    order.push_back(core_->key(uint32_t(e.gated), uint32_t(e.unit)));
  }
  o_.dg_seed = nullptr;
  o_.dg_seed_n = 0;
  order.insert(order.end(), x_.residents.begin(), x_.residents.end());
  for (uint32_t k = 0; k < x_.keys; ++k) order.push_back(k);
  core_->seat(order, x_.disk_tier ? &x_.disk : nullptr);
  if (o_.dg_score_profile_len) {  // checked by the layout; its counts are read here only, before the first token
    std::vector<uint32_t> units;
    for (uint32_t g = 0; g < G; ++g) units.push_back(core_->units(g));
    const ScoreProfile v = check_score_profile(o_.dg_score_profile, o_.dg_score_profile_len, units, x_.score_identity);
    core_->seed_transitions(v.cells);
    score_prov_ = v.provenance;
  }
  o_.dg_score_profile = nullptr;
  o_.dg_score_profile_len = 0;
  fill();
  tr_->upload_table(core_->table().data(), x_.keys);
  core_->audit();
  run_.assign(G, 1);
  kept_.assign(G, {});
  base_l_.assign(G, DgLayerCounts{});
  fold(false);
  svc_ = std::make_unique<DgService>(core_.get(), m_, x_.B, o_.dg_wait_timeout_ms, o_.device);
  if (o_.dg_diag) {
    tr_->enable_diag(G);
    svc_->enable_timeline();
    diag_rows_.assign(G, LayerDiag{});
  }
  svc_->set_hooks({[this] { tr_->poll_checks(); }, [this] { tr_->drain_checks(); }});
  svc_->start();
  tr_->set_service_thread(svc_->thread_id());
}

// The stats-v1 document of a device-gated context (reference src/dg_ctx.cpp:1359-1545): the host contract's keys, the
// exclusive object and the device_gated object. Counters of what this library does not serve (priors, window
// prefetches, placement rounds, make-resident, layer tokens) are 0, as the reference writes them when those are off;
// so are score_deferred and score_last_ns (this library ranks only at the boundary, where score_ns counts the
// selection); backend is "hip".
Json HipDgCtx::format_stats(const ss_dg_stats& s, const ss_exclusive_stats& x,
                            const std::vector<ss_layer_stats>& layers, uint32_t pol, const Extras& extra) const {
  static const std::pair<const char*, uint64_t ss_dg_stats::*> kFields[] = {
      {"tokens", &ss_dg_stats::tokens}, {"lookups", &ss_dg_stats::lookups}, {"misses", &ss_dg_stats::misses},
      {"covered", &ss_dg_stats::covered}, {"fetched", &ss_dg_stats::fetched},
      {"prefetched", &ss_dg_stats::prefetched}, {"prefetch_used", &ss_dg_stats::prefetch_used},
      {"pred_invalid", &ss_dg_stats::pred_invalid}, {"resurrected", &ss_dg_stats::resurrected},
      {"bank_serves", &ss_dg_stats::bank_serves}, {"collected_mid", &ss_dg_stats::collected_mid},
      {"evicted", &ss_dg_stats::evicted}, {"evict_short", &ss_dg_stats::evict_short},
      {"writebacks_done", &ss_dg_stats::writebacks_done}, {"stalled", &ss_dg_stats::stalled},
      {"wb_deferred", &ss_dg_stats::wb_deferred}, {"wb_cancelled", &ss_dg_stats::wb_cancelled},
      {"wb_forced", &ss_dg_stats::wb_forced}, {"wb_boundary_flushed", &ss_dg_stats::wb_boundary_flushed},
      {"wb_issued_bytes", &ss_dg_stats::wb_issued_bytes}, {"wb_completed_bytes", &ss_dg_stats::wb_completed_bytes},
      {"wb_cancelled_bytes", &ss_dg_stats::wb_cancelled_bytes},
      {"wb_boundary_flushed_bytes", &ss_dg_stats::wb_boundary_flushed_bytes},
      {"wb_forced_wait_ns", &ss_dg_stats::wb_forced_wait_ns}, {"winpf_hints", &ss_dg_stats::winpf_hints},
      {"winpf_hint_rows", &ss_dg_stats::winpf_hint_rows}, {"prior_issued", &ss_dg_stats::prior_issued},
      {"prior_used", &ss_dg_stats::prior_used}, {"prior_late", &ss_dg_stats::prior_late},
      {"prior_reverted", &ss_dg_stats::prior_reverted}, {"l1_candidates", &ss_dg_stats::l1_candidates},
      {"l1_issued", &ss_dg_stats::l1_issued}, {"l1_used", &ss_dg_stats::l1_used}, {"l1_late", &ss_dg_stats::l1_late},
      {"l1_reverted", &ss_dg_stats::l1_reverted}, {"l1_priced_out", &ss_dg_stats::l1_priced_out},
      {"l1_skipped_ahead", &ss_dg_stats::l1_skipped_ahead}, {"prior_budget_stops", &ss_dg_stats::prior_budget_stops},
      {"pf_reverted", &ss_dg_stats::pf_reverted}, {"pf_revert_bytes", &ss_dg_stats::pf_revert_bytes},
      {"pred_skipped_ahead", &ss_dg_stats::pred_skipped_ahead},
      {"pred_shadow_file_predicted", &ss_dg_stats::pred_shadow_file_predicted},
      {"pred_shadow_file_demanded", &ss_dg_stats::pred_shadow_file_demanded},
      {"pred_shadow_file_hit", &ss_dg_stats::pred_shadow_file_hit},
      {"pred_shadow_file_predicted_bytes", &ss_dg_stats::pred_shadow_file_predicted_bytes},
      {"pred_shadow_file_demanded_bytes", &ss_dg_stats::pred_shadow_file_demanded_bytes},
      {"pred_shadow_file_hit_bytes", &ss_dg_stats::pred_shadow_file_hit_bytes},
      {"pf_strict_refused", &ss_dg_stats::pf_strict_refused}, {"landing_issued", &ss_dg_stats::landing_issued},
      {"landing_promoted", &ss_dg_stats::landing_promoted}, {"landing_late", &ss_dg_stats::landing_late},
      {"landing_wait_ns", &ss_dg_stats::landing_wait_ns}, {"landing_expired", &ss_dg_stats::landing_expired},
      {"landing_dropped_full", &ss_dg_stats::landing_dropped_full},
      {"landing_read_bytes", &ss_dg_stats::landing_read_bytes},
      {"landing_cancelled", &ss_dg_stats::landing_cancelled},
      {"landing_expired_layer", &ss_dg_stats::landing_expired_layer},
      {"landing_skipped_passed", &ss_dg_stats::landing_skipped_passed},
      {"landing_yields", &ss_dg_stats::landing_yields},
      {"landing_aborted_bytes", &ss_dg_stats::landing_aborted_bytes},
      {"score_fallbacks", &ss_dg_stats::score_fallbacks}, {"scored_victims", &ss_dg_stats::scored_victims},
      {"score_layers", &ss_dg_stats::score_layers}, {"score_candidates", &ss_dg_stats::score_candidates},
      {"score_saturated", &ss_dg_stats::score_saturated}, {"score_ns", &ss_dg_stats::score_ns},
      {"score_deferred", &ss_dg_stats::score_deferred}, {"score_last_ns", &ss_dg_stats::score_last_ns},
      {"resident_units", &ss_dg_stats::resident_units}, {"resident_evicted", &ss_dg_stats::resident_evicted},
      {"resident_bytes", &ss_dg_stats::resident_bytes}, {"resident_ns", &ss_dg_stats::resident_ns},
      {"mkres_file_reads", &ss_dg_stats::mkres_file_reads}, {"mkres_file_bytes", &ss_dg_stats::mkres_file_bytes},
      {"mkres_read_ns", &ss_dg_stats::mkres_read_ns}, {"mkres_h2d_bytes", &ss_dg_stats::mkres_h2d_bytes},
      {"mkres_wb_bytes", &ss_dg_stats::mkres_wb_bytes}, {"round_count", &ss_dg_stats::round_count},
      {"round_units", &ss_dg_stats::round_units}, {"round_bytes", &ss_dg_stats::round_bytes},
      {"round_ns", &ss_dg_stats::round_ns}, {"round_cancelled", &ss_dg_stats::round_cancelled},
      {"lm_tokens", &ss_dg_stats::lm_tokens}, {"lm_parts", &ss_dg_stats::lm_parts},
      {"lm_mid_evictions", &ss_dg_stats::lm_mid_evictions}, {"lm_early_admits", &ss_dg_stats::lm_early_admits}};
  static const std::pair<const char*, uint64_t ss_dg_stats::*> kDiskFields[] = {
      {"disk_reads", &ss_dg_stats::disk_reads}, {"disk_read_bytes", &ss_dg_stats::disk_read_bytes},
      {"disk_read_ns", &ss_dg_stats::disk_read_ns}, {"disk_stage_waits", &ss_dg_stats::disk_stage_waits},
      {"disk_drops", &ss_dg_stats::disk_drops}, {"disk_discards", &ss_dg_stats::disk_discards},
      {"inclusive_kept", &ss_dg_stats::inclusive_kept}, {"inclusive_drops", &ss_dg_stats::inclusive_drops},
      {"disk_wait_ns", &ss_dg_stats::disk_wait_ns}, {"disk_overlapped", &ss_dg_stats::disk_overlapped},
      {"disk_carried", &ss_dg_stats::disk_carried}, {"disk_carried_bytes", &ss_dg_stats::disk_carried_bytes},
      {"disk_max_in_flight", &ss_dg_stats::disk_max_in_flight}, {"clean_drops", &ss_dg_stats::clean_drops},
      {"clean_drop_bytes", &ss_dg_stats::clean_drop_bytes}, {"bank_kept", &ss_dg_stats::bank_kept}};
  Json j = Json::object();
  j["schema"] = Json::string("strix-stream/stats-v1");
  j["backend"] = Json::string("hip");
  j["forwards"] = Json::number(s.tokens);
  Json direct = Json::array();
  for (const auto& f : files_) direct.push(Json::boolean(f->direct()));
  j["sources_direct"] = direct;
  ss_layer_stats t{};
  Json ls = Json::array();
  for (const ss_layer_stats& l : layers) {
    add_stats(t, l);
    ls.push(stats_object(l));
  }
  j["total"] = stats_object(t);
  j["layers"] = ls;
  Json e = Json::object();
  e["writebacks"] = Json::number(x.writebacks);
  e["writeback_bytes"] = Json::number(x.writeback_bytes);
  e["deferred"] = Json::number(x.deferred);
  e["wb_deferred"] = Json::number(fold_.wb_deferred);  // since open, as the other exclusive counters
  e["rereads"] = Json::number(uint64_t(0));
  e["promoted"] = Json::number(x.promoted);
  e["free_blocks"] = Json::number(x.free_blocks);
  e["min_free_blocks"] = Json::number(x.min_free_blocks);
  e["blocks"] = Json::number(uint64_t(x_.blocks));
  j["exclusive"] = e;
  Json g = Json::object();
  for (const auto& f : kFields) g[f.first] = Json::number(s.*f.second);
    g["free_slots"] = Json::number(uint64_t(uint64_t(s.free_slots)));
  g["blocks"] = Json::number(uint64_t(uint64_t(x_.blocks)));
  g["slots"] = Json::number(uint64_t(uint64_t(x_.slots)));
  g["pf_revert_unused"] = Json::number(uint64_t(0));
  g["pf_strict_admit"] = Json::number(uint64_t(0));
  g["pf_legacy"] = Json::number(uint64_t(1));
  g["landing_blocks"] = Json::number(uint64_t(x_.L));
  g["landing_max_queued"] = Json::number(uint64_t(x_.L ? x_.landing_queued : 0));
  g["landing_ttl"] = Json::number(uint64_t(x_.landing_ttl));
  g["landing_failed"] = Json::number(extra.landing_failed);
  g["policy"] = Json::string(pol == 2 ? "auto" : pol == 1 ? "scored" : "lru");
  g["cuda_module_loading"] = Json::string("unknown");  // (a CUDA setting; HIP has no such mode)
  if (x_.L && !x_.landing_chunk) g["landing_chunk"] = Json::string("whole");
  else g["landing_chunk"] = Json::number(uint64_t(x_.L ? x_.landing_chunk : 0));
  if (!score_prov_.empty()) g["score_profile"] = Json::string(score_prov_);
  if (x_.disk_tier || x_.I) {  // three tiers or clean copies: only then, so the two-tier document is unchanged
    Json tt = Json::object();
    for (const auto& f : kDiskFields) tt[f.first] = Json::number(s.*f.second);
    tt["unit_subread_bytes"] = Json::number(uint64_t(0));
    tt["clean_evict"] = Json::number(uint64_t(uint64_t(o_.dg_clean_evict != 0)));
    tt["bank_keep"] = Json::number(uint64_t(o_.dg_bank_keep));
    tt["bank_keep_drops"] = Json::number(extra.keep_drops);
    tt["bank_keep_rereads"] = Json::number(extra.keep_rereads);
    tt["disk_queue"] = Json::number(uint64_t(uint64_t(x_.disk_queue)));
    tt["disk_queue_resolved"] = Json::number(uint64_t(uint64_t(x_.disk_queue)));
    tt["disk_locations"] = Json::number(uint64_t(uint64_t(x_.disk_tier ? 1 : 0)));
    tt["disk_units_open"] = Json::number(uint64_t(uint64_t(x_.F)));
    tt["staging"] = Json::number(uint64_t(uint64_t(x_.S)));
    tt["inclusive_blocks"] = Json::number(uint64_t(uint64_t(x_.I)));
    tt["disk_queue_adapt"] = Json::string(adapt_ == 1 ? "on" : adapt_ == 2 ? "declined: " + adapt_why_ : "off");
    if (adapt_ == 1)
      tr_->read_controller([&](const ReadDepthController& c) {
        Json a = Json::object();
        const std::pair<const char*, uint64_t> nums[] = {
            {"depth", c.depth()}, {"bound", c.bound()}, {"calibrating", c.calibrating()}, {"changes", c.changes},
            {"calibrations", c.calibrations}, {"windows", c.windows}, {"decisions", c.verdicts()},
            {"reads_1", c.reads_1}, {"bytes_1", c.bytes_1}, {"busy_ns_1", c.ns_1}, {"reads_u", c.reads_u},
            {"bytes_u", c.bytes_u}, {"busy_ns_u", c.ns_u}};
        for (const auto& f : nums) a[f.first] = Json::number(f.second);
        static const char* const why[] = {"start", "keep_u", "keep_1", "split", "recheck", "drift"};
        a["ring"] = Json::array();
        for (const ReadDepthController::Verdict& v : c.recent()) {
          Json e = Json::object();
          e["seq"] = Json::number(v.seq);
          e["reads"] = Json::number(v.reads);
          e["from"] = Json::number(uint64_t(v.from));
          e["to"] = Json::number(uint64_t(v.to));
          e["gbps_u"] = Json::number_f(v.gbps_u);  // (bytes / ns = GB/s)
          e["gbps_1"] = Json::number_f(v.gbps_1);
          e["reason"] = Json::string(why[int(v.why)]);
          a["ring"].push(e);
        }
        tt["disk_depth"] = a;
      });
    g["three_tier"] = tt;
  }
  j["device_gated"] = g;
  return j;
}

void HipDgCtx::read_key(uint32_t k, char* dst) const {
  for (uint32_t p = 0; p < x_.part_bytes.size(); ++p) read_part(k, p, 0, x_.part_bytes[p], dst + x_.part_offset[p]);
}

void HipDgCtx::read_part(uint32_t k, uint32_t p, uint64_t off, uint64_t bytes, char* dst) const {
  const uint32_t g = core_->gated_of(k);
  const int L = x_.gated[g];
  const int u = int(k - x_.unit_base[g]);
  const Part& part = d_.layers[size_t(L)].parts[p];
  const SourceFile& f = *files_[size_t(part.source)];
  const uint64_t F = part.offset + uint64_t(u) * part.stride + off;
  require(F + bytes <= f.size(), SS_E_IO,
          "unit (" + std::to_string(L) + ", " + std::to_string(u) + ") is past the end of its source");
  const uint64_t al = std::max<uint64_t>(d_.sources[size_t(part.source)].align, 512);
  if (!f.direct() || (F % al == 0 && bytes % al == 0 && reinterpret_cast<uintptr_t>(dst) % al == 0)) {
    f.pread_all(dst, bytes, F);
  } else {  // a buffered read of an unaligned range
    SourceFile bf(f.path(), false);
    bf.pread_all(dst, bytes, F);
  }
}

void HipDgCtx::check_key(uint32_t k, const char* dst) const {
  const uint32_t g = core_->gated_of(k);
  const Layer& l = d_.layers[size_t(x_.gated[g])];
  const uint32_t u = k - x_.unit_base[g];
  if (l.hash.empty()) return;
  require(xxh64(dst, size_t(x_.unit_bytes)) == l.hash[size_t(u)], SS_E_HASH,
          "unit (" + std::to_string(l.index) + ", " + std::to_string(u) + ") bytes read from its file differ from the "
          "descriptor hash");
}

// Open-time fill, in parallel: every key from its file into its home. Units homed on the device are read into a free
// spare block (the spare blocks hold nothing before the first write-back, so they serve as the fill's staging and
// the fill pins no memory of its own; one per worker), then copied into their arena slot; the other units are read
// straight into their pinned block. With verify_hash the unit's XXH64 is checked against the descriptor; with
// verify_hash = 2 its checkpoints are kept in HBM for the device check of every later landing.
void HipDgCtx::fill() {
  const uint32_t G = uint32_t(x_.gated.size());
  std::vector<uint64_t> digests(x_.keys, 0);
  bool have_hash = true;
  for (int L : x_.gated) have_hash = have_hash && !d_.layers[size_t(L)].hash.empty();
  const bool dverify = o_.verify_hash == 2 && have_hash;
  uint64_t n_ckpt = 0;
  std::vector<uint64_t> ckpt_host;
  if (dverify) {
    n_ckpt = tsa_checkpoint_count(x_.part_bytes.data(), uint32_t(x_.part_bytes.size()), verify_seg_bytes(x_.unit_bytes));
    ckpt_dev_ = static_cast<uint64_t*>(dev_->alloc_device(uint64_t(x_.keys) * n_ckpt * 32, "verify checkpoints"));
    ckpt_host.assign(size_t(uint64_t(x_.keys) * n_ckpt * 4), 0);
  }
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned max_threads = std::min<unsigned>(16, hw);
  std::vector<uint32_t> dev_keys, host_keys, file_keys;
  for (uint32_t k = 0; k < x_.keys; ++k) {
    const DgCore::Where h = core_->where(k);
    (h == DgCore::Where::Resident ? dev_keys : h == DgCore::Where::File ? file_keys : host_keys).push_back(k);
  }
  // three-tier: the file homes stay in their files; with a hash check each is read once here, through a staging
  // buffer per worker, for its hash (and its checkpoints), never kept
  if (!o_.verify_hash || !have_hash) file_keys.clear();
  const std::vector<int32_t> spare = core_->free_block_ids();
  require(dev_keys.empty() || !spare.empty(), SS_E_CAPACITY, "device-gated: no free block to stage the fill through");
  const std::vector<uint32_t>* keys = nullptr;
  std::atomic<uint32_t> next{0};
  std::mutex err_mu;
  std::string err;
  ss_status err_st = SS_OK;
  auto work = [&](char* stage) {
    hipStream_t st = nullptr;
    try {
      dev_->bind();
      if (stage) st = dev_->stream_create();
      for (;;) {
        const uint32_t i = next.fetch_add(1);
        if (i >= keys->size()) break;
        {
          std::lock_guard<std::mutex> lk(err_mu);
          if (err_st != SS_OK) break;
        }
        const uint32_t k = (*keys)[i];
        const uint32_t g = core_->gated_of(k);
        const int L = x_.gated[g];
        const int u = int(k - x_.unit_base[g]);
        const Layer& l = d_.layers[size_t(L)];
        const DgCore::Where home = core_->where(k);
        const bool on_dev = home == DgCore::Where::Resident;
        char* dst = home == DgCore::Where::Pinned ? tr_->block_ptr(core_->block_of(k)) : stage;
        read_key(k, dst);
        if (o_.verify_hash && !l.hash.empty()) {
          tsa_unit hu{};
          for (size_t p = 0; p < x_.part_bytes.size(); ++p) {
            hu.ext[p].ptr = dst + x_.part_offset[p];
            hu.ext[p].bytes = x_.part_bytes[p];
          }
          hu.n_ext = uint32_t(x_.part_bytes.size());
          uint64_t dig = 0;
          if (dverify) {
            const ss_status s = tsa_xxh64_checkpoints(&hu, verify_seg_bytes(x_.unit_bytes),
                                                      ckpt_host.data() + uint64_t(k) * n_ckpt * 4,
                                                      n_ckpt, &dig);
            require(s == SS_OK, s, "device-gated: checkpoints of a unit");
          } else {
            dig = xxh64(dst, size_t(x_.unit_bytes));
          }
          digests[k] = l.hash[size_t(u)];
          require(dig == l.hash[size_t(u)], SS_E_HASH,
                  "unit (" + std::to_string(L) + ", " + std::to_string(u) + ") bytes differ from the descriptor hash");
        }
        if (on_dev) {
          const int32_t slot = core_->slot_of(k);
          for (size_t p = 0; p < x_.part_bytes.size(); ++p)
            copy_h2d(static_cast<char*>(arena_[p]) + uint64_t(slot) * x_.part_bytes[p], dst + x_.part_offset[p],
                     x_.part_bytes[p], st);
          stream_sync(st);
        }
      }
    } catch (const Error& e) {
      std::lock_guard<std::mutex> lk(err_mu);
      if (err_st == SS_OK) {
        err_st = e.status();
        err = e.what();
      }
    } catch (const std::exception& e) {
      std::lock_guard<std::mutex> lk(err_mu);
      if (err_st == SS_OK) {
        err_st = SS_E_BACKEND;
        err = e.what();
      }
    }
    if (st) dev_->stream_destroy(st);
  };
  // phase 1: the device homes, one spare block per worker; phase 2: the block homes; phase 3: the file homes, one
  // staging buffer per worker
  for (int phase = 0; phase < 3 && err_st == SS_OK; ++phase) {
    keys = phase == 0 ? &dev_keys : phase == 1 ? &host_keys : &file_keys;
    next = 0;
    const size_t cap = phase == 0 ? spare.size() : phase == 1 ? size_t(max_threads) : size_t(x_.S);
    const unsigned n = unsigned(std::min<size_t>({size_t(max_threads), cap, keys->size()}));
    std::vector<std::thread> th;
    for (unsigned i = 0; i < n; ++i)
      th.emplace_back(work, phase == 0 ? tr_->block_ptr(spare[i])
                            : phase == 2 ? tr_->block_ptr(int32_t(x_.blocks + i)) : nullptr);
    for (auto& t : th) t.join();
  }
  if (err_st != SS_OK) fail(err_st, err);
  if (dverify) {
    hip_check(hipMemcpy(ckpt_dev_, ckpt_host.data(), ckpt_host.size() * 8, hipMemcpyHostToDevice),
              "hipMemcpy (checkpoints)");
    tr_->enable_verify(digests, ckpt_dev_, n_ckpt, G * x_.B + o_.dg_prefetch_per_token + 64, dw_);
  }
  (void)G;
}

void HipDgCtx::release() noexcept {
  if (svc_) svc_->stop_join();
  if (tr_) tr_->stop_reads();  // the readers use this context's sources and layout
  if (dev_) (void)hipDeviceSynchronize();
  svc_.reset();
  core_.reset();
  tr_.reset();
  if (!dev_) return;
  for (void* a : arena_) dev_->free_device(a);
  dev_->free_device(slot_of_dev_);
  dev_->free_device(ctl_dev_);
  dev_->free_device(ckpt_dev_);
  dev_->free_pinned(mapped_host_);
  for (void* c : block_chunks_) dev_->free_pinned(c);
  arena_.clear();
  block_chunks_.clear();
  dev_.reset();
}

}  // namespace

std::unique_ptr<DgCtx> open_dg_ctx(const Desc& d, const Plan& p, const ss_options& o) {
  require(o.forward_mode == SS_FORWARD_DEVICE_GATED, SS_E_INVALID,
          "device-gated: forward_mode is not SS_FORWARD_DEVICE_GATED");
  return std::make_unique<HipDgCtx>(d, p, o);
}

}  // namespace tsa
