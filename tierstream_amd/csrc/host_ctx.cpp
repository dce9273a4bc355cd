#include "host_ctx.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>

#include "copy_runs.hpp"
#include "stats_json.hpp"
#include "tsa_device.hpp"

namespace tsa {
namespace {

constexpr uint64_t kHostAlign = 4096;
constexpr uint64_t kSegBytes = 2 * 1024;  // device check checkpoints: 32 B per 2 KiB segment (1.6 % of a unit)
constexpr size_t kCheckBatch = 32;         // landed units per device check launch

uint64_t now_ns() {
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count());
}

// The four XXH64 accumulators at every multiple of `seg` below a unit's whole-stripe span, taken while its bytes
// stream through the host hash once (the tsa.h checkpoint layout of a one-extent unit).
class CheckpointHasher {
 public:
  CheckpointHasher(uint64_t unit_bytes, uint64_t seg, uint64_t* states) : seg_(seg), states_(states) {
    const uint64_t span = unit_bytes / 32 * 32;
    count_ = seg ? std::max<uint64_t>(1, (span + seg - 1) / seg) : 0;
  }
  void feed(const void* p, uint64_t n) {
    const char* c = static_cast<const char*>(p);
    while (n) {
      take_checkpoints();
      uint64_t step = n;
      if (states_ && next_ < count_) step = std::min(step, next_ * seg_ - pos_);
      if (!step) step = n;
      h_.update(c, size_t(step));
      pos_ += step;
      c += step;
      n -= step;
    }
    take_checkpoints();
  }
  uint64_t digest() const { return h_.digest(); }

 private:
  void take_checkpoints() {
    for (; states_ && next_ < count_ && pos_ == next_ * seg_; ++next_) std::memcpy(states_ + 4 * next_, h_.acc(), 32);
  }
  Xxh64 h_;
  uint64_t seg_, count_ = 0, next_ = 0, pos_ = 0;
  uint64_t* states_;
};

}  // namespace

HostCtx::HostCtx(const Desc& d, const ss_budget& b, const Plan& p, const ss_options& o)
    : d_(d), plan_(p), o_(o), place_(d_, plan_, o_) {
  (void)b;
  place_.attach(this);
  try {
    init();
  } catch (...) {
    cleanup();
    throw;
  }
}

HostCtx::~HostCtx() { cleanup(); }

hipEvent_t HostCtx::pooled_event() {
  if (!ev_pool_.empty()) {
    hipEvent_t e = ev_pool_.back();
    ev_pool_.pop_back();
    return e;
  }
  hipEvent_t e = dev_->event_create();
  all_events_.push_back(e);
  return e;
}

void HostCtx::init() {
  require(o_.verify_hash >= 0 && o_.verify_hash <= 2, SS_E_INVALID, "open: verify_hash must be 0, 1 or 2");
  if (!o_.reader_threads) o_.reader_threads = 2;
  if (!o_.staging_buffers) o_.staging_buffers = 4;
  if (!o_.staging_bytes) o_.staging_bytes = uint64_t(256) << 20;
  if (!o_.copy_piece_bytes) o_.copy_piece_bytes = uint64_t(64) << 20;
  uint64_t align = kHostAlign;
  for (const auto& s : d_.sources) align = std::max(align, s.align);
  require(o_.staging_bytes >= 4 * align, SS_E_INVALID, "open: staging_bytes must be >= 4 x the source alignment");
  o_.staging_bytes = round_up(o_.staging_bytes, align);

  dev_ = std::make_unique<HipDevice>(o_.device);
  copy_ = dev_->stream_create_dedicated();
  for (int i = 1; i < kCopyStreams; ++i) {
    copyx_.push_back(dev_->stream_create_dedicated());
    joinx_ev_.push_back(dev_->event_create());
    vreadyx_ev_.push_back(dev_->event_create());
  }
  for (const auto& s : d_.sources) files_.push_back(std::make_unique<SourceFile>(s.path, o_.direct_io != 0));
  for (uint32_t i = 0; i < o_.staging_buffers; ++i) {
    staging_.push_back(Staging{dev_->alloc_pinned(o_.staging_bytes, "staging buffer"), nullptr});
    staging_.back().ev = dev_->event_create();
    staging_free_.push_back(i);
  }

  // pinned blocks: the pinned tier's layout (one allocation per chunk), then each class's spares in 1 GiB chunks
  {
    const PinnedLayout pl = pinned_layout(d_, plan_.tier);
    const size_t first_chunk = host_chunks_.size();
    for (uint64_t bytes : pl.chunk_bytes) host_chunks_.push_back(dev_->alloc_pinned(bytes, "pinned tier"));
    const auto& blocks = place_.blocks();
    const auto& cls_bytes = place_.block_class_bytes();
    block_addr_.assign(blocks.size(), nullptr);
    block_alloc_.assign(blocks.size(), -1);
    std::vector<uint64_t> left(cls_bytes.size(), 0);
    for (const BlockHome& b : blocks)
      if (b.home < 0) ++left[size_t(b.cls)];
    char* cursor = nullptr;
    uint64_t in_chunk = 0;
    int32_t cursor_cls = -1;
    for (size_t i = 0; i < blocks.size(); ++i) {
      const BlockHome& b = blocks[i];
      if (b.cls >= 0) ++excl_blocks_;
      if (b.home >= 0) {
        block_addr_[i] = at(host_chunks_[first_chunk + size_t(pl.chunk_of[size_t(b.home)])],
                            pl.offset_of[size_t(b.home)]);
        block_alloc_[i] = int32_t(first_chunk + size_t(pl.chunk_of[size_t(b.home)]));
        continue;
      }
      const uint64_t bytes = cls_bytes[size_t(b.cls)];
      if (!in_chunk || cursor_cls != b.cls) {
        const uint64_t n = std::min(std::max<uint64_t>(1, kPinnedChunk / bytes), left[size_t(b.cls)]);
        host_chunks_.push_back(dev_->alloc_pinned(n * bytes, "spare blocks"));
        cursor = static_cast<char*>(host_chunks_.back());
        in_chunk = n;
        cursor_cls = b.cls;
      }
      block_addr_[i] = cursor;
      block_alloc_[i] = int32_t(host_chunks_.size() - 1);
      cursor += bytes;
      --in_chunk;
      --left[size_t(b.cls)];
    }
  }
  if (place_.exclusive()) {
    wb_ = dev_->stream_create_dedicated();
    blocks_ev_ = dev_->event_create();
    wb_mark_ev_ = dev_->event_create();
  }

  L_.resize(d_.layers.size());
  for (size_t L = 0; L < d_.layers.size(); ++L) {
    const Layer& l = d_.layers[L];
    LayerDev& s = L_[L];
    s.release_ev = dev_->event_create();
    s.ready_ev = dev_->event_create();
    s.ids_ev = dev_->event_create();
    if (!l.n_units) continue;
    s.stride = d_.unit_stride(int(L));
    if (place_.pool_slots(int(L))) s.pool = dev_->alloc_device(uint64_t(place_.pool_slots(int(L))) * s.stride, "pool");
    for (int v = 0; v < 2; ++v) {
      s.table_host[v] = static_cast<uint64_t*>(dev_->alloc_pinned(8 * uint64_t(l.n_units), "unit table"));
      std::memset(s.table_host[v], 0, 8 * size_t(l.n_units));
      s.table_dev[v] = dev_->alloc_device(8 * uint64_t(l.n_units), "unit table");
      s.table_ev[v] = dev_->event_create();
    }
  }
  for (const auto& rc : place_.ring_classes()) {
    ring_base_.push_back(dev_->alloc_device(rc.stride * rc.count, "stream ring"));
    for (uint32_t i = 0; i < rc.count; ++i) {
      ring_addr_.push_back(at(ring_base_.back(), rc.stride * i));
      ring_alloc_.push_back(int32_t(ring_base_.size() - 1));
    }
  }

  if (o_.verify_hash == 2) {  // the device check of every landed unit: checkpoint tables and the launch slots
    dverify_ = true;
    seg_bytes_ = kSegBytes;
    checks_.assign(size_t(d_.total_units), UnitCheck{});
    vcap_ = size_t(d_.total_units) + 8;
    vtable_host_ = static_cast<tsa_verify_unit*>(dev_->alloc_pinned(vcap_ * sizeof(tsa_verify_unit), "check table"));
    vfail_host_ = static_cast<uint32_t*>(dev_->alloc_pinned(vcap_ * 4, "check results"));
    vtable_dev_ = dev_->alloc_device(vcap_ * sizeof(tsa_verify_unit), "check table");
    vfail_dev_ = static_cast<uint32_t*>(dev_->alloc_device(vcap_ * 4, "check results"));
    ventry_flush_.assign(vcap_, 0);
    hip_check(hipMemsetAsync(vfail_dev_, 0, vcap_ * 4, copy_), "hipMemsetAsync");
    vdone_ev_ = dev_->event_create();
    vready_ev_ = dev_->event_create();
    vstream_ = dev_->stream_create_dedicated();
    stream_sync(copy_);
  }

  if (place_.ra_on()) {  // host read-ahead: buffers of the largest unit a file read can bring, each with its event
    for (uint32_t i = 0; i < o_.readahead_units; ++i) {
      ra_ev_.push_back(dev_->event_create());
      ra_buf_.push_back(dev_->alloc_pinned(place_.ra_bytes(), "read-ahead buffer"));
      ra_free_.push_back(int32_t(o_.readahead_units - 1 - i));  // buffer 0 taken first
    }
    ra_index_.resize(d_.layers.size());
    for (size_t L = 0; L < d_.layers.size(); ++L) ra_index_[L].assign(size_t(d_.layers[L].n_units), -1);
  }

  reads_.set_readers(int(o_.reader_threads));
  for (uint32_t i = 0; i < o_.reader_threads; ++i) readers_.emplace_back([this] { reader_loop(); });

  // the pinned tier from the files, then the residents (from their pinned copies where they have one)
  for (size_t i = 0; i < place_.blocks().size(); ++i) {
    const BlockHome& b = place_.blocks()[i];
    if (b.home < 0) continue;
    auto c = std::make_shared<Copy>();
    const size_t L = size_t(std::upper_bound(d_.unit_base.begin(), d_.unit_base.end(), b.home) - d_.unit_base.begin()) - 1;
    c->layer = int32_t(L);
    c->unit = int32_t(b.home - d_.unit_base[L]);
    c->to_host = true;
    c->dst = block_addr_[i];
    fills_.push_back(c);
    submit(c);
  }
  for (const CopyPtr& c : fills_) await(*c);
  fills_.clear();
  {
    PendGuard g{this};
    place_.place_residents();
    flush_copies();
  }
  for (const CopyPtr& c : fills_) await(*c);
  for (const CopyPtr& c : fills_) release_event(*c);
  fills_.clear();
  sync_copies();
  if (dverify_) collect_verify();  // the residents' device check, one batch at open
}

void HostCtx::cleanup() noexcept {
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    reads_.stop();
  }
  for (auto& t : readers_) t.join();
  readers_.clear();
  if (!dev_) return;
  (void)hipDeviceSynchronize();
  for (auto& s : L_) {
    dev_->free_device(s.pool);
    dev_->event_destroy(s.release_ev);
    dev_->event_destroy(s.ready_ev);
    dev_->event_destroy(s.ids_ev);
    dev_->free_pinned(s.ids_host);
    for (int v = 0; v < 2; ++v) {
      dev_->free_pinned(s.table_host[v]);
      dev_->free_device(s.table_dev[v]);
      dev_->event_destroy(s.table_ev[v]);
    }
  }
  for (void* b : ring_base_) dev_->free_device(b);
  for (void* c : host_chunks_) dev_->free_pinned(c);
  for (auto& s : staging_) {
    dev_->free_pinned(s.host);
    dev_->event_destroy(s.ev);
  }
  for (void* b : ra_buf_) dev_->free_pinned(b);
  for (hipEvent_t e : ra_ev_) dev_->event_destroy(e);
  for (hipEvent_t e : all_events_) dev_->event_destroy(e);
  dev_->event_destroy(blocks_ev_);
  dev_->event_destroy(wb_mark_ev_);
  for (auto& c : checks_) dev_->free_device(c.states_dev);
  dev_->free_pinned(vtable_host_);
  dev_->free_pinned(vfail_host_);
  dev_->free_device(vtable_dev_);
  dev_->free_device(vfail_dev_);
  dev_->event_destroy(vdone_ev_);
  dev_->event_destroy(vready_ev_);
  for (hipEvent_t e : vflush_ev_) dev_->event_destroy(e);
  for (hipEvent_t e : prof_made_) dev_->event_destroy(e);
  dev_->stream_destroy(vstream_);
  for (hipEvent_t e : joinx_ev_) dev_->event_destroy(e);
  for (hipEvent_t e : vreadyx_ev_) dev_->event_destroy(e);
  dev_->stream_destroy(copy_);
  for (hipStream_t x : copyx_) dev_->stream_destroy(x);
  dev_->stream_destroy(wb_);
  L_.clear();
  dev_.reset();
}

// ---- placement orders -------------------------------------------------------------------------------------------------

void* HostCtx::spot_addr(int layer, const DevSpot& s) const {
  if (s.kind == DevSpot::kRing) return ring_addr_[size_t(s.index)];
  if (s.kind == DevSpot::kPool) return at(L_[size_t(layer)].pool, uint64_t(s.index) * L_[size_t(layer)].stride);
  return nullptr;
}

// Exclusive mode: victims' slots to their new blocks on the write-back stream. Blocks freed in an earlier forward are
// written only after that forward's copies out of them (blocks_ev_, recorded at its end on the copy stream).
void HostCtx::write_back(const WriteBackOrder& w) {
  if (wb_gate_) {
    ord_.wait(wb_, blocks_ev_);
    wb_gate_ = false;
  }
  hipEvent_t ev = pooled_event();
  if (size_t(w.batch) >= wb_ev_.size()) wb_ev_.resize(size_t(w.batch) + 1, nullptr);
  wb_ev_[size_t(w.batch)] = ev;
  const uint64_t ub = d_.layers[size_t(w.layer)].unit_bytes;
  for (size_t i = 0; i < w.slots.size(); ++i)
    copy_d2h(block_addr_[size_t(w.blocks[i])], spot_addr(w.layer, DevSpot{DevSpot::kPool, w.slots[i]}), ub, wb_);
  ord_.record(ev, wb_);
}

bool HostCtx::fetch(const FetchOrder& f) {
  auto c = std::make_shared<Copy>();
  c->layer = f.layer;
  c->unit = f.unit;
  c->speculative = f.speculative;
  c->dst = spot_addr(f.layer, f.dst);
  c->src = f.src_block >= 0 ? block_addr_[size_t(f.src_block)] : nullptr;
  c->src_alloc = f.src_block >= 0 ? block_alloc_[size_t(f.src_block)] : -1;
  c->dst_alloc = f.dst.kind == DevSpot::kRing ? ring_alloc_[size_t(f.dst.index)] : -2 - f.layer;
  c->after[0] = f.after_release >= 0 ? L_[size_t(f.after_release)].release_ev : nullptr;
  c->after[1] = f.after_writeback >= 0 ? wb_ev_[size_t(f.after_writeback)] : nullptr;
  c->after[2] = f.src_writeback >= 0 ? wb_ev_[size_t(f.src_writeback)] : nullptr;
  c->done_ev = pooled_event();
  if (f.job >= 0) {
    if (size_t(f.job) >= jobs_.size()) jobs_.resize(size_t(f.job) + 1);
    jobs_[size_t(f.job)] = c;
  } else {
    fills_.push_back(c);
  }
  if (ra_on() && f.job >= 0 && f.src_block < 0) {
    const int32_t i = ra_index_[size_t(f.layer)][size_t(f.unit)];
    if (i >= 0) {
      RaEntry& e = *ra_entries_[size_t(i)];
      if (f.speculative) {
        if (f.dst.kind == DevSpot::kPool) {  // a speculative admission reads the file as any speculative fetch
          std::lock_guard<std::mutex> lk(q_mu_);
          ra_abandon_locked(e);
        }  // (a speculative ring fetch leaves the request alone)
      } else if (ra_land(e, c)) {
        return true;
      }
    }
  }
  submit(c);
  return false;
}

void HostCtx::promote(int32_t job) {
  const CopyPtr& c = jobs_[size_t(job)];
  std::lock_guard<std::mutex> lk(q_mu_);
  if (c->state.load() != Copy::kQueued || !c->speculative) return;
  if (reads_.raise(ReadClass::kGuess, c)) c->speculative = false;  // a demand now: ahead of every other queued read
}

void HostCtx::retire(int32_t job) {
  Copy& c = *jobs_[size_t(job)];
  int queued = Copy::kQueued;
  if (!c.state.compare_exchange_strong(queued, Copy::kCancelled)) await_quiet(c);
  done_cv_.notify_all();
}

bool HostCtx::settle(int32_t job, bool) {
  Copy& c = *jobs_[size_t(job)];
  int queued = Copy::kQueued;
  if (c.speculative && c.state.compare_exchange_strong(queued, Copy::kCancelled)) return false;
  await_quiet(c);
  const int st = c.state.load();
  if (st == Copy::kFailed && fwd_failed_ == SS_OK) {
    fwd_failed_ = c.status;
    fwd_error_ = c.what;
  }
  return st == Copy::kDone;
}

// ---- copies and reads ---------------------------------------------------------------------------------------------

void HostCtx::submit(const CopyPtr& c) {
  if (c->src && !c->to_host) {  // a pinned block: issued when the engine call returns (flush_copies)
    pend_.push_back(c);
    c->state.store(Copy::kDone);
    return;
  }
  std::lock_guard<std::mutex> lk(q_mu_);
  reads_.push(c->speculative ? ReadClass::kGuess : ReadClass::kDemand, c);
}

// Host memory (a pinned block, a read-ahead buffer) into c's destination on the next copy stream (an SDMA queue), in
// pieces of copy_piece_bytes, behind the destination's waits; after_ev (if any) is recorded behind the copy too.
void HostCtx::issue_copy(Copy& c, const void* src, hipEvent_t after_ev) {
  std::lock_guard<std::mutex> lk(copy_mu_);
  issue_copy_locked(c, src, after_ev);
}

void HostCtx::issue_copy_locked(Copy& c, const void* src, hipEvent_t after_ev) {
  const uint64_t n = d_.layers[size_t(c.layer)].unit_bytes;
  const hipStream_t cs = next_copy_stream();
  wait_slot_check(cs, c.dst);
  for (hipEvent_t e : c.after) ord_.wait(cs, e);
  for (uint64_t off = 0; off < n; off += o_.copy_piece_bytes)
    copy_h2d(at(c.dst, off), at(src, off), std::min(o_.copy_piece_bytes, n - off), cs);
  ord_.record(c.done_ev, cs);
  if (after_ev) ord_.record(after_ev, cs);
  if (dverify_) verify_landed(c);
}

void HostCtx::flush_copies() {
  if (pend_.empty()) return;
  std::lock_guard<std::mutex> lk(copy_mu_);
  // Copies behind a write-back of this forward (into a victim's slot, or out of a block being written) go after the
  // others the engine call ordered: the write-back, a device-to-host copy on its own stream, runs while the copy
  // streams move the rest instead of holding the stream it waits on.
  std::stable_partition(pend_.begin(), pend_.end(), [](const CopyPtr& c) { return !c->after[1] && !c->after[2]; });
  std::vector<CopyRunItem> items(pend_.size());
  for (size_t k = 0; k < pend_.size(); ++k) {
    const Copy& c = *pend_[k];
    items[k] = CopyRunItem{c.layer, c.src_alloc, c.dst_alloc, uint64_t(reinterpret_cast<uintptr_t>(c.src)),
                           uint64_t(reinterpret_cast<uintptr_t>(c.dst))};
  }
  size_t i = 0;
  try {
    while (i < pend_.size()) {
      const uint64_t n = d_.layers[size_t(pend_[i]->layer)].unit_bytes;
      const uint64_t cap = std::max(o_.copy_piece_bytes, n);  // a run of small units stays one piece
      const size_t j = copy_run_end(items.data(), items.size(), i, n, cap);
      issue_run(i, j, j > i + 1 ? (items[j - 1].dst - items[i].dst) + n : n);
      i = j;
    }
  } catch (...) {
    for (; i < pend_.size(); ++i) {  // never issued: their waits would see nothing
      pend_[i]->state.store(Copy::kFailed);
      pend_[i]->status = SS_E_BACKEND;
    }
    pend_.clear();
    throw;
  }
  pend_.clear();
}

void HostCtx::issue_run(size_t first, size_t end, uint64_t span) {
  Copy& lead = *pend_[first];
  pinned_units_ += end - first;
  ++pinned_copies_;
  if (end == first + 1) {
    issue_copy_locked(lead, lead.src, nullptr);
    return;
  }
  const hipStream_t cs = next_copy_stream();
  hipEvent_t waited[16];
  size_t n_waited = 0;
  for (size_t k = first; k < end; ++k) {
    Copy& c = *pend_[k];
    wait_slot_check(cs, c.dst);
    for (hipEvent_t e : c.after) {
      if (!e || std::find(waited, waited + n_waited, e) != waited + n_waited) continue;
      ord_.wait(cs, e);
      if (n_waited < 16) waited[n_waited++] = e;
    }
  }
  for (uint64_t off = 0; off < span; off += o_.copy_piece_bytes)
    copy_h2d(at(lead.dst, off), at(lead.src, off), std::min(o_.copy_piece_bytes, span - off), cs);
  ord_.record(lead.done_ev, cs);
  for (size_t k = first; k < end; ++k) {
    Copy& c = *pend_[k];
    if (k != first) {
      ev_pool_.push_back(c.done_ev);
      c.done_ev = lead.done_ev;
      c.owns_ev = false;
    }
    if (dverify_) verify_landed(c);
  }
}

// Engine-stream waits for jobs' copies: each distinct event once (the units of one run share theirs).
void HostCtx::wait_jobs(const std::vector<int32_t>& jobs, hipStream_t es) {
  std::vector<hipEvent_t> seen;
  for (int32_t j : jobs) {
    Copy& c = *jobs_[size_t(j)];
    await(c);
    if (!c.done_ev || std::find(seen.begin(), seen.end(), c.done_ev) != seen.end()) continue;
    ord_.wait(es, c.done_ev);
    seen.push_back(c.done_ev);
  }
}

void HostCtx::finish(Copy& c, int state, ss_status st, const std::string& what) noexcept {
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    c.status = st;
    try {
      c.what = what;
    } catch (...) {
    }
    c.state.store(state);
    if (c.reading) reads_.ended(c.ran_as);
    c.reading = false;
  }
  done_cv_.notify_all();
}

void HostCtx::await_quiet(Copy& c) {
  if (c.state.load() >= Copy::kDone) return;  // (an ended copy never changes state again: no lock needed)
  std::unique_lock<std::mutex> lk(q_mu_);
  done_cv_.wait(lk, [&] { return c.state.load() >= Copy::kDone; });
}

void HostCtx::await(Copy& c) {
  await_quiet(c);
  if (c.state.load() == Copy::kFailed) fail(c.status, c.what);
}

// One reader thread: it starts whatever read the scheduler gives it, runs it outside the lock, and reports the
// outcome (a read-ahead read through its request, which may have a landing waiting for it).
void HostCtx::reader_loop() {
  try {
    dev_->bind();
  } catch (...) {  // (a device that cannot be bound fails the first copy this thread issues)
  }
  for (;;) {
    CopyPtr c;
    {
      std::unique_lock<std::mutex> lk(q_mu_);
      ReadClass cls;
      if (!reads_.wait_next(lk, &c, &cls)) return;
      int queued = Copy::kQueued;
      if (!c->state.compare_exchange_strong(queued, Copy::kRunning)) {  // cancelled while it queued: never read
        reads_.ended(cls);
        done_cv_.notify_all();
        continue;
      }
      c->reading = true;
      c->ran_as = cls;
    }
    ReadOutcome r;
    try {
      read_file_unit(*c);
    } catch (const Error& e) {
      r = ReadOutcome{Copy::kFailed, e.status(), e.what()};
    } catch (const std::bad_alloc&) {
      r = ReadOutcome{Copy::kFailed, SS_E_NOMEM, "out of host memory"};
    } catch (const std::exception& e) {
      r = ReadOutcome{Copy::kFailed, SS_E_BACKEND, e.what()};
    }
    if (c->ra) ra_read_ended(*c, r.state, r.status, r.what);  // (its landing first: the read counts as ended after)
    else finish(*c, r.state, r.status, r.what);
  }
}

void HostCtx::test_hold_readers(bool hold) {
  std::lock_guard<std::mutex> lk(q_mu_);
  reads_.hold(hold);
}

// ss_test_inject (the reference's one-shot fault injections, src/stream_ctx.cpp:508-1015): 1 queueing a read-ahead
// read fails, 2 queueing a landing fails, 3 a landing's copy fails before it starts, 4 after its first piece (its buffer
// is quarantined), 5 a read-ahead read fails, 8 fails after a part, 9 reads bytes that fail the hash. The
// synchronization mutations 6, 7 and 10 (a copy skipping a wait) are not offered. Any other value arms nothing.
void HostCtx::test_inject(int what) {
  require(what != 6 && what != 7 && what != 10, SS_E_UNSUPPORTED,
          "ss_test_inject: mutations that skip a copy's wait (6, 7, 10) are not offered by this library");
  inject_.store(what);
}

bool HostCtx::take_inject(int what) {
  int armed = what;
  return inject_.load() == what && inject_.compare_exchange_strong(armed, 0);
}

void HostCtx::test_ra_quiesce() {
  for (auto& e : ra_entries_)
    if (e->producer) await_quiet(*e->producer);
}

size_t HostCtx::take_staging() {
  std::unique_lock<std::mutex> lk(staging_mu_);
  staging_cv_.wait(lk, [&] { return !staging_free_.empty(); });
  const size_t i = staging_free_.back();
  staging_free_.pop_back();
  return i;
}

void HostCtx::give_staging(size_t i) {
  {
    std::lock_guard<std::mutex> lk(staging_mu_);
    staging_free_.push_back(i);
  }
  staging_cv_.notify_one();
}

void HostCtx::read_file_unit(Copy& c) {
  const Layer& l = d_.layers[size_t(c.layer)];
  const bool hash = o_.verify_hash && !l.hash.empty();
  if (c.to_host) {
    uint64_t digest = 0;
    if (c.ra) ev_sync(ra_ev_[size_t(c.ra->buf)]);  // the buffer's last copy out has completed
    if (c.ra && take_inject(5)) fail(SS_E_IO, "read-ahead: injected read failure");
    read_into_host(c.layer, c.unit, c.dst, hash, &digest, &c.bytes_read);
    if (c.ra && take_inject(9)) digest = ~digest;
    require(!hash || digest == l.hash[size_t(c.unit)], SS_E_HASH,
            "unit (" + std::to_string(c.layer) + ", " + std::to_string(c.unit) + ") bytes differ from the descriptor hash");
    return;
  }
  stage_to_device(c);
}

// The checkpoint states a host hash of (layer, unit) records for the device check: one set of four accumulators per
// check segment, or none when device checks are off or the unit has no descriptor hash.
std::vector<uint64_t> HostCtx::checkpoint_buffer(const Layer& l, bool hash) const {
  if (!dverify_ || !hash) return {};
  const uint64_t span = l.unit_bytes / 32 * 32;
  return std::vector<uint64_t>(4 * std::max<uint64_t>(1, (span + seg_bytes_ - 1) / seg_bytes_), 0);
}

// Keeps a unit's checkpoints in HBM (the first time a host hash certified them; copy_mu_ held).
void HostCtx::keep_checkpoints_locked(int64_t g, const std::vector<uint64_t>& states) {
  if (checks_[size_t(g)].states_dev) return;
  UnitCheck k;
  k.n_states = states.size() / 4;
  k.states_dev = static_cast<uint64_t*>(dev_->alloc_device(states.size() * 8, "check checkpoints"));
  hip_check(hipMemcpy(k.states_dev, states.data(), states.size() * 8, hipMemcpyHostToDevice), "hipMemcpy");
  checks_[size_t(g)] = k;
}

const SourceFile& HostCtx::part_source(int layer, int unit, const Part& part, uint64_t* off) const {
  const SourceFile& f = *files_[size_t(part.source)];
  *off = part.offset + uint64_t(unit) * part.stride;
  require(*off + part.bytes <= f.size(), SS_E_IO,
          "unit (" + std::to_string(layer) + ", " + std::to_string(unit) + ") part " + part.name +
              " is past the end of its source");
  return f;
}

// A unit's file bytes into host memory at dst, part after part. A part whose offset, length and destination suit the
// file's alignment is read straight into dst and hashed there; any other part goes window by window through a staging
// buffer (an aligned covering read), each window's piece hashed in the staging buffer while it is still in cache, then
// copied out to dst. got (if given) counts the bytes read so far, also when a read fails part-way. With device checks
// on, the checkpoints the hash recorded are kept in HBM once its digest matches the descriptor.
void HostCtx::read_into_host(int layer, int unit, void* dst, bool hash, uint64_t* digest, uint64_t* got) {
  const Layer& l = d_.layers[size_t(layer)];
  std::vector<uint64_t> states = checkpoint_buffer(l, hash);
  CheckpointHasher h(l.unit_bytes, seg_bytes_, states.empty() ? nullptr : states.data());
  uint64_t pos = 0;
  for (const Part& part : l.parts) {
    uint64_t off = 0;
    const SourceFile& f = part_source(layer, unit, part, &off);
    const uint64_t al = std::max<uint64_t>(d_.sources[size_t(part.source)].align, 512);
    char* out = at(dst, pos);
    const bool straight = !f.direct() || (off % al == 0 && part.bytes % al == 0 && uintptr_t(out) % al == 0);
    if (straight) {
      f.pread_all(out, part.bytes, off);
      if (got) *got += part.bytes;
      if (hash) h.feed(out, part.bytes);
    } else {
      const uint64_t cap = (o_.staging_bytes - 2 * al) / al * al;
      for_each_cover_window(off, part.bytes, al, cap, [&](const CoverWindow& w) {
        struct Lease {  // the staging buffer goes back however the window ends
          HostCtx& x;
          size_t i;
          ~Lease() { x.give_staging(i); }
        } lease{*this, take_staging()};
        char* buf = static_cast<char*>(staging_[lease.i].host);
        ev_sync(staging_[lease.i].ev);  // its last copy out has completed
        require(f.pread_some(buf, w.span, w.a0) >= w.lead + w.len, SS_E_IO,
                "short read of " + f.path() + " at " + std::to_string(w.a0));
        if (hash) h.feed(buf + w.lead, w.len);
        std::memcpy(out + w.at, buf + w.lead, size_t(w.len));
        if (got) *got += w.len;
      });
    }
    pos += part.bytes;
    if (got && take_inject(8)) fail(SS_E_IO, "read-ahead: injected failure after a part");
  }
  if (digest) *digest = h.digest();
  if (!states.empty() && h.digest() == l.hash[size_t(unit)]) {
    std::lock_guard<std::mutex> lk(copy_mu_);
    keep_checkpoints_locked(gidx(layer, unit), states);
  }
}

// A reader thread: the unit's file bytes, staging buffer by staging buffer, onto the device on the copy stream (the
// destination's waits before its first piece), hashed on the way.
void HostCtx::stage_to_device(Copy& c) {
  const Layer& l = d_.layers[size_t(c.layer)];
  const bool hash = o_.verify_hash && !l.hash.empty();
  std::vector<uint64_t> states = checkpoint_buffer(l, hash);
  CheckpointHasher h(l.unit_bytes, seg_bytes_, states.empty() ? nullptr : states.data());
  uint64_t pos = 0;
  bool ordered = false;  // the destination's waits go before its first piece
  for (const Part& part : l.parts) {
    uint64_t off = 0;
    const SourceFile& f = part_source(c.layer, c.unit, part, &off);
    const uint64_t al = f.direct() ? std::max<uint64_t>(d_.sources[size_t(part.source)].align, 512) : 1;
    const uint64_t cap = (o_.staging_bytes - 2 * std::max<uint64_t>(al, kHostAlign)) / kHostAlign * kHostAlign;
    for_each_cover_window(off, part.bytes, al, cap, [&](const CoverWindow& w) {
      struct Lease {  // the staging buffer goes back however the window ends
        HostCtx& x;
        size_t i;
        ~Lease() { x.give_staging(i); }
      } lease{*this, take_staging()};
      Staging& st = staging_[lease.i];
      ev_sync(st.ev);  // its last copy out has completed
      require(f.pread_some(st.host, w.span, w.a0) >= w.lead + w.len, SS_E_IO,
              "short read of " + f.path() + " at " + std::to_string(w.a0));
      const char* piece = at(st.host, w.lead);
      if (hash) h.feed(piece, w.len);
      std::lock_guard<std::mutex> lk(copy_mu_);
      if (!ordered) {
        wait_slot_check(copy_, c.dst);
        for (hipEvent_t e : c.after) ord_.wait(copy_, e);
        ordered = true;
      }
      copy_h2d(at(c.dst, pos + w.at), piece, w.len, copy_);
      ord_.record(st.ev, copy_);
    });
    pos += part.bytes;
  }
  require(!hash || h.digest() == l.hash[size_t(c.unit)], SS_E_HASH,
          "unit (" + std::to_string(c.layer) + ", " + std::to_string(c.unit) + ") bytes differ from the descriptor hash");
  std::lock_guard<std::mutex> lk(copy_mu_);
  if (!states.empty()) keep_checkpoints_locked(gidx(c.layer, c.unit), states);
  ord_.record(c.done_ev, copy_);
  if (dverify_) verify_landed(c);
}

// ---- host read-ahead (readahead_units; reference src/stream_ctx.cpp:732-1017, docs/design.md 3.6) -----------------------
// A forward's file-backed units that wait for a ring slot (or that ss_host_prefetch names) are read ahead into pinned
// read-ahead buffers, one unit each, by the reader threads below demand reads; when the unit gets its slot, the copy
// lands from the buffer (at once if the read ended, else when it does: a read still queued then becomes a demand
// read). Placement never depends on it: the same slots, tables and groups, only where the bytes come from.

void HostCtx::read_ahead(int layer, int unit) {
  if (!ra_on() || ra_frozen_) return;
  ra_entries_.push_back(std::make_unique<RaEntry>());
  RaEntry& e = *ra_entries_.back();
  e.layer = layer;
  e.unit = unit;
  ra_index_[size_t(layer)][size_t(unit)] = int32_t(ra_entries_.size() - 1);
  ra_wait_.push_back(&e);
}

// Waiting requests take free buffers, oldest first; one whose unit got a copy or a pinned source meanwhile is dropped.
void HostCtx::ra_pump() {
  if (!ra_on() || ra_frozen_) return;
  while (!ra_wait_.empty()) {
    RaEntry& e = *ra_wait_.front();
    bool drop;
    {
      std::lock_guard<std::mutex> lk(q_mu_);
      drop = e.st != RaEntry::kWaiting;
      if (!drop && !place_.ra_wanted(e.layer, e.unit)) {
        e.st = RaEntry::kAbandoned;
        drop = true;
      }
    }
    if (drop) {
      ra_wait_.pop_front();
      continue;
    }
    auto p = std::make_shared<Copy>();
    p->layer = e.layer;
    p->unit = e.unit;
    p->to_host = true;
    p->ra = &e;
    {
      std::lock_guard<std::mutex> lk(q_mu_);
      if (ra_free_.empty()) return;  // the next engine call tries again
      e.buf = ra_free_.back();
      ra_free_.pop_back();
      p->dst = ra_buf_[size_t(e.buf)];
      e.producer = p;
      if (take_inject(1)) {  // queueing the read failed: it ends at once, and the unit's fetch reads its file
        p->status = SS_E_NOMEM;
        p->what = "read-ahead: queueing a read failed";
        p->state.store(Copy::kFailed);
        ra_give_buf_locked(e);
        e.st = RaEntry::kFailed;
      } else {
        e.st = RaEntry::kReading;
        reads_.push(ReadClass::kAhead, p);
      }
    }
    ra_wait_.pop_front();
  }
}

void HostCtx::ra_give_buf_locked(RaEntry& e) {
  if (e.buf < 0) return;
  ra_free_.push_back(e.buf);
  e.buf = -1;
}

void HostCtx::ra_abandon_locked(RaEntry& e) {
  switch (e.st) {
    case RaEntry::kWaiting:
      e.st = RaEntry::kAbandoned;
      break;
    case RaEntry::kReady:  // read, never to land
      ra_give_buf_locked(e);
      e.st = RaEntry::kAbandoned;
      break;
    case RaEntry::kReading: {
      int queued = Copy::kQueued;
      if (e.producer->state.compare_exchange_strong(queued, Copy::kCancelled)) {  // never started: no read at all
        reads_.remove(ReadClass::kAhead, e.producer);
        ra_give_buf_locked(e);
      }  // (running: its end gives the buffer back)
      e.st = RaEntry::kAbandoned;
      break;
    }
    default:  // Landing (its copy decides), Consumed, Abandoned, Failed
      break;
  }
}

// The unit got its slot (a demand fetch, child: its job): lands from the buffer when the read ended or runs, else
// (never started, or failed: a fallback) the caller reads the file.
bool HostCtx::ra_land(RaEntry& e, const CopyPtr& child) {
  bool issue = false, attached = false, fallback = false, lost = false;
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    switch (e.st) {
      case RaEntry::kWaiting:  // not started: the ordinary read starts as early
        e.st = RaEntry::kAbandoned;
        break;
      case RaEntry::kReady:
        e.child = child;
        child->state.store(Copy::kRunning);
        attached = true;
        if (take_inject(2)) {  // the landing fails for good (no fallback that depends on timing)
          e.st = RaEntry::kFailed;
          ra_give_buf_locked(e);
          lost = true;
        } else {
          e.st = RaEntry::kLanding;
          issue = true;
        }
        break;
      case RaEntry::kReading: {
        e.st = RaEntry::kLanding;
        e.child = child;
        attached = true;
        reads_.raise(ReadClass::kAhead, e.producer);  // still queued: a demand waits behind it now
        break;
      }
      case RaEntry::kFailed:
        fallback = true;
        break;
      default:
        break;
    }
  }
  if (fallback) ++ra_st_.fallback;
  if (lost) finish(*child, Copy::kFailed, SS_E_NOMEM, "read-ahead: queueing a landing failed");
  if (issue) ra_issue_child(e, *child);
  return attached;
}

// The copy out of the read-ahead buffer into the child's slot (the child is running); the buffer is read again only
// after this copy (its event).
void HostCtx::ra_issue_child(RaEntry& e, Copy& child) {
  int state = Copy::kDone;
  ss_status st = SS_OK;
  std::string what;
  bool quarantine = false;  // a copy out of the buffer may still run: it is never read into again
  try {
    if (take_inject(3)) fail(SS_E_IO, "read-ahead: injected copy failure");
    if (take_inject(4)) {
      quarantine = true;
      issue_first_piece(child, ra_buf_[size_t(e.buf)]);
      fail(SS_E_IO, "read-ahead: injected copy failure after its first piece");
    }
    issue_copy(child, ra_buf_[size_t(e.buf)], ra_ev_[size_t(e.buf)]);
  } catch (const Error& x) {
    state = Copy::kFailed, st = x.status(), what = x.what();
  } catch (const std::exception& x) {
    state = Copy::kFailed, st = SS_E_BACKEND, what = x.what();
  }
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    e.st = state == Copy::kDone ? RaEntry::kConsumed : RaEntry::kFailed;
    if (quarantine) e.buf = -1;
    else ra_give_buf_locked(e);
  }
  finish(child, state, st, what);
}

// (ss_test_inject 4) only the first piece of a landing's copy, behind the destination's waits.
void HostCtx::issue_first_piece(Copy& c, const void* src) {
  std::lock_guard<std::mutex> lk(copy_mu_);
  const hipStream_t cs = next_copy_stream();
  wait_slot_check(cs, c.dst);
  for (hipEvent_t e : c.after) ord_.wait(cs, e);
  copy_h2d(c.dst, src, std::min(o_.copy_piece_bytes, d_.layers[size_t(c.layer)].unit_bytes), cs);
}

// A read-ahead read ended (state kDone or kFailed; a reader thread): its request moves on - a landing waiting for it
// is issued now, or fails with it (the forward fails: its copy had no other source) - and only then the read counts
// as ended.
void HostCtx::ra_read_ended(Copy& p, int state, ss_status st, const std::string& what) {
  RaEntry& e = *p.ra;
  CopyPtr issue, failed, lost;
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    const bool ok = state == Copy::kDone;
    switch (e.st) {
      case RaEntry::kReading:
        if (ok) {
          e.st = RaEntry::kReady;
        } else {
          e.st = RaEntry::kFailed;
          ra_give_buf_locked(e);
        }
        break;
      case RaEntry::kLanding: {
        int queued = Copy::kQueued;
        if (!e.child->state.compare_exchange_strong(queued, Copy::kRunning)) {  // its copy was cancelled meanwhile
          ra_give_buf_locked(e);
          break;
        }
        if (ok && !take_inject(2)) {
          issue = e.child;
        } else {
          (ok ? lost : failed) = e.child;  // (ok: its landing could not be queued)
          e.st = RaEntry::kFailed;
          ra_give_buf_locked(e);
        }
        break;
      }
      case RaEntry::kAbandoned:
        ra_give_buf_locked(e);
        break;
      default:
        break;
    }
  }
  if (issue) ra_issue_child(e, *issue);
  if (failed) finish(*failed, Copy::kFailed, st, "read-ahead: " + what);
  if (lost) finish(*lost, Copy::kFailed, SS_E_NOMEM, "read-ahead: queueing a landing failed");
  finish(p, state, st, what);
}

// ss_end: no new request; the ones not landing are abandoned; every read ends (a landing's copy is issued by its
// read's end); then each request counts once and the file bytes it read count in the layer's bytes_disk.
void HostCtx::ra_end_forward() {
  if (!ra_on()) return;
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    ra_frozen_ = true;
    for (auto& e : ra_entries_) ra_abandon_locked(*e);
  }
  ra_wait_.clear();
  done_cv_.notify_all();
  for (auto& e : ra_entries_)
    if (e->producer) await_quiet(*e->producer);
  for (auto& e : ra_entries_) {
    ++ra_st_.requested;
    const int ps = e->producer ? e->producer->state.load() : int(Copy::kCancelled);
    const uint64_t b = e->producer ? e->producer->bytes_read : 0;
    ra_st_.bytes += b;
    place_.add_disk_bytes(e->layer, b);
    if (ps == Copy::kDone) {
      ++ra_st_.read;
      if (e->st == RaEntry::kConsumed) ++ra_st_.landed;
      else ++ra_st_.unused;
    } else if (ps == Copy::kFailed) {
      ++ra_st_.failed;
    }
    ra_index_[size_t(e->layer)][size_t(e->unit)] = -1;
  }
  ra_entries_.clear();
  ra_frozen_ = false;
}

// ---- device checks (verify_hash = 2) --------------------------------------------------------------------------------

// The landed unit joins the pending batch (copy_mu_ held: its copies are enqueued). kCheckBatch units are launched
// together on the verify stream behind both copy streams; the rest at ss_end, where results are collected.
void HostCtx::verify_landed(const Copy& c) {
  const Layer& l = d_.layers[size_t(c.layer)];
  const UnitCheck& k = checks_[size_t(gidx(c.layer, c.unit))];
  if (l.hash.empty() || !k.states_dev) return;
  require(vused_ < vcap_, SS_E_BACKEND, "device check: launch table full (internal)");
  const size_t i = vused_++;
  tsa_verify_unit& v = vtable_host_[i];
  std::memset(&v, 0, sizeof v);
  v.ext[0].ptr = c.dst;
  v.ext[0].bytes = l.unit_bytes;
  v.n_ext = 1;
  v.seg_first = k.n_states;  // (the unit's checkpoint count until the flush turns it into the prefix sum)
  v.states = k.states_dev;
  v.digest = l.hash[size_t(c.unit)];
  v.total = l.unit_bytes;
  vunits_.push_back({c.layer, c.unit});
  vdst_[c.dst] = i;
  if (vused_ - vflushed_ >= kCheckBatch) flush_verify();
}

void HostCtx::wait_slot_check(hipStream_t s, const void* dst) {
  const auto it = vdst_.find(dst);
  if (it == vdst_.end()) return;
  if (it->second >= vflushed_) flush_verify();
  ord_.wait(s, vflush_ev_[ventry_flush_[it->second]]);
  vdst_.erase(it);
}

void HostCtx::join_copies() {
  for (size_t i = 0; i < copyx_.size(); ++i) {
    ord_.record(joinx_ev_[i], copyx_[i]);
    ord_.wait(copy_, joinx_ev_[i]);
  }
}

void HostCtx::sync_copies() {
  stream_sync(copy_);
  for (hipStream_t x : copyx_) stream_sync(x);
}

void HostCtx::flush_verify() {
  const size_t n = vused_ - vflushed_;
  if (!n) return;
  uint64_t segs = 0;
  for (size_t i = vflushed_; i < vused_; ++i) {
    const uint64_t count = vtable_host_[i].seg_first;
    vtable_host_[i].seg_first = segs;
    segs += count;
  }
  ord_.record(vready_ev_, copy_);
  ord_.wait(vstream_, vready_ev_);
  for (size_t i = 0; i < copyx_.size(); ++i) {
    ord_.record(vreadyx_ev_[i], copyx_[i]);
    ord_.wait(vstream_, vreadyx_ev_[i]);
  }
  tsa_verify_unit* vd = static_cast<tsa_verify_unit*>(vtable_dev_) + vflushed_;
  copy_h2d(vd, vtable_host_ + vflushed_, n * sizeof(tsa_verify_unit), vstream_);
  TimedCheck t{nullptr, nullptr, 0, uint32_t(n)};
  if (prof_verify_) {
    for (hipEvent_t* e : {&t.start, &t.stop}) {
      if (prof_free_.empty()) prof_made_.push_back(*e = dev_->event_create_timed());
      else *e = prof_free_.back(), prof_free_.pop_back();
    }
    for (size_t i = vflushed_; i < vused_; ++i) t.bytes += vtable_host_[i].total;
  }
  hip_check(hipError_t(launch_verify(vd, uint32_t(n), segs, seg_bytes_, vfail_dev_ + vflushed_, vstream_, t.start,
                                     t.stop)),
            "device check launch");
  if (t.start) prof_pending_.push_back(t);
  if (vflushes_ == vflush_ev_.size()) vflush_ev_.push_back(dev_->event_create());
  ord_.record(vflush_ev_[vflushes_], vstream_);
  for (size_t i = vflushed_; i < vused_; ++i) ventry_flush_[i] = vflushes_;
  ++vflushes_;
  vflushed_ = vused_;
}

void HostCtx::prof_drain(bool wait) {
  size_t kept = 0;
  for (const TimedCheck& t : prof_pending_) {
    if (wait) hip_check(hipEventSynchronize(t.stop), "hipEventSynchronize (check timing)");
    else if (hipEventQuery(t.stop) != hipSuccess) {
      prof_pending_[kept++] = t;
      continue;
    }
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, t.start, t.stop), "hipEventElapsedTime (check timing)");
    ++prof_sum_.verifies;
    prof_sum_.verify_units += t.units;
    prof_sum_.verify_bytes += t.bytes;
    prof_sum_.verify_ns += uint64_t(double(ms) * 1e6);
    prof_free_.push_back(t.start);
    prof_free_.push_back(t.stop);
  }
  prof_pending_.resize(kept);
}

void HostCtx::profile_enable(int on) {
  std::lock_guard<std::mutex> lk(copy_mu_);
  prof_drain(true);
  prof_verify_ = (on == 1) || (on & TSA_TEST_PROF_VERIFY);
  prof_sum_ = tsa_test_profile{};
}

tsa_test_profile HostCtx::profile_read(bool wait) {
  std::lock_guard<std::mutex> lk(copy_mu_);
  prof_drain(wait);
  tsa_test_profile out = prof_sum_;
  out.pending = prof_pending_.size();
  return out;
}

void HostCtx::collect_verify() {
  size_t n;
  {
    std::lock_guard<std::mutex> lk(copy_mu_);
    n = vused_;
    if (!n) return;
    flush_verify();
    copy_d2h(vfail_host_, vfail_dev_, 4 * n, vstream_);
    hip_check(hipMemsetAsync(vfail_dev_, 0, 4 * n, vstream_), "hipMemsetAsync");
    ord_.record(vdone_ev_, vstream_);
  }
  ev_sync(vdone_ev_);
  std::vector<std::pair<int, int>> units;
  {
    std::lock_guard<std::mutex> lk(copy_mu_);
    units.swap(vunits_);
    vused_ = vflushed_ = 0;
    vdst_.clear();
    vflushes_ = 0;
  }
  uint64_t bad = 0;
  std::string first;
  for (size_t i = 0; i < n; ++i)
    if (vfail_host_[i] && bad++ == 0) first = "(" + std::to_string(units[i].first) + ", " + std::to_string(units[i].second) + ")";
  verify_fail_total_ += bad;
  require(bad == 0, SS_E_HASH,
          "device verify: " + std::to_string(bad) + " landed unit(s) differ from the descriptor hash in HBM, first " +
              first);
}

// ---- the forward ----------------------------------------------------------------------------------------------------

void HostCtx::check_layer(int layer, const char* what) const {
  require(layer >= 0 && layer < n_layers(), SS_E_INVALID, std::string(what) + ": layer out of range");
}

// One engine stream per forward: every event the library records or waits on sits on it.
void HostCtx::check_stream(void* stream, const char* what) {
  if (!fwd_stream_set_) {
    fwd_stream_ = stream;
    fwd_stream_set_ = true;
    ord_.forget(static_cast<hipStream_t>(stream));  // (a new stream may reuse an earlier forward's handle)
    return;
  }
  require(stream == fwd_stream_, SS_E_INVALID,
          std::string(what) + ": a forward must use one engine stream (join other streams into it first)");
}

void HostCtx::seed(int layer, const int32_t* units, int n) {
  check_layer(layer, "seed");
  fills_.clear();
  std::vector<int32_t> placed;
  {
    PendGuard g{this};
    placed = place_.seed(layer, units, n);
    flush_copies();
  }
  ss_status failed = SS_OK;
  std::string error;
  std::vector<char> ok(placed.size(), 0);
  for (size_t i = 0; i < placed.size(); ++i) {
    Copy& c = *fills_[i];
    await_quiet(c);
    ok[i] = c.state.load() == Copy::kDone;
    if (!ok[i]) {
      place_.seed_landed(layer, placed[i], false);  // a seed whose read failed must not stay resident
      if (failed == SS_OK) {
        failed = c.status;
        error = c.what;
      }
    }
  }
  for (const CopyPtr& c : fills_) release_event(*c);
  fills_.clear();
  bool synced = true;
  try {
    sync_copies();
  } catch (const Error& e) {
    synced = false;
    if (failed == SS_OK) {
      failed = e.status();
      error = e.what();
    }
  }
  for (size_t i = 0; synced && i < placed.size(); ++i)
    if (ok[i]) place_.seed_landed(layer, placed[i], true);  // exclusive: its copy out of its block has completed
  if (failed != SS_OK) fail(failed, error);
}

void HostCtx::begin(const uint32_t* rows, int n_layers) { place_.begin(rows, n_layers); }

void HostCtx::routes(int layer, const int32_t* ids, int n) {
  check_layer(layer, "routes");
  PendGuard g{this};
  place_.routes(layer, ids, n);
  flush_copies();
  ra_pump();
}

void HostCtx::routes_all(int layer) {
  check_layer(layer, "layer_all");
  PendGuard g{this};
  place_.routes_all(layer);
  flush_copies();
  ra_pump();
}

// The ids are copied back on the engine stream right behind the router and taken at the next call that needs them.
void HostCtx::routes_dev(int layer, const int32_t* ids_dev, int n, void* stream) {
  check_layer(layer, "routes_dev");
  require(place_.in_forward(), SS_E_INVALID, "routes_dev: outside a forward (call ss_begin)");
  LayerDev& s = L_[size_t(layer)];
  require(n >= 0 && s.ids_n < 0 && !place_.routes_given(layer), SS_E_INVALID, "routes_dev: given twice or bad count");
  if (size_t(n) > s.ids_cap) {
    dev_->free_pinned(s.ids_host);
    s.ids_host = nullptr;
    s.ids_cap = std::max<size_t>(size_t(n), 1024);
    s.ids_host = static_cast<int32_t*>(dev_->alloc_pinned(4 * s.ids_cap, "device routes"));
  }
  check_stream(stream, "routes_dev");
  copy_d2h(s.ids_host, ids_dev, 4 * uint64_t(n), static_cast<hipStream_t>(stream));
  ord_.record(s.ids_ev, static_cast<hipStream_t>(stream));
  s.ids_n = n;
}

void HostCtx::ingest_dev_routes(int layer) {
  LayerDev& s = L_[size_t(layer)];
  if (s.ids_n < 0) return;
  ev_sync(s.ids_ev);
  const int n = s.ids_n;
  s.ids_n = -1;
  PendGuard g{this};
  place_.routes(layer, s.ids_host, n);
  flush_copies();
}

void HostCtx::prefetch(int layer, const int32_t* ids, int n, bool speculative) {
  check_layer(layer, "prefetch");
  PendGuard g{this};
  place_.prefetch(layer, ids, n, speculative);
  flush_copies();
  ra_pump();
}

void HostCtx::prefetch_layer(int layer) {
  check_layer(layer, "prefetch_layer");
  std::vector<int32_t> all(static_cast<size_t>(d_.layers[size_t(layer)].n_units));
  for (size_t u = 0; u < all.size(); ++u) all[u] = int32_t(u);
  PendGuard g{this};
  place_.prefetch(layer, all.data(), int(all.size()), false);
  flush_copies();
  ra_pump();
}

// Read-ahead of file-backed units of a layer, no device slot (a checked no-op while readahead_units is 0).
void HostCtx::host_prefetch(int layer, const int32_t* ids, int n) {
  check_layer(layer, "host_prefetch");
  place_.host_prefetch(layer, ids, n);
  ra_pump();
}

void HostCtx::host_prefetch_layer(int layer) {
  check_layer(layer, "host_prefetch_layer");
  if (!place_.ra_on()) return;
  std::vector<int32_t> all(static_cast<size_t>(d_.layers[size_t(layer)].n_units));
  for (size_t u = 0; u < all.size(); ++u) all[u] = int32_t(u);
  host_prefetch(layer, all.data(), int(all.size()));
}

void HostCtx::acquire(int layer, void* stream, bool wait_all, ss_layer_view* out) {
  check_layer(layer, "acquire");
  require(place_.in_forward(), SS_E_INVALID, "acquire: outside a forward");
  require(d_.layers[size_t(layer)].n_units > 0, SS_E_INVALID, "acquire: layer has no units");
  require(!place_.acquired(layer), SS_E_INVALID, "acquire: layer acquired twice in one forward");
  check_stream(stream, "acquire");
  ingest_dev_routes(layer);
  ra_pump();
  require(place_.routes_given(layer), SS_E_INVALID,
          "acquire: no routes for layer " + std::to_string(layer) + " (ss_layer_routes / ss_layer_all first)");
  const hipStream_t es = static_cast<hipStream_t>(stream);
  LayerDev& s = L_[size_t(layer)];
  PendGuard g{this};
  const HostPlacement::Acquire a = place_.acquire(layer, wait_all);
  flush_copies();
  if (a.wait_ready) ord_.wait(es, s.ready_ev);  // the copies an earlier forward issued into this layer's pool
  if (!a.wait_jobs.empty()) {
    const uint64_t t0 = now_ns();
    wait_jobs(a.wait_jobs, es);
    place_.add_wait_ns(layer, now_ns() - t0);
  }
  const std::vector<DevSpot>& t = place_.take_table(layer);
  s.version ^= 1;
  const int v = s.version;
  ev_sync(s.table_ev[v]);  // the acquire before last has released its table
  for (size_t u = 0; u < t.size(); ++u) s.table_host[v][u] = uint64_t(reinterpret_cast<uintptr_t>(spot_addr(layer, t[u])));
  copy_h2d(s.table_dev[v], s.table_host[v], 8 * uint64_t(t.size()), es);
  const auto& groups = place_.groups(layer);
  s.group_view.clear();
  for (const auto& g : groups) s.group_view.push_back(ss_group{g.data(), int(g.size())});
  out->table_dev = static_cast<const uint64_t*>(s.table_dev[v]);
  out->table_host = s.table_host[v];
  out->n_units = int(t.size());
  out->groups = s.group_view.data();
  out->n_groups = int(s.group_view.size());
}

void HostCtx::group_wait(int layer, int group, void* stream) {
  check_layer(layer, "group_wait");
  require(place_.acquired(layer) && !place_.released(layer), SS_E_INVALID, "group_wait: layer not acquired");
  require(group >= 0 && size_t(group) < place_.groups(layer).size(), SS_E_INVALID, "group_wait: no such group");
  check_stream(stream, "group_wait");
  const std::vector<int32_t> jobs = place_.group_jobs(layer, group);
  if (jobs.empty()) return;
  const uint64_t t0 = now_ns();
  wait_jobs(jobs, static_cast<hipStream_t>(stream));
  place_.add_wait_ns(layer, now_ns() - t0);
}

void HostCtx::release(int layer, void* stream) {
  check_layer(layer, "release");
  require(place_.acquired(layer) && !place_.released(layer), SS_E_INVALID,
          "release: layer not acquired or already released");
  check_stream(stream, "release");
  LayerDev& s = L_[size_t(layer)];
  ord_.record(s.release_ev, static_cast<hipStream_t>(stream));
  ord_.record(s.table_ev[s.version], static_cast<hipStream_t>(stream));  // its table is read until here
  PendGuard g{this};
  place_.release(layer);
  flush_copies();
  ra_pump();
}

void HostCtx::end() {
  require(place_.in_forward(), SS_E_INVALID, "end: no forward open");
  for (int L = 0; L < n_layers(); ++L)
    require(d_.layers[size_t(L)].n_units == 0 || !place_.acquired(L) || place_.released(L), SS_E_INVALID,
            "end: layer " + std::to_string(L) + " acquired but not released");
  fwd_failed_ = SS_OK;
  fwd_error_.clear();
  ra_end_forward();
  flush_copies();
  const HostPlacement::Ended e = place_.end();  // settles every job of the forward
  flush_copies();
  {
    std::lock_guard<std::mutex> lk(copy_mu_);
    join_copies();  // the once-per-forward marks below stand for the copies on both streams
    if (place_.exclusive()) {
      // the next forward's write-backs reuse blocks this one freed: they wait for blocks_ev_ (every copy out of them);
      // a later read of a block written back in this forward follows its write-back
      if (e.writeback_batches) {
        ord_.record(wb_mark_ev_, wb_);
        ord_.wait(copy_, wb_mark_ev_);
      }
      ord_.record(blocks_ev_, copy_);
      wb_gate_ = true;
    }
    // this forward's pool copies are issued but may still be in flight: the next acquire of those layers waits
    for (int L : e.landed_layers) ord_.record(L_[size_t(L)].ready_ev, copy_);
  }
  for (hipEvent_t ev : wb_ev_) ev_pool_.push_back(ev);
  wb_ev_.clear();
  for (const CopyPtr& c : jobs_)
    if (c) release_event(*c);
  jobs_.clear();
  fwd_stream_set_ = false;
  fwd_stream_ = nullptr;
  if (hook_) {
    ss_layer_stats tot{};
    for (const ss_layer_stats& s : place_.forward_stats()) add_stats(tot, s);
    hook_(hook_user_, &tot, place_.forward_stats().data(), n_layers());
  }
  publish();  // (a forward whose read failed is folded and published too)
  if (dverify_ && fwd_failed_ == SS_OK) collect_verify();
  if (fwd_failed_ != SS_OK) fail(fwd_failed_, fwd_error_);
}

// ss_check_unit (a test hook): the unit's bytes where this forward's table puts them must equal its file bytes and
// hash to the descriptor's digest. The device bytes come back a part at a time and are compared as they arrive, so a
// mismatch names the part and its first differing byte.
void HostCtx::check_unit(int layer, int unit) {
  check_layer(layer, "check_unit");
  const Layer& l = d_.layers[size_t(layer)];
  require(place_.acquired(layer) && !place_.released(layer), SS_E_INVALID, "check_unit: layer not acquired");
  require(unit >= 0 && unit < l.n_units, SS_E_INVALID, "check_unit: unit out of range");
  const LayerDev& s = L_[size_t(layer)];
  const char* dev = reinterpret_cast<const char*>(uintptr_t(s.table_host[s.version][unit]));
  require(dev != nullptr, SS_E_INVALID, "check_unit: unit not available in this forward");
  if (const int32_t j = place_.job_of(layer, unit); j >= 0) {  // its copy, if this forward made one, has landed
    await(*jobs_[size_t(j)]);
    ev_sync(jobs_[size_t(j)]->done_ev);
  }
  sync_copies();
  std::vector<char> file_buf(size_t(round_up(l.unit_bytes, kHostAlign) + kHostAlign));
  char* file = reinterpret_cast<char*>(round_up(uint64_t(uintptr_t(file_buf.data())), kHostAlign));
  read_into_host(layer, unit, file, false, nullptr);
  const std::string who = "(" + std::to_string(layer) + ", " + std::to_string(unit) + ")";
  uint64_t biggest = 0;
  for (const Part& part : l.parts) biggest = std::max(biggest, part.bytes);
  std::vector<char> landed(static_cast<size_t>(biggest));
  Xxh64 h;
  uint64_t pos = 0;
  for (const Part& part : l.parts) {
    hip_check(hipMemcpy(landed.data(), dev + pos, size_t(part.bytes), hipMemcpyDeviceToHost), "hipMemcpy (check_unit)");
    const auto diff = std::mismatch(landed.begin(), landed.begin() + std::ptrdiff_t(part.bytes), file + pos);
    require(diff.first == landed.begin() + std::ptrdiff_t(part.bytes), SS_E_HASH,
            "check_unit: landed bytes of " + who + " differ from the source (part " + part.name + ", byte " +
                std::to_string(diff.first - landed.begin()) + ")");
    h.update(landed.data(), size_t(part.bytes));
    pos += part.bytes;
  }
  require(l.hash.empty() || h.digest() == l.hash[size_t(unit)], SS_E_HASH,
          "check_unit: landed bytes of " + who + " differ from the descriptor hash");
}

Region HostCtx::region_of(uint64_t addr) const {
  Region r;
  if (!addr) return r;
  for (size_t L = 0; L < L_.size(); ++L) {
    const LayerDev& s = L_[L];
    if (!s.pool) continue;
    const uint64_t b = uint64_t(uintptr_t(s.pool)), n = uint64_t(place_.pool_slots(int(L))) * s.stride;
    if (addr >= b && addr < b + n) return Region{1, int(L), addr - b};
  }
  const auto& rc = place_.ring_classes();
  for (size_t k = 0; k < rc.size(); ++k) {
    const uint64_t b = uint64_t(uintptr_t(ring_base_[k]));
    if (addr >= b && addr < b + rc[k].stride * rc[k].count) return Region{2, int(k), addr - b};
  }
  return r;
}

// ---- counters, the stats-v1 document and the snapshot ---------------------------------------------------------------

ss_layer_stats HostCtx::total() const {
  ss_layer_stats t{};
  for (const auto& s : place_.stats()) add_stats(t, s);
  return t;
}

void HostCtx::stats_reset() {
  place_.reset_stats();
  ra_st_ = RaCounts{};
  if (!place_.in_forward()) publish();
}

void HostCtx::publish() {
  if (!snap_armed_.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(snap_mu_);
  snap_.layers = place_.stats();
  snap_.x = place_.exclusive_stats();
  snap_.ra = ra_st_;
  snap_.forwards = place_.forwards();
  ++snap_.seq;
}

bool HostCtx::snapshot(ss_layer_stats* total, ss_snapshot_info* info) const {
  snap_armed_.store(true, std::memory_order_relaxed);
  ss_layer_stats t{};
  ss_snapshot_info i{};
  {
    std::lock_guard<std::mutex> lk(snap_mu_);
    if (snap_.seq == 0) return false;
    for (const ss_layer_stats& l : snap_.layers) add_stats(t, l);
    i.sequence = snap_.seq;
    i.forwards = snap_.forwards;
    if (ra_on()) {
      const RaCounts& r = snap_.ra;
      i.readahead_requested = r.requested;
      i.readahead_read = r.read;
      i.readahead_landed = r.landed;
      i.readahead_unused = r.unused;
      i.readahead_failed = r.failed;
      i.readahead_fallback = r.fallback;
      i.readahead_bytes = r.bytes;
    }
    if (place_.exclusive()) {
      const ss_exclusive_stats& x = snap_.x;
      i.exclusive_writebacks = x.writebacks;
      i.exclusive_writeback_bytes = x.writeback_bytes;
      i.exclusive_deferred = x.deferred;
      i.exclusive_promoted = x.promoted;
      i.exclusive_free_blocks = x.free_blocks;
      i.exclusive_min_free_blocks = x.min_free_blocks;
      i.exclusive_rereads = x.rereads;
      i.exclusive_discards = x.discards;
    }
  }
  if (ra_on()) {  // (fixed at open)
    i.flags |= SS_SNAPSHOT_READAHEAD;
    i.readahead_buffers = ra_buf_.size();
    i.readahead_buffer_bytes = place_.ra_bytes();
  }
  if (place_.exclusive()) {
    i.flags |= SS_SNAPSHOT_EXCLUSIVE;
    i.exclusive_blocks = excl_blocks_;
  }
  i.struct_size = uint32_t(sizeof i);
  if (total) *total = t;
  if (info) *info = i;
  return true;
}

bool HostCtx::snapshot_json(Json* out) const {
  snap_armed_.store(true, std::memory_order_relaxed);
  Published p;
  {
    std::lock_guard<std::mutex> lk(snap_mu_);
    if (snap_.seq == 0) return false;
    p = snap_;
  }
  *out = format_stats(p.forwards, p.layers.data(), p.x, p.ra);
  return true;
}

Json HostCtx::stats_json() const {
  return format_stats(place_.forwards(), place_.stats().data(), place_.exclusive_stats(), ra_st_);
}

// The stats-v1 document (its keys and layout: reference src/stream_ctx.cpp:1826-1885).
Json HostCtx::format_stats(uint64_t forwards, const ss_layer_stats* layers, const ss_exclusive_stats& x,
                           const RaCounts& ra) const {
  Json doc = Json::object();
  doc["schema"] = Json::string("strix-stream/stats-v1");
  doc["backend"] = Json::string("hip");
  doc["forwards"] = Json::number(forwards);
  Json direct = Json::array();
  for (const auto& f : files_) direct.push(Json::boolean(f->direct()));
  doc["sources_direct"] = direct;
  ss_layer_stats sum{};
  Json per_layer = Json::array();
  for (int L = 0; L < n_layers(); ++L) {
    add_stats(sum, layers[L]);
    per_layer.push(stats_object(layers[L]));
  }
  doc["total"] = stats_object(sum);
  doc["layers"] = per_layer;
  if (ra_on()) {  // (readahead_units 0: no such object)
    Json r = Json::object();
    const std::pair<const char*, uint64_t> fields[] = {
        {"buffers", ra_buf_.size()}, {"buffer_bytes", place_.ra_bytes()}, {"requested", ra.requested},
        {"read", ra.read},           {"landed", ra.landed},               {"unused", ra.unused},
        {"failed", ra.failed},       {"fallback", ra.fallback},           {"bytes", ra.bytes}};
    for (const auto& f : fields) r[f.first] = Json::number(f.second);
    doc["readahead"] = r;
  }
  if (place_.exclusive()) {
    Json e = Json::object();
    const std::pair<const char*, uint64_t> fields[] = {
        {"writebacks", x.writebacks}, {"writeback_bytes", x.writeback_bytes}, {"discards", x.discards},
        {"deferred", x.deferred},     {"rereads", x.rereads},                 {"promoted", x.promoted},
        {"free_blocks", x.free_blocks}, {"min_free_blocks", x.min_free_blocks}, {"blocks", excl_blocks_}};
    for (const auto& f : fields) e[f.first] = Json::number(f.second);
    doc["exclusive"] = e;
  }
  return doc;
}

}  // namespace tsa
