#include "host_ctx.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>

#include "stats_json.hpp"
#include "tsa_device.hpp"

namespace tsa {
namespace {

constexpr uint64_t kHostAlign = 4096;
constexpr uint64_t kDefaultSegBytes = 8 * 1024;  // device verify checkpoints: 32 B per segment (0.4 % of a unit)
constexpr size_t kVerifyBatch = 32;                // landed units per device verify launch

bool resident_tier(uint8_t t) { return t == SS_TIER_RESIDENT || t == SS_TIER_RESIDENT_BACKED; }

uint64_t now_ns() {
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count());
}

void add(ss_layer_stats& a, const ss_layer_stats& b) {
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

// Checkpoints of one contiguous unit while its bytes stream through the host hasher: the four accumulators at every
// multiple of `seg` below the unit's whole-stripe span (tsa.h layout for one extent).
class SegHasher {
 public:
  SegHasher(uint64_t unit_bytes, uint64_t seg, uint64_t* states)
      : seg_(seg), span_(unit_bytes / 32 * 32), states_(states) {
    nseg_ = seg ? (span_ + seg - 1) / seg : 0;
    if (seg && nseg_ == 0) nseg_ = 1;
  }
  void feed(const void* p, uint64_t n) {
    const char* c = static_cast<const char*>(p);
    while (n) {
      mark();
      uint64_t take = n;
      if (states_ && k_ < nseg_) take = std::min(take, k_ * seg_ - pos_);
      if (take == 0) take = n;  // (past the last checkpoint)
      h_.update(c, size_t(take));
      pos_ += take;
      c += take;
      n -= take;
    }
    mark();
  }
  uint64_t digest() const { return h_.digest(); }

 private:
  void mark() {
    while (states_ && k_ < nseg_ && pos_ == k_ * seg_) {
      std::memcpy(states_ + 4 * k_, h_.acc(), 32);
      ++k_;
    }
  }
  Xxh64 h_;
  uint64_t seg_, span_, nseg_ = 0, k_ = 0, pos_ = 0;
  uint64_t* states_;
};

}  // namespace

HostCtx::HostCtx(const Desc& d, const ss_budget& b, const Plan& p, const ss_options& o) : d_(d), plan_(p), o_(o) {
  (void)b;
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
  require(int64_t(plan_.tier.size()) == d_.total_units, SS_E_INVALID, "open: plan does not match the descriptor");
  excl_ = plan_.budget.tier_mode == SS_TIER_MODE_EXCLUSIVE;
  require(!(excl_ && !o_.fill_residents), SS_E_INVALID, "open: the exclusive tier mode needs fill_residents = 1");
  require(!(excl_ && o_.exclusive_discard && d_.tiers == Tiers::Pinned), SS_E_INVALID,
          "open: exclusive_discard needs a descriptor whose tiers allow disk (tiers = \"pinned\" refuses it)");
  require(o_.readahead_units == 0, SS_E_UNSUPPORTED,
          "open: host read-ahead (readahead_units) is not part of this library's serve path");
  require(o_.verify_hash >= 0 && o_.verify_hash <= 2, SS_E_INVALID, "open: verify_hash must be 0, 1 or 2");
  dev_ = std::make_unique<HipDevice>(o_.device);
  copy_ = dev_->stream_create_dedicated();
  copy2_ = dev_->stream_create_dedicated();
  join_ev_ = dev_->event_create();
  if (!o_.reader_threads) o_.reader_threads = 2;
  if (!o_.staging_buffers) o_.staging_buffers = 4;
  if (!o_.staging_bytes) o_.staging_bytes = uint64_t(256) << 20;
  if (!o_.copy_piece_bytes) o_.copy_piece_bytes = uint64_t(64) << 20;
  uint64_t max_align = kHostAlign;
  for (const auto& s : d_.sources) max_align = std::max(max_align, s.align);
  require(o_.staging_bytes >= 4 * max_align, SS_E_INVALID, "open: staging_bytes must be >= 4 x the source alignment");
  o_.staging_bytes = round_up(o_.staging_bytes, max_align);
  for (const auto& s : d_.sources) files_.push_back(std::make_unique<SourceFile>(s.path, o_.direct_io != 0));

  for (uint32_t i = 0; i < o_.staging_buffers; ++i) {
    Staging s;
    s.host = dev_->alloc_pinned(o_.staging_bytes, "staging buffer");
    staging_.push_back(s);
    staging_.back().ev = dev_->event_create();
    staging_free_.push_back(i);
  }

  pinned_of_.assign(size_t(d_.total_units), nullptr);
  {
    const PinnedLayout pl = pinned_layout(d_, plan_.tier);
    for (uint64_t bytes : pl.chunk_bytes) pinned_chunks_.push_back(dev_->alloc_pinned(bytes, "pinned tier"));
    for (int64_t g = 0; g < d_.total_units; ++g)
      if (pl.chunk_of[size_t(g)] >= 0)
        pinned_of_[size_t(g)] = at(pinned_chunks_[size_t(pl.chunk_of[size_t(g)])], pl.offset_of[size_t(g)]);
  }

  if (excl_) {
    wb_ = dev_->stream_create_dedicated();
    blocks_ev_ = dev_->event_create();
    wb_mark_ev_ = dev_->event_create();
    wb_pending_.assign(size_t(d_.total_units), nullptr);
    for (const SpareClass& c : plan_.spares) block_bytes_.push_back(c.block_bytes);
    free_blocks_.resize(block_bytes_.size());
    layer_class_.assign(d_.layers.size(), -1);
    std::vector<uint64_t> class_total(block_bytes_.size(), 0);
    for (size_t L = 0; L < d_.layers.size(); ++L) {
      const Layer& l = d_.layers[L];
      if (!l.streamable || !l.n_units) continue;
      const auto it = std::find(block_bytes_.begin(), block_bytes_.end(), host_stride(l.unit_bytes));
      require(it != block_bytes_.end(), SS_E_INVALID, "open: exclusive plan without a block class (internal)");
      layer_class_[L] = int(it - block_bytes_.begin());
      for (int u = 0; u < l.n_units; ++u)
        if (pinned_of_[size_t(gidx(int(L), u))]) ++class_total[size_t(layer_class_[L])];
    }
    uint64_t free_total = 0;
    for (size_t k = 0; k < plan_.spares.size(); ++k) {
      const uint64_t bytes = plan_.spares[k].block_bytes;
      const uint64_t per_chunk = std::max<uint64_t>(1, kPinnedChunk / bytes);
      class_total[k] += plan_.spares[k].blocks;
      free_blocks_[k].reserve(size_t(class_total[k]));
      std::vector<void*> blocks;
      for (uint64_t left = plan_.spares[k].blocks; left > 0;) {
        const uint64_t n = std::min(per_chunk, left);
        void* chunk = dev_->alloc_pinned(n * bytes, "spare blocks");
        spare_chunks_.push_back(chunk);
        for (uint64_t i = 0; i < n; ++i) blocks.push_back(at(chunk, i * bytes));
        left -= n;
      }
      for (size_t i = blocks.size(); i-- > 0;) free_blocks_[k].push_back(blocks[i]);  // lowest address on top
      spares_of_.push_back(plan_.spares[k].blocks);
      free_total += plan_.spares[k].blocks;
      n_blocks_ += class_total[k];
    }
    xst_.free_blocks = xst_.min_free_blocks = free_total;
    wb_units_.reserve(size_t(d_.total_units));
  }

  L_.resize(d_.layers.size());
  for (size_t L = 0; L < d_.layers.size(); ++L) {
    const Layer& l = d_.layers[L];
    LayerState& s = L_[L];
    s.release_ev = dev_->event_create();
    s.ready_ev = dev_->event_create();
    s.ids_ev = dev_->event_create();
    if (l.n_units == 0) continue;
    int planned = 0;
    for (int u = 0; u < l.n_units; ++u)
      if (resident_tier(plan_.tier[size_t(gidx(int(L), u))])) ++planned;
    const int cap = l.streamable ? std::min(l.n_units, planned + int(plan_.dynamic_slots_per_layer)) : l.n_units;
    s.rs = std::make_unique<Residency>(l.n_units, cap, o_.policy, o_.score_window);
    if (cap) s.pool = dev_->alloc_device(uint64_t(cap) * d_.unit_stride(int(L)), "resident pool");
    for (int v = 0; v < 2; ++v) {
      s.table_host[v] = static_cast<uint64_t*>(dev_->alloc_pinned(8 * uint64_t(l.n_units), "unit table"));
      std::memset(s.table_host[v], 0, 8 * size_t(l.n_units));
      s.table_dev[v] = dev_->alloc_device(8 * uint64_t(l.n_units), "unit table");
      s.table_ev[v] = dev_->event_create();
    }
    s.loc.assign(size_t(l.n_units), None);
    s.slot.assign(size_t(l.n_units), -1);
    s.job.assign(size_t(l.n_units), nullptr);
    s.spec_unclaimed.assign(size_t(l.n_units), 0);
    s.count.assign(size_t(l.n_units), 0);
  }

  for (const RingClass& rc : plan_.rings) {
    if (!rc.slots) continue;
    void* base = dev_->alloc_device(rc.stride * rc.slots, "stream ring");
    ring_classes_.push_back({rc.stride, ring_.size(), rc.slots, 0, base});
    for (uint32_t i = 0; i < rc.slots; ++i) {
      RingSlot slot;
      slot.dev = at(base, rc.stride * i);
      slot.stride = rc.stride;
      ring_.push_back(slot);
    }
  }
  ring_owner_ev_.assign(ring_.size(), nullptr);
  stats_.assign(d_.layers.size(), ss_layer_stats{});
  fwd_stats_.assign(d_.layers.size(), ss_layer_stats{});

  if (o_.verify_hash == 2) {  // device verify of every landed unit: checkpoint tables and the per-forward launch slots
    dverify_ = true;
    seg_bytes_ = kDefaultSegBytes;
    checks_.assign(size_t(d_.total_units), UnitCheck{});
    vcap_ = size_t(d_.total_units) + 8;
    vtable_host_ = static_cast<tsa_verify_unit*>(dev_->alloc_pinned(vcap_ * sizeof(tsa_verify_unit), "verify table"));
    vfail_host_ = static_cast<uint32_t*>(dev_->alloc_pinned(vcap_ * 4, "verify results"));
    vtable_dev_ = dev_->alloc_device(vcap_ * sizeof(tsa_verify_unit), "verify table");
    vfail_dev_ = static_cast<uint32_t*>(dev_->alloc_device(vcap_ * 4, "verify results"));
    ventry_flush_.assign(vcap_, 0);
    hip_check(hipMemsetAsync(vfail_dev_, 0, vcap_ * 4, copy_), "hipMemsetAsync");
    vdone_ev_ = dev_->event_create();
    vready_ev_ = dev_->event_create();
    vready2_ev_ = dev_->event_create();
    vstream_ = dev_->stream_create_dedicated();
    stream_sync(copy_);  // (the zeroed results before any check on the verify stream)
  }

  for (uint32_t i = 0; i < o_.reader_threads; ++i) workers_.emplace_back([this] { worker(); });

  // Fill: the pinned tier first (host), then residents (from their pinned copy if any, else the file).
  std::vector<HostJobPtr> fill;
  for (size_t L = 0; L < d_.layers.size(); ++L)
    for (int u = 0; u < d_.layers[L].n_units; ++u) {
      const void* pa = pinned_of_[size_t(gidx(int(L), u))];
      if (!pa) continue;
      auto j = std::make_shared<HostJob>();
      j->layer = int(L);
      j->unit = u;
      j->dst = const_cast<void*>(pa);
      j->host_dst = true;
      fill.push_back(j);
      submit(j);
    }
  for (const auto& j : fill) wait_job(*j);
  fill.clear();
  for (size_t L = 0; L < d_.layers.size(); ++L) {
    const Layer& l = d_.layers[L];
    LayerState& s = L_[L];
    if (!s.rs) continue;
    for (int u = 0; u < l.n_units; ++u) {
      if (l.streamable && !resident_tier(plan_.tier[size_t(gidx(int(L), u))])) continue;
      const int slot = s.rs->place(u, !l.streamable || o_.pin_planned != 0);
      require(slot >= 0, SS_E_CAPACITY, "open: resident pool full (internal)");
      if (o_.fill_residents) {
        HostJobPtr j = make_job(int(L), u, at(s.pool, uint64_t(slot) * d_.unit_stride(int(L))), false);
        fill.push_back(j);
        submit(j);
      }
    }
  }
  for (const auto& j : fill) wait_job(*j);
  for (const auto& j : fill)
    if (j->done_ev) ev_pool_.push_back(j->done_ev);
  stream_sync(copy_);
  stream_sync(copy2_);
  if (dverify_) collect_verify();  // the residents' device check (one batch at open)
}

void HostCtx::cleanup() noexcept {
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    stop_ = true;
  }
  q_cv_.notify_all();
  for (auto& t : workers_) t.join();
  workers_.clear();
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
  for (const auto& r : ring_classes_) dev_->free_device(r.base);
  for (void* c : pinned_chunks_) dev_->free_pinned(c);
  for (void* c : spare_chunks_) dev_->free_pinned(c);
  for (auto& s : staging_) {
    dev_->free_pinned(s.host);
    dev_->event_destroy(s.ev);
  }
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
  dev_->event_destroy(vready2_ev_);
  for (hipEvent_t e : vflush_ev_) dev_->event_destroy(e);
  if (vstream_) dev_->stream_destroy(vstream_);
  dev_->event_destroy(join_ev_);
  dev_->stream_destroy(copy_);
  dev_->stream_destroy(copy2_);
  dev_->stream_destroy(wb_);
  L_.clear();
  dev_.reset();
}

// ---- reader threads -------------------------------------------------------------------------------------------------

void HostCtx::worker() {
  try {
    dev_->bind();
  } catch (...) {
  }
  while (true) {
    HostJobPtr j;
    {
      std::unique_lock<std::mutex> lk(q_mu_);
      // demands first; a speculative read only while no demand waits and at most one runs
      q_cv_.wait(lk, [&] { return stop_ || !demand_q_.empty() || (!spec_q_.empty() && demand_running_ <= 1); });
      if (stop_ && demand_q_.empty() && spec_q_.empty()) return;
      if (!demand_q_.empty()) {
        j = demand_q_.front();
        demand_q_.pop_front();
        ++demand_running_;
        j->ran_as_demand = true;
      } else if (!spec_q_.empty() && demand_running_ <= 1) {
        j = spec_q_.front();
        spec_q_.pop_front();
        j->ran_as_demand = false;
      } else {
        continue;
      }
      int expect = HostJob::Queued;
      if (!j->state.compare_exchange_strong(expect, HostJob::Running)) {
        if (j->ran_as_demand) --demand_running_;
        done_cv_.notify_all();
        continue;  // cancelled while queued
      }
    }
    int final_state = HostJob::Done;
    try {
      run_job(*j);
    } catch (const Error& e) {
      j->err_status = e.status();
      j->err = e.what();
      final_state = HostJob::Failed;
    } catch (const std::bad_alloc&) {
      j->err_status = SS_E_NOMEM;
      final_state = HostJob::Failed;
    } catch (const std::exception& e) {
      j->err_status = SS_E_BACKEND;
      j->err = e.what();
      final_state = HostJob::Failed;
    }
    {
      std::lock_guard<std::mutex> lk(q_mu_);
      j->state.store(final_state);
      if (j->ran_as_demand) --demand_running_;
    }
    done_cv_.notify_all();
    q_cv_.notify_all();
  }
}

void HostCtx::submit(const HostJobPtr& j) {
  if (j->from_pinned && !j->host_dst) {
    // pinned tier -> HBM: issued now on the copy stream (an SDMA queue), no host wait and no reader thread
    const uint64_t n = d_.layers[size_t(j->layer)].unit_bytes;
    try {
      std::lock_guard<std::mutex> lk(copy_mu_);
      const hipStream_t cs = next_copy_stream();
      wait_slot_check(cs, j->dst);
      stream_wait(cs, j->dst_release_ev);
      stream_wait(cs, j->dst_wb_ev);
      stream_wait(cs, j->src_wait_ev);
      for (uint64_t off = 0; off < n; off += o_.copy_piece_bytes)
        copy_h2d(at(j->dst, off), at(j->host_src, off), std::min<uint64_t>(o_.copy_piece_bytes, n - off), cs);
      ev_record(j->done_ev, cs);
      if (dverify_) verify_landed(*j);
    } catch (const Error& e) {
      fail_job(*j, e.status(), e.what());
      throw;
    }
    j->state.store(HostJob::Done);
    return;
  }
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    (j->spec ? spec_q_ : demand_q_).push_back(j);
  }
  q_cv_.notify_all();
}

void HostCtx::fail_job(HostJob& j, ss_status st, const char* msg) noexcept {
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    j.err_status = st;
    try {
      j.err = msg;
    } catch (...) {
    }
    j.state.store(HostJob::Failed);
  }
  done_cv_.notify_all();
}

void HostCtx::promote(const HostJobPtr& j) {
  std::lock_guard<std::mutex> lk(q_mu_);
  if (j->state.load() != HostJob::Queued || !j->spec) return;
  const auto it = std::find(spec_q_.begin(), spec_q_.end(), j);
  if (it == spec_q_.end()) return;
  spec_q_.erase(it);
  demand_q_.push_front(j);
  j->spec = false;
  q_cv_.notify_one();
}

void HostCtx::wait_job(HostJob& j) {
  wait_job_quiet(j);
  if (j.state.load() == HostJob::Failed) fail(j.err_status, j.err);
}

void HostCtx::wait_job_quiet(HostJob& j) {
  std::unique_lock<std::mutex> lk(q_mu_);
  done_cv_.wait(lk, [&] {
    const int s = j.state.load();
    return s == HostJob::Done || s == HostJob::Cancelled || s == HostJob::Failed;
  });
}

void HostCtx::run_job(HostJob& j) {
  const Layer& l = d_.layers[size_t(j.layer)];
  const bool hash = o_.verify_hash && !l.hash.empty();
  if (j.host_dst) {
    uint64_t digest = 0;
    read_unit_host(j.layer, j.unit, j.dst, hash, &digest);
    if (hash && digest != l.hash[size_t(j.unit)])
      fail(SS_E_HASH, "unit (" + std::to_string(j.layer) + ", " + std::to_string(j.unit) +
                          ") bytes differ from the descriptor hash");
    return;
  }
  read_unit_device(j);
}

void HostCtx::read_unit_host(int layer, int unit, void* dst, bool hash, uint64_t* digest) {
  const Layer& l = d_.layers[size_t(layer)];
  const int64_t g = gidx(layer, unit);
  uint64_t* states = nullptr;
  std::vector<uint64_t> st;
  if (dverify_ && hash) {
    st.assign(4 * std::max<uint64_t>(1, (l.unit_bytes / 32 * 32 + seg_bytes_ - 1) / seg_bytes_), 0);
    states = st.data();
  }
  SegHasher h(l.unit_bytes, seg_bytes_, states);
  uint64_t pos = 0;
  for (const Part& part : l.parts) {
    const SourceFile& f = *files_[size_t(part.source)];
    const uint64_t al = std::max<uint64_t>(d_.sources[size_t(part.source)].align, 512);
    const uint64_t F = part.offset + uint64_t(unit) * part.stride;
    char* out = at(dst, pos);
    require(F + part.bytes <= f.size(), SS_E_IO,
            "unit (" + std::to_string(layer) + ", " + std::to_string(unit) + ") part " + part.name +
                " is past the end of its source");
    const bool in_place = !f.direct() || (F % al == 0 && part.bytes % al == 0 && uintptr_t(out) % al == 0);
    if (in_place) {
      f.pread_all(out, part.bytes, F);
    } else {  // an aligned covering range through a staging buffer
      const uint64_t cap = (o_.staging_bytes - 2 * al) / al * al;
      for (uint64_t c = 0; c < part.bytes;) {
        const uint64_t len = std::min(cap, part.bytes - c);
        const uint64_t a0 = (F + c) / al * al, delta = F + c - a0, a1 = round_up(F + c + len, al);
        size_t i;
        {
          std::unique_lock<std::mutex> lk(staging_mu_);
          staging_cv_.wait(lk, [&] { return !staging_free_.empty(); });
          i = staging_free_.back();
          staging_free_.pop_back();
        }
        try {
          ev_sync(staging_[i].ev);
          require(f.pread_some(staging_[i].host, a1 - a0, a0) >= delta + len, SS_E_IO, "short read");
          std::memcpy(out + c, at(staging_[i].host, delta), size_t(len));
        } catch (...) {
          {
            std::lock_guard<std::mutex> lk(staging_mu_);
            staging_free_.push_back(i);
          }
          staging_cv_.notify_one();
          throw;
        }
        {
          std::lock_guard<std::mutex> lk(staging_mu_);
          staging_free_.push_back(i);
        }
        staging_cv_.notify_one();
        c += len;
      }
    }
    if (hash) h.feed(out, part.bytes);
    pos += part.bytes;
  }
  if (digest) *digest = h.digest();
  if (states && h.digest() == l.hash[size_t(unit)] && !checks_[size_t(g)].states_dev) {
    // the checkpoints are certified by the descriptor hash: kept on the device for every later landing of the unit
    UnitCheck c;
    c.n_states = st.size() / 4;
    c.states_dev = static_cast<uint64_t*>(dev_->alloc_device(st.size() * 8, "verify checkpoints"));
    hip_check(hipMemcpy(c.states_dev, st.data(), st.size() * 8, hipMemcpyHostToDevice), "hipMemcpy (checkpoints)");
    std::lock_guard<std::mutex> lk(copy_mu_);
    checks_[size_t(g)] = c;
  }
}

void HostCtx::read_unit_device(HostJob& j) {
  const Layer& l = d_.layers[size_t(j.layer)];
  const bool hash = o_.verify_hash && !l.hash.empty();
  const int64_t g = gidx(j.layer, j.unit);
  std::vector<uint64_t> st;
  uint64_t* states = nullptr;
  if (dverify_ && hash) {
    st.assign(4 * std::max<uint64_t>(1, (l.unit_bytes / 32 * 32 + seg_bytes_ - 1) / seg_bytes_), 0);
    states = st.data();
  }
  SegHasher h(l.unit_bytes, seg_bytes_, states);
  uint64_t pos = 0;
  bool waited = false;
  for (const Part& part : l.parts) {
    const SourceFile& f = *files_[size_t(part.source)];
    const uint64_t al = f.direct() ? std::max<uint64_t>(d_.sources[size_t(part.source)].align, 512) : 1;
    const uint64_t F = part.offset + uint64_t(j.unit) * part.stride;
    require(F + part.bytes <= f.size(), SS_E_IO,
            "unit (" + std::to_string(j.layer) + ", " + std::to_string(j.unit) + ") part " + part.name +
                " is past the end of its source");
    const uint64_t cap = (o_.staging_bytes - 2 * std::max<uint64_t>(al, kHostAlign)) / kHostAlign * kHostAlign;
    for (uint64_t c = 0; c < part.bytes;) {
      const uint64_t len = std::min(cap, part.bytes - c);
      const uint64_t a0 = (F + c) / al * al, delta = F + c - a0, a1 = round_up(F + c + len, al);
      size_t i;
      {
        std::unique_lock<std::mutex> lk(staging_mu_);
        staging_cv_.wait(lk, [&] { return !staging_free_.empty(); });
        i = staging_free_.back();
        staging_free_.pop_back();
      }
      auto give_back = [&] {
        {
          std::lock_guard<std::mutex> lk(staging_mu_);
          staging_free_.push_back(i);
        }
        staging_cv_.notify_one();
      };
      try {
        ev_sync(staging_[i].ev);  // the buffer's previous H2D has completed
        require(f.pread_some(staging_[i].host, a1 - a0, a0) >= delta + len, SS_E_IO, "short read");
        const char* src = at(staging_[i].host, delta);
        if (hash) h.feed(src, len);
        std::lock_guard<std::mutex> lk(copy_mu_);
        if (!waited) {
          wait_slot_check(copy_, j.dst);
          stream_wait(copy_, j.dst_release_ev);
          stream_wait(copy_, j.dst_wb_ev);
          waited = true;
        }
        copy_h2d(at(j.dst, pos + c), src, len, copy_);
        ev_record(staging_[i].ev, copy_);
      } catch (...) {
        give_back();
        throw;
      }
      give_back();
      c += len;
    }
    pos += part.bytes;
  }
  if (hash && h.digest() != l.hash[size_t(j.unit)])
    fail(SS_E_HASH, "unit (" + std::to_string(j.layer) + ", " + std::to_string(j.unit) +
                        ") bytes differ from the descriptor hash");
  std::lock_guard<std::mutex> lk(copy_mu_);
  if (states && !checks_[size_t(g)].states_dev) {
    UnitCheck c;
    c.n_states = st.size() / 4;
    c.states_dev = static_cast<uint64_t*>(dev_->alloc_device(st.size() * 8, "verify checkpoints"));
    hip_check(hipMemcpy(c.states_dev, st.data(), st.size() * 8, hipMemcpyHostToDevice), "hipMemcpy (checkpoints)");
    checks_[size_t(g)] = c;
  }
  ev_record(j.done_ev, copy_);
  if (dverify_) verify_landed(j);
}

// verify_hash = 2: the checkpoint-parallel check of the unit just landed at j.dst joins the pending batch (copy_mu_
// held by the caller: its copies are on the copy stream already). A batch of kVerifyBatch units is launched at once on
// the verify stream, behind the copy stream's work so far; the rest at ss_end, where the results are collected. One
// launch per unit on the copy stream made every next copy wait for the check (a 9 MiB unit: 1,152 quads, 134 us).
void HostCtx::verify_landed(const HostJob& j) {
  const Layer& l = d_.layers[size_t(j.layer)];
  const UnitCheck& c = checks_[size_t(gidx(j.layer, j.unit))];
  if (l.hash.empty() || !c.states_dev) return;  // (no descriptor hash: nothing to verify against)
  require(vused_ < vcap_, SS_E_BACKEND, "device verify: launch table full (internal)");
  const size_t i = vused_++;
  tsa_verify_unit& v = vtable_host_[i];
  std::memset(&v, 0, sizeof v);
  v.ext[0].ptr = j.dst;
  v.ext[0].bytes = l.unit_bytes;
  v.n_ext = 1;
  v.seg_first = c.n_states;  // (its checkpoint count until the flush turns it into the launch's prefix sum)
  v.states = c.states_dev;
  v.digest = l.hash[size_t(j.unit)];
  v.total = l.unit_bytes;
  vunits_.push_back({j.layer, j.unit});
  vdst_[j.dst] = i;
  if (vused_ - vflushed_ >= kVerifyBatch) flush_verify();
}

void HostCtx::wait_slot_check(hipStream_t s, const void* dst) {
  const auto it = vdst_.find(dst);
  if (it == vdst_.end()) return;
  const size_t i = it->second;
  if (i >= vflushed_) flush_verify();  // (its batch was still pending: launch it now)
  stream_wait(s, vflush_ev_[ventry_flush_[i]]);
  vdst_.erase(it);
}

void HostCtx::join_copies() {
  ev_record(join_ev_, copy2_);
  stream_wait(copy_, join_ev_);
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
  ev_record(vready_ev_, copy_);  // (the verify stream follows both copy streams; neither waits for the other)
  ev_record(vready2_ev_, copy2_);
  stream_wait(vstream_, vready_ev_);
  stream_wait(vstream_, vready2_ev_);
  tsa_verify_unit* vd = static_cast<tsa_verify_unit*>(vtable_dev_) + vflushed_;
  copy_h2d(vd, vtable_host_ + vflushed_, n * sizeof(tsa_verify_unit), vstream_);
  hip_check(hipError_t(launch_verify(vd, uint32_t(n), segs, seg_bytes_, vfail_dev_ + vflushed_, vstream_)),
            "device verify launch");
  if (vflushes_ == vflush_ev_.size()) vflush_ev_.push_back(dev_->event_create());
  ev_record(vflush_ev_[vflushes_], vstream_);
  for (size_t i = vflushed_; i < vused_; ++i) ventry_flush_[i] = vflushes_;
  ++vflushes_;
  vflushed_ = vused_;
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
    ev_record(vdone_ev_, vstream_);
  }
  ev_sync(vdone_ev_);
  std::string bad;
  uint64_t nbad = 0;
  std::vector<std::pair<int, int>> units;
  {
    std::lock_guard<std::mutex> lk(copy_mu_);
    units.swap(vunits_);
    vused_ = vflushed_ = 0;
    vdst_.clear();  // (every launch has completed: ev_sync above)
    vflushes_ = 0;
  }
  for (size_t i = 0; i < n; ++i)
    if (vfail_host_[i]) {
      ++nbad;
      if (bad.empty())
        bad = "(" + std::to_string(units[i].first) + ", " + std::to_string(units[i].second) + ")";
    }
  verify_fail_total_ += nbad;
  require(nbad == 0, SS_E_HASH,
          "device verify: " + std::to_string(nbad) + " landed unit(s) differ from the descriptor hash in HBM, first " +
              bad);
}

// ---- placement ------------------------------------------------------------------------------------------------------

HostJobPtr HostCtx::make_job(int layer, int unit, void* dst, bool spec) {
  auto j = std::make_shared<HostJob>();
  j->layer = layer;
  j->unit = unit;
  j->spec = spec;
  j->dst = dst;
  j->dst_release_ev = L_[size_t(layer)].release_ev;
  j->host_src = pinned_of_[size_t(gidx(layer, unit))];
  j->from_pinned = j->host_src != nullptr;
  if (excl_ && j->from_pinned) {
    j->src_wait_ev = wb_pending_[size_t(gidx(layer, unit))];
    if (j->src_wait_ev) ++xst_.rereads;
  }
  j->done_ev = pooled_event();
  return j;
}

void HostCtx::fetch_into_persistent(int layer, int unit, int slot, bool spec, hipEvent_t dst_wb_ev) {
  LayerState& s = L_[size_t(layer)];
  HostJobPtr j = make_job(layer, unit, at(s.pool, uint64_t(slot) * d_.unit_stride(layer)), spec);
  j->dst_wb_ev = dst_wb_ev;
  fwd_jobs_.push_back(j);
  s.loc[size_t(unit)] = Persistent;
  s.slot[size_t(unit)] = slot;
  s.job[size_t(unit)] = j;
  (j->from_pinned ? fwd_stats_[size_t(layer)].bytes_pinned : fwd_stats_[size_t(layer)].bytes_disk) +=
      d_.layers[size_t(layer)].unit_bytes;
  submit(j);
}

uint64_t HostCtx::writeback_blocks(int layer, bool speculative) const {
  const int cls = block_class(layer);
  if (cls < 0) return 0;
  uint64_t f = free_blocks_[size_t(cls)].size();
  if (speculative) {  // a guess leaves half of the spares to demands
    const uint64_t reserve = (spares_of_[size_t(cls)] + 1) / 2;
    f = f > reserve ? f - reserve : 0;
  }
  return f;
}

int HostCtx::eviction_cap(int layer, bool speculative) const {
  if (!excl_) return -1;
  if (block_class(layer) < 0) return 0;
  if (o_.exclusive_discard && !speculative) return -1;
  return int(std::min<uint64_t>(writeback_blocks(layer, speculative), uint64_t(INT32_MAX)));
}

// Exclusive mode: victims leave their slots for free blocks (D2H on the write-back stream) before anything is written
// into those slots; past the free blocks (exclusive_discard) they are discarded to their files.
hipEvent_t HostCtx::write_back(int layer, const Admission& a, bool speculative, size_t* n_wb) {
  const LayerState& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  const int cls = block_class(layer);
  const uint64_t room = writeback_blocks(layer, speculative);
  if (cls < 0 || (!o_.exclusive_discard && room < a.evicted.size()))
    fail(SS_E_BACKEND, "exclusive: more victims than free blocks (internal)");
  const size_t nw = size_t(std::min<uint64_t>(room, a.evicted.size()));
  *n_wb = nw;
  for (size_t i = 0; i < a.evicted.size(); ++i)
    if (pinned_of_[size_t(gidx(layer, a.evicted[i]))] != nullptr)
      fail(SS_E_BACKEND, "exclusive: an evicted resident still owns a block (internal)");
  xst_.discards += a.evicted.size() - nw;
  if (!nw) return nullptr;
  if (wb_gate_) {  // blocks freed by earlier forwards: their last H2D reader is before blocks_ev_ on the copy stream
    stream_wait(wb_, blocks_ev_);
    wb_gate_ = false;
  }
  hipEvent_t ev = pooled_event();
  wb_evs_.push_back(ev);
  for (size_t i = 0; i < nw; ++i) {
    const int64_t g = gidx(layer, a.evicted[i]);
    void* b = free_blocks_[size_t(cls)].back();
    free_blocks_[size_t(cls)].pop_back();
    pinned_of_[size_t(g)] = b;
    copy_d2h(b, at(s.pool, uint64_t(a.evicted_slot[i]) * d_.unit_stride(layer)), l.unit_bytes, wb_);
    ++xst_.writebacks;
    xst_.writeback_bytes += l.unit_bytes;
  }
  ev_record(ev, wb_);
  for (size_t i = 0; i < nw; ++i) {
    const int64_t g = gidx(layer, a.evicted[i]);
    wb_pending_[size_t(g)] = ev;
    wb_units_.push_back(g);
  }
  return ev;
}

void HostCtx::fetch_admitted(int layer, const Admission& a, bool spec) {
  size_t n_wb = 0;
  hipEvent_t ev = excl_ && !a.evicted.empty() ? write_back(layer, a, spec, &n_wb) : nullptr;
  for (size_t k = 0; k < a.admitted.size(); ++k) {
    hipEvent_t wait = nullptr;  // a write into a written-back victim's slot waits for the write-back
    if (ev)
      for (size_t i = 0; i < n_wb && !wait; ++i)
        if (a.evicted_slot[i] == a.admitted_slot[k]) wait = ev;
    fetch_into_persistent(layer, a.admitted[k], a.admitted_slot[k], spec, wait);
  }
}

void HostCtx::free_block(int layer, int unit) {
  const int64_t g = gidx(layer, unit);
  void* b = const_cast<void*>(pinned_of_[size_t(g)]);
  if (!b) return;
  free_blocks_[size_t(block_class(layer))].push_back(b);
  pinned_of_[size_t(g)] = nullptr;
  ++xst_.promoted;
}

bool HostCtx::fetch_into_ring(int layer, int unit, bool spec) {
  const uint64_t stride = d_.unit_stride(layer);
  auto rc = std::find_if(ring_classes_.begin(), ring_classes_.end(),
                         [&](const RingClassState& r) { return r.stride == stride; });
  if (rc == ring_classes_.end()) return false;
  for (size_t k = 0; k < rc->count; ++k) {  // round robin from the cursor
    const size_t i = rc->first + (rc->cursor + k) % rc->count;
    if (ring_[i].owner >= 0) continue;
    rc->cursor = (i - rc->first + 1) % rc->count;
    LayerState& s = L_[size_t(layer)];
    HostJobPtr j = make_job(layer, unit, ring_[i].dev, spec);
    fwd_jobs_.push_back(j);
    j->dst_release_ev = ring_owner_ev_[i];  // the layer that released the slot last
    ring_[i].owner = layer;
    ring_[i].job = j;
    s.loc[size_t(unit)] = Ring;
    s.slot[size_t(unit)] = int32_t(i);
    s.job[size_t(unit)] = j;
    (j->from_pinned ? fwd_stats_[size_t(layer)].bytes_pinned : fwd_stats_[size_t(layer)].bytes_disk) +=
        d_.layers[size_t(layer)].unit_bytes;
    submit(j);
    return true;
  }
  return false;
}

void HostCtx::dispatch_pending() {
  for (size_t L = 0; L < L_.size(); ++L) {
    LayerState& s = L_[L];
    if (s.pending.empty()) continue;
    size_t k = 0;
    while (k < s.pending.size() && fetch_into_ring(int(L), s.pending[k], false)) ++k;
    s.pending.erase(s.pending.begin(), s.pending.begin() + std::ptrdiff_t(k));
    if (!s.pending.empty()) return;  // layer order: a later layer never overtakes an earlier one
  }
}

void* HostCtx::unit_addr(int layer, int unit) const {
  const LayerState& s = L_[size_t(layer)];
  if (s.loc[size_t(unit)] == Ring) return ring_[size_t(s.slot[size_t(unit)])].dev;
  const int slot = s.rs->slot(unit);
  if (slot < 0) return nullptr;
  return at(s.pool, uint64_t(slot) * d_.unit_stride(layer));
}

Region HostCtx::region_of(uint64_t addr) const {
  Region r;
  if (!addr) return r;
  for (size_t L = 0; L < L_.size(); ++L) {
    const LayerState& s = L_[L];
    if (!s.pool || !s.rs) continue;
    const uint64_t b = uint64_t(uintptr_t(s.pool)), n = uint64_t(s.rs->capacity()) * d_.unit_stride(int(L));
    if (addr >= b && addr < b + n) return Region{1, int(L), addr - b};
  }
  for (size_t k = 0; k < ring_classes_.size(); ++k) {
    const uint64_t b = uint64_t(uintptr_t(ring_classes_[k].base));
    if (addr >= b && addr < b + ring_classes_[k].stride * ring_classes_[k].count) return Region{2, int(k), addr - b};
  }
  return r;
}

// ---- forward API ------------------------------------------------------------------------------------------------------

void HostCtx::check_stream(void* stream, const char* what) {
  if (!fwd_stream_set_) {
    fwd_stream_ = stream;
    fwd_stream_set_ = true;
    return;
  }
  require(stream == fwd_stream_, SS_E_INVALID,
          std::string(what) + ": a forward must use one engine stream (join other streams into it first)");
}

void HostCtx::host_prefetch(int layer, const int32_t* ids, int n) {
  check_layer(layer, "host_prefetch");
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "host_prefetch: bad ids");
  // readahead_units is 0 in every context this library opens (a nonzero value is refused at open): nothing to read
}

void HostCtx::host_prefetch_layer(int layer) { check_layer(layer, "host_prefetch_layer"); }

void HostCtx::check_layer(int layer, const char* what) const {
  require(layer >= 0 && layer < n_layers(), SS_E_INVALID, std::string(what) + ": layer out of range");
}

void HostCtx::open_forward() {
  if (fwd_open_) return;
  for (auto& s : L_) {
    std::fill(s.loc.begin(), s.loc.end(), int8_t(None));
    std::fill(s.slot.begin(), s.slot.end(), -1);
    std::fill(s.job.begin(), s.job.end(), nullptr);
    std::fill(s.spec_unclaimed.begin(), s.spec_unclaimed.end(), char(0));
    std::fill(s.count.begin(), s.count.end(), 0u);
    s.routed.clear();
    s.pending.clear();
    s.hits.clear();
    s.groups.clear();
    s.group_view.clear();
    s.routes_given = s.acquired = s.released = s.skip = false;
    s.ids_n = -1;
  }
  std::fill(fwd_stats_.begin(), fwd_stats_.end(), ss_layer_stats{});
  fwd_open_ = true;
}

void HostCtx::seed(int layer, const int32_t* units, int n) {
  check_layer(layer, "seed");
  require(!in_forward_ && !fwd_open_, SS_E_INVALID, "seed: only between forwards");
  LayerState& s = L_[size_t(layer)];
  require(s.rs != nullptr, SS_E_INVALID, "seed: layer has no units");
  require(n >= 0 && (units || n == 0), SS_E_INVALID, "seed: bad unit list");
  for (int i = 0; i < n; ++i)
    require(units[i] >= 0 && units[i] < d_.layers[size_t(layer)].n_units, SS_E_INVALID, "seed: unit out of range");
  std::vector<HostJobPtr> jobs;
  std::vector<int32_t> placed;
  ss_status failed = SS_OK;
  std::string err;
  try {
    for (int i = 0; i < n; ++i) {
      const int u = units[i];
      if (s.rs->slot(u) >= 0 || plan_.tier[size_t(gidx(layer, u))] == SS_TIER_PAIR) continue;
      const int slot = s.rs->place(u, false);
      if (slot < 0) break;  // seeds never evict
      placed.push_back(u);
      HostJobPtr j = make_job(layer, u, at(s.pool, uint64_t(slot) * d_.unit_stride(layer)), false);
      jobs.push_back(j);
      submit(j);
    }
  } catch (const Error& e) {
    failed = e.status();
    err = e.what();
  }
  std::vector<int32_t> landed;
  for (int32_t u : placed) {
    bool ok = false;
    for (const auto& j : jobs)
      if (j->unit == u) {
        wait_job_quiet(*j);
        ok = j->state.load() == HostJob::Done;
      }
    if (!ok) s.rs->drop(u);
    else landed.push_back(u);
  }
  for (const auto& j : jobs)
    if (j->state.load() != HostJob::Done && failed == SS_OK) {
      failed = j->err_status;
      err = j->err;
    }
  for (const auto& j : jobs)
    if (j->done_ev) ev_pool_.push_back(j->done_ev);
  stream_sync(copy_);
  stream_sync(copy2_);
  if (excl_)
    for (int32_t u : landed) free_block(layer, u);
  if (failed != SS_OK) fail(failed, err);
}

void HostCtx::begin(const uint32_t* rows, int n) {
  require(!in_forward_, SS_E_INVALID, "begin: previous forward not ended");
  require(rows == nullptr || n == n_layers(), SS_E_INVALID, "begin: rows_per_layer needs one per layer");
  open_forward();
  if (rows)
    for (size_t L = 0; L < L_.size(); ++L) L_[L].skip = rows[L] == 0;
  if (excl_) {
    uint64_t f = 0;
    for (const auto& v : free_blocks_) f += v.size();
    xst_.free_blocks = f;
    xst_.min_free_blocks = std::min(xst_.min_free_blocks, f);
  }
  in_forward_ = true;
}

void HostCtx::ingest_routes(int layer, const int32_t* ids, int n) {
  LayerState& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  require(s.rs != nullptr, SS_E_INVALID, "routes: layer " + std::to_string(layer) + " has no units");
  require(!s.routes_given, SS_E_INVALID, "routes: given twice for layer " + std::to_string(layer));
  require(!s.skip, SS_E_INVALID, "routes: layer " + std::to_string(layer) + " is skipped in this forward");
  s.routes_given = true;  // (an out-of-range id below leaves the layer's routes given, as the reference does)
  for (int i = 0; i < n; ++i) {
    if (ids[i] < 0) continue;
    require(ids[i] < l.n_units, SS_E_INVALID, "routes: unit id " + std::to_string(ids[i]) + " out of range");
    ++s.count[size_t(ids[i])];
  }
  ss_layer_stats& st = fwd_stats_[size_t(layer)];
  std::vector<int32_t> misses, to_admit;
  std::vector<char> busy(size_t(l.n_units), 0);
  for (int u = 0; u < l.n_units; ++u) {
    if (s.loc[size_t(u)] != None) busy[size_t(u)] = 1;
    if (!s.count[size_t(u)] || plan_.tier[size_t(gidx(layer, u))] == SS_TIER_PAIR) continue;
    busy[size_t(u)] = 1;  // a hit of this route is never the victim of one of its misses
    s.routed.push_back(u);
    if (s.loc[size_t(u)] != None) {  // prefetched in this forward
      if (s.spec_unclaimed[size_t(u)]) {
        s.spec_unclaimed[size_t(u)] = 0;
        ++st.spec_used;
        if (s.job[size_t(u)]) promote(s.job[size_t(u)]);
      } else {
        ++st.prefetched;
      }
      misses.push_back(u);
    } else if (s.rs->slot(u) >= 0) {
      s.hits.push_back(u);
    } else {
      to_admit.push_back(u);
      misses.push_back(u);
    }
  }
  st.routed += s.routed.size();
  st.hits += s.hits.size();
  const Admission a = s.rs->admit(to_admit, busy, true, eviction_cap(layer, false));
  xst_.deferred += uint64_t(a.deferred);
  fetch_admitted(layer, a, false);
  for (int32_t u : a.transient)
    if (!fetch_into_ring(layer, u, false)) {
      s.pending.push_back(u);
      s.loc[size_t(u)] = Ring;  // placed when a ring slot frees
    }
  st.admitted += a.admitted.size();
  st.transient += a.transient.size();
  st.evicted += a.evicted.size();
  s.rs->observe(s.routed, misses);
}

void HostCtx::routes(int layer, const int32_t* ids, int n) {
  check_layer(layer, "routes");
  require(in_forward_, SS_E_INVALID, "routes: outside a forward (call ss_begin)");
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "routes: bad ids");
  ingest_routes(layer, ids, n);
}

void HostCtx::routes_dev(int layer, const int32_t* ids_dev, int n, void* stream) {
  check_layer(layer, "routes_dev");
  require(in_forward_, SS_E_INVALID, "routes_dev: outside a forward (call ss_begin)");
  LayerState& s = L_[size_t(layer)];
  require(n >= 0 && s.ids_n < 0 && !s.routes_given, SS_E_INVALID, "routes_dev: given twice or bad count");
  if (size_t(n) > s.ids_cap) {
    dev_->free_pinned(s.ids_host);
    s.ids_host = nullptr;
    s.ids_cap = std::max<size_t>(size_t(n), 1024);
    s.ids_host = static_cast<int32_t*>(dev_->alloc_pinned(4 * s.ids_cap, "device routes"));
  }
  check_stream(stream, "routes_dev");
  copy_d2h(s.ids_host, ids_dev, 4 * uint64_t(n), static_cast<hipStream_t>(stream));
  ev_record(s.ids_ev, static_cast<hipStream_t>(stream));
  s.ids_n = n;
}

void HostCtx::ingest_dev_routes(int layer) {
  LayerState& s = L_[size_t(layer)];
  if (s.ids_n < 0) return;
  ev_sync(s.ids_ev);
  const int n = s.ids_n;
  s.ids_n = -1;
  ingest_routes(layer, s.ids_host, n);
}

void HostCtx::routes_all(int layer) {
  check_layer(layer, "layer_all");
  require(in_forward_, SS_E_INVALID, "layer_all: outside a forward (call ss_begin)");
  const int n = d_.layers[size_t(layer)].n_units;
  std::vector<int32_t> ids(static_cast<size_t>(n));
  for (int u = 0; u < n; ++u) ids[size_t(u)] = u;
  ingest_routes(layer, ids.data(), n);
}

void HostCtx::prefetch(int layer, const int32_t* ids, int n, bool speculative) {
  check_layer(layer, "prefetch");
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "prefetch: bad ids");
  open_forward();  // allowed between forwards: the reads belong to the next forward
  LayerState& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  require(s.rs != nullptr, SS_E_INVALID, "prefetch: layer has no units");
  if (s.routes_given || s.acquired) return;
  ss_layer_stats& st = fwd_stats_[size_t(layer)];
  uint32_t issued = 0;
  std::vector<char> busy(size_t(l.n_units), 0);
  for (int u = 0; u < l.n_units; ++u) busy[size_t(u)] = s.loc[size_t(u)] != None;
  for (int i = 0; i < n; ++i) {
    if (speculative && issued >= o_.lookahead_budget) break;
    const int32_t u = ids[i];
    if (u < 0 || u >= l.n_units) continue;
    if (s.loc[size_t(u)] != None || s.rs->slot(u) >= 0) continue;
    if (plan_.tier[size_t(gidx(layer, u))] == SS_TIER_PAIR) continue;
    const Admission a = speculative && !o_.spec_persistent
                            ? Admission{}
                            : s.rs->admit({u}, busy, true, eviction_cap(layer, speculative));
    xst_.deferred += uint64_t(a.deferred);
    if (!a.admitted.empty()) {
      fetch_admitted(layer, a, speculative);
      st.evicted += a.evicted.size();
    } else if (!fetch_into_ring(layer, u, speculative)) {
      if (speculative) break;  // ring full: speculation never waits
      s.pending.push_back(u);
      s.loc[size_t(u)] = Ring;
    }
    busy[size_t(u)] = 1;
    if (speculative) {
      s.spec_unclaimed[size_t(u)] = 1;
      ++st.spec_issued;
    }
    ++issued;
  }
}

void HostCtx::prefetch_layer(int layer) {
  check_layer(layer, "prefetch_layer");
  const int n = d_.layers[size_t(layer)].n_units;
  std::vector<int32_t> ids(static_cast<size_t>(n));
  for (int u = 0; u < n; ++u) ids[size_t(u)] = u;
  prefetch(layer, ids.data(), n, false);
}

void HostCtx::acquire(int layer, void* stream, bool wait_all, ss_layer_view* out) {
  check_layer(layer, "acquire");
  require(in_forward_, SS_E_INVALID, "acquire: outside a forward");
  require(out != nullptr, SS_E_INVALID, "acquire: null view");
  LayerState& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  require(s.rs != nullptr, SS_E_INVALID, "acquire: layer has no units");
  require(!s.acquired, SS_E_INVALID, "acquire: layer acquired twice in one forward");
  check_stream(stream, "acquire");
  hipStream_t es = static_cast<hipStream_t>(stream);
  ingest_dev_routes(layer);
  require(s.routes_given, SS_E_INVALID,
          "acquire: no routes for layer " + std::to_string(layer) + " (ss_layer_routes / ss_layer_all first)");
  dispatch_pending();
  require(s.pending.empty(), SS_E_CAPACITY,
          "acquire: the stream ring cannot hold layer " + std::to_string(layer) + "'s " +
              std::to_string(s.pending.size()) +
              " remaining transient units (release earlier layers or plan more ring slots)");
  if (s.ready_wait) {  // copies issued for this layer in an earlier forward: one device-side wait
    stream_wait(es, s.ready_ev);
    s.ready_wait = false;
  }
  // groups: 0 = resident before this forward; then the fetched units by route count (desc), id
  std::vector<int32_t> fetched;
  for (int32_t u : s.routed)
    if (s.job[size_t(u)]) fetched.push_back(u);
  std::stable_sort(fetched.begin(), fetched.end(),
                   [&](int32_t a, int32_t b) { return s.count[size_t(a)] > s.count[size_t(b)]; });
  s.groups.clear();
  s.groups.push_back(s.hits);
  const size_t gsz = o_.group_units ? o_.group_units : std::max<size_t>(fetched.size(), 1);
  for (size_t k = 0; k < fetched.size(); k += gsz) {
    std::vector<int32_t> g(fetched.begin() + std::ptrdiff_t(k),
                           fetched.begin() + std::ptrdiff_t(std::min(fetched.size(), k + gsz)));
    std::sort(g.begin(), g.end());
    s.groups.push_back(g);
  }
  if (wait_all) {
    const uint64_t t0 = now_ns();
    for (int32_t u : fetched) {
      wait_job(*s.job[size_t(u)]);
      stream_wait(es, s.job[size_t(u)]->done_ev);
    }
    fwd_stats_[size_t(layer)].wait_ns += now_ns() - t0;
  }
  s.version ^= 1;
  const int v = s.version;
  ev_sync(s.table_ev[v]);  // this version's previous upload has been read
  uint64_t* t = s.table_host[v];
  for (int u = 0; u < l.n_units; ++u) {
    void* a = nullptr;
    if (s.job[size_t(u)] ? s.count[size_t(u)] != 0 : s.rs->slot(u) >= 0) a = unit_addr(layer, u);
    t[u] = uint64_t(reinterpret_cast<uintptr_t>(a));
  }
  copy_h2d(s.table_dev[v], t, 8 * uint64_t(l.n_units), es);
  s.group_view.clear();
  for (const auto& g : s.groups) s.group_view.push_back({g.data(), int(g.size())});
  s.acquired = true;
  out->table_dev = static_cast<const uint64_t*>(s.table_dev[v]);
  out->table_host = t;
  out->n_units = l.n_units;
  out->groups = s.group_view.data();
  out->n_groups = int(s.group_view.size());
}

void HostCtx::group_wait(int layer, int group, void* stream) {
  check_layer(layer, "group_wait");
  LayerState& s = L_[size_t(layer)];
  require(s.acquired && !s.released, SS_E_INVALID, "group_wait: layer not acquired");
  require(group >= 0 && size_t(group) < s.groups.size(), SS_E_INVALID, "group_wait: no such group");
  check_stream(stream, "group_wait");
  if (group == 0) return;
  const uint64_t t0 = now_ns();
  for (int32_t u : s.groups[size_t(group)]) {
    wait_job(*s.job[size_t(u)]);
    stream_wait(static_cast<hipStream_t>(stream), s.job[size_t(u)]->done_ev);
  }
  fwd_stats_[size_t(layer)].wait_ns += now_ns() - t0;
}

void HostCtx::retire_ring(int layer) {
  LayerState& s = L_[size_t(layer)];
  for (size_t i = 0; i < ring_.size(); ++i) {
    if (ring_[i].owner != layer) continue;
    HostJob& j = *ring_[i].job;
    int expect = HostJob::Queued;
    if (!j.state.compare_exchange_strong(expect, HostJob::Cancelled)) wait_job_quiet(j);
    done_cv_.notify_all();
    ring_owner_ev_[i] = s.release_ev;
    ring_[i].owner = -1;
    ring_[i].job.reset();
  }
}

void HostCtx::release(int layer, void* stream) {
  check_layer(layer, "release");
  LayerState& s = L_[size_t(layer)];
  require(s.acquired && !s.released, SS_E_INVALID, "release: layer not acquired or already released");
  check_stream(stream, "release");
  hipStream_t es = static_cast<hipStream_t>(stream);
  ev_record(s.release_ev, es);
  ev_record(s.table_ev[s.version], es);
  s.released = true;
  for (int u = 0; u < d_.layers[size_t(layer)].n_units; ++u)
    if (s.spec_unclaimed[size_t(u)]) {
      s.spec_unclaimed[size_t(u)] = 0;
      ++fwd_stats_[size_t(layer)].spec_dropped;
    }
  retire_ring(layer);
  dispatch_pending();
}

void HostCtx::end() {
  require(in_forward_, SS_E_INVALID, "end: no forward open");
  for (size_t L = 0; L < L_.size(); ++L)
    require(!L_[L].acquired || L_[L].released, SS_E_INVALID,
            "end: layer " + std::to_string(L) + " acquired but not released");
  ss_status failed = SS_OK;
  std::string err;
  for (const auto& j : fwd_jobs_) {
    int expect = HostJob::Queued;
    if (j->spec && j->state.compare_exchange_strong(expect, HostJob::Cancelled)) continue;
    wait_job_quiet(*j);
    if (j->state.load() == HostJob::Failed && failed == SS_OK) {
      failed = j->err_status;
      err = j->err;
    }
  }
  done_cv_.notify_all();
  for (size_t L = 0; L < L_.size(); ++L) {
    LayerState& s = L_[L];
    if (!s.rs) continue;
    for (int u = 0; u < d_.layers[L].n_units; ++u) {
      if (s.spec_unclaimed[size_t(u)]) ++fwd_stats_[L].spec_dropped;
      if (s.loc[size_t(u)] == Persistent && s.job[size_t(u)] && s.job[size_t(u)]->state.load() != HostJob::Done)
        s.rs->drop(u);  // admitted, but its read never ran or failed: not resident
    }
    for (size_t i = 0; i < ring_.size(); ++i)
      if (ring_[i].owner == int(L)) {
        ring_[i].owner = -1;
        ring_[i].job.reset();
      }
  }
  if (excl_) {
    for (size_t L = 0; L < L_.size(); ++L) {
      LayerState& s = L_[L];
      if (!s.rs) continue;
      for (int u = 0; u < d_.layers[L].n_units; ++u)
        if (s.loc[size_t(u)] == Persistent && s.job[size_t(u)] && s.job[size_t(u)]->from_pinned &&
            s.job[size_t(u)]->state.load() == HostJob::Done)
          free_block(int(L), u);
    }
    {
      std::lock_guard<std::mutex> lk(copy_mu_);
      if (!wb_evs_.empty()) {
        ev_record(wb_mark_ev_, wb_);
        stream_wait(copy_, wb_mark_ev_);
        stream_wait(copy2_, wb_mark_ev_);
      }
      join_copies();
      ev_record(blocks_ev_, copy_);
      wb_gate_ = true;
    }
    for (int64_t g : wb_units_) wb_pending_[size_t(g)] = nullptr;
    wb_units_.clear();
    for (hipEvent_t e : wb_evs_) ev_pool_.push_back(e);
    wb_evs_.clear();
    uint64_t f = 0;
    for (const auto& v : free_blocks_) f += v.size();
    xst_.free_blocks = f;
  }
  {
    std::lock_guard<std::mutex> lk(copy_mu_);
    join_copies();
    for (size_t L = 0; L < L_.size(); ++L) {
      LayerState& s = L_[L];
      if (!s.rs) continue;
      bool any = false;
      for (int u = 0; u < d_.layers[L].n_units && !any; ++u)
        any = s.loc[size_t(u)] == Persistent && s.job[size_t(u)] && s.job[size_t(u)]->state.load() == HostJob::Done;
      if (any) {  // this forward's persistent copies: the next acquire of the layer waits for them device-side
        ev_record(s.ready_ev, copy_);
        s.ready_wait = true;
      }
    }
  }
  for (const auto& j : fwd_jobs_)
    if (j->done_ev) ev_pool_.push_back(j->done_ev);
  fwd_jobs_.clear();
  fwd_stream_set_ = false;
  fwd_stream_ = nullptr;
  ss_layer_stats tot{};
  for (size_t L = 0; L < L_.size(); ++L) {
    add(stats_[L], fwd_stats_[L]);
    add(tot, fwd_stats_[L]);
  }
  if (hook_) hook_(hook_user_, &tot, fwd_stats_.data(), n_layers());
  in_forward_ = false;
  fwd_open_ = false;
  ++forward_;
  publish();  // (also a forward whose read failed: its numbers are folded)
  if (dverify_ && failed == SS_OK) collect_verify();  // throws SS_E_HASH naming the first unit that differs
  if (failed != SS_OK) fail(failed, err);
}

void HostCtx::check_unit(int layer, int unit) {
  check_layer(layer, "check_unit");
  LayerState& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  require(s.acquired && !s.released, SS_E_INVALID, "check_unit: layer not acquired");
  require(unit >= 0 && unit < l.n_units, SS_E_INVALID, "check_unit: unit out of range");
  void* a = reinterpret_cast<void*>(uintptr_t(s.table_host[s.version][unit]));
  require(a != nullptr, SS_E_INVALID, "check_unit: unit not available in this forward");
  if (s.job[size_t(unit)]) {
    wait_job(*s.job[size_t(unit)]);
    ev_sync(s.job[size_t(unit)]->done_ev);
  }
  stream_sync(copy_);
  stream_sync(copy2_);
  std::vector<char> got(size_t(l.unit_bytes));
  std::vector<char> want(size_t(round_up(l.unit_bytes, kHostAlign)) + kHostAlign);
  hip_check(hipMemcpy(got.data(), a, got.size(), hipMemcpyDeviceToHost), "hipMemcpy (check_unit)");
  char* w = reinterpret_cast<char*>(round_up(uint64_t(reinterpret_cast<uintptr_t>(want.data())), kHostAlign));
  read_unit_host(layer, unit, w, false, nullptr);
  require(std::memcmp(got.data(), w, got.size()) == 0, SS_E_HASH,
          "check_unit: landed bytes of (" + std::to_string(layer) + ", " + std::to_string(unit) +
              ") differ from the source");
  if (!l.hash.empty())
    require(xxh64(got.data(), got.size()) == l.hash[size_t(unit)], SS_E_HASH,
            "check_unit: landed bytes of (" + std::to_string(layer) + ", " + std::to_string(unit) +
                ") differ from the descriptor hash");
}

ss_layer_stats HostCtx::total() const {
  ss_layer_stats t{};
  for (const auto& s : stats_) add(t, s);
  return t;
}

void HostCtx::stats_reset() {
  std::fill(stats_.begin(), stats_.end(), ss_layer_stats{});
  if (!in_forward_) publish();
}

// ---- stats-v1 and the snapshot (reference src/stream_ctx.cpp:1762-1885) ------------------------------------------

void HostCtx::publish() {
  if (!snap_armed_.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(snap_mu_);
  if (snap_.layers.size() != stats_.size()) snap_.layers.resize(stats_.size());
  std::copy(stats_.begin(), stats_.end(), snap_.layers.begin());
  snap_.x = xst_;
  snap_.forwards = forward_;
  ++snap_.seq;
}

bool HostCtx::snapshot(ss_layer_stats* total, ss_snapshot_info* info) const {
  snap_armed_.store(true, std::memory_order_relaxed);
  ss_layer_stats t{};
  ss_snapshot_info i{};
  {
    std::lock_guard<std::mutex> lk(snap_mu_);
    if (snap_.seq == 0) return false;
    for (const ss_layer_stats& l : snap_.layers) add(t, l);
    i.sequence = snap_.seq;
    i.forwards = snap_.forwards;
    if (excl_) {
      i.exclusive_writebacks = snap_.x.writebacks;
      i.exclusive_writeback_bytes = snap_.x.writeback_bytes;
      i.exclusive_deferred = snap_.x.deferred;
      i.exclusive_promoted = snap_.x.promoted;
      i.exclusive_free_blocks = snap_.x.free_blocks;
      i.exclusive_min_free_blocks = snap_.x.min_free_blocks;
      i.exclusive_rereads = snap_.x.rereads;
      i.exclusive_discards = snap_.x.discards;
    }
  }
  if (excl_) {
    i.flags |= SS_SNAPSHOT_EXCLUSIVE;
    i.exclusive_blocks = n_blocks_;
  }
  i.struct_size = uint32_t(sizeof i);
  if (total) *total = t;
  if (info) *info = i;
  return true;
}

bool HostCtx::snapshot_json(Json* out) const {
  snap_armed_.store(true, std::memory_order_relaxed);
  Published p;
  p.layers.resize(stats_.size());
  {
    std::lock_guard<std::mutex> lk(snap_mu_);
    if (snap_.seq == 0) return false;
    std::copy(snap_.layers.begin(), snap_.layers.end(), p.layers.begin());
    p.x = snap_.x;
    p.forwards = snap_.forwards;
  }
  *out = format_stats(p.forwards, p.layers.data(), p.x);
  return true;
}

Json HostCtx::stats_json() const { return format_stats(forward_, stats_.data(), xst_); }

Json HostCtx::format_stats(uint64_t forwards, const ss_layer_stats* layers, const ss_exclusive_stats& x) const {
  Json j = Json::object();
  j["schema"] = Json::string("strix-stream/stats-v1");
  j["backend"] = Json::string("hip");
  j["forwards"] = Json::number(forwards);
  Json direct = Json::array();
  for (const auto& f : files_) direct.push(Json::boolean(f->direct()));
  j["sources_direct"] = direct;
  ss_layer_stats t{};
  Json ls = Json::array();
  for (size_t L = 0; L < stats_.size(); ++L) {
    add(t, layers[L]);
    ls.push(stats_object(layers[L]));
  }
  j["total"] = stats_object(t);
  j["layers"] = ls;
  if (excl_) {
    Json e = Json::object();
    e["writebacks"] = Json::number(x.writebacks);
    e["writeback_bytes"] = Json::number(x.writeback_bytes);
    e["discards"] = Json::number(x.discards);
    e["deferred"] = Json::number(x.deferred);
    e["rereads"] = Json::number(x.rereads);
    e["promoted"] = Json::number(x.promoted);
    e["free_blocks"] = Json::number(x.free_blocks);
    e["min_free_blocks"] = Json::number(x.min_free_blocks);
    e["blocks"] = Json::number(n_blocks_);
    j["exclusive"] = e;
  }
  return j;
}

ss_exclusive_stats HostCtx::exclusive_stats() const {
  ss_exclusive_stats x = xst_;
  x.struct_size = uint32_t(sizeof x);
  return x;
}

}  // namespace tsa
