#include "hsa_copy.hpp"

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>
#include <immintrin.h>

#include <string>
#include <thread>
#include <type_traits>

#include "common.hpp"
#include "hip_rt.hpp"

namespace tsa {

// The runtime entry points this file calls, from the HSA runtime library already in the process.
struct HsaCopier::Api {
  decltype(&hsa_init) init = nullptr;
  decltype(&hsa_shut_down) shut_down = nullptr;
  decltype(&hsa_iterate_agents) iterate_agents = nullptr;
  decltype(&hsa_agent_get_info) agent_get_info = nullptr;
  decltype(&hsa_system_get_info) system_get_info = nullptr;
  decltype(&hsa_signal_create) signal_create = nullptr;
  decltype(&hsa_signal_destroy) signal_destroy = nullptr;
  decltype(&hsa_signal_store_screlease) signal_store = nullptr;
  decltype(&hsa_signal_load_scacquire) signal_load = nullptr;
  decltype(&hsa_amd_memory_async_copy) async_copy = nullptr;
  decltype(&hsa_amd_profiling_async_copy_enable) prof_enable = nullptr;
  decltype(&hsa_amd_profiling_get_async_copy_time) prof_time = nullptr;
  std::string missing;

  static const Api& get() {
    static const Api a = load();
    return a;
  }
  static Api load() {
    Api a;
    void* h = dlopen("libhsa-runtime64.so.1", RTLD_NOW | RTLD_NOLOAD);
    if (!h) h = dlopen("libhsa-runtime64.so.1", RTLD_NOW);
    if (!h) {
      a.missing = "libhsa-runtime64.so.1";
      return a;
    }
    const auto sym = [&](auto& fn, const char* name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
      if (!fn && a.missing.empty()) a.missing = name;
    };
    sym(a.init, "hsa_init");
    sym(a.shut_down, "hsa_shut_down");
    sym(a.iterate_agents, "hsa_iterate_agents");
    sym(a.agent_get_info, "hsa_agent_get_info");
    sym(a.system_get_info, "hsa_system_get_info");
    sym(a.signal_create, "hsa_signal_create");
    sym(a.signal_destroy, "hsa_signal_destroy");
    sym(a.signal_store, "hsa_signal_store_screlease");
    sym(a.signal_load, "hsa_signal_load_scacquire");
    sym(a.async_copy, "hsa_amd_memory_async_copy");
    sym(a.prof_enable, "hsa_amd_profiling_async_copy_enable");
    sym(a.prof_time, "hsa_amd_profiling_get_async_copy_time");
    return a;
  }
};

namespace {
void hsa_check(hsa_status_t s, const char* what) {
  require(s == HSA_STATUS_SUCCESS || s == HSA_STATUS_INFO_BREAK, SS_E_BACKEND,
          std::string("HSA: ") + what + " failed (status " + std::to_string(int(s)) + ")");
}
}  // namespace

HsaCopier::HsaCopier(int hip_device) : api_(&Api::get()) {
  require(api_->missing.empty(), SS_E_BACKEND, "HSA: the runtime's " + api_->missing + " is not available");
  hsa_check(api_->init(), "hsa_init");
  try {
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, hip_device), "hipGetDeviceProperties");
    struct Find {
      const Api* api;
      uint32_t domain, bus, dev;
      hsa_agent_t gpu{}, cpu{};
      bool has_gpu = false, has_cpu = false;
    } f{api_, uint32_t(prop.pciDomainID), uint32_t(prop.pciBusID), uint32_t(prop.pciDeviceID)};
    hsa_check(api_->iterate_agents(
                  [](hsa_agent_t a, void* data) {
                    Find& f = *static_cast<Find*>(data);
                    hsa_device_type_t t;
                    if (f.api->agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS)
                      return HSA_STATUS_ERROR;
                    if (t == HSA_DEVICE_TYPE_CPU && !f.has_cpu) {
                      f.cpu = a;
                      f.has_cpu = true;
                    } else if (t == HSA_DEVICE_TYPE_GPU && !f.has_gpu) {
                      uint32_t bdf = 0, domain = 0;
                      if (f.api->agent_get_info(a, hsa_agent_info_t(HSA_AMD_AGENT_INFO_BDFID), &bdf) !=
                              HSA_STATUS_SUCCESS ||
                          f.api->agent_get_info(a, hsa_agent_info_t(HSA_AMD_AGENT_INFO_DOMAIN), &domain) !=
                              HSA_STATUS_SUCCESS)
                        return HSA_STATUS_ERROR;
                      if (domain == f.domain && (bdf >> 8) == f.bus && ((bdf >> 3) & 0x1fu) == f.dev) {
                        f.gpu = a;
                        f.has_gpu = true;
                      }
                    }
                    return HSA_STATUS_SUCCESS;
                  },
                  &f),
              "hsa_iterate_agents");
    require(f.has_gpu && f.has_cpu, SS_E_BACKEND,
            "HSA: no GPU agent at the PCI location of HIP device " + std::to_string(hip_device) + " (or no CPU agent)");
    gpu_ = f.gpu;
    cpu_ = f.cpu;
    uint64_t hz = 0;
    hsa_check(api_->system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &hz), "timestamp frequency");
    ticks_per_ns_ = hz ? double(hz) / 1e9 : 1.0;
    e_.emplace_back();  // index 0: "nothing"
  } catch (...) {
    api_->shut_down();
    throw;
  }
}

HsaCopier::~HsaCopier() {
  wait_all();
  for (size_t i = 1; i < e_.size(); ++i) (void)api_->signal_destroy(e_[i].s);
  (void)api_->shut_down();
}

void HsaCopier::wait_all() const {
  std::lock_guard<std::mutex> lk(mu_);
  for (size_t i = 1; i < e_.size(); ++i)
    for (uint32_t spins = 0; api_->signal_load(e_[i].s) != 0; ++spins) {
      if (spins < 4096) _mm_pause();
      else std::this_thread::yield();
    }
}

bool HsaCopier::done_locked(uint32_t sig) const { return sig == 0 || api_->signal_load(e_[sig].s) == 0; }

bool HsaCopier::done(uint32_t sig) const {
  if (sig == 0) return true;
  std::lock_guard<std::mutex> lk(mu_);
  return done_locked(sig);
}

void HsaCopier::ref(uint32_t sig) {
  if (sig == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  ++e_[sig].refs;
}

void HsaCopier::unref(uint32_t sig) {
  if (sig == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  release_locked(sig);
}

void HsaCopier::release_locked(uint32_t sig) {
  Entry& e = e_[sig];
  require(e.refs > 0, SS_E_BACKEND, "HSA: a copy signal released more often than held");
  if (--e.refs == 0) retiring_.push_back(sig);
}

uint32_t HsaCopier::take_locked() {
  if (free_.empty()) {  // recycle the unreferenced signals whose copies have ended
    std::vector<uint32_t> ended;
    size_t keep = 0;
    for (uint32_t s : retiring_) {
      if (done_locked(s)) ended.push_back(s);
      else retiring_[keep++] = s;
    }
    retiring_.resize(keep);
    for (uint32_t s : ended) {  // an ended copy's polls have run: its dependencies may be recycled too
      free_.push_back(s);
      std::vector<uint32_t> deps;
      deps.swap(e_[s].deps);
      for (uint32_t d : deps) release_locked(d);
    }
  }
  uint32_t i;
  if (!free_.empty()) {
    i = free_.back();
    free_.pop_back();
  } else {
    Entry e;
    hsa_check(api_->signal_create(0, 0, nullptr, &e.s), "hsa_signal_create");
    e_.push_back(e);
    i = uint32_t(e_.size() - 1);
  }
  e_[i].refs = 1;
  api_->signal_store(e_[i].s, 1);
  return i;
}

uint32_t HsaCopier::copy(void* dst, const void* src, uint64_t bytes, bool to_host, const uint32_t* deps,
                         uint32_t n_deps) {
  std::lock_guard<std::mutex> lk(mu_);
  const uint32_t i = take_locked();
  dep_buf_.clear();
  for (uint32_t d = 0; d < n_deps; ++d)
    if (!done_locked(deps[d])) {
      dep_buf_.push_back(e_[deps[d]].s);
      ++e_[deps[d]].refs;
      e_[i].deps.push_back(deps[d]);
    }
  // (the runtime refuses a dependency array with a count of 0 unless it is null)
  const uint32_t nd = uint32_t(dep_buf_.size());
  const hsa_signal_t* dp = nd ? dep_buf_.data() : nullptr;
  const hsa_status_t st = to_host ? api_->async_copy(dst, cpu_, src, gpu_, bytes, nd, dp, e_[i].s)
                                  : api_->async_copy(dst, gpu_, src, cpu_, bytes, nd, dp, e_[i].s);
  if (st != HSA_STATUS_SUCCESS) {
    api_->signal_store(e_[i].s, 0);
    e_[i].refs = 1;
    release_locked(i);  // (ended: its dependencies go with it at the next recycling)
    hsa_check(st, to_host ? "a device-to-host copy" : "a host-to-device copy");
  }
  return i;
}

void HsaCopier::profiling(bool on) { hsa_check(api_->prof_enable(on), "copy profiling"); }

bool HsaCopier::copy_ns(uint32_t sig, uint64_t* ns) const {
  if (sig == 0) return false;
  std::lock_guard<std::mutex> lk(mu_);
  hsa_amd_profiling_async_copy_time_t t{};
  if (!done_locked(sig) || api_->prof_time(e_[sig].s, &t) != HSA_STATUS_SUCCESS || t.end < t.start) return false;
  *ns = uint64_t(double(t.end - t.start) / ticks_per_ns_ + 0.5);
  return true;
}

}  // namespace tsa
