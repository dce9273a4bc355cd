// The opaque handles of the C ABI and the context-call guard (poisoning rules of reference src/capi.cpp:481-508: a
// library error leaves the context usable; SS_E_BACKEND / SS_E_NOMEM or an unexpected exception poisons it).
#pragma once

#include <memory>

#include "common.hpp"
#include "model.hpp"

namespace tsa {
class HostCtx;
class DgCtx;
}  // namespace tsa

struct ss_desc {
  tsa::Desc d;
};
struct ss_plan {
  tsa::Plan p;
  const ss_desc* desc;
};
struct ss_ctx {
  std::unique_ptr<tsa::HostCtx> host;  // SS_FORWARD_HOST
  std::unique_ptr<tsa::DgCtx> dg;      // SS_FORWARD_DEVICE_GATED (exactly one of the two)
  ~ss_ctx();
};

namespace tsa {

bool ctx_poisoned(const ss_ctx* c);
void lookahead_select(const float* scores, int rows, int n_experts, int top_k, int32_t* out, int max_out,
                      int* n_out);
void ctx_poison(ss_ctx* c);

template <class F>
ss_status ctx_guard(ss_ctx* c, F&& f) noexcept {
  if (!c) {
    set_last_error("null context");
    return SS_E_INVALID;
  }
  if (ctx_poisoned(c)) {
    set_last_error("context poisoned by an earlier device, allocation or internal failure: close it");
    return SS_E_BACKEND;
  }
  try {
    f();
    return SS_OK;
  } catch (const Error& e) {
    if (e.status() == SS_E_BACKEND || e.status() == SS_E_NOMEM) ctx_poison(c);
    set_last_error(e.what());
    return e.status();
  } catch (const std::bad_alloc&) {
    ctx_poison(c);
    set_last_error("out of host memory (context poisoned)");
    return SS_E_NOMEM;
  } catch (const std::exception& e) {
    ctx_poison(c);
    set_last_error(e.what());
    return SS_E_BACKEND;
  }
}

}  // namespace tsa
