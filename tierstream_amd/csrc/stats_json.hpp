// The per-layer counters as a stats-v1 object (reference src/stream_ctx.cpp:1828-1843): the same keys for the host
// contract and device-gated documents.
#pragma once

#include "json.hpp"
#include "strix_stream/ss.h"

namespace tsa {

inline Json stats_object(const ss_layer_stats& s) {
  Json j = Json::object();
  j["routed"] = Json::number(s.routed);
  j["hits"] = Json::number(s.hits);
  j["admitted"] = Json::number(s.admitted);
  j["transient"] = Json::number(s.transient);
  j["evicted"] = Json::number(s.evicted);
  j["prefetched"] = Json::number(s.prefetched);
  j["spec_issued"] = Json::number(s.spec_issued);
  j["spec_used"] = Json::number(s.spec_used);
  j["spec_dropped"] = Json::number(s.spec_dropped);
  j["bytes_pinned"] = Json::number(s.bytes_pinned);
  j["bytes_disk"] = Json::number(s.bytes_disk);
  j["wait_ns"] = Json::number(s.wait_ns);
  return j;
}

}  // namespace tsa
