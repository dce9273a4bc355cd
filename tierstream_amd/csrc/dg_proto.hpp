// Device-gated decode: the words the GPU and the library share. The record layouts are the reference's
// (src/dg_proto.hpp:14-25: DgRecord 288 bytes, DgPredRecord 272 bytes) so a record dump reads the same; the placement
// is this library's: records, export flags and the completion words live in fine-grained coherent host memory (the
// service thread polls them), while ready words, the sequence, the sticky abort and the error words live in HBM (only
// the GPU polls ready). The service publishes a layer's ready word with a stream value-write ordered after its copies,
// or, with the device check of landed units on, the layer's last check kernel writes it (and the landed units' slot
// entries) when it ends.
#pragma once

#include <cstdint>

namespace tsa {

constexpr uint32_t kDgMaxIds = 64;

struct DgRecord {
  uint32_t n_ids, n_pred_promised, mask_lo, mask_hi;
  uint32_t seq, pad[3];
  uint32_t ids[kDgMaxIds];
};
struct DgPredRecord {
  uint32_t n_pred, pad[3];
  uint32_t pred[kDgMaxIds];
};
static_assert(sizeof(DgRecord) == 288 && sizeof(DgPredRecord) == 272, "record layout");

// Device error codes (err_aux = the gated layer, or the step's sequence for kDgDesync).
// kDgHash (this library's device verify, no reference counterpart): a landed unit's bytes in HBM differ from its
// descriptor hash (err_aux = the gated layer whose copies landed it).
enum DgErrCode : uint32_t {
  kDgOk = 0, kDgTimeout = 1, kDgBadId = 2, kDgHostAbort = 3, kDgDesync = 4, kDgAbsent = 5, kDgHash = 6
};

// Every address the control kernels use, fixed at open (a captured graph replays for the context's life).
struct DgDevWords {
  // HBM
  uint32_t* seq = nullptr;
  uint32_t* abort = nullptr;
  uint32_t* err_count = nullptr;
  uint32_t* err_code = nullptr;
  uint32_t* err_aux = nullptr;
  uint32_t* any_miss = nullptr;    // [G]
  uint32_t* ready = nullptr;       // [G]
  uint32_t* absent_err = nullptr;
  const int32_t* slot_of = nullptr;
  const uint32_t* unit_base = nullptr;  // [G + 1]
  uint64_t* stamps = nullptr;      // [4 G]: export end, wait entry, ready seen (0: no miss), wait exit (wall clock)
  // fine-grained host memory, device addresses
  DgRecord* rec = nullptr;          // [G]
  DgPredRecord* prec = nullptr;     // [G]
  uint32_t* flag = nullptr;         // [G]
  uint32_t* pflag = nullptr;        // [G]
  uint32_t* done = nullptr;
  uint32_t* m_err_code = nullptr;
  uint32_t* m_err_aux = nullptr;
  uint32_t* m_err_count = nullptr;
  uint32_t* host_abort = nullptr;
  uint32_t* host_seq = nullptr;
  uint32_t* began = nullptr;
  uint64_t timeout_ticks = 0;       // the wait kernel's deadline in wall-clock ticks (100 MHz)
};

// Host view of the same fine-grained words.
struct DgMappedHost {
  DgRecord* rec = nullptr;
  DgPredRecord* prec = nullptr;
  uint32_t* flag = nullptr;
  uint32_t* pflag = nullptr;
  uint32_t* done = nullptr;
  uint32_t* err_code = nullptr;
  uint32_t* err_aux = nullptr;
  uint32_t* err_count = nullptr;
  uint32_t* host_abort = nullptr;
  uint32_t* host_seq = nullptr;
  uint32_t* began = nullptr;
};

inline uint32_t load_acquire(const uint32_t* p) { return __atomic_load_n(p, __ATOMIC_ACQUIRE); }
inline void store_release(uint32_t* p, uint32_t v) { __atomic_store_n(p, v, __ATOMIC_RELEASE); }

// Launchers (hipError_t as int; none synchronizes or allocates; all legal under stream capture).
int dg_launch_begin(const DgDevWords& d, void* stream);
int dg_launch_export(const DgDevWords& d, uint32_t g, const int32_t* ids, uint32_t n, uint32_t n_pred, void* stream);
int dg_launch_predict(const DgDevWords& d, uint32_t g, const int32_t* ids, uint32_t n, void* stream);
int dg_launch_wait(const DgDevWords& d, uint32_t g, void* stream);
int dg_launch_end(const DgDevWords& d, void* stream);
// A one-lane store of v into a device word on the stream (the ready / entry publication when value-writes are off).
int dg_launch_store(uint32_t* word, uint32_t v, void* stream);
// Three-tier reads in flight: one lane polls a reader's word in fine-grained host memory until it holds gen, so the
// copies enqueued behind it on the stream start once the staging buffer's file read returned. The token's abort words
// and the wait deadline end it too (a deadline sets kDgTimeout with err_aux = aux, the gated layer of the read).
int dg_launch_await(const DgDevWords& d, const uint32_t* word, uint32_t gen, uint32_t aux, void* stream);

}  // namespace tsa
