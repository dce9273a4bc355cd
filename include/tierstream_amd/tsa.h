/*
 * tierstream MI355X extensions: the device-side byte path that has no function in the reference ABI, plus the small
 * plumbing calls tests and tools use instead of a framework (device memory, streams, events).
 *
 * None of these replaces a reference entry point; each names the reference code whose work it moves to the device:
 *  - tsa_xxh64_digest / tsa_xxh64_verify: the host XXH64 of landed units (reference src/xxh64.cpp:39-112, called from
 *    src/stream_ctx.cpp:511-544 and :622-660, src/dg_load.cpp:424-432) and the test-only ss_check_unit
 *    (src/stream_ctx.cpp:1711-1735), as kernels over HBM.
 *  - tsa_scatter: the per-part copies of a device-gated miss into each part's arena slot (reference
 *    src/dg_ctx.cpp:163-168) as one staged copy plus a kernel that writes every part with 128-bit stores.
 *  - tsa_xxh64_checkpoints: the host side of tsa_xxh64_verify (the four XXH64 accumulators at segment starts).
 *  - tsa_xxh64_verify_slots: the same check for units landed in a device-gated arena, addressed by (key, slot) with
 *    the arguments passed by value (the check a device-gated context runs before each layer's ready word).
 *
 * Every pointer named *_dev is device memory; every launch is asynchronous on `stream` (a hipStream_t, NULL = the
 * null stream) and allocates nothing. Return: SS_OK, SS_E_INVALID (argument checks, done on the host before any
 * launch), SS_E_BACKEND (a HIP error), SS_E_NOMEM.
 */
#ifndef TIERSTREAM_AMD_TSA_H
#define TIERSTREAM_AMD_TSA_H

#include <stddef.h>
#include <stdint.h>

#include "../strix_stream/ss.h"

#ifdef __cplusplus
extern "C" {
#endif

#define TSA_MAX_EXTENTS 4

/* A byte range; a unit's bytes are its extents back to back. Every extent starts 8-byte aligned and every extent but
 * the last is a multiple of 32 bytes (XXH64 stripes never straddle two extents). */
typedef struct tsa_extent {
  const void* ptr;
  uint64_t bytes;
} tsa_extent;
typedef struct tsa_unit {
  tsa_extent ext[TSA_MAX_EXTENTS];
  uint32_t n_ext;
  uint32_t reserved;
} tsa_unit;

/* XXH64 (seed 0) of each unit's bytes into digests_dev[i]. units_dev: n entries in device memory. */
SS_API ss_status tsa_xxh64_digest(const tsa_unit* units_dev, uint32_t n, uint64_t* digests_dev, void* stream);

/* Host XXH64 (seed 0) of host bytes: the same function the library checks descriptor hashes with. */
SS_API uint64_t tsa_xxh64_host(const void* data, uint64_t bytes);

/* Checkpoint layout of a unit: for each extent e, its segments are [k*seg, min((k+1)*seg, span_e)) with span_e =
 * bytes_e (the last extent: bytes rounded down to 32, and at least one segment); the checkpoint of a segment is the
 * four accumulators before its first stripe. tsa_checkpoint_count gives the count for extent byte sizes. */
SS_API uint64_t tsa_checkpoint_count(const uint64_t* extent_bytes, uint32_t n_ext, uint64_t seg_bytes);
/* Host: the checkpoints (4 x uint64 each, segment order) and the digest of host bytes laid out as `unit`. */
SS_API ss_status tsa_xxh64_checkpoints(const tsa_unit* unit_host, uint64_t seg_bytes, uint64_t* states,
                                       uint64_t n_states, uint64_t* digest);

typedef struct tsa_verify_unit {
  tsa_extent ext[TSA_MAX_EXTENTS];
  uint32_t n_ext;
  uint32_t reserved;
  uint64_t seg_first;           /* first segment of this unit in the launch (prefix sum, ascending) */
  const uint64_t* states;       /* device: the unit's checkpoints (tsa_xxh64_checkpoints) */
  uint64_t digest;              /* the descriptor hash */
  uint64_t total;               /* the unit's bytes */
} tsa_verify_unit;
/* fail_dev[i] |= 1 when unit i's device bytes do not reproduce its checkpoints and digest (2: bad launch table).
 * n_segments = the units' checkpoint counts summed; seg_bytes as for the checkpoints. The caller zeroes fail_dev. */
SS_API ss_status tsa_xxh64_verify(const tsa_verify_unit* units_dev, uint32_t n_units, uint64_t n_segments,
                                  uint64_t seg_bytes, uint32_t* fail_dev, void* stream);

/* Units laid out as a device-gated arena: part p of the unit in slot s at arena[p] + s x part_bytes[p] (every arena
 * pointer 8-byte aligned, every part_bytes a multiple of 8, every part but the last a multiple of 32); key k's
 * checkpoints (its parts as the extents, tsa_xxh64_checkpoints) at states_dev + k x count x 4, its digest at
 * digests_dev[k]. */
typedef struct tsa_arena_verify {
  const void* arena[TSA_MAX_EXTENTS];
  uint64_t part_bytes[TSA_MAX_EXTENTS];
  uint32_t n_parts;
  uint32_t reserved;
  uint64_t seg_bytes;
  const uint64_t* states_dev;
  const uint64_t* digests_dev;
} tsa_arena_verify;
/* fail_dev[i] |= 1 when unit (keys[i], slots[i]) differs from its checkpoints and digest. keys and slots are host
 * arrays of n entries (any n: launches of up to 64 units each). The caller zeroes fail_dev. */
SS_API ss_status tsa_xxh64_verify_slots(const tsa_arena_verify* a, const uint32_t* keys, const int32_t* slots, uint32_t n,
                                        uint32_t* fail_dev, void* stream);
/* The same check fused with the staged units' scatter (a device-gated context with verify_hash = 2 and parts under
 * 8 MiB): unit i's bytes lie back to back at src_dev + i x (its parts' bytes), 8-byte aligned; each is written to
 * (keys[i], slots[i])'s arena slot while it is hashed, so its bytes cross HBM once each way. Replaces the reference's
 * per-part copies (src/dg_ctx.cpp:163-168) followed by a separate check. */
SS_API ss_status tsa_xxh64_scatter_verify_slots(const tsa_arena_verify* a, const uint32_t* keys, const int32_t* slots,
                                                uint32_t n, const void* src_dev, uint32_t* fail_dev, void* stream);

/* One staged unit: src_dev holds the unit's bytes back to back; part p goes to dst[p] (parts[p] bytes). Every pointer
 * 16-byte aligned, every part a multiple of 16 bytes. block_first: prefix sum of the jobs' 16 KiB blocks. */
typedef struct tsa_scatter_job {
  const void* src;
  void* dst[TSA_MAX_EXTENTS];
  uint64_t bytes[TSA_MAX_EXTENTS];
  uint32_t n_parts;
  uint32_t reserved;
  uint64_t block_first;
} tsa_scatter_job;
#define TSA_SCATTER_BLOCK_BYTES 16384u
/* Blocks a job needs (its parts' bytes / 16 KiB, rounded up per part). */
SS_API uint64_t tsa_scatter_blocks(const uint64_t* part_bytes, uint32_t n_parts);
SS_API ss_status tsa_scatter(const tsa_scatter_job* jobs_dev, uint32_t n_jobs, uint64_t n_blocks, void* stream);

/* Synthetic bytes, counter-based: kind 0 = uniform bytes (word i of the stream = a splitmix64 of (seed, stream_id,
 * i)), kind 1 = bfloat16 N(0, sigma) by Box-Muller over the same words, kind 2 = Q4 blocks of 18 bytes (an fp16
 * scale, then 16 bytes of packed 4-bit values; sigma unused). offset: the stream's first byte written (a multiple of
 * 8); bytes: a multiple of 8. */
SS_API ss_status tsa_synth(void* dst_dev, uint64_t bytes, uint64_t seed, uint64_t stream_id, uint64_t offset,
                           uint32_t kind, float sigma, void* stream);

/* ---- plumbing (tests, tools) ---- */
SS_API ss_status tsa_device_count(int* n);
SS_API ss_status tsa_set_device(int device);
SS_API ss_status tsa_malloc(void** p, uint64_t bytes);
SS_API ss_status tsa_free(void* p);
SS_API ss_status tsa_host_alloc(void** p, uint64_t bytes);  /* pinned, coarse-grained */
SS_API ss_status tsa_host_free(void* p);
/* kind: 0 host->device, 1 device->host, 2 device->device, 3 default (inferred) */
SS_API ss_status tsa_memcpy(void* dst, const void* src, uint64_t bytes, int kind, void* stream);
SS_API ss_status tsa_memset(void* dst, int value, uint64_t bytes, void* stream);
SS_API ss_status tsa_stream_create(void** stream);
SS_API ss_status tsa_stream_destroy(void* stream);
SS_API ss_status tsa_stream_sync(void* stream);
SS_API ss_status tsa_device_sync(void);
SS_API ss_status tsa_event_create(void** ev);              /* timing event (no system-scope fence when recorded) */
SS_API ss_status tsa_event_destroy(void* ev);
SS_API ss_status tsa_event_record(void* ev, void* stream);
SS_API ss_status tsa_event_sync(void* ev);
SS_API ss_status tsa_event_elapsed_ms(void* start, void* stop, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* TIERSTREAM_AMD_TSA_H */
