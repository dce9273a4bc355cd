/*
 * Test hooks of libtierstream_amd (the counterpart of reference include/strix_stream/ss_test.h: calls tests link by
 * name that an engine never needs). None changes state.
 */
#ifndef TIERSTREAM_AMD_TSA_TEST_H
#define TIERSTREAM_AMD_TSA_TEST_H

#include <stdint.h>

#include "../strix_stream/ss.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Host contract: where a table address points. kind 1 = layer `index`'s resident pool, 2 = stream ring class `index`
 * (ascending slot size), 0 = neither; offset = bytes from that region's base (slot = offset / unit stride). */
SS_API ss_status tsa_test_region_of(const ss_ctx* c, uint64_t addr, int* kind, int* index, uint64_t* offset);
/* Device-gated: the host mirror of slot_of (one int32 per gated key, -1 = not on the device); *n = keys. */
SS_API ss_status tsa_test_dg_table(const ss_ctx* c, int32_t* out, uint32_t cap, uint32_t* n);
/* verify_hash = 2: landed units whose device check failed, since open. */
SS_API uint64_t tsa_test_verify_failures(const ss_ctx* c);

#ifdef __cplusplus
}
#endif

#endif
