/*
 * flash_mhc_probe.h -- HBM ceiling probe used by bench.py.
 *
 * No counterpart in the reference: a measurement helper, not part of the
 * K1/K3/K4 path.  It streams 16-byte vectors over device buffers so the
 * benchmark can report the achievable read, write and copy bandwidth of the
 * GPU it runs on next to the kernels' achieved bandwidth.
 */
#ifndef FLASH_MHC_PROBE_H_
#define FLASH_MHC_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMHC_PROBE_READ 0  /* read nbytes from src (nontemporal), write nothing but one word to dst */
#define FMHC_PROBE_WRITE 1 /* write nbytes to dst */
#define FMHC_PROBE_COPY 2  /* copy nbytes from src to dst (nontemporal) */

/* nbytes must be a positive multiple of 16; src/dst 16-byte aligned device
 * pointers of at least nbytes (dst >= 16 bytes for FMHC_PROBE_READ).
 * Returns 0 or an FMHC_ERR_* code of flash_mhc_hip.h. */
int fmhc_stream_probe(int kind, const void* src, void* dst, int64_t nbytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_MHC_PROBE_H_ */
