/*
 * flash_mhc_probe.h -- HBM ceiling probe and cache flush used by bench.py.
 *
 * No counterpart in the reference: a measurement helper, not part of the
 * K1/K3/K4 path, built into its own library (libflash_mhc_probe.so), which the
 * ops never load.  It streams 16-byte vectors over device buffers so the
 * benchmark can report the achievable read, write and copy bandwidth of the
 * GPU it runs on next to the kernels' achieved bandwidth, and evict the
 * caches before a cold-cache timing.
 */
#ifndef FLASH_MHC_PROBE_H_
#define FLASH_MHC_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMHC_PROBE_ABI_VERSION 2

#define FMHC_PROBE_READ 0         /* read nbytes from src (nontemporal), write nothing but one word to dst */
#define FMHC_PROBE_WRITE 1        /* write nbytes to dst (nontemporal stores, as the kernels' outputs) */
#define FMHC_PROBE_COPY 2         /* copy nbytes from src to dst (nontemporal loads and stores) */
#define FMHC_PROBE_READ_CACHED 3  /* FMHC_PROBE_READ with ordinary loads (allocate in L2 / memory-side cache) */
#define FMHC_PROBE_WRITE_CACHED 4 /* FMHC_PROBE_WRITE with ordinary stores */

/* nbytes must be a positive multiple of 16; src/dst 16-byte aligned device
 * pointers of at least nbytes (dst >= 16 bytes for the read kinds).
 * Returns 0 or an FMHC_ERR_* code of flash_mhc_hip.h. */
int fmhc_stream_probe(int kind, const void* src, void* dst, int64_t nbytes, void* stream);

/* FMHC_PROBE_ABI_VERSION of the built probe library. */
int fmhc_probe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_MHC_PROBE_H_ */
