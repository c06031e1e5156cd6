/* dsmoe_probe.h - measurement tooling beside libdsmoe.so, not part of the
 * layer's ABI (no counterpart in the reference, which has no measurement
 * hooks).  Built into its own library, libdsmoe_probe.so, which only
 * bench.py --dma-mb loads.
 *
 * dsmoe_probe_dma_read reads exactly `bytes` (a multiple of 1 MiB, src 16-byte
 * aligned) with the direct global -> LDS loads the grouped GEMMs issue
 * (global_load_lds_dwordx4), one workgroup per MiB, and writes one word per
 * workgroup to sink (bytes / 1 MiB words), so a traffic counter's reading per
 * dispatch (FETCH_SIZE) can be set against the bytes actually read.  Returns
 * 0, -1 for bad arguments or -4 for a launch error. */
#ifndef DSMOE_PROBE_H
#define DSMOE_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int dsmoe_probe_dma_read(const void* src, size_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSMOE_PROBE_H */
