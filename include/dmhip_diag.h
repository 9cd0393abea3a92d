/* dmhip_diag.h -- launch-floor probes for gfx950 (libdmhip_diag.so).
 *
 * Measurement only: not part of the drop-in surface (include/dmhip.h) and
 * with no counterpart in the reference.  bench.py uses them to state what a
 * single short GEMV launch can reach on the device: the back-to-back
 * duration of an empty kernel, and of a kernel that only reads the bytes a
 * GEMV would read.  Each call runs on the current HIP device, on a stream of
 * its own, and returns 0 on success or the HIP error code.
 */
#ifndef DMHIP_DIAG_H
#define DMHIP_DIAG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mean duration in microseconds of `launches` back-to-back launches of an
   empty kernel of `workgroups` x `threads` (threads a multiple of 64, at most
   1024), timed with events around the whole sequence after three untimed
   launches. */
int dmhip_diag_time_empty(uint32_t workgroups, uint32_t threads, size_t launches, double *us);

/* The same for a kernel that reads n bytes (a multiple of 16) with 16-byte
   loads, four per lane issued before any use, and keeps nothing: launch i
   reads sources[i % count] (16-byte aligned device addresses), so rotating
   copies larger than the 256 MB MALL give cold reads. */
int dmhip_diag_time_read(const void *const *sources, size_t count, size_t n, size_t launches, double *us);

#ifdef __cplusplus
}
#endif

#endif
