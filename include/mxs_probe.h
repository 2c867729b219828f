/* libmxs_probe.so: HBM rate probes for bench.py (measurement only, not part of the NF4 path's
 * interface in include/mxs_nf4.h).  Error codes are those of mxs_nf4.h. */
#ifndef MXS_PROBE_H
#define MXS_PROBE_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Measurement only, no counterpart in the reference: streams over n_chunks 16-byte chunks that
 * report what HBM delivers for an access pattern (bench.py's hbm_ceiling).  kind 0: the
 * standalone dequant's pattern without its arithmetic (4-byte non-temporal loads from src,
 * 16-byte non-temporal stores of the dword repeated to dst; 4 + 16 bytes per chunk); kind 1:
 * 16-byte loads from src only (dst receives 4 bytes per 64 chunks); kind 2: 16-byte stores to
 * dst only (src unused, may be NULL).  dst 16-byte aligned; src 16-byte aligned for kind 1. */
int mxs_hbm_probe(int kind, const void* src, void* dst, int64_t n_chunks, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MXS_PROBE_H */
