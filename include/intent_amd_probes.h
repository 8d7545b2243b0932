/* Measurement probes of libintent_amd.so: bench-only entry points, not
 * operators. They have no counterpart in the reference; bench.py's --probe
 * modes call them to measure what bounds the operators on the box they run
 * on (the HBM read floor of a streaming kernel, the sustained MFMA rate).
 * Same conventions as intent_amd.h: device pointers, a HIP stream (NULL for
 * the default stream), an int status (INTENT_OK or a negative code).
 */
#ifndef INTENT_AMD_PROBES_H
#define INTENT_AMD_PROBES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16) of `buf` once with the plainest coalesced
 * 16-byte loads, each workgroup of 256 lanes covering 256 * unroll * 16
 * contiguous bytes (unroll in {1, 2, 4, 8, 16}). Its duration is the HBM read
 * floor that a streaming kernel over the same bytes is compared with.
 * store = 0: `sink` (at least 256 uint32, device) is written only on a hash
 * coincidence. store = 1: every wave also writes 8 bytes of its result to
 * sink[2w], sink[2w + 1] (w: the wave's index in the grid), as a GEMV writes
 * its outputs; sink_words must be at least 8 * ceil(bytes / (4096 * unroll)) (four waves per
 * workgroup). store + 2 (2 or 3): the same with non-temporal loads (the cache policy of the
 * decode kernels' weight loads).
 */
int intent_hbm_read_probe(const void* buf, int64_t bytes, int unroll, int store, uint32_t* sink, int64_t sink_words,
                          void* stream);

/* `workgroups` groups of four waves each issue `iters` rounds of four
 * independent register-only 32x32 MFMAs (kind 0: f16, 32768 flops each; kind
 * 1: i8, 65536 ops each). The rate it reaches is the matrix cores' sustained
 * ceiling at the clock the chip holds under that load, the practical bound
 * for the compute-bound kernels. `sink` (256 uint32, device) is written only
 * on a value coincidence.
 */
int intent_mfma_peak_probe(int kind, int64_t iters, int64_t workgroups, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INTENT_AMD_PROBES_H */
