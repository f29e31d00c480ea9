/* gk_probe.h -- measurement probe used by bench.py and the tests
 * (tests/csrc/libgk_probe.so, built by tests/csrc/build_probe.py).  Not part
 * of the block-FP8 library and not a reference interface: it has no
 * counterpart in the reference, which publishes no performance figures.
 *
 * gk_probe_stream_read reads `bytes` of device memory at `src` (16-byte
 * aligned, a multiple of 16) with `workgroups` workgroups of 256 lanes and
 * 16-byte non-temporal loads, and writes nothing to `sink` (a device word)
 * unless the data folds to a sentinel.  Asynchronous on `stream` (hipStream_t
 * as void*).  Returns 0, 1 for bad arguments, 2 for a launch error.
 *
 * gk_probe_bf16x2_check runs the kernels' paired fp32 -> bf16 rounding (the
 * hardware conversion plus its NaN fix-up) over all 2^32 float bit patterns,
 * each as the low and the high value, against the software round-to-nearest-
 * even (NaN -> 0x7fc0), and adds to `counts` (two zeroed device uint64 words,
 * 8-byte aligned) the mismatches and the values checked (2^33).  Asynchronous;
 * returns 0, 1 for a bad pointer, 2 for a launch error.
 *
 * gk_probe_e4m3_check does the same for the activation quantizer's hardware
 * E4M3 encode (both halves of the packed word) against the software
 * round-to-nearest-even encoder on every fp32 with |v| <= 464 (the
 * quantizer's quotients stay below it): it adds the mismatches and the
 * values checked (2 x 0x43E80001). */
#ifndef GK_PROBE_H
#define GK_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int gk_probe_stream_read(const void* src, size_t bytes, void* sink, int workgroups, void* stream);
int gk_probe_bf16x2_check(void* counts, void* stream);
int gk_probe_e4m3_check(void* counts, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GK_PROBE_H */
