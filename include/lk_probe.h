/*
 * Measurement probes: the memory-system floors the decode kernels are
 * measured against (bench.py --workload stream_floor). They have no reference
 * counterpart and are not part of the product library: they are built into
 * their own local_kimi_amd/liblkprobe.so, which only the benchmark loads.
 *
 * Return codes are the LK_OK / LK_ERR_* values of lk_w4a16.h; the message of
 * the last failure on the calling host thread is lk_probe_last_error().
 */
#ifndef LK_PROBE_H
#define LK_PROBE_H

#include "lk_w4a16.h"

#ifdef __cplusplus
extern "C" {
#endif

/* lk_probe_stream_read reads `count` (1..32) device regions once with 16-byte
 * non-temporal loads, one launch; regions and bytes are HOST arrays of device
 * pointers and byte counts (each region 16-byte aligned, a positive multiple
 * of 16 bytes); sink is device memory of 256 uint32 words, written only in the
 * practically impossible case that a thread's folded words equal a fixed
 * value (it keeps the loads live). lk_probe_empty launches an empty kernel
 * (one wave). */
LK_API int lk_probe_stream_read(const void* const* regions, const int64_t* bytes, int count,
                                uint32_t* sink, void* stream);
LK_API int lk_probe_empty(void* stream);
LK_API const char* lk_probe_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* LK_PROBE_H */
