/* Measurement helper of libsas.so, used by bench.py to state the fp32
 * atomic-add peak that the backward kernel's row-gradient adds are priced
 * against. It has no counterpart in the reference (its callers: the
 * benchmark only) and is not part of the attention interface in sas.h. */
#ifndef SAS_BENCH_H
#define SAS_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Launch `workgroups` x 256 threads on `stream`; every wave adds 1.0f,
 * `iters` times, to a run of 64 consecutive floats of a row of `dst`
 * ([rows, row_len] fp32, row_len a multiple of 64), rows chosen by a stride
 * walk: workgroups * 256 * iters fp32 atomic adds in all. Returns SAS_OK, or
 * SAS_EINVAL / SAS_ELAUNCH with sas_last_error() set. */
int sas_bench_atomic_add_v1(float* dst, int32_t rows, int32_t row_len, int32_t workgroups, int32_t iters,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAS_BENCH_H */
