// Measurement helper for bench.py: the device's fp32 atomic-add rate, the
// bound the backward kernel's row-gradient adds run against. No counterpart
// in the reference; not on any attention path.
//
// Each wave adds 1.0 to 64 consecutive floats of one row (a 256-byte run,
// the backward's pattern: one add per channel of a cache row) per
// instruction, rows chosen by a stride walk over `rows` rows of `row_len`
// floats. The result of the add is unused, so each is one
// global_atomic_add_f32 without return.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/sas.h"
#include "../../include/sas_bench.h"
#include "sas_common.h"

namespace {

__global__ void __launch_bounds__(256) sas_bench_atomic_kernel(float* dst, int rows, int runs_per_row,
                                                               int iters) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int row_len = runs_per_row * 64;
  for (int i = 0; i < iters; ++i) {
    const int run = wave * 7919 + i * 104729;   // co-prime strides spread the runs
    const int r = (int)((unsigned)run % (unsigned)(rows * runs_per_row));
    atomicAdd(dst + (size_t)(r / runs_per_row) * row_len + (r % runs_per_row) * 64 + lane, 1.0f);
  }
}

}  // namespace

extern "C" int sas_bench_atomic_add_v1(float* dst, int32_t rows, int32_t row_len, int32_t workgroups,
                                       int32_t iters, void* stream) {
  sas::clear_error();
  if (!dst || rows < 1 || row_len < 64 || row_len % 64 || workgroups < 1 || iters < 1)
    return sas::set_error(SAS_EINVAL, "bench atomic: bad arguments");
  hipLaunchKernelGGL(sas_bench_atomic_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream, dst, rows,
                     row_len / 64, iters);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "bench atomic launch: %s", hipGetErrorString(e));
  return SAS_OK;
}
