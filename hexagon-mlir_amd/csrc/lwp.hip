// Light-weight region profiling on the GPU timeline.
//
// The reference instruments each region of a compiled kernel with begin and
// end hooks that append a record {id, cycles low word, cycles high word} to
// a buffer, later written out as {"entries": [{"id", "cyc"}]}
// (test/utils/dsp/include/prof_utils.cc:37-60) and folded into per-region
// totals by test/python/process_lwp.py:20-60.  Here a region is a stream of
// kernels, so a hook is a one-wave kernel enqueued on the same stream: it
// reads the GPU's constant-rate wall clock when it runs, after every kernel
// enqueued before it has finished, and stores the same three-word record at
// a slot the host assigns.
#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {

__global__ __launch_bounds__(64) void lwp_mark(uint32_t* rec, int64_t slot, uint32_t id) {
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x;
  if (lane < 3) {
    const uint32_t w = lane == 0 ? id : (lane == 1 ? (uint32_t)t : (uint32_t)(t >> 32));
    rec[slot * 3 + lane] = w;
  }
}

}  // namespace

hipError_t launch_lwp_mark(uint32_t* records, int64_t slot, uint32_t id, hipStream_t stream) {
  hipLaunchKernelGGL(lwp_mark, dim3(1), dim3(64), 0, stream, records, slot, id);
  return hipGetLastError();
}

}  // namespace hxmi
