// Routing capture for HIP graphs: each MoE layer's topk_ids of a decode step copied into a
// device ring, one launch per layer, so that a captured graph keeps recording on every replay.
//
// Same capture semantics as tools/routecap/routecap.py:83-100: the layer-0 call of a step
// advances the step counter ctr and stores it as the slot's step number (slot = ctr % ring);
// every layer's ids go to ring[layer][slot] as int16, padded with -1 to the ring's width.
// There the capture is five torch ops per layer (fill, copy, two index_copy_, an add at layer
// 0); here it is one single-workgroup launch. The host reads the ring back between steps and
// keeps every slot whose step has finished.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlu.h"

namespace rlu {

constexpr int RT = 256;

__global__ __launch_bounds__(RT) void route_capture_k(const int* __restrict__ ids, int n,
                                                      int layer, int ring, int width,
                                                      int16_t* __restrict__ ring_ids,
                                                      long long* __restrict__ ring_step,
                                                      long long* __restrict__ ctr) {
  const long long c = ctr[0] + (layer == 0 ? 1 : 0);
  __syncthreads();                                  // every thread holds c before ctr moves
  const int slot = (int)(c % ring);
  if (layer == 0 && threadIdx.x == 0) {
    ctr[0] = c;
    ring_step[slot] = c;
  }
  int16_t* dst = ring_ids + ((size_t)layer * ring + slot) * width;
  for (int i = threadIdx.x; i < width; i += RT) dst[i] = i < n ? (int16_t)ids[i] : (int16_t)-1;
}

}  // namespace rlu

extern "C" {

// tools/routecap/routecap.py:83-100 (the capture fn, as torch ops there)
int rlu_route_capture(const int* topk_ids, int n, int layer, int nlayer, int ring, int width,
                      short* ring_ids, long long* ring_step, long long* ctr,
                      hipStream_t stream) {
  if (n < 0 || width <= 0 || n > width || ring <= 0 || layer < 0 || layer >= nlayer) return -1;
  if ((n > 0 && !topk_ids) || !ring_ids || !ring_step || !ctr) return -1;
  hipLaunchKernelGGL(rlu::route_capture_k, dim3(1), dim3(rlu::RT), 0, stream, topk_ids, n,
                     layer, ring, width, (int16_t*)ring_ids, ring_step, ctr);
  return (int)hipGetLastError();
}

}  // extern "C"
