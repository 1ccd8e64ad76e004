// The streamed prefill grouped GEMM (prefill.hip), launched by the tiled entry points of
// gemm_tiled.hip for the K it is built for.
#pragma once
#include <hip/hip_runtime.h>

namespace rlu {

// Launches the streamed kernel over a tile list (tiles of <= 8 blocks) when K and N have a
// built configuration, and returns 0; returns -1 (nothing launched) otherwise.
int launch_prefill_stream(const void* qx, const float* xs, const void* wq, const float* ws,
                          const int* sorted_ids, const int* expert_ids, const int* tiles,
                          const int* ntiles, int max_tiles, const float* topk_weights, void* y,
                          int mtk, int top_k, int K, int N, hipStream_t stream);

}  // namespace rlu
