// The streamed prefill grouped GEMM (prefill.hip), launched by the tiled entry points of
// gemm_tiled.hip for the K it is built for.
#pragma once
#include <hip/hip_runtime.h>

namespace rlu {

// The second weight set and align of a two-set launch: the tiles whose block count carries
// bit 16 take their expert ids, sorted ids, weights and block scales from here.
struct PfSecond {
  const void* wq;
  const float* ws;
  const int* sorted_ids;
  const int* expert_ids;
};

// K and N with a built configuration of the plain streamed kernel.
bool prefill_stream_built(int K, int N);

// Launches the streamed kernel over a tile list (tiles of <= 8 blocks) when K and N have a
// built configuration, and returns 0; returns -1 (nothing launched) otherwise. second: null
// for a one-set tile list.
int launch_prefill_stream(const void* qx, const float* xs, const void* wq, const float* ws,
                          const int* sorted_ids, const int* expert_ids, const PfSecond* second,
                          const int* tiles, const int* ntiles, int max_tiles,
                          const float* topk_weights, void* y, int mtk, int top_k, int K, int N,
                          hipStream_t stream);

// The same kernel for gate_up with SiLU-mul-quant in its epilogue: writes q2 [mtk, N / 2] e4m3
// and s2 [mtk, N / 256] (group-128 scales) instead of the bf16 output. Returns -1 (nothing
// launched) when K and N have no built configuration.
bool prefill_stream_act_built(int K, int N);
int launch_prefill_stream_act(const void* qx, const float* xs, const void* wq, const float* ws,
                              const int* sorted_ids, const int* expert_ids,
                              const PfSecond* second, const int* tiles, const int* ntiles,
                              int max_tiles, void* q2, float* s2, int mtk, int top_k, int K,
                              int N, hipStream_t stream);

}  // namespace rlu
