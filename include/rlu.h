/* librlu.so -- C-ABI of the MI355X (gfx950) MoE decode hot path.
 *
 * Plain pointers, sizes and a hipStream_t; no torch types. Every entry point returns 0 on
 * success, a negative code on a bad argument (nothing is launched), or the value of
 * hipGetLastError() after the launch. No entry point allocates, synchronizes or reads device
 * memory from the host, so all of them can be captured into a HIP graph; every kernel runs on
 * the caller's stream.
 *
 * Each declaration names the reference interface it replaces (paths relative to the
 * davetha/r9700-lru-expert-cache checkout).
 */
#ifndef RLU_H
#define RLU_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device LRU expert cache -------------------------------------------------------------
 * Replaces kernels/lru/r4d_lru.hip:579-589 (r4d_lru_manage), :596-610 (r4d_lru_fused) and
 * :612-629 (r4d_lru_gather) with identical signatures, argument meaning and return codes.
 * Bound from Python as in patches/.../fused_moe/experts/r4d_mxfp4_moe.py.lru.diff:184-200:
 *   manage: [void*] + [int]*5 + [void*]*9
 *   fused:  [void*] + [int]*5 + [void*]*8 + [int]*3 + [void*]*7
 *   gather: [void*, void*, long]*6 + [void*, void*, int, int, void*]
 *
 * State (per layer, caller-owned, never reallocated): table[E] int32 expert->slot or -1,
 * map_cold[E] int32 expert->expert when not resident else -1, slot_expert[S] int32,
 * slot_stamp[S] int64, routed[E] uint8 (scratch, left holding this step's routed flags),
 * step[1] int64, miss[cap][2] int32 (expert, slot), n_miss[1] int32.
 * Limits: 1 <= E <= 1024, 1 <= S <= 1024, 0 <= max_inserts <= 1024, mk >= 0.
 * Returns -1 outside them. fused additionally needs bs, L, NB > 0; L and NB must be the sizes
 * moe_align_block_size allocates (L = mk < E ? min(mk*bs, mk+E*(bs-1)) : mk+E*(bs-1),
 * NB = ceil(L/bs)); writes past L / NB are dropped rather than performed.
 * Align output order is stable (ascending token index inside each bucket) at every mk.
 * gather: every size must be > 0 and a multiple of 16, chunks and lanes > 0; grid is
 * (chunks, lanes); sources may be pinned host memory (device pointer from
 * hipHostGetDevicePointer) or device memory.
 */
int r4d_lru_manage(const int* topk_ids, int mk, int E, int S, int max_distinct,
                   int max_inserts, int* table, int* map_cold, int* slot_expert,
                   long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                   int* n_miss, hipStream_t stream);

int r4d_lru_fused(const int* topk_ids, int mk, int E, int S, int max_distinct,
                  int max_inserts, int* table, int* map_cold, int* slot_expert,
                  long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                  int* n_miss, int bs, int L, int NB, int* sorted_hot, int* eids_hot,
                  int* npad_hot, int* sorted_cold, int* eids_cold, int* npad_cold,
                  hipStream_t stream);

int r4d_lru_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                   void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                   void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                   const int* miss, const int* n_miss, int chunks, int lanes,
                   hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RLU_H */
