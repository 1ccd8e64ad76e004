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
 * :612-629 (r4d_lru_gather) with identical signatures and argument meaning. The return codes
 * are the reference's with one narrower limit: r4d_lru_manage also returns -1 for E > 1024
 * (the reference's manager took any E; its fused kernel, like both here, stops at 1024, and the
 * 512-expert model is far inside it). A negative mk means no tokens, as in the reference.
 * Bound from Python as in patches/.../fused_moe/experts/r4d_mxfp4_moe.py.lru.diff:184-200:
 *   manage: [void*] + [int]*5 + [void*]*9
 *   fused:  [void*] + [int]*5 + [void*]*8 + [int]*3 + [void*]*7
 *   gather: [void*, void*, long]*6 + [void*, void*, int, int, void*]
 *
 * State (per layer, caller-owned, never reallocated): table[E] int32 expert->slot or -1,
 * map_cold[E] int32 expert->expert when not resident else -1, slot_expert[S] int32,
 * slot_stamp[S] int64, routed[E] uint8 (scratch, left holding this step's routed flags),
 * step[1] int64, miss[cap][2] int32 (expert, slot), n_miss[1] int32.
 * Limits: 1 <= E <= 1024, 1 <= S <= 1024, 0 <= max_inserts <= 1024 (and mk >= 0 for fused).
 * Returns -1 outside them; manage treats mk < 0 as mk = 0. fused additionally needs bs, L,
 * NB > 0; L and NB must be the sizes moe_align_block_size allocates
 * (L = mk < E ? min(mk*bs, mk+E*(bs-1)) : mk+E*(bs-1), NB = ceil(L/bs)); writes past L / NB are dropped rather than performed.
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

/* No counterpart in the reference: r4d_lru_fused plus, in the same launch (workgroups 1..rows,
 * one row each, beside the cache's workgroup 0), the per-token-group-128 e4m3 quant of the
 * layer's hidden state x [rows, K] bf16 (ldx elements apart) into q [rows, K] and scale
 * [rows, K / 128] -- the quant the reference launched separately before its first GEMM
 * (patches/.../r4dhip.py.diff:22-34), bit for bit rlu_quant_fp8_group with group 128.
 * Returns r4d_lru_fused's codes, -1 for bad rows / K / ldx / null buffers, -2 K % 128. */
int rlu_lru_fused_quant(const int* topk_ids, int mk, int E, int S, int max_distinct,
                        int max_inserts, int* table, int* map_cold, int* slot_expert,
                        long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                        int* n_miss, int bs, int L, int NB, int* sorted_hot, int* eids_hot,
                        int* npad_hot, int* sorted_cold, int* eids_cold, int* npad_cold,
                        const void* x, int rows, int K, int ldx, void* q, float* scale,
                        hipStream_t stream);

int r4d_lru_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                   void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                   void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                   const int* miss, const int* n_miss, int chunks, int lanes,
                   hipStream_t stream);

/* The bucket split of the three-way gather overlap (docs/REVIEW.md:281-301 proposes it; the
 * reference has no kernel for it). From the hot align's eids_hot[nb] (slot per block, -1 =
 * skip) and this step's miss list (miss[cap][2] = (expert, slot), n_miss[0] entries): eids_res
 * keeps the blocks whose slot was resident before the manager ran, eids_new the blocks whose
 * slot the manager installed; the other entry of each pair is -1. A grouped GEMM over eids_res
 * (and the cold align) may run while r4d_lru_gather copies; one over eids_new runs after it.
 * Together they write the rows one GEMM over eids_hot writes, bit for bit.
 * Limits: nb >= 0, miss_cap >= 0, 1 <= S <= 1024; -1 outside them. */
int rlu_lru_split_fresh(const int* eids_hot, int nb, const int* miss, const int* n_miss,
                        int miss_cap, int S, int* eids_res, int* eids_new, hipStream_t stream);

/* ---- activation quant, SiLU-mul-quant, top-k reduction ----------------------------------
 * bf16 activations (uint16 bit patterns), e4m3fn outputs (one byte each), float32 scales.
 * group = 128: one scale per 128 columns (per-token-group-128, the GEMM input format of this
 * path); group = 0: one scale per row (the reference's per-token form). Scale rule for both:
 * max(amax / 448, 1 / (448 * 512)); q = e4m3(clamp(x / scale, +-448)), nearest-even.
 * Returns -1 on bad sizes (K or d not a multiple of 8, ld too small), -2 on a bad group,
 * -3 when a per-row (group 0) row is too long for one workgroup.
 */

/* Replaces the activation quant of patches/.../mxfp4/r4dhip.py.diff:22-34 (fp8_quant_shared
 * -> vLLM scaled_fp8_quant) and kernels/fp8_target_lmhead.py:72-73 (vLLM
 * per_token_group_quant_fp8). x [rows, K] with row stride ldx (elements); q [rows, K];
 * scale [rows, K/128] or [rows]. */
int rlu_quant_fp8_group(const void* x, int rows, int K, int ldx, int group, void* q,
                        float* scale, hipStream_t stream);

/* Replaces kernels/fused_silu_mul_quant.py:75-101 (silu_mul_quant): x [rows, 2d] bf16 = gate |
 * up with row stride ldx; act = bf16(bf16(silu(g)) * u) is written to `act` [rows, d] when it
 * is not null; q [rows, d]; scale [rows, d/128] or [rows]. */
int rlu_silu_mul_quant(const void* x, int rows, int d, int ldx, int group, void* q,
                       float* scale, void* act, hipStream_t stream);

/* Replaces vLLM's ops.moe_sum as called at patches/.../r4d_mxfp4_moe.py.lru.diff:696:
 * out[m, :] = bf16(sum_k in[m * top_k + k, :]) with float32 accumulation in k order.
 * H % 8 == 0. */
int rlu_moe_sum(const void* in, int M, int top_k, int H, void* out, hipStream_t stream);

/* ---- fp8 block-scaled GEMMs on MFMA ----------------------------------------------------------
 * Replaces the closed r4d_gemm_moe_mxfp4a8_nt_b16 behind the op r4d_mxfp4_moe_gemm_into
 * (patches/.../r4d_mxfp4_moe.py.lru.diff:363-395; argument order of
 * tests/k1/moe_ref_harness.py:55-56,221-226), for e4m3 weights with 128x128 float32 block scales:
 *   qx [mtk/top_k, K] e4m3, xs [mtk/top_k, K/128] f32, wq [E, N, K] e4m3 in fragment order
 *   (rlu_shuffle_fp8_weight; the closed kernel likewise took pre-shuffled weights), ws [E, N/128, K/128]
 *   f32, wref unused (the reference's second scale slot), y [mtk, N] bf16, sorted_ids [em],
 *   expert_ids [em/16], num_post_pad [1] (read on the device), topk_weights [mtk] f32 or null.
 * Row contract of the reference kernel: sorted ids >= mtk are padding, expert id -1 skips the
 * block, only named rows are written, y[row] *= topk_weights[row] when given.
 * wv = workgroups per CU of a persistent grid (0: one workgroup per item group, balanced by the
 * hardware dispatcher), sk = waves of a workgroup that split
 * one tile's K range (1, 2, 4; 0: the largest that divides K/128), npw = 16-column tiles per
 * item (1, 2, 4, 8). Partial sums are added in a fixed order, so a given sk is deterministic.
 * Returns -1 bad sizes, -2 K or N not a multiple of 128, -4 sk unsupported or not dividing
 * K/128, -5 bad wv, -6 bad npw; the closed launcher aborted instead. */
int r4d_gemm_moe_fp8blk_nt_b16(const void* qx, const float* xs, const void* wq,
                               const float* ws, const void* wref, void* y,
                               const int* sorted_ids, const int* expert_ids,
                               const int* num_post_pad, const float* topk_weights, int em,
                               int mtk, int top_k, int K, int N, int wv, int sk, int npw,
                               hipStream_t stream);

/* No counterpart in the reference as one call: the two r4d_mxfp4_moe_gemm_into calls of
 * _gemm_split (patches/.../r4d_mxfp4_moe.py.lru.diff:584-592) -- resident slots, then the full
 * expert tensor -- in one launch. Block list 1 (sorted_hot, eids_hot, npad_hot, em entries)
 * runs against wq_hot / ws_hot, block list 2 against wq / ws (device or pinned host memory).
 * Same row contract, arguments, checks and codes as r4d_gemm_moe_fp8blk_nt_b16, so its output
 * equals the two calls with the same sk bit for bit. */
int rlu_moe_gemm_split(const void* qx, const float* xs, const void* wq_hot, const float* ws_hot,
                       const int* sorted_hot, const int* eids_hot, const int* npad_hot,
                       const void* wq, const float* ws, const int* sorted_cold,
                       const int* eids_cold, const int* npad_cold, const float* topk_weights,
                       void* y, int em, int mtk, int top_k, int K, int N, int wv, int sk,
                       int npw, hipStream_t stream);

/* No counterpart in the reference, which runs gate_up into ic1 [mtk, N] and then
 * fused_silu_mul_quant (r4d_mxfp4_moe.py.lru.diff:659-696, kernels/fused_silu_mul_quant.py:
 * 26-101): rlu_moe_gemm_split of gate_up (npw 2) with the SiLU-mul in its epilogue. act bf16
 * [mtk, N/2] = bf16(silu(g) x u) of the GEMM's bf16 outputs g (columns [0, N/2)) and u
 * ([N/2, N)), the activation rlu_silu_mul_quant computes from rlu_moe_gemm_split's y, bit for
 * bit, on every row the aligns name (other rows untouched). wq == NULL runs the hot list alone.
 * N % 256 == 0; other checks and codes as rlu_moe_gemm_split (no topk_weights, no npw). */
int rlu_moe_gemm_split_act(const void* qx, const float* xs, const void* wq_hot,
                           const float* ws_hot, const int* sorted_hot, const int* eids_hot,
                           const int* npad_hot, const void* wq, const float* ws,
                           const int* sorted_cold, const int* eids_cold, const int* npad_cold,
                           void* act, int em, int mtk, int top_k, int K, int N, int wv, int sk,
                           hipStream_t stream);

/* No counterpart in the reference (see rlu_moe_gemm_split_act): the down projection of the split
 * GEMM reading the bf16 activation act [mtk, K] instead of q2 / s2. Each workgroup quantizes
 * the rows of its block per 128-column group exactly as rlu_silu_mul_quant (group 128) does,
 * so y equals rlu_moe_gemm_split (sk 1, any npw, top_k 1) on that kernel's q2 / s2, bit for bit,
 * with topk_weights as there. wq == NULL runs the hot list alone. K % 128 == 0, K <= 768,
 * N % 256 == 0; -1 / -2 on bad sizes or null operands. */
int rlu_moe_gemm_split_qin(const void* act, const void* wq_hot, const float* ws_hot,
                           const int* sorted_hot, const int* eids_hot, const int* npad_hot,
                           const void* wq, const float* ws, const int* sorted_cold,
                           const int* eids_cold, const int* npad_cold,
                           const float* topk_weights, void* y, int em, int mtk, int K, int N,
                           hipStream_t stream);

/* Replaces fp8hip_gemm_w8a8_launch behind gemm_fp8_block (kernels/fp8_target_lmhead.py:70-74):
 * y [M, N] bf16 = qx [M, K] (xs [M, K/128]) x w [N, K] (ws [N/128, K/128])^T, 1 <= M <= 16,
 * w in fragment order (rlu_shuffle_fp8_weight), as fp8hip takes shuffle_weight_gfx1201 output. */
int rlu_gemm_fp8blk_m16(const void* qx, const float* xs, const void* w, const float* ws,
                        void* y, int M, int N, int K, int wv, int npw, hipStream_t stream);

/* Replaces shuffle_weight_gfx1201 (the load-time weight shuffle behind pack_fp8_block,
 * kernels/fp8_target_lmhead.py:44-66) for gfx950: row-major e4m3 [rows, K] -> MFMA fragment
 * order, the layout every GEMM above reads. Byte (n, k), n = 16 nt + r,
 * k = 128 kb + 64 h + 16 c + j, lands at ((nt (K/128) + kb) 2 + h) 1024 + (16 c + r) 16 + j:
 * a permutation inside each 16-row strip, so stacked experts [E, N, K] shuffle as rows = E N.
 * rows % 16 == 0, K % 128 == 0, out must not overlap w. Returns -1 / -2 on bad sizes. */
int rlu_shuffle_fp8_weight(const void* w, void* out, long long rows, int K, hipStream_t stream);

/* No counterpart in the reference (its closed launcher had one kernel for every M): the grouped
 * GEMM for the MFMA regime (prefill chunks, tens of rows per expert). Step 1 builds the tile
 * list from an align output (expert_ids [nb_max], num_post_pad): every run of 16-row blocks of
 * one expert is cut into tiles of at most 8 blocks, tiles[2 i] = first block, tiles[2 i + 1] =
 * block count, ntiles[0] = count; tiles must hold 2 nb_max ints; nb_max <= 8192. */
int rlu_moe_gemm_tiles(const int* expert_ids, const int* num_post_pad, int nb_max, int* tiles,
                       int* ntiles, hipStream_t stream);

/* Step 2: the same product, row contract and per-step accumulation as
 * r4d_gemm_moe_fp8blk_nt_b16 with sk = 1 (equal to it bit for bit), one workgroup per 128-row x
 * 256-column tile so an expert's weights are read once per tile. max_tiles bounds the device
 * count (the align output's block count). N % 256 == 0. wv = 0 picks the streamed kernel where
 * one is built for K (K = 2560: gate_up of the 2560-wide model, K = 768: its down projection;
 * persistent, one workgroup per CU walking (tile, 256-column strip) items with the weight stream
 * kept in flight across items), else the general tiled kernel at 2 workgroups per CU; wv in
 * 1..16 forces the general kernel at wv workgroups per CU. Every choice gives the same bits.
 * Returns -1 (bad sizes, or a NULL pointer other than topk_weights when mtk > 0), -2 (K % 128
 * or N % 256), -5 (wv outside 0..16). */
int rlu_moe_gemm_fp8blk_tiled(const void* qx, const float* xs, const void* wq, const float* ws,
                              const int* sorted_ids, const int* expert_ids, const int* tiles,
                              const int* ntiles, int max_tiles, const float* topk_weights,
                              void* y, int mtk, int top_k, int K, int N, int wv,
                              hipStream_t stream);

/* No counterpart in the reference (which runs rlu_moe_gemm_fp8blk_tiled's output through the
 * separate SiLU-mul-quant, r4d_mxfp4_moe.py.lru.diff:640-657): gate_up with SiLU-mul-quant in
 * the epilogue. q2 [mtk, N/2] e4m3 and s2 [mtk, N/256] float (group-128 scales) equal
 * rlu_silu_mul_quant(group 128) of rlu_moe_gemm_fp8blk_tiled's bf16 output bit for bit, rows
 * the align does not name untouched; the [mtk, N] bf16 intermediate is never written. Built
 * for K = 2560 and N % 256 == 0: other shapes return -6 before any other check, so a call with
 * mtk = 0 is a capability query (0: built; nothing is launched). Otherwise -1 / -2 as
 * rlu_moe_gemm_fp8blk_tiled. */
int rlu_moe_gemm_fp8blk_tiled_silu_quant(const void* qx, const float* xs, const void* wq,
                                         const float* ws, const int* sorted_ids,
                                         const int* expert_ids, const int* tiles,
                                         const int* ntiles, int max_tiles, void* q2, float* s2,
                                         int mtk, int top_k, int K, int N, hipStream_t stream);

/* No counterpart in the reference (its _gemm_split, r4d_mxfp4_moe.py.lru.diff:584-593, makes
 * one r4d_mxfp4_moe_gemm_into call per align): the prefill GEMMs over both of a layer's
 * aligns in one launch -- align 0 over weights wq0 / ws0 (the resident slots), align
 * 1 over wq1 / ws1 (the full tensor the non-resident experts are read from, device or pinned
 * host memory), both indexing the rows of qx and writing the same output.
 *   rlu_moe_gemm_tiles_split: the tile list of both aligns, align 0's tiles then align 1's with
 *     bit 16 of the block count set; tiles holds 2 (nb_max0 + nb_max1) ints; nb_max <= 8192
 *     each (-1 otherwise, or on a NULL pointer).
 *   rlu_moe_gemm_fp8blk_tiled_split / _split_silu_quant: rlu_moe_gemm_fp8blk_tiled (wv = 0) /
 *     rlu_moe_gemm_fp8blk_tiled_silu_quant on each align, in one launch, equal to the two calls
 *     bit for bit; max_tiles = nb_max0 + nb_max1. Built for the streamed kernel's shapes (K =
 *     2560 or 768 and N % 256 == 0; K = 2560 for _silu_quant): other shapes return -6 before
 *     any other check, so a call with mtk = 0 is a capability query. Every pointer but
 *     topk_weights is required (-1); otherwise -1 / -2 as rlu_moe_gemm_fp8blk_tiled. */
int rlu_moe_gemm_tiles_split(const int* expert_ids0, const int* num_post_pad0, int nb_max0,
                             const int* expert_ids1, const int* num_post_pad1, int nb_max1,
                             int* tiles, int* ntiles, hipStream_t stream);
int rlu_moe_gemm_fp8blk_tiled_split(const void* qx, const float* xs, const void* wq0,
                                    const float* ws0, const int* sorted_ids0,
                                    const int* expert_ids0, const void* wq1, const float* ws1,
                                    const int* sorted_ids1, const int* expert_ids1,
                                    const int* tiles, const int* ntiles, int max_tiles,
                                    const float* topk_weights, void* y, int mtk, int top_k,
                                    int K, int N, hipStream_t stream);
int rlu_moe_gemm_fp8blk_tiled_split_silu_quant(const void* qx, const float* xs, const void* wq0,
                                               const float* ws0, const int* sorted_ids0,
                                               const int* expert_ids0, const void* wq1,
                                               const float* ws1, const int* sorted_ids1,
                                               const int* expert_ids1, const int* tiles,
                                               const int* ntiles, int max_tiles, void* q2,
                                               float* s2, int mtk, int top_k, int K, int N,
                                               hipStream_t stream);

/* No counterpart in the reference (which runs the down GEMM into ic3 and then vLLM's moe_sum,
 * r4d_mxfp4_moe.py.lru.diff:690-696): the decode down projection with moe_sum folded in.
 * out[t] (bf16 [M, N]) = sum over k in k order, in float32, of bf16(down row (t, k) x
 * topk_weights[t, k]) -- the values rlu_moe_gemm_split (sk = 1) writes into ic3 followed by
 * rlu_moe_sum, bit for bit. q2 e4m3 [M top_k, K], s2 float [M top_k, K/128]; topk_ids int32
 * [M, top_k] (every id in [0, E)); table int32 [E] (expert -> slot or -1, the cache state after
 * this step's manager); expert e comes from slot table[e] of w_hot / s_hot when resident, else
 * from w_full / s_full (device or pinned host memory), both in fragment order with 128x128
 * block scales. Every pointer is required (NULL returns -1). Built for K = 768 and top_k = 10
 * (-6 otherwise); N % 128 == 0 (-2 otherwise). Returns -1 / -2 / -6 or a HIP error code. */
int rlu_moe_down_sum(const void* q2, const float* s2, const int* topk_ids,
                     const float* topk_weights, const int* table, const void* w_hot,
                     const float* s_hot, const void* w_full, const float* s_full, void* out,
                     int M, int top_k, int K, int N, int E, hipStream_t stream);

/* No counterpart in the reference (see rlu_moe_down_sum; the reference quantizes the activation
 * in its own launch, kernels/fused_silu_mul_quant.py:75-101): rlu_moe_down_sum from the bf16
 * SiLU-mul activation act [M top_k, K] (rlu_moe_gemm_split_act's output) instead of q2 / s2.
 * Each workgroup quantizes its token's rows per 128-column group exactly as rlu_silu_mul_quant
 * (group 128) does, so out equals rlu_moe_down_sum on that kernel's q2 / s2, bit for bit. Same
 * limits and return codes. */
int rlu_moe_down_sum_act(const void* act, const int* topk_ids, const float* topk_weights,
                         const int* table, const void* w_hot, const float* s_hot,
                         const void* w_full, const float* s_full, void* out, int M, int top_k,
                         int K, int N, int E, hipStream_t stream);

/* No counterpart in the reference. For callers that cannot allocate -- code recorded into a HIP
 * graph, serving loops and harnesses that forbid hipMalloc: rlu_moe_gemm_tiles followed by
 * rlu_moe_gemm_fp8blk_tiled (same kernels, same results bit for bit) with the tile list kept in
 * this library's own per-device scratch array (64 KB of device memory per GPU, held until the
 * process ends) instead of a caller workspace. Nothing is allocated, nothing is freed. nb =
 * the align output's block count (expert_ids holds nb entries), at most 8192 (131072 sorted
 * ids): larger returns -7 and launches nothing. The scratch address is looked up once per
 * device, on the first call with that device current -- make that first call outside graph
 * capture. Every call on one GPU shares its scratch (each call rewrites all it reads), so
 * calls that overlap on one GPU -- concurrent streams, or graphs replayed concurrently -- race;
 * calls in stream order do not. Returns -1 / -2 / -5 as rlu_moe_gemm_fp8blk_tiled, -7 nb >
 * 8192, or a HIP error code. */
int rlu_moe_gemm_fp8blk_tiled_noalloc(const void* qx, const float* xs, const void* wq,
                                      const float* ws, const int* sorted_ids,
                                      const int* expert_ids, const int* num_post_pad, int nb,
                                      const float* topk_weights, void* y, int mtk, int top_k,
                                      int K, int N, int wv, hipStream_t stream);

/* Replaces the closed r4d_gemm_w4a16_nt_m64 behind draft_w4_lmhead_gemm / gemm_w4a16
 * (kernels/draft_w4_lmhead.py:351-403), in this build's gfx950 W4 format:
 *   y [M, N] bf16 = x [M, K] bf16 . (scale * (q - zero))^T, 1 <= M <= 16,
 *   wq [N/16][K/128][64][16] bytes of int4 codes in bf16-MFMA B-operand order, sz
 *   [N/16][K/128][16] u32 = bf16 scale | int16 zero << 16 (w4.pack_w4a16 writes both).
 * wv: workgroups per CU of the persistent grid (0: 2). Returns -1 bad M / K / N / wv,
 * -2 K % 128, N % 32 or K > 4096. */
int rlu_gemm_w4_m16(const void* x, int M, int K, const void* wq, const unsigned* sz, void* y,
                    int N, int wv, hipStream_t stream);

/* Replaces quantize_w4 + pack_w4a16 (kernels/draft_w4_lmhead.py:154-198,228-259), with this
 * build's own quantizer, in the format rlu_gemm_w4_m16 reads: w [N, K] (row stride ld elements,
 * 16-byte aligned rows; dtype 0 bf16, 1 f32, 2 f16) -> wq [n_pad/16][K/128][64][16] codes and
 * sz [n_pad/16][K/128][16] words; rows N..n_pad-1 are packed as zeros. Per (row, 128-column
 * group): 10 clip fractions f of the range (s = bf16(f (hi - lo) / 15)) x the centred integer
 * zero and its two neighbours, codes clamp(rint(w / s) + z, 0, 15), least squared error (summed
 * in a fixed order) wins; a constant group stores s = bf16(|v|). Deterministic: the same bytes on
 * every run. Returns -1 bad sizes or null pointers, -2 K % 128 or n_pad % 16, -3 bad dtype,
 * -4 misaligned w / ld / wq / sz. */
int rlu_pack_w4(const void* w, int dtype, long long ld, int N, int K, int n_pad, void* wq,
                unsigned* sz, hipStream_t stream);

/* Replaces the capture fn of tools/routecap/routecap.py:83-100 (five torch ops per layer
 * there, one launch here; safe to record into a HIP graph). Copies one MoE layer's n routed
 * expert ids (topk_ids, int32) into ring_ids[layer][slot][0..width) as int16, padded with -1.
 * The layer-0 call of a step first advances *ctr and stores it in ring_step[slot];
 * slot = *ctr % ring. ring_ids is [nlayer][ring][width] int16, ring_step [ring] int64
 * (-1 = never written), ctr [1] int64 (0 at start). Returns -1 for n outside [0, width],
 * layer outside [0, nlayer), ring <= 0 or a null buffer. */
int rlu_route_capture(const int* topk_ids, int n, int layer, int nlayer, int ring, int width,
                      short* ring_ids, long long* ring_step, long long* ctr,
                      hipStream_t stream);

/* No counterpart in the reference: a self-test for callers who check the device before use.
 * The prefill SiLU-mul-quant epilogue rounds float32 to bfloat16 with gfx950's one-instruction
 * conversion, where every other kernel uses an integer nearest-even rounding; this runs both
 * over all 2^32 float32 bit patterns and adds the number that differ to *bad (the caller
 * zeroes it). 0 means the kernels' results do not depend on which rounding they use. Returns
 * -1 for a null pointer, else the launch status. */
int rlu_selftest_bf16(unsigned long long* bad, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RLU_H */
