// The grouped fp8 GEMM in the MFMA regime (prefill: tens of rows per expert), same operands,
// row contract and numerics as moe_gemm_k (gemm.hip), tiled for weight reuse:
//
//   tiles_k        from moe_align_block_size output (expert_ids per 16-row block, num_post_pad)
//                  builds the tile list: each run of blocks of one expert is cut into tiles of
//                  at most TMB blocks; a tile is (first block, block count). Blocks of expert -1
//                  make no tile. Given two aligns (a layer's resident and non-resident rows),
//                  it lists the second one's tiles after the first one's, with bit 16 of the
//                  block count set; only the streamed kernel (prefill.hip) reads such a list.
//   tiled_k        one workgroup (8 waves) computes a TMB*16-row x 256-column tile: per 128-deep
//                  K step it stages the tile's activation rows (gathered through sorted_ids) and
//                  the 16 weight strips (fragment order, 2 KB contiguous each) in LDS, double-
//                  buffered with one barrier per step; wave w runs the MFMAs of blocks
//                  w % 2, w % 2 + 2, ... (interleaved, so a short tile still splits evenly) and
//                  strips 4 (w / 2) .. 4 (w / 2) + 3. The expert's weights stream from HBM
//                  once per tile instead of once per 16-row block. Accumulation is acc += mfma * (xs * ws) per step,
//                  as in moe_gemm_k, so both kernels give the same sums up to the association of
//                  the (shared) per-step products -- each output is the same sequence of fma's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "gemm_common.h"
#include "numerics.h"
#include "prefill.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {
namespace tiled {

constexpr int TMB = 8;           // 16-row blocks per tile
constexpr int TBN = 256;         // columns per tile (16 strips of 16)
constexpr int NSTRIP = TBN / 16;
constexpr int NTHR = 512;        // 8 waves: 2 interleaved block sets x 4 column quarters
constexpr int MAXNB = 8192;      // blocks the tile builder handles (L = 131072 sorted ids)
constexpr int TB_THR = 1024;
constexpr int NXCD = 8;          // XCDs of an MI355X

// ---- tile list ---------------------------------------------------------------------------
// The tiles of one align, written from tile index base on with the list number in bit 16 of
// the block count; returns base plus their count (to every thread). se / wtot are the
// workgroup's LDS; the call ends with a barrier, so the next list may rewrite them.
__device__ __forceinline__ int list_tiles(const int* __restrict__ eids, int nb, int list, int base,
                                          int* se, int (*wtot)[TB_THR / WAVE], int* done,
                                          int* __restrict__ tiles) {
  const int t = threadIdx.x, lane = lane_id(), wv = t / WAVE;
  for (int b = t; b < nb; b += TB_THR) se[b] = eids[b];
  __syncthreads();
  const int per = (nb + TB_THR - 1) / TB_THR;
  const int lo = t * per;
  const int hi = lo + per < nb ? lo + per : nb;
  // run start of each block = the last block at or before it where the expert id changes
  int last = -1;
  for (int b = lo; b < hi; ++b)
    if (b == 0 || se[b] != se[b - 1]) last = b;
  // the run start entering this thread's segment: an exclusive max-scan of the segments' last
  // run starts, inside the wave by DPP and over the preceding waves' maxima
  const int wmax = wave_incl_max(last);
  if (lane == WAVE - 1) wtot[0][wv] = wmax;
  __syncthreads();
  int pmax = -1;
  for (int i = 0; i < wv; ++i) pmax = max(pmax, wtot[0][i]);
  int carry = __shfl_up(max(wmax, pmax), 1);
  if (lane == 0) carry = pmax;
  int rs = carry;
  int cnt = 0;
  for (int b = lo; b < hi; ++b) {
    if (b == 0 || se[b] != se[b - 1]) rs = b;
    cnt += se[b] >= 0 && (b - rs) % TMB == 0;
  }
  // this thread's first tile index: an exclusive sum-scan of the tile counts, the same way
  const int wsum = wave_incl_scan(cnt);
  if (lane == WAVE - 1) wtot[1][wv] = wsum;
  __syncthreads();
  int psum = 0;
  for (int i = 0; i < wv; ++i) psum += wtot[1][i];
  int pos = base + psum + wsum - cnt;
  rs = carry;
  for (int b = lo; b < hi; ++b) {
    if (b == 0 || se[b] != se[b - 1]) rs = b;
    if (se[b] >= 0 && (b - rs) % TMB == 0) {
      int n = 1;
      while (n < TMB && b + n < nb && se[b + n] == se[b]) ++n;
      tiles[2 * pos] = b;
      tiles[2 * pos + 1] = n | list << 16;
      ++pos;
    }
  }
  if (t == TB_THR - 1) *done = base + psum + wsum;
  __syncthreads();
  return *done;
}

// The tile list of align 0 (eids0) and, when eids1 is given, of align 1 after it: a tile is
// (first block, block count | align << 16), at most 8 blocks of one expert.
__global__ __launch_bounds__(TB_THR) void tiles_k(const int* __restrict__ eids0,
                                                  const int* __restrict__ npad0, int nb_max0,
                                                  const int* __restrict__ eids1,
                                                  const int* __restrict__ npad1, int nb_max1,
                                                  int* __restrict__ tiles,
                                                  int* __restrict__ ntiles) {
  __shared__ int se[MAXNB];
  __shared__ int wtot[2][TB_THR / WAVE];            // per wave: max of run starts, tile count
  __shared__ int done;
  const int nb0 = min(npad0[0] >> 4, nb_max0);
  int n = list_tiles(eids0, nb0, 0, 0, se, wtot, &done, tiles);
  if (eids1) {
    const int nb1 = min(npad1[0] >> 4, nb_max1);
    n = list_tiles(eids1, nb1, 1, n, se, wtot, &done, tiles);
  }
  if (threadIdx.x == 0) ntiles[0] = n;
}

// ---- the tiled GEMM ------------------------------------------------------------------------
struct Smem {
  v4u a[2][TMB * 128];           // [buf][block][half][lane]: 16 B per lane per half
  v4u b[2][NSTRIP * 128];        // [buf][strip][half][lane]
  float xs[2][TMB * 16];         // activation scale of each tile row at the staged step
  int row[TMB * 16];             // sorted id of each tile row (>= mtk: padding)
};

template <bool TWT>
__global__ __launch_bounds__(NTHR) void tiled_k(const uint8_t* __restrict__ qx,
                                                const float* __restrict__ xs,
                                                const uint8_t* __restrict__ wq,
                                                const float* __restrict__ ws,
                                                const int* __restrict__ sorted_ids,
                                                const int* __restrict__ eids,
                                                const int* __restrict__ tiles,
                                                const int* __restrict__ ntiles_p,
                                                uint16_t* __restrict__ y,
                                                const float* __restrict__ tw, int mtk, int top_k,
                                                int K, int N) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem& S = *reinterpret_cast<Smem*>(smem_raw);
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wv = uniform(t / WAVE);
  const int rh = wv & 1, ch = wv >> 1;             // blocks rh, rh + 2, ...; strips 4 ch ..
  const int r16 = lane & 15, c4 = lane >> 4;
  const int ncb = N / TBN;
  const int nkg = K / 128;
  // XCD-aware order: workgroups are dispatched round-robin over the XCDs, so workgroup b runs
  // on XCD b % 8. Each XCD takes a contiguous range of tiles with all their column blocks, so
  // a tile's gathered activation rows come into one L2 instead of one per column block.
  const int nx = gridDim.x % NXCD == 0 ? NXCD : 1;
  const int xcd = blockIdx.x % nx, per = gridDim.x / nx;
  const int nt = ntiles_p[0];
  const int i0 = (int)((long long)nt * xcd / nx) * ncb;
  const int i1 = (int)((long long)nt * (xcd + 1) / nx) * ncb;

  for (int item = i0 + blockIdx.x / nx; item < i1; item += per) {
    const int ti = item / ncb, cb = item - ti * ncb;
    const int b0 = tiles[2 * ti], nbk = tiles[2 * ti + 1];
    const int e = eids[b0];
    const int n0 = cb * TBN;
    __syncthreads();                                // previous item's epilogue reads of row[]
    if (t < TMB * 16) {
      const int blk = t >> 4;
      S.row[t] = blk < nbk ? sorted_ids[(b0 + blk) * 16 + (t & 15)] : mtk;
    }
    __syncthreads();
    const uint8_t* wbase = wq + ((size_t)e * N + n0) * K;
    // this wave's strips 4 ch .. 4 ch + 3 lie in the 128-column scale block n0 / 128 + ch / 2
    const float* wsr = ws + ((size_t)e * (N / 128) + n0 / 128 + (ch >> 1)) * nkg;

    // staging: unit u (16 B) of A = (block u >> 7, half (u >> 6) & 1, lane u & 63), 2 per
    // thread; of B = (strip u >> 7, the strip's 2 KB in fragment order), 4 per thread
    constexpr int QA = TMB * 128 / NTHR, QB = NSTRIP * 128 / NTHR;
    v4u ra[QA], rb[QB];
    float rx = 0.f;
    auto load = [&](int kb) {
#pragma unroll
      for (int q = 0; q < QA; ++q) {
        const int u = t + NTHR * q;
        const int blk = u >> 7, l = u & 63, h = (u >> 6) & 1;
        const int so = S.row[blk * 16 + (l & 15)];
        ra[q] = v4u{0u, 0u, 0u, 0u};
        if (so < mtk)
          ra[q] = *reinterpret_cast<const v4u*>(qx + (size_t)(so / top_k) * K + kb * 128 +
                                                64 * h + 16 * (l >> 4));
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int u = t + NTHR * q;
        rb[q] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(
            wbase + (size_t)(u >> 7) * 16 * K + (size_t)kb * 2048 + (u & 127) * 16));
      }
      if (t < TMB * 16) {
        const int so = S.row[t];
        rx = so < mtk ? xs[(size_t)(so / top_k) * nkg + kb] : 0.f;
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int q = 0; q < QA; ++q) S.a[buf][t + NTHR * q] = ra[q];
#pragma unroll
      for (int q = 0; q < QB; ++q) S.b[buf][t + NTHR * q] = rb[q];
      if (t < TMB * 16) S.xs[buf][t] = rx;
    };

    v4f acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[j][s] = v4f{0.f, 0.f, 0.f, 0.f};

    load(0);
    store(0);
    __syncthreads();
    for (int kb = 0; kb < nkg; ++kb) {
      const int buf = kb & 1;
      if (kb + 1 < nkg) load(kb + 1);
      const float wsv = wsr[kb];
      v8i bf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        bf[s] = pack8(S.b[buf][(4 * ch + s) * 128 + lane], S.b[buf][(4 * ch + s) * 128 + 64 + lane]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int blk = rh + 2 * j;
        if (blk < nbk) {
          const v8i af = pack8(S.a[buf][blk * 128 + lane], S.a[buf][blk * 128 + 64 + lane]);
          const v4f xr = *reinterpret_cast<const v4f*>(&S.xs[buf][blk * 16 + 4 * c4]);
          v4f f;
#pragma unroll
          for (int i = 0; i < 4; ++i) f[i] = xr[i] * wsv;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const v4f d = mfma_f8(af, bf[s]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[j][s][i] = fmaf(d[i], f[i], acc[j][s][i]);
          }
        }
      }
      if (kb + 1 < nkg) store(buf ^ 1);
      __syncthreads();
    }
    // epilogue: rows this lane holds, routed weight, bf16, live rows only
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = rh + 2 * j;
      if (blk < nbk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int so = S.row[blk * 16 + 4 * c4 + i];
          if (so < mtk) {
            const float wgt = TWT ? tw[so] : 1.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s)
              y[(size_t)so * N + n0 + (4 * ch + s) * 16 + r16] = f32_to_bf16(acc[j][s][i] * wgt);
          }
        }
      }
    }
  }
}

// ---- the no-allocation entry's workspace -----------------------------------------------------
// The tile list of one call: 2 ints per tile (at most one tile per block) and the count, for up
// to MAXNB blocks -- 64 KB per GPU, held until the process ends. Host code never uses the
// array's name as an address: each device's address comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that pointer reaches the kernels.
constexpr int SCRATCH_INTS = 2 * MAXNB + 64;
static __device__ __align__(256) int scratch[SCRATCH_INTS];

constexpr int MAXDEV = 64;
static std::mutex scratch_mu;
static int* scratch_dev[MAXDEV];

// this device's scratch address; 0 or a HIP error code
static int scratch_ptr(int** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAXDEV) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    scratch_dev[dev] = static_cast<int*>(p);
  }
  *out = scratch_dev[dev];
  return 0;
}

static int check_gemm_args(int mtk, int top_k, int K, int N, int max_tiles, int wv) {
  if (mtk < 0 || top_k < 1 || K <= 0 || N <= 0 || max_tiles <= 0) return -1;
  if (K % 128 || N % TBN) return -2;
  if (wv < 0 || wv > 16) return -5;
  return 0;
}

// The streamed kernel (prefill.hip) where K and N have a built configuration, tiled_k
// otherwise; both give the same bits.
static void launch_tiled(const void* qx, const float* xs, const void* wq, const float* ws,
                         const int* sorted_ids, const int* expert_ids, const int* tiles,
                         const int* ntiles, int max_tiles, const float* topk_weights, void* y,
                         int mtk, int top_k, int K, int N, int wv, hipStream_t stream) {
  if (wv == 0 && rlu::launch_prefill_stream(qx, xs, wq, ws, sorted_ids, expert_ids, nullptr,
                                            tiles, ntiles, max_tiles, topk_weights, y, mtk,
                                            top_k, K, N, stream) == 0)
    return;
  const int items = max_tiles * (N / TBN);
  int grid = rlu::device_cus() * (wv ? wv : 2);
  if (grid > items) grid = items;
  if (grid >= NXCD) grid -= grid % NXCD;           // whole XCD rounds (see tiled_k)
  const size_t lds = sizeof(Smem);
  if (topk_weights)
    hipLaunchKernelGGL(tiled_k<true>, dim3(grid), dim3(NTHR), lds, stream, (const uint8_t*)qx,
                       xs, (const uint8_t*)wq, ws, sorted_ids, expert_ids, tiles, ntiles,
                       (uint16_t*)y, topk_weights, mtk, top_k, K, N);
  else
    hipLaunchKernelGGL(tiled_k<false>, dim3(grid), dim3(NTHR), lds, stream, (const uint8_t*)qx,
                       xs, (const uint8_t*)wq, ws, sorted_ids, expert_ids, tiles, ntiles,
                       (uint16_t*)y, nullptr, mtk, top_k, K, N);
}

}  // namespace tiled
}  // namespace rlu

extern "C" {

int rlu_moe_gemm_tiles(const int* expert_ids, const int* num_post_pad, int nb_max, int* tiles,
                       int* ntiles, hipStream_t stream) {
  using namespace rlu::tiled;
  if (nb_max <= 0 || nb_max > MAXNB || !expert_ids || !num_post_pad || !tiles || !ntiles)
    return -1;
  hipLaunchKernelGGL(tiles_k, dim3(1), dim3(TB_THR), 0, stream, expert_ids, num_post_pad, nb_max,
                     nullptr, nullptr, 0, tiles, ntiles);
  return (int)hipGetLastError();
}

int rlu_moe_gemm_fp8blk_tiled(const void* qx, const float* xs, const void* wq, const float* ws,
                              const int* sorted_ids, const int* expert_ids, const int* tiles,
                              const int* ntiles, int max_tiles, const float* topk_weights,
                              void* y, int mtk, int top_k, int K, int N, int wv,
                              hipStream_t stream) {
  using namespace rlu::tiled;
  const int rc = check_gemm_args(mtk, top_k, K, N, max_tiles, wv);
  if (rc) return rc;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq || !ws || !sorted_ids || !expert_ids || !tiles || !ntiles || !y)
    return -1;
  launch_tiled(qx, xs, wq, ws, sorted_ids, expert_ids, tiles, ntiles, max_tiles, topk_weights, y,
               mtk, top_k, K, N, wv, stream);
  return (int)hipGetLastError();
}

// rlu_moe_gemm_tiles + rlu_moe_gemm_fp8blk_tiled with the tile list in this library's
// per-device scratch array instead of a caller workspace: nothing is allocated.
int rlu_moe_gemm_fp8blk_tiled_noalloc(const void* qx, const float* xs, const void* wq,
                                      const float* ws, const int* sorted_ids,
                                      const int* expert_ids, const int* num_post_pad, int nb,
                                      const float* topk_weights, void* y, int mtk, int top_k,
                                      int K, int N, int wv, hipStream_t stream) {
  using namespace rlu::tiled;
  if (!expert_ids || !num_post_pad) return -1;
  const int rc = check_gemm_args(mtk, top_k, K, N, nb, wv);
  if (rc) return rc;
  if (nb > MAXNB) return -7;                        // beyond the scratch tile list
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq || !ws || !sorted_ids || !y) return -1;
  int* ws_tiles = nullptr;
  const int e = scratch_ptr(&ws_tiles);
  if (e) return e;
  int* ws_count = ws_tiles + 2 * MAXNB;
  hipLaunchKernelGGL(tiles_k, dim3(1), dim3(TB_THR), 0, stream, expert_ids, num_post_pad, nb,
                     nullptr, nullptr, 0, ws_tiles, ws_count);
  launch_tiled(qx, xs, wq, ws, sorted_ids, expert_ids, ws_tiles, ws_count, nb, topk_weights, y,
               mtk, top_k, K, N, wv, stream);
  return (int)hipGetLastError();
}

// The gate_up GEMM with SiLU-mul-quant fused into its epilogue (prefill.hip, ACT): q2 / s2
// equal rlu_silu_mul_quant (group 128) of rlu_moe_gemm_fp8blk_tiled's bf16 output bit for bit,
// without that [mtk, N] output. Built for K = 2560 (gate_up of the 2560-wide model) and N % 256
// == 0; other shapes return -6 before anything else is checked, so a call with mtk = 0 is a
// capability query (0: built, nothing launched).
int rlu_moe_gemm_fp8blk_tiled_silu_quant(const void* qx, const float* xs, const void* wq,
                                         const float* ws, const int* sorted_ids,
                                         const int* expert_ids, const int* tiles,
                                         const int* ntiles, int max_tiles, void* q2, float* s2,
                                         int mtk, int top_k, int K, int N,
                                         hipStream_t stream) {
  using namespace rlu::tiled;
  if (!rlu::prefill_stream_act_built(K, N)) return -6;
  const int rc = check_gemm_args(mtk, top_k, K, N, max_tiles, 0);
  if (rc) return rc;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq || !ws || !sorted_ids || !expert_ids || !tiles || !ntiles || !q2 || !s2)
    return -1;
  if (rlu::launch_prefill_stream_act(qx, xs, wq, ws, sorted_ids, expert_ids, nullptr, tiles,
                                     ntiles, max_tiles, q2, s2, mtk, top_k, K, N, stream))
    return -6;
  return (int)hipGetLastError();
}

// ---- two aligns in one launch (a layer's resident slots and its non-resident experts) ------

// The tile list of both aligns: align 0's tiles, then align 1's with bit 16 of the block
// count set. tiles holds 2 (nb_max0 + nb_max1) ints.
int rlu_moe_gemm_tiles_split(const int* expert_ids0, const int* num_post_pad0, int nb_max0,
                             const int* expert_ids1, const int* num_post_pad1, int nb_max1,
                             int* tiles, int* ntiles, hipStream_t stream) {
  using namespace rlu::tiled;
  if (nb_max0 <= 0 || nb_max0 > MAXNB || nb_max1 <= 0 || nb_max1 > MAXNB || !expert_ids0 ||
      !num_post_pad0 || !expert_ids1 || !num_post_pad1 || !tiles || !ntiles)
    return -1;
  hipLaunchKernelGGL(tiles_k, dim3(1), dim3(TB_THR), 0, stream, expert_ids0, num_post_pad0,
                     nb_max0, expert_ids1, num_post_pad1, nb_max1, tiles, ntiles);
  return (int)hipGetLastError();
}

// rlu_moe_gemm_fp8blk_tiled over align 0 (weights wq0 / ws0) and align 1 (wq1 / ws1) in one
// launch of the streamed kernel, from rlu_moe_gemm_tiles_split's list; the output equals the
// two calls bit for bit. Built for the streamed kernel's shapes (K 2560 or 768, N % 256 == 0):
// other shapes return -6 before anything else is checked (mtk = 0: a capability query).
int rlu_moe_gemm_fp8blk_tiled_split(const void* qx, const float* xs, const void* wq0,
                                    const float* ws0, const int* sorted_ids0,
                                    const int* expert_ids0, const void* wq1, const float* ws1,
                                    const int* sorted_ids1, const int* expert_ids1,
                                    const int* tiles, const int* ntiles, int max_tiles,
                                    const float* topk_weights, void* y, int mtk, int top_k,
                                    int K, int N, hipStream_t stream) {
  using namespace rlu::tiled;
  if (!rlu::prefill_stream_built(K, N)) return -6;
  const int rc = check_gemm_args(mtk, top_k, K, N, max_tiles, 0);
  if (rc) return rc;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq0 || !ws0 || !sorted_ids0 || !expert_ids0 || !wq1 || !ws1 ||
      !sorted_ids1 || !expert_ids1 || !tiles || !ntiles || !y)
    return -1;
  const rlu::PfSecond second{wq1, ws1, sorted_ids1, expert_ids1};
  if (rlu::launch_prefill_stream(qx, xs, wq0, ws0, sorted_ids0, expert_ids0, &second, tiles,
                                 ntiles, max_tiles, topk_weights, y, mtk, top_k, K, N, stream))
    return -6;
  return (int)hipGetLastError();
}

// rlu_moe_gemm_fp8blk_tiled_silu_quant over two aligns in one launch, as
// rlu_moe_gemm_fp8blk_tiled_split; K = 2560 and N % 256 == 0, else -6 (mtk = 0: a query).
int rlu_moe_gemm_fp8blk_tiled_split_silu_quant(const void* qx, const float* xs, const void* wq0,
                                               const float* ws0, const int* sorted_ids0,
                                               const int* expert_ids0, const void* wq1,
                                               const float* ws1, const int* sorted_ids1,
                                               const int* expert_ids1, const int* tiles,
                                               const int* ntiles, int max_tiles, void* q2,
                                               float* s2, int mtk, int top_k, int K, int N,
                                               hipStream_t stream) {
  using namespace rlu::tiled;
  if (!rlu::prefill_stream_act_built(K, N)) return -6;
  const int rc = check_gemm_args(mtk, top_k, K, N, max_tiles, 0);
  if (rc) return rc;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq0 || !ws0 || !sorted_ids0 || !expert_ids0 || !wq1 || !ws1 ||
      !sorted_ids1 || !expert_ids1 || !tiles || !ntiles || !q2 || !s2)
    return -1;
  const rlu::PfSecond second{wq1, ws1, sorted_ids1, expert_ids1};
  if (rlu::launch_prefill_stream_act(qx, xs, wq0, ws0, sorted_ids0, expert_ids0, &second, tiles,
                                     ntiles, max_tiles, q2, s2, mtk, top_k, K, N, stream))
    return -6;
  return (int)hipGetLastError();
}

}  // extern "C"
