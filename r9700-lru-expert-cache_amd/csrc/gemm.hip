// fp8 e4m3 x fp8 e4m3 GEMMs with 128x128 float32 weight-block scales and per-(row, 128-column)
// activation scales, on gfx950 matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4 with unit
// E8M0 scales; the float32 block scales are applied per 128-deep K step in the accumulator).
//
//   moe_gemm_k<NPW, SKW, DENSE=false>  the grouped expert GEMM of the MoE path: rows come from
//       moe_align_block_size output (sorted_ids / expert_ids / num_post_pad, block 16), the
//       contract of the reference's r4d_mxfp4_moe_gemm_into (patches/.../r4d_mxfp4_moe.py.lru
//       .diff:363-395, probed in tests/k1/moe_ref_harness.py:282-321): a row id >= mtk is
//       padding and is skipped, an expert id of -1 skips its block, num_post_pad is read on
//       the device, only rows named in sorted_ids are written, and an optional routed weight
//       tw[row] scales the output (GEMM2's epilogue).
//   moe_gemm_k<NPW, SKW, DENSE=true>   y[M, N] = A[M, K] W[N, K]^T for M <= 16: the fp8
//       lm_head GEMV (kernels/fp8_target_lmhead.py:70-74).
//
// Weights are stored once, at load time, in gfx950 MFMA fragment order (shuffle_k below; the
// reference does the same for its gfx1201 WMMA kernels, kernels/fp8_target_lmhead.py:44-66):
// byte (n, k), n = 16 nt + r, k = 128 kb + 64 h + 16 c + j, sits at
//   ((nt * (K / 128) + kb) * 2 + h) * 1024 + (16 c + r) * 16 + j,
// so lane l = 16 c + r of a wave reads its 16 bytes of one 128-deep step of a 16-row strip at
// l * 16: every weight load instruction of a wave is 1 KB contiguous, and a strip's K range is
// one contiguous run. Activations stay row-major (they are gathered by sorted_ids).
//
// Work split: an item is (one 16-row block, one tile of 16 * NPW columns); SKW waves of a
// workgroup split its K range (item_mma in gemm_item.h) and add their partial sums in LDS in
// split order, so a given SKW is deterministic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "gemm_item.h"
#include "numerics.h"
#include "quant_row.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {

constexpr int GWV = 4;      // waves per workgroup
constexpr int QIN_MAXG = 6;   // 128-column groups of the activation MODE 2 reads (K <= 768):
                              // its rows' loads stay live across the first weight steps
static_assert(PMS >= QIN_MAXG, "item_mma_pm covers every K MODE 2 takes");
// MODE 2's shape: workgroups of 8 waves, 2 strips (32 columns) per wave, so a workgroup covers
// 256 columns of one block and quantizes the block's rows once for them; the wave's two strips
// stream through a ring of 3 pair-steps (item_mma_pm). 127 registers: four waves per SIMD, so
// both workgroups a CU can hold are resident and every live workgroup of a decode launch runs
// at once. Measured on the 52-layer B=4 step against 4 waves x 4 strips with a 6-deep ring
// (228 registers, two waves per SIMD): 3.305-3.308 against 3.348-3.352 ms; 4 waves x 2 strips:
// 3.417-3.421; 8 waves x 2 strips with a 6-deep ring (three waves per SIMD, one workgroup per
// CU): 3.432-3.441.
constexpr int QIN_NPW = 2;    // strips per wave in MODE 2
constexpr int QIN_RING = 3;   // pair-steps in MODE 2's weight ring
constexpr int QIN_G = 8;      // waves per workgroup in MODE 2 (items of one block)

// MODE 0: y [mtk, N] = the GEMM (routed weights optional).
// MODE 1 (gate_up with its activation, NPW / 2 gate + NPW / 2 up strips per item): y
// [mtk, N / 2] = bf16(silu(g) x u) of the GEMM's bf16 outputs g (column c) and u (column
// N / 2 + c), computed as silu_mul_quant_k computes them from the [mtk, N] output.
// MODE 2 (down from the activation, SKW = 1, the G items of a workgroup in one block): qx is
// the bf16 activation [mtk, K] and xs is not read; the workgroup first quantizes its block's 16
// rows per 128-column group exactly as silu_mul_quant_k does (same amax, scale and rounding)
// into LDS, which the MFMAs then read, so the output equals MODE 0 on that kernel's q2 / s2.
template <int NPW, int SKW, bool DENSE, int MODE = 0, int G = GWV>
__global__ __launch_bounds__(G * WAVE) void moe_gemm_k(
    const uint8_t* __restrict__ qx, const float* __restrict__ xs, WSet s0, WSet s1, int nsets,
    uint16_t* __restrict__ y, const float* __restrict__ tw, int mtk, int top_k, int K, int N) {
  constexpr bool PAIR = MODE == 1, AL = MODE == 2;
  constexpr int NH = PAIR ? 2 : 1;                  // weight-scale rows per item
  constexpr int IPG = G / SKW;                      // items per workgroup pass
  extern __shared__ float lds[];                    // [G][nsteps][NH][16] scales, then
                                                    // partials (SKW > 1) or the A rows (AL)
  const int lane = lane_id();
  const int wv = uniform(threadIdx.x / WAVE);       // wave-uniform: item metadata in SGPRs
  const int sub = wv / SKW, ks = wv % SKW;
  const int nsteps = AL ? PMS : item_steps<NPW, SKW>(K);   // AL: item_mma_pm's fixed steps
  const int NT = PAIR ? 8 * NPW : 16 * NPW;         // output columns per item
  const int ntiles = (PAIR ? N / 2 : N) / NT;
  // both lists' num_post_pad in one round trip (a launch with one list passes it twice)
  const int np0 = DENSE ? 16 : s0.npad[0];
  const int np1 = DENSE ? 0 : s1.npad[0];
  const int nb0 = np0 >> 4;
  const int nb1 = (DENSE || nsets < 2) ? 0 : (np1 >> 4);
  const int nitems = (nb0 + nb1) * ntiles;
  const int ngroups = (nitems + IPG - 1) / IPG;
  float* sx = lds + (size_t)wv * nsteps * 16 * NH;
  float* red = lds + (size_t)G * nsteps * 16 * NH;  // [2][G][NPW * 4][64]
  const int als = K + 16;                           // AL: LDS row stride of the A rows
  uint8_t* alds = reinterpret_cast<uint8_t*>(red);  // AL: [16][als] e4m3, then [16][K/128] f32
  float* xsl = reinterpret_cast<float*>(alds + 16 * als);
  const int r16 = lane & 15;
  int parity = 0;

  // MODE 2 takes its item groups in an XCD-aware order. Workgroup g runs on XCD g % 8 (the
  // dispatcher deals workgroups round-robin over the 8 XCDs), so XCD x gets the contiguous run
  // [x per, (x + 1) per) of the groups: the ten groups of one block then share one L2, which
  // fetches the block's activation rows once instead of once per XCD (the launch rounds its
  // grid up to a multiple of 8 workgroups; indices past ngroups are dead).
  const int per = (ngroups + 7) >> 3;
  const int nloop = AL ? 8 * per : ngroups;
  for (int grp = blockIdx.x; grp < nloop; grp += gridDim.x, parity ^= 1) {
    const int lg = AL ? (grp & 7) * per + (grp >> 3) : grp;
    const int item = lg * IPG + sub;
    bool live = item < nitems;
    int b = live ? item / ntiles : 0;
    const int n0 = live ? (item - b * ntiles) * NT : 0;
    const bool second = b >= nb0;
    if (second) b -= nb0;
    const uint8_t* __restrict__ wq = second ? s1.wq : s0.wq;
    const float* __restrict__ ws = second ? s1.ws : s0.ws;
    const int* __restrict__ sids = second ? s1.sorted_ids : s0.sorted_ids;
    // the block's expert id and its 16 row ids in one round trip (b is 0 for a dead item, and
    // every sorted-id array holds at least one block): this lane's A row (operand layout) and
    // the four output rows it holds (D layout: rows 4 c4 + i, column r16)
    int so = DENSE ? r16 : mtk;
    int sod[4] = {mtk, mtk, mtk, mtk};
    if (!DENSE) {
      int ids[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) ids[i] = sids[b * 16 + i];
#pragma unroll
      for (int i = 0; i < 16; ++i) so = r16 == i ? ids[i] : so;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int v = ids[i];
#pragma unroll
        for (int c = 1; c < 4; ++c) v = (lane >> 4) == c ? ids[4 * c + i] : v;
        sod[i] = v;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) sod[i] = 4 * (lane >> 4) + i;
    }
    const int eid = (DENSE || !live) ? 0 : (second ? s1.expert_ids : s0.expert_ids)[b];
    live = live && eid >= 0;
    v4f acc[NPW];
#pragma unroll
    for (int s = 0; s < NPW; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
    float twv[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (AL) {
      // MODE 2: the G items of the workgroup share block b (ntiles % G == 0, no item past
      // nitems), so the workgroup quantizes the block's 16 rows into LDS together -- 16-lane
      // group q takes row q % 16 and every (G / 4)-th 128-column group from q / 16 on, lane
      // l16 columns [8 l16, 8 l16 + 8) of each. The rows' loads go out before the item's first
      // weight steps (pre), so that waiting for them does not wait for the weights (the
      // counter retires in order); the quant runs while the weights are in flight (pro), then
      // one workgroup barrier
      constexpr int GS = G / 4;                     // 128-column group stride of a 16-lane group
      static_assert(G % 4 == 0 && SKW == 1, "16-lane groups cover the block's 16 rows");
      const int q16 = (int)threadIdx.x / 16, r = q16 % 16, g0 = q16 / 16;
      const int l16 = lane & 15, ng = K / 128;
      const int sr = sids[b * 16 + r];
      const bool ok = sr < mtk;
      const uint16_t* src =
          reinterpret_cast<const uint16_t*>(qx) + (size_t)(ok ? sr : 0) * K + 8 * l16;
      constexpr int NP = (QIN_MAXG + GS - 1) / GS;
      uint4 raw[NP];
      auto pre = [&]() __attribute__((always_inline)) {   // the rows' loads, ahead of weights
        if (eid >= 0) {
#pragma unroll
          for (int p = 0; p < NP; ++p)              // padding rows are zeros, not loaded
            raw[p] = (ok && g0 + p * GS < ng)
                         ? *reinterpret_cast<const uint4*>(src + (g0 + p * GS) * 128)
                         : uint4{0u, 0u, 0u, 0u};
        }
      };
      auto pro = [&]() __attribute__((always_inline)) {
        if (eid >= 0) {
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const int g = g0 + p * GS;
            if (g < ng) {
              float v[8];
              unpack8_bf16(raw[p], v);
              uint32_t m = 0;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                v[j] = ok ? v[j] : 0.f;
                m = max(m, abs_bits(v[j]));
              }
              const float sc = scale_of(row_max_u32(m));
              *reinterpret_cast<uint2*>(alds + r * als + g * 128 + 8 * l16) = quant8(v, sc);
              if (l16 == 0) xsl[r * ng + g] = sc;
            }
          }
        }
        lds_barrier();
      };
      static_assert(!AL || NPW % 2 == 0, "MODE 2 runs item_mma_pm: strips in pairs");
      if (live)
        item_mma_pm<NPW / 2, QIN_RING>(wq, ws, so, eid, n0, tw, mtk, K, N, sx, acc, sod, twv,
                                       alds, als, xsl, pro, pre);
      else {
        pre();
        pro();
      }
    } else if (live) {
      item_mma<NPW, SKW, DENSE, ring_of(NPW), PAIR, AL>(qx, xs, wq, ws, so, eid, n0, tw, mtk,
                                                        top_k, K, N, ks, sx, acc, sod, twv);
    }
    if (SKW > 1)
      splitk_reduce<NPW, SKW>(acc, red + (size_t)parity * G * NPW * 4 * WAVE, wv, ks);
    if (live && ks == 0) {
      // epilogue: rows this lane holds, routed weight, bf16, only live rows
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = sod[i];
        if (o < mtk) {
          if constexpr (PAIR) {
#pragma unroll
            for (int s = 0; s < NPW / 2; ++s) {
              const float g = bf16_to_f32(f32_to_bf16(acc[s][i] * twv[i]));
              const float u = bf16_to_f32(f32_to_bf16(acc[s + NPW / 2][i] * twv[i]));
              y[(size_t)o * (N / 2) + n0 + s * 16 + r16] =
                  f32_to_bf16(__fmul_rn(silu_bf16(g), u));
            }
          } else {
#pragma unroll
            for (int s = 0; s < NPW; ++s)
              y[(size_t)o * N + n0 + s * 16 + r16] = f32_to_bf16(acc[s][i] * twv[i]);
          }
        }
      }
    }
    if constexpr (AL)
      lds_barrier();                                // the A rows are rewritten by the next group
    else
      wave_lds_sync();                              // sx is rewritten by the next item
  }
}

// Row-major [rows, K] e4m3 -> fragment order; one thread per 16-byte unit of the output.
__global__ __launch_bounds__(256) void shuffle_k(const v4u* __restrict__ w, v4u* __restrict__ out,
                                                 size_t units, int K) {
  const size_t u = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int l = (int)(u & 63), h = (int)((u >> 6) & 1);
  const size_t t = u >> 7;                         // 16-row x 128-deep tile
  const int kb_n = K / 128;
  const size_t nt = t / kb_n;
  const int kb = (int)(t - nt * kb_n);
  const size_t row = nt * 16 + (l & 15);
  const size_t col = (size_t)kb * 128 + h * 64 + (l >> 4) * 16;
  out[u] = w[(row * K + col) / 16];
}

// K / 128 split over the waves of a workgroup: the largest of 4, 2, 1 that divides it.
static int pick_sk(int nkg, int sk) {
  if (sk > 0) return sk;
  if (nkg % 4 == 0) return 4;
  if (nkg % 2 == 0) return 2;
  return 1;
}

// MODE 1 is built for npw 2 (any sk), MODE 2 for npw QIN_NPW with sk 1 (-6 / -4 otherwise).
template <bool DENSE, int MODE = 0>
int launch(int npw, int sk, int grid, hipStream_t st, const uint8_t* qx, const float* xs,
           WSet s0, WSet s1, int nsets, uint16_t* y, const float* tw, int mtk, int top_k,
           int K, int N) {
  const int kpw = K / 128 / sk;
  const int d = ring_of(npw);
  const int nsteps = MODE == 2 ? PMS : (kpw + d - 1) / d * d;
  constexpr int G = MODE == 2 ? QIN_G : GWV;
  const size_t tail = MODE == 2 ? (size_t)16 * (K + 16) + (size_t)16 * (K / 128) * 4
                                : (sk > 1 ? 2 * (size_t)G * npw * 4 * WAVE * 4 : 0);
  const size_t lds = (size_t)G * nsteps * 16 * (MODE == 1 ? 2 : 1) * 4 + tail;
#define RLU_L(P, SK)                                                                          \
  hipLaunchKernelGGL((moe_gemm_k<P, SK, DENSE, MODE, G>), dim3(grid), dim3(G * WAVE), lds,    \
                     st, qx, xs, s0, s1, nsets, y, tw, mtk, top_k, K, N)
#define RLU_SK(P)                   \
  switch (sk) {                     \
    case 1: RLU_L(P, 1); break;     \
    case 2: RLU_L(P, 2); break;     \
    case 4: RLU_L(P, 4); break;     \
    default: return -4;             \
  }
  if constexpr (MODE == 1) {
    if (npw != 2) return -6;
    RLU_SK(2);
  } else if constexpr (MODE == 2) {
    if (npw != QIN_NPW) return -6;
    if (sk != 1) return -4;
    RLU_L(QIN_NPW, 1);
  } else {
    switch (npw) {
      case 1: RLU_SK(1); break;
      case 2: RLU_SK(2); break;
      case 4: RLU_SK(4); break;
      case 8: RLU_SK(8); break;
      default: return -6;
    }
  }
#undef RLU_SK
#undef RLU_L
  return (int)hipGetLastError();
}


// wv = 0: one workgroup per item group (the hardware dispatcher balances the CUs); otherwise a
// persistent grid of wv workgroups per CU
static int grid_for(int items, int sk, int wv) {
  const int ipg = GWV / sk;
  const int need = (items + ipg - 1) / ipg;
  const int g = wv ? device_cus() * wv : need;
  return g < need ? g : (need > 0 ? need : 1);
}

static bool bad_npw(int npw) { return npw != 1 && npw != 2 && npw != 4 && npw != 8; }

// sk valid for K: supported, divides K / 128, at most MAXKPW steps per wave
static bool bad_sk(int K, int sk) {
  const int nkg = K / 128;
  return (sk != 1 && sk != 2 && sk != 4) || nkg % sk || nkg / sk > MAXKPW;
}

}  // namespace rlu

extern "C" {

// Grouped GEMM with the reference op's argument order (r4d_mxfp4_moe.py.lru.diff:389-395):
// y[mtk, N] bf16 rows named by sorted_ids[0:npad] <- qx[mtk/top_k, K] e4m3 (scales xs[., K/128])
// x wq[E, N, K] e4m3 in fragment order (block scales ws[E, N/128, K/128]); wref is not used.
int r4d_gemm_moe_fp8blk_nt_b16(const void* qx, const float* xs, const void* wq,
                               const float* ws, const void* wref, void* y,
                               const int* sorted_ids, const int* expert_ids,
                               const int* num_post_pad, const float* topk_weights, int em,
                               int mtk, int top_k, int K, int N, int wv, int sk, int npw,
                               hipStream_t stream) {
  (void)wref;
  if (em < 1 || mtk < 0 || top_k < 1 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (rlu::bad_npw(npw)) return -6;
  sk = rlu::pick_sk(K / 128, sk);
  if (rlu::bad_sk(K, sk)) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq || !ws || !y || !sorted_ids || !expert_ids || !num_post_pad) return -1;
  const int nb = (em + 15) / 16;
  const int items = nb * (N / (16 * npw));
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)wq, ws, sorted_ids, expert_ids, num_post_pad};
  return rlu::launch<false>(npw, sk, grid, stream, (const uint8_t*)qx, xs, s0, s0, 1,
                            (uint16_t*)y, topk_weights, mtk, top_k, K, N);
}

// The hot/cold split of one GEMM (the two r4d_mxfp4_moe_gemm_into calls of _gemm_split,
// r4d_mxfp4_moe.py.lru.diff:584-592) in one launch: block list 1 (sorted_hot / eids_hot /
// npad_hot) against the slot buffers wq_hot / ws_hot, block list 2 against the full expert
// tensor wq / ws (device or pinned host memory). Both lists have em entries. Same checks and
// codes as r4d_gemm_moe_fp8blk_nt_b16.
int rlu_moe_gemm_split(const void* qx, const float* xs, const void* wq_hot, const float* ws_hot,
                       const int* sorted_hot, const int* eids_hot, const int* npad_hot,
                       const void* wq, const float* ws, const int* sorted_cold,
                       const int* eids_cold, const int* npad_cold, const float* topk_weights,
                       void* y, int em, int mtk, int top_k, int K, int N, int wv, int sk,
                       int npw, hipStream_t stream) {
  if (em < 1 || mtk < 0 || top_k < 1 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (rlu::bad_npw(npw)) return -6;
  sk = rlu::pick_sk(K / 128, sk);
  if (rlu::bad_sk(K, sk)) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
  if (!qx || !xs || !wq_hot || !ws_hot || !sorted_hot || !eids_hot || !npad_hot || !wq || !ws ||
      !sorted_cold || !eids_cold || !npad_cold || !y)
    return -1;
  // live blocks are numbered densely (hot list, then cold list) and each holds at least one of
  // the mtk rows, so there are at most min(2 ceil(em / 16), mtk) of them: the grid covers no
  // more (workgroups past the live ones still cost a dispatch and a scalar load each)
  const int nb = (em + 15) / 16;
  const int nblive = 2 * nb < mtk ? 2 * nb : mtk;
  const int items = nblive * (N / (16 * npw));
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)wq_hot, ws_hot, sorted_hot, eids_hot, npad_hot};
  const rlu::WSet s1{(const uint8_t*)wq, ws, sorted_cold, eids_cold, npad_cold};
  return rlu::launch<false>(npw, sk, grid, stream, (const uint8_t*)qx, xs, s0, s1, 2,
                            (uint16_t*)y, topk_weights, mtk, top_k, K, N);
}

// gate_up of the split GEMM with SiLU-mul in its epilogue: act [mtk, N / 2] bf16 =
// bf16(silu(g) x u) of the GEMM's bf16 outputs g = columns [0, N / 2), u = [N / 2, N), the
// activation silu_mul_quant computes from rlu_moe_gemm_split's output, bit for bit, on the
// rows the aligns name (no [mtk, N] intermediate, and no activation launch). wq == NULL runs
// the hot list alone. npw is 2 (two strips: a gate column block and its up block); N % 256.
int rlu_moe_gemm_split_act(const void* qx, const float* xs, const void* wq_hot,
                           const float* ws_hot, const int* sorted_hot, const int* eids_hot,
                           const int* npad_hot, const void* wq, const float* ws,
                           const int* sorted_cold, const int* eids_cold, const int* npad_cold,
                           void* act, int em, int mtk, int top_k, int K, int N, int wv, int sk,
                           hipStream_t stream) {
  if (em < 1 || mtk < 0 || top_k < 1 || K <= 0 || N <= 0) return -1;
  if (!qx || !xs || !wq_hot || !ws_hot || !sorted_hot || !eids_hot || !npad_hot || !act)
    return -1;
  const int nsets = wq ? 2 : 1;
  if (nsets == 2 && (!ws || !sorted_cold || !eids_cold || !npad_cold)) return -1;
  if (K % 128 || N % 256) return -2;
  sk = rlu::pick_sk(K / 128, sk);
  if (rlu::bad_sk(K, sk)) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
  const int nb = (em + 15) / 16;
  const int nblive = nsets * nb < mtk ? nsets * nb : mtk;
  const int items = nblive * (N / 32);
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)wq_hot, ws_hot, sorted_hot, eids_hot, npad_hot};
  const rlu::WSet s1{(const uint8_t*)wq, ws, sorted_cold, eids_cold, npad_cold};
  return rlu::launch<false, 1>(2, sk, grid, stream, (const uint8_t*)qx, xs, s0, nsets == 2 ? s1 : s0,
                               nsets, (uint16_t*)act, nullptr, mtk, top_k, K, N);
}

// down of the split GEMM from the bf16 activation act [mtk, K] (rlu_moe_gemm_split_act's
// output): each workgroup quantizes its block's rows per 128-column group as silu_mul_quant
// does (same scales and codes) and runs the down GEMM on them, so y equals
// rlu_moe_gemm_split (sk 1, any npw) on silu_mul_quant's q2 / s2, bit for bit. Routed weights
// as there; wq == NULL runs the hot list alone. K <= 768, N % 256 == 0.
int rlu_moe_gemm_split_qin(const void* act, const void* wq_hot, const float* ws_hot,
                           const int* sorted_hot, const int* eids_hot, const int* npad_hot,
                           const void* wq, const float* ws, const int* sorted_cold,
                           const int* eids_cold, const int* npad_cold,
                           const float* topk_weights, void* y, int em, int mtk, int K, int N,
                           hipStream_t stream) {
  if (em < 1 || mtk < 0 || K <= 0 || N <= 0) return -1;
  if (!act || !wq_hot || !ws_hot || !sorted_hot || !eids_hot || !npad_hot || !y) return -1;
  const int nsets = wq ? 2 : 1;
  if (nsets == 2 && (!ws || !sorted_cold || !eids_cold || !npad_cold)) return -1;
  if (K % 128 || N % (16 * rlu::QIN_NPW * rlu::QIN_G) || K > 128 * rlu::QIN_MAXG) return -2;
  if (mtk == 0) return 0;
  const int nb = (em + 15) / 16;
  const int nblive = nsets * nb < mtk ? nsets * nb : mtk;
  const int items = nblive * (N / (16 * rlu::QIN_NPW));
  const int grid = ((items + rlu::QIN_G - 1) / rlu::QIN_G + 7) / 8 * 8;   // XCD-aware order
  const rlu::WSet s0{(const uint8_t*)wq_hot, ws_hot, sorted_hot, eids_hot, npad_hot};
  const rlu::WSet s1{(const uint8_t*)wq, ws, sorted_cold, eids_cold, npad_cold};
  return rlu::launch<false, 2>(rlu::QIN_NPW, 1, grid, stream, (const uint8_t*)act, nullptr, s0,
                               nsets == 2 ? s1 : s0, nsets, (uint16_t*)y, topk_weights, mtk, 1,
                               K, N);
}

// Dense fp8 block-scaled GEMM for M <= 16 (the target lm_head): y[M, N] bf16 <- qx[M, K] e4m3
// (xs[M, K/128]) x w[N, K] e4m3 in fragment order (ws[N/128, K/128]).
int rlu_gemm_fp8blk_m16(const void* qx, const float* xs, const void* w, const float* ws,
                        void* y, int M, int N, int K, int wv, int npw, hipStream_t stream) {
  if (M < 1 || M > 16 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (rlu::bad_npw(npw)) return -6;
  const int sk = rlu::pick_sk(K / 128, 0);
  if (rlu::bad_sk(K, sk)) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (!qx || !xs || !w || !ws || !y) return -1;
  const int items = N / (16 * npw);
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)w, ws, nullptr, nullptr, nullptr};
  return rlu::launch<true>(npw, sk, grid, stream, (const uint8_t*)qx, xs, s0, s0, 1,
                           (uint16_t*)y, nullptr, M, 1, K, N);
}

// Row-major [rows, K] e4m3 -> gfx950 fragment order (the layout every GEMM here reads).
// rows % 16 == 0, K % 128 == 0, out must not overlap w. Returns -1 / -2 on bad sizes.
int rlu_shuffle_fp8_weight(const void* w, void* out, long long rows, int K, hipStream_t stream) {
  if (rows <= 0 || K <= 0 || !w || !out) return -1;
  if (rows % 16 || K % 128) return -2;
  const size_t units = (size_t)rows * K / 16;
  const size_t blocks = (units + 255) / 256;
  hipLaunchKernelGGL(rlu::shuffle_k, dim3((unsigned)blocks), dim3(256), 0, stream,
                     (const rlu::v4u*)w, (rlu::v4u*)out, units, K);
  return (int)hipGetLastError();
}

}  // extern "C"
