// fp8 e4m3 x fp8 e4m3 GEMMs with 128x128 float32 weight-block scales and per-(row, 128-column)
// activation scales, on gfx950 matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4 with unit
// E8M0 scales; the float32 block scales are applied per 128-deep K step in the accumulator).
//
//   moe_gemm_k<NPW, DENSE=false>  the grouped expert GEMM of the MoE path: rows come from
//       moe_align_block_size output (sorted_ids / expert_ids / num_post_pad, block 16), the
//       contract of the reference's r4d_mxfp4_moe_gemm_into (patches/.../r4d_mxfp4_moe.py.lru
//       .diff:363-395, probed in tests/k1/moe_ref_harness.py:282-321): a row id >= mtk is
//       padding and is skipped, an expert id of -1 skips its block, num_post_pad is read on
//       the device, only rows named in sorted_ids are written, and an optional routed weight
//       tw[row] scales the output (GEMM2's epilogue).
//   moe_gemm_k<NPW, DENSE=true>   y[M, N] = A[M, K] W[N, K]^T for M <= 16: the fp8 lm_head
//       GEMV (kernels/fp8_target_lmhead.py:70-74).
//
// Work split: an item is (one 16-row block, one tile of 16*NPW columns, all of K); each wave
// owns items gw, gw + total_waves, ... of a persistent grid, so the grid never depends on the
// device-side block count. Per 128-deep K step a lane issues two 16-byte loads of its
// activation row and two per 16-column weight tile, in the same lane -> K byte pattern
// (lane l: row/column l % 16, bytes 16 (l / 16) .. +16 and 64 + 16 (l / 16) .. +16), so one
// MFMA contracts the full 128 and weights need no pre-shuffle: W stays row-major [N, K].
// Loads for step kg + 1 are issued before the MFMAs of step kg.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int GWV = 4;   // waves per workgroup

__device__ __forceinline__ v8i pack8(uint4 lo, uint4 hi) {
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

__device__ __forceinline__ v4f mfma_f8(v8i a, v8i b, v4f c) {
  // formats 0/0 = e4m3 x e4m3; E8M0 scale 127 = 2^0 on both operands
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// One weight set with its align output; the split call passes two (resident slots + the
// full expert tensor) and runs both block lists in one launch.
struct WSet {
  const uint8_t* wq;
  const float* ws;
  const int* sorted_ids;
  const int* expert_ids;
  const int* npad;
};

// Registers hold up to KCMAX 128-deep K steps of loads per wave (all issued before the first
// MFMA of the chunk): A 32 B + B 32 B x NPW per lane per step.
template <int NPW>
struct Kc {
  static constexpr int MAX = NPW == 1 ? 8 : NPW == 2 ? 6 : NPW == 4 ? 3 : 2;
};

// An item is (one 16-row block, one 16*NPW-column tile). The GWV waves of a workgroup work on
// GWV/SKW items at once; the SKW waves of an item split its K range and their partial sums
// are added in LDS in split order (deterministic), by the split-0 wave, which writes the rows.
template <int NPW, int SKW, bool DENSE>
__global__ __launch_bounds__(GWV * WAVE) void moe_gemm_k(
    const uint8_t* __restrict__ qx, const float* __restrict__ xs, WSet s0, WSet s1, int nsets,
    uint16_t* __restrict__ y, const float* __restrict__ tw, int mtk, int top_k, int K, int N) {
  constexpr int KCM = Kc<NPW>::MAX;
  constexpr int IPG = GWV / SKW;                    // items per workgroup pass
  extern __shared__ float lds[];                    // [GWV][kpw][16] scales, then partials
  const int lane = lane_id();
  const int wv = threadIdx.x / WAVE;
  const int sub = wv / SKW, ks = wv % SKW;
  const int nkg = K / 128;
  const int kpw = nkg / SKW;                        // K steps of this wave
  const int NT = 16 * NPW;
  const int ntiles = N / NT;
  const int nb0 = DENSE ? 1 : (s0.npad[0] >> 4);
  const int nb1 = (DENSE || nsets < 2) ? 0 : (s1.npad[0] >> 4);
  const int nitems = (nb0 + nb1) * ntiles;
  const int ngroups = (nitems + IPG - 1) / IPG;
  float* sx = lds + (size_t)wv * kpw * 16;
  float* red = lds + (size_t)GWV * kpw * 16;        // [2][GWV][NPW*4][64]
  const int r16 = lane & 15, c4 = lane >> 4;
  int parity = 0;

  for (int grp = blockIdx.x; grp < ngroups; grp += gridDim.x, parity ^= 1) {
    const int item = grp * IPG + sub;
    bool live = item < nitems;
    int b = live ? item / ntiles : 0;
    const int n0 = live ? (item - b * ntiles) * NT : 0;
    const bool second = b >= nb0;
    if (second) b -= nb0;
    const uint8_t* __restrict__ wq = second ? s1.wq : s0.wq;
    const float* __restrict__ ws = second ? s1.ws : s0.ws;
    const int* __restrict__ sorted_ids = second ? s1.sorted_ids : s0.sorted_ids;
    const int eid = (DENSE || !live) ? 0 : uniform((second ? s1.expert_ids : s0.expert_ids)[b]);
    live = live && eid >= 0;
    v4f acc[NPW];
#pragma unroll
    for (int s = 0; s < NPW; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
    int sod[4] = {mtk, mtk, mtk, mtk};
    if (live) {
      // this lane's A row (operand layout) and the four output rows it holds (D layout)
      const int so = DENSE ? r16 : sorted_ids[b * 16 + r16];
      const bool valid = so < mtk;
      const int arow = valid ? so / top_k : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) sod[i] = DENSE ? 4 * c4 + i : sorted_ids[b * 16 + 4 * c4 + i];
      const int kg0 = ks * kpw;
      for (int k = c4; k < kpw; k += 4)
        sx[k * 16 + r16] = valid ? xs[(size_t)arow * nkg + kg0 + k] : 0.0f;
      wave_lds_sync();
      const uint8_t* A = qx + (size_t)arow * K + kg0 * 128 + 16 * c4;
      const uint8_t* W = wq + ((size_t)eid * N + n0 + r16) * K + kg0 * 128 + 16 * c4;
      const float* wsr = ws + ((size_t)eid * (N / 128) + n0 / 128) * nkg + kg0;
      const uint4 z4 = make_uint4(0, 0, 0, 0);
      for (int c0 = 0; c0 < kpw; c0 += KCM) {
        uint4 a0[KCM], a1[KCM], b0[KCM][NPW], b1[KCM][NPW];
#pragma unroll
        for (int j = 0; j < KCM; ++j) {             // the whole chunk's loads in flight
          if (c0 + j < kpw) {
            const int o = (c0 + j) * 128;
            a0[j] = valid ? *reinterpret_cast<const uint4*>(A + o) : z4;
            a1[j] = valid ? *reinterpret_cast<const uint4*>(A + o + 64) : z4;
#pragma unroll
            for (int s = 0; s < NPW; ++s) {
              b0[j][s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K + o);
              b1[j][s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K + o + 64);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < KCM; ++j) {
          if (c0 + j < kpw) {
            const int k = c0 + j;
            const float wsc = wsr[k];
            const v4f sxv = *reinterpret_cast<const v4f*>(sx + k * 16 + 4 * c4);
            const v8i av = pack8(a0[j], a1[j]);
#pragma unroll
            for (int s = 0; s < NPW; ++s) {
              const v4f d = mfma_f8(av, pack8(b0[j][s], b1[j][s]), v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[s][i] = fmaf(d[i], sxv[i] * wsc, acc[s][i]);
            }
          }
        }
      }
    }
    if (SKW > 1) {
      float* rb = red + (size_t)parity * GWV * NPW * 4 * WAVE;
      if (ks > 0) {
#pragma unroll
        for (int s = 0; s < NPW; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i) rb[((size_t)wv * NPW * 4 + s * 4 + i) * WAVE + lane] = acc[s][i];
      }
      lds_barrier();
      if (ks == 0) {
#pragma unroll
        for (int x = 1; x < SKW; ++x)
#pragma unroll
          for (int s = 0; s < NPW; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[s][i] += rb[((size_t)(wv + x) * NPW * 4 + s * 4 + i) * WAVE + lane];
      }
    }
    if (live && ks == 0) {
      // epilogue: rows this lane holds, routed weight, bf16, only live rows
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = sod[i];
        if (o < mtk) {
          const float wgt = tw ? tw[o] : 1.0f;
#pragma unroll
          for (int s = 0; s < NPW; ++s)
            y[(size_t)o * N + n0 + s * 16 + r16] = f32_to_bf16(acc[s][i] * wgt);
        }
      }
    }
    wave_lds_sync();                                // sx is rewritten by the next item
  }
}

static int pick_sk(int nkg, int sk) {
  if (sk > 0) return sk;
  if (nkg % 4 == 0) return 4;
  if (nkg % 2 == 0) return 2;
  return 1;
}

template <bool DENSE>
int launch(int npw, int sk, int grid, hipStream_t st, const uint8_t* qx, const float* xs,
           WSet s0, WSet s1, int nsets, uint16_t* y, const float* tw, int mtk, int top_k,
           int K, int N) {
  const int nkg = K / 128;
  const size_t lds =
      ((size_t)GWV * (nkg / sk) * 16 + (sk > 1 ? 2 * (size_t)GWV * npw * 4 * WAVE : 0)) * 4;
#define RLU_L(P, SK)                                                                            \
  hipLaunchKernelGGL((moe_gemm_k<P, SK, DENSE>), dim3(grid), dim3(GWV * WAVE), lds, st, qx, xs, \
                     s0, s1, nsets, y, tw, mtk, top_k, K, N)
#define RLU_SK(P)                   \
  switch (sk) {                     \
    case 1: RLU_L(P, 1); break;     \
    case 2: RLU_L(P, 2); break;     \
    case 4: RLU_L(P, 4); break;     \
    default: return -4;             \
  }
  switch (npw) {
    case 1: RLU_SK(1); break;
    case 2: RLU_SK(2); break;
    case 4: RLU_SK(4); break;
    case 8: RLU_SK(8); break;
    default: return -6;
  }
#undef RLU_SK
#undef RLU_L
  return (int)hipGetLastError();
}

static int num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

// persistent grid: enough workgroups to fill every CU wv deep, never more than the items need
static int grid_for(int items, int sk, int wv) {
  const int per_cu = wv ? wv : 3;
  const int ipg = GWV / sk;
  const int need = (items + ipg - 1) / ipg;
  const int g = num_cus() * per_cu;
  return g < need ? g : (need > 0 ? need : 1);
}

}  // namespace rlu

extern "C" {

// Grouped GEMM with the reference op's argument order (r4d_mxfp4_moe.py.lru.diff:389-395):
// y[mtk, N] bf16 rows named by sorted_ids[0:npad] <- qx[mtk/top_k, K] e4m3 (scales xs[., K/128])
// x wq[E, N, K] e4m3 (block scales ws[E, N/128, K/128]); wref is not used by the fp8 format.
// wv: workgroups per CU of the persistent grid (0 = default 3); sk: K split over the waves of a
// workgroup, 1/2/4 (0 = the largest that divides K/128); npw: 16-column tiles per item, 1/2/4/8.
int r4d_gemm_moe_fp8blk_nt_b16(const void* qx, const float* xs, const void* wq,
                               const float* ws, const void* wref, void* y,
                               const int* sorted_ids, const int* expert_ids,
                               const int* num_post_pad, const float* topk_weights, int em,
                               int mtk, int top_k, int K, int N, int wv, int sk, int npw,
                               hipStream_t stream) {
  (void)wref;
  if (em < 1 || mtk < 0 || top_k < 1 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (npw != 1 && npw != 2 && npw != 4 && npw != 8) return -6;
  sk = rlu::pick_sk(K / 128, sk);
  if ((sk != 1 && sk != 2 && sk != 4) || (K / 128) % sk) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
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
                       void* y, int em, int mtk, int top_k, int K, int N, int wv, int npw,
                       hipStream_t stream) {
  if (em < 1 || mtk < 0 || top_k < 1 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (npw != 1 && npw != 2 && npw != 4 && npw != 8) return -6;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
  const int sk = rlu::pick_sk(K / 128, 0);
  const int nb = (em + 15) / 16;
  const int items = 2 * nb * (N / (16 * npw));
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)wq_hot, ws_hot, sorted_hot, eids_hot, npad_hot};
  const rlu::WSet s1{(const uint8_t*)wq, ws, sorted_cold, eids_cold, npad_cold};
  return rlu::launch<false>(npw, sk, grid, stream, (const uint8_t*)qx, xs, s0, s1, 2,
                            (uint16_t*)y, topk_weights, mtk, top_k, K, N);
}

// Dense fp8 block-scaled GEMM for M <= 16 (the target lm_head): y[M, N] bf16 <- qx[M, K] e4m3
// (xs[M, K/128]) x w[N, K] e4m3 (ws[N/128, K/128]). Same checks as above; M in 1..16.
int rlu_gemm_fp8blk_m16(const void* qx, const float* xs, const void* w, const float* ws,
                        void* y, int M, int N, int K, int wv, int npw, hipStream_t stream) {
  if (M < 1 || M > 16 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (npw != 1 && npw != 2 && npw != 4 && npw != 8) return -6;
  if (wv < 0 || wv > 16) return -5;
  const int sk = rlu::pick_sk(K / 128, 0);
  const int items = N / (16 * npw);
  const int grid = rlu::grid_for(items, sk, wv);
  const rlu::WSet s0{(const uint8_t*)w, ws, nullptr, nullptr, nullptr};
  return rlu::launch<true>(npw, sk, grid, stream, (const uint8_t*)qx, xs, s0, s0, 1,
                           (uint16_t*)y, nullptr, M, 1, K, N);
}

}  // extern "C"
