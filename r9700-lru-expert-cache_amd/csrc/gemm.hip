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

template <int NPW, bool DENSE>
__global__ __launch_bounds__(GWV * WAVE) void moe_gemm_k(
    const uint8_t* __restrict__ qx, const float* __restrict__ xs,
    const uint8_t* __restrict__ wq, const float* __restrict__ ws, uint16_t* __restrict__ y,
    const int* __restrict__ sorted_ids, const int* __restrict__ expert_ids,
    const int* __restrict__ npad, const float* __restrict__ tw, int mtk, int top_k, int K,
    int N, int total_waves) {
  extern __shared__ float lds_xs[];                 // [GWV][nkg][16]
  const int lane = lane_id();
  const int wv = threadIdx.x / WAVE;
  const int gw = blockIdx.x * GWV + wv;
  const int nkg = K / 128;
  const int NT = 16 * NPW;
  const int ntiles = N / NT;
  const int nblocks = DENSE ? 1 : (npad[0] >> 4);
  const int nitems = nblocks * ntiles;
  float* sx = lds_xs + (size_t)wv * nkg * 16;
  const int r16 = lane & 15, c4 = lane >> 4;

  for (int item = gw; item < nitems; item += total_waves) {
    const int b = item / ntiles;
    const int n0 = (item - b * ntiles) * NT;
    const int eid = DENSE ? 0 : uniform(expert_ids[b]);
    if (eid < 0) continue;
    // this lane's A row (operand layout) and the four output rows it holds (D layout)
    const int so = DENSE ? r16 : sorted_ids[b * 16 + r16];
    const bool valid = so < mtk;
    const int arow = valid ? so / top_k : 0;
    int sod[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sod[i] = DENSE ? 4 * c4 + i : sorted_ids[b * 16 + 4 * c4 + i];
    // stage the activation scales of the 16 rows as [kg][row]
    for (int kg = c4; kg < nkg; kg += 4) sx[kg * 16 + r16] = valid ? xs[(size_t)arow * nkg + kg] : 0.0f;
    wave_lds_sync();

    const uint8_t* A = qx + (size_t)arow * K + 16 * c4;
    const uint8_t* W = wq + ((size_t)eid * N + n0 + r16) * K + 16 * c4;
    const float* wsr = ws + ((size_t)eid * (N / 128) + n0 / 128) * nkg;

    v4f acc[NPW];
#pragma unroll
    for (int s = 0; s < NPW; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    uint4 a0 = valid ? *reinterpret_cast<const uint4*>(A) : z4;
    uint4 a1 = valid ? *reinterpret_cast<const uint4*>(A + 64) : z4;
    uint4 b0[NPW], b1[NPW];
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      b0[s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K);
      b1[s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K + 64);
    }
    for (int kg = 0; kg < nkg; ++kg) {
      const v8i av = pack8(a0, a1);
      v8i bv[NPW];
#pragma unroll
      for (int s = 0; s < NPW; ++s) bv[s] = pack8(b0[s], b1[s]);
      if (kg + 1 < nkg) {                           // next step's loads in flight now
        const int o = (kg + 1) * 128;
        a0 = valid ? *reinterpret_cast<const uint4*>(A + o) : z4;
        a1 = valid ? *reinterpret_cast<const uint4*>(A + o + 64) : z4;
#pragma unroll
        for (int s = 0; s < NPW; ++s) {
          b0[s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K + o);
          b1[s] = *reinterpret_cast<const uint4*>(W + (size_t)s * 16 * K + o + 64);
        }
      }
      const float wsc = wsr[kg];
      const v4f sxv = *reinterpret_cast<const v4f*>(sx + kg * 16 + 4 * c4);
      v4f sc;
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] = sxv[i] * wsc;
#pragma unroll
      for (int s = 0; s < NPW; ++s) {
        const v4f d = mfma_f8(av, bv[s], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[s][i] = fmaf(d[i], sc[i], acc[s][i]);
      }
    }
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
    wave_lds_sync();                                // sx is rewritten by the next item
  }
}

template <bool DENSE>
int launch(int npw, int grid, size_t lds, hipStream_t st, const uint8_t* qx, const float* xs,
           const uint8_t* wq, const float* ws, uint16_t* y, const int* sid, const int* eids,
           const int* npad, const float* tw, int mtk, int top_k, int K, int N) {
  const int tot = grid * GWV;
#define RLU_L(P)                                                                                \
  hipLaunchKernelGGL((moe_gemm_k<P, DENSE>), dim3(grid), dim3(GWV * WAVE), lds, st, qx, xs, wq, \
                     ws, y, sid, eids, npad, tw, mtk, top_k, K, N, tot)
  switch (npw) {
    case 1: RLU_L(1); break;
    case 2: RLU_L(2); break;
    case 4: RLU_L(4); break;
    case 8: RLU_L(8); break;
    default: return -6;
  }
#undef RLU_L
  return (int)hipGetLastError();
}

int num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

}  // namespace rlu

extern "C" {

// Grouped GEMM with the reference op's argument order (r4d_mxfp4_moe.py.lru.diff:389-395):
// y[mtk, N] bf16 rows named by sorted_ids[0:npad] <- qx[mtk/top_k, K] e4m3 (scales xs[., K/128])
// x wq[E, N, K] e4m3 (block scales ws[E, N/128, K/128]); wref is not used by the fp8 format.
// wv: workgroups per CU of the persistent grid (0 = default 4); sk: must be 1 (no split-K);
// npw: 16-column tiles per wave, 1/2/4/8.
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
  if (sk != 1) return -4;
  if (wv < 0 || wv > 16) return -5;
  if (mtk == 0) return 0;
  const int nb = (em + 15) / 16;
  const int items = nb * (N / (16 * npw));
  const int per_cu = wv ? wv : 4;
  int grid = rlu::num_cus() * per_cu;
  const int need = (items + rlu::GWV - 1) / rlu::GWV;
  if (grid > need) grid = need;
  const size_t lds = (size_t)rlu::GWV * (K / 128) * 16 * sizeof(float);
  return rlu::launch<false>(npw, grid, lds, stream, (const uint8_t*)qx, xs, (const uint8_t*)wq,
                            ws, (uint16_t*)y, sorted_ids, expert_ids, num_post_pad,
                            topk_weights, mtk, top_k, K, N);
}

// Dense fp8 block-scaled GEMM for M <= 16 (the target lm_head): y[M, N] bf16 <- qx[M, K] e4m3
// (xs[M, K/128]) x w[N, K] e4m3 (ws[N/128, K/128]). Same checks as above; M in 1..16.
int rlu_gemm_fp8blk_m16(const void* qx, const float* xs, const void* w, const float* ws,
                        void* y, int M, int N, int K, int wv, int npw, hipStream_t stream) {
  if (M < 1 || M > 16 || K <= 0 || N <= 0) return -1;
  if (K % 128 || N % 128) return -2;
  if (npw != 1 && npw != 2 && npw != 4 && npw != 8) return -6;
  if (wv < 0 || wv > 16) return -5;
  const int items = N / (16 * npw);
  const int per_cu = wv ? wv : 4;
  int grid = rlu::num_cus() * per_cu;
  const int need = (items + rlu::GWV - 1) / rlu::GWV;
  if (grid > need) grid = need;
  const size_t lds = (size_t)rlu::GWV * (K / 128) * 16 * sizeof(float);
  return rlu::launch<true>(npw, grid, lds, stream, (const uint8_t*)qx, xs, (const uint8_t*)w,
                           ws, (uint16_t*)y, nullptr, nullptr, nullptr, nullptr, M, 1, K, N);
}

}  // extern "C"
