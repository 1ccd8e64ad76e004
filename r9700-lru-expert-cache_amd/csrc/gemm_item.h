// One wave's share of one grouped-GEMM item: the core of the decode kernel moe_gemm_k
// (gemm.hip), for the MoE GEMMs and the fp8 lm_head.
//
// An item is (one 16-row block, 16 * NPW output columns starting at n0). SKW waves split its K
// range; wave ks streams steps [ks * kpw, (ks + 1) * kpw) of every strip through a ring of D
// register stages: loads for step k + D are issued after the MFMAs of step k. The block's
// metadata (expert id, 16 sorted ids) arrives through scalar loads, which the vector-memory
// counter does not track, and the activation scale times the weight-block scale is staged per
// step in LDS (sx), so after the metadata the whole K range is in flight with no further round
// trip. The float32 block scales are applied per step in the accumulator,
// acc += mfma * (xs * ws), the same association for every NPW at a given SKW.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "numerics.h"
#include "wave.h"

namespace rlu {

constexpr int MAXKPW = 24;  // 128-deep K steps per wave (K / 128 / SKW)
constexpr int XM = 8;       // 4 * XM >= MAXKPW + max ring depth - 1

// K steps of one wave, padded to the ring depth D (the padding steps carry zero scales)
template <int NPW, int SKW, int D = ring_of(NPW)>
__host__ __device__ __forceinline__ int item_steps(int K) {
  const int kpw = K / 128 / SKW;
  return (kpw + D - 1) / D * D;
}

// Accumulates this wave's K share of the item into acc (D layout: lane l holds rows
// 4 (l / 16) + i, column l % 16 of each strip) and returns the item's row ids for those rows
// (sod; mtk = padding) and, for wave ks == 0 when tw is given, their routed weights (twv).
// so / sod: this lane's A row and its four output rows, which the caller takes from the
// block's 16 sorted ids, loaded together with the expert id.
// sx: this wave's item_steps() x 16 floats of LDS (x 2 with PAIR). D: register ring depth.
// PAIR (gate_up with its activation): the first NPW / 2 strips are gate columns n0 + 16 s,
// the others the matching up columns N / 2 + n0 + 16 (s - NPW / 2), each half with its own
// weight-block scales, so a lane holds gate and up of the same (row, column).
// AL: the A operand is the block's 16 rows in LDS (alds: row r at r * als bytes, xsl: their
// K / 128 scales per row), for SKW = 1; qx / xs are not read. pre() runs before the first
// weight loads are issued (loads that must not queue behind them), pro() once the first D
// weight steps are in flight and before anything reads LDS: with AL they fill alds / xsl.
struct NoPro {
  __device__ void operator()() const {}
};

template <int NPW, int SKW, bool DENSE, int D = ring_of(NPW), bool PAIR = false, bool AL = false,
          class PRO = NoPro, class PRE = NoPro>
__device__ __forceinline__ void item_mma(const uint8_t* __restrict__ qx,
                                         const float* __restrict__ xs,
                                         const uint8_t* __restrict__ wq,
                                         const float* __restrict__ ws,
                                         int so, int eid, int n0,
                                         const float* __restrict__ tw, int mtk, int top_k, int K,
                                         int N, int ks, float* sx, v4f (&acc)[NPW],
                                         int (&sod)[4], float (&twv)[4],
                                         const uint8_t* alds = nullptr, int als = 0,
                                         const float* xsl = nullptr, const PRO& pro = PRO(),
                                         const PRE& pre = PRE()) {
  static_assert(!PAIR || (NPW % 2 == 0 && !DENSE), "gate / up pairs");
  static_assert(!AL || (SKW == 1 && !DENSE), "A from LDS: one wave per item");
  constexpr int NH = PAIR ? 2 : 1;                  // weight-scale rows per item
  constexpr int HALF = NPW / 2 > 0 ? NPW / 2 : 1;   // strips per half with PAIR
  const int lane = lane_id();
  const int r16 = lane & 15, c4 = lane >> 4;
  const int nkg = K / 128;
  const int kpw = nkg / SKW;
  const int nsteps = item_steps<NPW, SKW, D>(K);
  if (tw && ks == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) twv[i] = tw[sod[i] < mtk ? sod[i] : 0];
  }
  const bool valid = so < mtk;
  const int arow = valid ? so / top_k : 0;
  const int kg0 = ks * kpw;
  // activation scale x weight-block scale for step k = 4 m + c4 of row r16 (per half with
  // PAIR); issued before the weight loads so that staging them waits for nothing else
  const float* xrow = AL ? xsl + (size_t)r16 * nkg : xs + (size_t)arow * nkg + kg0;
  // strip s's first column and its offset from strip 0 in the fragment-order weights
  auto scol = [&](int s) __attribute__((always_inline)) {
    return PAIR ? (s < NPW / 2 ? n0 + 16 * s : N / 2 + n0 + 16 * (s - NPW / 2)) : n0 + 16 * s;
  };
  const float* wsr[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h)
    wsr[h] = ws + ((size_t)eid * (N / 128) + scol(h * HALF) / 128) * nkg + kg0;
  float xv[XM], wv_[NH][XM];
#pragma unroll
  for (int m = 0; m < XM; ++m) {
    if (4 * m < nsteps) {                           // uniform; the product waits for the store
      const int k = min(4 * m + c4, kpw - 1);
      if (!AL) xv[m] = xrow[k];
#pragma unroll
      for (int h = 0; h < NH; ++h) wv_[h][m] = wsr[h][k];
    }
  }
  const uint8_t* A = AL ? alds + (size_t)r16 * als + 16 * c4
                        : qx + (size_t)arow * K + kg0 * 128 + 16 * c4;
  const uint8_t* W = wq + ((size_t)eid * N + n0) * K + (size_t)kg0 * 2048 + lane * 16;
  v4u ra[D][2], rb[D][NPW][2];
  auto issue = [&](int j, int k) {
    if (!AL) {
      ra[j][0] = *reinterpret_cast<const v4u*>(A + k * 128);
      ra[j][1] = *reinterpret_cast<const v4u*>(A + k * 128 + 64);
    }
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      const v4u* p = reinterpret_cast<const v4u*>(W + (size_t)(scol(s) - n0) * K +
                                                  (size_t)k * 2048);
      rb[j][s][0] = __builtin_nontemporal_load(p);
      rb[j][s][1] = __builtin_nontemporal_load(p + 64);
    }
  };
  auto step = [&](int j, int k) {
    v4f f[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h)
      f[h] = *reinterpret_cast<const v4f*>(sx + (k * NH + h) * 16 + 4 * c4);
    // ring padding (k >= kpw, scale 0) reads the last real step's A, as the register path
    // does: the LDS past a row's K bytes is not the row's (0 x a NaN code would be NaN)
    const int ka = k < kpw ? k : kpw - 1;
    const v8i av = AL ? pack8(*reinterpret_cast<const v4u*>(A + ka * 128),
                              *reinterpret_cast<const v4u*>(A + ka * 128 + 64))
                      : pack8(ra[j][0], ra[j][1]);
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      const v4f d = mfma_f8(av, pack8(rb[j][s][0], rb[j][s][1]));
      const int h = PAIR ? s / HALF : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[s][i] = fmaf(d[i], f[h][i], acc[s][i]);
    }
  };
  pre();
#pragma unroll
  for (int j = 0; j < D; ++j) issue(j, min(j, kpw - 1));
  pro();
  if (AL) {
#pragma unroll
    for (int m = 0; m < XM; ++m)
      if (4 * m < nsteps) xv[m] = xrow[min(4 * m + c4, kpw - 1)];
  }
#pragma unroll
  for (int m = 0; m < XM; ++m) {
    const int k = 4 * m + c4;
    if (4 * m < nsteps && k < nsteps)
#pragma unroll
      for (int h = 0; h < NH; ++h)
        sx[(k * NH + h) * 16 + r16] = (k < kpw && valid) ? xv[m] * wv_[h][m] : 0.f;
  }
  wave_lds_sync();
  int c0 = 0;
  for (; c0 + D < nsteps; c0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      step(j, c0 + j);
      issue(j, min(c0 + j + D, kpw - 1));
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) step(j, c0 + j);
}

// The down projection's item from the A rows in LDS (item_mma with SKW 1 and AL), with the
// weight loads in the order they lie in memory. The wave's 2 NP strips (12 KB each, adjacent)
// go as NP pairs, each pair's 24 KB front to back (step k of strips 2p and 2p + 1 side by
// side), through a ring of R pair-steps that runs on across the pairs. Read that way a wave of
// four strips streams its bytes about 6% faster than step by step across all four (12 KB
// apart). Each strip still accumulates its steps in ascending k from zero with the same
// scales, so the result equals item_mma's bit for bit (K <= 128 PMS; steps past K / 128 carry
// zero scales and repeat the last real step's operands, as item_mma's ring padding does).
constexpr int PMS = 6;

template <int NP, int R, class PRO, class PRE>
__device__ __forceinline__ void item_mma_pm(const uint8_t* __restrict__ wq,
                                            const float* __restrict__ ws, int so, int eid,
                                            int n0, const float* __restrict__ tw, int mtk, int K,
                                            int N, float* sx, v4f (&acc)[2 * NP], int (&sod)[4],
                                            float (&twv)[4], const uint8_t* alds, int als,
                                            const float* xsl, const PRO& pro, const PRE& pre) {
  const int lane = lane_id();
  const int r16 = lane & 15, c4 = lane >> 4;
  const int kpw = K / 128;
  if (tw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) twv[i] = tw[sod[i] < mtk ? sod[i] : 0];
  }
  const bool valid = so < mtk;
  // weight-block scale of step k = 4 m + c4 (the four strips share one 128-column block)
  const float* wsr = ws + ((size_t)eid * (N / 128) + n0 / 128) * kpw;
  float xv[2], wv_[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) wv_[m] = wsr[min(4 * m + c4, kpw - 1)];
  const uint8_t* A = alds + (size_t)r16 * als + 16 * c4;
  const uint8_t* W = wq + ((size_t)eid * N + n0) * K + lane * 16;
  v4u rb[R][2][2];
  auto issue = [&](int j, int t) __attribute__((always_inline)) {
    const int p = t / PMS, k = min(t % PMS, kpw - 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const v4u* q = reinterpret_cast<const v4u*>(W + (size_t)(32 * p + 16 * s) * K +
                                                  (size_t)k * 2048);
      rb[j][s][0] = __builtin_nontemporal_load(q);
      rb[j][s][1] = __builtin_nontemporal_load(q + 64);
    }
  };
  auto step = [&](int j, int t) __attribute__((always_inline)) {
    const int p = t / PMS, k = t % PMS;
    const v4f f = *reinterpret_cast<const v4f*>(sx + k * 16 + 4 * c4);
    const int ka = k < kpw ? k : kpw - 1;
    const v8i av = pack8(*reinterpret_cast<const v4u*>(A + ka * 128),
                         *reinterpret_cast<const v4u*>(A + ka * 128 + 64));
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const v4f d = mfma_f8(av, pack8(rb[j][s][0], rb[j][s][1]));
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[2 * p + s][i] = fmaf(d[i], f[i], acc[2 * p + s][i]);
    }
  };
  pre();
#pragma unroll
  for (int j = 0; j < R; ++j) issue(j, j);
  pro();
#pragma unroll
  for (int m = 0; m < 2; ++m) xv[m] = xsl[(size_t)r16 * kpw + min(4 * m + c4, kpw - 1)];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int k = 4 * m + c4;
    if (k < PMS) sx[k * 16 + r16] = (k < kpw && valid) ? xv[m] * wv_[m] : 0.f;
  }
  wave_lds_sync();
#pragma unroll
  for (int t = 0; t < NP * PMS; ++t) {
    // a later pair reads A and the scales from LDS again: kept from the first pair they
    // would hold 72 more registers and cost the second wave per SIMD
    if (t > 0 && t % PMS == 0) asm volatile("" ::: "memory");
    step(t % R, t);
    if (t + R < NP * PMS) issue(t % R, t + R);
  }
}

// Split-K: waves ks > 0 of each item add their partial sums into wave ks == 0 through LDS, in
// split order (deterministic). rbuf: nwaves x NPW x 4 x 64 floats; every wave of the workgroup
// takes part (one LDS barrier).
template <int NPW, int SKW>
__device__ __forceinline__ void splitk_reduce(v4f (&acc)[NPW], float* rbuf, int wv, int ks) {
  const int lane = lane_id();
  if (ks > 0) {
#pragma unroll
    for (int s = 0; s < NPW; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rbuf[((size_t)wv * NPW * 4 + s * 4 + i) * WAVE + lane] = acc[s][i];
  }
  lds_barrier();
  if (ks == 0) {
#pragma unroll
    for (int x = 1; x < SKW; ++x)
#pragma unroll
      for (int s = 0; s < NPW; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[s][i] += rbuf[((size_t)(wv + x) * NPW * 4 + s * 4 + i) * WAVE + lane];
  }
}

}  // namespace rlu
