// Row-level e4m3 quant pieces shared by the quant kernels and the LRU launch's quant
// workgroups: each lane owns 8 consecutive bf16 columns, so a 16-lane DPP row covers exactly one
// 128-column group and the group amax is a 4-step DPP reduction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.h"
#include "wave.h"

namespace rlu {

__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp<0xb1>((int)v, (int)v));
  v = max(v, (uint32_t)dpp<0x4e>((int)v, (int)v));
  v = max(v, (uint32_t)dpp<0x141>((int)v, (int)v));
  v = max(v, (uint32_t)dpp<0x140>((int)v, (int)v));
  return v;
}

// |x| of non-negative floats compares like its bit pattern
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

__device__ __forceinline__ float scale_of(uint32_t amax_bits) {
  const float s = __fdiv_rn(__uint_as_float(amax_bits), E4M3_MAX);
  return s > MIN_SCALE ? s : MIN_SCALE;
}

// a / s rounded to nearest, for s >= MIN_SCALE, without a division per value: with r =
// RN(1 / s), q0 = RN(a r) is within an ulp or two of a / s, e = a - q0 s is exact (one FMA),
// and RN(q0 + e r) is the correctly rounded quotient (Markstein's correction; P. Markstein,
// IBM J. Res. Dev. 34(1), 1990). It carries the sign of a, as the quotient does (the FMA turns
// -0 + +0 into +0). Where the correction cannot apply, the uncorrected q0 gives the same e4m3
// code: |q0| >= 448 (the clamp decides; that covers q0 = Inf), and an infinite s (an infinite
// amax), where q0 = a * 0 is what the division gives. Every kernel here quantizes bf16 values
// with a scale made from their bf16 amax; that whole input space, both signs, is checked
// against IEEE division code for code by the GPU tests.
struct RecipScale {
  float s, r;
  bool fin;
  __device__ __forceinline__ explicit RecipScale(float s_)
      : s(s_), r(__fdiv_rn(1.0f, s_)), fin(s_ < __builtin_inff()) {}
  __device__ __forceinline__ float quot(float a) const {
    const float q0 = __fmul_rn(a, r);
    const float e = __fmaf_rn(-q0, s, a);
    const float q1 = __builtin_copysignf(__fmaf_rn(e, r, q0), a);
    return (fin && fabsf(q0) < E4M3_MAX) ? q1 : q0;
  }
};

// quantize 8 values with one scale -> 8 e4m3 bytes: e4m3(clamp(a / s, +-448)), nearest even
__device__ __forceinline__ uint2 quant8(const float (&a)[8], float s) {
  const RecipScale rs(s);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x0 = rs.quot(a[2 * j]), x1 = rs.quot(a[2 * j + 1]);
    x0 = fminf(fmaxf(x0, -E4M3_MAX), E4M3_MAX);
    x1 = fminf(fmaxf(x1, -E4M3_MAX), E4M3_MAX);
    w[j] = f32x2_to_e4m3(x0, x1);
  }
  return make_uint2(w[0] | (w[1] << 16), w[2] | (w[3] << 16));
}

__device__ __forceinline__ void unpack8_bf16(const uint4 r, float (&v)[8]) {
  const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(u[j] << 16);
    v[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
  }
}

__device__ __forceinline__ void load8_bf16(const uint16_t* p, float (&v)[8]) {
  unpack8_bf16(*reinterpret_cast<const uint4*>(p), v);
}

// group == 128: one scale per 128 columns; group == 0: one scale per row. K % 8 == 0 and, for
// group 128, K % 128 == 0 (checked by the entry point).
// one row of per-token-group-128 quant by a 256-thread workgroup: q[c] = e4m3(x[c] / s_g),
// s_g = max(amax_g / 448, 1 / (448 * 512)) for each 128-column group g
__device__ __forceinline__ void group_quant_row128(const uint16_t* __restrict__ xr, int K,
                                                   uint8_t* __restrict__ qr,
                                                   float* __restrict__ sr) {
  for (int base = 0; base < K; base += 256 * 8) {   // uniform trip count over the block
    const int c = base + (int)threadIdx.x * 8;
    const bool in = c < K;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (in) load8_bf16(xr + c, v);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = max(m, abs_bits(v[j]));
    const float s = scale_of(row_max_u32(m));
    if (in) {
      *reinterpret_cast<uint2*>(qr + c) = quant8(v, s);
      if ((threadIdx.x & 15) == 0) sr[c / 128] = s;
    }
  }
}

// The same quant of one row by one wave: lane l owns columns [8 l, 8 l + 8) of each 512-column
// pass, and the loads of QP passes are in flight together. Identical results to
// group_quant_row128 (same groups, same amax reduction, same rounding).
constexpr int QP = 8;
__device__ __forceinline__ void wave_quant_row128(const uint16_t* __restrict__ xr, int K,
                                                  uint8_t* __restrict__ qr,
                                                  float* __restrict__ sr) {
  const int lane = lane_id();
  for (int base = 0; base < K; base += QP * WAVE * 8) {
    uint4 raw[QP];
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int c = base + (p * WAVE + lane) * 8;
      raw[p] = c < K ? *reinterpret_cast<const uint4*>(xr + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int c = base + (p * WAVE + lane) * 8;
      float v[8];
      unpack8_bf16(raw[p], v);
      uint32_t m = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = max(m, abs_bits(v[j]));
      const float s = scale_of(row_max_u32(m));
      if (c < K) {
        *reinterpret_cast<uint2*>(qr + c) = quant8(v, s);
        if ((lane & 15) == 0) sr[c / 128] = s;
      }
    }
  }
}

}  // namespace rlu
