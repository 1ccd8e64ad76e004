// W4 quantizer + packer on gfx950: an lm_head weight [N, K] (bf16, f32 or f16) -> this build's
// int4 group-128 format (the one w4.hip's GEMV reads), in one pass, at load time. It replaces
// quantize_w4 + pack_w4a16 of kernels/draft_w4_lmhead.py:154-198,228-259, with this build's own
// quantizer (bf16 scale, integer zero) and layout.
//
// One wave per tile of 16 rows x 128 columns (one group of 16 rows). Lane l = 16 c + r holds
// row r's 32 values k = 32 i + 8 c + j (i, j = 0..3, 0..7) -- exactly the values whose codes sit
// in the 16 bytes it stores (the B-operand order of v_mfma_f32_16x16x32_bf16: dword i, nibble t
// of the low half = j 2t, of the high half = j 2t + 1). So each lane quantizes its own nibbles
// and writes them with one 16-byte store; a wave writes its tile's 1 KB contiguously, and the
// lanes of column quarter 0 write the tile's 16 scale/zero words.
//
// Quantizer, per (row, group), every operation one float32 rounding (no contraction):
//   width = hi - lo, mid = (lo + hi) / 2 (hi, lo from cross-lane min/max: exact);
//   for each fraction f (1.0, 0.95, ..., 0.55): s = bf16(f * width / 15) (skipped if 0),
//   u = rint(w / s), z0 = rint(7.5 - mid / s); for z in z0, z0 - 1, z0 + 1 (clamped to
//   +-1024): q = clamp(u + z, 0, 15), err = sum ((q - z) s - w)^2 -- each lane sums its 32
//   terms in (i, j) order, the four lanes of a row combine as (p0 + p1) + (p2 + p3) through two
//   xor shuffles (the same float on all four, by commutativity) -- and the first least error
//   wins. A constant group (width 0) stores s = bf16(|v|), z = (v < 0), codes rint(v / s) + z;
//   an all-zero group (and every padding row past N) s = 0, z = 0, codes 0.
// The codes of the best candidate so far are kept packed, so nothing is recomputed.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlu.h"
#include "wave.h"

namespace rlu {
namespace w4pack {

constexpr int NFRAC = 10;
constexpr int ZMAX = 1024;
__constant__ unsigned FRACTION_BITS[NFRAC] = {0x3F800000u, 0x3F733333u, 0x3F666666u,
                                              0x3F59999Au, 0x3F4CCCCDu, 0x3F400000u,
                                              0x3F333333u, 0x3F266666u, 0x3F19999Au,
                                              0x3F0CCCCDu};

__device__ __forceinline__ float bf16_rne(float x) {     // finite, non-negative x
  unsigned b = __float_as_uint(x);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return __uint_as_float(b & 0xFFFF0000u);
}

__device__ __forceinline__ float row_sum4(float p) {     // (p0 + p1) + (p2 + p3) on every lane
  p = p + __shfl_xor(p, 16);
  return p + __shfl_xor(p, 32);
}

// 8 consecutive values of one row at element offset `off`, as float
template <int DT>
__device__ __forceinline__ void load8(const void* w, long long off, float* v) {
  if constexpr (DT == 1) {                                // float32
    const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const float*>(w) + off);
    const uint4 b = *reinterpret_cast<const uint4*>(static_cast<const float*>(w) + off + 4);
    const unsigned u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(u[j]);
  } else {                                                // 16-bit: bf16 (0) or f16 (2)
    const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + off);
    const unsigned u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == 0) {
        v[2 * j] = __uint_as_float(u[j] << 16);
        v[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
      } else {
        v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[j] & 0xFFFFu));
        v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[j] >> 16));
      }
    }
  }
}

// the four dwords of a lane's codes: dword i, nibble t of the low half = j 2t, high = j 2t + 1
__device__ __forceinline__ void pack_codes(const float* q, unsigned* d) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned x = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      x |= (unsigned)q[8 * i + 2 * t] << (4 * t);
      x |= (unsigned)q[8 * i + 2 * t + 1] << (16 + 4 * t);
    }
    d[i] = x;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void pack_k(const void* __restrict__ w, long long ld, int N,
                                              int G, int ntiles, uint4* __restrict__ wq,
                                              unsigned* __restrict__ sz) {
#pragma clang fp contract(off)
  const int tile = blockIdx.x * (256 / WAVE) + (int)(threadIdx.x / WAVE);
  if (tile >= ntiles) return;                             // whole waves only
  const int lane = lane_id();
  const int c = lane >> 4, r = lane & 15;
  const int strip = tile / G, g = tile - strip * G;
  const int row = strip * 16 + r;

  float v[32];
  if (row < N) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      load8<DT>(w, (long long)row * ld + 128 * g + 32 * i + 8 * c, v + 8 * i);
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) v[e] = 0.0f;
  }
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int e = 1; e < 32; ++e) {
    lo = fminf(lo, v[e]);
    hi = fmaxf(hi, v[e]);
  }
  lo = fminf(lo, __shfl_xor(lo, 16));
  lo = fminf(lo, __shfl_xor(lo, 32));
  hi = fmaxf(hi, __shfl_xor(hi, 16));
  hi = fmaxf(hi, __shfl_xor(hi, 32));
  const float width = hi - lo;
  const float mid = (lo + hi) / 2.0f;

  unsigned best[4] = {0u, 0u, 0u, 0u};
  float best_s = 0.0f, best_z = 0.0f;
  if (width > 0.0f) {
    float best_err = __builtin_inff();
    for (int fi = 0; fi < NFRAC; ++fi) {
      const float f = __uint_as_float(FRACTION_BITS[fi]);
      const float s = bf16_rne((f * width) / 15.0f);
      if (!(s > 0.0f)) continue;                          // row-uniform: all 4 lanes agree
      float u[32];
#pragma unroll
      for (int e = 0; e < 32; ++e) u[e] = __builtin_rintf(v[e] / s);
      const float z0 = fminf(fmaxf(__builtin_rintf(7.5f - mid / s), -(float)ZMAX), (float)ZMAX);
#pragma unroll
      for (int sh = 0; sh < 3; ++sh) {
        const float dz = sh == 0 ? 0.0f : sh == 1 ? -1.0f : 1.0f;
        const float z = fminf(fmaxf(z0 + dz, -(float)ZMAX), (float)ZMAX);
        float q[32];
        float p = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
          q[e] = fminf(fmaxf(u[e] + z, 0.0f), 15.0f);
          const float d = (q[e] - z) * s - v[e];
          const float d2 = d * d;
          p = e == 0 ? d2 : p + d2;
        }
        const float err = row_sum4(p);
        if (err < best_err) {
          best_err = err;
          best_s = s;
          best_z = z;
          pack_codes(q, best);
        }
      }
    }
  } else if (lo != 0.0f) {                                // constant, nonzero
    best_s = bf16_rne(fabsf(lo));
    best_z = lo < 0.0f ? 1.0f : 0.0f;
    float q[32];
#pragma unroll
    for (int e = 0; e < 32; ++e)
      q[e] = fminf(fmaxf(__builtin_rintf(v[e] / best_s) + best_z, 0.0f), 15.0f);
    pack_codes(q, best);
  }
  wq[(size_t)tile * WAVE + lane] = make_uint4(best[0], best[1], best[2], best[3]);
  if (c == 0)
    sz[(size_t)tile * 16 + r] =
        (__float_as_uint(best_s) >> 16) | ((unsigned)(int)best_z << 16);
}

}  // namespace w4pack
}  // namespace rlu

extern "C" {

int rlu_pack_w4(const void* w, int dtype, long long ld, int N, int K, int n_pad, void* wq,
                unsigned* sz, hipStream_t stream) {
  using namespace rlu::w4pack;
  if (N < 1 || K < 1 || n_pad < N || ld < K || !w || !wq || !sz) return -1;
  if (K % 128 || n_pad % 16) return -2;
  if (dtype < 0 || dtype > 2) return -3;
  const int esz = dtype == 1 ? 4 : 2;
  if (ld % (16 / esz) || reinterpret_cast<uintptr_t>(w) % 16 ||
      reinterpret_cast<uintptr_t>(wq) % 16 || reinterpret_cast<uintptr_t>(sz) % 4)
    return -4;
  const int G = K / 128;
  const long long tiles = (long long)(n_pad / 16) * G;
  if (tiles > (1LL << 31) - 256) return -1;
  const int ntiles = (int)tiles;
  const dim3 grid((ntiles + 3) / 4), block(256);
  uint4* o = static_cast<uint4*>(wq);
  switch (dtype) {
    case 0: hipLaunchKernelGGL(pack_k<0>, grid, block, 0, stream, w, ld, N, G, ntiles, o, sz); break;
    case 1: hipLaunchKernelGGL(pack_k<1>, grid, block, 0, stream, w, ld, N, G, ntiles, o, sz); break;
    default: hipLaunchKernelGGL(pack_k<2>, grid, block, 0, stream, w, ld, N, G, ntiles, o, sz); break;
  }
  return (int)hipGetLastError();
}

}  // extern "C"
