// W4 draft lm_head GEMV on gfx950: y[M, N] bf16 = x[M, K] bf16 . dequant(W[N, K])^T, M <= 16,
// for the int4 group-128 asymmetric weight of kernels/draft_w4_lmhead.py (quantize_w4 :154-198,
// op :351-403), in this build's own gfx950 format:
//
//   codes   q in 0..15, w ~ scale * (q - zero) per (row, 128-column group).
//   wq      [N/16][K/128][64 lanes][16 B]: the 1 KB of one 16-row x 128-deep tile in
//           v_mfma_f32_16x16x32_bf16 B-operand order. Lane l = 16 c + r (row r of the tile)
//           holds four dwords, one per 32-deep MFMA i, each covering k = 128 g + 32 i + 8 c + j
//           (j = 0..7): bits 4t..4t+3 hold j = 2t and bits 16+4t..19+4t hold j = 2t+1.
//   sz      [N/16][K/128][16] u32: bf16 scale bits in the low half, the integer zero (int16,
//           |zero| <= 1024) in the high half; row within the tile is the last axis.
//
// Dequant: ((D >> 4t) & 0x000F000F) | 0x43004300 is the bf16 pair (128 + q_2t, 128 + q_2t+1),
// exact; one v_and_or_b32 per pair, the shifts done 64 bits (two dwords) at a time. The MFMA
// then gives d = sum_k x_k (128 + q_k) per group, and the group's contribution is
// scale * (d - (128 + zero) * sum_k x_k). Per tile only scale * d is accumulated; the offset and
// zero terms of all of a wave's groups come out once per item through an f32 MFMA of the
// per-(row, group) activation sums (computed once per workgroup) against scale * (128 + zero).
// Activations stay bf16 (the reference widened bf16 to f16 for its gfx1201 WMMA).
//
// Work split: an item is SS 16-row strips (16 SS columns). SKW waves split K; a workgroup of 8
// waves runs 8 / SKW items at once. x (<= 16 rows, zero-padded) is staged once per workgroup in
// LDS in A-operand fragment order, so each A read is a conflict-free 1 KB ds_read_b128 shared by
// the SS strips of a group; each wave computes the per-(row, group) sums of x for its groups with
// an MFMA of ones. Per group a wave dequantizes its SS 1 KB tiles and runs SS
// independent MFMA chains. Its register ring is one item deep: after consuming a tile it issues
// the same tile of its next item, so a whole item (SS x G / SKW KB per wave) is in flight behind
// the one being computed. The K splits' partial sums are added in LDS in a fixed order
// (deterministic) and the split-0 wave writes the item's bf16 logits.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "numerics.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {
namespace w4 {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int WAVES = 8;
constexpr int SS = 2;          // strips per item
constexpr int MAXGQ = 8;       // groups per wave: K / 128 / split <= 8, so K <= 4096
constexpr int MAXK = 4096;     // x in LDS: 16 rows x K bf16 = 2 K * 16 bytes
constexpr int BUF_WORD3 = 0x00020000;   // raw buffer descriptor word 3 on gfx9 (no format)
constexpr int SLC = 2;                  // buffer cache policy: streaming (the codes are read once)

__device__ __forceinline__ v4f mfma_bf16(v4u a, v4u b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                 __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}

// (v & mask) | magic in one VALU op; the mask rides in an SGPR and the magic in a VGPR (a VOP3
// op on gfx9 takes no literal and one scalar operand), which the compiler would not pick itself
__device__ __forceinline__ unsigned and_or(unsigned v, unsigned mask, unsigned magic) {
  unsigned r;
  asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(magic));
  return r;
}

// 64-bit right shift by a constant, as one instruction (the compiler splits a 64-bit shift
// into two 32-bit ones, alignbit + shift)
template <int S>
__device__ __forceinline__ unsigned long long shr64(unsigned long long v) {
  unsigned long long r;
  asm volatile("v_lshrrev_b64 %0, %1, %2" : "=v"(r) : "i"(S), "v"(v));
  return r;
}

// the 16 bf16 pairs (128 + q_2t, 128 + q_2t+1) of one tile lane: b[i] feeds MFMA i. One 64-bit
// shift serves two dwords: the bits that cross into the low dword land at bit 20 and above,
// which the mask drops.
__device__ __forceinline__ void dequant(v4u w, unsigned mask, unsigned magic, v4u* b) {
  const unsigned long long p0 = ((unsigned long long)w.y << 32) | w.x;
  const unsigned long long p1 = ((unsigned long long)w.w << 32) | w.z;
  const unsigned long long a4 = shr64<4>(p0), a8 = shr64<8>(p0), a12 = shr64<12>(p0);
  const unsigned long long c4 = shr64<4>(p1), c8 = shr64<8>(p1), c12 = shr64<12>(p1);
  b[0] = v4u{and_or(w.x, mask, magic), and_or((unsigned)a4, mask, magic),
             and_or((unsigned)a8, mask, magic), and_or((unsigned)a12, mask, magic)};
  b[1] = v4u{and_or(w.y, mask, magic), and_or((unsigned)(a4 >> 32), mask, magic),
             and_or((unsigned)(a8 >> 32), mask, magic), and_or((unsigned)(a12 >> 32), mask, magic)};
  b[2] = v4u{and_or(w.z, mask, magic), and_or((unsigned)c4, mask, magic),
             and_or((unsigned)c8, mask, magic), and_or((unsigned)c12, mask, magic)};
  b[3] = v4u{and_or(w.w, mask, magic), and_or((unsigned)(c4 >> 32), mask, magic),
             and_or((unsigned)(c8 >> 32), mask, magic), and_or((unsigned)(c12 >> 32), mask, magic)};
}

template <int SKW, int GQ>
__global__ __launch_bounds__(WAVES * WAVE) void gemv_k(const uint16_t* __restrict__ x, int M,
                                                       int K, const v4u* __restrict__ wq,
                                                       const unsigned* __restrict__ sz,
                                                       uint16_t* __restrict__ y, int N) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int U = SS * GQ;                        // units (1 KB tiles) per item per wave
  constexpr int IPG = WAVES / SKW;                  // items per workgroup pass
  const int G = K / 128;
  v4u* xa = reinterpret_cast<v4u*>(smem);                       // [G][4][64] fragments
  float* red = reinterpret_cast<float*>(smem + (size_t)G * 256 * 16);  // [WAVES][SS*4][64]
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wv = uniform(t / WAVE);
  const int sub = wv / SKW, ks = wv % SKW;          // item slot in the workgroup, K split
  const int r16 = lane & 15, c4 = lane >> 4;
  const int g0 = ks * GQ;
  const unsigned mask = uniform(0x000F000F), magic = 0x43004300u;

  // x -> LDS in A-operand order: unit (g, i, l) = row l % 16, k = 128 g + 32 i + 8 (l / 16)
  for (int u = t; u < G * 256; u += WAVES * WAVE) {
    const int l = u & 63, gi = u >> 6;
    const int row = l & 15;
    const int k = (gi >> 2) * 128 + (gi & 3) * 32 + (l >> 4) * 8;
    v4u v = {0u, 0u, 0u, 0u};
    if (row < M) v = *reinterpret_cast<const v4u*>(x + (size_t)row * K + k);
    xa[u] = v;
  }
  __syncthreads();
  // per-(row, group) sums of x as the A operand of the zero-correction MFMA (f32 16x16x4):
  // lane (c4, r16) holds minus the sum of row r16 over group g0 + c4 + 4 j (0 past GQ). The
  // x fragments in A order, read as a B operand, are x transposed, so an MFMA of ones against
  // them leaves row r16's sum in every register of lane (c4, r16).
  constexpr int NJ = (GQ + 3) / 4;
  float xs_a[NJ];
  {
    const v4u ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    float s[GQ];
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) d = mfma_bf16(ones, xa[((g0 + g) * 4 + i) * 64 + lane], d);
      s[g] = d[0];
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float v = 0.f;
#pragma unroll
      for (int g = 4 * j; g < GQ && g < 4 * j + 4; ++g) v = c4 == g - 4 * j ? s[g] : v;
      xs_a[j] = -v;
    }
  }

  const int nitems = N / (16 * SS);
  const int stride = gridDim.x * IPG;
  int item = blockIdx.x * IPG + sub;
  v4u rw[U];
  unsigned rs[U];
  // buffer loads: the tile offset is wave-uniform and rides in an SGPR (no per-load vector
  // address arithmetic); the host keeps the byte sizes below 2^31
  const int ntile = nitems * SS * G;
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void*)wq, 0, ntile * 1024, BUF_WORD3);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc((void*)sz, 0, ntile * 64, BUF_WORD3);
  auto load = [&](int it, int g, int s2) {
    const int itc = it < nitems ? it : nitems - 1;  // past the end: re-read the last item
    const int tile = __builtin_amdgcn_readfirstlane((itc * SS + s2) * G + g0 + g);
    rw[g * SS + s2] = __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16, tile * 1024, SLC);
    rs[g * SS + s2] = __builtin_amdgcn_raw_buffer_load_b32(rz, r16 * 4, tile * 64, 0);
  };
#pragma unroll
  for (int g = 0; g < GQ; ++g)
#pragma unroll
    for (int s2 = 0; s2 < SS; ++s2) load(item, g, s2);
  // every wave of the workgroup runs the same number of passes (the barriers below)
  for (int pass = blockIdx.x; pass * IPG < nitems; pass += gridDim.x) {
    v4f acc[SS];
    unsigned zs[SS][NJ];            // scale/zero word of group g0 + c4 + 4 j, column r16
#pragma unroll
    for (int s2 = 0; s2 < SS; ++s2) {
      acc[s2] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) zs[s2][j] = 0u;
    }
    const int next = item + stride;
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      v4u a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = xa[((g0 + g) * 4 + i) * 64 + lane];
#pragma unroll
      for (int s2 = 0; s2 < SS; ++s2) {
        const int j = g * SS + s2;
        const unsigned sv = rs[j];
        v4u b[4];
        dequant(rw[j], mask, magic, b);
        v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) d = mfma_bf16(a[i], b[i], d);
        const float sc = __uint_as_float(sv << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[s2][i] = fmaf(sc, d[i], acc[s2][i]);
        if (c4 == g % 4) zs[s2][g / 4] = sv;        // for the zero correction below
        load(next, g, s2);                          // the same tile of the next item
      }
    }
    // offset and zero: acc -= sum_g xsum[row, g] * scale[g, col] * (128 + zero[g, col]), the
    // wave's GQ groups as the K of f32 MFMAs (the product of a bf16 scale and an integer
    // below 2^11 is exact in f32)
#pragma unroll
    for (int s2 = 0; s2 < SS; ++s2)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const unsigned sv = zs[s2][j];
        const float z = __uint_as_float(sv << 16) * (128.0f + (float)(short)(sv >> 16));
        acc[s2] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs_a[j], z, acc[s2], 0, 0, 0);
      }
    // K splits -> the split-0 wave of the item, in split order; the buffer is single, so a
    // second barrier keeps the next pass's writes behind this pass's reads
    if (SKW > 1) {
      float* rb = red;
      if (ks > 0) {
#pragma unroll
        for (int s2 = 0; s2 < SS; ++s2)
#pragma unroll
          for (int i = 0; i < 4; ++i) rb[((size_t)wv * SS * 4 + s2 * 4 + i) * WAVE + lane] = acc[s2][i];
      }
      lds_barrier();
      if (ks == 0) {
#pragma unroll
        for (int q = 1; q < SKW; ++q)
#pragma unroll
          for (int s2 = 0; s2 < SS; ++s2)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[s2][i] += rb[((size_t)(wv + q) * SS * 4 + s2 * 4 + i) * WAVE + lane];
      }
      lds_barrier();
    }
    if (ks == 0 && item < nitems) {
#pragma unroll
      for (int s2 = 0; s2 < SS; ++s2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 4 * c4 + i;
          if (row < M) y[(size_t)row * N + (item * SS + s2) * 16 + r16] = f32_to_bf16(acc[s2][i]);
        }
    }
    item = next;
  }
}

}  // namespace w4
}  // namespace rlu

extern "C" {

int rlu_gemm_w4_m16(const void* x, int M, int K, const void* wq, const unsigned* sz, void* y,
                    int N, int wv, hipStream_t stream) {
  using namespace rlu::w4;
  if (M < 1 || M > 16 || K <= 0 || N <= 0 || wv < 0 || wv > 16) return -1;
  if (K % 128 || N % (16 * SS) || K > MAXK) return -2;
  if ((long long)N * K / 2 >= (1LL << 31)) return -2;   // buffer byte offsets are 32-bit
  if (!x || !wq || !sz || !y) return -1;
  const int G = K / 128;
  const int skw = G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
  const int gq = G / skw;
  if (gq > MAXGQ) return -2;
  const int ipg = WAVES / skw;
  const int nitems = N / (16 * SS);
  const int passes = (nitems + ipg - 1) / ipg;
  int grid = rlu::device_cus() * (wv ? wv : 1);
  if (grid > passes) grid = passes;
  const size_t lds = (size_t)G * 256 * 16 + (size_t)WAVES * SS * 4 * rlu::WAVE * 4;
#define RLU_W4(SK, GQ)                                                                        \
  hipLaunchKernelGGL((gemv_k<SK, GQ>), dim3(grid), dim3(WAVES * rlu::WAVE), lds, stream,       \
                     (const uint16_t*)x, M, K, (const rlu::v4u*)wq, sz, (uint16_t*)y, N)
#define RLU_W4_GQ(SK)                                                                         \
  switch (gq) {                                                                               \
    case 1: RLU_W4(SK, 1); break;                                                             \
    case 2: RLU_W4(SK, 2); break;                                                             \
    case 3: RLU_W4(SK, 3); break;                                                             \
    case 4: RLU_W4(SK, 4); break;                                                             \
    case 5: RLU_W4(SK, 5); break;                                                             \
    case 6: RLU_W4(SK, 6); break;                                                             \
    case 7: RLU_W4(SK, 7); break;                                                             \
    case 8: RLU_W4(SK, 8); break;                                                             \
    default: return -2;                                                                       \
  }
  switch (skw) {
    case 1: RLU_W4_GQ(1); break;
    case 2: RLU_W4_GQ(2); break;
    default: RLU_W4_GQ(4); break;
  }
#undef RLU_W4_GQ
#undef RLU_W4
  return (int)hipGetLastError();
}

}  // extern "C"
