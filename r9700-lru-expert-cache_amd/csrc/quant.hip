// Activation quantizers and the top-k reduction of the MoE decode path, for gfx950.
//
//   group_quant_k     per-token-group-128 (or per-token) e4m3 quant of bf16 activations --
//                     the GEMM1 input (patches/.../mxfp4/r4dhip.py.diff:22-34 does it per token
//                     with vLLM's scaled_fp8_quant; this path uses 128-column groups).
//   silu_mul_quant_k  silu(gate) * up + the same quant, one pass (kernels/fused_silu_mul_quant.py
//                     :26-57): silu rounded to bf16 before the multiply, the product rounded to
//                     bf16, amax over the rounded product, scale = max(amax / 448, 1/(448*512)),
//                     q = e4m3(clamp(a / scale, +-448)) with a true division.
//   moe_sum_k         out[m] = sum_k in[m * top_k + k] (vLLM's moe_sum, called at
//                     patches/.../r4d_mxfp4_moe.py.lru.diff:696), float32 accumulation in k order.
//
// Layout: one workgroup per row; each lane owns 8 consecutive columns, so a 16-lane DPP row
// covers exactly one 128-column group and the group amax is a 4-step DPP reduction
// (quant_row.h).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "numerics.h"
#include "quant_row.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {

constexpr int QT = 256;   // threads per row

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* sh) {
  v = row_max_u32(v);
  v = max(max((uint32_t)readlane((int)v, 0), (uint32_t)readlane((int)v, 16)),
          max((uint32_t)readlane((int)v, 32), (uint32_t)readlane((int)v, 48)));
  if (lane_id() == 0) sh[threadIdx.x / WAVE] = v;
  lds_barrier();
  uint32_t r = 0;
  for (int i = 0; i < QT / WAVE; ++i) r = max(r, sh[i]);
  return r;
}

__global__ __launch_bounds__(QT) void group_quant_k(const uint16_t* __restrict__ x, int K,
                                                    int ldx, int group,
                                                    uint8_t* __restrict__ q,
                                                    float* __restrict__ scale) {
  __shared__ uint32_t sh[QT / WAVE];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (size_t)row * ldx;
  uint8_t* qr = q + (size_t)row * K;
  if (group == 0) {
    uint32_t m = 0;
    for (int c = threadIdx.x * 8; c < K; c += QT * 8) {
      float v[8];
      load8_bf16(xr + c, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) m = max(m, abs_bits(v[j]));
    }
    const float s = scale_of(block_max_u32(m, sh));
    if (threadIdx.x == 0) scale[row] = s;
    for (int c = threadIdx.x * 8; c < K; c += QT * 8) {
      float v[8];
      load8_bf16(xr + c, v);
      *reinterpret_cast<uint2*>(qr + c) = quant8(v, s);
    }
    return;
  }
  group_quant_row128(xr, K, qr, scale + (size_t)row * (K / 128));
}

// x [rows, 2d] bf16 (gate | up), ldx elements apart; q [rows, d]; scale [rows, d/group or 1];
// act [rows, d] bf16 or null.
__global__ __launch_bounds__(QT) void silu_mul_quant_k(const uint16_t* __restrict__ x, int d,
                                                       int ldx, int group,
                                                       uint8_t* __restrict__ q,
                                                       float* __restrict__ scale,
                                                       uint16_t* __restrict__ act) {
  __shared__ uint32_t sh[QT / WAVE];
  const int row = blockIdx.x;
  const uint16_t* g = x + (size_t)row * ldx;
  const uint16_t* u = g + d;
  uint8_t* qr = q + (size_t)row * d;
  auto compute8 = [&](int c, float (&a)[8]) {
    float gv[8], uv[8];
    load8_bf16(g + c, gv);
    load8_bf16(u + c, uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = bf16_to_f32(f32_to_bf16(__fmul_rn(silu_bf16(gv[j]), uv[j])));
    if (act) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)f32_to_bf16(a[2 * j]) | ((uint32_t)f32_to_bf16(a[2 * j + 1]) << 16);
      *reinterpret_cast<uint4*>(act + (size_t)row * d + c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  if (group == 0) {
    // per-token: the row is held in registers between the amax and the quant (d <= QT*8*4)
    float a[4][8];
    uint32_t m = 0;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = (it * QT + threadIdx.x) * 8;
      if (c < d) {
        compute8(c, a[it]);
#pragma unroll
        for (int j = 0; j < 8; ++j) m = max(m, abs_bits(a[it][j]));
      }
    }
    const float s = scale_of(block_max_u32(m, sh));
    if (threadIdx.x == 0) scale[row] = s;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = (it * QT + threadIdx.x) * 8;
      if (c < d) *reinterpret_cast<uint2*>(qr + c) = quant8(a[it], s);
    }
    return;
  }
  const int ng = d / 128;
  for (int base = 0; base < d; base += QT * 8) {
    const int c = base + threadIdx.x * 8;
    const bool in = c < d;
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (in) compute8(c, a);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = max(m, abs_bits(a[j]));
    const float s = scale_of(row_max_u32(m));
    if (in) {
      *reinterpret_cast<uint2*>(qr + c) = quant8(a, s);
      if ((threadIdx.x & 15) == 0) scale[(size_t)row * ng + c / 128] = s;
    }
  }
}

// The group-128 form of silu_mul_quant_k laid out by (row, 128-column group) units rather than
// by rows: a 16-lane group takes one unit (lane l on columns [8 l, 8 l + 8), so the DPP row is the
// quant group), a workgroup 16 units, and the grid strides over all rows x d / 128 units. Same
// arithmetic as silu_mul_quant_k, bit for bit; a row-per-workgroup launch leaves most of its
// threads idle at d = 768 and spends its time dispatching workgroups once rows run to
// thousands (a prefill chunk's 40960).
constexpr int SQ_UNITS = 16;                         // units per 256-thread workgroup

__global__ __launch_bounds__(QT) void silu_mul_quant_g128_k(const uint16_t* __restrict__ x,
                                                            int rows, int d, int ldx,
                                                            uint8_t* __restrict__ q,
                                                            float* __restrict__ scale,
                                                            uint16_t* __restrict__ act) {
  const int ng = d / 128;
  const long long units = (long long)rows * ng;
  const int l16 = (int)threadIdx.x & 15;
  // every lane of a 16-lane group has the same unit, so a group runs whole or not at all
  for (long long u = (long long)blockIdx.x * SQ_UNITS + threadIdx.x / 16; u < units;
       u += (long long)gridDim.x * SQ_UNITS) {
    const int row = (int)(u / ng), grp = (int)(u - (long long)row * ng);
    const int c = grp * 128 + 8 * l16;
    const uint16_t* g = x + (size_t)row * ldx;
    float gv[8], uv[8], a[8];
    load8_bf16(g + c, gv);
    load8_bf16(g + d + c, uv);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = bf16_to_f32(f32_to_bf16(__fmul_rn(silu_bf16(gv[j]), uv[j])));
      m = max(m, abs_bits(a[j]));
    }
    const float s = scale_of(row_max_u32(m));
    *reinterpret_cast<uint2*>(q + (size_t)row * d + c) = quant8(a, s);
    if (l16 == 0) scale[(size_t)row * ng + grp] = s;
    if (act) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)f32_to_bf16(a[2 * j]) | ((uint32_t)f32_to_bf16(a[2 * j + 1]) << 16);
      *reinterpret_cast<uint4*>(act + (size_t)row * d + c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// out [M, H] = sum over k of in [M * top_k + k, H]; one wave per 512 columns of a row, grid
// (M, ceil(H / 512)): a decode call's few rows spread over as many CUs as the row has pieces.
// A thread's SUMK rows are loaded together: with top_k 10 all ten loads are in flight at once
// (the rows are read in one memory round trip instead of ten, 3.82 -> 3.71 ms per 52-layer
// B=4 step), then added in k order. The rows are read once, so the loads are nontemporal: at
// 4096 x 10 rows of 2560 read from HBM, 75.4 -> 45.4 us against plain loads (44.0 -> 41.0 us
// inside the prefill layer step, right after down wrote the rows), bit-identical; the B=4 step
// is unchanged. 256-thread workgroups over the rows in row-major order read the chunk in 42.7
// us (6.5 us under plain loads inside the layer step) but made the B=4 step 0.15 us a layer
// slower.
constexpr int SUMK = 10;
constexpr int SUM_THR = WAVE;

__device__ __forceinline__ void load8_bf16_nt(const uint16_t* p, float (&v)[8]) {
  const v4u r = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  unpack8_bf16(make_uint4(r.x, r.y, r.z, r.w), v);
}

__global__ __launch_bounds__(SUM_THR) void moe_sum_k(const uint16_t* __restrict__ in,
                                                     int top_k, int H,
                                                     uint16_t* __restrict__ out) {
  const int m = blockIdx.x;
  const int c = (blockIdx.y * SUM_THR + threadIdx.x) * 8;
  if (c >= H) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint16_t* src = in + (size_t)m * top_k * H + c;
  int k0 = 0;
  for (; k0 + SUMK <= top_k; k0 += SUMK) {         // SUMK rows' loads in flight, then k order
    v4u r[SUMK];
#pragma unroll
    for (int u = 0; u < SUMK; ++u)
      r[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + (size_t)(k0 + u) * H));
#pragma unroll
    for (int u = 0; u < SUMK; ++u) {
      float v[8];
      unpack8_bf16(make_uint4(r[u].x, r[u].y, r[u].z, r[u].w), v);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], v[j]);
    }
  }
  for (int k = k0; k < top_k; ++k) {
    float v[8];
    load8_bf16_nt(src + (size_t)k * H, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], v[j]);
  }
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = (uint32_t)f32_to_bf16(acc[2 * j]) | ((uint32_t)f32_to_bf16(acc[2 * j + 1]) << 16);
  *reinterpret_cast<uint4*>(out + (size_t)m * H + c) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Self-test of f32_to_bf16_hw: every float32 bit pattern through both roundings; a thread
// takes patterns 2 t and 2 t + 1 (opaque to the compiler, so nothing is folded between them)
// and counts the patterns whose two results differ.
__global__ __launch_bounds__(256) void bf16_selftest_k(unsigned long long* __restrict__ bad) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;     // 0 .. 2^31 - 1
  uint32_t u0 = 2u * t, u1 = 2u * t + 1u;
  asm volatile("" : "+v"(u0), "+v"(u1));
  const float a = __uint_as_float(u0), b = __uint_as_float(u1);
  const int n = (f32_to_bf16_hw(a) != f32_to_bf16(a)) + (f32_to_bf16_hw(b) != f32_to_bf16(b));
  if (n) atomicAdd(bad, (unsigned long long)n);
}

}  // namespace rlu

extern "C" {

int rlu_quant_fp8_group(const void* x, int rows, int K, int ldx, int group, void* q,
                        float* scale, hipStream_t stream) {
  if (rows < 0 || K <= 0 || K % 8 || ldx < K || ldx % 8) return -1;
  if (!(group == 0 || (group == 128 && K % 128 == 0))) return -2;
  if (group == 0 && K > rlu::QT * 8 * 64) return -3;
  if (rows == 0) return 0;
  if (!x || !q || !scale) return -1;
  hipLaunchKernelGGL(rlu::group_quant_k, dim3(rows), dim3(rlu::QT), 0, stream,
                     (const uint16_t*)x, K, ldx, group, (uint8_t*)q, scale);
  return (int)hipGetLastError();
}

int rlu_silu_mul_quant(const void* x, int rows, int d, int ldx, int group, void* q,
                       float* scale, void* act, hipStream_t stream) {
  if (rows < 0 || d <= 0 || d % 8 || ldx < 2 * d || ldx % 8) return -1;
  if (!(group == 0 || (group == 128 && d % 128 == 0))) return -2;
  if (group == 0 && d > rlu::QT * 8 * 4) return -3;
  if (rows == 0) return 0;
  if (!x || !q || !scale) return -1;                // act is optional
  if (group == 128) {
    const long long units = (long long)rows * (d / 128);
    long long grid = (units + rlu::SQ_UNITS - 1) / rlu::SQ_UNITS;
    const long long cap = 16LL * rlu::device_cus();
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(rlu::silu_mul_quant_g128_k, dim3((unsigned)grid), dim3(rlu::QT), 0,
                       stream, (const uint16_t*)x, rows, d, ldx, (uint8_t*)q, scale,
                       (uint16_t*)act);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(rlu::silu_mul_quant_k, dim3(rows), dim3(rlu::QT), 0, stream,
                     (const uint16_t*)x, d, ldx, group, (uint8_t*)q, scale, (uint16_t*)act);
  return (int)hipGetLastError();
}

int rlu_moe_sum(const void* in, int M, int top_k, int H, void* out, hipStream_t stream) {
  if (M < 0 || top_k <= 0 || H <= 0 || H % 8) return -1;
  if (M == 0) return 0;
  if (!in || !out) return -1;
  hipLaunchKernelGGL(rlu::moe_sum_k, dim3(M, (H + rlu::SUM_THR * 8 - 1) / (rlu::SUM_THR * 8)),
                     dim3(rlu::SUM_THR), 0, stream, (const uint16_t*)in, top_k, H,
                     (uint16_t*)out);
  return (int)hipGetLastError();
}

// Counts the float32 inputs (of all 2^32) on which f32_to_bf16_hw and f32_to_bf16 differ into
// *bad (which the caller zeroes); 0 means the one-instruction rounding may stand in for the
// integer one. Returns -1 for a null pointer, else the launch status.
int rlu_selftest_bf16(unsigned long long* bad, hipStream_t stream) {
  if (!bad) return -1;
  hipLaunchKernelGGL(rlu::bf16_selftest_k, dim3(1u << 23), dim3(256), 0, stream, bad);
  return (int)hipGetLastError();
}

}  // extern "C"
