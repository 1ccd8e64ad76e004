// The decode down projection with moe_sum folded in, token-major: out[t] = sum over k of
// bf16(down(q2[t top_k + k]) x tw[t, k]), summed in float32 in k order and rounded to bf16 --
// the values rlu_moe_gemm_split (sk = 1) writes into ic3 followed by moe_sum_k, bit for bit,
// without the [mtk, N] intermediate or the moe_sum launch.
//
// A workgroup owns one token and W x 16 output columns. Each 16-column strip has KS waves, and
// each of them walks its share of the token's top_k experts in k order (top_k a compile-time
// constant: the loop is unrolled, so the experts' addresses and routed weights sit in scalar
// registers, loaded up front). Per expert a wave runs the K steps of the grouped GEMM for the
// token's A rows (one MFMA per step: 16 rows x 16 columns, of which row k is the one kept) with
// the same per-step fma as moe_gemm_k, multiplies by the routed weight and rounds to bf16; the
// strip's values are then added in k order into one float32 sum. The token's activation
// fragments for every K step are loaded once and serve all its experts; the weights stream
// through a ring of RE x NS stages (RE experts' K ranges) that runs on across a wave's
// experts, so the next RE experts' strips are in flight while expert k is summed. With the
// experts split over two waves per strip (KSPLIT) a workgroup keeps twice the weight bytes in
// flight: the kernel is bound by its loads' latency at these few tokens. Experts come from the
// layer's cache table: a resident expert from its slot, any other from the full tensor
// (device or pinned host memory).
//
// Each expert strip is read once per token that routes to it; workgroups are laid out so that
// the tokens of one column range run on one XCD at the same time and share its L2. The ACT form
// takes the bf16 SiLU-mul activation and quantizes it itself (no silu_mul_quant launch).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "numerics.h"
#include "quant_row.h"
#include "wave.h"

namespace rlu {
namespace dsum {

constexpr int NXCD = 8;
constexpr int BUF_WORD3 = 0x00020000;      // raw buffer descriptor word 3 on gfx9 (no format)
constexpr int NTP = 2;                     // buffer cache policy: streaming
constexpr int MAXK = 16;                   // top_k the kernel takes (A rows of one MFMA)
constexpr int KSPLIT = 2;                  // waves per column strip (the experts split)
constexpr int RE = 2;                      // experts of a wave in flight at once: B=1 step
                                           // 2.588-2.591 -> 2.579-2.582 ms (3 deep: 2.588)

// ACT: qa is the bf16 activation [M top_k, K] (the SiLU-mul output) and sa is not read; the
// workgroup quantizes the token's rows per 128-column group into LDS first, exactly as
// silu_mul_quant_g128_k does (same amax, scale and rounding), and the waves take their A
// fragments and the rows' scales from there.
// KS: waves per column strip, each taking TK / KS of the token's experts (wave w % W owns the
// strip, wave w / W the experts [(w / W) TK / KS, ...)). With KS > 1 the rounded per-expert
// values go through LDS and the strip's first wave adds all TK of them in k order, so the sum
// is the same; the point is twice the weight bytes in flight per workgroup.
template <int NS, int W, int TK, bool ACT = false, int KS = 1>
__global__ __launch_bounds__(W * KS * WAVE) void down_sum_k(
    const void* __restrict__ qa, const float* __restrict__ sa, const int* __restrict__ ids,
    const float* __restrict__ tw, const int* __restrict__ table,
    const uint8_t* __restrict__ hw, const float* __restrict__ hs,
    const uint8_t* __restrict__ cw, const float* __restrict__ cs,
    uint16_t* __restrict__ out, int M, int N, int E) {
  constexpr int K = NS * 128;
  constexpr int TKH = TK / KS;                     // experts per wave
  static_assert(TK <= MAXK, "top_k rows fit one MFMA");
  static_assert(TK % KS == 0, "experts split evenly over a strip's waves");
  constexpr int ALS = K + 16;                      // ACT: LDS row stride of the quantized rows
  __shared__ uint8_t alds[ACT ? TK * ALS : 16];
  __shared__ float xsl[ACT ? TK * NS : 4];
  __shared__ float ys[KS > 1 ? TK * W * 16 : 1];  // KS > 1: [k][column] rounded values
  const int lane = lane_id(), wi = uniform((int)(threadIdx.x / WAVE));
  const int w = wi % W, kb = wi / W * TKH;        // column strip, first expert of this wave
  const int r16 = lane & 15, c4 = lane >> 4;
  // workgroup -> (token, column group): the tokens of one column group are consecutive within
  // an XCD's share of the grid (workgroup b runs on XCD b % 8)
  const int ncg = N / (16 * W);
  const int G = (int)gridDim.x;
  const int nx = G % NXCD == 0 ? NXCD : 1;
  const int pos = ((int)blockIdx.x % nx) * (G / nx) + (int)blockIdx.x / nx;
  const int cg = pos / M, t = pos - cg * M;
  const int col0 = (cg * W + w) * 16;

  // this wave's experts kb + kk (scalar loads, all up front) and where their weights live
  const uint8_t* wp[TKH];
  const float* sp[TKH];
  float twk[TKH];
#pragma unroll
  for (int kk = 0; kk < TKH; ++kk) {
    int e = ids[t * TK + kb + kk];
    e = e < 0 || e >= E ? 0 : e;
    const int s = table[e];
    wp[kk] = (s >= 0 ? hw + (size_t)s * N * K : cw + (size_t)e * N * K) + (size_t)col0 * K;
    sp[kk] = (s >= 0 ? hs + (size_t)s * (N / 128) * NS : cs + (size_t)e * (N / 128) * NS) +
             (size_t)(col0 / 128) * NS;
    twk[kk] = tw[t * TK + kb + kk];
  }
  // the token's A rows: row r16 of the MFMA is (t, k = r16); rows past top_k repeat row 0
  const int arow = t * TK + (r16 < TK ? r16 : 0);
  v4u ra[NS][2];
  if constexpr (!ACT) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const uint8_t* p = reinterpret_cast<const uint8_t*>(qa) + (size_t)arow * K + j * 128 +
                         16 * c4;
      ra[j][0] = *reinterpret_cast<const v4u*>(p);
      ra[j][1] = *reinterpret_cast<const v4u*>(p + 64);
    }
  }
  v4u rb[RE][NS][2];
  const int voff = lane * 16;
  auto issue = [&](int x, int j, __amdgpu_buffer_rsrc_t b) __attribute__((always_inline)) {
    rb[x][j][0] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(b, voff, j * 2048, NTP));
    rb[x][j][1] = __builtin_bit_cast(
        v4u, __builtin_amdgcn_raw_buffer_load_b128(b, voff + 1024, j * 2048, NTP));
  };
  auto wbuf = [&](int kk) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)wp[kk < TKH ? kk : TKH - 1], 0,
                                             kk < TKH ? 16 * K : 0, BUF_WORD3);
  };
  // expert k's per-step scales (activation row (t, k) x weight block), vector loads issued one
  // expert ahead, so waiting for them waits only for weight loads already consumed
  float fx[2][NS], fw[2][NS];
  auto load_scales = [&](int kk, int q) __attribute__((always_inline)) {
    const int kq = kk < TKH ? kk : TKH - 1, r = kb + kq;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      if constexpr (ACT)                           // row r's scale, from LDS
        fx[q][j] = xsl[r * NS + j];
      else
        fx[q][j] = sa[(size_t)(t * TK + r) * NS + j];
      fw[q][j] = sp[kq][j];
    }
  };
  // ACT: the workgroup quantizes the token's top_k rows into LDS once. The rows' loads go out
  // before the first expert's weight loads, so that waiting for them (the counter retires in
  // order) does not wait for the weights: the quant runs while those are in flight. 16-lane
  // group q takes (row, 128-column group) pairs q, q + NG, ... and lane l16 columns
  // [8 l16, 8 l16 + 8) of each, as silu_mul_quant_g128_k does.
  constexpr int NG = W * KS * WAVE / 16, NPR = TK * NS, NPASS = (NPR + NG - 1) / NG;
  const int q16 = (int)threadIdx.x / 16, l16 = lane & 15;
  uint4 raw[ACT ? NPASS : 1];
  if constexpr (ACT) {
    const uint16_t* act = reinterpret_cast<const uint16_t*>(qa) + (size_t)t * TK * K;
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
      const int pr = q16 + p * NG, r = pr / NS, g = pr - r * NS;
      if (pr < NPR)
        raw[p] = *reinterpret_cast<const uint4*>(act + (size_t)r * K + g * 128 + 8 * l16);
    }
  }
#pragma unroll
  for (int x = 0; x < RE; ++x)
#pragma unroll
    for (int j = 0; j < NS; ++j) issue(x, j, wbuf(x));
  if constexpr (ACT) {
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
      const int pr = q16 + p * NG, r = pr / NS, g = pr - r * NS;
      if (pr < NPR) {                              // uniform over each 16-lane group
        float v[8];
        unpack8_bf16(raw[p], v);
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = max(m, abs_bits(v[i]));
        const float sc = scale_of(row_max_u32(m));
        *reinterpret_cast<uint2*>(alds + r * ALS + g * 128 + 8 * l16) = quant8(v, sc);
        if (l16 == 0) xsl[r * NS + g] = sc;
      }
    }
    __syncthreads();
    const int ar = r16 < TK ? r16 : 0;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      ra[j][0] = *reinterpret_cast<const v4u*>(alds + ar * ALS + j * 128 + 16 * c4);
      ra[j][1] = *reinterpret_cast<const v4u*>(alds + ar * ALS + j * 128 + 64 + 16 * c4);
    }
  }
  load_scales(0, 0);
  float sum = 0.f;
#pragma unroll
  for (int kk = 0; kk < TKH; ++kk) {
    const int q = kk & 1;
    load_scales(kk + 1, q ^ 1);
    const __amdgpu_buffer_rsrc_t bn = wbuf(kk + RE);   // past the last: no records, no reads
    const int xr = kk % RE;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const float f = fx[q][j] * fw[q][j];
      const v4f d = mfma_f8(pack8(ra[j][0], ra[j][1]), pack8(rb[xr][j][0], rb[xr][j][1]));
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], f, acc[i]);
      asm volatile("" : "+v"(acc));
      issue(xr, j, bn);
      __builtin_amdgcn_sched_barrier(0);
    }
    // row k sits in lanes c4 = k / 4, element k % 4: round it as the GEMM epilogue does, then
    // add it in k order in the lanes of c4 = 0 (moved there, or through LDS with KS > 1)
    if constexpr (KS == 1) {
      const int k = kk;
      const float y = bf16_to_f32(f32_to_bf16(acc[k & 3] * twk[kk]));
      sum = __fadd_rn(sum, __shfl(y, r16 + 16 * (k >> 2)));
    } else {
      const int k = kb + kk, e4 = k & 3;          // wave-uniform
      const float a = e4 == 0 ? acc[0] : e4 == 1 ? acc[1] : e4 == 2 ? acc[2] : acc[3];
      const float y = bf16_to_f32(f32_to_bf16(a * twk[kk]));
      if (c4 == (k >> 2)) ys[k * (W * 16) + w * 16 + r16] = y;
    }
  }
  if constexpr (KS > 1) {
    __syncthreads();
    if (kb == 0 && c4 == 0) {
#pragma unroll
      for (int k = 0; k < TK; ++k) sum = __fadd_rn(sum, ys[k * (W * 16) + w * 16 + r16]);
    }
  }
  if (kb == 0 && c4 == 0) out[(size_t)t * N + col0 + r16] = f32_to_bf16(sum);
}

}  // namespace dsum
}  // namespace rlu

extern "C" {

// No counterpart in the reference, which runs the down GEMM into ic3 and then vLLM's moe_sum
// (r4d_mxfp4_moe.py.lru.diff:690-696). See include/rlu.h.
int rlu_moe_down_sum(const void* q2, const float* s2, const int* topk_ids,
                     const float* topk_weights, const int* table, const void* w_hot,
                     const float* s_hot, const void* w_full, const float* s_full, void* out,
                     int M, int top_k, int K, int N, int E, hipStream_t stream) {
  using namespace rlu;
  if (M < 0 || top_k < 1 || top_k > dsum::MAXK || K <= 0 || N <= 0 || E <= 0) return -1;
  if (!q2 || !s2 || !topk_ids || !topk_weights || !table || !w_hot || !s_hot || !w_full ||
      !s_full || !out)
    return -1;
  if (K % 128 || N % 128) return -2;               // 128x128 weight blocks
  if (K != 768 || top_k != 10) return -6;          // built for the 768-deep down, top-10
  if (M == 0) return 0;
  constexpr int W = 4, KS = dsum::KSPLIT;
  const int grid = M * (N / (16 * W));
  hipLaunchKernelGGL((dsum::down_sum_k<6, W, 10, false, KS>), dim3(grid), dim3(W * KS * WAVE), 0,
                     stream, q2,
                     s2, topk_ids, topk_weights, table, (const uint8_t*)w_hot, s_hot,
                     (const uint8_t*)w_full, s_full, (uint16_t*)out, M, N, E);
  return (int)hipGetLastError();
}

// rlu_moe_down_sum from the bf16 SiLU-mul activation act [M top_k, K] instead of q2 / s2: the
// kernel quantizes each token's rows as silu_mul_quant (group 128) does, so out is the same
// bit for bit. Same limits and codes. No counterpart in the reference; see include/rlu.h.
int rlu_moe_down_sum_act(const void* act, const int* topk_ids, const float* topk_weights,
                         const int* table, const void* w_hot, const float* s_hot,
                         const void* w_full, const float* s_full, void* out, int M, int top_k,
                         int K, int N, int E, hipStream_t stream) {
  using namespace rlu;
  if (M < 0 || top_k < 1 || top_k > dsum::MAXK || K <= 0 || N <= 0 || E <= 0) return -1;
  if (!act || !topk_ids || !topk_weights || !table || !w_hot || !s_hot || !w_full || !s_full ||
      !out)
    return -1;
  if (K % 128 || N % 128) return -2;
  if (K != 768 || top_k != 10) return -6;
  if (M == 0) return 0;
  constexpr int W = 4, KS = dsum::KSPLIT;
  const int grid = M * (N / (16 * W));
  hipLaunchKernelGGL((dsum::down_sum_k<6, W, 10, true, KS>), dim3(grid), dim3(W * KS * WAVE), 0,
                     stream, act, nullptr, topk_ids, topk_weights, table, (const uint8_t*)w_hot, s_hot,
                     (const uint8_t*)w_full, s_full, (uint16_t*)out, M, N, E);
  return (int)hipGetLastError();
}

}  // extern "C"
