// Scalar numerics shared by the gfx950 kernels: bf16 and e4m3 conversions and the float32
// exponential used by SiLU. Every routine here has a CPU restatement in the oracle that it
// matches bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rlu {

constexpr float E4M3_MAX = 448.0f;
constexpr float MIN_SCALE = 1.0f / (448.0f * 512.0f);  // vLLM's min_scaling_factor for e4m3

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// nearest-even float32 -> bfloat16 bits (NaN stays NaN)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  // a select, not a branch: the NaN test would otherwise split every conversion of a GEMM
  // epilogue into two exec-masked paths
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}

// f32_to_bf16 in one instruction: gfx950's v_cvt_pk_bf16_f32 gives the same bits for every
// one of the 2^32 float32 inputs (nearest even; NaN payload kept with the quiet bit set;
// denormals rounded, not flushed), which the library's self-test rlu_selftest_bf16 checks
// on the device. Inline assembly: clang's vector conversion to __bf16 did not lower to it
// correctly (it dropped one element of a pair). Used where the rounding sits on a kernel's
// critical path (the prefill SiLU-mul-quant epilogue); elsewhere a faster epilogue only bunched
// the stores that follow it and measured slower.
__device__ __forceinline__ uint16_t f32_to_bf16_hw(float f) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, 0" : "=v"(r) : "v"(f));
  return (uint16_t)r;
}

// two float32 -> two e4m3fn bytes (nearest-even), packed in the low 16 bits. Inputs are
// already clamped to +-448 by every caller, so saturation behaviour never comes into play.
__device__ __forceinline__ uint32_t f32x2_to_e4m3(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// e^x: Cody-Waite reduction x = n ln2 + r (ln2 split hi/lo), degree-7 Taylor polynomial of
// e^r in Horner form, 2^n applied in two exact halves; every operation rounded on its own
// (no contraction), so the CPU restatement reproduces it bit for bit.
__device__ __forceinline__ float exp_f32(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return __builtin_inff();
  if (x < -103.972076f) return 0.0f;
  const float n = __builtin_rintf(__fmul_rn(x, 1.44269504f));
  float r = __fsub_rn(x, __fmul_rn(n, 0.693145752f));
  r = __fsub_rn(r, __fmul_rn(n, 1.42860677e-06f));
  float p = 1.0f / 5040.0f;
  p = __fadd_rn(__fmul_rn(p, r), 1.0f / 720.0f);
  p = __fadd_rn(__fmul_rn(p, r), 1.0f / 120.0f);
  p = __fadd_rn(__fmul_rn(p, r), 1.0f / 24.0f);
  p = __fadd_rn(__fmul_rn(p, r), 1.0f / 6.0f);
  p = __fadd_rn(__fmul_rn(p, r), 0.5f);
  p = __fadd_rn(__fmul_rn(p, r), 1.0f);
  p = __fadd_rn(__fmul_rn(p, r), 1.0f);
  int ni = (int)n;
  ni = ni < -200 ? -200 : (ni > 200 ? 200 : ni);
  const int h = ni >= 0 ? ni / 2 : -((-ni + 1) / 2);   // floor(ni / 2)
  return __fmul_rn(__fmul_rn(p, __builtin_ldexpf(1.0f, h)), __builtin_ldexpf(1.0f, ni - h));
}

// bf16(g / (1 + e^-g)), computed in float32
__device__ __forceinline__ float silu_bf16(float g) {
  const float s = __fdiv_rn(g, __fadd_rn(1.0f, exp_f32(-g)));
  return bf16_to_f32(f32_to_bf16(s));
}

// silu_bf16 with the one-instruction rounding (the same bits)
__device__ __forceinline__ float silu_bf16_hw(float g) {
  const float s = __fdiv_rn(g, __fadd_rn(1.0f, exp_f32(-g)));
  return bf16_to_f32(f32_to_bf16_hw(s));
}

}  // namespace rlu
