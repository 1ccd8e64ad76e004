// Wave64 / workgroup primitives shared by the gfx950 kernels of librlu.so.
//
// Cross-lane traffic uses DPP (data-parallel primitives: a VALU operand modifier, a few cycles)
// and v_readlane into scalar registers, never ds_bpermute, whose LDS round trip costs ~100
// cycles per step. Results the whole wave needs come back as wave-uniform values.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rlu {

constexpr int WAVE = 64;

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// number of set bits of m in lanes below this one
__device__ __forceinline__ int mbcnt(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Workgroup barrier that orders LDS only: global loads and stores still in flight are not
// waited for, so a barrier never stalls on store acknowledgements.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders LDS writes of some lanes before LDS reads of other lanes of the same wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// ---- DPP ---------------------------------------------------------------------------------
// dpp_ctrl encodings (GFX9): quad_perm 0x00-0xff, row_shr:n 0x110+n, row_mirror 0x140,
// row_half_mirror 0x141, row_bcast:15 0x142, row_bcast:31 0x143.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ int dpp(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  const int lo = dpp<CTRL>((int)(uint32_t)v, (int)(uint32_t)v);
  const int hi = dpp<CTRL>((int)(uint32_t)(v >> 32), (int)(uint32_t)(v >> 32));
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__device__ __forceinline__ int readlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  return ((uint64_t)(uint32_t)readlane((int)(uint32_t)(v >> 32), l) << 32) |
         (uint32_t)readlane((int)(uint32_t)v, l);
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

struct OpMin64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return b < a ? b : a; } };
struct OpMax64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return b > a ? b : a; } };

// every lane of each 16-lane row ends with the row's reduction
template <class Op>
__device__ __forceinline__ uint64_t row_reduce64(uint64_t v, Op op) {
  v = op(v, dpp64<0xb1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp64<0x4e>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp64<0x141>(v));  // row_half_mirror
  v = op(v, dpp64<0x140>(v));  // row_mirror
  return v;
}
template <class Op>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, Op op) {  // wave-uniform
  v = row_reduce64(v, op);
  uint64_t r = readlane64(v, 0);
  r = op(r, readlane64(v, 16));
  r = op(r, readlane64(v, 32));
  return op(r, readlane64(v, 48));
}

// unsigned minimum and maximum over the wave, both at once (wave-uniform results)
__device__ __forceinline__ void wave_minmax_u32(uint32_t& mn, uint32_t& mx) {
#define RLU_MM(C)                                            \
  {                                                          \
    const uint32_t a = (uint32_t)dpp<C>((int)mn, (int)mn);   \
    const uint32_t b = (uint32_t)dpp<C>((int)mx, (int)mx);   \
    mn = a < mn ? a : mn;                                    \
    mx = b > mx ? b : mx;                                    \
  }
  RLU_MM(0xb1) RLU_MM(0x4e) RLU_MM(0x141) RLU_MM(0x140)
#undef RLU_MM
  const uint32_t n0 = (uint32_t)readlane((int)mn, 0), n1 = (uint32_t)readlane((int)mn, 16);
  const uint32_t n2 = (uint32_t)readlane((int)mn, 32), n3 = (uint32_t)readlane((int)mn, 48);
  const uint32_t x0 = (uint32_t)readlane((int)mx, 0), x1 = (uint32_t)readlane((int)mx, 16);
  const uint32_t x2 = (uint32_t)readlane((int)mx, 32), x3 = (uint32_t)readlane((int)mx, 48);
  mn = min(min(n0, n1), min(n2, n3));
  mx = max(max(x0, x1), max(x2, x3));
}

__device__ __forceinline__ int row_sum(int v) {
  v += dpp<0xb1>(v, v);
  v += dpp<0x4e>(v, v);
  v += dpp<0x141>(v, v);
  v += dpp<0x140>(v, v);
  return v;
}
__device__ __forceinline__ int wave_sum(int v) {  // wave-uniform
  v = row_sum(v);
  return readlane(v, 0) + readlane(v, 16) + readlane(v, 32) + readlane(v, 48);
}

// inclusive prefix sum inside each 16-lane row
__device__ __forceinline__ int row_incl_scan(int v) {
  v += dpp<0x111>(0, v);
  v += dpp<0x112>(0, v);
  v += dpp<0x114>(0, v);
  v += dpp<0x118>(0, v);
  return v;
}
// inclusive prefix sum over the wave
__device__ __forceinline__ int wave_incl_scan(int v) {
  v = row_incl_scan(v);
  v += dpp<0x142, 0xa>(0, v);  // row_bcast:15 -> rows 1 and 3
  v += dpp<0x143, 0xc>(0, v);  // row_bcast:31 -> rows 2 and 3
  return v;
}

// inclusive prefix max over the wave, for values >= -1 (lanes with no source take -1)
__device__ __forceinline__ int wave_incl_max(int v) {
  v = max(v, dpp<0x111>(-1, v));
  v = max(v, dpp<0x112>(-1, v));
  v = max(v, dpp<0x114>(-1, v));
  v = max(v, dpp<0x118>(-1, v));
  v = max(v, dpp<0x142, 0xa>(-1, v));
  v = max(v, dpp<0x143, 0xc>(-1, v));
  return v;
}

// Lanes of this wave holding the same `key` as this lane (all lanes call it; lanes with
// valid == false match nothing and get 0). Bit-sliced: one ballot per key bit.
__device__ __forceinline__ uint64_t match_any(int key, bool valid, int nbits) {
  uint64_t m = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = ((key >> b) & 1) != 0;
    const uint64_t bal = __ballot(valid && bit);
    m &= bit ? bal : ~bal;
  }
  return valid ? m : 0ull;
}

}  // namespace rlu
