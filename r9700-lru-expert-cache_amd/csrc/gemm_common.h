// Operand types, the fp8 MFMA and the weight-set descriptor shared by the grouped GEMMs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rlu {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v8i pack8(v4u lo, v4u hi) {
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

__device__ __forceinline__ v4f mfma_f8(v8i a, v8i b) {
  // formats 0/0 = e4m3 x e4m3; E8M0 scale 127 = 2^0 on both operands
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                          0, 127, 0, 127);
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

// Register ring depth: D steps of A (32 B) + NPW weight strips (32 B each) per lane.
__host__ __device__ constexpr int ring_of(int npw) {
  return npw == 1 ? 8 : npw == 2 ? 5 : npw == 4 ? 3 : 2;
}

// CUs of the current device, looked up once per device (256 on MI355X).
static inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

}  // namespace rlu
