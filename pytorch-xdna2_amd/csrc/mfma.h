// CDNA4 (gfx950) MFMA building blocks: bf16 32x32x16 with fp32 accumulation.
//
// v_mfma_f32_32x32x16_bf16, per 64-lane wave:
//   A fragment (32 x 16): lane l holds A[l % 32][8*(l/32) .. 8*(l/32)+7]
//   B fragment (16 x 32): lane l holds B[8*(l/32) .. +7][l % 32]
//   D (32 x 32, 16 fp32 per lane): register i of lane l holds
//       D[8*(i/4) + 4*(l/32) + (i%4)][l % 32]
// A and B share one k-assignment per (lane half, slot), so any consistent
// permutation of k in both operands gives the same sum.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace xdna {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// 16-byte register vector (HIP's uint4 is a struct over a union, which keeps arrays of it
// in scratch memory; this native vector type stays in VGPRs)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline f32x16_t mfma_32x32x16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ inline bf16x8_t as_bf16x8(const uint4& u) { return __builtin_bit_cast(bf16x8_t, u); }
__device__ inline bf16x8_t as_bf16x8(const u32x4_t& u) { return __builtin_bit_cast(bf16x8_t, u); }

// Row (within a 32x32 tile) of accumulator register i for lane l.
__device__ inline int mfma_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

__device__ inline f32x16_t zero_acc() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

}  // namespace xdna
