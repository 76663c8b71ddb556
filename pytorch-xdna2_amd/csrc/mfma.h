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

// ---------------------------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16, per 64-lane wave:
//   A fragment (16 x 32): lane l holds A[l % 16][8*(l/16) .. 8*(l/16)+7]
//   B fragment (32 x 16): lane l holds B[8*(l/16) .. +7][l % 16]
//   D (16 x 16, 4 fp32 per lane): register r of lane l holds D[4*(l/16) + r][l % 16]
// ---------------------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The MFMA as an inline-assembly statement on an AGPR quad updated in place: with 64
// accumulators filling the 256 AGPRs, the compiler's allocation of the builtin's results
// renames them through v_accvgpr copies every k-step.  The compiler then does not see an
// MFMA, so the hazards it would pad are padded by the kernel (mfma16_fence): wait states
// between the last MFMA writing an accumulator and any other read of it (VALU, stores), and
// between VALU writes of an accumulator (its initial value) and the first MFMA reading it.
// Operands A and B must come straight from LDS reads, whose completion the compiler's
// s_waitcnt covers for inline-assembly operands as for any instruction (an operand written
// by a VALU instruction would need 2 wait states before the MFMA, which nothing pads
// here); a kernel updates each accumulator once per k-step of many MFMAs, so no MFMA reads
// a result of the MFMA just before it.
// kInit: the first k-step's MFMA, accumulating onto the inline constant 0 (no zero-filled
// accumulators to set up)
template <bool kInit>
__device__ inline void mfma16_acc(f32x4_t& c, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (kInit)
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// 24 wait states (the longest MFMA dependency in the gfx9 family needs 19), then every
// accumulator of the set passed through volatile statements, so that no read or MFMA of
// them can be scheduled before the wait states
template <int MI, int NJ>
__device__ inline void mfma16_fence(f32x4_t (&acc)[MI][NJ]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) asm volatile("; mfma16 fence" : "+a"(acc[i][j]));
}

// ---------------------------------------------------------------------------------------
// gfx950's 16-byte LDS DMA (buffer_load_dwordx4 ... lds): one instruction per wave writes
// 64 x 16 bytes contiguously at an LDS base (lane L at base + 16 L; a lane whose offset is
// past the buffer's range writes zeros), with no register staging and no LDS store.
// ---------------------------------------------------------------------------------------
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource of `bytes` bytes at `base`: stride 0 (offsets in bytes), the dword-3
// flags of __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000).
__device__ inline i32x4_t lds_dma_rsrc(const void* base, int bytes) {
  const uint64_t b = uint64_t(base);
  return i32x4_t{int(uint32_t(b)), int(uint32_t(b >> 32) & 0xFFFF), bytes, 0x00020000};
}

// One 16-byte LDS DMA of byte offset voff of the resource into lds + 16 L (the LDS base
// and the resource are wave-uniform: lane 0's are used).  Issued from
// inline assembly on purpose: for the compiler's builtin, its wait insertion makes every
// later LDS read wait for all outstanding DMA (vmcnt(0)) whatever the read's address, which
// serializes a multi-buffered pipeline.  The caller tracks completion with counted
// s_waitcnt vmcnt (lds_dma_wait) before the barrier that publishes a buffer.  M0 (the LDS
// base) is set inside the statement; kernels that use this helper use M0 for nothing else.
__device__ inline void lds_dma16(const i32x4_t& rsrc, const uint16_t* lds, int voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      uint32_t(uintptr_t((__attribute__((address_space(3))) const uint16_t*)lds)));
  const i32x4_t rs = {__builtin_amdgcn_readfirstlane(rsrc[0]), __builtin_amdgcn_readfirstlane(rsrc[1]),
                      __builtin_amdgcn_readfirstlane(rsrc[2]), __builtin_amdgcn_readfirstlane(rsrc[3])};
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rs)
               : "m0");
}

// LDS byte address of a shared-memory pointer, made wave-uniform (an SGPR value)
__device__ inline uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(uint32_t(uintptr_t((__attribute__((address_space(3))) const void*)p)));
}

// lds_dma16 with the destination's LDS byte address and the resource already wave-uniform
// (computed once outside a loop: no per-load readfirstlane or address-space conversion)
__device__ inline void lds_dma16_m0(const i32x4_t& rs, uint32_t m0, int voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rs)
               : "m0");
}

// a resource descriptor made wave-uniform
__device__ inline i32x4_t uniform_rsrc(const i32x4_t& r) {
  return i32x4_t{__builtin_amdgcn_readfirstlane(r[0]), __builtin_amdgcn_readfirstlane(r[1]),
                 __builtin_amdgcn_readfirstlane(r[2]), __builtin_amdgcn_readfirstlane(r[3])};
}

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt at their maxima), gfx9 encoding
template <int n>
__device__ inline void lds_dma_wait() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) alone: this wave's LDS reads have returned
__device__ inline void lds_reads_wait() { __builtin_amdgcn_s_waitcnt((7 << 4) | (0 << 8) | 15 | (3 << 14)); }

__device__ inline f32x16_t zero_acc() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

}  // namespace xdna
