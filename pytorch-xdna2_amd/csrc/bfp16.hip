// BFP16 ("bfp16ebs8") weight codec on the device: the reference's on-device weight
// format for its NPU conv3x3w kernels, produced bit-exactly from OIHW bf16 weights.
//
// Format (reference spec xdna_train/_designs/conv3x3w_host.py:49-82, host code
// xdna_train/_native/conv_pack.cpp:398-443 and, for the dX weights, :474-519): for
// output channels [128 n_block, +128) the (K x 128) matrix with K order (chunk, dy, dx,
// c) is laid out in blocks [kb = chunk*9 + tap][n / 16][k / 8][2][8 n][8 k]; each run of
// 8 consecutive k is one block of 9 bytes: the largest biased fp32 exponent of the 8
// values, then 8 int8 mantissas clamp(round_half_even(v * 2^(133 - e_max)), -128, 127).
// Channels past Cin / Cout are zeros.  The dX form reads w'[ci][co][dy][dx] =
// w[co][ci][2-dy][2-dx] (flip + swap) directly.
//
// The quantization is integer arithmetic on the bf16 bits: with significand M (hidden
// bit included; subnormals M = mantissa, exponent 1) the scaled value is
// M * 2^(E - e_max - 1), i.e. M shifted right by d = e_max + 1 - E with round-half-even;
// exact for every input, so no floating-point mode can change a byte.  Inf saturates
// to 127 / -128; NaN gives 0 (the reference's int conversion of NaN on x86).
//
// One thread per (kb, n/16, k/8): 16 blocks = 144 contiguous bytes, nine 16-byte stores.
#include "common.h"
#include "mfma.h"
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kBfpN = 128;                        // output channels per block
constexpr int64_t kBfpBytesPerChunk = 9 * 8 * 8 * 2 * 8 * 9;  // 82,944

// int8 mantissa (as a byte) of bf16 bits h in a block whose largest exponent is emax
__device__ inline uint32_t bfp16_mantissa(uint16_t h, int emax) {
  const int e = (h >> 7) & 0xFF;
  const int m7 = h & 0x7F;
  const bool neg = (h >> 15) != 0;
  if (e == 0xFF) {
    if (m7 != 0) return 0u;                       // NaN
    return neg ? 0x80u : 0x7Fu;                   // -inf -> -128, +inf -> 127
  }
  const int M = (e ? 128 : 0) + m7;
  const int E = e ? e : 1;
  const int d = min(emax + 1 - E, 31);            // >= 0
  int q = M >> d;
  if (d > 0) {
    const int rem = M & ((1 << d) - 1), half = 1 << (d - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
  }
  int v = neg ? -q : q;
  v = v > 127 ? 127 : (v < -128 ? -128 : v);
  return uint32_t(v) & 0xFFu;
}

template <bool kDx>
__global__ __launch_bounds__(256) void bfp16_weights_kernel(const uint16_t* __restrict__ w,
                                                            uint8_t* __restrict__ dst, int Cout,
                                                            int Cin, int ld_n, int chunks,
                                                            int n_block) {
  // this conv: output channels n < Cout, input channels c < Cin; element (n, c, tap) is
  // w[n][c][tap] (forward) or w[c][n][8 - tap] of the forward weight (dX; ld_n = Cin_fwd)
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= chunks * 9 * 64) return;
  const int k8 = t & 7, n16 = (t >> 3) & 7, kb = t >> 6;
  const int chunk = kb / 9, tap = kb - chunk * 9;
  uint32_t out[36];
#pragma unroll
  for (int i = 0; i < 36; ++i) out[i] = 0;
#pragma unroll
  for (int blk = 0; blk < 16; ++blk) {
    const int n = kBfpN * n_block + n16 * 16 + blk;  // blk = two * 8 + nl
    uint16_t h[8];
    int emax = 0;
#pragma unroll
    for (int kl = 0; kl < 8; ++kl) {
      const int c = chunk * kKStep + k8 * 8 + kl;
      uint16_t v = 0;
      if (c < Cin && n < Cout)
        v = kDx ? w[(int64_t(c) * ld_n + n) * 9 + (8 - tap)] : w[(int64_t(n) * ld_n + c) * 9 + tap];
      h[kl] = v;
      emax = max(emax, (v >> 7) & 0xFF);
    }
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const uint32_t byte = i == 0 ? uint32_t(emax) : bfp16_mantissa(h[i - 1], emax);
      const int p = blk * 9 + i;                  // compile-time after unrolling
      out[p >> 2] |= byte << ((p & 3) * 8);
    }
  }
  u32x4_t* o = reinterpret_cast<u32x4_t*>(dst + int64_t(t) * 144);
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    u32x4_t v = {out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
    o[i] = v;
  }
}

// dst[8 b + i] = float(int8 mantissa i of block b) * 2^(e_b - 133)
__global__ __launch_bounds__(256) void bfp16_decode_kernel(const uint8_t* __restrict__ src,
                                                           float* __restrict__ dst, int64_t nblocks) {
  const int64_t b = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t* s = src + b * 9;
  const int e = s[0];
#pragma unroll
  for (int i = 0; i < 8; ++i) dst[b * 8 + i] = ldexpf(float(int8_t(s[1 + i])), e - 133);
}

// ---------------------------------------------------------------------------------
// Quantization in place of the format: every aligned run of 8 bf16 values becomes the
// values its bfp16ebs8 block decodes to, q * 2^(e_max - 133), as bf16 bits.  This is what
// the reference's NPU conv computes with (weights through the codec above, activations
// through the core's round-to-nearest-even conversion of 8-channel blocks; the emulation
// is restated in benchmarks/bfp16_training_gate.py:33-44).  The result is exact: |q| <= 128
// has at most 8 significant bits and e_max >= 1 puts its last bit at or above 2^-132, so
// it is a bf16 value (subnormal below 2^-126); a block whose largest exponent is 254 can
// round -1.99 * 2^127 to -128 * 2^121 = -2^128, which overflows to -inf, as the decode does
// in fp32.  Non-finite inputs: NaN stays NaN (0x7FC0; the reference's conv gives NaN
// outputs for NaN operands), +-inf saturate to +-127 / -128 at e_max = 255 and decode to
// +-inf; the other values of such a block are quantized against e_max = 255, as the codec
// does.
// ---------------------------------------------------------------------------------
__device__ inline uint32_t bfp16_value_bits(int q, int emax) {
  if (q == 0) return 0u;
  const uint32_t s = q < 0 ? 0x8000u : 0u;
  const int mag = q < 0 ? -q : q;                 // 1 .. 128
  const int k = 31 - __builtin_clz(uint32_t(mag));  // floor(log2 mag): 0 .. 7
  const int E = emax - 6 + k;                     // biased bf16 exponent of the value
  if (E >= 255) return s | 0x7F80u;               // overflow: inf
  if (E >= 1) return s | (uint32_t(E) << 7) | (uint32_t(mag << (7 - k)) & 0x7Fu);
  return s | uint32_t(mag << emax);               // subnormal: (mag << emax) * 2^-133, < 2^7
}

__device__ inline uint32_t bfp16_quant_bits(uint16_t h, int emax) {
  if ((h & 0x7F80u) == 0x7F80u && (h & 0x7Fu)) return 0x7FC0u;  // NaN
  return bfp16_value_bits(int(int8_t(uint8_t(bfp16_mantissa(h, emax)))), emax);
}

// one thread per 8-value block (16 bytes)
__global__ __launch_bounds__(256) void bfp16_quant8_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                           int64_t nblocks) {
  for (int64_t b = int64_t(blockIdx.x) * 256 + threadIdx.x; b < nblocks; b += int64_t(gridDim.x) * 256) {
    const u32x4_t v = src[b];
    uint16_t h[8];
    int emax = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[2 * i] = uint16_t(v[i] & 0xFFFFu);
      h[2 * i + 1] = uint16_t(v[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) emax = max(emax, (h[i] >> 7) & 0xFF);
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = bfp16_quant_bits(h[2 * i], emax) | (bfp16_quant_bits(h[2 * i + 1], emax) << 16);
    dst[b] = o;
  }
}

bool bfp16_args_ok(const char* what, const void* w, const void* dst, int Cout, int Cin, int chunks,
                   int n_block) {
  if (!w || !dst || Cout < 1 || Cin < 1 || chunks < 1 || n_block < 0 || chunks > (1 << 20)) {
    set_error(std::string(what) + ": invalid arguments");
    return false;
  }
  if (reinterpret_cast<uintptr_t>(dst) & 15) {
    set_error(std::string(what) + ": dst must be 16-byte aligned");
    return false;
  }
  return true;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

size_t xdna_conv3x3w_weights_bfp16_bytes(int chunks) {
  return chunks < 1 ? 0 : size_t(chunks) * size_t(kBfpBytesPerChunk);
}

int xdna_conv3x3w_pack_weights_bfp16(const uint16_t* w, uint8_t* dst, int Cout, int Cin, int chunks,
                                     int n_block, void* stream) {
  if (!bfp16_args_ok("xdna_conv3x3w_pack_weights_bfp16", w, dst, Cout, Cin, chunks, n_block)) return -1;
  if (!admit_launch("xdna_conv3x3w_pack_weights_bfp16")) return -1;
  const int threads = chunks * 9 * 64;
  bfp16_weights_kernel<false><<<unsigned(ceil_div(threads, 256)), 256, 0, as_stream(stream)>>>(
      w, dst, Cout, Cin, Cin, chunks, n_block);
  return check_launch("xdna_conv3x3w_pack_weights_bfp16");
}

int xdna_conv3x3w_pack_weights_dx_bfp16(const uint16_t* w, uint8_t* dst, int Cout_fwd, int Cin_fwd,
                                        int chunks, int n_block, void* stream) {
  if (!bfp16_args_ok("xdna_conv3x3w_pack_weights_dx_bfp16", w, dst, Cout_fwd, Cin_fwd, chunks, n_block))
    return -1;
  if (!admit_launch("xdna_conv3x3w_pack_weights_dx_bfp16")) return -1;
  const int threads = chunks * 9 * 64;
  // the dX conv: input channels Cout_fwd, output channels Cin_fwd
  bfp16_weights_kernel<true><<<unsigned(ceil_div(threads, 256)), 256, 0, as_stream(stream)>>>(
      w, dst, Cin_fwd, Cout_fwd, Cin_fwd, chunks, n_block);
  return check_launch("xdna_conv3x3w_pack_weights_dx_bfp16");
}

int xdna_bfp16_quantize8_bf16(const uint16_t* src, uint16_t* dst, int64_t nblocks, void* stream) {
  if (nblocks < 0 || (nblocks > 0 && (!src || !dst))) {
    set_error("xdna_bfp16_quantize8_bf16: invalid arguments");
    return -1;
  }
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) {
    set_error("xdna_bfp16_quantize8_bf16: buffers must be 16-byte aligned");
    return -1;
  }
  if (nblocks == 0) return 0;
  if (!admit_launch("xdna_bfp16_quantize8_bf16")) return -1;
  bfp16_quant8_kernel<<<unsigned(std::min<int64_t>(ceil_div(nblocks, 256), 16384)), 256, 0, as_stream(stream)>>>(
      reinterpret_cast<const u32x4_t*>(src), reinterpret_cast<u32x4_t*>(dst), nblocks);
  return check_launch("xdna_bfp16_quantize8_bf16");
}

int xdna_bfp16_decode_f32(const uint8_t* src, float* dst, int64_t nblocks, void* stream) {
  if (nblocks < 0 || (nblocks > 0 && (!src || !dst))) {
    set_error("xdna_bfp16_decode_f32: invalid arguments");
    return -1;
  }
  if (nblocks == 0) return 0;
  if (!admit_launch("xdna_bfp16_decode_f32")) return -1;
  bfp16_decode_kernel<<<unsigned(ceil_div(nblocks, 256)), 256, 0, as_stream(stream)>>>(src, dst, nblocks);
  return check_launch("xdna_bfp16_decode_f32");
}

}  // extern "C"
