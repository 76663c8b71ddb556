// conv3x3w layouts on the device: NCHW bf16 <-> padded-grid row tiles.
//
// Layout (reference spec xdna_train/_designs/conv3x3w_host.py:32-46, 85-140;
// host implementation xdna_train/_native/conv_pack.cpp:632-743):
//   packed input  [groups][chunks][2126][64] bf16.  Virtual image vb = b*S + s,
//   grid row of data column j at image row y is p = (vb*(H+2) + y + 1)*wp + j + 1.
//   Group g holds rows [2048 g, 2048 g + 2126): its last 78 rows duplicate the
//   first 78 of group g+1.  Channels beyond C in the last chunk, border rows and
//   the tail of the last group are never written (the caller zero-fills once).
//   raw output rows [p][128]: output pixel (y, t) of virtual image vb sits at row
//   (vb*(H+2) + y)*wp + first + t, first = 0 (S == 1) or 1 (strips).
//
// Both kernels are HBM-bound byte moves.  One thread per packed row (pixel x chunk):
// consecutive threads take consecutive image columns, so each of the (up to) 64
// channel loads of a wave is one contiguous run of NCHW, and each thread writes its
// own 128-byte row with 16-byte stores.  Unpack is the mirror image.
#include "common.h"
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

template <bool kVecStore>
__global__ __launch_bounds__(256) void pack_rows_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int C, int H, int W, int S,
    int So, int Wg, int wp, int halo_zero, int chunks, int g0, int ng, int v0, int64_t plo,
    int64_t phi, int64_t n_threads) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_threads) return;
  const int j = int(t % Wg);
  t /= Wg;
  const int y = int(t % H);
  t /= H;
  const int chunk = int(t % chunks);
  const int vb = v0 + int(t / chunks);
  const int cc = min(C - chunk * kKStep, kKStep);
  if (cc <= 0) return;
  const int b = vb / S, s = vb % S;
  const int x = (S == 1 ? 0 : s * So - 1) + j;  // source column of data column j
  if (x < 0 || x >= W) return;
  const int64_t p = (int64_t(vb) * (H + 2) + y + 1) * wp + 1 + j;
  if (p < plo || p >= phi) return;
  const int64_t g = p / kGroupOutRows;
  const int r = int(p - g * kGroupOutRows);
  const bool main_w = g >= g0 && g < int64_t(g0) + ng;
  const bool halo_w = g > g0 && g <= int64_t(g0) + ng && r + kGroupOutRows < kGroupRows;
  if (!main_w && !halo_w) return;

  uint32_t v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = 0;
  const bool zero = halo_zero && S > 1 && (j == 0 || j == Wg - 1);
  if (!zero) {
    const int64_t plane = int64_t(H) * W;
    const uint16_t* sp = src + ((int64_t(b) * C + chunk * kKStep) * H + y) * W + x;
#pragma unroll
    for (int c = 0; c < kKStep; ++c) {
      if (c < cc) {
        const uint32_t h = sp[c * plane];
        v[c >> 1] |= (c & 1) ? (h << 16) : h;
      }
    }
  }
  uint16_t* rows[2];
  int nrows = 0;
  if (main_w) rows[nrows++] = dst + ((int64_t(g - g0) * chunks + chunk) * kGroupRows + r) * kKStep;
  if (halo_w)
    rows[nrows++] =
        dst + ((int64_t(g - 1 - g0) * chunks + chunk) * kGroupRows + r + kGroupOutRows) * kKStep;
  for (int k = 0; k < nrows; ++k) {
    uint16_t* d = rows[k];
    if (kVecStore && cc == kKStep) {
      uint4* d4 = reinterpret_cast<uint4*>(d);
#pragma unroll
      for (int q = 0; q < 8; ++q) d4[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
#pragma unroll
      for (int c = 0; c < kKStep; ++c)
        if (c < cc) d[c] = uint16_t((c & 1) ? (v[c >> 1] >> 16) : (v[c >> 1] & 0xFFFF));
    }
  }
}

template <bool kVecLoad>
__global__ __launch_bounds__(256) void unpack_rows_kernel(
    const uint16_t* __restrict__ c, uint16_t* __restrict__ dst, int H, int W, int S, int So,
    int wp, int cout_valid, int C_total, int c_start, int64_t p0, int64_t p1, int v0, int TW,
    int64_t n_threads) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_threads) return;
  const int tc = int(t % TW);
  t /= TW;
  const int y = int(t % H);
  const int vb = v0 + int(t / H);
  const int b = vb / S, s = vb % S;
  const int first = S == 1 ? 0 : 1;
  const int cols = S == 1 ? W : min(So, W - s * So);
  if (tc >= cols) return;
  const int64_t p = (int64_t(vb) * (H + 2) + y) * wp + first + tc;
  if (p < p0 || p >= p1) return;
  const int x = (S == 1 ? 0 : s * So) + tc;
  const uint16_t* row = c + (p - p0) * kRawN;
  const int64_t plane = int64_t(H) * W;
  uint16_t* out = dst + ((int64_t(b) * C_total + c_start) * H + y) * W + x;
  if (kVecLoad) {
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int q = 0; q < kRawN / 8; ++q) {
      if (q * 8 < cout_valid) {
        const uint4 w = r4[q];
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int n = q * 8 + e;
          if (n < cout_valid) out[n * plane] = uint16_t((e & 1) ? (u[e >> 1] >> 16) : (u[e >> 1] & 0xFFFF));
        }
      }
    }
  } else {
    for (int n = 0; n < cout_valid; ++n) out[n * plane] = row[n];
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int pack_launch(const char* what, const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                int S, int So, int halo_zero, int chunks, int g0, int ng, void* stream) {
  if (B < 0 || C < 0 || H < 0 || W < 0 || chunks < 0 || S < 1 || g0 < 0 || ng < 0 ||
      (S > 1 && So < 1)) {
    set_error(std::string(what) + ": invalid geometry");
    return -1;
  }
  if (B == 0 || C == 0 || H == 0 || W == 0 || chunks == 0 || ng == 0) return 0;
  const int Wg = S == 1 ? W : So + 2;
  const int wp = Wg + 2;
  const int64_t Bv = int64_t(B) * S;
  const int64_t img = int64_t(H + 2) * wp;
  const int64_t plo = int64_t(g0) * kGroupOutRows;
  const int64_t phi = int64_t(g0 + ng) * kGroupOutRows + (kGroupRows - kGroupOutRows);
  const int64_t v0 = plo / img;
  const int64_t v1 = std::min<int64_t>((phi - 1) / img + 1, Bv);
  if (v1 <= v0) return 0;
  if (!admit_launch(what)) return -1;
  const int64_t n = (v1 - v0) * chunks * H * Wg;
  const int threads = 256;
  const int64_t blocks = ceil_div(n, threads);
  if (aligned16(dst))
    pack_rows_kernel<true><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        src, dst, C, H, W, S, So, Wg, wp, halo_zero, chunks, g0, ng, int(v0), plo, phi, n);
  else
    pack_rows_kernel<false><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        src, dst, C, H, W, S, So, Wg, wp, halo_zero, chunks, g0, ng, int(v0), plo, phi, n);
  return check_launch(what);
}

int unpack_launch(const char* what, const uint16_t* c, uint16_t* dst, int B, int H, int W, int S,
                  int So, int cout_valid, int C_total, int c_start, int64_t p0, int64_t p1,
                  void* stream) {
  if (B < 0 || H < 0 || W < 0 || S < 1 || cout_valid < 0 || cout_valid > kRawN ||
      c_start < 0 || c_start + cout_valid > C_total || (S > 1 && So < 1)) {
    set_error(std::string(what) + ": invalid geometry");
    return -1;
  }
  if (B == 0 || H == 0 || W == 0 || cout_valid == 0 || p1 <= p0) return 0;
  const int Wg = S == 1 ? W : So + 2;
  const int wp = Wg + 2;
  const int64_t Bv = int64_t(B) * S;
  const int64_t img = int64_t(H + 2) * wp;
  const int64_t v0 = p0 / img;
  const int64_t v1 = std::min<int64_t>((p1 - 1) / img + 1, Bv);
  if (v1 <= v0) return 0;
  if (!admit_launch(what)) return -1;
  const int TW = S == 1 ? W : So;
  const int64_t n = (v1 - v0) * H * TW;
  const int threads = 256;
  const int64_t blocks = ceil_div(n, threads);
  if (aligned16(c))
    unpack_rows_kernel<true><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        c, dst, H, W, S, So, wp, cout_valid, C_total, c_start, p0, p1, int(v0), TW, n);
  else
    unpack_rows_kernel<false><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        c, dst, H, W, S, So, wp, cout_valid, C_total, c_start, p0, p1, int(v0), TW, n);
  return check_launch(what);
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_conv3x3w_pack_input_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                                  int chunks, void* stream) {
  const int64_t m_total = int64_t(B) * (H + 2) * (W + 2);
  const int groups = int(ceil_div(m_total, kGroupOutRows));
  return pack_launch("xdna_conv3x3w_pack_input_bf16", src, dst, B, C, H, W, 1, W, 0, chunks, 0,
                     groups, stream);
}

int xdna_conv3x3w_pack_input_range_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H,
                                        int W, int chunks, int g0, int ng, void* stream) {
  return pack_launch("xdna_conv3x3w_pack_input_range_bf16", src, dst, B, C, H, W, 1, W, 0, chunks,
                     g0, ng, stream);
}

int xdna_conv3x3w_pack_input_strips_range_bf16(const uint16_t* src, uint16_t* dst, int B, int C,
                                               int H, int W, int S, int So, int halo_zero,
                                               int chunks, int g0, int ng, void* stream) {
  return pack_launch("xdna_conv3x3w_pack_input_strips_range_bf16", src, dst, B, C, H, W, S, So,
                     halo_zero, chunks, g0, ng, stream);
}

int xdna_conv3x3w_unpack_output_bf16(const uint16_t* c, uint16_t* dst, int B, int H, int W,
                                     int cout_valid, int C_total, int c_start, void* stream) {
  const int64_t m_total = int64_t(B) * (H + 2) * (W + 2);
  return unpack_launch("xdna_conv3x3w_unpack_output_bf16", c, dst, B, H, W, 1, W, cout_valid,
                       C_total, c_start, 0, m_total, stream);
}

int xdna_conv3x3w_unpack_output_range_bf16(const uint16_t* c, uint16_t* dst, int B, int H, int W,
                                           int cout_valid, int C_total, int c_start, int p0,
                                           int p1, void* stream) {
  return unpack_launch("xdna_conv3x3w_unpack_output_range_bf16", c, dst, B, H, W, 1, W,
                       cout_valid, C_total, c_start, p0, p1, stream);
}

int xdna_conv3x3w_unpack_output_strips_range_bf16(const uint16_t* c, uint16_t* dst, int B, int H,
                                                  int W, int S, int So, int cout_valid,
                                                  int C_total, int c_start, int p0, int p1,
                                                  void* stream) {
  return unpack_launch("xdna_conv3x3w_unpack_output_strips_range_bf16", c, dst, B, H, W, S, So,
                       cout_valid, C_total, c_start, p0, p1, stream);
}

int xdna_conv3x3w_geometry(int B, int Cin, int H, int W, int64_t* out7) {
  if (B < 1 || Cin < 1 || H < 1 || W < 1) {
    set_error("xdna_conv3x3w_geometry: invalid shape");
    return -1;
  }
  const ConvGeom g = conv_geom(B, H, W);
  out7[0] = g.st.S;
  out7[1] = g.st.So;
  out7[2] = g.st.Wg;
  out7[3] = g.st.wp;
  out7[4] = g.groups;
  out7[5] = ceil_div(Cin, kKStep);
  out7[6] = g.m_total;
  return 0;
}

}  // extern "C"
