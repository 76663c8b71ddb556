// Resampling of NCHW bf16 planes: nearest-neighbour 2x upsampling and its gradient (the
// style generator's "nearest up x2" layers), and the stride-2 sampling that runs 3x3 /
// stride-2 convs through the stride-1 conv kernels (below).
//
// Upsampling: for an exact factor of 2, PyTorch's nearest source index floor(dst * 0.5) is
// dst / 2 (its scale 1/2 is exact in fp32), so
//   y[p][oy][ox] = x[p][oy / 2][ox / 2],
// and the gradient sums each 2x2 block of dy in fp32 in row-major order, (0,0), (0,1),
// (1,0), (1,1), then rounds once to bf16, as PyTorch's backward accumulates in float.
// The reference runs both from PyTorch's CPU kernels through its zero-copy fallback
// (torch_xdna_device.cpp:5124-5260).
//
// One thread per input pixel: the forward reads 2 bytes and writes two 4-byte pairs, the
// backward reads two 4-byte pairs and writes 2 bytes (output columns 2*ix are even, so
// the pairs are 4-byte aligned).  HBM-bound.
#include "common.h"
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

__global__ __launch_bounds__(256) void upsample2x_kernel(const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int64_t n, int H,
                                                         int W) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int64_t row = i / W;  // plane * H + iy
    const int ix = int(i - row * W);
    const uint32_t v = x[i];
    const uint32_t pair = v | (v << 16);
    uint32_t* o = reinterpret_cast<uint32_t*>(y + (2 * row) * (2 * int64_t(W)) + 2 * ix);
    o[0] = pair;
    o[W] = pair;  // the next output row: 2W elements = W pairs further
  }
  (void)H;
}

__global__ __launch_bounds__(256) void upsample2x_bwd_kernel(const uint16_t* __restrict__ dy,
                                                             uint16_t* __restrict__ dx, int64_t n, int H,
                                                             int W) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int64_t row = i / W;
    const int ix = int(i - row * W);
    const uint32_t* g = reinterpret_cast<const uint32_t*>(dy + (2 * row) * (2 * int64_t(W)) + 2 * ix);
    const uint32_t a = g[0], b = g[W];
    float s = __uint_as_float(a << 16);
    s += __uint_as_float(a & 0xFFFF0000u);
    s += __uint_as_float(b << 16);
    s += __uint_as_float(b & 0xFFFF0000u);
    dx[i] = f32_to_bf16(s);
  }
  (void)H;
}

// Stride-2 sampling for 3x3 / stride-2 / pad-1 convs run through the stride-1 kernels:
// y[p][oy][ox] = full[p][2 oy][2 ox] (forward: every other output of the stride-1 conv),
// and the spread of a gradient onto the stride-1 grid, full[p][y][x] = dy[p][y/2][x/2] at
// even (y, x) and 0 elsewhere (the input / weight gradients then run at stride 1; the
// zeros add nothing to their sums).  Full planes H x W, sampled ceil(H/2) x ceil(W/2).
//
// Widths that are multiples of 4 (every ResNet and style-network plane) take the vector
// forms: one thread per 8 bytes of the full grid (4 pixels) and 4 bytes of the sampled one
// (2 pixels), 32-bit index arithmetic; other widths take one thread per element.

// y[r][2q .. 2q+1] = full[row(r)][4q], full[row(r)][4q + 2]; r = plane * Ho + oy, Wq = W / 4
__global__ __launch_bounds__(256) void subsample2_vec_kernel(const uint2* __restrict__ full,
                                                             uint32_t* __restrict__ y, uint32_t n, uint32_t Wq,
                                                             uint32_t H, uint32_t Ho) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
    const uint32_t r = i / Wq, q = i - r * Wq;
    const uint32_t p = r / Ho, oy = r - p * Ho;
    const uint2 v = full[(p * H + 2u * oy) * Wq + q];
    y[i] = (v.x & 0xFFFFu) | (v.y << 16);
  }
}

// full[row][4q .. 4q+3] = (dy[p][y/2][2q], 0, dy[p][y/2][2q+1], 0) on even rows y, zeros on
// odd ones; row = plane * H + y, Wq = W / 4 = Wo / 2
__global__ __launch_bounds__(256) void dilate2_vec_kernel(const uint32_t* __restrict__ dy,
                                                          uint2* __restrict__ full, uint32_t n, uint32_t Wq,
                                                          uint32_t H, uint32_t Ho) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
    const uint32_t row = i / Wq, q = i - row * Wq;
    const uint32_t p = row / H, yy = row - p * H;
    uint2 o = make_uint2(0u, 0u);
    if ((yy & 1u) == 0) {
      const uint32_t v = dy[(p * Ho + yy / 2u) * Wq + q];
      o = make_uint2(v & 0xFFFFu, v >> 16);
    }
    full[i] = o;
  }
}

// vector forms apply: W % 4 == 0, both buffers 8-byte aligned, index range in 32 bits
bool resample_vec(const void* a, const void* b, int64_t planes, int H, int W) {
  return W % 4 == 0 && ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 7) == 0 &&
         planes * H * int64_t(W) < (int64_t(1) << 31);
}
__global__ __launch_bounds__(256) void subsample2_kernel(const uint16_t* __restrict__ full,
                                                         uint16_t* __restrict__ y, int64_t n, int H, int W) {
  const int Ho = (H + 1) / 2, Wo = (W + 1) / 2;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int64_t row = i / Wo;  // plane * Ho + oy
    const int ox = int(i - row * Wo);
    const int64_t p = row / Ho;
    const int oy = int(row - p * Ho);
    y[i] = full[(p * H + 2 * oy) * int64_t(W) + 2 * ox];
  }
}

__global__ __launch_bounds__(256) void dilate2_kernel(const uint16_t* __restrict__ dy,
                                                      uint16_t* __restrict__ full, int64_t n, int H, int W) {
  const int Ho = (H + 1) / 2, Wo = (W + 1) / 2;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int64_t row = i / W;  // plane * H + y
    const int x = int(i - row * W);
    const int64_t p = row / H;
    const int y = int(row - p * H);
    const bool even = ((x | y) & 1) == 0;
    const uint16_t v = dy[even ? (p * Ho + y / 2) * int64_t(Wo) + x / 2 : 0];
    full[i] = even ? v : uint16_t(0);
  }
}

bool resample_args(const char* what, const void* src, const void* dst, int64_t planes, int H, int W) {
  if (planes < 0 || H < 0 || W < 0 || ((planes * H * W) > 0 && (!src || !dst))) {
    set_error(std::string(what) + ": invalid arguments");
    return false;
  }
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 3) {
    set_error(std::string(what) + ": buffers must be 4-byte aligned");
    return false;
  }
  return true;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_upsample_nearest2x_bf16(const uint16_t* x, uint16_t* y, int64_t planes, int H, int W, void* stream) {
  if (!resample_args("xdna_upsample_nearest2x_bf16", x, y, planes, H, W)) return -1;
  const int64_t n = planes * H * W;
  if (n == 0) return 0;
  if (!admit_launch("xdna_upsample_nearest2x_bf16")) return -1;
  upsample2x_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 65536)), 256, 0, as_stream(stream)>>>(x, y, n,
                                                                                                          H, W);
  return check_launch("xdna_upsample_nearest2x_bf16");
}

int xdna_upsample_nearest2x_bwd_bf16(const uint16_t* dy, uint16_t* dx, int64_t planes, int H, int W,
                                     void* stream) {
  if (!resample_args("xdna_upsample_nearest2x_bwd_bf16", dy, dx, planes, H, W)) return -1;
  const int64_t n = planes * H * W;
  if (n == 0) return 0;
  if (!admit_launch("xdna_upsample_nearest2x_bwd_bf16")) return -1;
  upsample2x_bwd_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 65536)), 256, 0, as_stream(stream)>>>(
      dy, dx, n, H, W);
  return check_launch("xdna_upsample_nearest2x_bwd_bf16");
}

int xdna_subsample2_bf16(const uint16_t* full, uint16_t* y, int64_t planes, int H, int W, void* stream) {
  if (planes < 0 || H < 0 || W < 0 || (planes * H * W > 0 && (!full || !y))) {
    set_error("xdna_subsample2_bf16: invalid arguments");
    return -1;
  }
  const int64_t n = planes * ((H + 1) / 2) * ((W + 1) / 2);
  if (n == 0) return 0;
  if (!admit_launch("xdna_subsample2_bf16")) return -1;
  if (resample_vec(full, y, planes, H, W)) {
    const uint32_t nv = uint32_t(n / 2);  // 2 output pixels per thread (Wo = W / 2 is even)
    subsample2_vec_kernel<<<unsigned(std::min<int64_t>(ceil_div(nv, 256), 65536)), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<const uint2*>(full), reinterpret_cast<uint32_t*>(y), nv, uint32_t(W / 4), uint32_t(H),
        uint32_t((H + 1) / 2));
  } else {
    subsample2_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 65536)), 256, 0, as_stream(stream)>>>(full, y,
                                                                                                            n, H, W);
  }
  return check_launch("xdna_subsample2_bf16");
}

int xdna_dilate2_bf16(const uint16_t* dy, uint16_t* full, int64_t planes, int H, int W, void* stream) {
  if (planes < 0 || H < 0 || W < 0 || (planes * H * W > 0 && (!full || !dy))) {
    set_error("xdna_dilate2_bf16: invalid arguments");
    return -1;
  }
  const int64_t n = planes * H * W;
  if (n == 0) return 0;
  if (!admit_launch("xdna_dilate2_bf16")) return -1;
  if (resample_vec(dy, full, planes, H, W)) {
    const uint32_t nv = uint32_t(n / 4);  // 4 full-grid pixels per thread
    dilate2_vec_kernel<<<unsigned(std::min<int64_t>(ceil_div(nv, 256), 65536)), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<const uint32_t*>(dy), reinterpret_cast<uint2*>(full), nv, uint32_t(W / 4), uint32_t(H),
        uint32_t((H + 1) / 2));
  } else {
    dilate2_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 65536)), 256, 0, as_stream(stream)>>>(dy, full, n,
                                                                                                         H, W);
  }
  return check_launch("xdna_dilate2_bf16");
}

}  // extern "C"
