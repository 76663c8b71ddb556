// Kernels of the fused training regions on gfx950: the frozen-feature (perceptual) loss of
// the reference's xdna_train/regions.py:1-425 (its host kernels: _native/region_kernels.cpp:
// 51-340), re-designed for device memory.  The region's convolutions are the 3x3 conv path
// with a fused ReLU epilogue; what is left for these kernels is one pass per tensor:
//
//   * 2x2 / stride-2 max-pool (PyTorch's rule: the first maximum of the window in row-major
//     order wins, a NaN wins over any number);
//   * tap loss terms as fp32 partial sums over a fixed partition of the elements (one slab
//     per tap, each pre-scaled), and one fixed-order finish into the scalar loss, so the
//     loss never leaves the device and the same inputs give the same bits;
//   * the backward of ReLU, max-pool and the tap terms in one elementwise pass:
//       out = mask ? bf16(base + extra + scale * go * (a - b)) : 0
//     with base the incoming gradient or, through a max-pool, the pooled gradient routed
//     to the window's maximum (recomputed from the pool input, same rule as the forward),
//     and mask the ReLU result's positivity (threshold_backward: a NaN result passes);
//   * the Gram-matrix style term: sum of (G / chw - T)^2, and the symmetric matrix S with
//     which the gradient with respect to the features F (G = F F^T) is one product, S F.
//
// bf16 storage, fp32 arithmetic, one rounding per output, as the reference's region
// contract states (regions.py:29-32).  Scalars that come from autograd (the loss's
// incoming gradient) are read on the device, so a region's backward needs no host sync and
// can be captured in a graph.
#include "common.h"

#include <algorithm>
#include <cmath>
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kRegionThreads = 256;
constexpr int kLossParts = 2048;  // partial sums per tap term (fixed partition)

__device__ inline float go_value(const void* go, int go_dtype) {
  if (go_dtype == 1) return *static_cast<const float*>(go);
  if (go_dtype == 2) return bf16_to_f32(*static_cast<const uint16_t*>(go));
  return 1.0f;
}

// Row-major index (0..3) of the window maximum: (0,0), (0,1), (1,0), (1,1); a value
// replaces the running maximum when it is larger or NaN (PyTorch's max_pool2d rule).
__device__ inline int window_argmax(const uint16_t* w0, int W, float& m) {
  const float v[4] = {bf16_to_f32(w0[0]), bf16_to_f32(w0[1]), bf16_to_f32(w0[W]), bf16_to_f32(w0[W + 1])};
  m = -INFINITY;
  int k = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (v[j] > m || v[j] != v[j]) {
      m = v[j];
      k = j;
    }
  return k;
}

__global__ __launch_bounds__(kRegionThreads) void maxpool2_kernel(const uint16_t* __restrict__ x,
                                                                  uint16_t* __restrict__ y, int64_t planes, int H,
                                                                  int W, int Ho, int Wo) {
  const int64_t n = planes * Ho * Wo;
  for (int64_t i = int64_t(blockIdx.x) * kRegionThreads + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kRegionThreads) {
    const int64_t p = i / (int64_t(Ho) * Wo);
    const int r = int(i - p * Ho * Wo);
    const int oy = r / Wo, ox = r - oy * Wo;
    float m;
    window_argmax(x + (p * H + 2 * oy) * W + 2 * ox, W, m);
    y[i] = f32_to_bf16(m);
  }
}

struct BwdArgs {
  const uint16_t* r;      // ReLU result (mask), or null
  const uint16_t* g;      // incoming gradient at this shape, or null
  const uint16_t* gp;     // incoming gradient at the pooled shape, or null
  const uint16_t* px;     // max-pool input (for the window maxima), with gp
  const uint16_t* extra;  // another gradient term at this shape, or null
  const uint16_t* ta;     // tap term a - b, or null
  const uint16_t* tb;
  const void* go;
  int go_dtype;
  float scale;
  uint16_t* out;
  int64_t planes;
  int H, W, Ho, Wo;
};

__global__ __launch_bounds__(kRegionThreads) void region_bwd_kernel(BwdArgs a) {
  const int64_t n = a.planes * a.H * a.W;
  const float s = a.ta ? a.scale * go_value(a.go, a.go_dtype) : 0.0f;
  for (int64_t i = int64_t(blockIdx.x) * kRegionThreads + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kRegionThreads) {
    if (a.r && bf16_to_f32(a.r[i]) <= 0.0f) {
      a.out[i] = 0;
      continue;
    }
    float v = 0.0f;
    if (a.g) {
      v = bf16_to_f32(a.g[i]);
    } else if (a.gp) {
      const int64_t p = i / (int64_t(a.H) * a.W);
      const int rem = int(i - p * a.H * a.W);
      const int y = rem / a.W, x = rem - y * a.W;
      const int oy = y >> 1, ox = x >> 1;
      if (oy < a.Ho && ox < a.Wo) {
        float m;
        const int k = window_argmax(a.px + (p * a.H + 2 * oy) * a.W + 2 * ox, a.W, m);
        if (k == ((y & 1) << 1) + (x & 1)) v = bf16_to_f32(a.gp[(p * a.Ho + oy) * a.Wo + ox]);
      }
    }
    if (a.extra) v += bf16_to_f32(a.extra[i]);
    if (a.ta) v += s * (bf16_to_f32(a.ta[i]) - bf16_to_f32(a.tb[i]));
    a.out[i] = f32_to_bf16(v);
  }
}

// part[blockIdx.x] = scale * sum over this block's elements of d^2, d = a - b (kind 0, both
// bf16) or d = a / chw - t (kind 1: a the bf16 Gram matrices [batch][cc], t fp32 targets
// with batch stride t_bstride, 0 for one target broadcast over the batch).  Block b sums
// elements b * 256 + tid + k * gridDim.x * 256 in that order per thread, then a fixed tree.
__global__ __launch_bounds__(kRegionThreads) void sqdiff_kernel(int kind, const uint16_t* __restrict__ a,
                                                                const uint16_t* __restrict__ b,
                                                                const float* __restrict__ t, int64_t t_bstride,
                                                                int64_t cc, float chw, int64_t n, float scale,
                                                                float* __restrict__ part) {
  float s = 0.0f;
  for (int64_t i = int64_t(blockIdx.x) * kRegionThreads + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kRegionThreads) {
    float d;
    if (kind == 0) {
      d = bf16_to_f32(a[i]) - bf16_to_f32(b[i]);
    } else {
      const int64_t bi = i / cc;
      d = bf16_to_f32(a[i]) / chw - t[bi * t_bstride + (i - bi * cc)];
    }
    s = fmaf(d, d, s);
  }
  __shared__ float red[kRegionThreads];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = kRegionThreads / 2; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = scale * red[0];
}

// loss = sum of part[0 .. n) in fp64, thread-strided then a fixed tree; written as fp32
// and bf16 scalars (either may be null).
constexpr int kFinishThreads = 1024;

__global__ __launch_bounds__(kFinishThreads) void finish_kernel(const float* __restrict__ part, int n,
                                                                float* __restrict__ out_f32,
                                                                uint16_t* __restrict__ out_bf16) {
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += kFinishThreads) s += double(part[i]);
  __shared__ double red[kFinishThreads];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = kFinishThreads / 2; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (out_f32) *out_f32 = float(red[0]);
    if (out_bf16) *out_bf16 = f32_to_bf16(float(red[0]));
  }
}

// S = bf16(coef * go * (d_ij + d_ji) / chw), d = G / chw - t, over C x C matrices: with
// G = F F^T, the gradient of coef / 2 * sum d^2 with respect to F is S F (both operands of
// the Gram product carry F), so one product gives it (coef = 2 w / N for w times a mean).
// Block (tj, ti, b) takes the 32 x 32 tile at rows ti*32, columns tj*32 of matrix b and
// stages the mirrored tile (rows tj*32, columns ti*32) of d in LDS, so both reads and the
// write are coalesced.
constexpr int kGT = 32;

__global__ __launch_bounds__(kRegionThreads) void gram_grad_kernel(const uint16_t* __restrict__ G,
                                                                   const float* __restrict__ t, int64_t t_bstride,
                                                                   int C, float chw, float coef, const void* go,
                                                                   int go_dtype, uint16_t* __restrict__ S) {
  const float c = coef * go_value(go, go_dtype);
  const int64_t cc = int64_t(C) * C;
  const int b = blockIdx.z, i0 = blockIdx.y * kGT, j0 = blockIdx.x * kGT;
  const uint16_t* Gb = G + b * cc;
  const float* tb = t + b * t_bstride;
  __shared__ float mir[kGT][kGT + 1];  // mir[x][y] = d at row j0 + y, column i0 + x
  const int tx = threadIdx.x % kGT, ty = threadIdx.x / kGT;  // 32 x 8
  for (int y = ty; y < kGT; y += kRegionThreads / kGT) {
    const int r = j0 + y, col = i0 + tx;
    float d = 0.0f;
    if (r < C && col < C) d = bf16_to_f32(Gb[int64_t(r) * C + col]) / chw - tb[int64_t(r) * C + col];
    mir[tx][y] = d;
  }
  __syncthreads();
  for (int y = ty; y < kGT; y += kRegionThreads / kGT) {
    const int r = i0 + y, col = j0 + tx;
    if (r >= C || col >= C) continue;
    const int64_t e = int64_t(r) * C + col;
    const float d = bf16_to_f32(Gb[e]) / chw - tb[e];
    S[b * cc + e] = f32_to_bf16(c * (d + mir[y][tx]) / chw);
  }
}

unsigned grid_for(int64_t n) { return unsigned(std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, kRegionThreads), 16384))); }

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_region_maxpool2_bf16(const uint16_t* x, uint16_t* y, int64_t planes, int H, int W, void* stream) {
  if (planes < 0 || H < 0 || W < 0) {
    set_error("xdna_region_maxpool2_bf16: invalid arguments");
    return -1;
  }
  const int Ho = H / 2, Wo = W / 2;
  if (planes == 0 || Ho == 0 || Wo == 0) return 0;  // nothing to write
  if (!x || !y) {
    set_error("xdna_region_maxpool2_bf16: null operand");
    return -1;
  }
  if (!admit_launch("xdna_region_maxpool2_bf16")) return -1;
  maxpool2_kernel<<<grid_for(planes * Ho * Wo), kRegionThreads, 0, as_stream(stream)>>>(x, y, planes, H, W, Ho, Wo);
  return check_launch("xdna_region_maxpool2_bf16");
}

int xdna_region_backward_bf16(const uint16_t* r, const uint16_t* g, const uint16_t* gp, const uint16_t* px,
                              const uint16_t* extra, const uint16_t* ta, const uint16_t* tb, float scale,
                              const void* go, int go_dtype, uint16_t* out, int64_t planes, int H, int W,
                              void* stream) {
  if (planes < 0 || H < 0 || W < 0 || (g && gp) || (gp && !px) || (!ta != !tb) || go_dtype < 0 || go_dtype > 2 ||
      (go_dtype != 0 && !go)) {
    set_error("xdna_region_backward_bf16: invalid arguments");
    return -1;
  }
  const int64_t n = planes * H * W;
  if (n == 0) return 0;
  if (!out) {
    set_error("xdna_region_backward_bf16: null output");
    return -1;
  }
  if (!admit_launch("xdna_region_backward_bf16")) return -1;
  BwdArgs a{r, g, gp, px, extra, ta, tb, go, go_dtype, scale, out, planes, H, W, H / 2, W / 2};
  region_bwd_kernel<<<grid_for(n), kRegionThreads, 0, as_stream(stream)>>>(a);
  return check_launch("xdna_region_backward_bf16");
}

int xdna_region_loss_parts(void) { return kLossParts; }

int xdna_region_sqdiff_bf16(const uint16_t* a, const uint16_t* b, int64_t n, float scale, float* part,
                            void* stream) {
  if (!a || !b || !part || n < 0) {
    set_error("xdna_region_sqdiff_bf16: invalid arguments");
    return -1;
  }
  if (!admit_launch("xdna_region_sqdiff_bf16")) return -1;
  sqdiff_kernel<<<kLossParts, kRegionThreads, 0, as_stream(stream)>>>(0, a, b, nullptr, 0, 1, 1.0f, n, scale,
                                                                     part);
  return check_launch("xdna_region_sqdiff_bf16");
}

int xdna_region_gram_sqdiff_bf16(const uint16_t* G, const float* t, int64_t t_bstride, int64_t batch, int64_t cc,
                                 float chw, float scale, float* part, void* stream) {
  if (!G || !t || !part || batch < 0 || cc < 1 || t_bstride < 0 || !(chw > 0.0f)) {
    set_error("xdna_region_gram_sqdiff_bf16: invalid arguments");
    return -1;
  }
  if (!admit_launch("xdna_region_gram_sqdiff_bf16")) return -1;
  sqdiff_kernel<<<kLossParts, kRegionThreads, 0, as_stream(stream)>>>(1, G, nullptr, t, t_bstride, cc, chw,
                                                                     batch * cc, scale, part);
  return check_launch("xdna_region_gram_sqdiff_bf16");
}

int xdna_region_loss_finish(const float* part, int n, float* out_f32, uint16_t* out_bf16, void* stream) {
  if (!part || n < 0 || (!out_f32 && !out_bf16)) {
    set_error("xdna_region_loss_finish: invalid arguments");
    return -1;
  }
  if (!admit_launch("xdna_region_loss_finish")) return -1;
  finish_kernel<<<1, kFinishThreads, 0, as_stream(stream)>>>(part, n, out_f32, out_bf16);
  return check_launch("xdna_region_loss_finish");
}

int xdna_region_gram_grad_bf16(const uint16_t* G, const float* t, int64_t t_bstride, int64_t batch, int C,
                               float chw, float coef, const void* go, int go_dtype, uint16_t* S, void* stream) {
  if (!G || !t || !S || batch < 0 || C < 1 || t_bstride < 0 || !(chw > 0.0f) || go_dtype < 0 || go_dtype > 2 ||
      (go_dtype != 0 && !go)) {
    set_error("xdna_region_gram_grad_bf16: invalid arguments");
    return -1;
  }
  if (batch == 0) return 0;
  if (batch > 65535) {
    set_error("xdna_region_gram_grad_bf16: batch too large");
    return -1;
  }
  if (!admit_launch("xdna_region_gram_grad_bf16")) return -1;
  const unsigned nt = unsigned(ceil_div(C, kGT));
  gram_grad_kernel<<<dim3(nt, nt, unsigned(batch)), kRegionThreads, 0, as_stream(stream)>>>(G, t, t_bstride, C, chw,
                                                                                        coef, go, go_dtype, S);
  return check_launch("xdna_region_gram_grad_bf16");
}

}  // extern "C"
