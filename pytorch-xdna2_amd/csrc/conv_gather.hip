// General 2-D convolution (any kernel size, stride and padding; dilation 1, groups 1) in
// bf16 with fp32 accumulation: forward, input gradient and weight gradient as MFMA GEMMs
// whose operands are gathered from NCHW / OIHW on the fly (implicit im2col; nothing is
// materialised).  These are the convolutions outside the 3x3 / stride-1 path: strided
// 3x3, 1x1 and 9x9 layers (the style network's encoder and output layers, ResNet's
// downsampling).  The reference sends them to PyTorch's CPU kernels through its
// fallback (convolution_overrideable_xdna, torch_xdna_device.cpp:4524-4606, 4608-4885).
//
//   forward: C[co][p]          = sum_{k=(ci,ky,kx)} w[co][k] * x[b][ci][oy*sh-ph+ky][ox*sw-pw+kx]
//   dgrad:   C[ci][q]          = sum_{k=(co,ky,kx)} w[co][ci][ky][kx] * dy[b][co][oy][ox],
//                                oy = (iy+ph-ky)/sh where that divides and lands inside
//   wgrad:   C[co][j=(ci,ky,kx)] = sum_{p=(b,oy,ox)} dy[b][co][oy][ox] * x[b][ci][oy*sh-ph+ky][ox*sw-pw+kx]
//
// Tiles: TM (32 / 64 / 128) rows x 128 columns x 32 k per workgroup of four waves; both
// operands are staged k-contiguous in LDS ([row][k], pitch 40) so every MFMA fragment is
// one 16-byte read; the next k-tile's gathers are issued into registers while the
// current one is multiplied (double-buffered LDS, one barrier per k-tile).  The weight
// gradient splits its pixel reduction over blockIdx.z into fp32 partials, summed in a
// fixed order by a second kernel (deterministic).
#include "common.h"
#include "mfma.h"
#include "../../include/xdna_hip.h"

#include <algorithm>

namespace xdna {
namespace {

enum GDir { kGFwd = 0, kGDgrad = 1, kGWgrad = 2 };
constexpr int kGTN = 128, kGTK = 32, kGPitch = 40;

struct GArgs {
  const uint16_t* x;     // [B][Cin][H][W]
  const uint16_t* w;     // [Cout][Cin][KH][KW]
  const uint16_t* dy;    // [B][Cout][Ho][Wo]
  const uint16_t* bias;  // [Cout] (forward) or null
  uint16_t* out;         // forward: y; dgrad: dx
  float* part;           // wgrad: [nsplit][M][N]
  int B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw, Ho, Wo;
  int M, N, K, kt_per, nsplit;
};

// Element (row, k) of operand A and (col, k) of operand B, with the per-thread row state
// precomputed once.  Out-of-range elements are zero.
struct RowState {
  bool valid;
  int b, y0, x0;   // fwd B: image, oy*sh-ph, ox*sw-pw;  dgrad B: image, iy+ph, ix+pw
  int ci, ky, kx;  // wgrad B: the (ci, ky, kx) of the column
};

template <int DIR>
__device__ inline RowState b_row(const GArgs& a, int n) {
  RowState r{};
  r.valid = n < a.N;
  const int nn = r.valid ? n : 0;
  if (DIR == kGFwd) {
    const int hw = a.Ho * a.Wo;
    r.b = nn / hw;
    const int rem = nn - r.b * hw, oy = rem / a.Wo, ox = rem - oy * a.Wo;
    r.y0 = oy * a.sh - a.ph;
    r.x0 = ox * a.sw - a.pw;
  } else if (DIR == kGDgrad) {
    const int hw = a.H * a.W;
    r.b = nn / hw;
    const int rem = nn - r.b * hw, iy = rem / a.W, ix = rem - iy * a.W;
    r.y0 = iy + a.ph;
    r.x0 = ix + a.pw;
  } else {
    const int khw = a.KH * a.KW;
    r.ci = nn / khw;
    const int rem = nn - r.ci * khw;
    r.ky = rem / a.KW;
    r.kx = rem - r.ky * a.KW;
  }
  return r;
}

// Every gather below is branch-free: the address of an out-of-range element is replaced by
// the operand's first element and the loaded value is masked, so all loads of a k-tile
// are in flight together (a branch per element would serialise them, one memory latency
// each).
// offsets are 32-bit: every operand holds fewer than 2^31 elements (checked on entry)
__device__ inline uint32_t ld_masked(const uint16_t* base, int off, bool ok) {
  const uint32_t v = base[ok ? off : 0];
  return ok ? v : 0u;
}

// B operand: elements (n, k0 .. k0+15) packed as bf16 pairs into u[8].  S1: unit strides
// (dgrad needs no division then).
template <int DIR, bool S1>
__device__ inline void gather_b(const GArgs& a, const RowState& r, int k0, uint32_t (&u)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = 0;
  if (DIR == kGFwd) {
    const int khw = a.KH * a.KW;
    int ci = k0 / khw, rem = k0 - ci * khw;
    int ky = rem / a.KW, kx = rem - ky * a.KW;
    const int img = r.b * a.Cin;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int iy = r.y0 + ky, ix = r.x0 + kx;
      const bool ok = r.valid & (k0 + e < a.K) & (iy >= 0) & (iy < a.H) & (ix >= 0) & (ix < a.W);
      u[e >> 1] |= ld_masked(a.x, ((img + ci) * a.H + iy) * a.W + ix, ok) << ((e & 1) * 16);
      if (++kx == a.KW) { kx = 0; if (++ky == a.KH) { ky = 0; ++ci; } }
    }
  } else if (DIR == kGDgrad) {
    const int khw = a.KH * a.KW;
    int co = k0 / khw, rem = k0 - co * khw;
    int ky = rem / a.KW, kx = rem - ky * a.KW;
    const int img = r.b * a.Cout;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int ty = r.y0 - ky, tx = r.x0 - kx;
      int oy, ox;
      bool ok = r.valid & (k0 + e < a.K) & (ty >= 0) & (tx >= 0);
      if (S1) {
        oy = ty;
        ox = tx;
      } else {
        oy = ty / a.sh;
        ox = tx / a.sw;
        ok = ok & (oy * a.sh == ty) & (ox * a.sw == tx);
      }
      ok = ok & (oy < a.Ho) & (ox < a.Wo);
      u[e >> 1] |= ld_masked(a.dy, ((img + co) * a.Ho + oy) * a.Wo + ox, ok) << ((e & 1) * 16);
      if (++kx == a.KW) { kx = 0; if (++ky == a.KH) { ky = 0; ++co; } }
    }
  } else {
    const int hw = a.Ho * a.Wo;
    int b = k0 / hw, rem = k0 - b * hw;
    int oy = rem / a.Wo, ox = rem - oy * a.Wo;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int iy = oy * a.sh - a.ph + r.ky, ix = ox * a.sw - a.pw + r.kx;
      const bool ok = r.valid & (k0 + e < a.K) & (iy >= 0) & (iy < a.H) & (ix >= 0) & (ix < a.W);
      u[e >> 1] |= ld_masked(a.x, ((b * a.Cin + r.ci) * a.H + iy) * a.W + ix, ok) << ((e & 1) * 16);
      if (++ox == a.Wo) { ox = 0; if (++oy == a.Ho) { oy = 0; ++b; } }
    }
  }
}

// A operand: row m, KPT consecutive k from k0, packed as bf16 pairs
template <int DIR, int KPT>
__device__ inline void gather_a(const GArgs& a, int m, int k0, uint32_t (&u)[KPT / 2]) {
#pragma unroll
  for (int i = 0; i < KPT / 2; ++i) u[i] = 0;
  const bool mok = m < a.M;
  if (DIR == kGFwd) {
    const int row = m * a.K;
#pragma unroll
    for (int e = 0; e < KPT; ++e)
      u[e >> 1] |= ld_masked(a.w, row + k0 + e, mok & (k0 + e < a.K)) << ((e & 1) * 16);
  } else if (DIR == kGDgrad) {
    // w[co][m][ky][kx] for k = (co, ky, kx)
    const int khw = a.KH * a.KW;
    int co = k0 / khw, r = k0 - co * khw;
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      u[e >> 1] |= ld_masked(a.w, (co * a.Cin + m) * khw + r, mok & (k0 + e < a.K)) << ((e & 1) * 16);
      if (++r == khw) { r = 0; ++co; }
    }
  } else {
    // dy[b][m][oy][ox] for k = (b, oy, ox)
    const int hw = a.Ho * a.Wo;
    int b = k0 / hw, rem = k0 - b * hw;
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      u[e >> 1] |= ld_masked(a.dy, (b * a.Cout + m) * hw + rem, mok & (k0 + e < a.K)) << ((e & 1) * 16);
      if (++rem == hw) { rem = 0; ++b; }
    }
  }
}

template <int DIR, int TM, bool S1>
__global__ __launch_bounds__(256) void conv_gather_kernel(GArgs a) {
  constexpr int WMW = TM == 32 ? 1 : 2;        // waves along M
  constexpr int WNW = 4 / WMW;                 // waves along N
  constexpr int MT = TM / WMW / 32;            // 32-row MFMA tiles per wave
  constexpr int NT = kGTN / WNW / 32;          // 32-column MFMA tiles per wave
  constexpr int TPR = 256 / TM;                // threads per A row
  constexpr int KPT = kGTK / TPR;              // A elements per thread
  __shared__ __attribute__((aligned(16))) uint16_t as[2][TM * kGPitch];
  __shared__ __attribute__((aligned(16))) uint16_t bs[2][kGTN * kGPitch];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WMW, wn = wave / WMW;
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * kGTN;
  const int split = blockIdx.z;
  const int ktiles = (a.K + kGTK - 1) / kGTK;
  const int kt0 = split * a.kt_per, kt1 = min(ktiles, kt0 + a.kt_per);
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  // staging roles: A row tid / TPR (KPT k from (tid % TPR) * KPT), B row tid / 2 (16 k)
  const int am = m0 + tid / TPR, ak = (tid % TPR) * KPT;
  const int bn = tid >> 1, bk = (tid & 1) * 16;
  const RowState br = b_row<DIR>(a, n0 + bn);

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = zero_acc();

  uint32_t ua[KPT / 2], ub[8];
  auto store = [&](int buf) {
    uint16_t* ad = &as[buf][(tid / TPR) * kGPitch + ak];
#pragma unroll
    for (int i = 0; i < KPT / 2; i += 2) {
      uint2 v = make_uint2(ua[i], ua[i + 1]);
      *reinterpret_cast<uint2*>(ad + 2 * i) = v;
    }
    uint16_t* bd = &bs[buf][bn * kGPitch + bk];
    *reinterpret_cast<uint4*>(bd) = make_uint4(ub[0], ub[1], ub[2], ub[3]);
    *reinterpret_cast<uint4*>(bd + 8) = make_uint4(ub[4], ub[5], ub[6], ub[7]);
  };

  if (kt0 < kt1) {
    gather_a<DIR, KPT>(a, am, kt0 * kGTK + ak, ua);
    gather_b<DIR, S1>(a, br, kt0 * kGTK + bk, ub);
    store(0);
  }
  __syncthreads();
  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) {
      gather_a<DIR, KPT>(a, am, (kt + 1) * kGTK + ak, ua);
      gather_b<DIR, S1>(a, br, (kt + 1) * kGTK + bk, ub);
    }
#pragma unroll
    for (int ks = 0; ks < kGTK / 16; ++ks) {
      u32x4_t fa[MT], fb[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        fa[i] = *reinterpret_cast<const u32x4_t*>(&as[cur][(wm * MT * 32 + i * 32 + lr) * kGPitch + ks * 16 + lk]);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        fb[j] = *reinterpret_cast<const u32x4_t*>(&bs[cur][(wn * NT * 32 + j * 32 + lr) * kGPitch + ks * 16 + lk]);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = mfma_32x32x16(as_bf16x8(fa[i]), as_bf16x8(fb[j]), acc[i][j]);
    }
    if (more) store(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lanes 0..31 hold 32 consecutive columns (n) of one row (m)
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = n0 + wn * NT * 32 + j * 32 + lr;
    if (n >= a.N) continue;
    if (DIR == kGWgrad) {
      float* P = a.part + int64_t(split) * a.M * a.N;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * MT * 32 + i * 32 + mfma_row(r, lane);
          if (m < a.M) P[int64_t(m) * a.N + n] = acc[i][j][r];
        }
    } else {
      // n -> (b, pixel): NCHW offset of channel 0; channel m adds m * plane
      const int plane = DIR == kGFwd ? a.Ho * a.Wo : a.H * a.W;
      const int C = DIR == kGFwd ? a.Cout : a.Cin;
      const int b = n / plane, pix = n - b * plane;
      uint16_t* o = a.out + int64_t(b) * C * plane + pix;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * MT * 32 + i * 32 + mfma_row(r, lane);
          if (m >= a.M) continue;
          float v = acc[i][j][r];
          if (DIR == kGFwd && a.bias) v += bf16_to_f32(a.bias[m]);
          o[int64_t(m) * plane] = f32_to_bf16(v);
        }
    }
  }
}

// gw[m][n] = bf16(sum over splits of part[s][m][n]): the 256 threads are 8 groups of 32
// consecutive outputs; group z sums splits z, z + 8, ... and the groups are added in
// order through LDS (a fixed association per output, so the result is deterministic;
// eight loads in flight per output where one thread per output waited on each split).
__global__ __launch_bounds__(256) void gather_reduce_kernel(const float* __restrict__ part,
                                                            uint16_t* __restrict__ gw, int64_t mn,
                                                            int nsplit) {
  constexpr int ZG = 8, EPB = 256 / ZG;
  const int z = threadIdx.x / EPB, e = threadIdx.x % EPB;
  __shared__ float red[256];
  for (int64_t base = int64_t(blockIdx.x) * EPB; base < mn; base += int64_t(gridDim.x) * EPB) {
    const int64_t i = base + e;
    float s = 0.0f;
    if (i < mn)
      for (int k = z; k < nsplit; k += ZG) s += part[int64_t(k) * mn + i];
    red[threadIdx.x] = s;
    __syncthreads();
    if (z == 0) {
      for (int q = 1; q < ZG; ++q) s += red[q * EPB + e];
      if (i < mn) gw[i] = f32_to_bf16(s);
    }
    __syncthreads();
  }
}

bool gconv_args(const char* what, GArgs& a, int B, int Cin, int Cout, int H, int W, int KH, int KW,
                int sh, int sw, int ph, int pw) {
  if (B < 1 || Cin < 1 || Cout < 1 || H < 1 || W < 1 || KH < 1 || KW < 1 || sh < 1 || sw < 1 || ph < 0 ||
      pw < 0) {
    set_error(std::string(what) + ": invalid shape");
    return false;
  }
  a.B = B; a.Cin = Cin; a.Cout = Cout; a.H = H; a.W = W; a.KH = KH; a.KW = KW;
  a.sh = sh; a.sw = sw; a.ph = ph; a.pw = pw;
  a.Ho = (H + 2 * ph - KH) / sh + 1;
  a.Wo = (W + 2 * pw - KW) / sw + 1;
  if (H + 2 * ph < KH || W + 2 * pw < KW || a.Ho < 1 || a.Wo < 1) {
    set_error(std::string(what) + ": kernel larger than the padded input");
    return false;
  }
  // element counts and offsets inside each operand must fit the kernel's int arithmetic,
  // with headroom for the (masked) offsets of out-of-range elements
  const int64_t lim = int64_t(1) << 30;
  if (int64_t(B) * Cin * H * W >= lim || int64_t(B) * Cout * a.Ho * a.Wo >= lim ||
      int64_t(Cout) * Cin * KH * KW >= lim) {
    set_error(std::string(what) + ": tensor too large");
    return false;
  }
  return true;
}

int tile_m(int M) { return M <= 32 ? 32 : M <= 64 ? 64 : 128; }

template <int DIR, bool S1>
void launch_gather_s(GArgs& a, dim3 grid, int tm, hipStream_t st) {
  if (tm == 32) conv_gather_kernel<DIR, 32, S1><<<grid, 256, 0, st>>>(a);
  else if (tm == 64) conv_gather_kernel<DIR, 64, S1><<<grid, 256, 0, st>>>(a);
  else conv_gather_kernel<DIR, 128, S1><<<grid, 256, 0, st>>>(a);
}

template <int DIR>
int launch_gather(GArgs& a, hipStream_t st) {
  const int tm = tile_m(a.M);
  const dim3 grid(unsigned(ceil_div(a.N, kGTN)), unsigned(ceil_div(a.M, tm)), unsigned(a.nsplit));
  // unit strides only change the dgrad gather (no division); one instantiation otherwise
  if (DIR == kGDgrad && a.sh == 1 && a.sw == 1) launch_gather_s<DIR, true>(a, grid, tm, st);
  else launch_gather_s<DIR, false>(a, grid, tm, st);
  return check_launch("conv gather");
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_conv2d_fwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* y, int B,
                         int Cin, int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph, int pw,
                         void* stream) {
  GArgs a{};
  if (!gconv_args("xdna_conv2d_fwd_bf16", a, B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw)) return -1;
  a.x = x; a.w = w; a.bias = bias; a.out = y;
  a.M = Cout; a.N = B * a.Ho * a.Wo; a.K = Cin * KH * KW;
  if (int64_t(B) * a.Ho * a.Wo >= (int64_t(1) << 31) || ceil_div(a.N, kGTN) > 0x7fffffff) {
    set_error("xdna_conv2d_fwd_bf16: output too large");
    return -1;
  }
  a.nsplit = 1;
  a.kt_per = int(ceil_div(a.K, kGTK));
  if (!admit_launch("xdna_conv2d_fwd_bf16")) return -1;
  return launch_gather<kGFwd>(a, as_stream(stream));
}

int xdna_conv2d_dgrad_bf16(const uint16_t* dy, const uint16_t* w, uint16_t* dx, int B, int Cin, int Cout,
                           int H, int W, int KH, int KW, int sh, int sw, int ph, int pw, void* stream) {
  GArgs a{};
  if (!gconv_args("xdna_conv2d_dgrad_bf16", a, B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw)) return -1;
  a.dy = dy; a.w = w; a.out = dx;
  a.M = Cin; a.N = B * H * W; a.K = Cout * KH * KW;
  a.nsplit = 1;
  a.kt_per = int(ceil_div(a.K, kGTK));
  if (!admit_launch("xdna_conv2d_dgrad_bf16")) return -1;
  return launch_gather<kGDgrad>(a, as_stream(stream));
}

int xdna_conv2d_wgrad_bf16(const uint16_t* x, const uint16_t* dy, uint16_t* gw, uint16_t* gb, int B, int Cin,
                           int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph, int pw,
                           void* stream) {
  GArgs a{};
  if (!gconv_args("xdna_conv2d_wgrad_bf16", a, B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw)) return -1;
  a.x = x; a.dy = dy;
  a.M = Cout; a.N = Cin * KH * KW; a.K = B * a.Ho * a.Wo;
  // split the pixel reduction until the grid covers the CUs twice (fixed-order partial sums)
  const int64_t tiles = ceil_div(a.M, tile_m(a.M)) * ceil_div(a.N, kGTN);
  const int64_t ktiles = ceil_div(a.K, kGTK);
  int64_t ns = std::max<int64_t>(1, std::min<int64_t>(ktiles, ceil_div(512, tiles)));
  ns = std::min<int64_t>(ns, 4096);
  a.kt_per = int(ceil_div(ktiles, ns));
  a.nsplit = int(ceil_div(ktiles, a.kt_per));
  const int64_t mn = int64_t(a.M) * a.N;
  if (!admit_launch("xdna_conv2d_wgrad_bf16")) return -1;
  a.part = static_cast<float*>(xdna_hip_cache_alloc(size_t(a.nsplit) * size_t(mn) * sizeof(float)));
  if (!a.part) return -1;
  hipStream_t st = as_stream(stream);
  if (launch_gather<kGWgrad>(a, st)) {
    xdna_hip_cache_free(a.part);
    return -1;
  }
  gather_reduce_kernel<<<unsigned(std::min<int64_t>(ceil_div(mn, 32), 8192)), 256, 0, st>>>(a.part, gw, mn,
                                                                                         a.nsplit);
  // stream-ordered reuse: the next user of the block runs after the reduce
  xdna_hip_cache_free(a.part);
  if (check_launch("xdna_conv2d_wgrad_bf16")) return -1;
  if (gb) return xdna_conv3x3_bias_grad_bf16(dy, gb, B, Cout, a.Ho, a.Wo, stream);
  return 0;
}

}  // extern "C"
