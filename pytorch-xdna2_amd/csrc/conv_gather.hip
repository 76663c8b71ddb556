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
#include <atomic>

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
  int x_bytes, w_bytes, dy_bytes;  // operand extents (each under 2^31 bytes)
};

// Buffer resources over the three operands: a load at an out-of-range offset returns
// zero without a memory access, which is how every masked element below is read.
struct GRs {
  __amdgpu_buffer_rsrc_t x, w, dy;
};

__device__ inline GRs g_rs(const GArgs& a) {
  GRs r;
  r.x = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), 0, a.x_bytes, 0x00020000);
  r.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.w), 0, a.w_bytes, 0x00020000);
  r.dy = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.dy), 0, a.dy_bytes, 0x00020000);
  return r;
}

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

// Every gather below is branch-free: a masked element's offset is replaced by one past
// the resource's end, so the hardware returns zero without a memory access, and all loads
// of a k-tile are in flight together (a branch per element would serialise them, one
// memory latency each; redirecting masked loads to element 0 instead queued them all on
// that one address).  Offsets are 32-bit: every operand holds fewer than 2^30 elements
// (checked on entry).
constexpr int kOob = int(0x80000000u);

__device__ inline uint32_t ld_masked(__amdgpu_buffer_rsrc_t rs, int off, bool ok) {
  return __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? off * 2 : kOob, 0, 0);
}

// B operand: elements (n, k0 .. k0+15) packed as bf16 pairs into u[8].  S1: unit strides
// (dgrad needs no division then).
template <int DIR, bool S1>
__device__ inline void gather_b(const GArgs& a, const GRs& rs, const RowState& r, int k0, uint32_t (&u)[8]) {
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
      u[e >> 1] |= ld_masked(rs.x, ((img + ci) * a.H + iy) * a.W + ix, ok) << ((e & 1) * 16);
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
      u[e >> 1] |= ld_masked(rs.dy, ((img + co) * a.Ho + oy) * a.Wo + ox, ok) << ((e & 1) * 16);
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
      u[e >> 1] |= ld_masked(rs.x, ((b * a.Cin + r.ci) * a.H + iy) * a.W + ix, ok) << ((e & 1) * 16);
      if (++ox == a.Wo) { ox = 0; if (++oy == a.Ho) { oy = 0; ++b; } }
    }
  }
}

// A operand: row m, KPT consecutive k from k0, packed as bf16 pairs
template <int DIR, int KPT>
__device__ inline void gather_a(const GArgs& a, const GRs& rs, int m, int k0, uint32_t (&u)[KPT / 2]) {
#pragma unroll
  for (int i = 0; i < KPT / 2; ++i) u[i] = 0;
  const bool mok = m < a.M;
  if (DIR == kGFwd) {
    const int row = m * a.K;
#pragma unroll
    for (int e = 0; e < KPT; ++e)
      u[e >> 1] |= ld_masked(rs.w, row + k0 + e, mok & (k0 + e < a.K)) << ((e & 1) * 16);
  } else if (DIR == kGDgrad) {
    // w[co][m][ky][kx] for k = (co, ky, kx)
    const int khw = a.KH * a.KW;
    int co = k0 / khw, r = k0 - co * khw;
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      u[e >> 1] |= ld_masked(rs.w, (co * a.Cin + m) * khw + r, mok & (k0 + e < a.K)) << ((e & 1) * 16);
      if (++r == khw) { r = 0; ++co; }
    }
  } else {
    // dy[b][m][oy][ox] for k = (b, oy, ox)
    const int hw = a.Ho * a.Wo;
    int b = k0 / hw, rem = k0 - b * hw;
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      u[e >> 1] |= ld_masked(rs.dy, (b * a.Cout + m) * hw + rem, mok & (k0 + e < a.K)) << ((e & 1) * 16);
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
  const GRs rs = g_rs(a);

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
    gather_a<DIR, KPT>(a, rs, am, kt0 * kGTK + ak, ua);
    gather_b<DIR, S1>(a, rs, br, kt0 * kGTK + bk, ub);
    store(0);
  }
  __syncthreads();
  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) {
      gather_a<DIR, KPT>(a, rs, am, (kt + 1) * kGTK + ak, ua);
      gather_b<DIR, S1>(a, rs, br, (kt + 1) * kGTK + bk, ub);
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
    if (i < mn) s = sum_strided8(0.0f, part + i, mn, z, ZG, nsplit);
    red[threadIdx.x] = s;
    __syncthreads();
    if (z == 0) {
      for (int q = 1; q < ZG; ++q) s += red[q * EPB + e];
      if (i < mn) gw[i] = f32_to_bf16(s);
    }
    __syncthreads();
  }
}

// Weight gradient of stride-1 convs with at most 4 output channels (the style network's
// last layer, 9x9 32->3): gw[co][ci][ky][kx] = sum over pixels of dy[n][co][oy][ox] *
// x[n][ci][oy + ky - ph][ox + kx - pw].  As a GEMM its output dimension is the 3 output
// channels, which MFMA tiles would pad 10x; here each workgroup takes a run of output rows
// (n, oy), stages the row's Cin x KH input rows (zero-padded to Wo + KW - 1 columns) and
// its dY row in LDS as fp32, and each thread accumulates Cout sums for each of its
// (ci, ky, kx) taps with fp32 FMAs.  Partials per workgroup go through gather_reduce_kernel
// (fixed order).
constexpr int kFoMaxTaps = 16;  // taps per thread: Cin * KH * KW <= 4096

struct FoArgs {
  const uint16_t* x;
  const uint16_t* dy;
  float* part;  // [workgroups][Cout * Cin * KH * KW]
  int B, Ci, Co, H, W, KH, KW, ph, pw, Ho, Wo, Wp;
  int rows_per_wg;
  int64_t rows;
};

template <int CO>
__global__ __launch_bounds__(256) void wgrad_fewout_kernel(FoArgs a) {
  extern __shared__ float fsm[];
  const int nxr = a.Ci * a.KH;      // staged input rows
  float* xs = fsm;                  // [Ci * KH][Wp]
  float* ds = fsm + nxr * a.Wp;     // [CO][Wo]
  const int T = a.Ci * a.KH * a.KW;
  const int tid = threadIdx.x;
  int toff[kFoMaxTaps];
  float acc[kFoMaxTaps][CO];
#pragma unroll
  for (int j = 0; j < kFoMaxTaps; ++j) {
    const int t = tid + 256 * j;
    const int ci = t / (a.KH * a.KW), r = t - ci * (a.KH * a.KW);
    const int ky = r / a.KW, kx = r - ky * a.KW;
    toff[j] = t < T ? (ci * a.KH + ky) * a.Wp + kx : -1;
#pragma unroll
    for (int c = 0; c < CO; ++c) acc[j][c] = 0.f;
  }
  const int rows_per_pass = 256 / a.Wp;  // staged rows loaded per pass (Wp <= 256)
  const int lrow = tid / a.Wp, lcol = tid - lrow * a.Wp;
  const int64_t r0 = int64_t(blockIdx.x) * a.rows_per_wg;
  const int64_t r1 = min(a.rows, r0 + a.rows_per_wg);
  for (int64_t row = r0; row < r1; ++row) {
    const int n = int(row / a.Ho), oy = int(row - int64_t(n) * a.Ho);
    __syncthreads();  // the previous row's reads are done
    if (lrow < rows_per_pass) {
      const int ix = lcol - a.pw;
      for (int q = lrow; q < nxr; q += rows_per_pass) {
        const int ci = q / a.KH, ky = q - ci * a.KH;
        const int iy = oy + ky - a.ph;
        float v = 0.f;
        if (iy >= 0 && iy < a.H && ix >= 0 && ix < a.W)
          v = bf16_to_f32(a.x[((int64_t(n) * a.Ci + ci) * a.H + iy) * a.W + ix]);
        xs[q * a.Wp + lcol] = v;
      }
    }
    for (int i = tid; i < CO * a.Wo; i += 256) {
      const int c = i / a.Wo, ox = i - c * a.Wo;
      ds[i] = c < a.Co ? bf16_to_f32(a.dy[((int64_t(n) * a.Co + c) * a.Ho + oy) * a.Wo + ox]) : 0.f;
    }
    __syncthreads();
    for (int ox = 0; ox < a.Wo; ++ox) {
      float d[CO];
#pragma unroll
      for (int c = 0; c < CO; ++c) d[c] = ds[c * a.Wo + ox];
#pragma unroll
      for (int j = 0; j < kFoMaxTaps; ++j) {
        if (toff[j] < 0) break;
        const float xv = xs[toff[j] + ox];
#pragma unroll
        for (int c = 0; c < CO; ++c) acc[j][c] = fmaf(d[c], xv, acc[j][c]);
      }
    }
  }
  float* pb = a.part + int64_t(blockIdx.x) * a.Co * T;
#pragma unroll
  for (int j = 0; j < kFoMaxTaps; ++j) {
    const int t = tid + 256 * j;
    if (t >= T) break;
#pragma unroll
    for (int c = 0; c < CO; ++c)
      if (c < a.Co) pb[int64_t(c) * T + t] = acc[j][c];
  }
}

bool fewout_ok(int Cout, int Cin, int KH, int KW, int sh, int sw, int Wo) {
  const int Wp = Wo + KW - 1;
  return sh == 1 && sw == 1 && Cout <= 4 && int64_t(Cin) * KH * KW <= 256 * kFoMaxTaps && Wp <= 256 &&
         size_t(int64_t(Cin) * KH * Wp + 4 * Wo) * 4 <= 64 * 1024;
}

// Sliding-window form of the few-output weight gradient for odd kernel widths up to 9.
// A workgroup takes a run of rows_per_wg consecutive output rows (n, oy), in tiles of at
// most R rows within one image.  Per tile it stages the tile's input rows, Cin x (R + KH
// - 1) rows of Wo + KW - 1 columns (fp32, zero padding written out, odd row pitch so that
// consecutive rows start in different banks), and dY's Cout x R rows.  Thread p owns the
// row pair (ci, ky) = (p / KH, p % KH) and its KW x Cout sums; it walks each staged row
// with a KW-wide register window (a ring indexed by the unrolled column phase), so every
// output column costs one LDS read of x, Cout broadcast reads of dY and KW x Cout FMAs.
// The staging issues eight global loads before waiting on any.  Each workgroup writes its
// sums to its own partial slab; gather_reduce_kernel adds the slabs in a fixed order.
struct FsArgs {
  const uint16_t* x;
  const uint16_t* dy;
  float* part;      // [workgroups][Cout][Cin * KH * KW]
  int Ci, Co, H, W, KH, ph, pw, Ho, Wo;
  int pitch;        // staged row pitch in floats: odd, >= Wo + KW - 1
  int R;            // output rows per tile
  int rows_per_wg;
  int64_t rows;     // B * Ho
};

constexpr int kFsStage = 8;  // global loads in flight per thread while staging

template <int CO, int KW>
__global__ __launch_bounds__(512) void wgrad_slide_kernel(FsArgs a) {
  extern __shared__ float fsm[];
  const int Rs = a.R + a.KH - 1;
  float* xs = fsm;                        // [Ci][Rs][pitch]
  float* ds = fsm + a.Ci * Rs * a.pitch;  // [CO][R][Wo]
  const int P = a.Ci * a.KH, T = P * KW;
  const int nt = blockDim.x, tid = threadIdx.x;
  const int wp = a.Wo + KW - 1;
  const int rpp = nt / wp;  // staged rows per pass (wp <= nt)
  const int lrow = tid / wp, col = tid - lrow * wp;
  const int ix = col - a.pw;
  const bool colok = lrow < rpp && ix >= 0 && ix < a.W;
  const int64_t r0 = int64_t(blockIdx.x) * a.rows_per_wg;
  const int64_t r1 = min(a.rows, r0 + a.rows_per_wg);
  float* pb = a.part + int64_t(blockIdx.x) * a.Co * T;
  for (int p0 = 0; p0 < P; p0 += nt) {
    const int p = p0 + tid;
    const int ci = p / a.KH, ky = p - ci * a.KH;
    float acc[KW][CO];
#pragma unroll
    for (int k = 0; k < KW; ++k)
#pragma unroll
      for (int c = 0; c < CO; ++c) acc[k][c] = 0.f;
    for (int64_t row = r0; row < r1;) {
      const int n = int(row / a.Ho), oy0 = int(row - int64_t(n) * a.Ho);
      const int nr = int(min(min(r1 - row, int64_t(a.R)), int64_t(a.Ho - oy0)));
      const int srows = nr + a.KH - 1, nq = a.Ci * srows;
      __syncthreads();  // the previous tile's reads are done
      if (lrow < rpp) {
        int c = lrow / srows, rr = lrow - c * srows;
        for (int q = lrow; q < nq; q += kFsStage * rpp) {
          float v[kFsStage];
          int dst[kFsStage];
#pragma unroll
          for (int j = 0; j < kFsStage; ++j) {
            const bool in = q + j * rpp < nq;
            const int iy = oy0 - a.ph + rr;
            v[j] = in && colok && iy >= 0 && iy < a.H
                       ? bf16_to_f32(a.x[((int64_t(n) * a.Ci + c) * a.H + iy) * a.W + ix])
                       : 0.f;
            dst[j] = in ? (c * Rs + rr) * a.pitch + col : -1;
            rr += rpp;
            while (rr >= srows) {
              rr -= srows;
              ++c;
            }
          }
#pragma unroll
          for (int j = 0; j < kFsStage; ++j)
            if (dst[j] >= 0) xs[dst[j]] = v[j];
        }
      }
      for (int i = tid; i < CO * nr * a.Wo; i += nt) {
        const int q = i / a.Wo, ox = i - q * a.Wo;
        const int c = q / nr, r = q - c * nr;
        ds[(c * a.R + r) * a.Wo + ox] =
            c < a.Co ? bf16_to_f32(a.dy[((int64_t(n) * a.Co + c) * a.Ho + oy0 + r) * a.Wo + ox]) : 0.f;
      }
      __syncthreads();
      if (p < P) {
        for (int r = 0; r < nr; ++r) {
          const float* xr = xs + (ci * Rs + r + ky) * a.pitch;
          const float* dr = ds + r * a.Wo;
          float w[KW];
#pragma unroll
          for (int k = 0; k < KW - 1; ++k) w[k] = xr[k];
          for (int ox0 = 0; ox0 < a.Wo; ox0 += KW) {
#pragma unroll
            for (int u = 0; u < KW; ++u) {
              const int ox = ox0 + u;
              if (ox >= a.Wo) break;
              w[(u + KW - 1) % KW] = xr[ox + KW - 1];
              float d[CO];
#pragma unroll
              for (int c = 0; c < CO; ++c) d[c] = dr[c * a.R * a.Wo + ox];
#pragma unroll
              for (int k = 0; k < KW; ++k)
#pragma unroll
                for (int c = 0; c < CO; ++c) acc[k][c] = fmaf(d[c], w[(u + k) % KW], acc[k][c]);
            }
          }
        }
      }
      row += nr;
    }
    if (p < P) {
#pragma unroll
      for (int c = 0; c < CO; ++c)
#pragma unroll
        for (int k = 0; k < KW; ++k) pb[int64_t(c) * T + p * KW + k] = acc[k][c];
    }
  }
}

constexpr size_t kFsLdsBudget = 80 * 1024;  // two workgroups per CU
constexpr size_t kFsLdsMax = 160 * 1024;

size_t slide_lds(int Ci, int KH, int pitch, int R, int Wo) {
  return (size_t(Ci) * (R + KH - 1) * pitch + size_t(4) * R * Wo) * 4;
}

// The sliding form's geometry, or false when it does not apply (stride other than 1, more
// than 4 outputs, an even or wider kernel, rows wider than the block, or one tile beyond
// one CU's LDS).
bool slide_args(FsArgs& f, int B, int Cin, int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph,
                int pw, int Ho, int Wo, int& nt) {
  if (sh != 1 || sw != 1 || Cout > 4 || Cout < 1 || (KW != 3 && KW != 5 && KW != 7 && KW != 9)) return false;
  const int64_t P = int64_t(Cin) * KH;
  nt = int(std::min<int64_t>(512, ceil_div(P, 64) * 64));
  const int wp = Wo + KW - 1;
  if (wp > nt || P * KW > (int64_t(1) << 24)) return false;
  f.pitch = wp | 1;
  if (slide_lds(Cin, KH, f.pitch, 1, Wo) > kFsLdsMax) return false;
  f.Ci = Cin; f.Co = Cout; f.H = H; f.W = W; f.KH = KH; f.ph = ph; f.pw = pw; f.Ho = Ho; f.Wo = Wo;
  f.rows = int64_t(B) * Ho;
  // about two workgroups per CU; tiles as tall as the LDS budget allows
  f.rows_per_wg = int(ceil_div(f.rows, std::min<int64_t>(f.rows, 512)));
  f.R = 1;
  while (f.R < f.rows_per_wg && f.R < Ho && slide_lds(Cin, KH, f.pitch, f.R + 1, Wo) <= kFsLdsBudget) ++f.R;
  return true;
}

template <int CO>
int launch_slide(const FsArgs& f, int KW, unsigned grid, int nt, size_t lds, hipStream_t st) {
  const void* fn = KW == 3   ? reinterpret_cast<const void*>(&wgrad_slide_kernel<CO, 3>)
                   : KW == 5 ? reinterpret_cast<const void*>(&wgrad_slide_kernel<CO, 5>)
                   : KW == 7 ? reinterpret_cast<const void*>(&wgrad_slide_kernel<CO, 7>)
                             : reinterpret_cast<const void*>(&wgrad_slide_kernel<CO, 9>);
  if (lds > 64 * 1024 && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(kFsLdsMax)) !=
                             hipSuccess) {
    set_error("xdna_conv2d_wgrad_bf16: cannot raise the LDS limit of the few-output kernel");
    return -1;
  }
  if (KW == 3) wgrad_slide_kernel<CO, 3><<<grid, nt, lds, st>>>(f);
  else if (KW == 5) wgrad_slide_kernel<CO, 5><<<grid, nt, lds, st>>>(f);
  else if (KW == 7) wgrad_slide_kernel<CO, 7><<<grid, nt, lds, st>>>(f);
  else wgrad_slide_kernel<CO, 9><<<grid, nt, lds, st>>>(f);
  return 0;
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
  a.x_bytes = int(int64_t(B) * Cin * H * W * 2);
  a.w_bytes = int(int64_t(Cout) * Cin * KH * KW * 2);
  a.dy_bytes = int(int64_t(B) * Cout * a.Ho * a.Wo * 2);
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

// ---------------------------------------------------------------------------------------
// Direct form for few output channels (<= 32) at stride 1: the style network's 9x9 input
// and output layers (3 -> 32, 32 -> 3, and the 32 -> 3 layer's input gradient), where the
// gather GEMM pads M to 32 rows and fetches every operand element from global memory.
// Workgroup = (image, kDTR output rows, all columns).  The input rows it needs sit in LDS
// as a zero-padded grid of Wp = Wo + KW - 1 columns, pixel-major with 32 channels per
// position; output pixel (oy, ox) is grid position q = (oy - oy0) * Wp + ox and tap
// (ky, kx) reads position q + ky * Wp + kx, so a B fragment (32 consecutive q x 8
// channels) is one 16-byte LDS read per lane (columns ox >= Wo are computed and dropped).
// Prepared weights [chunk][ky][32 co][KW][32 ci] are staged one kernel row at a time; the
// next row is loaded into registers during the current row's MFMAs.  Two workgroups fit
// a CU (67 KB of LDS for the 9x9 layers at 36 x 36).
// ---------------------------------------------------------------------------------------
constexpr int kDTR = 4;        // output rows per workgroup
constexpr int kDCK = 32;       // channels per chunk
constexpr int kDPitch = 40;    // LDS pitch (elements) of one grid position / weight row
constexpr int kDMaxNB = 16;    // grid blocks of 32 positions (kDTR * Wp <= 512)
constexpr int kDXItems = 16;   // staging items (position x 8 channels) per thread

// 16-byte weight vectors per thread per kernel row: 32 rows x KW taps x 4 vectors,
// rounded up to whole rounds of 256 threads (the prepared rows are zero-padded to that, so
// every load and LDS write is unconditional); KW <= 16
__host__ __device__ constexpr int direct_wv(int kw) { return (32 * kw * 4 + 255) / 256; }

struct DArgs {
  const uint16_t* x;     // [B][Cin][H][W]
  const uint16_t* wp;    // prepared [chunks][KH][wv * 256 vectors of 8]: rows (co, kx) of 32 ci
  const uint16_t* bias;  // [Cout] or null
  uint16_t* out;         // [B][Cout][Ho][Wo]
  int B, Cin, Cout, H, W, KH, KW, ph, pw, Ho, Wo, Wp, chunks, nb, xpos, rtiles, wv;
  int x_bytes;           // under 2^31
};

// Prepared weights, one block of wv * 256 vectors per (chunk, ky): row r = co * KW + kx holds
// the 32 channels ci of w[co][ch*32+ci][ky][kx] (forward) or, flipped for the input
// gradient as a forward conv, of w[ch*32+ci][co][KH-1-ky][KW-1-kx]; zero padding.
__global__ __launch_bounds__(256) void direct_prep_kernel(const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ wp, int Cin, int Cout,
                                                          int KH, int KW, int flip, int blk, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int e = int(i % blk);
    const int64_t cb = i / blk;  // ch * KH + ky
    const int ky = int(cb % KH), ch = int(cb / KH);
    const int ci = e % kDCK, row = e / kDCK;
    const int co = row / KW, kx = row - co * KW;
    const int c = ch * kDCK + ci;
    uint16_t v = 0;
    if (co < 32 && co < Cout && c < Cin) {
      // flipped: the forward conv's weight tensor is [Cin][Cout][KH][KW] in this
      // direction's terms (its output channels are this conv's inputs)
      v = flip ? w[((int64_t(c) * Cout + co) * KH + (KH - 1 - ky)) * KW + (KW - 1 - kx)]
               : w[((int64_t(co) * Cin + c) * KH + ky) * KW + kx];
    }
    wp[i] = v;
  }
}

// KWT: the kernel width when known at compile time (the tap loop unrolls), 0: any width.
// NBW: grid blocks per wave (blocks wave, wave + 4, ...; a wave past the last block
// recomputes the last one and drops it, so no MFMA or LDS read sits behind a branch).
template <int KWT, int NBW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_direct_kernel(DArgs a) {
  constexpr int WV = KWT > 0 ? direct_wv(KWT) : direct_wv(16);
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs = smem;                               // [xpos][kDPitch]
  uint16_t* ws = smem + a.xpos * kDPitch;            // [WV * 256 / 4][kDPitch]
  const int b = blockIdx.x / a.rtiles, oy0 = (blockIdx.x % a.rtiles) * kDTR;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  const int trh = kDTR + a.KH - 1;                   // input rows staged
  const int KW = KWT > 0 ? KWT : a.KW;

  f32x16_t acc[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) acc[j] = zero_acc();
  int bpos[NBW];  // first grid position of each of this wave's blocks (clamped)
#pragma unroll
  for (int j = 0; j < NBW; ++j) bpos[j] = min(wave + 4 * j, a.nb - 1) * 32 + lr;

  u32x4_t wr[WV];
  auto load_w = [&](int ch, int ky) {
    const uint16_t* src = a.wp + (int64_t(ch) * a.KH + ky) * (a.wv * 256 * 8) + tid * 8;
#pragma unroll
    for (int j = 0; j < WV; ++j)
      if (KWT > 0 || j < a.wv) wr[j] = *reinterpret_cast<const u32x4_t*>(src + j * 256 * 8);
  };
  auto store_w = [&]() {
#pragma unroll
    for (int j = 0; j < WV; ++j) {
      // vector v = tid + 256 j: row v / 4, channels (v % 4) * 8
      const int v = tid + j * 256;
      if (KWT > 0 || j < a.wv) *reinterpret_cast<u32x4_t*>(ws + (v >> 2) * kDPitch + (v & 3) * 8) = wr[j];
    }
  };
  // masked elements (borders, padding channels, unused items) read through an
  // out-of-range offset: zero, no memory access
  const auto xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), 0, a.x_bytes, 0x00020000);
  const int plane = a.H * a.W;
  auto stage_x = [&](int ch) {
    const int items = a.xpos * (kDCK / 8);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t v[kDXItems / 2][4];
#pragma unroll
      for (int j = 0; j < kDXItems / 2; ++j) {
        const int i = tid + (half * (kDXItems / 2) + j) * 256;
        const int pos = i % a.xpos, cg = i / a.xpos;
        const int t = pos / a.Wp, c = pos - t * a.Wp;
        const int iy = oy0 - a.ph + t, ix = c - a.pw;
        const bool pok = i < items && t < trh && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
        const int c0 = ch * kDCK + cg * 8;
        const int base = ((b * a.Cin + c0) * plane + iy * a.W + ix) * 2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok0 = pok && c0 + 2 * e < a.Cin, ok1 = pok && c0 + 2 * e + 1 < a.Cin;
          const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(xrs, ok0 ? base + (2 * e) * plane * 2 : kOob, 0, 0);
          const uint32_t hi =
              __builtin_amdgcn_raw_buffer_load_b16(xrs, ok1 ? base + (2 * e + 1) * plane * 2 : kOob, 0, 0);
          v[j][e] = lo | (hi << 16);
        }
      }
#pragma unroll
      for (int j = 0; j < kDXItems / 2; ++j) {
        const int i = tid + (half * (kDXItems / 2) + j) * 256;
        if (i < items) {
          const int pos = i % a.xpos, cg = i / a.xpos;
          *reinterpret_cast<u32x4_t*>(xs + pos * kDPitch + cg * 8) = u32x4_t{v[j][0], v[j][1], v[j][2], v[j][3]};
        }
      }
    }
  };

  for (int ch = 0; ch < a.chunks; ++ch) {
    __syncthreads();  // the previous chunk's reads of xs / ws are done
    stage_x(ch);
    load_w(ch, 0);
    for (int ky = 0; ky < a.KH; ++ky) {
      if (ky > 0) __syncthreads();  // the previous kernel row's reads of ws are done
      store_w();
      __syncthreads();
      if (ky + 1 < a.KH) load_w(ch, ky + 1);
      const uint16_t* wa = ws + lr * KW * kDPitch + lk;
      const uint16_t* xb = xs + (ky * a.Wp) * kDPitch + lk;
#pragma unroll
      for (int kx = 0; kx < KW; ++kx) {
#pragma unroll
        for (int ks = 0; ks < kDCK / 16; ++ks) {
          const bf16x8_t af = as_bf16x8(*reinterpret_cast<const u32x4_t*>(wa + kx * kDPitch + ks * 16));
#pragma unroll
          for (int j = 0; j < NBW; ++j) {
            const bf16x8_t bf =
                as_bf16x8(*reinterpret_cast<const u32x4_t*>(xb + (bpos[j] + kx) * kDPitch + ks * 16));
            acc[j] = mfma_32x32x16(af, bf, acc[j]);
          }
        }
      }
    }
  }

  // lanes 0..31 hold 32 consecutive grid positions of one output channel per value
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int nbk = wave + 4 * j;
    if (nbk >= a.nb) continue;
    const int q = nbk * 32 + lr;
    const int orow = q / a.Wp, ox = q - orow * a.Wp, oy = oy0 + orow;
    if (orow >= kDTR || oy >= a.Ho || ox >= a.Wo) continue;
    uint16_t* o = a.out + (int64_t(b) * a.Cout * a.Ho + oy) * a.Wo + ox;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int co = mfma_row(r, lane);
      if (co < a.Cout) {
        float v = acc[j][r];
        if (a.bias) v += bf16_to_f32(a.bias[co]);
        o[int64_t(co) * a.Ho * a.Wo] = f32_to_bf16(v);
      }
    }
  }
}

size_t direct_lds(const DArgs& d);

// The direct form's geometry for a stride-1 conv of x [B][Cin][H][W] into Cout channels,
// or false when it does not apply (more than 32 outputs, fewer than 16 inputs, a grid
// wider than 128 columns, more staging than the fixed per-thread budget, or LDS beyond
// one CU).
bool direct_args(DArgs& d, int B, int Cin, int Cout, int H, int W, int KH, int KW, int ph, int pw) {
  // fewer than 16 input channels: the 32-channel chunk would be mostly padding (the
  // gather GEMM's k runs over the real channels only; measured faster for 3 channels)
  if (Cout > 32 || Cin < 16 || KW > 16 || KH < 1 || KW < 1 || ph < 0 || pw < 0) return false;
  d.B = B; d.Cin = Cin; d.Cout = Cout; d.H = H; d.W = W; d.KH = KH; d.KW = KW; d.ph = ph; d.pw = pw;
  d.Ho = H + 2 * ph - KH + 1;
  d.Wo = W + 2 * pw - KW + 1;
  if (d.Ho < 1 || d.Wo < 1) return false;
  d.Wp = d.Wo + KW - 1;
  d.nb = int(ceil_div(int64_t(kDTR) * d.Wp, 32));
  if (d.nb > kDMaxNB) return false;
  d.xpos = d.nb * 32 + (KH - 1) * d.Wp + KW - 1;
  if (d.xpos * (kDCK / 8) > kDXItems * 256) return false;
  d.chunks = int(ceil_div(Cin, kDCK));
  d.rtiles = int(ceil_div(d.Ho, kDTR));
  d.wv = direct_wv(KW == 9 ? 9 : 16);  // the generic kernel pads every width to 16
  if (direct_lds(d) > 160 * 1024) return false;
  if (int64_t(B) * d.rtiles > 0x7fffffff) return false;
  return true;
}

size_t direct_lds(const DArgs& d) { return size_t(d.xpos + d.wv * 256 / 4) * kDPitch * 2; }

std::atomic<int> g_conv2d_variant{0};  // 0 automatic, 1 gather GEMM only

// Runs the direct form (weights prepared into the cache allocator) or returns 1 when it
// does not apply.
int run_direct(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* out, int B, int Cin,
               int Cout, int H, int W, int KH, int KW, int ph, int pw, int flip, hipStream_t st) {
  DArgs d{};
  if (g_conv2d_variant.load() == 1 || !direct_args(d, B, Cin, Cout, H, W, KH, KW, ph, pw)) return 1;
  d.x_bytes = int(int64_t(B) * Cin * H * W * 2);  // the callers' operands are under 2^30 elements
  static const bool lds_ok = [] {
    bool ok = true;
    for (const void* f : {reinterpret_cast<const void*>(&conv_direct_kernel<0, 1>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<0, 2>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<0, 3>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<0, 4>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<9, 1>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<9, 2>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<9, 3>),
                          reinterpret_cast<const void*>(&conv_direct_kernel<9, 4>)})
      ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    return ok;
  }();
  if (!lds_ok) return 1;
  const int blk = d.wv * 256 * 8;
  const int64_t n = int64_t(d.chunks) * KH * blk;
  uint16_t* wp = static_cast<uint16_t*>(xdna_hip_cache_alloc(size_t(n) * 2));
  if (!wp) return -1;
  direct_prep_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 4096)), 256, 0, st>>>(w, wp, Cin, Cout, KH, KW,
                                                                                          flip, blk, n);
  d.x = x;
  d.wp = wp;
  d.bias = bias;
  d.out = out;
  const unsigned grid = unsigned(int64_t(B) * d.rtiles);
  const size_t lds = direct_lds(d);
  const int nbw = int(ceil_div(d.nb, 4));
#define XDNA_DIRECT(kw_, nbw_) conv_direct_kernel<kw_, nbw_><<<grid, 256, lds, st>>>(d)
  if (KW == 9) {
    if (nbw == 1) XDNA_DIRECT(9, 1);
    else if (nbw == 2) XDNA_DIRECT(9, 2);
    else if (nbw == 3) XDNA_DIRECT(9, 3);
    else XDNA_DIRECT(9, 4);
  } else {
    if (nbw == 1) XDNA_DIRECT(0, 1);
    else if (nbw == 2) XDNA_DIRECT(0, 2);
    else if (nbw == 3) XDNA_DIRECT(0, 3);
    else XDNA_DIRECT(0, 4);
  }
#undef XDNA_DIRECT
  // stream-ordered reuse: the next user of the block runs after the conv
  xdna_hip_cache_free(wp);
  return check_launch("conv direct");
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
  if (sh == 1 && sw == 1) {
    const int rc = run_direct(x, w, bias, y, B, Cin, Cout, H, W, KH, KW, ph, pw, 0, as_stream(stream));
    if (rc <= 0) return rc;
  }
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
  if (sh == 1 && sw == 1 && ph <= KH - 1 && pw <= KW - 1) {
    // at stride 1 the input gradient is the forward conv of dy with the flipped,
    // transposed weights and padding K - 1 - p, which gives back H x W
    const int rc = run_direct(dy, w, nullptr, dx, B, Cout, Cin, a.Ho, a.Wo, KH, KW, KH - 1 - ph, KW - 1 - pw, 1,
                              as_stream(stream));
    if (rc <= 0) return rc;
  }
  return launch_gather<kGDgrad>(a, as_stream(stream));
}

int xdna_conv2d_wgrad_bf16(const uint16_t* x, const uint16_t* dy, uint16_t* gw, uint16_t* gb, int B, int Cin,
                           int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph, int pw,
                           void* stream) {
  GArgs a{};
  if (!gconv_args("xdna_conv2d_wgrad_bf16", a, B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw)) return -1;
  a.x = x; a.dy = dy;
  hipStream_t st = as_stream(stream);
  FsArgs fs{};
  int fs_nt = 0;
  if (slide_args(fs, B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw, a.Ho, a.Wo, fs_nt)) {
    fs.x = x;
    fs.dy = dy;
    const int64_t nwg = ceil_div(fs.rows, fs.rows_per_wg);
    const int64_t mn = int64_t(Cout) * Cin * KH * KW;
    if (!admit_launch("xdna_conv2d_wgrad_bf16")) return -1;
    fs.part = static_cast<float*>(xdna_hip_cache_alloc(size_t(nwg) * size_t(mn) * sizeof(float)));
    if (!fs.part) return -1;
    const size_t lds = slide_lds(Cin, KH, fs.pitch, fs.R, fs.Wo);
    const unsigned grid = unsigned(nwg);
    const int rc = Cout == 1   ? launch_slide<1>(fs, KW, grid, fs_nt, lds, st)
                   : Cout == 2 ? launch_slide<2>(fs, KW, grid, fs_nt, lds, st)
                   : Cout == 3 ? launch_slide<3>(fs, KW, grid, fs_nt, lds, st)
                               : launch_slide<4>(fs, KW, grid, fs_nt, lds, st);
    if (rc) {
      xdna_hip_cache_free(fs.part);
      return -1;
    }
    gather_reduce_kernel<<<unsigned(std::min<int64_t>(ceil_div(mn, 32), 8192)), 256, 0, st>>>(fs.part, gw, mn,
                                                                                           int(nwg));
    xdna_hip_cache_free(fs.part);  // stream-ordered reuse
    if (check_launch("xdna_conv2d_wgrad_bf16")) return -1;
    if (gb) return xdna_conv3x3_bias_grad_bf16(dy, gb, B, Cout, a.Ho, a.Wo, stream);
    return 0;
  }
  if (fewout_ok(Cout, Cin, KH, KW, sh, sw, a.Wo)) {
    FoArgs f{x, dy, nullptr, B, Cin, Cout, H, W, KH, KW, ph, pw, a.Ho, a.Wo, a.Wo + KW - 1, 1,
             int64_t(B) * a.Ho};
    // about two workgroups per CU, at least one output row each
    const int64_t wgs = std::min<int64_t>(f.rows, 512);
    f.rows_per_wg = int(ceil_div(f.rows, wgs));
    const int64_t nwg = ceil_div(f.rows, f.rows_per_wg);
    const int64_t mn = int64_t(Cout) * Cin * KH * KW;
    if (!admit_launch("xdna_conv2d_wgrad_bf16")) return -1;
    f.part = static_cast<float*>(xdna_hip_cache_alloc(size_t(nwg) * size_t(mn) * sizeof(float)));
    if (!f.part) return -1;
    const size_t lds = size_t(int64_t(Cin) * KH * f.Wp + 4 * f.Wo) * 4;
    if (Cout == 1) wgrad_fewout_kernel<1><<<unsigned(nwg), 256, lds, st>>>(f);
    else if (Cout == 2) wgrad_fewout_kernel<2><<<unsigned(nwg), 256, lds, st>>>(f);
    else if (Cout == 3) wgrad_fewout_kernel<3><<<unsigned(nwg), 256, lds, st>>>(f);
    else wgrad_fewout_kernel<4><<<unsigned(nwg), 256, lds, st>>>(f);
    gather_reduce_kernel<<<unsigned(std::min<int64_t>(ceil_div(mn, 32), 8192)), 256, 0, st>>>(f.part, gw, mn,
                                                                                           int(nwg));
    xdna_hip_cache_free(f.part);  // stream-ordered reuse
    if (check_launch("xdna_conv2d_wgrad_bf16")) return -1;
    if (gb) return xdna_conv3x3_bias_grad_bf16(dy, gb, B, Cout, a.Ho, a.Wo, stream);
    return 0;
  }
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

int xdna_conv2d_set_variant(int variant) {
  if (variant < 0 || variant > 1) {
    set_error("xdna_conv2d_set_variant: variant must be 0 or 1");
    return -1;
  }
  g_conv2d_variant.store(variant);
  return 0;
}

}  // extern "C"
