// Shared helpers of the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <numeric>
#include <string>

namespace xdna {

// ---- errors (thread-local message, int status) --------------------------------

void set_error(const std::string& msg);
void clear_error();
// Counts a launch; returns false (error already set) when the process is poisoned
// or an injected failure fires.  Every C-ABI compute entry point calls it once
// before launching anything.
bool admit_launch(const char* what);
// Records a HIP error from a launch; poisons the process for errors that can leave
// device work behind.  Returns -1.
int launch_failed(const char* what, hipError_t err);
// Checks hipGetLastError() after kernel launches: 0 or -1.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- conv3x3w geometry (reference torch_xdna_device.cpp:1916-1937, 2112-2157) ----

constexpr int kGroupOutRows = 2048;
constexpr int kGroupRows = 2126;   // 2048 + 2*(36+2) + 2: the 3x3 window of a group
constexpr int kKStep = 64;         // channels per chunk
constexpr int kRawN = 128;         // channels per raw output row block
constexpr int kMaxWidth = 36;
constexpr int kMaxStrip = 34;

// Two row layouts share the group structure above.
//  kLayoutRef: the reference's conv3x3w layout.  Images wider than 36 are cut into S strips
//    of So <= 34 columns; a strip row holds Wg = So + 2 data columns (the strip's columns
//    and one neighbour column each side, zero at the image border) between two zero
//    columns (wp = Wg + 2, data column j at row position j + 1).
//  kLayoutTight: the same up to 36 columns; wider images as strips of So <= 36 columns
//    whose rows hold only the Wg = So + 2 data columns (wp = Wg, data column j at row
//    position j).  The taps of a real output column stay inside its strip row, so the
//    zero columns are never read: for 72 columns, 2 strips of 38 positions instead of 3
//    of 28 (8.5% more rows than pixels instead of 20%).
// Output column c of a strip is output row position c + first of its image row.
constexpr int kLayoutRef = 0;
constexpr int kLayoutTight = 1;
constexpr int kMaxStripTight = 36;

struct StripGeom {
  int S = 1, So = 0, Wg = 0, wp = 0;
  int lead = 1;   // row position of data column 0
  int first = 0;  // output row position of output column 0
};

inline StripGeom strip_geom(int W, int layout = kLayoutRef) {
  StripGeom g;
  if (W <= kMaxWidth) {
    g.S = 1; g.So = W; g.Wg = W; g.wp = W + 2;
  } else if (layout == kLayoutTight) {
    g.S = int(ceil_div(W, kMaxStripTight));
    g.So = int(ceil_div(W, g.S));
    g.Wg = g.So + 2;
    g.wp = g.Wg;
    g.lead = 0;
  } else {
    g.S = int(ceil_div(W, kMaxStrip));
    g.So = int(ceil_div(W, g.S));
    g.Wg = g.So + 2;
    g.wp = g.Wg + 2;
  }
  // output row p is centred on packed row p + wp + 1; output column c reads data column
  // c + (S > 1) at row position c + (S > 1) + lead
  g.first = (g.S > 1 ? 1 : 0) + g.lead - 1;
  return g;
}

struct ConvGeom {
  StripGeom st;
  int B = 0, H = 0, W = 0;
  int64_t img = 0;      // (H+2)*wp rows per virtual image
  int64_t m_total = 0;  // B*S*img
  int groups = 0;
};

inline ConvGeom conv_geom(int B, int H, int W, int layout = kLayoutRef) {
  ConvGeom g;
  g.st = strip_geom(W, layout);
  g.B = B; g.H = H; g.W = W;
  g.img = int64_t(H + 2) * g.st.wp;
  g.m_total = int64_t(B) * g.st.S * g.img;
  g.groups = int(ceil_div(g.m_total, kGroupOutRows));
  return g;
}

// ---- bf16 <-> fp32 -----------------------------------------------------------

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Round to nearest even; NaN -> quiet NaN 0x7FC0 (the c10::BFloat16 convention).
// gfx950 converts with v_cvt_pk_bf16_f32, which rounds to nearest even exactly as
// (u + 0x7FFF + lsb) >> 16 for every non-NaN input, subnormals included (checked over
// all 2^32 patterns on an MI355X); it keeps a NaN's sign and payload, hence the select.
__device__ inline uint16_t f32_to_bf16(float f) {
  const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  return f != f ? uint16_t(0x7FC0) : h;
}

// A buffer resource's record count from a byte extent, clamped to 2^31 - 1 with integer
// compares (HIP's min over int64_t resolves to the double overload, whose VALU result makes
// a resource built from it per-lane: every access through it then runs a waterfall loop).
__device__ inline int clamp_records(int64_t bytes) { return bytes < 0x7FFFFFFF ? int(bytes) : 0x7FFFFFFF; }

// A buffer resource over bytes from p, built from lane 0's values: a scalar resource even
// where the compiler cannot prove its inputs wave-uniform (a per-lane resource turns every
// access through it into a waterfall loop).  Callers pass wave-uniform values.
__device__ inline __amdgpu_buffer_rsrc_t uniform_buffer_rsrc(const void* p, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint64_t u = uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))))) |
                     (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))))) << 32);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), 0, __builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

// Split-K partial sums: init + src[z * stride] + src[(z + step) * stride] + ... over
// indices below n, added left to right in that order (the fixed association every
// deterministic reduce here keeps), with eight loads issued before their sums: a loop of
// single loads waits one memory latency per term.
__device__ inline float sum_strided8(float init, const float* __restrict__ src, int64_t stride, int z, int step,
                                     int n) {
  float s = init;
  int k = z;
  for (; k + 7 * step < n; k += 8 * step) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[int64_t(k + u * step) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; k < n; k += step) s += src[int64_t(k) * stride];
  return s;
}

// ---- activations fused into producers (norm outputs, region ops) -------------
// act 0: none, 1: ReLU (PyTorch's: NaN kept, -0 to +0), 2: LeakyReLU with slope
// (x > 0 ? x : x * slope).  Applied to the fp32 value before its one rounding.
__device__ inline float act_forward(int act, float slope, float v) {
  if (act == 1) return v <= 0.0f ? 0.0f : v;
  if (act == 2) return v > 0.0f ? v : v * slope;
  return v;
}

// The gradient through the activation, from its output y: ReLU masks where y <= 0
// (threshold_backward on the result: a NaN result passes the gradient), LeakyReLU scales
// by slope where y <= 0 (leaky_relu_backward on the result).
__device__ inline float act_backward(int act, float slope, float y, float g) {
  if (act == 1) return y <= 0.0f ? 0.0f : g;
  if (act == 2) return y > 0.0f ? g : g * slope;
  return g;
}

}  // namespace xdna
