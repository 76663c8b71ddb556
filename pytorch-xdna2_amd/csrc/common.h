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

struct StripGeom {
  int S = 1, So = 0, Wg = 0, wp = 0;
};

inline StripGeom strip_geom(int W) {
  StripGeom g;
  if (W <= kMaxWidth) {
    g.S = 1; g.So = W; g.Wg = W;
  } else {
    g.S = int(ceil_div(W, kMaxStrip));
    g.So = int(ceil_div(W, g.S));
    g.Wg = g.So + 2;
  }
  g.wp = g.Wg + 2;
  return g;
}

struct ConvGeom {
  StripGeom st;
  int B = 0, H = 0, W = 0;
  int64_t img = 0;      // (H+2)*wp rows per virtual image
  int64_t m_total = 0;  // B*S*img
  int groups = 0;
};

inline ConvGeom conv_geom(int B, int H, int W) {
  ConvGeom g;
  g.st = strip_geom(W);
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

}  // namespace xdna
