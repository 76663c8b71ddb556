// Column sums of a row-major bf16 matrix, out[n] = bf16(sum over rows r of x[r][n]) with
// fp32 accumulation and one rounding: the bias gradient of a Linear layer (autograd reduces
// addmm's output gradient [M, N] over its rows).  The reference reaches this sum through
// its zero-copy CPU fallback (torch_xdna_device.cpp:5124-5260); PyTorch-ROCm's reduction
// takes a fill and a reduction launch, 23-27 us on config 3's [8192, 1024 .. 4096] gradients.
//
// Two fixed-order stages, so equal inputs give equal bits: workgroup (c, s) sums rows
// [s R/S, (s+1) R/S) of a block of columns, each thread four consecutive columns (8-byte
// loads, rows in order) into fp32 partial s; then each column adds its S (at most 256)
// partials in a fixed association and rounds once.  One slice: the first stage writes the
// result itself.
#include "common.h"

#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kColThreads = 256;
constexpr int kColPer = 4;                            // columns per thread
constexpr int kColBlock = kColThreads * kColPer;      // columns per workgroup

// V: 4 columns per thread with 8-byte loads (N % 4 == 0, 8-byte aligned rows); else one
// column per thread.  Rows are read eight at a time, all eight loads issued before the sums,
// which take the rows in order.
template <bool V>
__global__ __launch_bounds__(kColThreads) void colsum_part_kernel(const uint16_t* __restrict__ x,
                                                                  float* __restrict__ part,
                                                                  uint16_t* __restrict__ out, int64_t R,
                                                                  int64_t N, int64_t rows_per) {
  constexpr int kRU = 8;
  const int64_t s = blockIdx.y;
  const int64_t r0 = s * rows_per, r1 = min(R, r0 + rows_per);
  if (V) {
    const int64_t n = (int64_t(blockIdx.x) * kColThreads + threadIdx.x) * kColPer;
    if (n >= N) return;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    for (int64_t r = r0; r < r1; r += kRU) {
      uint2 v[kRU];
#pragma unroll
      for (int u = 0; u < kRU; ++u)
        v[u] = r + u < r1 ? *reinterpret_cast<const uint2*>(x + (r + u) * N + n) : make_uint2(0, 0);
#pragma unroll
      for (int u = 0; u < kRU; ++u)
        if (r + u < r1) {
          a0 += __uint_as_float(v[u].x << 16);
          a1 += __uint_as_float(v[u].x & 0xFFFF0000u);
          a2 += __uint_as_float(v[u].y << 16);
          a3 += __uint_as_float(v[u].y & 0xFFFF0000u);
        }
    }
    if (out) {
      *reinterpret_cast<uint2*>(out + n) =
          make_uint2(uint32_t(f32_to_bf16(a0)) | (uint32_t(f32_to_bf16(a1)) << 16),
                     uint32_t(f32_to_bf16(a2)) | (uint32_t(f32_to_bf16(a3)) << 16));
    } else {
      *reinterpret_cast<float4*>(part + s * N + n) = make_float4(a0, a1, a2, a3);
    }
  } else {
    const int64_t n = int64_t(blockIdx.x) * kColThreads + threadIdx.x;
    if (n >= N) return;
    float a = 0.f;
    for (int64_t r = r0; r < r1; r += kRU) {
      float v[kRU];
#pragma unroll
      for (int u = 0; u < kRU; ++u) v[u] = r + u < r1 ? bf16_to_f32(x[(r + u) * N + n]) : 0.f;
#pragma unroll
      for (int u = 0; u < kRU; ++u)
        if (r + u < r1) a += v[u];
    }
    if (out) out[n] = f32_to_bf16(a);
    else part[s * N + n] = a;
  }
}

// out[n] = bf16(sum of the S slice partials of column n): a workgroup takes 32 columns; its
// 8 thread groups sum slices z, z + 8, ... (group z), and the 8 group sums are added in
// order through LDS: a fixed association per column.
constexpr int kFinCols = 32, kFinGroups = 8;
__global__ __launch_bounds__(kColThreads) void colsum_finish_kernel(const float* __restrict__ part,
                                                                    uint16_t* __restrict__ out, int64_t S,
                                                                    int64_t N) {
  __shared__ float red[kColThreads];
  const int z = threadIdx.x / kFinCols, e = threadIdx.x % kFinCols;
  const int64_t n = int64_t(blockIdx.x) * kFinCols + e;
  float a = 0.f;
  if (n < N) a = sum_strided8(0.0f, part + n, N, z, kFinGroups, int(S));
  red[threadIdx.x] = a;
  __syncthreads();
  if (z != 0 || n >= N) return;
  for (int q = 1; q < kFinGroups; ++q) a += red[q * kFinCols + e];
  out[n] = f32_to_bf16(a);
}

struct ColsumPlan {
  bool vec = false;
  int64_t col_blocks = 0, slices = 1, rows_per = 0;
};

ColsumPlan colsum_plan(const uint16_t* x, int64_t R, int64_t N) {
  ColsumPlan p;
  p.vec = (N % kColPer) == 0 && (reinterpret_cast<uintptr_t>(x) & 7) == 0;
  p.col_blocks = ceil_div(N, p.vec ? kColBlock : kColThreads);
  // about 512 workgroups, each at least 16 rows, at most 256 slices (64 left [8192, 1024]
  // on 64 workgroups: 14 us, 1.2 TB/s)
  p.slices = std::max<int64_t>(1, std::min<int64_t>({ceil_div(512, p.col_blocks), ceil_div(R, 16), 256}));
  p.rows_per = ceil_div(R, p.slices);
  p.slices = ceil_div(R, p.rows_per);
  return p;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

size_t xdna_colsum_workspace_bytes(const uint16_t* x, int64_t R, int64_t N) {
  if (R < 1 || N < 1) return 0;
  const ColsumPlan p = colsum_plan(x, R, N);
  return p.slices > 1 ? size_t(p.slices) * size_t(N) * sizeof(float) : 0;
}

int xdna_colsum_bf16(const uint16_t* x, uint16_t* out, int64_t R, int64_t N, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (!x || !out || R < 1 || N < 1 || R > (int64_t(1) << 40) || N > (int64_t(1) << 40)) {
    set_error("xdna_colsum_bf16: invalid arguments");
    return -1;
  }
  const ColsumPlan p = colsum_plan(x, R, N);
  const size_t need = p.slices > 1 ? size_t(p.slices) * size_t(N) * sizeof(float) : 0;
  if (need && (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15))) {
    set_error("xdna_colsum_bf16: workspace too small or not 16-byte aligned (xdna_colsum_workspace_bytes)");
    return -1;
  }
  if (p.slices > 65535) {
    set_error("xdna_colsum_bf16: too many row slices");
    return -1;
  }
  if (!admit_launch("colsum")) return -1;
  hipStream_t st = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  uint16_t* direct = p.slices == 1 ? out : nullptr;
  const dim3 grid(unsigned(p.col_blocks), unsigned(p.slices));
  if (p.vec)
    colsum_part_kernel<true><<<grid, kColThreads, 0, st>>>(x, part, direct, R, N, p.rows_per);
  else
    colsum_part_kernel<false><<<grid, kColThreads, 0, st>>>(x, part, direct, R, N, p.rows_per);
  if (p.slices > 1)
    colsum_finish_kernel<<<unsigned(ceil_div(N, kFinCols)), kColThreads, 0, st>>>(part, out, p.slices, N);
  return check_launch("colsum");
}

}  // extern "C"
