// Losses of plain training scripts on gfx950: mse_loss (mean or sum) and its backward, for
// fp32 or bf16 operands whose target is either the same shape or a batch-broadcast of a
// contiguous block (target.expand_as(input), as a style loss compares per-image Gram
// matrices with one target).  The reference runs both on its CPU through the zero-copy
// fallback (torch_xdna_device.cpp:5124-5260); PyTorch-ROCm's forms take three launches
// forward (squared differences, output fill, reduction) and two backward (zero fill,
// elementwise), each a few microseconds at these sizes.
//
// Forward, two launches: workgroup k sums the squared differences of a fixed slice of the
// elements (fp32 per thread, fixed tree across the workgroup) into partial k; one
// workgroup then adds the partials in index order (fp64) and writes the scalar.  The
// partition depends on n only, so equal inputs give equal bits.  (Finishing in the last
// workgroup of the first launch would need a device-scope fence per workgroup, whose L2
// write-back costs more than the second launch on this multi-XCD part.)
//
// Backward, one launch: grad[i] = norm * (a[i] - b[i % period]) * go, go the incoming
// gradient read on the device (no host sync; graph-capturable), norm = 2 / n (mean) or 2.
#include "common.h"

#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kLossThreads = 256;
constexpr int kMaxLossParts = 1024;
template <typename T>
__device__ inline float load_f(const T* p, int64_t i);
template <>
__device__ inline float load_f<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ inline float load_f<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

template <typename T>
__device__ inline void store_f(T* p, int64_t i, float v);
template <>
__device__ inline void store_f<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ inline void store_f<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// VEC consecutive elements starting at i (16-byte aligned when VEC > 1)
template <typename T, int VEC>
__device__ inline void load_vec(const T* p, int64_t i, float (&v)[VEC]) {
  if constexpr (VEC == 1) {
    v[0] = load_f<T>(p, i);
  } else if constexpr (sizeof(T) == 4) {
    static_assert(VEC == 4, "fp32 vectors are 4 elements");
    const float4 q = *reinterpret_cast<const float4*>(p + i);
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else {
    static_assert(VEC == 8, "bf16 vectors are 8 elements");
    const uint4 q = *reinterpret_cast<const uint4*>(p + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(w[k] << 16);
      v[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
    }
  }
}

__device__ inline float wave_reduce(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

struct MseArgs {
  const void* a;
  const void* b;
  int64_t n, period;  // b element of a's element i: b[i % period]
  int64_t slice;      // elements per workgroup (a multiple of VEC)
  float* part;        // [gridDim.x]
};

template <typename T, int VEC>
__global__ __launch_bounds__(kLossThreads) void mse_sum_kernel(MseArgs m) {
  const T* a = static_cast<const T*>(m.a);
  const T* b = static_cast<const T*>(m.b);
  const int tid = threadIdx.x;
  const int64_t lo = int64_t(blockIdx.x) * m.slice;
  const int64_t hi = min(m.n, lo + m.slice);
  float s = 0.0f;
  int64_t i = lo + int64_t(tid) * VEC;
  const int64_t step = int64_t(kLossThreads) * VEC;
  int64_t j = i % m.period;
  const int64_t jstep = step % m.period;
  for (; i < hi; i += step) {
    float va[VEC], vb[VEC];
    load_vec<T, VEC>(a, i, va);
    load_vec<T, VEC>(b, j, vb);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = va[k] - vb[k];
      s += d * d;
    }
    j += jstep;
    if (j >= m.period) j -= m.period;
  }
  __shared__ float red[kLossThreads / 64];
  s = wave_reduce(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kLossThreads / 64; ++w) t += red[w];
    m.part[blockIdx.x] = t;
  }
}

// out = scale * (the parts added in index order, fp64), in the operands' dtype
template <typename T>
__global__ __launch_bounds__(kLossThreads) void mse_finish_kernel(const float* __restrict__ part, int parts,
                                                                  double scale, T* __restrict__ out) {
  const int tid = threadIdx.x;
  double d = 0.0;
  for (int k = tid; k < parts; k += kLossThreads) d += double(part[k]);
  __shared__ double dred[kLossThreads];
  dred[tid] = d;
  __syncthreads();
  for (int w = kLossThreads / 2; w > 0; w >>= 1) {
    if (tid < w) dred[tid] += dred[tid + w];
    __syncthreads();
  }
  if (tid == 0) store_f<T>(out, 0, float(dred[0] * scale));
}

struct MseBwdArgs {
  const void* go;
  int go_dtype;  // 1 fp32, 2 bf16
  const void* a;
  const void* b;
  void* grad;
  int64_t n, period;
  float norm;
};

template <typename T, int VEC>
__global__ __launch_bounds__(kLossThreads) void mse_bwd_kernel(MseBwdArgs m) {
  const T* a = static_cast<const T*>(m.a);
  const T* b = static_cast<const T*>(m.b);
  T* g = static_cast<T*>(m.grad);
  const float go = m.go_dtype == 1 ? *static_cast<const float*>(m.go) : bf16_to_f32(*static_cast<const uint16_t*>(m.go));
  const int64_t step = int64_t(gridDim.x) * kLossThreads * VEC;
  int64_t i = (int64_t(blockIdx.x) * kLossThreads + threadIdx.x) * VEC;
  int64_t j = i % m.period;
  const int64_t jstep = step % m.period;
  for (; i < m.n; i += step) {
    float va[VEC], vb[VEC];
    load_vec<T, VEC>(a, i, va);
    load_vec<T, VEC>(b, j, vb);
    // PyTorch's order: norm * (a - b) * go in fp32
    if constexpr (VEC == 1) {
      store_f<T>(g, i, m.norm * (va[0] - vb[0]) * go);
    } else if constexpr (sizeof(T) == 4) {
      float4 q;
      q.x = m.norm * (va[0] - vb[0]) * go;
      q.y = m.norm * (va[1] - vb[1]) * go;
      q.z = m.norm * (va[2] - vb[2]) * go;
      q.w = m.norm * (va[3] - vb[3]) * go;
      *reinterpret_cast<float4*>(g + i) = q;
    } else {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = uint32_t(f32_to_bf16(m.norm * (va[2 * k] - vb[2 * k]) * go)) |
               (uint32_t(f32_to_bf16(m.norm * (va[2 * k + 1] - vb[2 * k + 1]) * go)) << 16);
      *reinterpret_cast<uint4*>(g + i) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    j += jstep;
    if (j >= m.period) j -= m.period;
  }
}

bool aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// elements per vector for dtype 1 (fp32) / 2 (bf16), or 1 when the operands or the period
// do not allow 16-byte vectors
int vec_width(int dtype, const void* a, const void* b, const void* out, int64_t n, int64_t period) {
  const int v = dtype == 1 ? 4 : 8;
  if (!aligned(a) || !aligned(b) || (out && !aligned(out)) || n % v != 0 || period % v != 0) return 1;
  return v;
}

bool mse_args_ok(const char* what, const void* a, const void* b, int dtype, int64_t n, int64_t period,
                 int reduction) {
  if (!a || !b || (dtype != 1 && dtype != 2) || n < 1 || period < 1 || period > n || n % period != 0 ||
      (reduction != 1 && reduction != 2)) {
    set_error(std::string(what) + ": invalid arguments");
    return false;
  }
  return true;
}

int mse_parts(int64_t n) {
  return int(std::max<int64_t>(1, std::min<int64_t>(kMaxLossParts, ceil_div(n, int64_t(kLossThreads) * 32))));
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

size_t xdna_mse_loss_workspace_bytes(int64_t n) {
  return n < 1 ? 0 : size_t(mse_parts(n)) * sizeof(float);
}

int xdna_mse_loss(const void* a, const void* b, int dtype, int64_t n, int64_t period, int reduction, void* out,
                  void* workspace, size_t workspace_bytes, void* stream) {
  if (!mse_args_ok("xdna_mse_loss", a, b, dtype, n, period, reduction)) return -1;
  const int parts0 = mse_parts(n);
  if (!out || !workspace || workspace_bytes < size_t(parts0) * sizeof(float)) {
    set_error("xdna_mse_loss: output or workspace missing or too small");
    return -1;
  }
  if (!admit_launch("xdna_mse_loss")) return -1;
  const int vec = vec_width(dtype, a, b, nullptr, n, period);
  MseArgs m;
  m.a = a;
  m.b = b;
  m.n = n;
  m.period = period;
  // a fixed slice per workgroup, a multiple of the vector width
  m.slice = ceil_div(ceil_div(n, int64_t(parts0)), int64_t(vec)) * vec;
  const int parts = int(ceil_div(n, m.slice));
  m.part = static_cast<float*>(workspace);
  const double scale = reduction == 1 ? 1.0 / double(n) : 1.0;
  hipStream_t st = as_stream(stream);
  const dim3 grid{unsigned(parts)};
  if (dtype == 1) {
    if (vec == 4) mse_sum_kernel<float, 4><<<grid, kLossThreads, 0, st>>>(m);
    else mse_sum_kernel<float, 1><<<grid, kLossThreads, 0, st>>>(m);
    mse_finish_kernel<float><<<1, kLossThreads, 0, st>>>(m.part, parts, scale, static_cast<float*>(out));
  } else {
    if (vec == 8) mse_sum_kernel<uint16_t, 8><<<grid, kLossThreads, 0, st>>>(m);
    else mse_sum_kernel<uint16_t, 1><<<grid, kLossThreads, 0, st>>>(m);
    mse_finish_kernel<uint16_t><<<1, kLossThreads, 0, st>>>(m.part, parts, scale, static_cast<uint16_t*>(out));
  }
  return check_launch("xdna_mse_loss");
}

int xdna_mse_loss_bwd(const void* go, int go_dtype, const void* a, const void* b, int dtype, int64_t n,
                      int64_t period, int reduction, void* grad, void* stream) {
  if (!mse_args_ok("xdna_mse_loss_bwd", a, b, dtype, n, period, reduction)) return -1;
  if (!go || (go_dtype != 1 && go_dtype != 2) || !grad) {
    set_error("xdna_mse_loss_bwd: the incoming gradient must be an fp32 or bf16 device scalar");
    return -1;
  }
  if (!admit_launch("xdna_mse_loss_bwd")) return -1;
  const int vec = vec_width(dtype, a, b, grad, n, period);
  MseBwdArgs m;
  m.go = go;
  m.go_dtype = go_dtype;
  m.a = a;
  m.b = b;
  m.grad = grad;
  m.n = n;
  m.period = period;
  m.norm = float(reduction == 1 ? 2.0 / double(n) : 2.0);
  const int64_t vecs = ceil_div(n, int64_t(vec));
  const dim3 grid(unsigned(std::max<int64_t>(1, std::min<int64_t>(ceil_div(vecs, int64_t(kLossThreads)), 8192))));
  hipStream_t st = as_stream(stream);
  if (dtype == 1) {
    if (vec == 4) mse_bwd_kernel<float, 4><<<grid, kLossThreads, 0, st>>>(m);
    else mse_bwd_kernel<float, 1><<<grid, kLossThreads, 0, st>>>(m);
  } else {
    if (vec == 8) mse_bwd_kernel<uint16_t, 8><<<grid, kLossThreads, 0, st>>>(m);
    else mse_bwd_kernel<uint16_t, 1><<<grid, kLossThreads, 0, st>>>(m);
  }
  return check_launch("xdna_mse_loss_bwd");
}

}  // extern "C"
