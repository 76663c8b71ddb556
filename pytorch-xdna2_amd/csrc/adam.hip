// Fused Adam / AdamW: one HBM pass per element (read p, g, m, v; write p, m, v).
//
// The reference reaches torch._fused_adam_ through its boxed CPU fallback
// (torch_xdna_device.cpp:5124-5260, 5273-5295) after _prefer_fused_optimizer
// (xdna_train/device.py:408-436) sets fused=True, so the arithmetic to match is
// PyTorch's CPU fused kernel.  Per element, in fp32 opmath with the step scalars
// computed in double:
//   g  = grad (/ grad_scale), negated if maximize
//   Adam:  g = fma(p, wd, g)           AdamW: p = p * float(1 - lr*wd)
//   m  = fma(w, g - m, m)              w = float(1 - beta1)  (lerp, |w| < 0.5)
//        fma(-(g - m), 1 - w, g)       (lerp, |w| >= 0.5)
//   v  = fma(float(1-beta2) * g, g, v * float(beta2))
//   den = sqrt(amsgrad ? max(max_v, v) : v) / float(sqrt(1 - beta2^t)) + float(eps)
//   p  = p - (float(lr / (1 - beta1^t)) * m) / den
// and p, m, v (max_v) are stored once in the tensor dtype.  The fused-multiply-add
// placement was fitted bit-exactly against torch 2.10's CPU _fused_adam_ on bf16 and
// fp32 tensors (tests/golden/make_adam_golden.py); its scalar tail (numel % 16) uses
// separate mul/add for v, which differs from this in the last fp32 bit only.
//
// Multi-tensor launch: up to kMaxTensors tensors per launch, passed by value; block
// b belongs to the tensor whose block range contains it.  8 elements per thread per
// iteration (16-byte bf16 vectors).
#include "common.h"
#include "../../include/xdna_hip.h"

#include <algorithm>
#include <cmath>
#include <vector>

namespace xdna {
namespace {

constexpr int kMaxTensors = 24;
constexpr int kThreads = 256;
constexpr int kVec = 8;
constexpr int kIters = 2;  // 4096 elements per workgroup (measured: 2 beats 1, 4 and 8 by 4-15 %)
constexpr int64_t kBlockElems = int64_t(kThreads) * kVec * kIters;

struct AdamArgs {
  void* p[kMaxTensors];
  void* g[kMaxTensors];
  void* m[kMaxTensors];
  void* v[kMaxTensors];
  void* mx[kMaxTensors];
  const float* step[kMaxTensors];
  int64_t numel[kMaxTensors];
  int32_t block_start[kMaxTensors + 1];
  int32_t vec_ok[kMaxTensors];
  int n;
};

struct AdamScalars {
  double lr, beta1, beta2, wd, eps;
  int amsgrad, maximize, adamw;
  // lr as a device scalar (torch's tensor-lr overloads), read where the step constants
  // are computed: 0 absent (lr above), 1 fp32, 2 fp64
  const void* lr_dev;
  int lr_dtype;
};

template <typename T> __device__ inline float ld(const T* p, int64_t i);
template <> __device__ inline float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ inline float ld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> __device__ inline void st(T* p, int64_t i, float v);
template <> __device__ inline void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ inline void st<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 8 consecutive elements <-> fp32 registers.
template <typename T> struct Vec8;
template <> struct Vec8<uint16_t> {
  __device__ static inline void load(const uint16_t* p, int64_t i, float* f) {
    const uint4 w = *reinterpret_cast<const uint4*>(p + i);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __uint_as_float(u[e] << 16);
      f[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
    }
  }
  __device__ static inline void store(uint16_t* p, int64_t i, const float* f) {
    uint32_t u[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      u[e] = uint32_t(f32_to_bf16(f[2 * e])) | (uint32_t(f32_to_bf16(f[2 * e + 1])) << 16);
    *reinterpret_cast<uint4*>(p + i) = make_uint4(u[0], u[1], u[2], u[3]);
  }
};
template <> struct Vec8<float> {
  __device__ static inline void load(const float* p, int64_t i, float* f) {
    const float4 a = *reinterpret_cast<const float4*>(p + i);
    const float4 b = *reinterpret_cast<const float4*>(p + i + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
  __device__ static inline void store(float* p, int64_t i, const float* f) {
    *reinterpret_cast<float4*>(p + i) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4*>(p + i + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
};

struct StepConsts {
  float step_size, bc2_sqrt, eps, beta2, one_minus_beta2, w, one_minus_w, wd, decay;
};

__device__ inline void adam_elem(float& p, float& g, float& m, float& v, float& mx,
                                 const StepConsts& k, const AdamScalars& s) {
  if (s.maximize) g = -g;
  if (s.wd != 0.0) {
    if (s.adamw) p = p * k.decay;
    else g = __builtin_fmaf(p, k.wd, g);
  }
  const float d = g - m;
  m = fabsf(k.w) < 0.5f ? __builtin_fmaf(k.w, d, m) : __builtin_fmaf(-d, k.one_minus_w, g);
  v = __builtin_fmaf(k.one_minus_beta2 * g, g, v * k.beta2);
  float src = v;
  if (s.amsgrad) {
    mx = fmaxf(mx, v);
    src = mx;
  }
  const float den = __builtin_sqrtf(src) / k.bc2_sqrt + k.eps;
  p = p - (k.step_size * m) / den;
}

// Bias corrections of this tensor's step, in double as torch's _fused_adam_ computes
// them (step_size = lr / (1 - beta1^t), sqrt(1 - beta2^t)).
__device__ inline StepConsts step_consts(const AdamScalars& s, float step_f) {
  const double step = double(step_f);
  const double bc1 = 1.0 - pow(s.beta1, step);
  const double bc2 = 1.0 - pow(s.beta2, step);
  // a tensor lr is used at its value as a double, as torch's CPU kernel reads it
  // (lr.item<double>())
  const double lr = s.lr_dtype == 1   ? double(*static_cast<const float*>(s.lr_dev))
                    : s.lr_dtype == 2 ? *static_cast<const double*>(s.lr_dev)
                                      : s.lr;
  StepConsts k;
  k.step_size = float(lr / bc1);
  k.bc2_sqrt = float(sqrt(bc2));
  k.eps = float(s.eps);
  k.beta2 = float(s.beta2);
  k.one_minus_beta2 = float(1.0 - s.beta2);
  k.w = float(1.0 - s.beta1);
  k.one_minus_w = 1.0f - k.w;
  k.wd = float(s.wd);
  k.decay = float(1.0 - lr * s.wd);
  return k;
}

// 16-byte raw vector <-> 8 fp32 values (bf16: 8 elements; fp32: 4 elements per vector,
// two vectors per 8).
template <typename T> struct Raw;
template <> struct Raw<uint16_t> {
  static constexpr int kVecs = 1;
  __device__ static inline void to_f32(const u32x4& w, const u32x4&, float* f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __uint_as_float(w[e] << 16);
      f[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
  }
};
template <> struct Raw<float> {
  static constexpr int kVecs = 2;
  __device__ static inline void to_f32(const u32x4& a, const u32x4& b, float* f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = __uint_as_float(a[e]);
      f[4 + e] = __uint_as_float(b[e]);
    }
  }
};

// One workgroup per kBlockElems elements of one tensor (block_start prefix).  A full
// item issues all its loads (kIters vectors each of p, g, m, v per thread, raw) before
// thread 0 computes the step constants (double-precision bias corrections) and the
// workgroup waits for them: the loads' latency covers that work.
template <typename T>
__global__ __launch_bounds__(kThreads) void fused_adam_kernel(AdamArgs a, AdamScalars s,
                                                              const float* grad_scale,
                                                              const float* found_inf) {
  if (found_inf && *found_inf == 1.0f) return;
  __shared__ StepConsts sk;
  int t = 0;
  while (t + 1 < a.n && int(blockIdx.x) >= a.block_start[t + 1]) ++t;
  T* P = static_cast<T*>(a.p[t]);
  T* G = static_cast<T*>(a.g[t]);
  T* M = static_cast<T*>(a.m[t]);
  T* V = static_cast<T*>(a.v[t]);
  T* MX = static_cast<T*>(a.mx[t]);
  const int64_t n = a.numel[t];
  const int64_t base = int64_t(blockIdx.x - a.block_start[t]) * kBlockElems;
  const int64_t i0 = base + int64_t(threadIdx.x) * kVec;
  constexpr int64_t kStride = int64_t(kThreads) * kVec;
  constexpr int RV = Raw<T>::kVecs;
  const bool full = a.vec_ok[t] && base + kBlockElems <= n && !s.amsgrad && !grad_scale;
  u32x4 rp[kIters][RV], rg[kIters][RV], rm[kIters][RV], rv[kIters][RV];
  if (full) {
#pragma unroll
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int q = 0; q < RV; ++q) {
        const int64_t j = i0 + it * kStride + q * (8 / RV);
        rp[it][q] = *reinterpret_cast<const u32x4*>(P + j);
        rg[it][q] = *reinterpret_cast<const u32x4*>(G + j);
        rm[it][q] = *reinterpret_cast<const u32x4*>(M + j);
        rv[it][q] = *reinterpret_cast<const u32x4*>(V + j);
      }
  }
  if (threadIdx.x == 0) sk = step_consts(s, *a.step[t]);
  __syncthreads();
  const StepConsts k = sk;
  if (full) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      float p[kVec], g[kVec], m[kVec], v[kVec];
      Raw<T>::to_f32(rp[it][0], rp[it][RV - 1], p);
      Raw<T>::to_f32(rg[it][0], rg[it][RV - 1], g);
      Raw<T>::to_f32(rm[it][0], rm[it][RV - 1], m);
      Raw<T>::to_f32(rv[it][0], rv[it][RV - 1], v);
      float mx_unused = 0.0f;
#pragma unroll
      for (int e = 0; e < kVec; ++e) adam_elem(p[e], g[e], m[e], v[e], mx_unused, k, s);
      const int64_t j = i0 + it * kStride;
      Vec8<T>::store(P, j, p);
      Vec8<T>::store(M, j, m);
      Vec8<T>::store(V, j, v);
    }
    return;
  }
  const float inv_scale_div = grad_scale ? *grad_scale : 1.0f;
  for (int it = 0; it < kIters; ++it) {
    const int64_t j0 = i0 + it * kStride;
    if (j0 >= n) break;
    if (a.vec_ok[t] && j0 + kVec <= n) {
      float p[kVec], g[kVec], m[kVec], v[kVec], mx[kVec];
      Vec8<T>::load(P, j0, p);
      Vec8<T>::load(G, j0, g);
      Vec8<T>::load(M, j0, m);
      Vec8<T>::load(V, j0, v);
      if (s.amsgrad) Vec8<T>::load(MX, j0, mx);
      if (grad_scale) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) g[e] = g[e] / inv_scale_div;
        Vec8<T>::store(G, j0, g);
      }
#pragma unroll
      for (int e = 0; e < kVec; ++e) adam_elem(p[e], g[e], m[e], v[e], mx[e], k, s);
      Vec8<T>::store(P, j0, p);
      Vec8<T>::store(M, j0, m);
      Vec8<T>::store(V, j0, v);
      if (s.amsgrad) Vec8<T>::store(MX, j0, mx);
    } else {
      for (int64_t i = j0; i < j0 + kVec && i < n; ++i) {
        float p = ld(P, i), g = ld(G, i), m = ld(M, i), v = ld(V, i);
        float mx = s.amsgrad ? ld(MX, i) : 0.0f;
        if (grad_scale) {
          g = g / inv_scale_div;
          st(G, i, g);
        }
        adam_elem(p, g, m, v, mx, k, s);
        st(P, i, p);
        st(M, i, m);
        st(V, i, v);
        if (s.amsgrad) st(MX, i, mx);
      }
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// t[i][j] += value for every element of up to kForeachMax fp32 tensors, one launch
// (workgroup i takes tensor i): the optimizers' per-step counter bump
// (torch._foreach_add_(state_steps, 1)) in one kernel instead of one per tensor.
constexpr int kForeachMax = 64;
struct ForeachArgs {
  float* t[kForeachMax];
  int64_t numel[kForeachMax];
};

__global__ __launch_bounds__(256) void foreach_add_f32_kernel(ForeachArgs a, float value) {
  float* t = a.t[blockIdx.x];
  const int64_t n = a.numel[blockIdx.x];
  for (int64_t j = threadIdx.x; j < n; j += 256) t[j] = t[j] + value;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

namespace xdna {
namespace {

int fused_adam_launch(int n_tensors, void* const* params, void* const* grads, void* const* exp_avgs,
                      void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, const float* const* steps,
                      const int64_t* numels, int dtype, const AdamScalars& s, const float* grad_scale,
                      const float* found_inf, void* stream) {
  if (n_tensors < 0 || (dtype != 0 && dtype != 1) || (s.adamw != 0 && s.adamw != 1)) {
    set_error("xdna_fused_adam: invalid arguments");
    return -1;
  }
  if (s.amsgrad && !max_exp_avg_sqs) {
    set_error("xdna_fused_adam: amsgrad needs max_exp_avg_sqs");
    return -1;
  }
  const int amsgrad = s.amsgrad;
  int done = 0;
  while (done < n_tensors) {
    AdamArgs a{};
    int64_t blocks = 0;
    int n = 0;
    while (done + n < n_tensors && n < kMaxTensors) {
      const int i = done + n;
      if (numels[i] < 0 || !steps[i]) {
        set_error("xdna_fused_adam: invalid tensor entry");
        return -1;
      }
      const int64_t nb = ceil_div(numels[i], kBlockElems);
      if (blocks + nb > (int64_t(1) << 30)) break;
      a.p[n] = params[i];
      a.g[n] = grads[i];
      a.m[n] = exp_avgs[i];
      a.v[n] = exp_avg_sqs[i];
      a.mx[n] = amsgrad ? max_exp_avg_sqs[i] : nullptr;
      a.step[n] = steps[i];
      a.numel[n] = numels[i];
      a.block_start[n] = int32_t(blocks);
      a.vec_ok[n] = aligned16(params[i]) && aligned16(grads[i]) && aligned16(exp_avgs[i]) &&
                    aligned16(exp_avg_sqs[i]) && (!amsgrad || aligned16(max_exp_avg_sqs[i]));
      blocks += nb;
      ++n;
    }
    a.block_start[n] = int32_t(blocks);
    a.n = n;
    done += n;
    if (blocks == 0) continue;
    if (!admit_launch("xdna_fused_adam")) return -1;
    if (dtype == 1)
      fused_adam_kernel<uint16_t><<<dim3(unsigned(blocks)), kThreads, 0, as_stream(stream)>>>(
          a, s, grad_scale, found_inf);
    else
      fused_adam_kernel<float><<<dim3(unsigned(blocks)), kThreads, 0, as_stream(stream)>>>(
          a, s, grad_scale, found_inf);
    if (check_launch("xdna_fused_adam")) return -1;
  }
  return 0;
}

}  // namespace
}  // namespace xdna

extern "C" int xdna_fused_adam(int n_tensors, void* const* params, void* const* grads,
                               void* const* exp_avgs, void* const* exp_avg_sqs,
                               void* const* max_exp_avg_sqs, const float* const* steps,
                               const int64_t* numels, int dtype, double lr, double beta1,
                               double beta2, double weight_decay, double eps, int amsgrad,
                               int maximize, int mode, const float* grad_scale,
                               const float* found_inf, void* stream) {
  const AdamScalars s{lr, beta1, beta2, weight_decay, eps, amsgrad ? 1 : 0, maximize ? 1 : 0, mode, nullptr, 0};
  return fused_adam_launch(n_tensors, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, steps, numels,
                           dtype, s, grad_scale, found_inf, stream);
}

extern "C" int xdna_fused_adam_tensor_lr(int n_tensors, void* const* params, void* const* grads,
                                         void* const* exp_avgs, void* const* exp_avg_sqs,
                                         void* const* max_exp_avg_sqs, const float* const* steps,
                                         const int64_t* numels, int dtype, const void* lr, int lr_dtype,
                                         double beta1, double beta2, double weight_decay, double eps,
                                         int amsgrad, int maximize, int mode, const float* grad_scale,
                                         const float* found_inf, void* stream) {
  if (!lr || (lr_dtype != 1 && lr_dtype != 2)) {
    set_error("xdna_fused_adam_tensor_lr: lr must be a device fp32 (1) or fp64 (2) scalar");
    return -1;
  }
  const AdamScalars s{0.0, beta1, beta2, weight_decay, eps, amsgrad ? 1 : 0, maximize ? 1 : 0, mode, lr, lr_dtype};
  return fused_adam_launch(n_tensors, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, steps, numels,
                           dtype, s, grad_scale, found_inf, stream);
}

extern "C" int xdna_foreach_add_scalar_f32(int n_tensors, float* const* tensors, const int64_t* numels,
                                           float value, void* stream) {
  if (n_tensors < 0 || (n_tensors > 0 && (!tensors || !numels))) {
    set_error("xdna_foreach_add_scalar_f32: invalid arguments");
    return -1;
  }
  for (int done = 0; done < n_tensors;) {
    ForeachArgs a;
    const int n = std::min(kForeachMax, n_tensors - done);
    for (int i = 0; i < n; ++i) {
      a.t[i] = tensors[done + i];
      a.numel[i] = numels[done + i];
      if (a.numel[i] < 0 || (a.numel[i] > 0 && !a.t[i])) {
        set_error("xdna_foreach_add_scalar_f32: invalid tensor");
        return -1;
      }
    }
    if (!admit_launch("xdna_foreach_add_scalar_f32")) return -1;
    foreach_add_f32_kernel<<<dim3(unsigned(n)), 256, 0, as_stream(stream)>>>(a, value);
    if (check_launch("xdna_foreach_add_scalar_f32")) return -1;
    done += n;
  }
  return 0;
}
