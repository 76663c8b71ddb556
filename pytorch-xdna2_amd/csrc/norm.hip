// Batch-norm statistics, normalisation and backward for bf16 activations, in the form
// instance_norm reaches them: PyTorch's instance_norm views [B, C, H, W] as
// [1, B*C, H, W] and calls native_batch_norm (training, no running statistics), so a
// "channel" here is one (image, channel) plane of H*W elements.  The instance-norm entry
// points take the C-element weight and bias directly (parameter index = channel % C) and
// sum the parameter gradients over the images themselves, which replaces PyTorch's
// repeat of the parameters and the reductions of its backward.  The reference serves
// these operators from PyTorch's CPU kernels through its zero-copy fallback
// (torch_xdna_device.cpp:5124-5260); on the GPU they decide the style step's time once
// the convolutions are fast (a wide, shallow reduction PyTorch-ROCm runs at ~35 us).
//
// Layout: x[n][c][l], n < N, c < C, l < L (contiguous).  One 64-lane wave per channel,
// four channels per workgroup; a channel's N*L elements are read from HBM once and
// re-read from cache by the later passes.  Statistics in fp32: mean, then the centred
// sum of squares (two passes), biased variance, invstd = 1 / sqrt(var + eps), as
// PyTorch's batch_norm_collect_statistics; y = (x - mean) * invstd * w + b rounded
// once to bf16.
#include "common.h"
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kNormWaves = 4;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// weight / bias element c of dtype wd (0 none -> default, 1 bf16, 2 fp32)
__device__ inline float param_at(const void* p, int wd, int64_t c, float dflt) {
  if (!p || wd == 0) return dflt;
  return wd == 1 ? bf16_to_f32(static_cast<const uint16_t*>(p)[c]) : static_cast<const float*>(p)[c];
}

__device__ inline void param_put(void* p, int wd, int64_t c, float v) {
  if (!p) return;
  if (wd == 1) static_cast<uint16_t*>(p)[c] = f32_to_bf16(v);
  else static_cast<float*>(p)[c] = v;
}

// The element loops below take each lane's elements l, l + 64, l + 128, ... of a plane in
// that order, as a plain strided loop would, four loads ahead (kU): the same fp32 sums, bit
// for bit, with the loads of four elements in flight instead of one.
constexpr int kU = 4;

// Parameters are indexed by channel % pC: pC = C for batch norm, the per-image channel
// count for instance norm (whose B*C "channels" share C weights; no repeated copies).
__global__ __launch_bounds__(64 * kNormWaves) void bn_fwd_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const void* __restrict__ b, int wd,
    uint16_t* __restrict__ y, float* __restrict__ save_mean, float* __restrict__ save_invstd,
    int64_t N, int64_t C, int64_t L, float eps, int64_t pC, int act, float slope) {
  const int lane = threadIdx.x & 63;
  const int64_t c = int64_t(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (c >= C) return;
  const int64_t cnt = N * L;
  float s = 0.f;
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* xp = x + (n * C + c) * L;
    for (int64_t l0 = lane; l0 < L; l0 += 64 * kU) {
      float v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = l0 + 64 * u < L ? bf16_to_f32(xp[l0 + 64 * u]) : 0.f;
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (l0 + 64 * u < L) s += v[u];
    }
  }
  const float mean = wave_sum(s) / float(cnt);
  float q = 0.f;
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* xp = x + (n * C + c) * L;
    for (int64_t l0 = lane; l0 < L; l0 += 64 * kU) {
      float v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = l0 + 64 * u < L ? bf16_to_f32(xp[l0 + 64 * u]) : 0.f;
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (l0 + 64 * u < L) {
          const float d = v[u] - mean;
          q += d * d;
        }
    }
  }
  const float var = wave_sum(q) / float(cnt);
  const float invstd = 1.0f / sqrtf(var + eps);
  if (lane == 0) {
    save_mean[c] = mean;
    save_invstd[c] = invstd;
  }
  const float scale = param_at(w, wd, c % pC, 1.f) * invstd;
  const float shift = param_at(b, wd, c % pC, 0.f) - mean * scale;
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* xp = x + (n * C + c) * L;
    uint16_t* yp = y + (n * C + c) * L;
    for (int64_t l0 = lane; l0 < L; l0 += 64 * kU) {
      float v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = l0 + 64 * u < L ? bf16_to_f32(xp[l0 + 64 * u]) : 0.f;
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (l0 + 64 * u < L) yp[l0 + 64 * u] = f32_to_bf16(act_forward(act, slope, fmaf(v[u], scale, shift)));
    }
  }
}

// One plane's backward (elements [o, o + L)): its sums of g and g * (x - mean), where g is
// dy through the activation (from its output yact), then, with dx set, dx from them.
__device__ inline void plane_bwd_sums(const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x,
                                      const uint16_t* __restrict__ yact, int act, float slope, int64_t o,
                                      int64_t L, float mean, int lane, float& sdy, float& sdot) {
  for (int64_t l0 = lane; l0 < L; l0 += 64 * kU) {
    float g[kU], xv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t l = l0 + 64 * u;
      const bool ok = l < L;
      const float d = ok ? bf16_to_f32(dy[o + l]) : 0.f;
      g[u] = ok && act ? act_backward(act, slope, bf16_to_f32(yact[o + l]), d) : d;
      xv[u] = ok ? bf16_to_f32(x[o + l]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (l0 + 64 * u < L) {
        sdy += g[u];
        sdot += g[u] * (xv[u] - mean);
      }
  }
}

__device__ inline void plane_bwd_dx(const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x,
                                    const uint16_t* __restrict__ yact, int act, float slope, int64_t o, int64_t L,
                                    float mean, float gmean, float proj, float gscale, int lane,
                                    uint16_t* __restrict__ dx) {
  for (int64_t l0 = lane; l0 < L; l0 += 64 * kU) {
    float g[kU], xm[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t l = l0 + 64 * u;
      const bool ok = l < L;
      const float d = ok ? bf16_to_f32(dy[o + l]) : 0.f;
      g[u] = ok && act ? act_backward(act, slope, bf16_to_f32(yact[o + l]), d) : d;
      xm[u] = (ok ? bf16_to_f32(x[o + l]) : 0.f) - mean;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (l0 + 64 * u < L) dx[o + l0 + 64 * u] = f32_to_bf16((g[u] - gmean - xm[u] * proj) * gscale);
  }
}

// dx = (dy - mean(dy) - (x - mean) * invstd^2 * mean(dy * (x - mean))) * invstd * w
// dw = invstd * sum(dy * (x - mean)),  db = sum(dy)   (PyTorch's batch_norm_backward)
// With pw / pb set (instance norm), each channel's dw / db terms go there in fp32 for a
// fixed-order sum over the images (norm_param_reduce_kernel) instead of to dw / db.
__global__ __launch_bounds__(64 * kNormWaves) void bn_bwd_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x, const void* __restrict__ w, int wd,
    const float* __restrict__ mean_in, const float* __restrict__ invstd_in, uint16_t* __restrict__ dx,
    void* __restrict__ dw, void* __restrict__ db, int64_t N, int64_t C, int64_t L, int64_t pC,
    float* __restrict__ pw, float* __restrict__ pb, const uint16_t* __restrict__ yact, int act, float slope) {
  const int lane = threadIdx.x & 63;
  const int64_t c = int64_t(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (c >= C) return;
  const float mean = mean_in[c], invstd = invstd_in[c];
  float sdy = 0.f, sdot = 0.f;
  for (int64_t n = 0; n < N; ++n) plane_bwd_sums(dy, x, yact, act, slope, (n * C + c) * L, L, mean, lane, sdy, sdot);
  sdy = wave_sum(sdy);
  sdot = wave_sum(sdot);
  if (lane == 0) {
    if (pw) {
      pw[c] = sdot * invstd;
      pb[c] = sdy;
    } else {
      param_put(dw, wd, c, sdot * invstd);
      param_put(db, wd, c, sdy);
    }
  }
  if (!dx) return;
  const float inv_cnt = 1.0f / float(N * L);
  const float gmean = sdy * inv_cnt;
  const float proj = sdot * inv_cnt * invstd * invstd;
  const float gscale = invstd * param_at(w, wd, c % pC, 1.f);
  for (int64_t n = 0; n < N; ++n)
    plane_bwd_dx(dy, x, yact, act, slope, (n * C + c) * L, L, mean, gmean, proj, gscale, lane, dx);
}

// Instance norm on planes of up to 64 NV elements held in registers (lane l: elements
// l + 64 i, i < NV), so each plane is read once, all its loads issued together.  The sums
// run over each lane's elements in the loops' order above and then the same lane sum, so
// the results are those kernels', bit for bit.
//
// Forward: a wave per plane, four planes per workgroup (bn_fwd_kernel with N = 1).
template <int NV>
__global__ __launch_bounds__(64 * kNormWaves) void in_fwd_regs_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const void* __restrict__ b, int wd,
    uint16_t* __restrict__ y, float* __restrict__ save_mean, float* __restrict__ save_invstd, int64_t P,
    int L, float eps, int64_t pC, int act, float slope) {
  const int lane = threadIdx.x & 63;
  const int64_t c = int64_t(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (c >= P) return;
  const uint16_t* xp = x + c * L;
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = lane + 64 * i < L ? bf16_to_f32(xp[lane + 64 * i]) : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < L) s += v[i];
  const float mean = wave_sum(s) / float(L);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < L) {
      const float d = v[i] - mean;
      q += d * d;
    }
  const float var = wave_sum(q) / float(L);
  const float invstd = 1.0f / sqrtf(var + eps);
  if (lane == 0) {
    save_mean[c] = mean;
    save_invstd[c] = invstd;
  }
  const float scale = param_at(w, wd, c % pC, 1.f) * invstd;
  const float shift = param_at(b, wd, c % pC, 0.f) - mean * scale;
  uint16_t* yp = y + c * L;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < L) yp[lane + 64 * i] = f32_to_bf16(act_forward(act, slope, fmaf(v[i], scale, shift)));
}

// Backward: a wave per plane, four planes per workgroup (bn_bwd_kernel with N = 1), the
// plane's dy, x (and the activation's output) in registers; each plane's dw / db terms go
// to pw / pb for norm_param_reduce_kernel's fixed-order sum over the images (pw null: not
// written).
template <int NV>
__global__ __launch_bounds__(64 * kNormWaves) void in_bwd_regs_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x, const void* __restrict__ w, int wd,
    const float* __restrict__ mean_in, const float* __restrict__ invstd_in, uint16_t* __restrict__ dx, int64_t P,
    int L, int64_t pC, float* __restrict__ pw, float* __restrict__ pb, const uint16_t* __restrict__ yact, int act,
    float slope) {
  const int lane = threadIdx.x & 63;
  const int64_t c = int64_t(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (c >= P) return;
  const int64_t o = c * L;
  float g[NV], xv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int l = lane + 64 * i;
    const bool ok = l < L;
    const float d = ok ? bf16_to_f32(dy[o + l]) : 0.f;
    g[i] = ok && act ? act_backward(act, slope, bf16_to_f32(yact[o + l]), d) : d;
    xv[i] = ok ? bf16_to_f32(x[o + l]) : 0.f;
  }
  const float mean = mean_in[c], invstd = invstd_in[c];
  float sdy = 0.f, sdot = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < L) {
      sdy += g[i];
      sdot += g[i] * (xv[i] - mean);
    }
  sdy = wave_sum(sdy);
  sdot = wave_sum(sdot);
  if (pw && lane == 0) {
    pw[c] = sdot * invstd;
    pb[c] = sdy;
  }
  if (!dx) return;
  const float inv_cnt = 1.0f / float(L);
  const float gmean = sdy * inv_cnt;
  const float proj = sdot * inv_cnt * invstd * invstd;
  const float gscale = invstd * param_at(w, wd, c % pC, 1.f);
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < L) dx[o + lane + 64 * i] = f32_to_bf16((g[i] - gmean - (xv[i] - mean) * proj) * gscale);
}

// per-lane register count of a plane of L elements (power of two), 0 past 2048 elements
inline int in_regs_nv(int64_t L) {
  for (int nv = 1; nv <= 32; nv *= 2)
    if (L <= 64 * nv) return nv;
  return 0;
}

// dw[c] = sum_b pw[b*C + c], db likewise, stored in dtype wd: one wave per parameter,
// lane l sums images l, l+64, ... and the wave adds the lanes in a fixed order (the
// result does not depend on timing).
__global__ __launch_bounds__(64 * kNormWaves) void norm_param_reduce_kernel(const float* __restrict__ pw,
                                                                           const float* __restrict__ pb,
                                                                           void* dw, void* db, int wd, int64_t B,
                                                                           int64_t C) {
  const int64_t c = int64_t(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= C) return;
  float sw = 0.f, sb = 0.f;
  for (int64_t b = lane; b < B; b += 64) {
    sw += pw[b * C + c];
    sb += pb[b * C + c];
  }
  sw = wave_sum(sw);
  sb = wave_sum(sb);
  if (lane == 0) {
    param_put(dw, wd, c, sw);
    param_put(db, wd, c, sb);
  }
}

bool norm_shape_ok(const char* what, int64_t N, int64_t C, int64_t L, int wd) {
  if (N < 0 || C < 0 || L < 0 || wd < 0 || wd > 2) {
    set_error(std::string(what) + ": invalid arguments");
    return false;
  }
  return true;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_batch_norm_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                             uint16_t* y, float* save_mean, float* save_invstd, int64_t N, int64_t C,
                             int64_t L, double eps, void* stream) {
  if (!norm_shape_ok("xdna_batch_norm_fwd_bf16", N, C, L, param_dtype)) return -1;
  if (C == 0) return 0;
  if (N * L == 0) {
    set_error("xdna_batch_norm_fwd_bf16: empty reduction");
    return -1;
  }
  if (!admit_launch("batch_norm fwd")) return -1;
  bn_fwd_kernel<<<dim3(unsigned(ceil_div(C, kNormWaves))), 64 * kNormWaves, 0, as_stream(stream)>>>(
      x, weight, bias, param_dtype, y, save_mean, save_invstd, N, C, L, float(eps), C, 0, 0.0f);
  return check_launch("batch_norm fwd");
}

int xdna_batch_norm_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight, int param_dtype,
                             const float* save_mean, const float* save_invstd, uint16_t* dx,
                             void* dweight, void* dbias, int64_t N, int64_t C, int64_t L, void* stream) {
  if (!norm_shape_ok("xdna_batch_norm_bwd_bf16", N, C, L, param_dtype)) return -1;
  if (C == 0) return 0;
  if ((dweight || dbias) && param_dtype == 0) {
    set_error("xdna_batch_norm_bwd_bf16: parameter gradients need param_dtype 1 or 2");
    return -1;
  }
  if (!admit_launch("batch_norm bwd")) return -1;
  bn_bwd_kernel<<<dim3(unsigned(ceil_div(C, kNormWaves))), 64 * kNormWaves, 0, as_stream(stream)>>>(
      dy, x, weight, param_dtype, save_mean, save_invstd, dx, dweight, dbias, N, C, L, C, nullptr, nullptr, nullptr,
      0, 0.0f);
  return check_launch("batch_norm bwd");
}

int xdna_instance_norm_act_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                    uint16_t* y, float* save_mean, float* save_invstd, int64_t B, int64_t C,
                                    int64_t L, double eps, int act, float slope, void* stream) {
  if (!norm_shape_ok("xdna_instance_norm_fwd_bf16", B, C, L, param_dtype)) return -1;
  if (act < 0 || act > 2) {
    set_error("xdna_instance_norm_fwd_bf16: activation must be 0, 1 or 2");
    return -1;
  }
  if (B == 0 || C == 0) return 0;
  if (L == 0) {
    set_error("xdna_instance_norm_fwd_bf16: empty reduction");
    return -1;
  }
  const int64_t ch = B * C;
  if (ceil_div(ch, kNormWaves) > 0x7fffffff) {
    set_error("xdna_instance_norm_fwd_bf16: too many planes");
    return -1;
  }
  if (!admit_launch("instance_norm fwd")) return -1;
  const dim3 grid(unsigned(ceil_div(ch, kNormWaves)));
  hipStream_t st = as_stream(stream);
  switch (in_regs_nv(L)) {
#define XDNA_INF(nv_)                                                                                  \
  case nv_:                                                                                          \
    in_fwd_regs_kernel<nv_><<<grid, 64 * kNormWaves, 0, st>>>(x, weight, bias, param_dtype, y, save_mean, \
                                                               save_invstd, ch, int(L), float(eps), C, act, slope); \
    break;
    XDNA_INF(1) XDNA_INF(2) XDNA_INF(4) XDNA_INF(8) XDNA_INF(16) XDNA_INF(32)
#undef XDNA_INF
    default:
      bn_fwd_kernel<<<grid, 64 * kNormWaves, 0, st>>>(x, weight, bias, param_dtype, y, save_mean, save_invstd, 1,
                                                      ch, L, float(eps), C, act, slope);
  }
  return check_launch("instance_norm fwd");
}

int xdna_instance_norm_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                uint16_t* y, float* save_mean, float* save_invstd, int64_t B, int64_t C,
                                int64_t L, double eps, void* stream) {
  return xdna_instance_norm_act_fwd_bf16(x, weight, bias, param_dtype, y, save_mean, save_invstd, B, C, L, eps, 0,
                                         0.0f, stream);
}

int xdna_instance_norm_act_bwd_bf16(const uint16_t* dy, const uint16_t* x, const uint16_t* y, const void* weight,
                                    int param_dtype, const float* save_mean, const float* save_invstd,
                                    uint16_t* dx, void* dweight, void* dbias, int64_t B, int64_t C, int64_t L,
                                    int act, float slope, void* stream) {
  if (!norm_shape_ok("xdna_instance_norm_bwd_bf16", B, C, L, param_dtype)) return -1;
  if (act < 0 || act > 2 || (act && !y)) {
    set_error("xdna_instance_norm_bwd_bf16: activation must be 0, 1 or 2, with its output");
    return -1;
  }
  if (B == 0 || C == 0) return 0;
  const bool params = dweight || dbias;
  if (params && (param_dtype == 0 || !dweight || !dbias)) {
    set_error("xdna_instance_norm_bwd_bf16: parameter gradients need both outputs and param_dtype 1 or 2");
    return -1;
  }
  const int64_t ch = B * C;
  if (ceil_div(ch, kNormWaves) > 0x7fffffff) {
    set_error("xdna_instance_norm_bwd_bf16: too many planes");
    return -1;
  }
  if (!admit_launch("instance_norm bwd")) return -1;
  hipStream_t st = as_stream(stream);
  float* part = nullptr;
  if (params) {
    part = static_cast<float*>(xdna_hip_cache_alloc(size_t(2 * ch) * sizeof(float)));
    if (!part) return -1;
  }
  const dim3 grid(unsigned(ceil_div(ch, kNormWaves)));
  float* const pw = part, *const pb = part ? part + ch : nullptr;
  switch (in_regs_nv(L)) {
#define XDNA_INB(nv_)                                                                                            \
  case nv_:                                                                                                    \
    in_bwd_regs_kernel<nv_><<<grid, 64 * kNormWaves, 0, st>>>(dy, x, weight, param_dtype, save_mean, save_invstd, \
                                                               dx, ch, int(L), C, pw, pb, y, act, slope);         \
    break;
    XDNA_INB(1) XDNA_INB(2) XDNA_INB(4) XDNA_INB(8) XDNA_INB(16) XDNA_INB(32)
#undef XDNA_INB
    default:
      bn_bwd_kernel<<<grid, 64 * kNormWaves, 0, st>>>(dy, x, weight, param_dtype, save_mean, save_invstd, dx,
                                                      nullptr, nullptr, 1, ch, L, C, pw, pb, y, act, slope);
  }
  if (params) {
    norm_param_reduce_kernel<<<dim3(unsigned(ceil_div(C, kNormWaves))), 64 * kNormWaves, 0, st>>>(
        part, part + ch, dweight, dbias, param_dtype, B, C);
    // stream-ordered reuse: the next user of the block runs after the reduce
    xdna_hip_cache_free(part);
  }
  return check_launch("instance_norm bwd");
}

int xdna_instance_norm_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight, int param_dtype,
                                const float* save_mean, const float* save_invstd, uint16_t* dx, void* dweight,
                                void* dbias, int64_t B, int64_t C, int64_t L, void* stream) {
  return xdna_instance_norm_act_bwd_bf16(dy, x, nullptr, weight, param_dtype, save_mean, save_invstd, dx, dweight,
                                         dbias, B, C, L, 0, 0.0f, stream);
}

}  // extern "C"
