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
    for (int64_t l = lane; l < L; l += 64) s += bf16_to_f32(xp[l]);
  }
  const float mean = wave_sum(s) / float(cnt);
  float q = 0.f;
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* xp = x + (n * C + c) * L;
    for (int64_t l = lane; l < L; l += 64) {
      const float d = bf16_to_f32(xp[l]) - mean;
      q += d * d;
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
    for (int64_t l = lane; l < L; l += 64)
      yp[l] = f32_to_bf16(act_forward(act, slope, fmaf(bf16_to_f32(xp[l]), scale, shift)));
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
  for (int64_t n = 0; n < N; ++n) {
    const int64_t o = (n * C + c) * L;
    for (int64_t l = lane; l < L; l += 64) {
      const float g = act ? act_backward(act, slope, bf16_to_f32(yact[o + l]), bf16_to_f32(dy[o + l]))
                          : bf16_to_f32(dy[o + l]);
      sdy += g;
      sdot += g * (bf16_to_f32(x[o + l]) - mean);
    }
  }
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
  for (int64_t n = 0; n < N; ++n) {
    const int64_t o = (n * C + c) * L;
    for (int64_t l = lane; l < L; l += 64) {
      const float xm = bf16_to_f32(x[o + l]) - mean;
      const float g = act ? act_backward(act, slope, bf16_to_f32(yact[o + l]), bf16_to_f32(dy[o + l]))
                          : bf16_to_f32(dy[o + l]);
      dx[o + l] = f32_to_bf16((g - gmean - xm * proj) * gscale);
    }
  }
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
  bn_fwd_kernel<<<dim3(unsigned(ceil_div(ch, kNormWaves))), 64 * kNormWaves, 0, as_stream(stream)>>>(
      x, weight, bias, param_dtype, y, save_mean, save_invstd, 1, ch, L, float(eps), C, act, slope);
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
  float* part = nullptr;
  if (params) {
    part = static_cast<float*>(xdna_hip_cache_alloc(size_t(2 * ch) * sizeof(float)));
    if (!part) return -1;
  }
  hipStream_t st = as_stream(stream);
  bn_bwd_kernel<<<dim3(unsigned(ceil_div(ch, kNormWaves))), 64 * kNormWaves, 0, st>>>(
      dy, x, weight, param_dtype, save_mean, save_invstd, dx, nullptr, nullptr, 1, ch, L, C, part,
      part ? part + ch : nullptr, y, act, slope);
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
