// Batch norm of convolutional networks in training mode: per-channel statistics over
// N * L elements (L = H * W), running-statistics update, normalisation, and the
// backward.  The reference serves native_batch_norm / native_batch_norm_backward from
// PyTorch's CPU kernels through its zero-copy fallback (torch_xdna_device.cpp:5124-5260);
// ResNet-style training reaches them with up to 128 * 64 * 64 =
// 524288 elements per channel, far past what one wave per channel (norm.hip) can take.
//
// Layout x[n][c][l] bf16, contiguous.  A channel's elements are cut into S ranges of whole
// images; workgroup (c, s) reduces one range.  Forward: pass 1 sums d = x - K and d^2 per
// range (K = the channel's first element, a shift that keeps the one-pass variance from
// cancelling), pass 2 combines the S partials of its channel in a fixed order (every
// workgroup of the channel computes the same totals), normalises its range, and
// workgroup (c, 0) writes save_mean / save_invstd and the running statistics.  Backward:
// pass 1 sums dy and dy * (x - mean) per range, pass 2 combines them and writes dx, and
// workgroup (c, 0) the parameter gradients.  All sums in fp32; outputs rounded once.
// Statistics as PyTorch's batch norm: biased variance for invstd = 1 / sqrt(var + eps),
// unbiased variance for the running update, running = (1 - momentum) * running +
// momentum * batch.
#include "common.h"
#include "../../include/xdna_hip.h"

#include <algorithm>

namespace xdna {
namespace {

constexpr int kBnThreads = 256;

__device__ inline float bn_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the workgroup (4 waves) in a fixed order; every thread gets the result.
__device__ inline float bn_block_sum(float v, float* lds) {
  v = bn_wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[w] = v;
  __syncthreads();
  return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

__device__ inline float bn_load_param(const void* p, int dt, int64_t c, float dflt) {
  if (!p || dt == 0) return dflt;
  return dt == 1 ? bf16_to_f32(static_cast<const uint16_t*>(p)[c]) : static_cast<const float*>(p)[c];
}

__device__ inline void bn_store_param(void* p, int dt, int64_t c, float v) {
  if (!p || dt == 0) return;
  if (dt == 1) static_cast<uint16_t*>(p)[c] = f32_to_bf16(v);
  else static_cast<float*>(p)[c] = v;
}

struct BnGeom {
  int64_t N, C, L;
  int S;          // ranges per channel
  int64_t nper;   // images per range
  int vec;        // 1: L % 8 == 0 and 16-byte aligned tensors (8-element vectors)
};

// Elements [n0 * L, n1 * L) of channel c, visited as (image, offset) pairs; f(xv[8], base)
// for 8-element vectors when g.vec, else f on single elements.
template <class F8, class F1>
__device__ inline void bn_visit(const BnGeom& g, int64_t c, F8 f8, F1 f1) {
  const int64_t n0 = int64_t(blockIdx.y) * g.nper, n1 = min(g.N, n0 + g.nper);
  if (g.vec) {
    const int64_t nv = g.L / 8;
    const int64_t total = (n1 - n0) * nv;
    for (int64_t i = threadIdx.x; i < total; i += kBnThreads) {
      const int64_t n = n0 + i / nv, v = i - (i / nv) * nv;
      f8((n * g.C + c) * g.L + v * 8);
    }
  } else {
    const int64_t total = (n1 - n0) * g.L;
    for (int64_t i = threadIdx.x; i < total; i += kBnThreads) {
      const int64_t n = n0 + i / g.L, l = i - (i / g.L) * g.L;
      f1((n * g.C + c) * g.L + l);
    }
  }
}

__device__ inline void unpack8(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
  }
}

// part[(c * S + s) * 2 + {0, 1}] = sum of d, sum of d^2 over range s, d = x - x[0][c][0]
__global__ __launch_bounds__(kBnThreads) void bn_stats_kernel(const uint16_t* __restrict__ x, BnGeom g,
                                                              float* __restrict__ part) {
  __shared__ float red[4];
  const int64_t c = blockIdx.x;
  const float k = bf16_to_f32(x[c * g.L]);
  float s1 = 0.f, s2 = 0.f;
  bn_visit(
      g, c,
      [&](int64_t o) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(x + o), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = f[e] - k;
          s1 += d;
          s2 = fmaf(d, d, s2);
        }
      },
      [&](int64_t o) {
        const float d = bf16_to_f32(x[o]) - k;
        s1 += d;
        s2 = fmaf(d, d, s2);
      });
  s1 = bn_block_sum(s1, red);
  s2 = bn_block_sum(s2, red);
  if (threadIdx.x == 0) {
    part[(c * g.S + blockIdx.y) * 2] = s1;
    part[(c * g.S + blockIdx.y) * 2 + 1] = s2;
  }
}

struct BnFwdArgs {
  const uint16_t* x;
  const void* w;
  const void* b;
  int wd;
  void* rmean;
  void* rvar;
  int rd;
  float momentum, eps;
  uint16_t* y;
  float* save_mean;
  float* save_invstd;
  const float* part;
  int act;      // activation applied before rounding (act_forward)
  float slope;
};

__global__ __launch_bounds__(kBnThreads) void bn_norm_kernel(BnFwdArgs a, BnGeom g) {
  __shared__ float tot[2];
  const int64_t c = blockIdx.x;
  if (threadIdx.x == 0) {
    float s1 = 0.f, s2 = 0.f;
    for (int s = 0; s < g.S; ++s) {
      s1 += a.part[(c * g.S + s) * 2];
      s2 += a.part[(c * g.S + s) * 2 + 1];
    }
    tot[0] = s1;
    tot[1] = s2;
  }
  __syncthreads();
  const float n = float(g.N * g.L);
  const float k = bf16_to_f32(a.x[c * g.L]);
  const float dmean = tot[0] / n;
  const float var = fmaxf(tot[1] / n - dmean * dmean, 0.f);  // biased
  const float mean = k + dmean;
  const float invstd = 1.0f / sqrtf(var + a.eps);
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    a.save_mean[c] = mean;
    a.save_invstd[c] = invstd;
    if (a.rmean) {
      const float rm = bn_load_param(a.rmean, a.rd, c, 0.f);
      bn_store_param(a.rmean, a.rd, c, a.momentum * mean + (1.0f - a.momentum) * rm);
    }
    if (a.rvar) {
      const float cnt = float(g.N * g.L);
      const float unbiased = cnt > 1.f ? var * cnt / (cnt - 1.f) : var;
      const float rv = bn_load_param(a.rvar, a.rd, c, 1.f);
      bn_store_param(a.rvar, a.rd, c, a.momentum * unbiased + (1.0f - a.momentum) * rv);
    }
  }
  const float scale = bn_load_param(a.w, a.wd, c, 1.f) * invstd;
  const float shift = bn_load_param(a.b, a.wd, c, 0.f) - mean * scale;
  bn_visit(
      g, c,
      [&](int64_t o) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(a.x + o), f);
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w4[e] = uint32_t(f32_to_bf16(act_forward(a.act, a.slope, fmaf(f[2 * e], scale, shift)))) |
                  (uint32_t(f32_to_bf16(act_forward(a.act, a.slope, fmaf(f[2 * e + 1], scale, shift)))) << 16);
        *reinterpret_cast<uint4*>(a.y + o) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      },
      [&](int64_t o) { a.y[o] = f32_to_bf16(act_forward(a.act, a.slope, fmaf(bf16_to_f32(a.x[o]), scale, shift))); });
}

// part[(c * S + s) * 2 + {0, 1}] = sum of dy, sum of dy * (x - mean) over range s
// (with act, dy is first taken through the activation's gradient from its output y)
__global__ __launch_bounds__(kBnThreads) void bn_bwd_stats_kernel(const uint16_t* __restrict__ dy,
                                                                  const uint16_t* __restrict__ x,
                                                                  const float* __restrict__ mean_in, BnGeom g,
                                                                  float* __restrict__ part,
                                                                  const uint16_t* __restrict__ y, int act,
                                                                  float slope) {
  __shared__ float red[4];
  const int64_t c = blockIdx.x;
  const float mean = mean_in[c];
  float s1 = 0.f, s2 = 0.f;
  bn_visit(
      g, c,
      [&](int64_t o) {
        float fd[8], fx[8];
        unpack8(*reinterpret_cast<const uint4*>(dy + o), fd);
        unpack8(*reinterpret_cast<const uint4*>(x + o), fx);
        if (act) {
          float fy[8];
          unpack8(*reinterpret_cast<const uint4*>(y + o), fy);
#pragma unroll
          for (int e = 0; e < 8; ++e) fd[e] = act_backward(act, slope, fy[e], fd[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s1 += fd[e];
          s2 = fmaf(fd[e], fx[e] - mean, s2);
        }
      },
      [&](int64_t o) {
        float d = bf16_to_f32(dy[o]);
        if (act) d = act_backward(act, slope, bf16_to_f32(y[o]), d);
        s1 += d;
        s2 = fmaf(d, bf16_to_f32(x[o]) - mean, s2);
      });
  s1 = bn_block_sum(s1, red);
  s2 = bn_block_sum(s2, red);
  if (threadIdx.x == 0) {
    part[(c * g.S + blockIdx.y) * 2] = s1;
    part[(c * g.S + blockIdx.y) * 2 + 1] = s2;
  }
}

struct BnBwdArgs {
  const uint16_t* dy;
  const uint16_t* x;
  const void* w;
  int wd;
  const float* mean;
  const float* invstd;
  uint16_t* dx;
  void* dw;
  void* db;
  const float* part;
  const uint16_t* y;  // the activation's output (act != 0)
  int act;
  float slope;
};

// dx = (dy - sum(dy)/n - (x - mean) * invstd^2 * sum(dy (x - mean))/n) * invstd * w,
// dw = invstd * sum(dy (x - mean)), db = sum(dy)   (PyTorch's batch_norm_backward)
__global__ __launch_bounds__(kBnThreads) void bn_bwd_kernel2(BnBwdArgs a, BnGeom g) {
  __shared__ float tot[2];
  const int64_t c = blockIdx.x;
  if (threadIdx.x == 0) {
    float s1 = 0.f, s2 = 0.f;
    for (int s = 0; s < g.S; ++s) {
      s1 += a.part[(c * g.S + s) * 2];
      s2 += a.part[(c * g.S + s) * 2 + 1];
    }
    tot[0] = s1;
    tot[1] = s2;
  }
  __syncthreads();
  const float sdy = tot[0], sdot = tot[1];
  const float mean = a.mean[c], invstd = a.invstd[c];
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    bn_store_param(a.dw, a.wd, c, sdot * invstd);
    bn_store_param(a.db, a.wd, c, sdy);
  }
  if (!a.dx) return;
  const float inv_cnt = 1.0f / float(g.N * g.L);
  const float gmean = sdy * inv_cnt;
  const float proj = sdot * inv_cnt * invstd * invstd;
  const float gscale = invstd * bn_load_param(a.w, a.wd, c, 1.f);
  bn_visit(
      g, c,
      [&](int64_t o) {
        float fd[8], fx[8];
        unpack8(*reinterpret_cast<const uint4*>(a.dy + o), fd);
        unpack8(*reinterpret_cast<const uint4*>(a.x + o), fx);
        if (a.act) {
          float fy[8];
          unpack8(*reinterpret_cast<const uint4*>(a.y + o), fy);
#pragma unroll
          for (int e = 0; e < 8; ++e) fd[e] = act_backward(a.act, a.slope, fy[e], fd[e]);
        }
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v0 = (fd[2 * e] - gmean - (fx[2 * e] - mean) * proj) * gscale;
          const float v1 = (fd[2 * e + 1] - gmean - (fx[2 * e + 1] - mean) * proj) * gscale;
          w4[e] = uint32_t(f32_to_bf16(v0)) | (uint32_t(f32_to_bf16(v1)) << 16);
        }
        *reinterpret_cast<uint4*>(a.dx + o) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      },
      [&](int64_t o) {
        float d = bf16_to_f32(a.dy[o]);
        if (a.act) d = act_backward(a.act, a.slope, bf16_to_f32(a.y[o]), d);
        const float v = (d - gmean - (bf16_to_f32(a.x[o]) - mean) * proj) * gscale;
        a.dx[o] = f32_to_bf16(v);
      });
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Ranges per channel: enough workgroups to cover the CUs several times, each range at
// least 4096 elements; whole images per range.
BnGeom bn_geom(int64_t N, int64_t C, int64_t L, bool vec) {
  BnGeom g;
  g.N = N;
  g.C = C;
  g.L = L;
  const int64_t want = std::max<int64_t>(1, (2048 + C - 1) / C);
  const int64_t by_size = std::max<int64_t>(1, N * L / 4096);
  g.S = int(std::min<int64_t>({N, want, by_size, 65535}));
  g.nper = (N + g.S - 1) / g.S;
  g.S = int((N + g.nper - 1) / g.nper);
  g.vec = vec && (L % 8) == 0 ? 1 : 0;
  return g;
}

bool bn_args_ok(const char* what, int64_t N, int64_t C, int64_t L, int wd) {
  if (N < 1 || C < 1 || L < 1 || C > 0x7fffffff || wd < 0 || wd > 2) {
    set_error(std::string(what) + ": invalid arguments");
    return false;
  }
  return true;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" int xdna_batch_norm_train_act_fwd_bf16(const uint16_t* x, const void* weight, const void* bias,
                                                  int param_dtype, void* running_mean, void* running_var,
                                                  int stat_dtype, double momentum, double eps, uint16_t* y,
                                                  float* save_mean, float* save_invstd, int64_t N, int64_t C,
                                                  int64_t L, int act, float slope, void* stream) {
  if (!bn_args_ok("xdna_batch_norm_train_fwd_bf16", N, C, L, param_dtype)) return -1;
  if (!x || !y || !save_mean || !save_invstd || stat_dtype < 0 || stat_dtype > 2 ||
      ((running_mean || running_var) && stat_dtype == 0) || act < 0 || act > 2) {
    set_error("xdna_batch_norm_train_fwd_bf16: invalid arguments");
    return -1;
  }
  const BnGeom g = bn_geom(N, C, L, aligned16(x) && aligned16(y));
  float* part = static_cast<float*>(xdna_hip_cache_alloc(size_t(C) * g.S * 2 * sizeof(float)));
  if (!part) return -1;
  if (!admit_launch("xdna_batch_norm_train_fwd_bf16")) {
    xdna_hip_cache_free(part);
    return -1;
  }
  hipStream_t st = as_stream(stream);
  const dim3 grid(unsigned(C), unsigned(g.S));
  bn_stats_kernel<<<grid, kBnThreads, 0, st>>>(x, g, part);
  BnFwdArgs a{x,     weight,    bias,        param_dtype, running_mean, running_var, stat_dtype,
              float(momentum), float(eps), y, save_mean, save_invstd, part, act, slope};
  bn_norm_kernel<<<grid, kBnThreads, 0, st>>>(a, g);
  xdna_hip_cache_free(part);  // stream-ordered reuse
  return check_launch("xdna_batch_norm_train_fwd_bf16");
}

extern "C" int xdna_batch_norm_train_fwd_bf16(const uint16_t* x, const void* weight, const void* bias,
                                              int param_dtype, void* running_mean, void* running_var,
                                              int stat_dtype, double momentum, double eps, uint16_t* y,
                                              float* save_mean, float* save_invstd, int64_t N, int64_t C,
                                              int64_t L, void* stream) {
  return xdna_batch_norm_train_act_fwd_bf16(x, weight, bias, param_dtype, running_mean, running_var, stat_dtype,
                                            momentum, eps, y, save_mean, save_invstd, N, C, L, 0, 0.0f, stream);
}

extern "C" int xdna_batch_norm_train_act_bwd_bf16(const uint16_t* dy, const uint16_t* x, const uint16_t* y,
                                                  const void* weight, int param_dtype, const float* save_mean,
                                                  const float* save_invstd, uint16_t* dx, void* dweight,
                                                  void* dbias, int64_t N, int64_t C, int64_t L, int act, float slope,
                                                  void* stream) {
  if (!bn_args_ok("xdna_batch_norm_train_bwd_bf16", N, C, L, param_dtype)) return -1;
  if (!dy || !x || !save_mean || !save_invstd || ((dweight || dbias) && param_dtype == 0) || act < 0 || act > 2 ||
      (act && !y)) {
    set_error("xdna_batch_norm_train_bwd_bf16: invalid arguments");
    return -1;
  }
  const BnGeom g =
      bn_geom(N, C, L, aligned16(dy) && aligned16(x) && (!dx || aligned16(dx)) && (!act || aligned16(y)));
  float* part = static_cast<float*>(xdna_hip_cache_alloc(size_t(C) * g.S * 2 * sizeof(float)));
  if (!part) return -1;
  if (!admit_launch("xdna_batch_norm_train_bwd_bf16")) {
    xdna_hip_cache_free(part);
    return -1;
  }
  hipStream_t st = as_stream(stream);
  const dim3 grid(unsigned(C), unsigned(g.S));
  bn_bwd_stats_kernel<<<grid, kBnThreads, 0, st>>>(dy, x, save_mean, g, part, y, act, slope);
  BnBwdArgs a{dy, x, weight, param_dtype, save_mean, save_invstd, dx, dweight, dbias, part, y, act, slope};
  bn_bwd_kernel2<<<grid, kBnThreads, 0, st>>>(a, g);
  xdna_hip_cache_free(part);
  return check_launch("xdna_batch_norm_train_bwd_bf16");
}

extern "C" int xdna_batch_norm_train_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight,
                                              int param_dtype, const float* save_mean, const float* save_invstd,
                                              uint16_t* dx, void* dweight, void* dbias, int64_t N, int64_t C,
                                              int64_t L, void* stream) {
  return xdna_batch_norm_train_act_bwd_bf16(dy, x, nullptr, weight, param_dtype, save_mean, save_invstd, dx,
                                            dweight, dbias, N, C, L, 0, 0.0f, stream);
}
