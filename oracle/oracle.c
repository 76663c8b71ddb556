/*
 * CPU oracle for the MI355X hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or the timed CPU baseline), never as the product
 * path.  Plain C restatements of the reference's algorithms, written for clarity:
 * straight loop nests, double accumulation for the convolutions.
 *
 * Each function names the reference code it restates.  How each is pinned (golden
 * vectors, the reference's own build in oracle/_ref, closed forms) is listed in the
 * test files under tests/ that exercise it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GROUP_OUT_ROWS 2048
#define GROUP_ROWS 2126
#define KSTEP 64
#define RAW_N 128

static float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f2bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* Strip geometry: conv3x3w_host.py:96-103 (strip_geometry), torch_xdna_device.cpp:1927-1937. */
void oracle_strip_geometry(int W, int* S, int* So) {
  if (W <= 36) {
    *S = 1;
    *So = W;
  } else {
    *S = (W + 33) / 34;
    *So = (W + *S - 1) / *S;
  }
}

/*
 * Packed input, groups [g0, g0+ng), written into dst = [ng][chunks][2126][64].
 * Layout: conv3x3w_host.py:32-46 (pack_input: padded-grid rows, zero border, per-group
 * windows of 2126 rows starting every 2048) and :106-131 (strip_batch: virtual image
 * b*S+s holds source columns [s*So-1, s*So+So+1), halo columns zeroed for halo_zero).
 * Write contract: conv_pack.cpp:625-631 (only real pixels and channels are written;
 * the caller zero-fills dst).
 */
void oracle_pack_strips_range(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                              int S, int So, int halo_zero, int chunks, int g0, int ng) {
  const int Wg = S == 1 ? W : So + 2;
  const int wp = Wg + 2;
  for (int vb = 0; vb < B * S; ++vb) {
    const int b = vb / S, s = vb % S;
    for (int y = 0; y < H; ++y) {
      for (int j = 0; j < Wg; ++j) {
        const int x = (S == 1 ? 0 : s * So - 1) + j;
        if (x < 0 || x >= W) continue;
        const int64_t p = ((int64_t)vb * (H + 2) + y + 1) * wp + j + 1;
        const int64_t g = p / GROUP_OUT_ROWS;
        const int64_t r = p % GROUP_OUT_ROWS;
        const int zero = halo_zero && S > 1 && (j == 0 || j == Wg - 1);
        for (int ch = 0; ch < C && ch < chunks * KSTEP; ++ch) {
          const int chunk = ch / KSTEP, c = ch % KSTEP;
          const uint16_t v = zero ? 0 : src[(((int64_t)b * C + ch) * H + y) * W + x];
          if (g >= g0 && g < (int64_t)g0 + ng)
            dst[((((g - g0) * chunks + chunk) * GROUP_ROWS) + r) * KSTEP + c] = v;
          if (g - 1 >= g0 && g - 1 < (int64_t)g0 + ng && r + GROUP_OUT_ROWS < GROUP_ROWS)
            dst[((((g - 1 - g0) * chunks + chunk) * GROUP_ROWS) + GROUP_OUT_ROWS + r) * KSTEP + c] = v;
        }
      }
    }
  }
}

/*
 * Raw output rows [p0, p1) (c points at row p0, 128 channels per row) -> channel slice
 * [c_start, c_start+cout_valid) of NCHW [B][C_total][H][W].
 * Layout: conv3x3w_host.py:85-90 (unpack_output: pixel (y, x) of image b at row
 * (b*(H+2)+y)*wp + x) and :134-140 (unpack_output_strips: strip s output column t is
 * virtual-image data column 1+t, image column s*So+t).
 */
void oracle_unpack_strips_range(const uint16_t* c, uint16_t* dst, int B, int H, int W, int S,
                                int So, int cout_valid, int C_total, int c_start, int64_t p0,
                                int64_t p1) {
  const int Wg = S == 1 ? W : So + 2;
  const int wp = Wg + 2;
  for (int vb = 0; vb < B * S; ++vb) {
    const int b = vb / S, s = vb % S;
    const int first = S == 1 ? 0 : 1;
    int cols = S == 1 ? W : W - s * So;
    if (S > 1 && cols > So) cols = So;
    for (int y = 0; y < H; ++y) {
      for (int t = 0; t < cols; ++t) {
        const int64_t p = ((int64_t)vb * (H + 2) + y) * wp + first + t;
        if (p < p0 || p >= p1) continue;
        const int x = (S == 1 ? 0 : s * So) + t;
        for (int n = 0; n < cout_valid; ++n)
          dst[(((int64_t)b * C_total + c_start + n) * H + y) * W + x] = c[(p - p0) * RAW_N + n];
      }
    }
  }
}

/*
 * 3x3 / stride 1 / pad 1 convolution, double accumulation of bf16 operands.
 * Forward: y[b][co][i][j] = sum x[b][ci][i+dy-1][j+dx-1] w[co][ci][dy][dx] (+ bias[co]).
 * This is the direct convolution the reference's own kernel tests compare against
 * (tests/run_conv3x3w_hw.py:21-30, run_conv3x3w_dw_hw.py:21-30); the CPU BF16 path
 * (torch_xdna_device.cpp:4594-4604) computes the same sum in fp32.
 */
void oracle_conv3x3_fwd(const uint16_t* x, const uint16_t* w, const uint16_t* bias, double* y,
                        int B, int Cin, int Cout, int H, int W) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int co = 0; co < Cout; ++co) {
      for (int i = 0; i < H; ++i)
        for (int j = 0; j < W; ++j) {
          double s = bias ? (double)bf16f(bias[co]) : 0.0;
          for (int ci = 0; ci < Cin; ++ci) {
            const uint16_t* xp = x + (((int64_t)b * Cin + ci) * H) * W;
            const uint16_t* wq = w + ((int64_t)co * Cin + ci) * 9;
            for (int dy = 0; dy < 3; ++dy) {
              const int yy = i + dy - 1;
              if (yy < 0 || yy >= H) continue;
              for (int dx = 0; dx < 3; ++dx) {
                const int xx = j + dx - 1;
                if (xx < 0 || xx >= W) continue;
                s += (double)bf16f(xp[(int64_t)yy * W + xx]) * (double)bf16f(wq[dy * 3 + dx]);
              }
            }
          }
          y[(((int64_t)b * Cout + co) * H + i) * W + j] = s;
        }
    }
}

/* Input gradient: dx[b][ci][i][j] = sum dy[b][co][i-dy+1][j-dx+1] w[co][ci][dy][dx]
 * (the adjoint of the forward sum, written without the flip+swap rewrite that the
 * reference's NPU path uses, conv_pack.cpp:470-473, so it checks that rewrite). */
void oracle_conv3x3_dgrad(const uint16_t* dy, const uint16_t* w, double* dx, int B, int Cin,
                          int Cout, int H, int W) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int ci = 0; ci < Cin; ++ci) {
      for (int i = 0; i < H; ++i)
        for (int j = 0; j < W; ++j) {
          double s = 0.0;
          for (int co = 0; co < Cout; ++co) {
            const uint16_t* gp = dy + (((int64_t)b * Cout + co) * H) * W;
            const uint16_t* wq = w + ((int64_t)co * Cin + ci) * 9;
            for (int ky = 0; ky < 3; ++ky) {
              const int oy = i - ky + 1;
              if (oy < 0 || oy >= H) continue;
              for (int kx = 0; kx < 3; ++kx) {
                const int ox = j - kx + 1;
                if (ox < 0 || ox >= W) continue;
                s += (double)bf16f(gp[(int64_t)oy * W + ox]) * (double)bf16f(wq[ky * 3 + kx]);
              }
            }
          }
          dx[(((int64_t)b * Cin + ci) * H + i) * W + j] = s;
        }
    }
}

/* Weight gradient gw[co][ci][dy][dx] = sum_{b,i,j} dy[b][co][i][j] x[b][ci][i+dy-1][j+dx-1]
 * (XdnaConv3x3wDwRuntime::compute, torch_xdna_device.cpp:2683-2751, in closed form),
 * and gb[co] = sum dy[b][co][i][j] (the CPU bias gradient, :4850-4877). gb may be NULL. */
void oracle_conv3x3_wgrad(const uint16_t* x, const uint16_t* dy, double* gw, double* gb, int B,
                          int Cin, int Cout, int H, int W) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int co = 0; co < Cout; ++co)
    for (int ci = 0; ci < Cin; ++ci) {
      for (int ky = 0; ky < 3; ++ky)
        for (int kx = 0; kx < 3; ++kx) {
          double s = 0.0;
          for (int b = 0; b < B; ++b) {
            const uint16_t* gp = dy + (((int64_t)b * Cout + co) * H) * W;
            const uint16_t* xp = x + (((int64_t)b * Cin + ci) * H) * W;
            for (int i = 0; i < H; ++i) {
              const int yy = i + ky - 1;
              if (yy < 0 || yy >= H) continue;
              for (int j = 0; j < W; ++j) {
                const int xx = j + kx - 1;
                if (xx < 0 || xx >= W) continue;
                s += (double)bf16f(gp[(int64_t)i * W + j]) * (double)bf16f(xp[(int64_t)yy * W + xx]);
              }
            }
          }
          gw[(((int64_t)co * Cin + ci) * 3 + ky) * 3 + kx] = s;
        }
    }
  if (gb) {
    for (int co = 0; co < Cout; ++co) {
      double s = 0.0;
      for (int b = 0; b < B; ++b)
        for (int64_t i = 0; i < (int64_t)H * W; ++i)
          s += (double)bf16f(dy[((int64_t)b * Cout + co) * H * W + i]);
      gb[co] = s;
    }
  }
}

/*
 * Fused Adam / AdamW step on one tensor, fp32 opmath, in place.  Restates PyTorch's
 * CPU _fused_adam_ / _fused_adamw_ (the kernel the reference's fallback runs for
 * fused=True groups: xdna_train/device.py:408-436, torch_xdna_device.cpp:5124-5260),
 * per element:
 *   g = grad / grad_scale (written back), negated if maximize
 *   Adam: g = fma(p, wd, g);   AdamW: p = p * float(1 - lr*wd)
 *   m = fma(w, g - m, m), w = float(1 - beta1)   [fma(-(g - m), 1 - w, g) if |w| >= 0.5]
 *   v = fma(float(1 - beta2) * g, g, v * float(beta2))
 *   den = sqrt(amsgrad ? max(max_v, v) : v) / float(sqrt(1 - beta2^t)) + float(eps)
 *   p = p - (float(lr / (1 - beta1^t)) * m) / den
 * dtype 0 = fp32 arrays, 1 = bf16 bit arrays; every stored value is rounded once.
 */
void oracle_adam(void* p_, void* g_, void* m_, void* v_, void* mx_, int64_t n, int dtype,
                 double step, double lr, double beta1, double beta2, double wd, double eps,
                 int amsgrad, int maximize, int adamw, double grad_scale, int has_scale) {
  const double bc1 = 1.0 - pow(beta1, step);
  const double bc2 = 1.0 - pow(beta2, step);
  const float step_size = (float)(lr / bc1);
  const float bc2_sqrt = (float)sqrt(bc2);
  const float w = (float)(1.0 - beta1);
  const float one_minus_w = 1.0f - w;
  const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2), e = (float)eps;
  const float wdf = (float)wd, decay = (float)(1.0 - lr * wd);
  for (int64_t i = 0; i < n; ++i) {
    float p, g, m, v, mx = 0.0f;
    if (dtype == 1) {
      p = bf16f(((uint16_t*)p_)[i]);
      g = bf16f(((uint16_t*)g_)[i]);
      m = bf16f(((uint16_t*)m_)[i]);
      v = bf16f(((uint16_t*)v_)[i]);
      if (amsgrad) mx = bf16f(((uint16_t*)mx_)[i]);
    } else {
      p = ((float*)p_)[i];
      g = ((float*)g_)[i];
      m = ((float*)m_)[i];
      v = ((float*)v_)[i];
      if (amsgrad) mx = ((float*)mx_)[i];
    }
    if (has_scale) {
      g = g / (float)grad_scale;
      if (dtype == 1) ((uint16_t*)g_)[i] = f2bf16(g);
      else ((float*)g_)[i] = g;
    }
    if (maximize) g = -g;
    if (wd != 0.0) {
      if (adamw) p = p * decay;
      else g = fmaf(p, wdf, g);
    }
    const float d = g - m;
    m = fabsf(w) < 0.5f ? fmaf(w, d, m) : fmaf(-d, one_minus_w, g);
    v = fmaf(omb2 * g, g, v * b2);
    float src = v;
    if (amsgrad) {
      mx = mx > v ? mx : v;
      src = mx;
    }
    const float den = sqrtf(src) / bc2_sqrt + e;
    p = p - (step_size * m) / den;
    if (dtype == 1) {
      ((uint16_t*)p_)[i] = f2bf16(p);
      ((uint16_t*)m_)[i] = f2bf16(m);
      ((uint16_t*)v_)[i] = f2bf16(v);
      if (amsgrad) ((uint16_t*)mx_)[i] = f2bf16(mx);
    } else {
      ((float*)p_)[i] = p;
      ((float*)m_)[i] = m;
      ((float*)v_)[i] = v;
      if (amsgrad) ((float*)mx_)[i] = mx;
    }
  }
}

/*
 * BFP16 ("bfp16ebs8") weight encoding for output channels [128 n_block, +128).
 * Spec: conv3x3w_host.py:49-82 (bfp16_encode: per 8 consecutive values, exponent byte =
 * largest biased fp32 exponent, mantissas = clip(rint(v / 2^(e-127-6)), -128, 127);
 * atb_shuffle: blocks [kb][n/16][k/8][2][8 n][8 k]; pack_weights: K order (chunk, dy, dx,
 * c), zero padding past Cin / Cout).  Host code: conv_pack.cpp:398-443 (forward: element
 * (n, c, t) = w[n][c][t], ld = Cin) and :474-519 (dx = 1: the dX conv's weights
 * w'[ci][co][t] = w[co][ci][8-t] read from the forward weight; Cout and Cin are the dX
 * conv's own channel counts, i.e. Cin_fwd and Cout_fwd, and ld = Cin_fwd).
 * The rounding is done in double, where v * 2^(133-e) is exact; NaN encodes as 0 (the
 * reference's int conversion of NaN on x86 gives INT_MIN, whose low byte is 0).
 */
void oracle_pack_weights_bfp16(const uint16_t* w, uint8_t* dst, int Cout, int Cin, int ld, int chunks,
                               int n_block, int dx) {
  uint8_t* out = dst;
  for (int kb = 0; kb < chunks * 9; ++kb) {
    const int chunk = kb / 9, tap = kb % 9;
    for (int n16 = 0; n16 < 8; ++n16)
      for (int k8 = 0; k8 < 8; ++k8)
        for (int two = 0; two < 2; ++two)
          for (int nl = 0; nl < 8; ++nl) {
            const int n = 128 * n_block + n16 * 16 + two * 8 + nl;
            float v[8];
            int emax = 0;
            for (int kl = 0; kl < 8; ++kl) {
              const int c = chunk * KSTEP + k8 * 8 + kl;
              uint16_t h = 0;
              if (c < Cin && n < Cout)
                h = dx ? w[((size_t)c * ld + n) * 9 + (8 - tap)] : w[((size_t)n * ld + c) * 9 + tap];
              v[kl] = bf16f(h);
              const int e = (h >> 7) & 0xFF;
              if (e > emax) emax = e;
            }
            *out++ = (uint8_t)emax;
            for (int kl = 0; kl < 8; ++kl) {
              double q = nearbyint(ldexp((double)v[kl], 133 - emax));
              if (isnan(q)) q = 0.0;
              if (q < -128.0) q = -128.0;
              if (q > 127.0) q = 127.0;
              *out++ = (uint8_t)(int8_t)(int)q;
            }
          }
  }
}

/*
 * BFP16 emulation of the reference NPU's conv arithmetic (the optional mode restated by
 * the reference's benchmarks/bfp16_training_gate.py:33-57; the NPU kernel
 * _designs/conv3x3w_kernel.cc:40-51, 105-108 and its loop order conv3x3w.py:172-177).
 *
 * Quantization: an aligned run of 8 values becomes the values of its bfp16ebs8 block, as
 * the codec above encodes it and the block decodes: q = clip(rint(v * 2^(133 - e_max)),
 * -128, 127), value q * 2^(e_max - 133), with e_max the largest biased exponent field of
 * the 8 (NaN stays NaN).  The value is formed in double and converted to float (exact, or
 * +-inf past the float range) and then to bf16 (exact: at most 8 significant bits).
 */
static void bfp16_quant8(const uint16_t* in, uint16_t* out) {
  int emax = 0;
  for (int i = 0; i < 8; ++i) {
    const int e = (in[i] >> 7) & 0xFF;
    if (e > emax) emax = e;
  }
  for (int i = 0; i < 8; ++i) {
    const float v = bf16f(in[i]);
    if (isnan(v)) {
      out[i] = 0x7FC0;
      continue;
    }
    double q = nearbyint(ldexp((double)v, 133 - emax));
    if (q < -128.0) q = -128.0;
    if (q > 127.0) q = 127.0;
    if (q == 0.0) q = 0.0; /* an int8 mantissa of 0 is +0 (nearbyint keeps the sign of -0.3) */
    out[i] = f2bf16((float)ldexp(q, emax - 133));
  }
}

void oracle_bfp16_quantize8(const uint16_t* src, uint16_t* dst, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b) bfp16_quant8(src + 8 * b, dst + 8 * b);
}

/* Round-to-nearest-even of a double to bf16 bits in one step (no float in between):
 * 8 significant bits in the normal range, multiples of 2^-133 below 2^-126. */
static uint16_t d2bf16(double x) {
  if (isnan(x)) return 0x7FC0;
  if (x == 0.0) return signbit(x) ? 0x8000 : 0;
  int e;
  (void)frexp(x, &e);                       /* |x| in [2^(e-1), 2^e) */
  const int lsb = e - 8 > -133 ? e - 8 : -133;
  const double r = ldexp(nearbyint(ldexp(x, -lsb)), lsb);
  return f2bf16((float)r);                  /* exact, or +-inf past the range */
}

/*
 * The emulated forward conv (3x3, stride 1, pad 1): x [B][Cin][H][W] quantized in runs of
 * 8 channels at each pixel (channels past Cin are zeros), w [Cout][Cin][3][3] in runs of 8
 * input channels at each (output channel, tap); per output, C = 0 and, for each 64-channel
 * chunk and within it each tap (dy, dx) in order, C = bf16(C + the chunk's 64-term sum in
 * double); then y = bf16(float(C) + float(bias)) (the reference's host bias add,
 * torch_xdna_device.cpp:2477-2480).  y holds bf16 bits.
 */
void oracle_conv3x3_bfp16_emul(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* y, int B,
                               int Cin, int Cout, int H, int W) {
  const int chunks = (Cin + KSTEP - 1) / KSTEP, cpad = chunks * KSTEP;
  const size_t plane = (size_t)H * W;
  /* quantized operands: xq [B][H][W][cpad] (channel runs contiguous), wq [Cout][9][cpad] */
  uint16_t* xq = (uint16_t*)malloc((size_t)B * plane * cpad * 2);
  uint16_t* wq = (uint16_t*)malloc((size_t)Cout * 9 * cpad * 2);
  if (!xq || !wq) {
    free(xq);
    free(wq);
    return;
  }
  uint16_t run[8];
  for (int b = 0; b < B; ++b)
    for (size_t p = 0; p < plane; ++p)
      for (int c0 = 0; c0 < cpad; c0 += 8) {
        for (int i = 0; i < 8; ++i)
          run[i] = c0 + i < Cin ? x[((size_t)b * Cin + c0 + i) * plane + p] : 0;
        bfp16_quant8(run, xq + ((size_t)b * plane + p) * cpad + c0);
      }
  for (int co = 0; co < Cout; ++co)
    for (int t = 0; t < 9; ++t)
      for (int c0 = 0; c0 < cpad; c0 += 8) {
        for (int i = 0; i < 8; ++i) run[i] = c0 + i < Cin ? w[((size_t)co * Cin + c0 + i) * 9 + t] : 0;
        bfp16_quant8(run, wq + ((size_t)co * 9 + t) * cpad + c0);
      }
  for (int b = 0; b < B; ++b)
    for (int co = 0; co < Cout; ++co)
      for (int yy = 0; yy < H; ++yy)
        for (int xx = 0; xx < W; ++xx) {
          double C = 0.0;
          for (int ch = 0; ch < chunks; ++ch)
            for (int t = 0; t < 9; ++t) {
              const int sy = yy + t / 3 - 1, sx = xx + t % 3 - 1;
              double s = 0.0;
              if (sy >= 0 && sy < H && sx >= 0 && sx < W) {
                const uint16_t* xr = xq + ((size_t)b * plane + (size_t)sy * W + sx) * cpad + ch * KSTEP;
                const uint16_t* wr = wq + ((size_t)co * 9 + t) * cpad + ch * KSTEP;
                for (int c = 0; c < KSTEP; ++c) s += (double)bf16f(xr[c]) * (double)bf16f(wr[c]);
              }
              C = (double)bf16f(d2bf16(C + s));
            }
          float out = (float)C;
          if (bias) out += bf16f(bias[co]);
          y[(((size_t)b * Cout + co) * H + yy) * W + xx] = f2bf16(out);
        }
  free(xq);
  free(wq);
}
