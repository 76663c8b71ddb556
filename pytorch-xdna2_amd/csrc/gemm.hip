// bf16 GEMM on gfx950 MFMA: C = alpha * A.B + beta * bias, fp32 accumulation, one
// bf16 rounding.  Replaces the reference's fixed-shape NPU GEMM and its CPU mm/addmm/
// bmm on aliases (torch_xdna_device.cpp:1330-1458, 3740-3790, 4360-4417): any shape,
// any element strides, so Linear's forward (B = W^T, k-contiguous), dX (B = W,
// n-contiguous) and dW (A = dY^T, m-contiguous) run without copies.
//
// Tiles: 128 x 128 x 32 per workgroup, four waves of 64 x 64 (2 x 2 MFMA 32x32x16).
// Both LDS tiles are stored k-contiguous ([row][k], pitch 40 elements) so every MFMA
// fragment is one 16-byte LDS read.  Staging picks per operand: 16-byte vector loads
// along k (k-contiguous source), 16-byte loads along m/n written transposed into LDS
// (m/n-contiguous source), or element loads (anything else, and the ragged edges).
#include "common.h"
#include "mfma.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

constexpr int kTM = 128, kTN = 128, kTK = 32, kLdsPitch = 40;

enum StageMode { kAlongK = 0, kAlongRow = 1, kScalar = 2 };

struct GemmArgs {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  const uint16_t* bias;
  int M, N, K;
  int64_t a_r, a_k, a_batch;  // A element (row=m, k) strides
  int64_t b_r, b_k, b_batch;  // B as [n][k]: element (row=n, k) strides
  int64_t c_m, c_n, c_batch;
  int bias_mode;
  int64_t bias_sm, bias_sn;
  float alpha, beta;
  int batch;
  int kt_per;   // k-tiles per split (blockIdx.z = batch index * nsplit + split)
  int nsplit;
  float* part;  // split-K: fp32 partial products [nsplit][batch][M][N], else null
  int rs_ok;    // 1: the epilogue stores through buffer resources (extents host-checked)
  int c_bytes, bias_bytes, part_bytes;  // byte extents of one batch's C / bias / partials
  int xcd_group;  // > 0: XCD-blocked tile order with groups of this many tile rows (gemm4)
};

// Workgroups go round-robin to the 8 XCDs (each with its own L2) in linear id order.  In
// launch order (x = column tile fastest) XCD x would take the column tiles x, x + 8, ...
// of every row, so each XCD would read all of A.  With xcd_group = G (the tile count a
// multiple of 8), XCD x takes tiles [x T/8, (x+1) T/8) of a grouped order (G tile rows at
// a time, rows fastest): a compact block of rows and columns per XCD, whose A and B tiles
// its L2 holds for the workgroups in flight.
constexpr int kGemmXcds = 8;

__device__ inline void gemm_tile_xy(const GemmArgs& g, int& bx, int& by) {
  bx = blockIdx.x;
  by = blockIdx.y;
  if (g.xcd_group <= 0) return;
  const int nx = gridDim.x, my = gridDim.y;
  const int T = nx * my;
  const int L = by * nx + bx;
  const int t = (L % kGemmXcds) * (T / kGemmXcds) + L / kGemmXcds;
  const int gsz = g.xcd_group * nx;
  const int grp = t / gsz, r = t - grp * gsz;
  const int gm = min(g.xcd_group, my - grp * g.xcd_group);
  by = grp * g.xcd_group + r % gm;
  bx = r / gm;
}

// Branch-free epilogue of one wave's MI x NJ block of 32 x 32 MFMA tiles (rows mb + i*32 +
// mfma_row(r, lane), columns nb + j*32 + lane % 32), through buffer resources: an element
// outside M x N gets an offset of kSkip or more, past the record count, so the hardware
// drops its store (and reads its bias as zero) and no store waits behind a branch.  Valid
// offsets stay below kSkip (rs_ok, checked on the host), so a valid row offset plus a
// skipped column offset, or two skipped ones, are dropped as well.
constexpr int kSkip = 0x40000000;

template <int MI, int NJ>
__device__ inline void store_block(const GemmArgs& g, int batch, int split, const f32x16_t (&acc)[MI][NJ],
                                   int mb, int nb, int lane) {
  const int lr = lane & 31;
  if (g.part) {
    float* P = g.part + (int64_t(split) * g.batch + batch) * g.M * g.N;
    const auto prs = uniform_buffer_rsrc(P, g.part_bytes);
    int noff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = nb + j * 32 + lr;
      noff[j] = n < g.N ? n * 4 : kSkip;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + i * 32 + mfma_row(r, lane);
        const int moff = m < g.M ? m * g.N * 4 : kSkip;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), prs, moff + noff[j], 0, 0);
        // one row of stores at a time: keeps the accumulators in place (no spills)
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  }
  const auto crs = uniform_buffer_rsrc(g.c + int64_t(batch) * g.c_batch, g.c_bytes);
  const bool bias = g.bias_mode != 0 && g.beta != 0.0f;
  const auto brs = uniform_buffer_rsrc(g.bias, bias ? g.bias_bytes : 0);
  int noff[NJ], nbo[NJ];
  float bn[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = nb + j * 32 + lr;
    noff[j] = n < g.N ? int(n * g.c_n * 2) : kSkip;
    nbo[j] = n < g.N ? int(n * g.bias_sn * 2) : kSkip;
    bn[j] = bias && g.bias_mode == 1 ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, nbo[j], 0, 0)) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mb + i * 32 + mfma_row(r, lane);
      const bool mok = m < g.M;
      const int moff = mok ? int(m * g.c_m * 2) : kSkip;
      const int mbo = mok ? int(m * g.bias_sm * 2) : kSkip;
      float bm = 0.0f;
      if (bias && g.bias_mode == 3) bm = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, mbo, 0, 0));
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float v = g.alpha * acc[i][j][r];
        if (bias) {
          float bv = g.bias_mode == 1 ? bn[j] : bm;
          if (g.bias_mode == 2) bv = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, mbo + nbo[j], 0, 0));
          v += g.beta * bv;
        }
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), crs, moff + noff[j], 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Stages rows [r0, r0+128) x k [k0, k0+32) of a row-major-by-strides operand into
// lds[row][k].  rows: valid row count; K: valid k count.
template <int kMode>
__device__ inline void stage(uint16_t* lds, const uint16_t* src, int64_t s_r, int64_t s_k, int r0,
                             int rows, int k0, int K, int tid) {
  if (kMode == kAlongK) {
    // 128 rows x 4 vectors of 8 k.
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int i = tid + it * 256;
      const int row = i >> 2, kv = (i & 3) * 8;
      const int r = r0 + row, k = k0 + kv;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r < rows) {
        const uint16_t* p = src + int64_t(r) * s_r + k;
        if (k + 8 <= K) {
          v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint32_t u[4] = {0, 0, 0, 0};
          for (int e = 0; e < 8; ++e)
            if (k + e < K) u[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
          v = make_uint4(u[0], u[1], u[2], u[3]);
        }
      }
      *reinterpret_cast<uint4*>(lds + row * kLdsPitch + kv) = v;
    }
  } else if (kMode == kAlongRow) {
    // 32 k x 16 vectors of 8 rows; each vector is written transposed.
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int i = tid + it * 256;
      const int kk = i >> 4, rv = (i & 15) * 8;
      const int r = r0 + rv, k = k0 + kk;
      uint32_t u[4] = {0, 0, 0, 0};
      if (k < K) {
        const uint16_t* p = src + int64_t(k) * s_k + r;
        if (r + 8 <= rows) {
          const uint4 v = *reinterpret_cast<const uint4*>(p);
          u[0] = v.x; u[1] = v.y; u[2] = v.z; u[3] = v.w;
        } else {
          for (int e = 0; e < 8; ++e)
            if (r + e < rows) u[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        lds[(rv + e) * kLdsPitch + kk] = uint16_t((e & 1) ? (u[e >> 1] >> 16) : (u[e >> 1] & 0xFFFF));
    }
  } else {
    // Element by element (strides without 16-byte vectors): all 16 loads of a thread are
    // issued before the first LDS write (a load-store loop waited one memory latency per
    // element), out-of-range elements read element 0 and are masked (no branches), and
    // consecutive lanes take the operand's unit-stride direction where it has one.
    constexpr int kPer = 128 * kTK / 256;
    const bool rows_fast = s_r == 1 && s_k != 1;
    uint32_t v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * 256;
      const int row = rows_fast ? (i & 127) : i / kTK;
      const int kk = rows_fast ? (i >> 7) : i % kTK;
      const int r = r0 + row, k = k0 + kk;
      const bool ok = r < rows && k < K;
      const uint32_t e = src[ok ? int64_t(r) * s_r + int64_t(k) * s_k : 0];
      v[j] = ok ? e : 0u;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * 256;
      const int row = rows_fast ? (i & 127) : i / kTK;
      const int kk = rows_fast ? (i >> 7) : i % kTK;
      lds[row * kLdsPitch + kk] = uint16_t(v[j]);
    }
  }
}

template <int kModeA, int kModeB>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t as[kTM * kLdsPitch];
  __shared__ __attribute__((aligned(16))) uint16_t bs[kTN * kLdsPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kTM, n0 = blockIdx.x * kTN;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  const int kbeg = split * g.kt_per * kTK, kend = min(g.K, kbeg + g.kt_per * kTK);
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero_acc();

  for (int k0 = kbeg; k0 < kend; k0 += kTK) {
    __syncthreads();
    stage<kModeA>(as, A, g.a_r, g.a_k, m0, g.M, k0, kend, tid);
    stage<kModeB>(bs, B, g.b_r, g.b_k, n0, g.N, k0, kend, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kTK / 16; ++ks) {
      bf16x8_t af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = as_bf16x8(*reinterpret_cast<const uint4*>(as + (wm * 64 + i * 32 + lr) * kLdsPitch + ks * 16 + lk));
        bfr[i] = as_bf16x8(*reinterpret_cast<const uint4*>(bs + (wn * 64 + i * 32 + lr) * kLdsPitch + ks * 16 + lk));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_32x32x16(af[i], bfr[j], acc[i][j]);
    }
  }

  if (g.rs_ok) {
    store_block<2, 2>(g, batch, split, acc, m0 + wm * 64, n0 + wn * 64, lane);
    return;
  }
  if (g.part) {
    float* P = g.part + (int64_t(split) * g.batch + batch) * g.M * g.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 64 + i * 32 + mfma_row(r, lane);
          if (m < g.M) P[int64_t(m) * g.N + n] = acc[i][j][r];
        }
      }
    return;
  }
  uint16_t* C = g.c + int64_t(batch) * g.c_batch;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + lr;
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + mfma_row(r, lane);
        if (m >= g.M) continue;
        float v = g.alpha * acc[i][j][r];
        if (g.bias_mode && g.beta != 0.0f) {
          float bv;
          if (g.bias_mode == 1) bv = bf16_to_f32(g.bias[int64_t(n) * g.bias_sn]);
          else if (g.bias_mode == 2) bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm + int64_t(n) * g.bias_sn]);
          else bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm]);
          v += g.beta * bv;
        }
        C[int64_t(m) * g.c_m + int64_t(n) * g.c_n] = f32_to_bf16(v);
      }
    }
}

// ---------------------------------------------------------------------------------------
// Large-tile variant: 256 x 256 output tile, k-tile 64, 8 waves (two per SIMD); wave
// (wm, wn) owns rows [wm*128, +128) x columns [wn*64, +64) (4 x 2 MFMA tiles).  Both
// operands are staged k-contiguous in LDS ([256][72] each, double-buffered, 144 KiB);
// the next k-tile is loaded into registers while the current one is multiplied.
// An operand whose rows are contiguous (kAlongRow: A = dY^T, B = W in dX) is read as
// 4 (k) x 8 (rows) blocks with 16-byte loads and transposed in registers (v_perm) into
// 8-byte LDS writes.
// ---------------------------------------------------------------------------------------
constexpr int kT2 = 256, kK2 = 64, kP2 = 72;
constexpr size_t kGemm2Lds = size_t(2) * 2 * kT2 * kP2 * 2;  // 2 buffers x (A, B)

typedef unsigned int g2u4 __attribute__((ext_vector_type(4)));
typedef unsigned int g2u2 __attribute__((ext_vector_type(2)));

// Registers of one operand's k-tile: 4 x 16 bytes per thread.
template <int kMode>
__device__ inline void g2_load(g2u4 (&r)[4], const uint16_t* src, int64_t s_r, int64_t s_k, int r0,
                               int rows, int k0, int K, int tid) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (kMode == kAlongK) {
      // vector v: row v / 8, k [k0 + (v % 8) * 8, +8)
      const int v = tid + j * 512;
      const int row = v >> 3, k = k0 + (v & 7) * 8;
      const int rr = r0 + row;
      g2u4 x = {0u, 0u, 0u, 0u};
      if (rr < rows) {
        const uint16_t* p = src + int64_t(rr) * s_r + k;
        if (k + 8 <= K) {
          x = *reinterpret_cast<const g2u4*>(p);
        } else {
          for (int e = 0; e < 8; ++e)
            if (k + e < K) x[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
        }
      }
      r[j] = x;
    } else {
      // thread t: rows [r0 + (t % 32) * 8, +8), k = k0 + (t / 32) * 4 + j (one 16-byte row run)
      const int rg = tid & 31, k = k0 + (tid >> 5) * 4 + j;
      const int rr = r0 + rg * 8;
      g2u4 x = {0u, 0u, 0u, 0u};
      if (k < K) {
        const uint16_t* p = src + int64_t(k) * s_k + rr;
        if (rr + 8 <= rows) {
          x = *reinterpret_cast<const g2u4*>(p);
        } else {
          for (int e = 0; e < 8; ++e)
            if (rr + e < rows) x[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
        }
      }
      r[j] = x;
    }
  }
}

template <int kMode>
__device__ inline void g2_store(uint16_t* lds, const g2u4 (&r)[4], int tid) {
  if (kMode == kAlongK) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int v = tid + j * 512;
      *reinterpret_cast<g2u4*>(lds + (v >> 3) * kP2 + (v & 7) * 8) = r[j];
    }
  } else {
    // r[j] holds rows rg*8 .. +7 at k = kq*4 + j; row e gets (k0..k3) as two dwords
    const int rg = tid & 31, kq = tid >> 5;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;  // high / low halves
      g2u2 w;
      w[0] = __builtin_amdgcn_perm(r[1][e >> 1], r[0][e >> 1], sel);
      w[1] = __builtin_amdgcn_perm(r[3][e >> 1], r[2][e >> 1], sel);
      *reinterpret_cast<g2u2*>(lds + (rg * 8 + e) * kP2 + kq * 4) = w;
    }
  }
}

template <int kModeA, int kModeB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm2_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kT2, n0 = blockIdx.x * kT2;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  const int kbeg = split * g.kt_per * kK2, kend = min(g.K, kbeg + g.kt_per * kK2);
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero_acc();

  g2u4 ra[4], rb[4];
  if (kbeg < kend) {
    g2_load<kModeA>(ra, A, g.a_r, g.a_k, m0, g.M, kbeg, kend, tid);
    g2_load<kModeB>(rb, B, g.b_r, g.b_k, n0, g.N, kbeg, kend, tid);
    g2_store<kModeA>(smem, ra, tid);
    g2_store<kModeB>(smem + kT2 * kP2, rb, tid);
  }
  __syncthreads();
  int cur = 0;
  for (int k0 = kbeg; k0 < kend; k0 += kK2) {
    const bool more = k0 + kK2 < kend;
    if (more) {
      g2_load<kModeA>(ra, A, g.a_r, g.a_k, m0, g.M, k0 + kK2, kend, tid);
      g2_load<kModeB>(rb, B, g.b_r, g.b_k, n0, g.N, k0 + kK2, kend, tid);
    }
    const uint16_t* as = smem + cur * 2 * kT2 * kP2;
    const uint16_t* bs = as + kT2 * kP2;
#pragma unroll
    for (int ks = 0; ks < kK2 / 16; ++ks) {
      bf16x8_t af[4], bfr[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(as + (wm * 128 + i * 32 + lr) * kP2 + ks * 16 + lk));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(bs + (wn * 64 + j * 32 + lr) * kP2 + ks * 16 + lk));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_32x32x16(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      uint16_t* nxt = smem + (cur ^ 1) * 2 * kT2 * kP2;
      g2_store<kModeA>(nxt, ra, tid);
      g2_store<kModeB>(nxt + kT2 * kP2, rb, tid);
    }
    __syncthreads();
    cur ^= 1;
  }

  if (g.rs_ok) {
    store_block<4, 2>(g, batch, split, acc, m0 + wm * 128, n0 + wn * 64, lane);
    return;
  }
  if (g.part) {
    float* P = g.part + (int64_t(split) * g.batch + batch) * g.M * g.N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + i * 32 + mfma_row(r, lane);
          if (m < g.M) P[int64_t(m) * g.N + n] = acc[i][j][r];
        }
      }
    return;
  }
  uint16_t* C = g.c + int64_t(batch) * g.c_batch;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + lr;
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 128 + i * 32 + mfma_row(r, lane);
        if (m >= g.M) continue;
        float v = g.alpha * acc[i][j][r];
        if (g.bias_mode && g.beta != 0.0f) {
          float bv;
          if (g.bias_mode == 1) bv = bf16_to_f32(g.bias[int64_t(n) * g.bias_sn]);
          else if (g.bias_mode == 2) bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm + int64_t(n) * g.bias_sn]);
          else bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm]);
          v += g.beta * bv;
        }
        C[int64_t(m) * g.c_m + int64_t(n) * g.c_n] = f32_to_bf16(v);
      }
    }
}

// ---------------------------------------------------------------------------------------
// Four-wave variant: the same 256 x 256 tile with k-tile 64, one wave per SIMD owning a
// 128 x 128 block (4 x 4 MFMA tiles, accumulators in the AGPR half of the register
// file): 8 fragment reads per 16 MFMAs.  Latency is covered by pipelining, not by a
// second wave: fragments are read one k-step ahead (across k-tiles too), the global loads
// of k-tile t+2 issue between the MFMAs of k-tile t's first two k-steps, and the barrier
// that opens k-step 3 frees this k-tile's LDS buffer for them.  Loads are unconditional
// (clamped addresses, zero-masked results), so the memory counters are static.  Needs
// whole 8-element vectors: K % 8 == 0 for k-contiguous operands, rows % 8 == 0 for
// row-contiguous ones (checked by the launcher).
// ---------------------------------------------------------------------------------------
constexpr int kT4 = 256, kK4 = 64, kP4 = 72;
// A row-contiguous operand's k-tile stays in its own layout, [k][row] with pitch kPR4,
// and its MFMA fragments are read with the transposing LDS read; it fits the region of a
// k-contiguous tile.  The pitch (144 dwords, 16 mod 64) puts the 4 k rows x 32 row
// elements of a half-wave read on distinct banks (272 elements overlapped two of them).
constexpr int kPR4 = kT4 + 32;
static_assert(kK4 * kPR4 <= kT4 * kP4, "a [k][row] tile fits the operand region");
typedef short g4i16x4 __attribute__((ext_vector_type(4)));
constexpr size_t kGemm4Lds = size_t(2) * 2 * kT4 * kP4 * 2;  // 2 buffers x (A, B)

// One operand's loads through a buffer resource: per thread 8 vectors of 16 bytes per
// k-tile.  The row part of each vector's offset is fixed for the workgroup (-1 for rows
// past the operand); the k part moves with the k-tile.  A vector outside the operand gets
// an offset past the resource's size, and the buffer load returns zeros for it: no
// branch and no select on the data.
struct G4Operand {
  __amdgpu_buffer_rsrc_t rs;
  int roff[8];   // row * s_r (elements), or -1
  int kq[8];     // k offset of vector j within a k-tile
  int s_k;
};

template <int kMode>
__device__ inline G4Operand g4_operand(const uint16_t* src, int64_t s_r, int64_t s_k, int r0, int rows,
                                       int K, int tid) {
  G4Operand o;
  // bytes up to the last element of the operand (< 2^31: checked by the launcher)
  const int64_t extent = ((int64_t(rows) - 1) * s_r + (int64_t(K) - 1) * s_k + 1) * 2;
  o.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src), 0, int(extent), 0x00020000);
  o.s_k = int(s_k);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int row;
    if (kMode == kAlongK) {
      // vector v = tid + 256 j: row v / 8, k [(v % 8) * 8, +8)
      const int v = tid + j * 256;
      row = r0 + (v >> 3);
      o.kq[j] = (v & 7) * 8;
    } else {
      // vector v = tid + 256 j: rows [r0 + (v % 32) * 8, +8) at k = v / 32
      const int v = tid + j * 256;
      row = r0 + (v & 31) * 8;
      o.kq[j] = v >> 5;
    }
    o.roff[j] = row < rows ? int(int64_t(row) * s_r) : -1;
  }
  return o;
}

__device__ inline void g4_load(u32x4_t (&r)[8], const G4Operand& o, int k0, int K) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = k0 + o.kq[j];
    const bool ok = o.roff[j] >= 0 && k < K;
    const int off = ok ? (o.roff[j] + k * o.s_k) * 2 : 0x7FFFFFF0;
    r[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(o.rs, off, 0, 0));
  }
}

template <int kMode>
__device__ inline void g4_store(uint16_t* lds, const u32x4_t (&r)[8], int tid) {
  if (kMode == kAlongK) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int v = tid + j * 256;
      *reinterpret_cast<u32x4_t*>(lds + (v >> 3) * kP4 + (v & 7) * 8) = r[j];
    }
  } else {
    // as loaded: 8 rows at one k per vector, into the [k][row] tile
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int v = tid + j * 256;
      *reinterpret_cast<u32x4_t*>(lds + (v >> 5) * kPR4 + (v & 31) * 8) = r[j];
    }
  }
}

// MFMA fragment of a k-tile: row rb + lane % 32, k = kk + 8 (lane / 32) .. +8.  From a
// [k][row] tile with two transposing reads: in 16-lane group g = lane / 16 (rows
// +16 (g % 2), k +8 (g / 2)), lane j supplies (k + j / 4, row + 4 (j % 4)) and every lane
// receives 4 consecutive k of its own row (layout measured on the MI355X).
template <int kMode>
__device__ inline u32x4_t g4_frag(const uint16_t* tile, int rb, int kk, int lane) {
  if (kMode == kAlongK)
    return *reinterpret_cast<const u32x4_t*>(tile + (rb + (lane & 31)) * kP4 + kk + (lane >> 5) * 8);
  const int g = lane >> 4, j = lane & 15;
  const uint16_t* p = tile + (kk + 8 * (g >> 1) + (j >> 2)) * kPR4 + rb + 16 * (g & 1) + 4 * (j & 3);
  const g4i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p));
  const g4i16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p + 4 * kPR4));
  const g2u2 a = __builtin_bit_cast(g2u2, lo), b = __builtin_bit_cast(g2u2, hi);
  return u32x4_t{a[0], a[1], b[0], b[1]};
}

template <int kModeA, int kModeB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm4_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  int tbx, tby;
  gemm_tile_xy(g, tbx, tby);
  const int m0 = tby * kT4, n0 = tbx * kT4;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  const int kbeg = split * g.kt_per * kK4, kend = min(g.K, kbeg + g.kt_per * kK4);
  const int ntiles = kend > kbeg ? (kend - kbeg + kK4 - 1) / kK4 : 0;
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero_acc();

  u32x4_t ra[8], rb[8];
  u32x4_t fa[2][4], fb[2][4];
  const G4Operand oa = g4_operand<kModeA>(A, g.a_r, g.a_k, m0, g.M, g.K, tid);
  const G4Operand ob = g4_operand<kModeB>(B, g.b_r, g.b_k, n0, g.N, g.K, tid);
  // k-tile t lives in LDS buffer t % 2: A at [256][kP4], then B
  auto abuf = [&](int t) { return smem + (t & 1) * 2 * kT4 * kP4; };
#define XDNA_G4_LOAD(t_)                                                                     \
  do {                                                                                       \
    const int k_ = kbeg + min((t_), ntiles - 1) * kK4;                                       \
    g4_load(ra, oa, k_, kend);                                                               \
    g4_load(rb, ob, k_, kend);                                                               \
  } while (0)
#define XDNA_G4_STORE(t_)                                                                    \
  do {                                                                                       \
    g4_store<kModeA>(abuf(t_), ra, tid);                                                     \
    g4_store<kModeB>(abuf(t_) + kT4 * kP4, rb, tid);                                         \
  } while (0)
#define XDNA_G4_FRAGS(buf_, t_, ks_)                                                         \
  do {                                                                                       \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                            \
      fa[buf_][i] = g4_frag<kModeA>(abuf(t_), wm * 128 + i * 32, (ks_) * 16, lane);          \
    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                            \
      fb[buf_][j] = g4_frag<kModeB>(abuf(t_) + kT4 * kP4, wn * 128 + j * 32, (ks_) * 16, lane); \
  } while (0)
#define XDNA_G4_MFMA(buf_)                                                                   \
  do {                                                                                       \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                            \
      _Pragma("unroll") for (int j = 0; j < 4; ++j)                                          \
        acc[i][j] = mfma_32x32x16(as_bf16x8(fa[buf_][i]), as_bf16x8(fb[buf_][j]), acc[i][j]); \
  } while (0)

  if (ntiles > 0) {
    // prologue: k-tiles 0 and 1 in LDS
    XDNA_G4_LOAD(0);
    XDNA_G4_STORE(0);
    XDNA_G4_LOAD(1);
    XDNA_G4_STORE(1);
    __syncthreads();
    XDNA_G4_FRAGS(0, 0, 0);
    constexpr int kMfma = 0x008, kVmemRd = 0x020, kDsRd = 0x100, kDsWr = 0x200;
    // LDS reads per k-step: one per fragment, two for a row-contiguous operand's
    constexpr int kRd = (kModeA == kAlongK ? 4 : 8) + (kModeB == kAlongK ? 4 : 8);
    for (int t = 0; t < ntiles; ++t) {
#pragma unroll
      for (int ks = 0; ks < 3; ++ks) {
        const int cur = ks & 1;
        XDNA_G4_FRAGS(cur ^ 1, t, ks + 1);
        if (ks == 0) XDNA_G4_LOAD(t + 2);    // k-tile t+2 into registers
        XDNA_G4_MFMA(cur);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
          if (i < kRd) __builtin_amdgcn_sched_group_barrier(kDsRd, 1, 0);
          if (ks == 0 && i < 8) __builtin_amdgcn_sched_group_barrier(kVmemRd, 2, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // every wave has read this k-tile's buffer for the last time (k-step 3's fragments)
      __syncthreads();
      XDNA_G4_FRAGS(0, t + 1, 0);            // k-tile t+1: stored one k-tile ago
      XDNA_G4_STORE(t + 2);                  // into this k-tile's buffer
      XDNA_G4_MFMA(1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        if (i < kRd) __builtin_amdgcn_sched_group_barrier(kDsRd, 1, 0);
        if (i >= 8) __builtin_amdgcn_sched_group_barrier(kDsWr, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#undef XDNA_G4_LOAD
#undef XDNA_G4_STORE
#undef XDNA_G4_FRAGS
#undef XDNA_G4_MFMA

  // buffer-resource epilogue only (the launcher checks rs_ok): a second, per-element
  // path would keep every accumulator live across both and spill them
  store_block<4, 4>(g, batch, split, acc, m0 + wm * 128, n0 + wn * 128, lane);
}

// Split-K epilogue: C[b][m][n] = bf16(alpha * sum over splits (in split order) of the fp32
// partials + beta * bias term), consecutive threads on consecutive n.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs g) {
  const int64_t mn = int64_t(g.M) * g.N;
  const int64_t n_all = mn * g.batch;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n_all; i += int64_t(gridDim.x) * 256) {
    const int b = int(i / mn);
    const int64_t r = i - int64_t(b) * mn;
    const int m = int(r / g.N), n = int(r - int64_t(m) * g.N);
    float acc = 0.0f;
    acc = sum_strided8(acc, g.part + i, n_all, 0, 1, g.nsplit);
    float v = g.alpha * acc;
    if (g.bias_mode && g.beta != 0.0f) {
      float bv;
      if (g.bias_mode == 1) bv = bf16_to_f32(g.bias[int64_t(n) * g.bias_sn]);
      else if (g.bias_mode == 2) bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm + int64_t(n) * g.bias_sn]);
      else bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm]);
      v += g.beta * bv;
    }
    g.c[int64_t(b) * g.c_batch + int64_t(m) * g.c_m + int64_t(n) * g.c_n] = f32_to_bf16(v);
  }
}

// The same epilogue four outputs at a time, for C rows of unit column stride and N % 4 == 0
// (8-byte-aligned C rows, 16-byte-aligned partials) and fewer than 2^31 groups of four: one
// 16-byte partial load per split and one 8-byte store per thread, 32-bit index math.  Each
// output is the scalar form's sum in the same split order, with the same alpha, bias and
// rounding, so the bits are the same.
__global__ __launch_bounds__(256) void gemm_reduce4_kernel(GemmArgs g) {
  const int n4 = g.N >> 2;
  const int rows = g.M * g.batch;  // (b, m) pairs, b-major
  const int64_t n_all = int64_t(g.M) * g.N * g.batch;
  const int total = rows * n4;
  const float4* part = reinterpret_cast<const float4*>(g.part);
  const int64_t zs = n_all >> 2;  // float4 stride of one split
  for (int i = int(blockIdx.x) * 256 + int(threadIdx.x); i < total; i += int(gridDim.x) * 256) {
    const int row = i / n4, q = i - row * n4;
    const int b = row / g.M, m = row - b * g.M;
    const int n = q << 2;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // four splits' loads issued before their sums, which stay in split order
    int z = 0;
    for (; z + 3 < g.nsplit; z += 4) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = part[int64_t(z + u) * zs + i];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc.x += v[u].x;
        acc.y += v[u].y;
        acc.z += v[u].z;
        acc.w += v[u].w;
      }
    }
    for (; z < g.nsplit; ++z) {
      const float4 v = part[int64_t(z) * zs + i];
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    float o[4] = {g.alpha * acc.x, g.alpha * acc.y, g.alpha * acc.z, g.alpha * acc.w};
    if (g.bias_mode && g.beta != 0.0f) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float bv;
        if (g.bias_mode == 1) bv = bf16_to_f32(g.bias[int64_t(n + e) * g.bias_sn]);
        else if (g.bias_mode == 2) bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm + int64_t(n + e) * g.bias_sn]);
        else bv = bf16_to_f32(g.bias[int64_t(m) * g.bias_sm]);
        o[e] += g.beta * bv;
      }
    }
    const uint2 packed = make_uint2(uint32_t(f32_to_bf16(o[0])) | (uint32_t(f32_to_bf16(o[1])) << 16),
                                    uint32_t(f32_to_bf16(o[2])) | (uint32_t(f32_to_bf16(o[3])) << 16));
    *reinterpret_cast<uint2*>(g.c + int64_t(b) * g.c_batch + int64_t(m) * g.c_m + n) = packed;
  }
}

// The split-K epilogue launch: the four-wide form where its conditions hold.
void launch_gemm_reduce(const GemmArgs& g, hipStream_t st) {
  const int64_t n_all = int64_t(g.batch) * g.M * g.N;
  const bool vec = g.c_n == 1 && (g.N % 4) == 0 && (reinterpret_cast<uintptr_t>(g.c) & 7) == 0 &&
                   (g.c_m % 4) == 0 && (g.batch <= 1 || (g.c_batch % 4) == 0) && n_all / 4 < (int64_t(1) << 31) &&
                   int64_t(g.M) * g.batch < (int64_t(1) << 31);
  if (vec) {
    gemm_reduce4_kernel<<<unsigned(std::min<int64_t>(ceil_div(n_all / 4, 256), 8192)), 256, 0, st>>>(g);
    return;
  }
  gemm_reduce_kernel<<<unsigned(std::min<int64_t>(ceil_div(n_all, 256), 4096)), 256, 0, st>>>(g);
}

// Operand described as [rows][k] with element strides (s_r, s_k).
int stage_mode(const void* base, int64_t s_r, int64_t s_k, int64_t s_batch, int batch) {
  const bool a16 = (reinterpret_cast<uintptr_t>(base) & 15) == 0;
  const bool batch_ok = batch <= 1 || (s_batch % 8) == 0;
  if (s_k == 1 && a16 && (s_r % 8) == 0 && batch_ok) return kAlongK;
  if (s_r == 1 && a16 && (s_k % 8) == 0 && batch_ok) return kAlongRow;
  return kScalar;
}

template <int MA, int MB>
bool gemm2_lds_ok() {
  static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm2_kernel<MA, MB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(kGemm2Lds)) == hipSuccess;
  return ok;
}

template <int MA, int MB>
bool launch2(dim3 grid, hipStream_t st, const GemmArgs& g) {
  if (!gemm2_lds_ok<MA, MB>()) return false;
  gemm2_kernel<MA, MB><<<grid, 512, kGemm2Lds, st>>>(g);
  return true;
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS variant of the four-wave kernel: the same 256 x 256 tile and wave layout,
// with k-tiles of 32 loaded by gfx950's 16-byte LDS DMA (buffer_load ... lds): a wave's
// load instruction writes 64 x 16 bytes contiguously at an LDS base (measured on the
// MI355X: lane L at base + 16 L; a lane past the buffer's range writes zeros), so the
// data never passes through registers and no LDS store is issued.  Four k-tile buffers
// (128 KB) let a k-tile's loads issue three k-tiles before its first read; a wave waits
// on its own loads with a counted s_waitcnt and the barrier publishes everyone's.
// Layouts, both unpadded with 16-byte pieces permuted so that MFMA fragment reads hit
// distinct banks (each lane loads the piece its LDS position holds):
//   k-contiguous operand, [256 rows][4 pieces of 8 k]: piece c of row r at r * 4 + (c ^ ((r >> 2) & 3));
//   row-contiguous operand, [32 k][32 pieces of 8 rows]: piece q of k row kr at kr * 32 + (q ^ 4 (kr & 3)).
// ---------------------------------------------------------------------------------------
constexpr int kK5 = 32, kNB5 = 4;
constexpr int kTile5 = kT4 * kK5;                          // elements of one operand's k-tile
constexpr size_t kGemm5Lds = size_t(kNB5) * 2 * kTile5 * 2;  // 4 buffers x (A, B): 128 KB

// One operand's DMA plan: per thread 4 loads of 16 bytes per k-tile (blocks 4 w + i of
// 1 KB, w the wave).  roff: the row part of the element offset (-1: rows past the
// operand), kq: the k offset within the k-tile.
struct G5Operand {
  i32x4_t rs;
  int roff[4];
  int kq[4];
  int s_k;
};

// kPerm16: the tile permutations of the 16x16x32 kernel (gemm6_kernel): k-contiguous,
// piece c of row r at c ^ 2 ((r >> 3) & 1), which the LDS serves without bank conflicts for
// reads of 16 rows x 4 pieces (the k-contiguous permutation above measured 2 conflict cycles
// per LDS-active cycle there); [k][row], for transposing reads that cover k rows R .. R+3
// and R+8 .. R+11 in one half-wave
template <int kMode, bool kPerm16 = false>
__device__ inline G5Operand g5_operand(const uint16_t* src, int64_t s_r, int64_t s_k, int r0, int rows, int K,
                                       int tid) {
  G5Operand o;
  const int64_t extent = ((int64_t(rows) - 1) * s_r + (int64_t(K) - 1) * s_k + 1) * 2;
  o.rs = lds_dma_rsrc(src, int(extent));
  o.s_k = int(s_k);
  const int lane = tid & 63, w = tid >> 6;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = 4 * w + i;
    if (kMode == kAlongK) {
      // block j: rows 16 j .. 16 j + 15, lane L at row 16 j + L / 4, position L % 4
      const int r = 16 * j + (lane >> 2);
      const int c = (lane & 3) ^ (kPerm16 ? 2 * ((r >> 3) & 1) : (r >> 2) & 3);
      o.roff[i] = r0 + r < rows ? int(int64_t(r0 + r) * s_r) : -1;
      o.kq[i] = c * 8;
    } else {
      // block j: k rows 2 j, 2 j + 1, lane L at k row 2 j + L / 32, position L % 32
      const int kr = 2 * j + (lane >> 5);
      const int q = (lane & 31) ^ (4 * (kr & 3) + (kPerm16 ? 2 * ((kr >> 3) & 1) : 0));
      o.roff[i] = r0 + 8 * q < rows ? (r0 + 8 * q) : -1;  // s_r == 1
      o.kq[i] = kr;
    }
  }
  return o;
}

// Byte offset of DMA load i of k-tile k0 .. k0 + 31 (masked past K: out of range).
__device__ inline int g5_off(const G5Operand& o, int i, int k0, int K) {
  const int k = k0 + o.kq[i];
  return o.roff[i] >= 0 && k < K ? (o.roff[i] + k * o.s_k) * 2 : 0x7FFFFFF0;
}

// The 4 DMA loads of k-tile k0 .. k0 + 31 (clamped, masked past K) into `tile`.
__device__ inline void g5_load(uint16_t* tile, const G5Operand& o, int k0, int K, int w) {
#pragma unroll
  for (int i = 0; i < 4; ++i) lds_dma16(o.rs, tile + (4 * w + i) * 512, g5_off(o, i, k0, K));
}

// MFMA fragment (rows rb + lane % 32, k = 16 ks + 8 (lane / 32) .. +8) from a k-tile.
template <int kMode>
__device__ inline u32x4_t g5_frag(const uint16_t* tile, int rb, int ks, int lane) {
  if (kMode == kAlongK) {
    const int r = rb + (lane & 31);
    const int c = (2 * ks + (lane >> 5)) ^ ((r >> 2) & 3);
    return *reinterpret_cast<const u32x4_t*>(tile + (r * 4 + c) * 8);
  }
  // transposing reads: in 16-lane group g = lane / 16 (rows +16 (g % 2), k +8 (g / 2)),
  // lane j supplies (k + j / 4, row + 4 (j % 4)); every lane receives 4 consecutive k of
  // its own row.  The high half (k + 4) keeps k % 4, so the same piece permutation.
  const int g = lane >> 4, j = lane & 15;
  const int kr = 16 * ks + 8 * (g >> 1) + (j >> 2);
  const int rr = rb + 16 * (g & 1) + 4 * (j & 3);
  const uint16_t* p = tile + (kr * 32 + ((rr >> 3) ^ (4 * (kr & 3)))) * 8 + (rr & 7);
  const g4i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p));
  const g4i16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p + 4 * 32 * 8));
  const g2u2 a = __builtin_bit_cast(g2u2, lo), b = __builtin_bit_cast(g2u2, hi);
  return u32x4_t{a[0], a[1], b[0], b[1]};
}


template <int kModeA, int kModeB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm5_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  int tbx, tby;
  gemm_tile_xy(g, tbx, tby);
  const int m0 = tby * kT4, n0 = tbx * kT4;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  // split-K ranges are whole k-tiles of 64 (kt_per counts those)
  const int kbeg = split * g.kt_per * kK4, kend = min(g.K, kbeg + g.kt_per * kK4);
  const int ntiles = kend > kbeg ? (kend - kbeg + kK5 - 1) / kK5 : 0;
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero_acc();

  if (ntiles > 0) {
    u32x4_t fa[2][4], fb[2][4];
    const G5Operand oa = g5_operand<kModeA>(A, g.a_r, g.a_k, m0, g.M, g.K, tid);
    const G5Operand ob = g5_operand<kModeB>(B, g.b_r, g.b_k, n0, g.N, g.K, tid);
    // k-tile t in buffer t % 4: A then B
    auto tbuf = [&](int t) { return smem + (t & (kNB5 - 1)) * 2 * kTile5; };
#define XDNA_G5_LOAD(t_)                                                                      \
  do {                                                                                        \
    const int k_ = kbeg + min((t_), ntiles - 1) * kK5;                                        \
    g5_load(tbuf(t_), oa, k_, kend, wave);                                                    \
    g5_load(tbuf(t_) + kTile5, ob, k_, kend, wave);                                           \
  } while (0)
#define XDNA_G5_FRAGS(buf_, t_, ks_)                                                          \
  do {                                                                                        \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                             \
      fa[buf_][i] = g5_frag<kModeA>(tbuf(t_), wm * 128 + i * 32, (ks_), lane);                \
    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                             \
      fb[buf_][j] = g5_frag<kModeB>(tbuf(t_) + kTile5, wn * 128 + j * 32, (ks_), lane);       \
  } while (0)
#define XDNA_G5_MFMA(buf_)                                                                    \
  do {                                                                                        \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                             \
      _Pragma("unroll") for (int j = 0; j < 4; ++j)                                           \
        acc[i][j] = mfma_32x32x16(as_bf16x8(fa[buf_][i]), as_bf16x8(fb[buf_][j]), acc[i][j]); \
  } while (0)

    // prologue: k-tiles 0..3 in flight (8 loads each, always issued: the counts stay
    // static); wait for k-tile 0's
#pragma unroll
    for (int t = 0; t < kNB5; ++t) XDNA_G5_LOAD(t);
    lds_dma_wait<8 * (kNB5 - 1)>();
    __builtin_amdgcn_s_barrier();
    XDNA_G5_FRAGS(0, 0, 0);
    constexpr int kMfma = 0x008, kVmemRd = 0x020, kDsRd = 0x100;
    constexpr int kRd = (kModeA == kAlongK ? 4 : 8) + (kModeB == kAlongK ? 4 : 8);
    for (int t = 0; t < ntiles; ++t) {
      // offsets of the DMA of k-tile t + kNB5 (computed among the first k-step's MFMAs,
      // issued after the barrier)
      const int kn = kbeg + min(t + kNB5, ntiles - 1) * kK5;
      int dofs[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dofs[i] = g5_off(oa, i, kn, kend);
        dofs[4 + i] = g5_off(ob, i, kn, kend);
      }
      // k-step 0 of k-tile t: k-step 1's fragments are read meanwhile
      XDNA_G5_FRAGS(1, t, 1);
      XDNA_G5_MFMA(0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        if (i < kRd) __builtin_amdgcn_sched_group_barrier(kDsRd, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // this wave's reads of buffer t are complete, and its loads of k-tile t+1 (two
      // k-tiles, 16 loads, may stay in flight); the barrier makes k-tile t+1 visible and
      // buffer t free
      lds_reads_wait();
      lds_dma_wait<8 * (kNB5 - 2)>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // k-step 1 of k-tile t in 8 slices of two MFMAs, each slice also issuing one DMA of
      // k-tile t + kNB5 (into buffer t % kNB5) and one fragment of k-tile t + 1, k-step 0
      // (past the end: never used); the slices are fenced so that the DMA, which the
      // scheduler cannot group, spreads over the MFMAs instead of delaying the first one
      uint16_t* const nbuf = tbuf(t + kNB5);
#pragma unroll
      for (int sl = 0; sl < 8; ++sl) {
        const int i = sl >> 1, j0 = 2 * (sl & 1);
        acc[i][j0] = mfma_32x32x16(as_bf16x8(fa[1][i]), as_bf16x8(fb[1][j0]), acc[i][j0]);
        acc[i][j0 + 1] = mfma_32x32x16(as_bf16x8(fa[1][i]), as_bf16x8(fb[1][j0 + 1]), acc[i][j0 + 1]);
        if (sl < 4) {
          lds_dma16(oa.rs, nbuf + (4 * wave + sl) * 512, dofs[sl]);
          fa[0][sl] = g5_frag<kModeA>(tbuf(t + 1), wm * 128 + sl * 32, 0, lane);
        } else {
          lds_dma16(ob.rs, nbuf + kTile5 + (4 * wave + sl - 4) * 512, dofs[sl]);
          fb[0][sl - 4] = g5_frag<kModeB>(tbuf(t + 1) + kTile5, wn * 128 + (sl - 4) * 32, 0, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // drain the clamped loads issued past the end before the workgroup can exit
    lds_dma_wait<0>();
#undef XDNA_G5_LOAD
#undef XDNA_G5_FRAGS
#undef XDNA_G5_MFMA
  }
  store_block<4, 4>(g, batch, split, acc, m0 + wm * 128, n0 + wn * 128, lane);
}

// ---------------------------------------------------------------------------------------
// gemm5's tile, DMA plan and LDS layout with v_mfma_f32_16x16x32_bf16.
// The MFMA-bound kernels run at the board's power limit, and the 16x16x32 form costs less
// energy per flop: one wave per SIMD issuing independent MFMAs on random bf16 operands
// sustains 2156 TFLOP/s against 1772 for 32x32x16, and this kernel runs at 2.08 GHz where
// gemm5_kernel runs at 1.79 (counters on config 3's M 8192, N 4096, K 4096 product).  Its
// MFMAs last 16 cycles instead of 32, so every LDS read and DMA is issued after a single
// MFMA: behind a group of MFMAs the same instructions left the pipe idle (44.6 % busy,
// 283.9 us; interleaved one by one, 234.9 us against gemm5's 264.6).
// A fragment (16 rows x 32 k): lane l holds row l % 16, k 8 (l / 16) .. +7: one 16-byte LDS
// read from a k-contiguous tile (row r, piece (l / 16) ^ 2 ((r >> 3) & 1) of the [256][4
// pieces] tile), two transposing reads from a [k][row] tile (g6_frag).  D (16 x 16, 4 fp32 per lane): register i of lane l
// holds D[4 (l / 16) + i][l % 16].  A wave's 128 x 128 is 8 x 8 tiles (64 MFMAs per 32-k
// k-tile, 64 x 4 accumulator registers).  Per k-tile: the first half of its MFMAs, then the
// wait and barrier that publish the next k-tile and free this one's buffer, then the second
// half with the next k-tile's DMA and fragment reads in fenced slices.
// ---------------------------------------------------------------------------------------
// epilogue of 16 x 16 tiles: rows mb + i*16 + 4 (lane / 16) + r, columns nb + j*16 + lane % 16.
// EK, the form fixed at compile time (gemm_epilogue_kind): C with no bias (0: alpha * acc), a
// bias per column (1: Linear's) or any bias form read at run time (2), or the split-K fp32
// partials (3).  Each value is computed as the run-time form would (same products, sums and
// rounding).  One form per kernel: the epilogue is straight-line code run once per tile, and
// the kernel carrying every form was twice the size (a single 256 x 256 tile at K = 32 took
// 15.5 against 8.9 us).
int gemm_epilogue_kind(const GemmArgs& g) {
  if (g.part) return 3;
  if (g.bias_mode == 0 || g.beta == 0.0f) return 0;
  return g.bias_mode == 1 ? 1 : 2;
}

template <int MI, int NJ, int EK>
__device__ inline void store_block16(const GemmArgs& g, int batch, int split, const f32x4_t (&acc)[MI][NJ],
                                     int mb, int nb, int lane) {
  const int lc = lane & 15, lq = lane >> 4;
  if constexpr (EK == 3) {
    float* P = g.part + (int64_t(split) * g.batch + batch) * g.M * g.N;
    const auto prs = __builtin_amdgcn_make_buffer_rsrc(P, 0, g.part_bytes, 0x00020000);
    int noff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = nb + j * 16 + lc;
      noff[j] = n < g.N ? n * 4 : kSkip;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mb + i * 16 + 4 * lq + r;
        const int moff = m < g.M ? m * g.N * 4 : kSkip;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), prs, moff + noff[j], 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  } else {
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(g.c + int64_t(batch) * g.c_batch, 0, g.c_bytes, 0x00020000);
  if constexpr (EK < 2) {
    int noff[NJ];
    float bn[NJ];
    const auto brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(g.bias), 0, EK ? g.bias_bytes : 0,
                                                       0x00020000);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = nb + j * 16 + lc;
      noff[j] = n < g.N ? int(n * g.c_n * 2) : kSkip;
      bn[j] = EK ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, n < g.N ? int(n * g.bias_sn * 2) : kSkip, 0, 0))
                 : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mb + i * 16 + 4 * lq + r;
        const int moff = m < g.M ? int(m * g.c_m * 2) : kSkip;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          float v = g.alpha * acc[i][j][r];
          if (EK) v += g.beta * bn[j];
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), crs, moff + noff[j], 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  }
  const bool bias = g.bias_mode != 0 && g.beta != 0.0f;
  const auto brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(g.bias), 0, bias ? g.bias_bytes : 0,
                                                     0x00020000);
  int noff[NJ], nbo[NJ];
  float bn[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = nb + j * 16 + lc;
    noff[j] = n < g.N ? int(n * g.c_n * 2) : kSkip;
    nbo[j] = n < g.N ? int(n * g.bias_sn * 2) : kSkip;
    bn[j] = bias && g.bias_mode == 1 ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, nbo[j], 0, 0)) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mb + i * 16 + 4 * lq + r;
      const bool mok = m < g.M;
      const int moff = mok ? int(m * g.c_m * 2) : kSkip;
      const int mbo = mok ? int(m * g.bias_sm * 2) : kSkip;
      float bm = 0.0f;
      if (bias && g.bias_mode == 3) bm = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, mbo, 0, 0));
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float v = g.alpha * acc[i][j][r];
        if (bias) {
          float bv = g.bias_mode == 1 ? bn[j] : bm;
          if (g.bias_mode == 2) bv = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, mbo + nbo[j], 0, 0));
          v += g.beta * bv;
        }
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), crs, moff + noff[j], 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// 16 x 32 fragment of a k-contiguous [256][4 pieces] k-tile: rows rb + lane % 16, piece lane / 16
// 16 x 32 fragment of a [k][row] k-tile (row-contiguous operand): two transposing reads.
// In 16-lane group g = lane / 16, lane j supplies (k row 8 g + 4 h + j / 4, rows rb + 4 (j % 4)
// .. +3) and receives row rb + j at k rows 8 g + 4 h .. +3 (h = 0, 1).  Piece q (8 rows) of
// k row kr sits at q ^ (4 (kr & 3) + 2 ((kr >> 3) & 1)): a half-wave's k rows R .. R+3 and
// R+8 .. R+11 fall on 16 distinct 16-byte positions of a 64-bank window.
template <int kMode>
__device__ inline u32x4_t g6_frag(const uint16_t* tile, int rb, int lane) {
  if (kMode == kAlongK) {
    const int r = rb + (lane & 15);
    const int c = (lane >> 4) ^ (2 * ((r >> 3) & 1));
    return *reinterpret_cast<const u32x4_t*>(tile + (r * 4 + c) * 8);
  }
  const int g = lane >> 4, j = lane & 15;
  const int kr = 8 * g + (j >> 2);
  const int rr = rb + 4 * (j & 3);
  const uint16_t* p = tile + (kr * 32 + ((rr >> 3) ^ (4 * (kr & 3) + 2 * ((kr >> 3) & 1)))) * 8 + (rr & 7);
  const g4i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p));
  const g4i16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) g4i16x4*)(p + 4 * 32 * 8));
  const g2u2 a = __builtin_bit_cast(g2u2, lo), b = __builtin_bit_cast(g2u2, hi);
  return u32x4_t{a[0], a[1], b[0], b[1]};
}

template <int kModeA, int kModeB, int EK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm6_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  int tbx, tby;
  gemm_tile_xy(g, tbx, tby);
  const int m0 = tby * kT4, n0 = tbx * kT4;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  const int kbeg = split * g.kt_per * kK4, kend = min(g.K, kbeg + g.kt_per * kK4);
  // an empty split still runs one k-tile: every load past kend is masked to zeros
  const int ntiles = kend > kbeg ? (kend - kbeg + kK5 - 1) / kK5 : 1;
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;

  f32x4_t acc[8][8];
  {
    // one fragment set, each fragment read again for the next k-tile after its last MFMA
    // of this one: rows 0..3 of A and the B columns during the second half, rows 4..7 of A
    // during the next first half.  Both halves run column by column, so a fragment is read
    // at least 16 MFMAs before its first use.
    u32x4_t fa[8], fb[8];
    const G5Operand oa = g5_operand<kModeA, true>(A, g.a_r, g.a_k, m0, g.M, g.K, tid);
    const G5Operand ob = g5_operand<kModeB, true>(B, g.b_r, g.b_k, n0, g.N, g.K, tid);
    auto tbuf = [&](int t) { return smem + (t & (kNB5 - 1)) * 2 * kTile5; };
    auto load = [&](int t) {
      const int k_ = kbeg + min(t, ntiles - 1) * kK5;
      g5_load(tbuf(t), oa, k_, kend, wave);
      g5_load(tbuf(t) + kTile5, ob, k_, kend, wave);
    };
#pragma unroll
    for (int t = 0; t < kNB5; ++t) load(t);
    lds_dma_wait<8 * (kNB5 - 1)>();
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = g6_frag<kModeA>(tbuf(0), wm * 128 + i * 16, lane);
#pragma unroll
    for (int j = 0; j < 8; ++j) fb[j] = g6_frag<kModeB>(tbuf(0) + kTile5, wn * 128 + j * 16, lane);
    // wave-uniform DMA state: resources and the LDS byte address of this wave's first
    // destination block (the loop adds buffer and block offsets as scalar arithmetic)
    const i32x4_t rsa = uniform_rsrc(oa.rs), rsb = uniform_rsrc(ob.rs);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds_w = lds_addr(smem) + uint32_t(4 * wave_u * 512 * 2);
    // k-tile t (kFirst: t == 0, whose MFMAs start the accumulators).  A 16x16x32 MFMA
    // occupies the matrix pipe for 16 cycles, so every LDS read and DMA is issued right
    // after one MFMA (never several after a group): the wave issues them while that MFMA
    // runs and the next MFMA is not held back.
    auto ktile = [&](int t, auto first) {
      constexpr bool kFirst = decltype(first)::value;
      // k of the DMA loads (k-tile t + kNB5): their offsets are formed in the second half
      const int kn = kbeg + min(t + kNB5, ntiles - 1) * kK5;
      const uint32_t m0n = lds_w + uint32_t(((t + kNB5) & (kNB5 - 1)) * 2 * kTile5 * 2);
      // first half (A rows 0..3) column by column; A rows 4..7 of this k-tile are read
      // after the second MFMA of columns 0..3
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mfma16_acc<kFirst>(acc[i][j], fa[i], fb[j]);
          if (i == 1 && j < 4) fa[4 + j] = g6_frag<kModeA>(tbuf(t), wm * 128 + (4 + j) * 16, lane);
          __builtin_amdgcn_sched_barrier(0);
        }
      // this wave's reads of buffer t are complete and its loads of k-tile t+1 have landed
      // (two k-tiles of loads may stay in flight): the barrier publishes k-tile t+1 and
      // frees buffer t
      lds_reads_wait();
      lds_dma_wait<8 * (kNB5 - 2)>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // second half (A rows 4..7) column by column: DMA j of k-tile t+kNB5 after the
      // column's first MFMA, k-tile t+1's A row j (j < 4) after its second, its B column j
      // after the last (the last use of this k-tile's B column j)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mfma16_acc<kFirst>(acc[4][j], fa[4], fb[j]);
        if (j < 4)
          lds_dma16_m0(rsa, m0n + uint32_t(j * 512 * 2), g5_off(oa, j, kn, kend));
        else
          lds_dma16_m0(rsb, m0n + uint32_t((kTile5 + (j - 4) * 512) * 2), g5_off(ob, j - 4, kn, kend));
        __builtin_amdgcn_sched_barrier(0);
        mfma16_acc<kFirst>(acc[5][j], fa[5], fb[j]);
        if (j < 4) fa[j] = g6_frag<kModeA>(tbuf(t + 1), wm * 128 + j * 16, lane);
        __builtin_amdgcn_sched_barrier(0);
        mfma16_acc<kFirst>(acc[6][j], fa[6], fb[j]);
        __builtin_amdgcn_sched_barrier(0);
        mfma16_acc<kFirst>(acc[7][j], fa[7], fb[j]);
        fb[j] = g6_frag<kModeB>(tbuf(t + 1) + kTile5, wn * 128 + j * 16, lane);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    ktile(0, std::true_type{});
    for (int t = 1; t < ntiles; ++t) ktile(t, std::false_type{});
    lds_dma_wait<0>();
  }
  mfma16_fence(acc);
  store_block16<8, 8, EK>(g, batch, split, acc, m0 + wm * 128, n0 + wn * 128, lane);
}

template <int MA, int MB>
bool launch6(dim3 grid, hipStream_t st, const GemmArgs& g) {
  const auto lds = [](const void* f) {
    return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(kGemm5Lds)) == hipSuccess;
  };
  static const bool ok = lds(reinterpret_cast<const void*>(&gemm6_kernel<MA, MB, 0>)) &&
                         lds(reinterpret_cast<const void*>(&gemm6_kernel<MA, MB, 1>)) &&
                         lds(reinterpret_cast<const void*>(&gemm6_kernel<MA, MB, 2>)) &&
                         lds(reinterpret_cast<const void*>(&gemm6_kernel<MA, MB, 3>));
  if (!ok) return false;
  switch (gemm_epilogue_kind(g)) {
    case 0: gemm6_kernel<MA, MB, 0><<<grid, 256, kGemm5Lds, st>>>(g); break;
    case 1: gemm6_kernel<MA, MB, 1><<<grid, 256, kGemm5Lds, st>>>(g); break;
    case 2: gemm6_kernel<MA, MB, 2><<<grid, 256, kGemm5Lds, st>>>(g); break;
    default: gemm6_kernel<MA, MB, 3><<<grid, 256, kGemm5Lds, st>>>(g); break;
  }
  return true;
}

template <int MA, int MB>
bool launch5(dim3 grid, hipStream_t st, const GemmArgs& g) {
  static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm5_kernel<MA, MB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(kGemm5Lds)) == hipSuccess;
  if (!ok) return false;
  gemm5_kernel<MA, MB><<<grid, 256, kGemm5Lds, st>>>(g);
  return true;
}

template <int MA, int MB>
bool launch4(dim3 grid, hipStream_t st, const GemmArgs& g) {
  static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm4_kernel<MA, MB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(kGemm4Lds)) == hipSuccess;
  if (!ok) return false;
  gemm4_kernel<MA, MB><<<grid, 256, kGemm4Lds, st>>>(g);
  return true;
}

std::atomic<int> g_gemm_variant{[] {
  const char* e = std::getenv("XDNA_GEMM_VARIANT");
  return e ? std::atoi(e) : 0;
}()};

// XCD-blocked tile order of the four-wave kernel: 1 (default) on, 0 launch order
// (XDNA_GEMM_XCD at start-up).
std::atomic<int> g_gemm_xcd{[] {
  const char* e = std::getenv("XDNA_GEMM_XCD");
  return e && std::atoi(e) == 0 ? 0 : 1;
}()};

template <int MA>
void launch_b(int mb, dim3 grid, hipStream_t st, const GemmArgs& g) {
  if (mb == kAlongK) gemm_kernel<MA, kAlongK><<<grid, 256, 0, st>>>(g);
  else if (mb == kAlongRow) gemm_kernel<MA, kAlongRow><<<grid, 256, 0, st>>>(g);
  else gemm_kernel<MA, kScalar><<<grid, 256, 0, st>>>(g);
}

// ---------------------------------------------------------------------------------------
// Batched products of small matrices (the style loss's Gram matrices G = F F^T and their
// gradients: C x C outputs over an HW-long k, C x HW and HW x C outputs over a C-long k,
// HW as small as 16 and odd): 64 x 64 output tiles, four waves of 32 x 32 (one 32x32x16
// accumulator each), k-tiles of 64 in LDS ([row][k], pitch 72) with the next k-tile's
// loads in registers during the current one's MFMAs and one barrier per k-tile.  The large
// tiles leave most of such an output empty and the 128 x 128 kernel stages its k-tiles
// without overlap, a memory latency each.  K is split over blockIdx.z while the grid is
// small, into fp32 partials that gemm_reduce_kernel adds in split order.  (A tile's last
// split adding them itself would need a device-scope fence per workgroup, whose L2
// write-back cost more than the separate launch on this multi-XCD part.)
// ---------------------------------------------------------------------------------------
constexpr int kSmT = 64, kSmK = 64, kSmP = 72;
// One operand's 64 x 64 k-tile in registers: 16 elements per thread.  kAlongK: two 16-byte
// vectors (8 k of one row); kAlongRow: two vectors of 8 rows at one k; kScalar: 16 single
// elements, consecutive lanes along the operand's unit-stride direction where it has one.
// Out-of-range elements are zero (no load).
struct SmRegs {
  uint32_t u[8];
};

template <int kMode>
__device__ inline void sm_load(SmRegs& r, const uint16_t* src, int64_t s_r, int64_t s_k, int r0, int rows, int k0,
                               int K, int tid) {
  if (kMode == kAlongK) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * 256;
      const int row = r0 + (i >> 3), k = k0 + (i & 7) * 8;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (row < rows && k < K) {
        const uint16_t* p = src + int64_t(row) * s_r + k;
        if (k + 8 <= K) {
          const uint4 v = *reinterpret_cast<const uint4*>(p);
          w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k + e < K) w[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) r.u[4 * j + q] = w[q];
    }
  } else if (kMode == kAlongRow) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * 256;
      const int k = k0 + (i >> 3), row = r0 + (i & 7) * 8;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (k < K && row < rows) {
        const uint16_t* p = src + int64_t(k) * s_k + row;
        if (row + 8 <= rows) {
          const uint4 v = *reinterpret_cast<const uint4*>(p);
          w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (row + e < rows) w[e >> 1] |= uint32_t(p[e]) << ((e & 1) * 16);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) r.u[4 * j + q] = w[q];
    }
  } else {
    const bool rows_fast = s_r == 1 && s_k != 1;
    uint32_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = tid + j * 256;
      const int rr = rows_fast ? (i & 63) : (i >> 6), kk = rows_fast ? (i >> 6) : (i & 63);
      const int row = r0 + rr, k = k0 + kk;
      const bool ok = row < rows && k < K;
      const uint32_t e = src[ok ? int64_t(row) * s_r + int64_t(k) * s_k : 0];
      v[j] = ok ? e : 0u;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) r.u[q] = v[2 * q] | (v[2 * q + 1] << 16);
  }
}

template <int kMode>
__device__ inline void sm_store(uint16_t* lds, const SmRegs& r, int64_t s_r, int64_t s_k, int tid) {
  if (kMode == kAlongK) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * 256;
      *reinterpret_cast<uint4*>(lds + (i >> 3) * kSmP + (i & 7) * 8) =
          make_uint4(r.u[4 * j], r.u[4 * j + 1], r.u[4 * j + 2], r.u[4 * j + 3]);
    }
  } else if (kMode == kAlongRow) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * 256;
      const int kk = i >> 3, rv = (i & 7) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        lds[(rv + e) * kSmP + kk] = uint16_t((e & 1) ? (r.u[4 * j + (e >> 1)] >> 16) : (r.u[4 * j + (e >> 1)] & 0xFFFF));
    }
  } else {
    const bool rows_fast = s_r == 1 && s_k != 1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = tid + j * 256;
      const int rr = rows_fast ? (i & 63) : (i >> 6), kk = rows_fast ? (i >> 6) : (i & 63);
      lds[rr * kSmP + kk] = uint16_t((j & 1) ? (r.u[j >> 1] >> 16) : (r.u[j >> 1] & 0xFFFF));
    }
  }
}

template <int kModeA, int kModeB>
__global__ __launch_bounds__(256) void gemm_small_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t as[2][kSmT * kSmP];
  __shared__ __attribute__((aligned(16))) uint16_t bs[2][kSmT * kSmP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kSmT, n0 = blockIdx.x * kSmT;
  const int batch = blockIdx.z / g.nsplit, split = blockIdx.z - batch * g.nsplit;
  const int kbeg = split * g.kt_per * kSmK, kend = min(g.K, kbeg + g.kt_per * kSmK);
  const uint16_t* A = g.a + int64_t(batch) * g.a_batch;
  const uint16_t* B = g.b + int64_t(batch) * g.b_batch;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc = zero_acc();
  SmRegs ra, rb;
  if (kbeg < kend) {
    sm_load<kModeA>(ra, A, g.a_r, g.a_k, m0, g.M, kbeg, kend, tid);
    sm_load<kModeB>(rb, B, g.b_r, g.b_k, n0, g.N, kbeg, kend, tid);
    sm_store<kModeA>(as[0], ra, g.a_r, g.a_k, tid);
    sm_store<kModeB>(bs[0], rb, g.b_r, g.b_k, tid);
  }
  __syncthreads();
  int buf = 0;
  for (int k0 = kbeg; k0 < kend; k0 += kSmK) {
    const bool more = k0 + kSmK < kend;
    if (more) {  // the next k-tile's loads fly during this one's MFMAs
      sm_load<kModeA>(ra, A, g.a_r, g.a_k, m0, g.M, k0 + kSmK, kend, tid);
      sm_load<kModeB>(rb, B, g.b_r, g.b_k, n0, g.N, k0 + kSmK, kend, tid);
    }
    const uint16_t* ab = as[buf] + (wm * 32 + lr) * kSmP + lk;
    const uint16_t* bb = bs[buf] + (wn * 32 + lr) * kSmP + lk;
#pragma unroll
    for (int ks = 0; ks < kSmK / 16; ++ks)
      acc = mfma_32x32x16(as_bf16x8(*reinterpret_cast<const uint4*>(ab + ks * 16)),
                          as_bf16x8(*reinterpret_cast<const uint4*>(bb + ks * 16)), acc);
    if (more) {  // the other buffer's last reads ended before the previous barrier
      sm_store<kModeA>(as[buf ^ 1], ra, g.a_r, g.a_k, tid);
      sm_store<kModeB>(bs[buf ^ 1], rb, g.b_r, g.b_k, tid);
    }
    __syncthreads();
    buf ^= 1;
  }

  // the tile, or (split-K) this split's fp32 partial tile
  const f32x16_t out[1][1] = {{acc}};
  store_block<1, 1>(g, batch, split, out, m0 + wm * 32, n0 + wn * 32, lane);
}

template <int MA>
void launch_small_b(int mb, dim3 grid, hipStream_t st, const GemmArgs& g) {
  if (mb == kAlongK) gemm_small_kernel<MA, kAlongK><<<grid, 256, 0, st>>>(g);
  else if (mb == kAlongRow) gemm_small_kernel<MA, kAlongRow><<<grid, 256, 0, st>>>(g);
  else gemm_small_kernel<MA, kScalar><<<grid, 256, 0, st>>>(g);
}

// Small products take gemm_small_kernel: a side of at most 128 or a k of at most 128, and
// a k up to 8192 (XDNA_GEMM_SMALL=0 at start-up, or xdna_gemm_set_small(0), turns it off).
std::atomic<int> g_gemm_small{[] {
  const char* e = std::getenv("XDNA_GEMM_SMALL");
  return e && std::atoi(e) == 0 ? 0 : 1;
}()};

// Device scratch of xdna_gemm_bf16_noalloc: its split-K partials live here instead of in
// blocks of the caching allocator.  Each GPU the library runs on holds its own copy until
// the process ends; host code reaches it only through the per-device address that
// hipGetSymbolAddress returns (the array's name is a host-side stand-in, not a device
// address).  Every split writes all of its slab before the reduce reads it, so nothing
// has to be cleared between calls.
static __device__ __align__(256) float scratch[XDNA_GEMM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxScratchDevices] = {};

// The current device's copy of `scratch`, looked up once per device with that device
// current.  NULL (error set) when the lookup fails.
float* scratch_of_current_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    launch_failed("xdna_gemm_bf16_noalloc: hipGetDevice", e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("xdna_gemm_bf16_noalloc: device index beyond the scratch table");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      launch_failed("xdna_gemm_bf16_noalloc: hipGetSymbolAddress(scratch)", e != hipSuccess ? e : hipErrorUnknown);
      return nullptr;
    }
    g_scratch[dev] = static_cast<float*>(p);
  }
  return g_scratch[dev];
}

// Where one call's split-K partials come from: the caching allocator (xdna_gemm_bf16) or
// the fixed device scratch (xdna_gemm_bf16_noalloc, `scratch` non-null).
struct PartialsSource {
  const char* who;
  float* scratch;
  float* take(size_t bytes) const {
    if (!scratch) return static_cast<float*>(xdna_hip_cache_alloc(bytes));
    if (bytes > size_t(XDNA_GEMM_NOALLOC_SCRATCH_BYTES)) {
      set_error(std::string(who) + ": the split-K partials of this product need " + std::to_string(bytes) +
                " bytes, above the " + std::to_string(size_t(XDNA_GEMM_NOALLOC_SCRATCH_BYTES)) +
                "-byte scratch (use xdna_gemm_bf16)");
      return nullptr;
    }
    return scratch;
  }
  // stream-ordered reuse: the next user of a cache block runs after the reduce
  void give_back(float* p) const {
    if (!scratch && p) xdna_hip_cache_free(p);
  }
};

int gemm_run(const PartialsSource& src, const uint16_t* A, const uint16_t* Bm, uint16_t* C,
             const uint16_t* bias, int batch, int M, int N, int K, int64_t lda_m, int64_t lda_k,
             int64_t stride_a, int64_t ldb_k, int64_t ldb_n, int64_t stride_b, int64_t ldc_m,
             int64_t ldc_n, int64_t stride_c, int bias_mode, int64_t bias_sm, int64_t bias_sn,
             float alpha, float beta, void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0 || bias_mode < 0 || bias_mode > 3 ||
      (bias_mode && !bias)) {
    set_error(std::string(src.who) + ": invalid arguments");
    return -1;
  }
  if (batch == 0 || M == 0 || N == 0) return 0;
  if (batch > 65535) {
    set_error(std::string(src.who) + ": batch too large");
    return -1;
  }
  GemmArgs g;
  g.xcd_group = 0;
  g.a = A;
  g.b = Bm;
  g.c = C;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.a_r = lda_m;
  g.a_k = lda_k;
  g.a_batch = stride_a;
  g.b_r = ldb_n;  // B is staged as [n][k]
  g.b_k = ldb_k;
  g.b_batch = stride_b;
  g.c_m = ldc_m;
  g.c_n = ldc_n;
  g.c_batch = stride_c;
  g.bias_mode = bias_mode;
  g.bias_sm = bias_sm;
  g.bias_sn = bias_sn;
  g.alpha = alpha;
  g.beta = beta;
  {
    // byte extents of one batch element's C, bias and partials: the buffer-resource
    // epilogue needs every offset below kSkip (else the per-element form runs)
    const auto ext = [](int64_t rows, int64_t s_r, int64_t cols, int64_t s_c) {
      return ((rows - 1) * s_r + (cols - 1) * s_c + 1) * 2;
    };
    const int64_t cb = ext(M, ldc_m, N, ldc_n);
    int64_t bb = 0;
    bool nonneg = ldc_m >= 0 && ldc_n >= 0;
    if (bias_mode == 1) bb = ext(1, 0, N, bias_sn), nonneg = nonneg && bias_sn >= 0;
    if (bias_mode == 2) bb = ext(M, bias_sm, N, bias_sn), nonneg = nonneg && bias_sm >= 0 && bias_sn >= 0;
    if (bias_mode == 3) bb = ext(M, bias_sm, 1, 0), nonneg = nonneg && bias_sm >= 0;
    const int64_t pb = int64_t(M) * N * 4;
    g.rs_ok = nonneg && cb < kSkip && bb < kSkip && pb < kSkip ? 1 : 0;
    g.c_bytes = int(std::min<int64_t>(cb, kSkip));
    g.bias_bytes = int(std::min<int64_t>(bb, kSkip));
    g.part_bytes = int(std::min<int64_t>(pb, kSkip));
  }
  const int ma = stage_mode(A, lda_m, lda_k, stride_a, batch);
  const int mb = stage_mode(Bm, ldb_n, ldb_k, stride_b, batch);
  if (!admit_launch("xdna_gemm_bf16")) return -1;
  g.batch = batch;
  // (two element-staged operands with a short k stay on the 128 x 128 tiles, which read each
  // element fewer times: 15 against 22 us for the style loss's 256-channel Gram product)
  if (g_gemm_small.load() && g_gemm_variant.load() == 0 && g.rs_ok && K > 0 && K <= 8192 &&
      (M <= 128 || N <= 128 || K <= 128) && !(ma == kScalar && mb == kScalar && K <= 128)) {
    // small products (gemm_small_kernel): K split while the grid is below two workgroups
    // per CU, each split keeping at least two k-tiles
    const int64_t tiles = ceil_div(M, kSmT) * ceil_div(N, kSmT) * int64_t(batch);
    const int ktiles = int(ceil_div(K, kSmK));
    int nsplit = 1;
    if (tiles < 256 && ktiles >= 4)
      nsplit = int(std::max<int64_t>(1, std::min<int64_t>({ceil_div(512, tiles), int64_t(ktiles / 2),
                                                           int64_t(65535 / std::max(batch, 1))})));
    g.kt_per = int(ceil_div(ktiles, nsplit));
    g.nsplit = int(ceil_div(ktiles, g.kt_per));
    g.part = nullptr;
    if (g.nsplit > 1) {
      g.part = src.take(size_t(g.nsplit) * size_t(batch) * size_t(M) * size_t(N) * sizeof(float));
      if (!g.part) return -1;
    }
    const dim3 grid(unsigned(ceil_div(N, kSmT)), unsigned(ceil_div(M, kSmT)), unsigned(batch * g.nsplit));
    hipStream_t sts = as_stream(stream);
    if (ma == kAlongK) launch_small_b<kAlongK>(mb, grid, sts, g);
    else if (ma == kAlongRow) launch_small_b<kAlongRow>(mb, grid, sts, g);
    else launch_small_b<kScalar>(mb, grid, sts, g);
    if (g.nsplit > 1) {
      launch_gemm_reduce(g, sts);
      src.give_back(g.part);  // stream-ordered reuse: the next user of the block runs after the reduce
    }
    return check_launch(src.who);
  }
  hipStream_t st2 = as_stream(stream);
  // Large tiles (256 x 256) when neither operand needs scalar staging and the grid still
  // has enough tiles: the four-wave kernel where its whole-vector loads fit the shape, else
  // the eight-wave one; xdna_gemm_set_variant overrides (1 small, 2 eight-wave, 3 four-wave,
  // 4 four-wave with direct-to-LDS loads).
  const int variant = g_gemm_variant.load();
  const int64_t tiles2 = ceil_div(N, kT2) * ceil_div(M, kT2) * int64_t(batch);
  const bool vec_ok = ma != kScalar && mb != kScalar;
  // buffer-resource offsets are 32-bit: each operand (one batch element) under 2 GiB
  const auto extent = [](int rows, int64_t s_r, int64_t s_k, int k) {
    return ((int64_t(rows) - 1) * s_r + (int64_t(k) - 1) * s_k + 1) * 2;
  };
  const bool fits4 = vec_ok && K > 0 && (K % 8) == 0 && (ma != kAlongRow || (M % 8) == 0) &&
                     (mb != kAlongRow || (N % 8) == 0) && extent(M, lda_m, lda_k, K) < (int64_t(1) << 31) &&
                     extent(N, ldb_n, ldb_k, K) < (int64_t(1) << 31);
  // Large tiles when the grid has enough of them, or when a long K can be split into
  // enough work (Gram-like products: measured 1.5x the small kernel at K = 51840).  The
  // four-wave kernel's longer prologue (one wave per SIMD) pays off from K = 1024 on
  // config 3's GEMMs (even there, ahead of the eight-wave kernel from K = 4096).
  const bool big = tiles2 >= 64 || K >= 16384;
  const bool use4 = fits4 && g.rs_ok && (variant == 3 || variant == 4 || variant == 5 || (variant == 0 && big && K >= 1024));
  // the direct-to-LDS form for every operand layout (config 3's nine products: 1441 against
  // 1502 us for the register-staged form, 1-7 % ahead on each, same bits); variant 3 keeps
  // the register-staged one
  const bool use5 = use4 && (variant == 4 || variant == 5 || variant == 0);
  // 16x16x32 MFMAs for every operand layout (config 3's nine products: 1284.6 against
  // 1352.2 us for the 32x32x16 form on one box, 0-8 % ahead on each but one level; same
  // bits); variant 4 keeps the 32x32x16 form
  const bool use6 = use5 && (variant == 5 || variant == 0);
  if (vec_ok && K > 0 && (use4 || variant == 2 || (variant == 0 && big))) {
    // split K while the grid is below the CU count (fp32 partials, fixed-order reduce)
    const int kt2 = int(ceil_div(K, kK2));
    g.nsplit = 1;
    g.kt_per = std::max(kt2, 1);
    g.part = nullptr;
    if (tiles2 < 256 && kt2 >= 8) {
      int sp = int(std::min<int64_t>(kt2 / 4, ceil_div(256, tiles2)));
      sp = std::max(1, std::min(sp, 65535 / std::max(batch, 1)));
      g.kt_per = int(ceil_div(kt2, sp));
      g.nsplit = int(ceil_div(kt2, g.kt_per));
    }
    if (g.nsplit > 1) {
      g.part = src.take(size_t(g.nsplit) * size_t(batch) * size_t(M) * size_t(N) * sizeof(float));
      if (!g.part) return -1;
    }
    const dim3 grid2(unsigned(ceil_div(N, kT2)), unsigned(ceil_div(M, kT2)), unsigned(batch * g.nsplit));
    bool ok;
    if (use4 && g_gemm_xcd.load() && (int64_t(grid2.x) * grid2.y) % kGemmXcds == 0)
      g.xcd_group = int(std::min<unsigned>(grid2.y, 8));
    if (use6) {
      if (ma == kAlongK) ok = mb == kAlongK ? launch6<kAlongK, kAlongK>(grid2, st2, g) : launch6<kAlongK, kAlongRow>(grid2, st2, g);
      else ok = mb == kAlongK ? launch6<kAlongRow, kAlongK>(grid2, st2, g) : launch6<kAlongRow, kAlongRow>(grid2, st2, g);
    } else if (use5) {
      if (ma == kAlongK) ok = mb == kAlongK ? launch5<kAlongK, kAlongK>(grid2, st2, g) : launch5<kAlongK, kAlongRow>(grid2, st2, g);
      else ok = mb == kAlongK ? launch5<kAlongRow, kAlongK>(grid2, st2, g) : launch5<kAlongRow, kAlongRow>(grid2, st2, g);
    } else if (use4) {
      if (ma == kAlongK) ok = mb == kAlongK ? launch4<kAlongK, kAlongK>(grid2, st2, g) : launch4<kAlongK, kAlongRow>(grid2, st2, g);
      else ok = mb == kAlongK ? launch4<kAlongRow, kAlongK>(grid2, st2, g) : launch4<kAlongRow, kAlongRow>(grid2, st2, g);
    } else if (ma == kAlongK) {
      ok = mb == kAlongK ? launch2<kAlongK, kAlongK>(grid2, st2, g) : launch2<kAlongK, kAlongRow>(grid2, st2, g);
    } else {
      ok = mb == kAlongK ? launch2<kAlongRow, kAlongK>(grid2, st2, g) : launch2<kAlongRow, kAlongRow>(grid2, st2, g);
    }
    if (!ok) {
      src.give_back(g.part);
      set_error(std::string(src.who) + ": cannot enable a large-tile kernel's LDS size");
      return -1;
    }
    if (g.nsplit > 1) {
      launch_gemm_reduce(g, st2);
      src.give_back(g.part);
    }
    return check_launch(src.who);
  }
  // Few output tiles and a long K (Gram matrices: [C x HW] x [HW x C]): split K over
  // blockIdx.z so the grid covers the CUs; fp32 partials are summed in split order.
  const int64_t tiles = ceil_div(N, kTN) * ceil_div(M, kTM) * int64_t(batch);
  const int ktiles = int(ceil_div(K, kTK));
  g.nsplit = 1;
  g.kt_per = std::max(ktiles, 1);
  g.part = nullptr;
  if (tiles < 256 && ktiles >= 8) {
    int s = int(std::min<int64_t>(ktiles / 4, ceil_div(512, tiles)));
    s = std::max(1, std::min(s, 65535 / std::max(batch, 1)));
    g.kt_per = int(ceil_div(ktiles, s));
    g.nsplit = int(ceil_div(ktiles, g.kt_per));
  }
  hipStream_t st = as_stream(stream);
  if (g.nsplit > 1) {
    g.part = src.take(size_t(g.nsplit) * size_t(batch) * size_t(M) * size_t(N) * sizeof(float));
    if (!g.part) return -1;
  }
  const dim3 grid(unsigned(ceil_div(N, kTN)), unsigned(ceil_div(M, kTM)), unsigned(batch * g.nsplit));
  if (ma == kAlongK) launch_b<kAlongK>(mb, grid, st, g);
  else if (ma == kAlongRow) launch_b<kAlongRow>(mb, grid, st, g);
  else launch_b<kScalar>(mb, grid, st, g);
  if (g.nsplit > 1) {
    launch_gemm_reduce(g, st);
    src.give_back(g.part);
  }
  return check_launch(src.who);
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" int xdna_gemm_bf16(const uint16_t* A, const uint16_t* Bm, uint16_t* C,
                              const uint16_t* bias, int batch, int M, int N, int K, int64_t lda_m,
                              int64_t lda_k, int64_t stride_a, int64_t ldb_k, int64_t ldb_n,
                              int64_t stride_b, int64_t ldc_m, int64_t ldc_n, int64_t stride_c,
                              int bias_mode, int64_t bias_sm, int64_t bias_sn, float alpha,
                              float beta, void* stream) {
  const PartialsSource src{"xdna_gemm_bf16", nullptr};
  return gemm_run(src, A, Bm, C, bias, batch, M, N, K, lda_m, lda_k, stride_a, ldb_k, ldb_n, stride_b, ldc_m,
                  ldc_n, stride_c, bias_mode, bias_sm, bias_sn, alpha, beta, stream);
}

extern "C" int xdna_gemm_bf16_noalloc(const uint16_t* A, const uint16_t* Bm, uint16_t* C,
                                      const uint16_t* bias, int batch, int M, int N, int K, int64_t lda_m,
                                      int64_t lda_k, int64_t stride_a, int64_t ldb_k, int64_t ldb_n,
                                      int64_t stride_b, int64_t ldc_m, int64_t ldc_n, int64_t stride_c,
                                      int bias_mode, int64_t bias_sm, int64_t bias_sn, float alpha,
                                      float beta, void* stream) {
  float* sp = scratch_of_current_device();
  if (!sp) return -1;
  const PartialsSource src{"xdna_gemm_bf16_noalloc", sp};
  return gemm_run(src, A, Bm, C, bias, batch, M, N, K, lda_m, lda_k, stride_a, ldb_k, ldb_n, stride_b, ldc_m,
                  ldc_n, stride_c, bias_mode, bias_sm, bias_sn, alpha, beta, stream);
}

extern "C" int xdna_gemm_set_small(int on) {
  if (on != 0 && on != 1) {
    set_error("xdna_gemm_set_small: 0 or 1");
    return -1;
  }
  g_gemm_small.store(on);
  return 0;
}

extern "C" int xdna_gemm_set_variant(int variant) {
  if (variant < 0 || variant > 5) {
    set_error("xdna_gemm_set_variant: variant must be 0..5");
    return -1;
  }
  g_gemm_variant.store(variant);
  return 0;
}
