// 3x3 stride-1 pad-1 bf16 convolution on gfx950: forward, dgrad and wgrad as MFMA
// implicit GEMMs with fp32 accumulation and one bf16 rounding.
//
// Forward / dgrad (reference: NPU design xdna_train/_designs/conv3x3w.py:8-29, 155-182
// and runtime torch_xdna_device.cpp:2317-2483, 2515-2522).  The input is the
// reference's packed padded-grid layout [groups][chunks][2126][64] (pack.hip).  For
// output grid row p the 3x3 window is the nine rows p + dy*wp + dx, so
//     out[co][p] = sum_{chunk, tap, c} Wt[co][(chunk*9 + tap)*64 + c] * X[p + off(tap)][c]
// is a GEMM with M = output channels, N = grid rows, K = chunks*9*64.  A workgroup
// owns 128 channels x TP rows of one group; per chunk it stages the TP + 2*wp + 2
// input rows of its window (the halo tile) in LDS once and reads the nine taps as
// shifted row windows of it.  Weights are prepared once per call into the A layout
// [co][chunk][tap][64] (for dgrad with the flip+swap map of conv_pack.cpp:470-473).
// The epilogue adds the bias in fp32, rounds once and writes NCHW directly (the
// reference's unpack, conv_pack.cpp:706-743, fused), 32 consecutive pixels per store.
//
// Wgrad (reference: XdnaConv3x3wDwRuntime::compute, torch_xdna_device.cpp:2683-2751;
// NPU design conv3x3w_dw.py).  Its reduction runs over pixels, so both operands are
// re-laid out channel-major on a padded grid of pitch wp8 = roundup(W+2, 8):
//     XT[ci][q]  = x[b][ci][yy-1][xx-1] at q = (b*(H+2) + yy)*wp8 + xx (zero border)
//     DT[co][p]  = dy[b][co][y][x]      at p = (b*(H+2) + y)*wp8 + x   (zero elsewhere)
//     gw[co][ci][dy][dx] = sum_p DT[co][p] * XT[ci][p + dy*wp8 + dx]
// With wp8 a multiple of 8 the dy shift keeps 16-byte alignment; the dx = 1, 2 shifts
// are built in registers from one 16-byte and one 4-byte LDS read (alignbit), so the
// staged window serves all nine taps.  Pixels are split across workgroups (split-K);
// partial sums go to a workspace and a second kernel adds them in a fixed order, so
// every call returns the same bits.  The bias gradient rides along in the
// first channel tile.
#include "common.h"
#include "mfma.h"
#include "../../include/xdna_hip.h"

#include <algorithm>
#include <atomic>
#include <utility>
#include <type_traits>
#include <cstdlib>

namespace xdna {
namespace {

constexpr int kTCo = 128;            // output channels per workgroup
constexpr int kPitch = 72;           // LDS row pitch (elements) of 64-wide tiles
constexpr int kMaxHalo = 2 * (kMaxWidth + 4) + 2;  // 2*wp + 2 for wp <= 38 -> 78

inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// ---------------------------------------------------------------------------------
// Weight preparation: OIHW bf16 -> Wt[co_pad][chunks*9*64] (k order chunk, tap, c).
// dgrad: the conv of dY (cin' = Cout channels) with w'[ci][co][t] = w[co][ci][8-t].
// ---------------------------------------------------------------------------------
// Both prepared forms from one read of the weight: a workgroup takes a block of CO output
// x 64 input channels of the OIHW weight (CO rows of 64 x 9 contiguous elements, read with
// 16-byte loads where the rows allow) into LDS, then writes the forward form's CO rows
// [tap][64 ci] of chunk ci0 / 64 and the input-gradient form's 64 rows [tap][CO co] (taps
// flipped) of chunk co0 / 64, each in 16-byte stores.  Blocks cover the padded extents of
// both forms; elements outside Cout x Cin are zeros.  wt or wtd may be null (that form is
// not written).  CO is 32 for weights that give a full grid of such blocks and 8 (a quarter
// of the work per workgroup, four times the workgroups) for smaller ones, whose time is the
// latency of one block.  (The element-per-thread form spent most of its time in 64-bit
// index divisions and 18-byte-strided gathers: up to 17 us for a 512-channel weight.)
constexpr int kPrepCi = 64, kPrepRow = kPrepCi * 9;  // 576 elements per block row

// one block (input channels [ci0, ci0 + 64), output channels [co0, co0 + CO)) of both forms
template <int CO>
__device__ inline void prep_block(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                  uint16_t* __restrict__ wtd, int Cout, int Cin, int co_pad_f, int chunks_f,
                                  int co_pad_d, int chunks_d, int vec, int ci0, int co0, uint16_t* tile) {
  constexpr int NT = CO * 8;  // threads
  const int tid = threadIdx.x;
  const bool full = vec && ci0 + kPrepCi <= Cin && co0 + CO <= Cout;
  if (full) {
    // CO rows x 72 pieces of 16 bytes, each row starting at a 16-byte boundary (Cin % 8 == 0)
#pragma unroll
    for (int e = tid; e < CO * (kPrepRow / 8); e += NT) {
      const int r = e / (kPrepRow / 8), q = e - r * (kPrepRow / 8);
      const uint4 v = *reinterpret_cast<const uint4*>(w + (int64_t(co0 + r) * Cin + ci0) * 9 + q * 8);
      *reinterpret_cast<uint4*>(tile + r * kPrepRow + q * 8) = v;
    }
  } else if (co0 < Cout && ci0 < Cin) {
    // a block at the weight's edge: element loads, 8 per thread in flight per round
    for (int e0 = tid * 8; e0 < CO * kPrepRow; e0 += NT * 8) {
      uint16_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + j, r = e / kPrepRow, q = e - r * kPrepRow;
        const int co = co0 + r, ci = ci0 + q / 9;
        v[j] = co < Cout && ci < Cin ? w[(int64_t(co) * Cin + ci) * 9 + q % 9] : uint16_t(0);
      }
      *reinterpret_cast<uint4*>(tile + e0) = make_uint4(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
                                                         v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16));
    }
  } else {
    // only padding: zeros, no loads
    for (int e0 = tid * 8; e0 < CO * kPrepRow; e0 += NT * 8)
      *reinterpret_cast<uint4*>(tile + e0) = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  // forward form: row co, k = (chunk ci0 / 64, tap, c); 8 consecutive c per store
  if (wt && co0 < co_pad_f && ci0 < chunks_f * kKStep) {
    for (int e = tid; e < CO * 72; e += NT) {
      const int r = e / 72, q = e - r * 72;
      const int tap = q >> 3, c0 = (q & 7) * 8;
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        u[j] = uint32_t(tile[r * kPrepRow + (c0 + 2 * j) * 9 + tap]) |
               (uint32_t(tile[r * kPrepRow + (c0 + 2 * j + 1) * 9 + tap]) << 16);
      uint16_t* dst = wt + (int64_t(co0 + r) * chunks_f + ci0 / kKStep) * kPrepRow + tap * kKStep + c0;
      *reinterpret_cast<uint4*>(dst) = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
  // input-gradient form: row ci, k = (chunk co0 / 64, tap, co), w'[ci][co][t] = w[co][ci][8 - t]
  if (wtd && ci0 < co_pad_d && co0 < chunks_d * kKStep) {
    const int cb = co0 % kKStep;  // this block's CO-channel part of the chunk
    for (int e = tid; e < kPrepCi * 9 * (CO / 8); e += NT) {
      const int r = e / (9 * (CO / 8)), q = e - r * (9 * (CO / 8));
      const int tap = q / (CO / 8), c0 = (q % (CO / 8)) * 8;
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        u[j] = uint32_t(tile[(c0 + 2 * j) * kPrepRow + r * 9 + (8 - tap)]) |
               (uint32_t(tile[(c0 + 2 * j + 1) * kPrepRow + r * 9 + (8 - tap)]) << 16);
      uint16_t* dst = wtd + (int64_t(ci0 + r) * chunks_d + co0 / kKStep) * kPrepRow + tap * kKStep + cb + c0;
      *reinterpret_cast<uint4*>(dst) = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
}

template <int CO>
__global__ __launch_bounds__(CO * 8) void prep_tiled_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                            uint16_t* __restrict__ wtd, int Cout, int Cin, int co_pad_f,
                                                            int chunks_f, int co_pad_d, int chunks_d, int vec) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[CO * kPrepRow];  // [co_l][ci_l * 9 + tap]
  prep_block<CO>(w, wt, wtd, Cout, Cin, co_pad_f, chunks_f, co_pad_d, chunks_d, vec, blockIdx.x * kPrepCi,
                 blockIdx.y * CO, tile);
}

// Several weights' forms in one launch (the optimizer step's refresh of every conv weight
// it wrote): job e owns blocks [block0, next job's block0), gx input-channel blocks per
// row of 8-output-channel blocks, as prep_tiled_kernel<8>'s grid.
constexpr int kPrepJobs = 32;
struct PrepJob {
  const uint16_t* w;
  uint16_t* wt;
  uint16_t* wtd;
  int Cout, Cin, co_pad_f, chunks_f, co_pad_d, chunks_d, gx, vec, block0;
};
struct PrepJobs {
  PrepJob j[kPrepJobs];
  int n;
};

__global__ __launch_bounds__(64) void prep_multi_kernel(PrepJobs jobs) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[8 * kPrepRow];
  const int bid = blockIdx.x;
  int e = 0;
  while (e + 1 < jobs.n && bid >= jobs.j[e + 1].block0) ++e;
  const PrepJob& J = jobs.j[e];
  const int lb = bid - J.block0;
  const int cy = lb / J.gx, cx = lb - cy * J.gx;
  prep_block<8>(J.w, J.wt, J.wtd, J.Cout, J.Cin, J.co_pad_f, J.chunks_f, J.co_pad_d, J.chunks_d, J.vec, cx * kPrepCi,
                cy * 8, tile);
}

// ---------------------------------------------------------------------------------
// Implicit GEMM on packed rows.
// ---------------------------------------------------------------------------------
struct RowsArgs {
  const uint16_t* xp;    // [groups][chunks][2126][64]
  const uint16_t* xsrc;  // NCHW [B][cin][H][W] (the small-grid kernel's NCHW form), else null
  int cin;               // input channels (NCHW form)
  const uint16_t* wt;    // [co_pad][K]
  const uint16_t* bias;  // [cout] or null
  uint16_t* out;         // NCHW [B][cout][H][W]
  float* part;           // split-K: fp32 partial sums [nsplit][cout][m_pad], else null
  int chunks, cout, wp, H, W, S, So;
  int first;             // output row position of output column 0 (the layout's)
  int ch_per;            // input chunks per split (blockIdx.z)
  int nrt, ncot;         // row tiles, channel tiles (blockIdx.x decodes to both)
  int64_t img, m_total, m_pad;
  int B;                 // images
  int out_rs;            // 1: stores through a buffer resource (every tile's span < 2^30 bytes)
  int bias_vec;          // 1: bias 8-byte aligned and cout % 4 == 0 (4-channel vector loads)
  int act;               // epilogue activation: 0 none, 1 ReLU
  // Output image: oH x oW.  osh = 0: the conv's own H x W.  osh = 1: the forward of a
  // 3x3 / stride-2 / pad-1 conv, ceil(H/2) x ceil(W/2): only grid pixels at even (y, x)
  // are stored, at (y/2, x/2) (the buffer-store epilogues and the split-K reduce).
  int osh, oH, oW;
};

// The epilogue's activation, applied to the fp32 sum before its one rounding.  ReLU keeps
// NaN and maps -0 to +0 (PyTorch's relu); rounding is monotonic and keeps the sign, so
// bf16(relu(v)) equals relu(bf16(v)) bit for bit: the fused result is the unfused one.
__device__ inline float rows_act(const RowsArgs& a, float v) { return a.act && v <= 0.0f ? 0.0f : v; }
// rows_act with the activation fixed at compile time (ReLU when kRelu)
template <bool kRelu>
__device__ inline float rows_act_c(float v) { return kRelu && v <= 0.0f ? 0.0f : v; }

// Branch-free NCHW epilogue.  The resource starts at the first image a tile touches; a
// store whose pixel or channel lies outside the output gets an offset of kOutSkip or more,
// past the resource's record count, and the hardware drops it, so no store waits behind a
// branch.  Valid offsets stay below kOutSkip (checked on the host), so the sum of a valid
// and a skipped part, or of two skipped parts, is dropped too.
constexpr int kOutSkip = 0x40000000;

struct OutMap {
  __amdgpu_buffer_rsrc_t rs;
  int b0;
  int64_t cp;  // elements of one image (cout * H * W)
};

__device__ inline OutMap out_map(const RowsArgs& a, int64_t p_first) {
  OutMap o;
  o.b0 = int(p_first / a.img / a.S);
  o.cp = int64_t(a.cout) * a.oH * a.oW;
  const int64_t left = (int64_t(a.B) - o.b0) * o.cp * 2;
  o.rs = __builtin_amdgcn_make_buffer_rsrc(a.out + o.b0 * o.cp, 0, int(left < kOutSkip ? left : kOutSkip - 1),
                                           0x00020000);
  return o;
}

// byte offset of padded-grid row p's output pixel (channel 0) from the map's base, or
// kOutSkip for a border / padding row; 32-bit arithmetic (grids of fewer than 2^31 rows,
// checked on the host with the map's 1 GiB span)
__device__ inline int out_pixel_off32(const RowsArgs& a, const OutMap& o, int p) {
  if (p >= int(a.m_total)) return kOutSkip;
  const int img = int(a.img);
  const int vb = p / img;
  const int rem = p - vb * img;
  const int y = rem / a.wp;
  const int col = rem - y * a.wp - a.first;
  const int b = a.S == 1 ? vb : vb / a.S, s = vb - b * a.S;
  const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
  if (y >= a.H || col < 0 || col >= cols) return kOutSkip;
  const int x = (a.S == 1 ? 0 : s * a.So) + col;
  if ((y | x) & a.osh) return kOutSkip;
  return ((b - o.b0) * int(o.cp) + (y >> a.osh) * a.oW + (x >> a.osh)) * 2;
}

constexpr int kXcds = 8;  // MI355X: workgroups go round-robin to 8 XCDs, each with its own L2

// blockIdx.x -> (row tile, channel tile).  Workgroup L runs on XCD L % 8; on each XCD the
// consecutive workgroups take all channel tiles of one row tile, so a window read from
// HBM once serves every channel tile from that XCD's L2 (row tile r lives on XCD r % 8;
// nrt is padded to a multiple of 8 in the grid, padding workgroups exit).
__device__ inline bool rows_tile(const RowsArgs& a, int& rt, int& ct) {
  const int L = blockIdx.x;
  const int x = L % kXcds, k = L / kXcds;
  rt = (k / a.ncot) * kXcds + x;
  ct = k % a.ncot;
  return rt < a.nrt;
}

// One workgroup: 128 output channels x TP grid rows of one group; wave (wm, wn) owns
// channels [wm*64, +64) x rows [wn*TP/2, +TP/2) (2 x TP/64 MFMA tiles).  Per input chunk
// the TP + 2*wp + 2 rows of the halo window sit in LDS (double-buffered: the next chunk's
// window is fetched into registers while this one is multiplied, one barrier per chunk);
// the nine taps are row offsets into it.  Weight fragments come straight from L2 into
// registers, two taps ahead (they are shared by every workgroup and stay L2-resident).
// The window prefetch is spread over taps 0..6, each slice issued after that tap's weight
// loads: the memory counter is in order, so a weight load never waits on a window load
// issued less than three taps earlier.  blockIdx.z selects a range of ch_per input chunks
// (split-K for small grids); a split writes fp32 partial sums for rows_reduce_kernel.
template <int TP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void conv_rows_kernel(RowsArgs a) {
  constexpr int kXRows = TP + kMaxHalo;
  constexpr int NT = TP / 64;                       // 32-row MFMA tiles per wave along N
  constexpr int kXv = (kXRows * 8 + 255) / 256;     // window vectors per thread
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kXRows * kPitch];

  constexpr int tiles_per_group = kGroupOutRows / TP;
  int rt, ct;
  if (!rows_tile(a, rt, ct)) return;
  const int g = rt / tiles_per_group;
  const int r0 = (rt % tiles_per_group) * TP;
  if (int64_t(g) * kGroupOutRows + r0 >= a.m_total) return;  // tail tile: no valid row
  const int co0 = ct * kTCo;
  const int ch0 = blockIdx.z * a.ch_per;
  const int ch1 = min(a.chunks, ch0 + a.ch_per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int K = a.chunks * 9 * kKStep;
  const int nvec = (TP + 2 * a.wp + 2) * 8;         // window vectors actually needed
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  // accumulators start at the bias (fp32), so the epilogue is one rounding and a store
  f32x16_t acc[2][NT];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    f32x16_t init = zero_acc();
    if (a.bias && !a.part) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * 64 + m * 32 + mfma_row(i, lane);
        init[i] = co < a.cout ? bf16_to_f32(a.bias[co]) : 0.0f;
      }
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = init;
  }

  // weight fragments of (chunk, tap): rows co0 + wm*64 + m*32 + lr, k = (ch*9+tap)*64 + ks*16 + lk
  const uint16_t* wrow0 = a.wt + int64_t(co0 + wm * 64 + lr) * K + lk;
  const uint16_t* wrow1 = wrow0 + int64_t(32) * K;
  u32x4_t wa[3][2][4];   // [set][m][ks]: tap t uses set t % 3 (9 taps per chunk keep the rotation)
  u32x4_t xr[kXv];

#define XDNA_ROWS_LOADW(set_, ch_, tap_)                                                     \
  do {                                                                                       \
    const int kb_ = ((ch_) * 9 + (tap_)) * kKStep;                                           \
    _Pragma("unroll") for (int ks = 0; ks < 4; ++ks) {                                       \
      wa[set_][0][ks] = *reinterpret_cast<const u32x4_t*>(wrow0 + kb_ + ks * 16);            \
      wa[set_][1][ks] = *reinterpret_cast<const u32x4_t*>(wrow1 + kb_ + ks * 16);            \
    }                                                                                        \
  } while (0)
// window vectors j with j * 7 / kXv == part_ (part_ < 0: all of them)
#define XDNA_ROWS_LOADX(ch_, part_)                                                          \
  do {                                                                                       \
    const uint16_t* src_ = a.xp + ((int64_t(g) * a.chunks + (ch_)) * kGroupRows + r0) * kKStep; \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j) {                                        \
      const int i = tid + j * 256;                                                           \
      if (((part_) < 0 || j * 7 / kXv == (part_)) && i < nvec)                               \
        xr[j] = *reinterpret_cast<const u32x4_t*>(src_ + (i >> 3) * kKStep + (i & 7) * 8);   \
    }                                                                                        \
  } while (0)
#define XDNA_ROWS_STOREX(buf_)                                                               \
  do {                                                                                       \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j) {                                        \
      const int i = tid + j * 256;                                                           \
      if (i < nvec) *reinterpret_cast<u32x4_t*>(&xs[buf_][(i >> 3) * kPitch + (i & 7) * 8]) = xr[j]; \
    }                                                                                        \
  } while (0)

  // weights two taps ahead
  XDNA_ROWS_LOADW(0, ch0, 0);
  XDNA_ROWS_LOADW(1, ch0, 1);
  XDNA_ROWS_LOADX(ch0, -1);
  XDNA_ROWS_STOREX(0);
  __syncthreads();

  for (int ch = ch0; ch < ch1; ++ch) {
    const int cur = (ch - ch0) & 1;
    const bool more = ch + 1 < ch1;
    const uint16_t* xb = &xs[cur][(wn * (TP / 2) + lr) * kPitch + lk];
    // B fragments are software-pipelined one 16-wide k-step ahead (36 steps per chunk:
    // 9 taps x 4), so LDS latency hides behind the 2*NT MFMAs of the current step.
    u32x4_t bq[2][NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
      bq[0][n] = *reinterpret_cast<const u32x4_t*>(xb + n * 32 * kPitch);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int set = tap % 3;
      // weights of tap + 2 first, so the window prefetch below can stay in flight
      if (tap < 7) {
        XDNA_ROWS_LOADW((tap + 2) % 3, ch, tap + 2);
      } else if (more) {
        XDNA_ROWS_LOADW((tap + 2) % 3, ch + 1, tap - 7);
      }
      if (tap < 7 && more) XDNA_ROWS_LOADX(ch + 1, tap);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int step = tap * 4 + ks;
        if (step + 1 < 36) {
          const int ntap = (step + 1) >> 2, nks = (step + 1) & 3;
          const int noff = ((ntap / 3) * a.wp + (ntap % 3)) * kPitch + nks * 16;
#pragma unroll
          for (int n = 0; n < NT; ++n)
            bq[(step + 1) & 1][n] = *reinterpret_cast<const u32x4_t*>(xb + noff + n * 32 * kPitch);
        }
        // keep the next step's LDS reads ahead of this step's MFMAs (the scheduler would
        // otherwise sink each read next to its use and expose its latency)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const bf16x8_t bfr = as_bf16x8(bq[step & 1][n]);
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m][n] = mfma_32x32x16(as_bf16x8(wa[set][m][ks]), bfr, acc[m][n]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (more) XDNA_ROWS_STOREX(cur ^ 1);
    __syncthreads();
  }
#undef XDNA_ROWS_LOADW
#undef XDNA_ROWS_LOADX
#undef XDNA_ROWS_STOREX

  if (a.part) {
    // split-K: fp32 partial sums, rows of 32 consecutive grid rows per store
    float* pz = a.part + int64_t(blockIdx.z) * a.cout * a.m_pad;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * (TP / 2) + n * 32 + lr;
      if (p >= a.m_total) continue;
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int co = co0 + wm * 64 + m * 32 + mfma_row(i, lane);
          if (co < a.cout) pz[int64_t(co) * a.m_pad + p] = acc[m][n][i];
        }
    }
    return;
  }

  // Epilogue: grid row -> NCHW pixel, one rounding; lanes 0..31 store 32 consecutive
  // grid rows (mostly consecutive image columns) of one channel.
  const int first = a.first;
  const int64_t plane = int64_t(a.H) * a.W;
  uint16_t* obase[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    obase[n] = nullptr;
    const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * (TP / 2) + n * 32 + lr;
    if (p >= a.m_total) continue;
    const int64_t vb = p / a.img;
    const int64_t rem = p - vb * a.img;
    const int y = int(rem / a.wp);
    const int col = int(rem - int64_t(y) * a.wp) - first;
    if (y >= a.H || col < 0) continue;
    const int b = int(vb / a.S), s = int(vb % a.S);
    const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
    if (col >= cols) continue;
    const int x = (a.S == 1 ? 0 : s * a.So) + col;
    obase[n] = a.out + int64_t(b) * a.cout * plane + int64_t(y) * a.W + x;
  }
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 64 + m * 32 + mfma_row(i, lane);
      if (co >= a.cout) continue;
#pragma unroll
      for (int n = 0; n < NT; ++n)
        if (obase[n]) obase[n][int64_t(co) * plane] = f32_to_bf16(rows_act(a, acc[m][n][i]));
    }
}

// Wide variant for cout >= 256: 256 output channels x 256 grid rows per workgroup, 8 waves
// (two per SIMD, so one wave's MFMAs run while the other waits).  Wave (wm, wn) owns
// channels [wm*64, +64) x rows [wn*128, +128): 2 x 4 MFMA tiles per 16-wide k-step.
// Both operands come from LDS: the chunk's halo window (single buffer, the next chunk's
// window prefetched into registers over taps 0..6) and the weights of one (chunk, tap)
// slab at a time in a 3-slot ring.  Slab T is loaded into registers at tap T-2 (16-byte
// coalesced loads, 256 rows x 128 bytes), stored to slot T % 3 at the start of tap T-1
// and read at tap T; a barrier opens every tap.  Fragments are read right before their
// MFMAs: the other wave of the SIMD covers the LDS latency.  Needs prepared weights
// padded to a multiple of 256 rows (fwd_plan pads so for cout > 128).
constexpr int kWCo = 256;                              // output channels per workgroup
constexpr int kWTp = 256;                              // grid rows per workgroup
constexpr int kWXRows = kWTp + kMaxHalo;
constexpr int kWSlot = kWCo * kPitch;                  // elements of one weight slot
constexpr size_t kWideLds = size_t(kWXRows * kPitch + 3 * kWSlot) * 2;

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void conv_rows2_kernel(RowsArgs a) {
  constexpr int kXv = (kWXRows * 8 + 511) / 512;       // window vectors per thread (6)
  constexpr int kWv = kWCo * 8 / 512;                  // weight vectors per thread per slab (4)
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs = smem;                                 // [kWXRows][kPitch]
  uint16_t* wsl = smem + kWXRows * kPitch;             // [3][kWCo][kPitch]

  constexpr int tiles_per_group = kGroupOutRows / kWTp;
  int rt, ct;
  if (!rows_tile(a, rt, ct)) return;
  const int g = rt / tiles_per_group;
  const int r0 = (rt % tiles_per_group) * kWTp;
  if (int64_t(g) * kGroupOutRows + r0 >= a.m_total) return;
  const int co0 = ct * kWCo;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int K = a.chunks * 9 * kKStep;
  const int nvec = (kWTp + 2 * a.wp + 2) * 8;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  const int T0 = 0, T1 = a.chunks * 9;

  f32x16_t acc[2][4];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    f32x16_t init = zero_acc();
    if (a.bias) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * 64 + m * 32 + mfma_row(i, lane);
        init[i] = co < a.cout ? bf16_to_f32(a.bias[co]) : 0.0f;
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[m][n] = init;
  }

  // weight slab T: rows co0 .. co0+255, k = [T*64, T*64+64); vector v = row v/8, piece v%8
  const uint16_t* wbase = a.wt + int64_t(co0) * K;
  u32x4_t wreg[kWv];
  u32x4_t xr[kXv];
#define XDNA_W2_LOAD(T_)                                                                     \
  do {                                                                                       \
    _Pragma("unroll") for (int j = 0; j < kWv; ++j) {                                        \
      const int v = tid + j * 512;                                                           \
      wreg[j] = *reinterpret_cast<const u32x4_t*>(wbase + int64_t(v >> 3) * K + (T_) * kKStep + (v & 7) * 8); \
    }                                                                                        \
  } while (0)
#define XDNA_W2_STORE(slot_)                                                                 \
  do {                                                                                       \
    _Pragma("unroll") for (int j = 0; j < kWv; ++j) {                                        \
      const int v = tid + j * 512;                                                           \
      *reinterpret_cast<u32x4_t*>(&wsl[(slot_) * kWSlot + (v >> 3) * kPitch + (v & 7) * 8]) = wreg[j]; \
    }                                                                                        \
  } while (0)
#define XDNA_X2_LOAD(ch_, part_)                                                             \
  do {                                                                                       \
    const uint16_t* src_ = a.xp + ((int64_t(g) * a.chunks + (ch_)) * kGroupRows + r0) * kKStep; \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j) {                                        \
      const int i = tid + j * 512;                                                           \
      if (((part_) < 0 || j * 7 / kXv == (part_)) && i < nvec)                               \
        xr[j] = *reinterpret_cast<const u32x4_t*>(src_ + (i >> 3) * kKStep + (i & 7) * 8);   \
    }                                                                                        \
  } while (0)
#define XDNA_X2_STORE()                                                                      \
  do {                                                                                       \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j) {                                        \
      const int i = tid + j * 512;                                                           \
      if (i < nvec) *reinterpret_cast<u32x4_t*>(&xs[(i >> 3) * kPitch + (i & 7) * 8]) = xr[j]; \
    }                                                                                        \
  } while (0)

  // prologue: slab 0 to slot 0, slab 1 in registers, window of chunk 0 in LDS
  XDNA_W2_LOAD(T0);
  XDNA_X2_LOAD(0, -1);
  XDNA_W2_STORE(0);
  XDNA_X2_STORE();
  if (T0 + 1 < T1) XDNA_W2_LOAD(T0 + 1);

  const uint16_t* xb = xs + (wn * 128 + lr) * kPitch + lk;
  for (int ch = 0; ch < a.chunks; ++ch) {
    const bool more = ch + 1 < a.chunks;
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int T = ch * 9 + tap;
      __syncthreads();  // tap T-1 done everywhere; slot T % 3 and the window are visible
      // slab T+1 (in registers since tap T-1) to its slot (last read at tap T-2), then
      // slab T+2 into the registers
      if (T + 1 < T1) XDNA_W2_STORE((T + 1) % 3);
      if (T + 2 < T1) XDNA_W2_LOAD(T + 2);
      if (tap < 7 && more) XDNA_X2_LOAD(ch + 1, tap);
      const uint16_t* wa = wsl + (T % 3) * kWSlot + (wm * 64 + lr) * kPitch + lk;
      const int toff = ((tap / 3) * a.wp + (tap % 3)) * kPitch;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4_t aq[2], bq[4];
#pragma unroll
        for (int m = 0; m < 2; ++m) aq[m] = *reinterpret_cast<const u32x4_t*>(wa + m * 32 * kPitch + ks * 16);
#pragma unroll
        for (int n = 0; n < 4; ++n) bq[n] = *reinterpret_cast<const u32x4_t*>(xb + toff + n * 32 * kPitch + ks * 16);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const bf16x8_t bfr = as_bf16x8(bq[n]);
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m][n] = mfma_32x32x16(as_bf16x8(aq[m]), bfr, acc[m][n]);
        }
      }
    }
    if (more) {
      __syncthreads();  // every wave is done reading this chunk's window
      XDNA_X2_STORE();
    }
  }
#undef XDNA_W2_LOAD
#undef XDNA_W2_STORE
#undef XDNA_X2_LOAD
#undef XDNA_X2_STORE

  const int first = a.first;
  const int64_t plane = int64_t(a.H) * a.W;
  uint16_t* obase[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    obase[n] = nullptr;
    const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * 128 + n * 32 + lr;
    if (p >= a.m_total) continue;
    const int64_t vb = p / a.img;
    const int64_t rem = p - vb * a.img;
    const int y = int(rem / a.wp);
    const int col = int(rem - int64_t(y) * a.wp) - first;
    if (y >= a.H || col < 0) continue;
    const int b = int(vb / a.S), s = int(vb % a.S);
    const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
    if (col >= cols) continue;
    const int x = (a.S == 1 ? 0 : s * a.So) + col;
    obase[n] = a.out + int64_t(b) * a.cout * plane + int64_t(y) * a.W + x;
  }
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 64 + m * 32 + mfma_row(i, lane);
      if (co >= a.cout) continue;
#pragma unroll
      for (int n = 0; n < 4; ++n)
        if (obase[n]) obase[n][int64_t(co) * plane] = f32_to_bf16(rows_act(a, acc[m][n][i]));
    }
}

// Four-wave kernels: one wave per SIMD, wave (wm, wn) of a WM x (4/WM) grid owning MT*32
// channels x NT*32 rows (MT x NT MFMA tiles, accumulators in the AGPR half of the
// register file).  A workgroup covers CO = WM*MT*32 channels x TP = (4/WM)*NT*32 rows:
//   <4,4,2>  256 channels x 256 rows (cout > 128): a 16-wide k-step reads 8 fragments for
//            16 MFMAs, half the LDS traffic per MFMA of the eight-wave form;
//   <2,4,2>  128 x 256 and <4,4,1> 128 x 512 (cout <= 128), <2,4,1> 64 x 512 (cout <= 64).
// With one wave per SIMD nothing else covers latency, so the kernel pipelines it:
//   * fragments are read one k-step ahead, across tap boundaries too: the slab of tap T+1
//     is in its slot two barriers before the last k-step of tap T reads its first
//     fragments (only a chunk boundary, where the window changes, waits);
//   * the one barrier per tap opens the last k-step, where slab T+3 replaces slab T in
//     LDS; slabs are loaded two taps before they are stored (register set = slab % 3, and
//     9 taps per chunk keep the rotation static);
//   * every LDS access and global load issues between two MFMAs (scheduling groups), so
//     the matrix cores do not idle while the wave issues memory instructions;
//   * every load and store is unconditional (slab and chunk indexes clamped, window rows
//     clamped to the window), so the memory counters the compiler waits on are static.
template <int MT, int NT, int WM>
struct Q4 {
  static constexpr int WN = 4 / WM;
  static constexpr int CO = WM * MT * 32;                    // channels per workgroup
  static constexpr int TP = WN * NT * 32;                    // grid rows per workgroup
  static constexpr int XRows = TP + kMaxHalo;                // window rows
  static constexpr int Slot = CO * kPitch;                   // elements of one weight slot
  static constexpr size_t Lds = size_t(XRows * kPitch + 3 * Slot) * 2;
};

template <int MT, int NT, int WM, int OCC, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
void conv_rows4_kernel(RowsArgs a) {
  using Q = Q4<MT, NT, WM>;
  constexpr int kXv = (Q::XRows * 8 + 255) / 256;      // window vectors per thread
  constexpr int kWv = Q::CO * 8 / 256;                 // weight vectors per thread per slab
  constexpr int kR = MT + NT, kM = MT * NT;            // fragment reads, MFMAs per k-step
  static_assert(kM >= kR && kWv >= 1, "tile too small for the schedule");
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs = smem;                                 // [XRows][kPitch]
  uint16_t* wsl = smem + Q::XRows * kPitch;            // [3][CO][kPitch]

  constexpr int tiles_per_group = kGroupOutRows / Q::TP;
  int rt, ct;
  if (!rows_tile(a, rt, ct)) return;
  const int g = rt / tiles_per_group;
  const int r0 = (rt % tiles_per_group) * Q::TP;
  if (int64_t(g) * kGroupOutRows + r0 >= a.m_total) return;
  const int co0 = ct * Q::CO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int K = a.chunks * 9 * kKStep;
  const int T1 = a.chunks * 9;
  const int nrows = Q::TP + 2 * a.wp + 2;              // window rows (<= XRows)
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    f32x16_t init = zero_acc();
    if (a.bias && a.bias_vec) {
      // a lane's 16 rows are 4 runs of 4 consecutive channels (mfma_row): one 8-byte load
      // per run through a buffer resource (channels past cout read as zero); 2-byte loads
      // per row measured 4.7 % slower over the sweep
      const __amdgpu_buffer_rsrc_t brs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.bias), 0, a.cout * 2, 0x00020000);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int co = co0 + wm * MT * 32 + m * 32 + 8 * q + 4 * (lane >> 5);
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(brs, co * 2, 0, 0));
        init[4 * q + 0] = __uint_as_float(v.x << 16);
        init[4 * q + 1] = __uint_as_float(v.x & 0xFFFF0000u);
        init[4 * q + 2] = __uint_as_float(v.y << 16);
        init[4 * q + 3] = __uint_as_float(v.y & 0xFFFF0000u);
      }
    } else if (a.bias) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * MT * 32 + m * 32 + mfma_row(i, lane);
        init[i] = co < a.cout ? bf16_to_f32(a.bias[co]) : 0.0f;
      }
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = init;
  }

  // weight vector j of a slab: row (tid >> 3) + 32 j, 8-element piece tid & 7
  const uint16_t* wsrc = a.wt + (int64_t(co0) + (tid >> 3)) * K + (tid & 7) * 8;
  const int wdst = (tid >> 3) * kPitch + (tid & 7) * 8;
  // window vector j: row min((tid + 256 j) >> 3, nrows - 1), piece tid & 7
  auto xoff = [&](int j) { return min((tid + j * 256) >> 3, nrows - 1) * 8 + (tid & 7); };
  const uint16_t* xsrc0 = a.xp + (int64_t(g) * a.chunks * kGroupRows + r0) * kKStep;

  u32x4_t wreg[3][kWv];
  u32x4_t xr[kXv];
  u32x4_t fa[2][MT], fb[2][NT];

#define XDNA_W4_LOAD(set_, T_)                                                               \
  do {                                                                                       \
    const uint16_t* s_ = wsrc + int64_t(min((T_), T1 - 1)) * kKStep;                         \
    _Pragma("unroll") for (int j = 0; j < kWv; ++j)                                          \
      wreg[set_][j] = *reinterpret_cast<const u32x4_t*>(s_ + int64_t(j * 32) * K);           \
  } while (0)
#define XDNA_W4_STORE(set_, slot_)                                                           \
  do {                                                                                       \
    uint16_t* d_ = wsl + (slot_) * Q::Slot + wdst;                                           \
    _Pragma("unroll") for (int j = 0; j < kWv; ++j)                                          \
      *reinterpret_cast<u32x4_t*>(d_ + j * 32 * kPitch) = wreg[set_][j];                     \
  } while (0)
// window vectors j of chunk ch_ with j * 7 / kXv == part_ (part_ < 0: all of them)
#define XDNA_X4_LOAD(ch_, part_)                                                             \
  do {                                                                                       \
    const uint16_t* s_ = xsrc0 + int64_t(ch_) * kGroupRows * kKStep;                         \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j)                                          \
      if ((part_) < 0 || j * 7 / kXv == (part_))                                             \
        xr[j] = *reinterpret_cast<const u32x4_t*>(s_ + xoff(j) * 8);                         \
  } while (0)
#define XDNA_X4_STORE()                                                                      \
  do {                                                                                       \
    _Pragma("unroll") for (int j = 0; j < kXv; ++j)                                          \
      *reinterpret_cast<u32x4_t*>(&xs[(xoff(j) >> 3) * kPitch + (xoff(j) & 7) * 8]) = xr[j]; \
  } while (0)
// fragments of (slot_, tap_, ks_) into buffer buf_
#define XDNA_F4_LOAD(buf_, slot_, tap_, ks_)                                                 \
  do {                                                                                       \
    const uint16_t* wa_ = wsl + (slot_) * Q::Slot + (wm * MT * 32 + lr) * kPitch + lk + (ks_) * 16; \
    const uint16_t* xb_ = xs + (wn * NT * 32 + lr + ((tap_) / 3) * a.wp + ((tap_) % 3)) * kPitch + lk + (ks_) * 16; \
    _Pragma("unroll") for (int m = 0; m < MT; ++m)                                           \
      fa[buf_][m] = *reinterpret_cast<const u32x4_t*>(wa_ + m * 32 * kPitch);                \
    _Pragma("unroll") for (int n = 0; n < NT; ++n)                                           \
      fb[buf_][n] = *reinterpret_cast<const u32x4_t*>(xb_ + n * 32 * kPitch);                \
  } while (0)
#define XDNA_M4(buf_)                                                                        \
  do {                                                                                       \
    _Pragma("unroll") for (int m = 0; m < MT; ++m)                                           \
      _Pragma("unroll") for (int n = 0; n < NT; ++n)                                         \
        acc[m][n] = mfma_32x32x16(as_bf16x8(fa[buf_][m]), as_bf16x8(fb[buf_][n]), acc[m][n]); \
  } while (0)

  // prologue: slabs 0..2 and the window of chunk 0 in LDS; slabs 3, 4 in registers
  XDNA_W4_LOAD(0, 0);
  XDNA_W4_LOAD(1, 1);
  XDNA_W4_LOAD(2, 2);
  XDNA_X4_LOAD(0, -1);
  XDNA_W4_STORE(0, 0);
  XDNA_W4_STORE(1, 1);
  XDNA_W4_STORE(2, 2);
  XDNA_X4_STORE();
  XDNA_W4_LOAD(0, 3);
  XDNA_W4_LOAD(1, 4);
  __syncthreads();
  XDNA_F4_LOAD(0, 0, 0, 0);

  // Slab S lives in slot S % 3 and, before that, in register set S % 3 (loaded at tap
  // S-5, two taps before it is stored; at most two sets hold data at a time); (tap % 3) ==
  // (T % 3), so every slot and set index below is a compile-time constant.  Slot T % 3 is
  // read for the last time at tap T, k-step 2 (the fragments of k-step 3): the barrier
  // that opens k-step 3 frees it for slab T+3, which is first read at tap T+2, k-step 3,
  // two barriers later.  Instruction order is pinned with scheduling groups so that every
  // LDS access and global load issues between two MFMAs of the current k-step.
  constexpr int kMfma = 0x008, kVmemRd = 0x020, kDsRd = 0x100, kDsWr = 0x200;
  constexpr int kRest = kM - kR;                                   // MFMAs after the reads
  constexpr int kPerRest = kRest > 0 ? (kWv + kRest - 1) / kRest : kWv;
  constexpr int kXwPer = (kXv + kR - 1) / kR;                      // window writes per MFMA
  for (int ch = 0; ch < a.chunks; ++ch) {
    const int chn = min(ch + 1, a.chunks - 1);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int T = ch * 9 + tap;
#pragma unroll
      for (int ks = 0; ks < 3; ++ks) {
        const int cur = ks & 1;
        XDNA_F4_LOAD(cur ^ 1, tap % 3, tap, ks + 1);
        if (ks == 1 && tap < 7) XDNA_X4_LOAD(chn, tap);
        XDNA_M4(cur);
#pragma unroll
        for (int i = 0; i < kR; ++i) {
          __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kDsRd, 1, 0);
          if (ks == 1 && i < 3) __builtin_amdgcn_sched_group_barrier(kVmemRd, 1, 0);
        }
        if (kRest > 0) __builtin_amdgcn_sched_group_barrier(kMfma, kRest, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      __syncthreads();
      if (tap < 8) XDNA_F4_LOAD(0, (tap + 1) % 3, tap + 1, 0);
      else XDNA_X4_STORE();                 // chunk boundary: the next window
      XDNA_W4_STORE(tap % 3, tap % 3);      // slab T+3
      XDNA_W4_LOAD((tap + 2) % 3, T + 5);
      XDNA_M4(1);
      // the next tap's fragment reads first (their slot is not the one being written)
#pragma unroll
      for (int i = 0; i < kR; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        if (tap < 8)
          __builtin_amdgcn_sched_group_barrier(kDsRd, 1, 0);
        else
          __builtin_amdgcn_sched_group_barrier(kDsWr, kXwPer, 0);
      }
#pragma unroll
      for (int i = 0; i < (kRest > 0 ? kRest : 1); ++i) {
        if (kRest > 0) __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kDsWr, kPerRest, 0);
        __builtin_amdgcn_sched_group_barrier(kVmemRd, kPerRest, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (tap == 8) {
        __syncthreads();
        XDNA_F4_LOAD(0, 0, 0, 0);
      }
    }
  }
#undef XDNA_W4_LOAD
#undef XDNA_W4_STORE
#undef XDNA_X4_LOAD
#undef XDNA_X4_STORE
#undef XDNA_F4_LOAD
#undef XDNA_M4

  if constexpr (EPI < 2) {
    const OutMap om = out_map(a, int64_t(g) * kGroupOutRows + r0);
    const int plane2 = a.oH * a.oW * 2;
    int poff[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
      poff[n] = out_pixel_off32(a, om, g * kGroupOutRows + r0 + wn * NT * 32 + n * 32 + lr);
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * MT * 32 + m * 32 + mfma_row(i, lane);
        const int coff = co < a.cout ? co * plane2 : kOutSkip;
#pragma unroll
        for (int n = 0; n < NT; ++n)
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(rows_act_c<EPI == 1>(acc[m][n][i])), om.rs, poff[n] + coff, 0, 0);
      }
    return;
  } else {
    const int first = a.first;
    const int64_t plane = int64_t(a.H) * a.W;
    uint16_t* obase[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      obase[n] = nullptr;
      const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * NT * 32 + n * 32 + lr;
      if (p >= a.m_total) continue;
      const int64_t vb = p / a.img;
      const int64_t rem = p - vb * a.img;
      const int y = int(rem / a.wp);
      const int col = int(rem - int64_t(y) * a.wp) - first;
      if (y >= a.H || col < 0) continue;
      const int b = int(vb / a.S), s = int(vb % a.S);
      const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
      if (col >= cols) continue;
      const int x = (a.S == 1 ? 0 : s * a.So) + col;
      obase[n] = a.out + int64_t(b) * a.cout * plane + int64_t(y) * a.W + x;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * MT * 32 + m * 32 + mfma_row(i, lane);
        if (co >= a.cout) continue;
#pragma unroll
        for (int n = 0; n < NT; ++n)
          if (obase[n]) obase[n][int64_t(co) * plane] = f32_to_bf16(rows_act(a, acc[m][n][i]));
      }
  }
}

// Four-wave rows kernels on v_mfma_f32_16x16x32_bf16: the tiles, LDS layout, weight-slab
// ring and window staging of conv_rows4_kernel, with 16 x 16 output tiles.  The MFMA-bound
// kernels run at the board's power limit and the 16x16x32 form costs less energy per flop
// (independent chains: 2156 against 1772 TFLOP/s for 32x32x16 on random bf16 operands), so
// the clock runs higher; its MFMAs last 16 cycles instead of 32, so every LDS access and
// global load is issued after a single MFMA, never after a group of them.
// Wave (wm, wn) owns MI 16-channel x NJ 16-row tiles; a k-step is 32 channels (two per
// tap).  One fragment set: A rows MI/2 .. MI-1 of a k-step are read during the first half
// of its MFMAs (rows 0 .. MI/2-1, column by column), the next k-step's B columns and A
// rows 0 .. MI/2-1 during the second half, each right after its last use.  The one
// barrier per tap sits between the halves of its second k-step: every wave has then
// read the tap's weight slot for the last time, so slab T+3 is stored into it during
// the second half (and, at a chunk's last tap, the next chunk's window, followed by a
// second barrier before its first fragment reads).
// f(std::integral_constant<int, t>) for t = 0, 1, ...: call sites with compile-time indexes
// (what a long unrolled loop does not guarantee)
template <typename F, int... t>
__device__ inline void for_each_index(std::integer_sequence<int, t...>, F&& f) {
  (f(std::integral_constant<int, t>{}), ...);
}

// LDS rows of 80 elements (160 bytes) where one workgroup per CU leaves room, with the
// 16 rows of a fragment read in the lane order that swaps bits 2 and 3 of the lane's row
// index: rocprofv3's bank-conflict counter and a probe of ds_read_b128 lane groupings on
// the MI355X show 16-row x 4-piece reads at a 144-byte pitch conflicting (about 2 conflict
// cycles per LDS-active cycle) and this form free of conflicts at any starting row (the tap
// offsets).  The MFMA then sees rows and channels in that order, which the accumulator
// mapping follows.  Two workgroups per CU keep the 144-byte pitch and the plain order.
template <int MI, int NJ, int WM, int OCC = 1>
struct Q6 {
  static constexpr int WN = 4 / WM;
  static constexpr int CO = WM * MI * 16;                    // channels per workgroup
  static constexpr int TP = WN * NJ * 16;                    // grid rows per workgroup
  static constexpr int XRows = TP + kMaxHalo;                // window rows
  static constexpr bool Swz = size_t(XRows + 3 * CO) * 160 * OCC <= 160 * 1024;
  static constexpr int Mode = Swz ? 1 : 2;                   // q6_row's lane order
  static constexpr int Pitch = Swz ? 80 : kPitch;            // LDS row pitch (elements)
  static constexpr int Slot = CO * Pitch;                    // elements of one weight slot
  static constexpr size_t Lds = size_t(XRows * Pitch + 3 * Slot) * 2;
};

// The lane order of a fragment's 16 rows: mode 1 (160-byte rows) bits 2 and 3 swapped;
// mode 2 (144-byte rows, two workgroups per CU) the two 2-bit halves swapped, with the
// k-step's 8-channel pieces taken in the order (0, 4, 1, 5), (2, 6, 3, 7) by lane groups 0..3
// (both operands alike, so the sum is unchanged): a probe of that layout on the MI355X reads
// without bank conflicts at any starting row.
template <int kMode>
__device__ inline int q6_row(int r) {
  if (kMode == 1) return (r & 3) | ((r & 4) << 1) | ((r & 8) >> 1);
  if (kMode == 2) return ((r >> 2) & 3) | ((r & 3) << 2);
  return r;
}

template <int MI, int NJ, int WM, int OCC, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
void conv_rows6_kernel(RowsArgs a) {
  using Q = Q6<MI, NJ, WM, OCC>;
  constexpr int kP = Q::Pitch;
  constexpr int kXv = (Q::XRows * 8 + 255) / 256;      // window vectors per thread
  constexpr int kWv = Q::CO * 8 / 256;                 // weight vectors per thread per slab
  constexpr int kH = MI / 2;                           // A rows per half
  constexpr int kQ = kH * NJ;                          // MFMAs per half
  static_assert(MI % 2 == 0 && NJ >= kH && kH >= 2 && kWv >= 1, "tile shape");
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs = smem;                                 // [XRows][kP]
  uint16_t* wsl = smem + Q::XRows * kP;                // [3][CO][kP]

  constexpr int tiles_per_group = kGroupOutRows / Q::TP;
  int rt, ct;
  if (!rows_tile(a, rt, ct)) return;
  const int g = rt / tiles_per_group;
  const int r0 = (rt % tiles_per_group) * Q::TP;
  if (int64_t(g) * kGroupOutRows + r0 >= a.m_total) return;
  const int co0 = ct * Q::CO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int K = a.chunks * 9 * kKStep;
  const int T1 = a.chunks * 9;
  const int nrows = Q::TP + 2 * a.wp + 2;              // window rows (<= XRows)
  const int l16 = lane & 15, lq = lane >> 4;
  // the fragment row this lane reads, and the first of the 4 channel rows (4 lq .. 4 lq + 3
  // of a 16-row tile in MFMA order) its accumulators hold
  const int l16s = q6_row<Q::Mode>(l16);
  int chr[4];  // channel row (within a 16-channel tile) of accumulator register r
#pragma unroll
  for (int r = 0; r < 4; ++r) chr[r] = q6_row<Q::Mode>(4 * lq + r);
  // this lane group's 8 channels of k-step ks: + kqs * ks
  constexpr int kqs = Q::Mode == 2 ? 16 : 32;
  const int kq0 = Q::Mode == 2 ? 8 * (lq >> 1) + 32 * (lq & 1) : 8 * lq;

  // accumulators start at the bias of their channel rows 4 lq .. 4 lq + 3
  f32x4_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    f32x4_t init = {0.0f, 0.0f, 0.0f, 0.0f};
    const int cb = co0 + wm * MI * 16 + i * 16;
    if (a.bias && a.bias_vec && Q::Mode != 2) {
      // 4 consecutive channels from chr[0] on
      const __amdgpu_buffer_rsrc_t brs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.bias), 0, a.cout * 2, 0x00020000);
      const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(brs, (cb + chr[0]) * 2, 0, 0));
      init[0] = __uint_as_float(v.x << 16);
      init[1] = __uint_as_float(v.x & 0xFFFF0000u);
      init[2] = __uint_as_float(v.y << 16);
      init[3] = __uint_as_float(v.y & 0xFFFF0000u);
    } else if (a.bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r) init[r] = cb + chr[r] < a.cout ? bf16_to_f32(a.bias[cb + chr[r]]) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = init;
  }
  mfma16_fence(acc);

  // weight vector j of a slab: row (tid >> 3) + 32 j, 8-element piece tid & 7
  const uint16_t* wsrc = a.wt + (int64_t(co0) + (tid >> 3)) * K + (tid & 7) * 8;
  const int wdst = (tid >> 3) * kP + (tid & 7) * 8;
  // window vector j: row min((tid + 256 j) >> 3, nrows - 1), piece tid & 7
  auto xoff = [&](int j) { return min((tid + j * 256) >> 3, nrows - 1) * 8 + (tid & 7); };
  const uint16_t* xsrc0 = a.xp + (int64_t(g) * a.chunks * kGroupRows + r0) * kKStep;
  // fragment bases: A row wm*MI*16 + l16s of a slot, B row wn*NJ*16 + l16s of the window,
  // this lane group's 8 channels of a k-step (kq0)
  const uint16_t* wfr = wsl + (wm * MI * 16 + l16s) * kP + kq0;
  const uint16_t* xfr = xs + (wn * NJ * 16 + l16s) * kP + kq0;
  const int wrow = a.wp * kP;

  u32x4_t wreg[3][kWv];
  u32x4_t xr[kXv];
  u32x4_t fa[MI], fb[NJ];

  auto w_load = [&](int set, int S) {
    const uint16_t* s_ = wsrc + int64_t(min(S, T1 - 1)) * kKStep;
#pragma unroll
    for (int v = 0; v < kWv; ++v) wreg[set][v] = *reinterpret_cast<const u32x4_t*>(s_ + int64_t(v * 32) * K);
  };
  auto w_load1 = [&](int set, int S, int v) {
    const uint16_t* s_ = wsrc + int64_t(min(S, T1 - 1)) * kKStep;
    wreg[set][v] = *reinterpret_cast<const u32x4_t*>(s_ + int64_t(v * 32) * K);
  };
  auto w_store1 = [&](int set, int slot, int v) {
    *reinterpret_cast<u32x4_t*>(wsl + slot * Q::Slot + wdst + v * 32 * kP) = wreg[set][v];
  };
  auto x_load1 = [&](int ch, int v) {
    xr[v] = *reinterpret_cast<const u32x4_t*>(xsrc0 + int64_t(ch) * kGroupRows * kKStep + xoff(v) * 8);
  };
  auto x_store1 = [&](int v) {
    *reinterpret_cast<u32x4_t*>(&xs[(xoff(v) >> 3) * kP + (xoff(v) & 7) * 8]) = xr[v];
  };
  auto frag_a = [&](int slot, int i, int ks) {
    return *reinterpret_cast<const u32x4_t*>(wfr + slot * Q::Slot + i * 16 * kP + ks * kqs);
  };
  auto frag_b = [&](int tap, int j, int ks) {
    return *reinterpret_cast<const u32x4_t*>(xfr + (tap / 3) * wrow + ((tap % 3) + j * 16) * kP + ks * kqs);
  };

  // prologue: slabs 0..2 and the window of chunk 0 in LDS; slabs 3, 4 in registers
  w_load(0, 0);
  w_load(1, 1);
  w_load(2, 2);
#pragma unroll
  for (int v = 0; v < kXv; ++v) x_load1(0, v);
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int v = 0; v < kWv; ++v) w_store1(s, s, v);
#pragma unroll
  for (int v = 0; v < kXv; ++v) x_store1(v);
  w_load(0, 3);
  w_load(1, 4);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kH; ++i) fa[i] = frag_a(0, i, 0);
#pragma unroll
  for (int j = 0; j < NJ; ++j) fb[j] = frag_b(0, j, 0);

  int ch = 0, chn = 0;
  // one k-step (tap, ks) of chunk ch; tap and ks are compile-time constants, so every
  // register-set index and every slot of the extra memory work below is static
  auto kstep = [&](auto tap_c, auto ks_c) {
        constexpr int tap = decltype(tap_c)::value, ks = decltype(ks_c)::value;
        const int T = ch * 9 + tap;
        // first half: A rows 0 .. kH-1 column by column; A rows kH + j read after the
        // second MFMA of column j
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int i = 0; i < kH; ++i) {
            mfma16_acc<false>(acc[i][j], fa[i], fb[j]);
            if (i == 1 && j < kH) fa[kH + j] = frag_a(tap % 3, kH + j, ks);
            __builtin_amdgcn_sched_barrier(0);
          }
        if (ks == 1) {
          // every wave has read slot tap % 3 (and, at tap 8, this chunk's window) for the
          // last time
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
        }
        // second half: A rows kH .. MI-1 column by column.  After column j's last MFMA its
        // B fragment is read for the next k-step (at a chunk's end, after the window
        // store and barrier below); after its second MFMA, A row j (j < kH) of the next
        // k-step.  Extra memory work, one instruction per MFMA slot: k-step 0 the next
        // chunk's window loads (taps 0..6 share them), k-step 1 slab T+3 into slot
        // tap % 3, slab T+5 into register set (tap + 2) % 3 and, at tap 8, the window store.
        constexpr int ntap = ks == 0 ? tap : (tap + 1) % 9;
        constexpr int nks = ks ^ 1;
        constexpr bool chunk_end = ks == 1 && tap == 8;
        // window loads of the next chunk, spread over taps 0..6
        constexpr int nx_lo = tap < 7 ? tap * kXv / 7 : kXv, nx_hi = tap < 7 ? (tap + 1) * kXv / 7 : kXv;
        constexpr int n_extra = ks == 0 ? nx_hi - nx_lo : 2 * kWv + (tap == 8 ? kXv : 0);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < kH; ++r) {
            const int q = j * kH + r;
            mfma16_acc<false>(acc[kH + r][j], fa[kH + r], fb[j]);
            if (r == kH - 1 && !chunk_end) fb[j] = frag_b(ntap, j, nks);
            if (r == 1 && j < kH) fa[j] = frag_a(ntap % 3, j, nks);
#pragma unroll
            for (int e = 0; e < 2 * kWv + kXv; ++e) {
              if (e >= n_extra || e * kQ / (n_extra > 0 ? n_extra : 1) != q) continue;
              if (ks == 0) {
                x_load1(chn, nx_lo + e);
              } else if (e < kWv) {
                w_store1(tap % 3, tap % 3, e);
              } else if (e < 2 * kWv) {
                w_load1((tap + 2) % 3, T + 5, e - kWv);
              } else {
                x_store1(e - 2 * kWv);
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        if (chunk_end) {
          __syncthreads();  // the next chunk's window is in place
#pragma unroll
          for (int j = 0; j < NJ; ++j) fb[j] = frag_b(0, j, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
  };
  for (; ch < a.chunks; ++ch) {
    chn = min(ch + 1, a.chunks - 1);
    for_each_index(std::make_integer_sequence<int, 9>{}, [&](auto tap_c) {
      kstep(tap_c, std::integral_constant<int, 0>{});
      kstep(tap_c, std::integral_constant<int, 1>{});
    });
  }

  mfma16_fence(acc);
  if constexpr (EPI < 2) {
    const OutMap om = out_map(a, int64_t(g) * kGroupOutRows + r0);
    const int plane2 = a.oH * a.oW * 2;
    int poff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      poff[j] = out_pixel_off32(a, om, g * kGroupOutRows + r0 + wn * NJ * 16 + j * 16 + l16s);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int co = co0 + wm * MI * 16 + i * 16 + chr[r];
        const int coff = co < a.cout ? co * plane2 : kOutSkip;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(rows_act_c<EPI == 1>(acc[i][j][r])), om.rs, poff[j] + coff, 0, 0);
      }
    return;
  } else {
    const int first = a.first;
    const int64_t plane = int64_t(a.H) * a.W;
    uint16_t* obase[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      obase[j] = nullptr;
      const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * NJ * 16 + j * 16 + l16s;
      if (p >= a.m_total) continue;
      const int64_t vb = p / a.img;
      const int64_t rem = p - vb * a.img;
      const int y = int(rem / a.wp);
      const int col = int(rem - int64_t(y) * a.wp) - first;
      if (y >= a.H || col < 0) continue;
      const int b = int(vb / a.S), s = int(vb % a.S);
      const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
      if (col >= cols) continue;
      const int x = (a.S == 1 ? 0 : s * a.So) + col;
      obase[j] = a.out + int64_t(b) * a.cout * plane + int64_t(y) * a.W + x;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int co = co0 + wm * MI * 16 + i * 16 + chr[r];
        if (co >= a.cout) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          if (obase[j]) obase[j][int64_t(co) * plane] = f32_to_bf16(rows_act(a, acc[i][j][r]));
      }
  }
}

// Small-grid variant: 64 output channels x TP grid rows per workgroup.  Per input chunk
// the halo window AND all nine taps of the workgroup's weights (64 x 576 bf16, 72 KiB)
// are staged in LDS with every load of the chunk in flight at once, so a chunk costs one
// memory latency instead of one per tap; the next chunk's loads are issued into
// registers before the current chunk is multiplied.  Wave (wm, wn) owns channels
// [wm*32, +32) x rows [wn*TP/2, +TP/2).  For convs whose grid is a few hundred
// workgroups or less, where the main kernel waits on its per-tap weight loads.
//
// EMUL: the reference NPU's arithmetic (conv3x3w_kernel.cc:40-51, 105-108; loop order
// conv3x3w.py:172-177): the running sum is kept as bf16 and rounded after every (chunk,
// tap), chunks outer and taps inner, and the bias is added after the last rounding (the
// reference's host bias add, torch_xdna_device.cpp:2477-2480).  Operands come in already
// quantized to BFP16 values; no split-K (it would change the rounding order).
//
// NCHW: the halo window is gathered from the NCHW input itself instead of packed rows
// (images up to 36 columns, input channels a multiple of 8): window row i is padded-grid
// row q = rt * TP + i of the packed layout (q = (b (H+2) + y + 1) wp + x + 1 for pixel
// (y, x) of image b, wp = W + 2), so the LDS window, and with it every product and sum, is
// the one the packed input gives, and no pack pass runs.  Item (row, 8-channel piece):
// consecutive threads take consecutive rows, so each of the piece's eight 2-byte channel
// loads of a wave reads one contiguous run of a channel plane; border, padding and
// past-the-end rows read zeros (an offset past the buffer's range).
constexpr int kSCo = 64;                  // output channels per workgroup
// LDS pitch of a staged weight row (672 elements, 16 banks mod 64): with the slab's pieces
// swizzled per row (sw_piece) both its writes (four lanes per row: the rows of a lane group
// on disjoint 16-bank windows) and the fragment reads (sixteen rows per lane group on
// distinct bank quads) are free of bank conflicts; the 584-element pitch put the rows of a
// write's lane group on overlapping banks
constexpr int kSWPitch = 9 * kKStep + 96;
// 16-byte piece p of staged weight row r sits at sw_piece(r, p): bits 0-1 of p XOR bits 2-3
// of r (a permutation inside each aligned block of 4 pieces)
__device__ inline int sw_piece(int r, int p) { return p ^ ((r >> 2) & 3); }

__device__ inline float round_bf16(float v) { return __uint_as_float(uint32_t(f32_to_bf16(v)) << 16); }

template <int TP, bool EMUL = false, bool NCHW = false, int EP = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void conv_small_kernel(RowsArgs a) {
  constexpr int kXRows = TP + kMaxHalo;
  constexpr int NT = TP / 64;                     // 32-row MFMA tiles per wave
  constexpr int kXv = (kXRows * 8 + 255) / 256;   // window vectors per thread
  constexpr int kWv = kSCo * 9 * 8 / 256;         // weight vectors per thread (18)
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs = smem;                            // [kXRows][kPitch]
  uint16_t* ws = smem + kXRows * kPitch;          // [kSCo][kSWPitch]

  constexpr int tiles_per_group = kGroupOutRows / TP;
  int rt, ct;
  if (!rows_tile(a, rt, ct)) return;
  const int g = rt / tiles_per_group;
  const int r0 = (rt % tiles_per_group) * TP;
  if (int64_t(g) * kGroupOutRows + r0 >= a.m_total) return;
  const int co0 = ct * kSCo;
  const int ch0 = blockIdx.z * a.ch_per;
  const int ch1 = min(a.chunks, ch0 + a.ch_per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int K = a.chunks * 9 * kKStep;
  const int nvec = (TP + 2 * a.wp + 2) * 8;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[NT];
  float bco[EMUL ? 16 : 1];  // EMUL: the bias of each accumulator row, added at the end
  if constexpr (EMUL) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 32 + mfma_row(i, lane);
      bco[i] = a.bias && co < a.cout ? bf16_to_f32(a.bias[co]) : 0.0f;
    }
  }
  {
    f32x16_t init = zero_acc();
    if (EMUL) {
      // the running sum starts at zero
    } else if (a.bias && !a.part && a.bias_vec) {
      // 4 runs of 4 consecutive channels per lane: 8-byte buffer loads (as the main kernel)
      const __amdgpu_buffer_rsrc_t brs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.bias), 0, a.cout * 2, 0x00020000);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int co = co0 + wm * 32 + 8 * q + 4 * (lane >> 5);
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(brs, co * 2, 0, 0));
        init[4 * q + 0] = __uint_as_float(v.x << 16);
        init[4 * q + 1] = __uint_as_float(v.x & 0xFFFF0000u);
        init[4 * q + 2] = __uint_as_float(v.y << 16);
        init[4 * q + 3] = __uint_as_float(v.y & 0xFFFF0000u);
      }
    } else if (a.bias && !a.part) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * 32 + mfma_row(i, lane);
        init[i] = co < a.cout ? bf16_to_f32(a.bias[co]) : 0.0f;
      }
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = init;
  }

  u32x4_t xr[kXv], wr[kWv];
  // NCHW: per window item j of this thread (row xrow[j], piece xpc[j]) the element offset of
  // its pixel in channel plane 0 of its image, or a negative value for a zero row
  const int nrows = TP + 2 * a.wp + 2;
  int xoff[NCHW ? kXv : 1], xpc[NCHW ? kXv : 1], xrow[NCHW ? kXv : 1];
  __amdgpu_buffer_rsrc_t xrs;
  int plane_bytes = 0;
  if constexpr (NCHW) {
    const int hw = a.H * a.W;
    plane_bytes = hw * 2;
    xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xsrc), 0,
                                            int(int64_t(a.B) * a.cin * hw * 2), 0x00020000);
    const int64_t q0 = int64_t(g) * kGroupOutRows + r0;
#pragma unroll
    for (int j = 0; j < kXv; ++j) {
      const int i = tid + j * 256;
      const int pc = i / nrows, row = i - pc * nrows;
      xpc[j] = pc;
      xrow[j] = row;
      const int64_t q = q0 + row;
      const int b = int(q / a.img);
      const int rem = int(q - int64_t(b) * a.img);
      const int yy = rem / a.wp, xx = rem - yy * a.wp;
      const bool ok = i < nvec && q < a.m_total && yy >= 1 && yy <= a.H && xx >= 1 && xx <= a.W;
      xoff[j] = ok ? (b * a.cin) * hw + (yy - 1) * a.W + (xx - 1) : -1;
    }
  }
  // Chunk staging with addresses fixed per thread (no per-chunk index math):
  //  * weights: thread t copies row t / 4 of the workgroup's 64-row slab, its 16-byte
  //    pieces t % 4 + 4 j (j < 18) of 72: one buffer offset per thread, 64 j bytes as an
  //    immediate, chunk ch's slab ch * 1152 bytes into the rows (scalar offset);
  //  * packed window: item (row t / 8 + 32 j, piece t % 8): one buffer offset per thread,
  //    the chunk's block and 4096 j bytes in the scalar offset; rows past the window are
  //    read (inside the group's 2126 rows, or past the buffer: zeros) and not stored.
  const int wrow = tid >> 2, wq = tid & 3;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.wt + int64_t(co0) * K), 0, kSCo * K * 2, 0x00020000);
  const int wvo = wrow * K * 2 + wq * 16;
  uint16_t* const wlds = ws + wrow * kSWPitch + sw_piece(wrow, wq) * 8;  // pieces wq + 4 j (j * 32 below)
  __amdgpu_buffer_rsrc_t prs;
  if constexpr (!NCHW) {
    const int64_t pbase = (int64_t(g) * a.chunks * kGroupRows + r0) * kKStep;
    const int64_t ptotal = (a.m_total + kGroupOutRows - 1) / kGroupOutRows * a.chunks * kGroupRows * kKStep;
    prs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xp + pbase), 0,
                                            clamp_records((ptotal - pbase) * 2), 0x00020000);
  }
  const int pvo = (tid >> 3) * 128 + (tid & 7) * 16;
  auto load_chunk = [&](int ch) {
    if constexpr (NCHW) {
#pragma unroll
      for (int j = 0; j < kXv; ++j) {
        const int c0 = ch * kKStep + 8 * xpc[j];
        // element offset of (pixel, channel c0), or past the range (reads zeros)
        const int off = xoff[j] >= 0 && c0 < a.cin ? 2 * (xoff[j] + c0 * (plane_bytes >> 1)) : 0x7FFFFFF0;
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          h[e] = uint32_t(__builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(
                                                           xrs, off, e * plane_bytes, 0)));
        xr[j] = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
      }
    } else {
      const int so = ch * (kGroupRows * kKStep * 2);
#pragma unroll
      for (int j = 0; j < kXv; ++j)
        xr[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(prs, pvo, so + j * 4096, 0));
    }
    const int wso = ch * (9 * kKStep * 2);
    static_assert(kWv == 18 && kSCo * 4 == 256, "weight staging: 4 threads per row, 18 pieces each");
#pragma unroll
    for (int j = 0; j < kWv; ++j)
      wr[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo + j * 64, wso, 0));
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int j = 0; j < kXv; ++j) {
      if constexpr (NCHW) {
        const int i = tid + j * 256;
        if (i < nvec) *reinterpret_cast<u32x4_t*>(&xs[xrow[j] * kPitch + xpc[j] * 8]) = xr[j];
      } else {
        const int row = (tid >> 3) + 32 * j;
        if (row < nrows) *reinterpret_cast<u32x4_t*>(&xs[row * kPitch + (tid & 7) * 8]) = xr[j];
      }
    }
#pragma unroll
    for (int j = 0; j < kWv; ++j) *reinterpret_cast<u32x4_t*>(wlds + j * 32) = wr[j];
  };

  load_chunk(ch0);
  // fragment k-step (tap, ks) of this lane: piece 8 tap + 2 ks + lk / 8 of weight row
  // wm * 32 + lr, at its swizzled place (the tap in the immediate offset)
  const uint16_t* wa_k[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    wa_k[ks] = ws + (wm * 32 + lr) * kSWPitch + sw_piece(wm * 32 + lr, 2 * ks + (lk >> 3)) * 8;
  const uint16_t* xb = xs + (wn * (TP / 2) + lr) * kPitch + lk;
  for (int ch = ch0; ch < ch1; ++ch) {
    __syncthreads();  // the previous chunk's reads of xs / ws are done
    store_chunk();
    __syncthreads();
    if (ch + 1 < ch1) load_chunk(ch + 1);
    // k-step s = (tap, 16-channel slice): its fragments are read kPre k-steps ahead into
    // a ring of registers (one wave per SIMD: an MFMA or two cannot cover an LDS read)
    constexpr int kPre = 3;
    u32x4_t aq[kPre + 1], bq[kPre + 1][NT];
    const uint16_t* xrow[3] = {xb, xb + a.wp * kPitch, xb + 2 * a.wp * kPitch};
    auto fetch = [&](int step) {
      const int tap = step >> 2, ks = step & 3, slot = step % (kPre + 1);
      aq[slot] = *reinterpret_cast<const u32x4_t*>(wa_k[ks] + tap * kKStep);
      const uint16_t* xq = xrow[tap / 3] + (tap % 3) * kPitch + ks * 16;
#pragma unroll
      for (int n = 0; n < NT; ++n) bq[slot][n] = *reinterpret_cast<const u32x4_t*>(xq + n * 32 * kPitch);
    };
#pragma unroll
    for (int step = 0; step < kPre; ++step) fetch(step);
#pragma unroll
    for (int step = 0; step < 36; ++step) {
      if (step + kPre < 36) fetch(step + kPre);
      __builtin_amdgcn_sched_barrier(0);
      const int slot = step % (kPre + 1);
      const bf16x8_t af = as_bf16x8(aq[slot]);
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] = mfma_32x32x16(af, as_bf16x8(bq[slot][n]), acc[n]);
      if constexpr (EMUL) {
        if ((step & 3) == 3) {  // the tap's 64 channels are in: C stored as bf16
#pragma unroll
          for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[n][i] = round_bf16(acc[n][i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (EMUL) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[n][i] += bco[i];
  }

  if constexpr (EP == 1) {
    float* pz = a.part + int64_t(blockIdx.z) * a.cout * a.m_pad;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * (TP / 2) + n * 32 + lr;
      if (p >= a.m_total) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wm * 32 + mfma_row(i, lane);
        if (co < a.cout) pz[int64_t(co) * a.m_pad + p] = acc[n][i];
      }
    }
    return;
  } else if constexpr (EP == 0 || EP == 3) {
    const OutMap om = out_map(a, int64_t(g) * kGroupOutRows + r0);
    const int plane2 = a.oH * a.oW * 2;
    int poff[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
      poff[n] = out_pixel_off32(a, om, g * kGroupOutRows + r0 + wn * (TP / 2) + n * 32 + lr);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 32 + mfma_row(i, lane);
      const int coff = co < a.cout ? co * plane2 : kOutSkip;
#pragma unroll
      for (int n = 0; n < NT; ++n)
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(rows_act_c<EP == 3>(acc[n][i])), om.rs, poff[n] + coff, 0, 0);
    }
    return;
  } else {
    const int first = a.first;
    const int64_t plane = int64_t(a.H) * a.W;
    uint16_t* obase[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      obase[n] = nullptr;
      const int64_t p = int64_t(g) * kGroupOutRows + r0 + wn * (TP / 2) + n * 32 + lr;
      if (p >= a.m_total) continue;
      const int64_t vb = p / a.img;
      const int64_t rem = p - vb * a.img;
      const int y = int(rem / a.wp);
      const int col = int(rem - int64_t(y) * a.wp) - first;
      if (y >= a.H || col < 0) continue;
      const int b = int(vb / a.S), s = int(vb % a.S);
      const int cols = a.S == 1 ? a.W : min(a.So, a.W - s * a.So);
      if (col >= cols) continue;
      const int x = (a.S == 1 ? 0 : s * a.So) + col;
      obase[n] = a.out + int64_t(b) * a.cout * plane + int64_t(y) * a.W + x;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 32 + mfma_row(i, lane);
      if (co >= a.cout) continue;
#pragma unroll
      for (int n = 0; n < NT; ++n)
        if (obase[n]) obase[n][int64_t(co) * plane] = f32_to_bf16(rows_act(a, acc[n][i]));
    }
  }
}

// Split-K epilogue: out[b][co][y][x] = bf16(bias[co] + sum over splits, in split order,
// of part[z][co][p(b, y, x)]).  blockIdx.y = plane b * cout + co (plane0 + that), threads
// over the plane's pixels (32-bit index math).
__global__ __launch_bounds__(256) void rows_reduce_kernel(RowsArgs a, int nsplit, int plane0) {
  const int plane = plane0 + int(blockIdx.y);
  const int b = plane / a.cout, co = plane - b * a.cout;
  const int pix = int(blockIdx.x) * 256 + int(threadIdx.x);
  if (pix >= a.oH * a.oW) return;
  // output pixel pix of the oH x oW image; its grid pixel (y, x) (stride-2 output: 2x)
  const int yo = pix / a.oW, xo = pix - yo * a.oW;
  const int y = yo << a.osh, x = xo << a.osh;
  const int s = a.S == 1 ? 0 : x / a.So;
  const int col = x - s * a.So + a.first;
  const int64_t p = (int64_t(b) * a.S + s) * a.img + int64_t(y) * a.wp + col;
  float v = a.bias ? bf16_to_f32(a.bias[co]) : 0.0f;
  const float* pp = a.part + int64_t(co) * a.m_pad + p;
  const int64_t zstride = int64_t(a.cout) * a.m_pad;
  v = sum_strided8(v, pp, zstride, 0, 1, nsplit);
  a.out[int64_t(plane) * a.oH * a.oW + pix] = f32_to_bf16(rows_act(a, v));
}

// ---------------------------------------------------------------------------------
// Channel-major padded grid for wgrad.
// ---------------------------------------------------------------------------------
struct CmGeom {
  int wp8 = 0;
  int64_t img = 0, npix = 0, ktiles = 0, q = 0;  // q: row length (elements)
};

constexpr int kTK = 64;  // pixels per wgrad k-tile

CmGeom cm_geom(int B, int H, int W) {
  CmGeom g;
  g.wp8 = int(ceil_div(W + 2, 8) * 8);
  g.img = int64_t(H + 2) * g.wp8;
  g.npix = int64_t(B) * g.img;
  g.ktiles = ceil_div(g.npix, kTK);
  g.q = g.ktiles * kTK + 2 * g.wp8 + 16;
  return g;
}

// dst[c][q] for c < c_pad, q < qlen; shift = 1 places pixel (y, x) at grid (y+1, x+1)
// (the conv input), shift = 0 at (y, x) (the output gradient).  Every element is
// written (zeros outside the image and for c >= C).
//
// Workgroups [0, nmain) each take grid rows [gy0, gy0 + rows_per) of planes_per
// consecutive (b, c) planes (planes_per > 1 only when whole planes fit): the source rows
// they need are one contiguous run of NCHW, read with 16-byte loads into LDS (placed so
// that 16-byte aligned global addresses stay 16-byte aligned in LDS), then written as
// 16-byte pieces of padded grid rows.  The remaining workgroups zero the rows c >= C and
// the tail of every row past the last image.
constexpr int kCmLdsElems = 8192;  // 16 KiB of staged source rows

// One operand of the channel-major pack (x with shift 1, or dY with shift 0).
struct CmOp {
  const uint16_t* src;
  uint16_t* dst;
  int C, c_pad, shift, rows_per, rblocks, planes_per;
  int64_t nmain, blocks;  // workgroups [0, nmain) pack planes, [nmain, blocks) zero-fill
};
struct CmArgs {
  CmOp op[2];
  int B, H, W, wp8;
  int64_t img, qlen;
};

__global__ __launch_bounds__(256) void pack_cm_kernel(CmArgs ca) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[kCmLdsElems + 16];
  int64_t bid = blockIdx.x;
  const int which = bid < ca.op[0].blocks ? 0 : 1;
  if (which) bid -= ca.op[0].blocks;
  const CmOp& op = ca.op[which];
  const uint16_t* __restrict__ src = op.src;
  uint16_t* __restrict__ dst = op.dst;
  const int B = ca.B, C = op.C, H = ca.H, W = ca.W, c_pad = op.c_pad, wp8 = ca.wp8, shift = op.shift;
  const int rows_per = op.rows_per, rblocks = op.rblocks, planes_per = op.planes_per;
  const int64_t img = ca.img, qlen = ca.qlen, nmain = op.nmain;
  const int64_t tail0 = int64_t(B) * img;  // first q past the last image
  if (bid >= nmain) {
    // zero fill: rows c < C from tail0 (a multiple of 8), rows c >= C whole
    const int64_t tvec = (qlen - tail0) / 8, rvec = qlen / 8;
    const int64_t n = int64_t(C) * tvec + int64_t(c_pad - C) * rvec;
    const uint4 z = make_uint4(0, 0, 0, 0);
    for (int64_t i = (bid - nmain) * 256 + threadIdx.x; i < n; i += (op.blocks - nmain) * 256) {
      int64_t o;
      if (i < int64_t(C) * tvec) {
        const int64_t c = i / tvec;
        o = c * qlen + tail0 + (i - c * tvec) * 8;
      } else {
        const int64_t k = i - int64_t(C) * tvec;
        const int64_t c = C + k / rvec;
        o = c * qlen + (k - (c - C) * rvec) * 8;
      }
      *reinterpret_cast<uint4*>(dst + o) = z;
    }
    return;
  }
  const int rb = int(bid % rblocks);
  const int64_t pl0 = (bid / rblocks) * planes_per;  // first source plane b*C + c
  const int np = int(std::min<int64_t>(planes_per, int64_t(B) * C - pl0));
  const int gy0 = rb * rows_per;
  const int gy1 = min(gy0 + rows_per, H + 2);
  const int vrow = wp8 / 8;
  const int nout_pl = (gy1 - gy0) * vrow;
  // source rows needed: yy = gy - shift for gy in [gy0, gy1), clipped to [0, H)
  const int ylo = max(gy0 - shift, 0), yhi = min(gy1 - shift, H);
  if (yhi > ylo) {
    const int64_t off = (pl0 * H + ylo) * W;  // element offset of the run
    const int len = ((np - 1) * H + yhi - ylo) * W;
    const int lead = int(off & 7);            // LDS index of element 0
    const int64_t abase = off - lead;         // 16-byte aligned start
    const int nvec = (lead + len + 7) >> 3;
    const bool full_ok = (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    for (int v = threadIdx.x; v < nvec; v += 256) {
      const int e0 = v * 8;
      if (full_ok && e0 >= lead && e0 + 8 <= lead + len) {
        *reinterpret_cast<uint4*>(lds + e0) = *reinterpret_cast<const uint4*>(src + abase + e0);
      } else {
        for (int e = e0; e < e0 + 8; ++e)
          if (e >= lead && e < lead + len) lds[e] = src[abase + e];
      }
    }
    __syncthreads();
    for (int v = threadIdx.x; v < np * nout_pl; v += 256) {
      const int k = v / nout_pl;
      const int vv = v - k * nout_pl;
      const int r = vv / vrow;
      const int x0 = (vv - r * vrow) * 8 - shift;
      const int yy = gy0 + r - shift;
      uint32_t u[4] = {0, 0, 0, 0};
      if (yy >= 0 && yy < H) {
        const uint16_t* lr = lds + lead + (k * H + yy - ylo) * W;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int xx = x0 + e;
          if (xx >= 0 && xx < W) u[e >> 1] |= uint32_t(lr[xx]) << (16 * (e & 1));
        }
      }
      const int64_t pl = pl0 + k;
      const int64_t b = pl / C, c = pl - b * C;
      uint16_t* d = dst + c * qlen + b * img + int64_t(gy0) * wp8 + int64_t(vv) * 8;
      *reinterpret_cast<uint4*>(d) = make_uint4(u[0], u[1], u[2], u[3]);
    }
  } else {
    // grid rows with no source row (a single plane): all zero
    const int64_t b = pl0 / C, c = pl0 - b * C;
    uint16_t* drow = dst + c * qlen + b * img + int64_t(gy0) * wp8;
    for (int v = threadIdx.x; v < nout_pl; v += 256)
      *reinterpret_cast<uint4*>(drow + int64_t(v) * 8) = make_uint4(0, 0, 0, 0);
  }
}

// Plans one operand of pack_cm_kernel.
CmOp pack_cm_plan(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W, int c_pad,
                  const CmGeom& cm, int shift) {
  // grid rows per workgroup: the source run (rows_per rows of W, plus alignment lead)
  // must fit the LDS buffer; small planes are batched while the grid stays large
  CmOp o;
  o.src = src;
  o.dst = dst;
  o.C = C;
  o.c_pad = c_pad;
  o.shift = shift;
  o.rows_per = std::max(1, std::min(H + 2, (kCmLdsElems - 8) / std::max(W, 1)));
  o.rblocks = int(ceil_div(H + 2, o.rows_per));
  const int64_t planes = int64_t(B) * C;
  o.planes_per = 1;
  if (o.rblocks == 1)
    o.planes_per = int(std::max<int64_t>(1, std::min<int64_t>((kCmLdsElems - 8) / (int64_t(H) * W), planes / 2048)));
  o.nmain = ceil_div(planes, o.planes_per) * o.rblocks;
  const int64_t nzero = int64_t(C) * ((cm.q - int64_t(B) * cm.img) / 8) + int64_t(c_pad - C) * (cm.q / 8);
  o.blocks = o.nmain + std::min<int64_t>(std::max<int64_t>(ceil_div(nzero, 256 * 4), 1), 4096);
  return o;
}

// Packs x (shift 1) and dY (shift 0) in one launch.
int pack_cm_launch2(const uint16_t* x, uint16_t* xt, int Cin, int ci_pad, const uint16_t* dy, uint16_t* dt,
                    int Cout, int co_pad, int B, int H, int W, const CmGeom& cm, hipStream_t st) {
  CmArgs ca;
  ca.op[0] = pack_cm_plan(x, xt, B, Cin, H, W, ci_pad, cm, 1);
  ca.op[1] = pack_cm_plan(dy, dt, B, Cout, H, W, co_pad, cm, 0);
  ca.B = B;
  ca.H = H;
  ca.W = W;
  ca.wp8 = cm.wp8;
  ca.img = cm.img;
  ca.qlen = cm.q;
  const int64_t blocks = ca.op[0].blocks + ca.op[1].blocks;
  if (blocks > int64_t(0x7fffffff)) {
    set_error("conv3x3 wgrad pack: too many planes");
    return -1;
  }
  pack_cm_kernel<<<dim3(unsigned(blocks)), 256, 0, st>>>(ca);
  return 0;
}

struct WgradArgs {
  const uint16_t* xt;  // [ci_pad][q]
  const uint16_t* dt;  // [co_pad][q]
  float* part;         // [splits][co_pad][9][ci_pad]
  float* bpart;        // [splits][co_pad]
  int64_t q;           // row length of xt and dt
  int wp8, ci_pad, co_pad;
  int kt_per_split, ktiles;
  int xpitch;          // LDS pitch of the staged x window (elements)
  int wlen;            // staged window length (elements): kTK + 2*wp8 + 8
  int nco_t, ntiles, splits;  // channel tiles (co tiles x ci tiles) and pixel splits
};

// blockIdx.x -> (co tile, ci tile, split).  Workgroup L runs on XCD L % 8; on each XCD the
// consecutive workgroups take every channel tile of one pixel split, so the split's x
// window and dY rows come from HBM once and serve all its tiles from that XCD's L2
// (split s lives on XCD s % 8; the grid is padded to a multiple of 8 splits).
__device__ inline bool wgrad_tile(const WgradArgs& a, int& co_t, int& ci_t, int& split) {
  const int L = blockIdx.x;
  const int x = L % kXcds, k = L / kXcds;
  const int tile = k % a.ntiles;
  split = (k / a.ntiles) * kXcds + x;
  co_t = tile % a.nco_t;
  ci_t = tile / a.nco_t;
  return split < a.splits;
}

// One workgroup (8 waves, 512 threads): 128 output channels x 64 input channels x 9 taps
// over the k-tiles of one split.  Wave (wm, wn) owns channels [wm*32, +32) x input
// channels [wn*32, +32) x all 9 taps (9 accumulator tiles), fed per 16-pixel step by one
// dY fragment and 3 x (16 + 4)-byte LDS reads of the x window (dx = 0, 1, 2 are built from
// each read with alignbit).  Fragments are software-pipelined one step ahead; the next
// k-tile is fetched into registers while the current one is multiplied, and LDS is
// double-buffered ([dY 128 x kPitch][x 64 x xpitch] per buffer): one barrier per k-tile.
// Two waves per SIMD.
constexpr int kWgThreads = 512;
constexpr int kWgMaxXv = 6;  // x-window vectors per thread (64 * wlen/8 <= 3072: wlen <= 384)

// XV: x-window vectors per thread (4: wlen <= 256, i.e. W <= 90; 6: wlen <= 384)
template <int XV>
__global__ __launch_bounds__(kWgThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void wgrad_kernel(WgradArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int buf_elems = kTCo * kPitch + 64 * a.xpitch;
  int co_t, ci_t, split;
  if (!wgrad_tile(a, co_t, ci_t, split)) return;
  const int co0 = co_t * kTCo;
  const int ci0 = ci_t * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  const int kt0 = split * a.kt_per_split;
  const int kt1 = min(a.ktiles, kt0 + a.kt_per_split);
  const int nvec_w = a.wlen / 8;
  const int nx = 64 * nvec_w;

  f32x16_t acc[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) acc[t] = zero_acc();
  float bsum = 0.0f;
  const bool do_bias = a.bpart && ci_t == 0 && wn == 0;

  u32x4_t dreg[2];
  u32x4_t xreg[XV];
  // global -> registers (k-tile kt), registers -> LDS buffer; macros keep the prefetch
  // arrays in registers (fully unrolled, constant indices)
#define XDNA_WG_LOAD(kt_)                                                                    \
  do {                                                                                       \
    const int64_t k0_ = int64_t(kt_) * kTK;                                                  \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                          \
      const int i = tid + j * kWgThreads;                                                    \
      dreg[j] = *reinterpret_cast<const u32x4_t*>(a.dt + int64_t(co0 + (i >> 3)) * a.q + k0_ + \
                                                  (i & 7) * 8);                              \
    }                                                                                        \
    _Pragma("unroll") for (int j = 0; j < XV; ++j) {                                         \
      const int i = tid + j * kWgThreads;                                                    \
      const int row = i / nvec_w, qv = i - row * nvec_w;                                     \
      if (i < nx)                                                                            \
        xreg[j] = *reinterpret_cast<const u32x4_t*>(a.xt + int64_t(ci0 + row) * a.q + k0_ +  \
                                                    qv * 8);                                 \
    }                                                                                        \
  } while (0)
#define XDNA_WG_STORE(buf_)                                                                  \
  do {                                                                                       \
    uint16_t* ds_ = smem + (buf_) * buf_elems;                                               \
    uint16_t* xs_ = ds_ + kTCo * kPitch;                                                     \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                          \
      const int i = tid + j * kWgThreads;                                                    \
      *reinterpret_cast<u32x4_t*>(ds_ + (i >> 3) * kPitch + (i & 7) * 8) = dreg[j];          \
    }                                                                                        \
    _Pragma("unroll") for (int j = 0; j < XV; ++j) {                                         \
      const int i = tid + j * kWgThreads;                                                    \
      const int row = i / nvec_w, qv = i - row * nvec_w;                                     \
      if (i < nx) *reinterpret_cast<u32x4_t*>(xs_ + row * a.xpitch + qv * 8) = xreg[j];      \
    }                                                                                        \
  } while (0)

  if (kt0 < kt1) {
    XDNA_WG_LOAD(kt0);
    XDNA_WG_STORE(0);
  }
  __syncthreads();
  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) XDNA_WG_LOAD(kt + 1);
    const uint16_t* ds = smem + cur * buf_elems;
    const uint16_t* xs = ds + kTCo * kPitch;
    const uint16_t* arow = ds + (wm * 32 + lr) * kPitch + lk;
    const uint16_t* xrow = xs + (wn * 32 + lr) * a.xpitch + lk;
    u32x4_t av[2], lo[2][3];
    uint32_t hi[2][3];
#define XDNA_WG_FRAGS(slot_, ks_)                                                            \
  do {                                                                                       \
    av[slot_] = *reinterpret_cast<const u32x4_t*>(arow + (ks_) * 16);                        \
    _Pragma("unroll") for (int dy = 0; dy < 3; ++dy) {                                       \
      const uint16_t* src_ = xrow + (ks_) * 16 + dy * a.wp8;                                 \
      lo[slot_][dy] = *reinterpret_cast<const u32x4_t*>(src_);                               \
      hi[slot_][dy] = *reinterpret_cast<const uint32_t*>(src_ + 8);                          \
    }                                                                                        \
  } while (0)
    XDNA_WG_FRAGS(0, 0);
#pragma unroll
    for (int ks = 0; ks < kTK / 16; ++ks) {
      const int sl = ks & 1;
      if (ks + 1 < kTK / 16) XDNA_WG_FRAGS(sl ^ 1, ks + 1);
      // keep the next step's LDS reads ahead of this step's MFMAs
      __builtin_amdgcn_sched_barrier(0);
      if (do_bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          bsum += __uint_as_float(av[sl][e] << 16) + __uint_as_float(av[sl][e] & 0xFFFF0000u);
      }
      const bf16x8_t af = as_bf16x8(av[sl]);
#pragma unroll
      for (int dy = 0; dy < 3; ++dy) {
        const u32x4_t l = lo[sl][dy];
        const uint32_t h = hi[sl][dy];
        u32x4_t s1, s2;
        s1[0] = __builtin_amdgcn_alignbit(l[1], l[0], 16);
        s1[1] = __builtin_amdgcn_alignbit(l[2], l[1], 16);
        s1[2] = __builtin_amdgcn_alignbit(l[3], l[2], 16);
        s1[3] = __builtin_amdgcn_alignbit(h, l[3], 16);
        s2[0] = l[1];
        s2[1] = l[2];
        s2[2] = l[3];
        s2[3] = h;
        acc[dy * 3 + 0] = mfma_32x32x16(af, as_bf16x8(l), acc[dy * 3 + 0]);
        acc[dy * 3 + 1] = mfma_32x32x16(af, as_bf16x8(s1), acc[dy * 3 + 1]);
        acc[dy * 3 + 2] = mfma_32x32x16(af, as_bf16x8(s2), acc[dy * 3 + 2]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#undef XDNA_WG_FRAGS
    if (more) XDNA_WG_STORE(cur ^ 1);
    __syncthreads();
  }
#undef XDNA_WG_LOAD
#undef XDNA_WG_STORE

  // Partials: part[split][co][tap][ci]; lanes 0..31 write 32 consecutive ci.
  float* pbase = a.part + int64_t(split) * a.co_pad * 9 * a.ci_pad;
  const int ci = ci0 + wn * 32 + lr;
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int co = co0 + wm * 32 + mfma_row(i, lane);
      pbase[(int64_t(co) * 9 + t) * a.ci_pad + ci] = acc[t][i];
    }
  if (do_bias) {
    // lanes l and l+32 hold the two k-halves of channel row l % 32
    const float other = __shfl_down(bsum, 32, 64);
    if (lane < 32) a.bpart[int64_t(split) * a.co_pad + co0 + wm * 32 + lane] = bsum + other;
  }
}

// gw[co][ci][0..8] = bf16(sum over splits of part[split][co][t][ci]) and gb likewise from
// bpart.  Thread (z, e) of a block owns the (co, ci) pair base + e with its nine taps and
// sums splits z, z + ZG, ... (nine independent loads per split, each coalesced over e);
// the ZG groups are added in order through LDS, a fixed association per output (the
// result is deterministic).  The bf16 results are staged in LDS and the block writes its
// pairs' outputs, one contiguous run of gw, consecutive threads on consecutive elements
// (OIHW keeps the nine taps of a pair together, the partials keep each tap's ci run
// together: the transposition happens in LDS).
template <int ZG>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ part,
                                                           const float* __restrict__ bpart,
                                                           uint16_t* __restrict__ gw,
                                                           uint16_t* __restrict__ gb, int Cout,
                                                           int Cin, int co_pad, int ci_pad,
                                                           int splits) {
  constexpr int EPB = 256 / ZG;
  const int z = threadIdx.x / EPB, e = threadIdx.x % EPB;
  const int64_t npair = int64_t(Cout) * Cin;
  const int64_t stride = int64_t(co_pad) * 9 * ci_pad;
  __shared__ float red[ZG > 1 ? 9 * 256 : 1];
  __shared__ uint16_t ob[9 * EPB];
  for (int64_t base = int64_t(blockIdx.x) * EPB; base < npair; base += int64_t(gridDim.x) * EPB) {
    const int64_t i = base + e;
    float s[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) s[t] = 0.0f;
    if (i < npair) {
      const int co = int(i / Cin), ci = int(i - int64_t(co) * Cin);
      const float* src = part + int64_t(co) * 9 * ci_pad + ci;
      // four splits' 36 loads issued before their sums, which stay in split order
      int k = z;
      for (; k + 3 * ZG < splits; k += 4 * ZG) {
        float v[4][9];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int t = 0; t < 9; ++t) v[u][t] = src[(k + u * ZG) * stride + t * ci_pad];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int t = 0; t < 9; ++t) s[t] += v[u][t];
      }
      for (; k < splits; k += ZG) {
        const float* q = src + k * stride;
#pragma unroll
        for (int t = 0; t < 9; ++t) s[t] += q[t * ci_pad];
      }
    }
    if (ZG > 1) {
#pragma unroll
      for (int t = 0; t < 9; ++t) red[t * 256 + threadIdx.x] = s[t];
      __syncthreads();
      if (z == 0)
        for (int g = 1; g < ZG; ++g)
#pragma unroll
          for (int t = 0; t < 9; ++t) s[t] += red[t * 256 + g * EPB + e];
    }
    if (z == 0)
#pragma unroll
      for (int t = 0; t < 9; ++t) ob[e * 9 + t] = f32_to_bf16(s[t]);
    __syncthreads();
    const int n_out = int(npair - base < EPB ? npair - base : int64_t(EPB)) * 9;
    for (int j = threadIdx.x; j < n_out; j += 256) gw[base * 9 + j] = ob[j];
    __syncthreads();  // red and ob are rewritten by the next pass
  }
  if (gb)
    for (int co = blockIdx.x * 256 + threadIdx.x; co < Cout; co += gridDim.x * 256) {
      float s = 0.0f;
      s = sum_strided8(0.0f, bpart + co, co_pad, 0, 1, splits);
      gb[co] = f32_to_bf16(s);
    }
}

// One thread per output element, for layers with few outputs: gw[co][ci][t] = bf16(sum
// over splits of part[split][co][t][ci]), gb likewise from bpart.  The 256 threads are ZG
// groups of 256 / ZG consecutive elements in partial order (coalesced reads): group z sums
// splits z, z + ZG, ... and the groups are added in order through LDS (a fixed
// association per output), with ZG loads in flight per output when the split count is
// large.  Nine times the threads of wgrad_reduce_kernel: small layers have few outputs and
// many splits.
template <int ZG>
__global__ __launch_bounds__(256) void wgrad_reduce_elem_kernel(const float* __restrict__ part,
                                                                const float* __restrict__ bpart,
                                                                uint16_t* __restrict__ gw,
                                                                uint16_t* __restrict__ gb, int Cout,
                                                                int Cin, int co_pad, int ci_pad,
                                                                int splits) {
  constexpr int EPB = 256 / ZG;
  const int z = threadIdx.x / EPB, e = threadIdx.x % EPB;
  const int64_t n = int64_t(Cout) * 9 * Cin;
  const int64_t stride = int64_t(co_pad) * 9 * ci_pad;
  __shared__ float red[256];
  for (int64_t base = int64_t(blockIdx.x) * EPB; base < n + Cout; base += int64_t(gridDim.x) * EPB) {
    const int64_t i = base + e;
    float s = 0.0f;
    if (i < n) {
      const int ci = int(i % Cin);
      const int t = int((i / Cin) % 9);
      const int co = int(i / (int64_t(Cin) * 9));
      const float* src = part + (int64_t(co) * 9 + t) * ci_pad + ci;
      s = sum_strided8(0.0f, src, stride, z, ZG, splits);
    } else if (i < n + Cout && gb) {
      const int co = int(i - n);
      s = sum_strided8(0.0f, bpart + co, co_pad, z, ZG, splits);
    }
    if (ZG > 1) {
      red[threadIdx.x] = s;
      __syncthreads();
      if (z == 0)
        for (int q = 1; q < ZG; ++q) s += red[q * EPB + e];
      __syncthreads();
    }
    if (z == 0) {
      if (i < n) {
        const int ci = int(i % Cin);
        const int t = int((i / Cin) % 9);
        const int co = int(i / (int64_t(Cin) * 9));
        gw[(int64_t(co) * Cin + ci) * 9 + t] = f32_to_bf16(s);
      } else if (i < n + Cout && gb) {
        gb[i - n] = f32_to_bf16(s);
      }
    }
  }
}

// Launches the split-K reduce of the weight gradient: the pair form (coalesced writes)
// from 65536 (co, ci) pairs on, with at most 16 splits per thread; the element form below
// (its parallelism is what layers with few outputs and many splits need).
void launch_wgrad_reduce(const float* part, const float* bpart, uint16_t* gw, uint16_t* gb, int Cout, int Cin,
                         int co_pad, int ci_pad, int splits, hipStream_t st) {
  const int64_t npair = int64_t(Cout) * Cin;
  if (npair >= 65536) {
    int zg = 1;
    while (zg < 8 && zg * 2 <= splits && ceil_div(splits, zg) > 16) zg *= 2;
    const unsigned grid = unsigned(std::max<int64_t>(std::min<int64_t>(ceil_div(npair, 256 / zg), 16384),
                                                     gb ? ceil_div(Cout, 256) : 1));
#define XDNA_WRED(zg_) wgrad_reduce_kernel<zg_><<<grid, 256, 0, st>>>(part, bpart, gw, gb, Cout, Cin, co_pad, ci_pad, splits)
    switch (zg) {
      case 1: XDNA_WRED(1); break;
      case 2: XDNA_WRED(2); break;
      case 4: XDNA_WRED(4); break;
      default: XDNA_WRED(8); break;
    }
#undef XDNA_WRED
    return;
  }
  const int64_t n = npair * 9 + Cout;
  const int zg = splits >= 64 ? 8 : splits >= 16 ? 4 : splits >= 4 ? 2 : 1;
  const unsigned grid = unsigned(std::min<int64_t>(ceil_div(n, 256 / zg), 8192));
#define XDNA_WRED(zg_) \
  wgrad_reduce_elem_kernel<zg_><<<grid, 256, 0, st>>>(part, bpart, gw, gb, Cout, Cin, co_pad, ci_pad, splits)
  switch (zg) {
    case 1: XDNA_WRED(1); break;
    case 2: XDNA_WRED(2); break;
    case 4: XDNA_WRED(4); break;
    default: XDNA_WRED(8); break;
  }
#undef XDNA_WRED
}

// Bias gradient on its own: one workgroup per channel, fixed-order tree.
// Bias gradient on its own, in two fixed-order stages: workgroup (c, p) sums channel c
// over images [p * ipp, (p + 1) * ipp) into part[c * P + p] (tree over its 256 threads);
// then one wave per channel sums its P parts.  Enough workgroups to fill the GPU even
// for a handful of channels (one workgroup per channel reduced 40 images of 36 x 36 in
// 55 us).
__global__ __launch_bounds__(256) void bias_grad_part_kernel(const uint16_t* __restrict__ dy,
                                                             float* __restrict__ part, int B, int C,
                                                             int64_t plane, int P, int ipp) {
  const int c = blockIdx.x, p = blockIdx.y;
  const int b0 = p * ipp, b1 = min(B, b0 + ipp);
  float s = 0.0f;
  for (int b = b0; b < b1; ++b) {
    const uint16_t* src = dy + (int64_t(b) * C + c) * plane;
    for (int64_t i = threadIdx.x; i < plane; i += 256) s += bf16_to_f32(src[i]);
  }
  __shared__ float red[256];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[int64_t(c) * P + p] = red[0];
}

__global__ __launch_bounds__(256) void bias_grad_sum_kernel(const float* __restrict__ part,
                                                            uint16_t* __restrict__ gb, int C, int P) {
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (c >= C) return;
  float s = 0.0f;
  for (int p = lane; p < P; p += 64) s += part[int64_t(c) * P + p];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0) gb[c] = f32_to_bf16(s);
}

// ---------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------

struct FwdPlan {
  ConvGeom geom;
  int chunks = 0, co_pad = 0;
  size_t packed_bytes = 0, wt_bytes = 0;
};

FwdPlan fwd_plan(int B, int Cin, int Cout, int H, int W) {
  FwdPlan p;
  p.geom = conv_geom(B, H, W);
  p.chunks = int(ceil_div(Cin, kKStep));
  // 128-row channel tiles; beyond 128 channels, a multiple of 256 for the wide kernel
  p.co_pad = Cout <= kTCo ? kTCo : int(ceil_div(Cout, kWCo) * kWCo);
  p.packed_bytes = align256(size_t(p.geom.groups) * p.chunks * kGroupRows * kKStep * 2);
  p.wt_bytes = align256(size_t(p.co_pad) * p.chunks * 9 * kKStep * 2);
  return p;
}

bool shape_ok(const char* what, int B, int Cin, int Cout, int H, int W) {
  if (B < 1 || Cin < 1 || Cout < 1 || H < 1 || W < 1) {
    set_error(std::string(what) + ": invalid shape");
    return false;
  }
  return true;
}

// The forward form (wt) and / or the input-gradient form (wtd) of an OIHW weight in one
// launch of prep_tiled_kernel.
// output-channel tile of the weight preparation: 0 by size, else 8 or 32
std::atomic<int> g_prep_co{0};

int launch_prep_tiled(const uint16_t* w, uint16_t* wt, uint16_t* wtd, int Cout, int Cin, void* stream) {
  if (!admit_launch("conv3x3 weight preparation")) return -1;
  const FwdPlan pf = fwd_plan(1, Cin, Cout, 1, 1), pd = fwd_plan(1, Cout, Cin, 1, 1);
  // extents: forward rows co_pad_f x chunks_f * 64 columns; gradient rows co_pad_d (over
  // ci) x chunks_d * 64 (over co)
  const int ci_ext = std::max(wt ? pf.chunks * kKStep : 0, wtd ? pd.co_pad : 0);
  const int co_ext = std::max(wt ? pf.co_pad : 0, wtd ? pd.chunks * kKStep : 0);
  const int vec = (Cin % 8 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) ? 1 : 0;
  const int64_t blocks32 = ceil_div(ci_ext, kPrepCi) * ceil_div(co_ext, 32);
  const int co_tile = g_prep_co.load() ? g_prep_co.load() : (blocks32 < 256 ? 8 : 32);
  const dim3 grid(unsigned(ceil_div(ci_ext, kPrepCi)), unsigned(ceil_div(co_ext, co_tile)));
  if (co_tile == 8)
    prep_tiled_kernel<8><<<grid, 64, 0, as_stream(stream)>>>(w, wt, wtd, Cout, Cin, pf.co_pad, pf.chunks, pd.co_pad,
                                                             pd.chunks, vec);
  else
    prep_tiled_kernel<32><<<grid, 256, 0, as_stream(stream)>>>(w, wt, wtd, Cout, Cin, pf.co_pad, pf.chunks, pd.co_pad,
                                                               pd.chunks, vec);
  return check_launch("conv3x3 weight preparation");
}

// prep_multi_kernel over n weights, in launches of up to kPrepJobs
int launch_prep_multi(int n, const uint16_t* const* w, uint16_t* const* wt, uint16_t* const* wtd, const int* cout,
                      const int* cin, void* stream) {
  for (int first = 0; first < n; first += kPrepJobs) {
    PrepJobs jobs{};
    jobs.n = std::min(kPrepJobs, n - first);
    int blocks = 0;
    for (int e = 0; e < jobs.n; ++e) {
      const int i = first + e;
      const FwdPlan pf = fwd_plan(1, cin[i], cout[i], 1, 1), pd = fwd_plan(1, cout[i], cin[i], 1, 1);
      const int ci_ext = std::max(wt[i] ? pf.chunks * kKStep : 0, wtd[i] ? pd.co_pad : 0);
      const int co_ext = std::max(wt[i] ? pf.co_pad : 0, wtd[i] ? pd.chunks * kKStep : 0);
      PrepJob& J = jobs.j[e];
      J = PrepJob{w[i], wt[i], wtd[i], cout[i], cin[i], pf.co_pad, pf.chunks, pd.co_pad, pd.chunks,
                  int(ceil_div(ci_ext, kPrepCi)),
                  (cin[i] % 8 == 0 && (reinterpret_cast<uintptr_t>(w[i]) & 15) == 0) ? 1 : 0, blocks};
      blocks += J.gx * int(ceil_div(co_ext, 8));
    }
    if (blocks == 0) continue;
    if (!admit_launch("conv3x3 weight preparation (several weights)")) return -1;
    prep_multi_kernel<<<unsigned(blocks), 64, 0, as_stream(stream)>>>(jobs);
    if (check_launch("conv3x3 weight preparation (several weights)")) return -1;
  }
  return 0;
}

int launch_prep(const uint16_t* w, uint16_t* wt, int Cout, int Cin, int co_pad, int chunks,
                int dgrad, void* stream) {
  (void)co_pad;
  (void)chunks;
  return dgrad ? launch_prep_tiled(w, nullptr, wt, Cout, Cin, stream)
               : launch_prep_tiled(w, wt, nullptr, Cout, Cin, stream);
}

// The rows kernels' epilogue form, a compile-time choice (the epilogue is straight-line code
// run once per tile, and a kernel carrying every form was twice the size): 0 buffer stores,
// 1 buffer stores with the fused ReLU, 2 per-element pointers (outputs past the buffer
// stores' 1 GiB range, or grids of 2^31 rows or more), activation read at run time.
int rows_epilogue(const RowsArgs& a) { return !a.out_rs ? 2 : a.act ? 1 : 0; }

template <int MT, int NT, int WM, int OCC = 1>
int launch_rows4(RowsArgs a, const ConvGeom& geom, int cout, hipStream_t st) {
  using Q = Q4<MT, NT, WM>;
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows4_kernel<MT, NT, WM, OCC, 0>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows4_kernel<MT, NT, WM, OCC, 1>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows4_kernel<MT, NT, WM, OCC, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess;
  if (!lds_ok) {
    set_error("conv3x3 rows: cannot enable the four-wave kernel's LDS size");
    return -1;
  }
  a.nrt = int(ceil_div(geom.m_total, Q::TP));
  a.ncot = int(ceil_div(cout, Q::CO));
  const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, 1);
  switch (rows_epilogue(a)) {
    case 0: conv_rows4_kernel<MT, NT, WM, OCC, 0><<<grid, 256, Q::Lds, st>>>(a); break;
    case 1: conv_rows4_kernel<MT, NT, WM, OCC, 1><<<grid, 256, Q::Lds, st>>>(a); break;
    default: conv_rows4_kernel<MT, NT, WM, OCC, 2><<<grid, 256, Q::Lds, st>>>(a); break;
  }
  return check_launch("conv3x3 rows");
}

template <int MI, int NJ, int WM, int OCC = 1>
int launch_rows6(RowsArgs a, const ConvGeom& geom, int cout, hipStream_t st) {
  using Q = Q6<MI, NJ, WM, OCC>;
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows6_kernel<MI, NJ, WM, OCC, 0>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows6_kernel<MI, NJ, WM, OCC, 1>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows6_kernel<MI, NJ, WM, OCC, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(Q::Lds)) == hipSuccess;
  if (!lds_ok) {
    set_error("conv3x3 rows: cannot enable the 16x16x32 kernel's LDS size");
    return -1;
  }
  a.nrt = int(ceil_div(geom.m_total, Q::TP));
  a.ncot = int(ceil_div(cout, Q::CO));
  const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, 1);
  switch (rows_epilogue(a)) {
    case 0: conv_rows6_kernel<MI, NJ, WM, OCC, 0><<<grid, 256, Q::Lds, st>>>(a); break;
    case 1: conv_rows6_kernel<MI, NJ, WM, OCC, 1><<<grid, 256, Q::Lds, st>>>(a); break;
    default: conv_rows6_kernel<MI, NJ, WM, OCC, 2><<<grid, 256, Q::Lds, st>>>(a); break;
  }
  return check_launch("conv3x3 rows");
}

// conv of packed input xp (cin channels) with prepared weights -> NCHW out (cout channels).
std::atomic<int> g_rows_variant{[] {
  const char* e = std::getenv("XDNA_ROWS_VARIANT");
  return e ? std::atoi(e) : 0;
}()};

RowsArgs rows_args(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* out, int B, int cin,
                   int cout, int H, int W, const ConvGeom& geom, int act) {
  RowsArgs a;
  a.act = act;
  a.osh = 0;
  a.oH = H;
  a.oW = W;
  a.xp = xp;
  a.xsrc = nullptr;
  a.cin = cin;
  a.wt = wt;
  a.bias = bias;
  a.out = out;
  a.part = nullptr;
  a.chunks = int(ceil_div(cin, kKStep));
  a.cout = cout;
  a.wp = geom.st.wp;
  a.H = H;
  a.W = W;
  a.S = geom.st.S;
  a.So = geom.st.So;
  a.first = geom.st.first;
  a.ch_per = a.chunks;
  a.img = geom.img;
  a.m_total = geom.m_total;
  a.m_pad = int64_t(geom.groups) * kGroupOutRows;
  a.B = B;
  a.bias_vec = bias && (reinterpret_cast<uintptr_t>(bias) & 7) == 0 && cout % 4 == 0 ? 1 : 0;
  {
    // images a tile of up to 512 grid rows can touch, and the bytes they span
    const int64_t span = (512 - 1) / geom.img + 2;
    a.out_rs = span * cout * int64_t(H) * W * 2 < kOutSkip && geom.m_total < (int64_t(1) << 31) ? 1 : 0;
  }
  return a;
}

// LDS of the small-grid kernel with TP-row tiles
constexpr size_t small_lds(int TP) { return size_t(TP + kMaxHalo) * kPitch * 2 + size_t(kSCo) * kSWPitch * 2; }

// The small-grid kernel's epilogue form, a compile-time choice: 0 buffer stores, 1 split-K
// partials, 2 per-element pointers (outputs past the buffer stores' 1 GiB range), 3 buffer
// stores with the fused ReLU.
int small_epilogue(const RowsArgs& a) { return a.part ? 1 : !a.out_rs ? 2 : a.act ? 3 : 0; }

template <int TP, bool EMUL, bool NCHW>
bool small_lds_set() {
  const auto set = [](const void* f) {
    return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(small_lds(TP))) == hipSuccess;
  };
  return set(reinterpret_cast<const void*>(&conv_small_kernel<TP, EMUL, NCHW, 0>)) &&
         set(reinterpret_cast<const void*>(&conv_small_kernel<TP, EMUL, NCHW, 1>)) &&
         set(reinterpret_cast<const void*>(&conv_small_kernel<TP, EMUL, NCHW, 2>)) &&
         set(reinterpret_cast<const void*>(&conv_small_kernel<TP, EMUL, NCHW, 3>));
}

bool small_nchw_lds_ok() {
  static const bool ok = small_lds_set<64, false, true>() && small_lds_set<128, false, true>();
  return ok;
}

template <bool EMUL>
bool small_lds_ok() {
  static const bool ok = small_lds_set<64, EMUL, false>() && small_lds_set<128, EMUL, false>();
  return ok;
}

template <int TP, bool EMUL, bool NCHW>
void launch_small_kernel(const RowsArgs& a, dim3 grid, hipStream_t st) {
  switch (small_epilogue(a)) {
    case 0: conv_small_kernel<TP, EMUL, NCHW, 0><<<grid, 256, small_lds(TP), st>>>(a); break;
    case 1: conv_small_kernel<TP, EMUL, NCHW, 1><<<grid, 256, small_lds(TP), st>>>(a); break;
    case 2: conv_small_kernel<TP, EMUL, NCHW, 2><<<grid, 256, small_lds(TP), st>>>(a); break;
    default: conv_small_kernel<TP, EMUL, NCHW, 3><<<grid, 256, small_lds(TP), st>>>(a); break;
  }
}

int launch_small(RowsArgs a, const ConvGeom& geom, int B, int cout, int variant, hipStream_t st);

// Whether launch_rows would run this conv on the small-grid kernel and the kernel's NCHW
// form can read the input in place: images up to 36 columns (one strip), input channels a
// multiple of 8 (whole 8-channel pieces), an input under 2 GiB (32-bit buffer offsets).
bool nchw_small_ok(int B, int cin, int cout, int H, int W) {
  if (B < 1 || cin < 1 || cout < 1 || H < 1 || W < 1 || W > kMaxWidth || cin % 8 != 0) return false;
  if (int64_t(B) * cin * H * W * 2 >= (int64_t(1) << 31)) return false;
  const int variant = g_rows_variant.load();
  if (variant == 2 || variant == 3) return true;
  if (variant != 0) return false;
  const ConvGeom geom = conv_geom(B, H, W, kLayoutTight);
  return ceil_div(geom.m_total, 256) * ceil_div(cout, kSCo) < 150;
}

int launch_rows_nchw(const uint16_t* x, const uint16_t* wt, const uint16_t* bias, uint16_t* out, int B, int cin,
                     int cout, int H, int W, int act, bool s2out, void* stream) {
  const ConvGeom geom = conv_geom(B, H, W, kLayoutTight);
  RowsArgs a = rows_args(nullptr, wt, bias, out, B, cin, cout, H, W, geom, act);
  a.xsrc = x;
  if (s2out) {
    a.osh = 1;
    a.oH = (H + 1) / 2;
    a.oW = (W + 1) / 2;
    if (!a.out_rs) {
      set_error("conv3x3 nchw: the stride-2 output needs the buffer-store epilogue (output too large)");
      return -1;
    }
  }
  if (!admit_launch("conv3x3 nchw")) return -1;
  const int v = g_rows_variant.load();
  return launch_small(a, geom, B, cout, v == 2 || v == 3 ? v : -1, as_stream(stream));
}

int launch_rows(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* out,
                int B, int cin, int cout, int H, int W, void* stream, int layout = kLayoutRef, int act = 0,
                bool s2out = false) {
  const ConvGeom geom = conv_geom(B, H, W, layout);
  RowsArgs a = rows_args(xp, wt, bias, out, B, cin, cout, H, W, geom, act);
  if (s2out) {
    a.osh = 1;
    a.oH = (H + 1) / 2;
    a.oW = (W + 1) / 2;
    if (!a.out_rs) {
      set_error("conv3x3 rows: the stride-2 output needs the buffer-store epilogue (output too large)");
      return -1;
    }
  }
  if (!admit_launch("conv3x3 rows")) return -1;
  hipStream_t st = as_stream(stream);
  // Kernel choice (xdna_conv3x3_set_rows_variant, or XDNA_ROWS_VARIANT at start-up,
  // overrides it: 1 main kernel, 2 / 3 small-grid kernel with 64 / 128-row tiles).  The
  // main kernel needs a grid of several workgroups per CU to hide its per-tap weight
  // loads; below that the small-grid kernel, which stages whole chunks, is faster.
  int variant = g_rows_variant.load();
  // the stride-2 output is stored by the buffer-store epilogues only: the main and the
  // eight-wave kernels (variants 1, 4; 5 up to 128 channels) have none
  if (s2out && (variant == 1 || variant == 4 || (variant == 5 && cout <= kTCo))) variant = 0;
  const unsigned ytiles = unsigned(ceil_div(cout, kTCo));
  if (variant == 0) {
    // Automatic choice (fitted to the sweep shapes on an MI355X).  Grids of a few hundred
    // 128-row tiles or less: the small-grid kernel (whole chunks staged per workgroup,
    // split-K below the CU count).  Otherwise the four-wave kernel whose modelled time
    //   ceil(workgroups / 256) * (tile channels * tile rows) * per-MFMA cost
    // is least (one workgroup per CU; the 128 x 256 and 64 x 512 tiles issue 8 MFMAs per 6
    // fragment reads instead of 16 per 8: cost 1.1).  Ties go to the first candidate.
    // Below ~150 workgroups of the 64 x 256 two-per-CU kernel: the small-grid kernel.  Up
    // to 256 output channels: the two-per-CU kernel (its second workgroup hides the
    // per-tap weight loads and the prologue of the other; measured 7 % ahead of the
    // one-per-CU tiles over the sweep's C <= 256 shapes).  Wider: the modelled choice.
    const int64_t wgs9 = ceil_div(geom.m_total, 256) * ceil_div(cout, kSCo);
    if (wgs9 < 150) {
      variant = -1;
    } else if (cout <= 2 * kTCo) {
      // its 16x16x32 form (variant 11) from 256 output channels on grids of 300 such
      // workgroups or more: 0.5-3.4 % less step time on the sweep's C256 shapes with H >= 36,
      // 2-4 us more on the small ones
      variant = cout > kTCo && wgs9 >= 300 ? 11 : 9;
    } else {
      // slots: workgroups one round holds (256 CUs x workgroups per CU)
      struct Cand { int v, co, tp, slots; double cost; };
      // (the 128 x 512 tile in its 16x16x32 form, variant 10: 2.8 % less time per conv
      // step than variant 7 on N64 C512 H72, 1-5 % on the sweep's other 512-channel shapes)
      const Cand all[] = {{10, 128, 512, 256, 1.0}, {5, 256, 256, 256, 1.0}, {6, 128, 256, 256, 1.1},
                          {9, 64, 256, 512, 1.05}};
      double best = 1e300;
      for (const Cand& c : all) {
        const int64_t wgs = ceil_div(geom.m_total, c.tp) * ceil_div(cout, c.co);
        const double t = double(ceil_div(wgs, c.slots)) * (c.slots / 256) * double(c.co) * c.tp * c.cost;
        if (t < best) {
          best = t;
          variant = c.v;
        }
      }
    }
  }
  const bool small = variant == 2 || variant == 3 || variant == -1;
  // four-wave kernels with 128- or 64-channel tiles: any cout (the prepared weights cover
  // every tile: 128 rows up to 128 channels, a multiple of 256 beyond)
  if (variant == 6) return launch_rows4<2, 4, 2>(a, geom, cout, st);
  if (variant == 7) return launch_rows4<4, 4, 1>(a, geom, cout, st);
  if (variant == 8) return launch_rows4<2, 4, 1>(a, geom, cout, st);
  // 64 x 256 tiles, two workgroups per CU (76 KB of LDS each)
  if (variant == 9) return launch_rows4<2, 2, 1, 2>(a, geom, cout, st);
  // the 16x16x32 forms of variants 7 and 9
  if (variant == 10) return launch_rows6<8, 8, 1>(a, geom, cout, st);
  if (variant == 11) return launch_rows6<4, 4, 1, 2>(a, geom, cout, st);
  // the wide kernels: 256-channel tiles (cout > 128 only: the weights are padded to 256
  // rows from there on); the four-wave form unless the eight-wave one is asked for
  const bool wide = cout > kTCo && (variant == 4 || variant == 5);
  if (wide) {
    if (variant != 4) return launch_rows4<4, 4, 2>(a, geom, cout, st);
    static const bool lds_wide =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_rows2_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(kWideLds)) == hipSuccess;
    if (!lds_wide) {
      set_error("conv3x3 rows: cannot enable the wide kernel's LDS size");
      return -1;
    }
    a.nrt = int(ceil_div(geom.m_total, kWTp));
    a.ncot = int(ceil_div(cout, kWCo));
    const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, 1);
    conv_rows2_kernel<<<grid, 512, kWideLds, st>>>(a);
    return check_launch("conv3x3 rows");
  }
  if (!small) {
    // Tile rows per workgroup: the largest of 256 / 128 / 64 that still puts a few
    // hundred workgroups on the 256 CUs.
    const int64_t wg256 = int64_t(geom.groups) * (kGroupOutRows / 256) * ytiles;
    const int64_t wg128 = int64_t(geom.groups) * (kGroupOutRows / 128) * ytiles;
    const int TP = wg256 >= 384 ? 256 : wg128 >= 384 ? 128 : 64;
    a.nrt = int(ceil_div(geom.m_total, TP));
    a.ncot = int(ytiles);
    const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, 1);
    if (TP == 256)
      conv_rows_kernel<256><<<grid, 256, 0, st>>>(a);
    else if (TP == 128)
      conv_rows_kernel<128><<<grid, 256, 0, st>>>(a);
    else
      conv_rows_kernel<64><<<grid, 256, 0, st>>>(a);
    return check_launch("conv3x3 rows");
  }
  return launch_small(a, geom, B, cout, variant, st);
}

// The small-grid kernel (variant 2 / 3 force its 64 / 128-row tiles; otherwise by grid
// size), with split-K below 64 workgroups; a.xsrc set: its NCHW form.
int launch_small(RowsArgs a, const ConvGeom& geom, int B, int cout, int variant, hipStream_t st) {
  const bool nchw = a.xsrc != nullptr;
  // 32-bit row indexes and weight-slab offsets in the kernel
  if (geom.m_total >= (int64_t(1) << 30) || int64_t(kSCo) * a.chunks * 9 * kKStep * 2 >= (int64_t(1) << 31)) {
    set_error("conv3x3 rows: grid or weights too large for the small-grid kernel");
    return -1;
  }
  if (nchw ? !small_nchw_lds_ok() : !small_lds_ok<false>()) {
    set_error("conv3x3 rows: cannot enable the small-grid kernel's LDS size");
    return -1;
  }
  const unsigned stiles = unsigned(ceil_div(cout, kSCo));
  const int64_t tp128_min = 128;  // measured on the sweep shapes
  const int TP = variant == 2 ? 64 : variant == 3 ? 128 : (ceil_div(geom.m_total, 128) * stiles >= tp128_min ? 128 : 64);
  const int64_t valid = ceil_div(geom.m_total, TP) * stiles;
  // Fewer workgroups than CUs: split the input chunks over blockIdx.z and sum the fp32
  // partials in a second pass (in split order).
  int nsplit = 1;
  if (valid <= 64 && a.chunks >= 2) {
    nsplit = int(std::min<int64_t>(a.chunks, ceil_div(256, valid)));
    a.ch_per = int(ceil_div(a.chunks, nsplit));
    nsplit = int(ceil_div(a.chunks, a.ch_per));
  }
  if (nsplit > 1) {
    const size_t pbytes = size_t(nsplit) * size_t(cout) * size_t(a.m_pad) * sizeof(float);
    a.part = static_cast<float*>(xdna_hip_cache_alloc(pbytes));
    if (!a.part) return -1;
  }
  a.nrt = int(ceil_div(geom.m_total, TP));
  a.ncot = int(stiles);
  const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, unsigned(nsplit));
  if (nchw && TP == 128)
    launch_small_kernel<128, false, true>(a, grid, st);
  else if (nchw)
    launch_small_kernel<64, false, true>(a, grid, st);
  else if (TP == 128)
    launch_small_kernel<128, false, false>(a, grid, st);
  else
    launch_small_kernel<64, false, false>(a, grid, st);
  if (nsplit > 1) {
    const unsigned pix_blocks = unsigned(ceil_div(int64_t(a.oH) * a.oW, 256));
    const int planes = B * cout;
    for (int p0 = 0; p0 < planes; p0 += 65535)
      rows_reduce_kernel<<<dim3(pix_blocks, unsigned(std::min(65535, planes - p0))), 256, 0, st>>>(a, nsplit, p0);
    // stream-ordered reuse: the next user of the block runs after the reduce
    xdna_hip_cache_free(a.part);
  }
  return check_launch("conv3x3 rows");
}

// The BFP16 emulation of the reference NPU's conv: the packed rows and the prepared
// weights quantized to BFP16 values (8-element blocks: 8 channels of a pixel, 8 channels
// of a (row, tap) of the weights, which are the codec's blocks), then the small-grid kernel
// in its EMUL form over every tile, without split-K.  The quantized copies are transient.
int launch_rows_emul(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* out, int B, int cin,
                     int cout, int H, int W, void* stream, int layout, int act) {
  const ConvGeom geom = conv_geom(B, H, W, layout);
  const int chunks = int(ceil_div(cin, kKStep));
  const size_t xbytes = size_t(geom.groups) * chunks * kGroupRows * kKStep * 2;
  const size_t wbytes = xdna_conv3x3_prepared_weight_bytes(cin, cout);
  if (!small_lds_ok<true>()) {
    set_error("conv3x3 BFP16 emulation: cannot enable the small-grid kernel's LDS size");
    return -1;
  }
  if (geom.m_total >= (int64_t(1) << 30) || int64_t(kSCo) * chunks * 9 * kKStep * 2 >= (int64_t(1) << 31)) {
    set_error("conv3x3 BFP16 emulation: grid or weights too large for the small-grid kernel");
    return -1;
  }
  uint16_t* xq = static_cast<uint16_t*>(xdna_hip_cache_alloc(xbytes));
  if (!xq) return -1;
  uint16_t* wq = static_cast<uint16_t*>(xdna_hip_cache_alloc(wbytes));
  if (!wq) {
    xdna_hip_cache_free(xq);
    return -1;
  }
  int rc = xdna_bfp16_quantize8_bf16(xp, xq, int64_t(xbytes / 16), stream);
  if (rc == 0) rc = xdna_bfp16_quantize8_bf16(wt, wq, int64_t(wbytes / 16), stream);
  if (rc == 0 && admit_launch("conv3x3 BFP16 emulation")) {
    RowsArgs a = rows_args(xq, wq, bias, out, B, cin, cout, H, W, geom, act);
    const unsigned stiles = unsigned(ceil_div(cout, kSCo));
    const int TP = ceil_div(geom.m_total, 128) * stiles >= 128 ? 128 : 64;
    a.nrt = int(ceil_div(geom.m_total, TP));
    a.ncot = int(stiles);
    const dim3 grid(unsigned(ceil_div(a.nrt, kXcds) * kXcds * a.ncot), 1, 1);
    if (TP == 128)
      launch_small_kernel<128, true, false>(a, grid, as_stream(stream));
    else
      launch_small_kernel<64, true, false>(a, grid, as_stream(stream));
    rc = check_launch("conv3x3 BFP16 emulation");
  } else if (rc == 0) {
    rc = -1;
  }
  // stream-ordered reuse: the next user of either block runs after the conv
  xdna_hip_cache_free(wq);
  xdna_hip_cache_free(xq);
  return rc;
}

struct WgradPlan {
  CmGeom cm;
  int ci_pad = 0, co_pad = 0, splits = 0, kt_per = 0, xpitch = 0, wlen = 0;
  size_t xt_bytes = 0, dt_bytes = 0, part_bytes = 0, bpart_bytes = 0;
  size_t lds_bytes = 0;
};

WgradPlan wgrad_plan(int B, int Cin, int Cout, int H, int W) {
  WgradPlan p;
  p.cm = cm_geom(B, H, W);
  p.ci_pad = int(ceil_div(Cin, 64) * 64);
  // 128-row channel tiles; beyond 128 channels, a multiple of 256 for the wide kernel
  p.co_pad = Cout <= kTCo ? kTCo : int(ceil_div(Cout, kWCo) * kWCo);
  const int64_t tiles = int64_t(p.ci_pad / 64) * (p.co_pad / kTCo);
  const int64_t out_elems = int64_t(p.co_pad) * 9 * p.ci_pad;
  // Split-K: pick the split count s that minimizes a simple model of the two kernels,
  //   rounds(s) * flops / (tiles * s * per-CU rate) + (write + read of s fp32 partials) / BW,
  // with rounds(s) = ceil(tiles * s / 256): one workgroup fits a CU (its LDS and 8 waves
  // of 256 registers), so a grid of 257 workgroups takes two full workgroup times.
  const double flops = 2.0 * 9.0 * double(B) * H * W * double(Cin) * double(Cout);
  const double cu_rate = 4.0e12, bw = 5.0e12;
  int64_t best = 1;
  double best_t = 1e30;
  const int64_t smax = std::min<int64_t>(p.cm.ktiles, 4096);
  for (int64_t s = 1; s <= smax; s = s < 512 ? s + 1 : s + s / 8) {
    const double rounds = double(ceil_div(tiles * s, 256));
    const double t = rounds * flops / (double(tiles * s) * cu_rate) + 2.0 * double(s) * double(out_elems) * 4.0 / bw;
    if (t < best_t) {
      best_t = t;
      best = s;
    }
  }
  p.kt_per = int(ceil_div(p.cm.ktiles, best));
  p.splits = int(ceil_div(p.cm.ktiles, p.kt_per));
  p.wlen = kTK + 2 * p.cm.wp8 + 8;
  p.xpitch = int(ceil_div(p.wlen, 16) * 16 + 8);
  p.xt_bytes = align256(size_t(p.ci_pad) * p.cm.q * 2);
  p.dt_bytes = align256(size_t(p.co_pad) * p.cm.q * 2);
  p.part_bytes = align256(size_t(p.splits) * out_elems * 4);
  p.bpart_bytes = align256(size_t(p.splits) * p.co_pad * 4);
  p.lds_bytes = 2 * (size_t(kTCo) * kPitch * 2 + size_t(64) * p.xpitch * 2);  // double-buffered
  return p;
}

constexpr size_t kMaxWgradLds = 160 * 1024;

// Output rows per k-tile of the rows weight gradient (64 or 128; XDNA_WGRAD_KT at start-up,
// xdna_conv3x3_set_wgrad_rows_kt).
std::atomic<int> g_wgrad_rows_kt{[] {
  const char* e = std::getenv("XDNA_WGRAD_KT");
  return e && std::atoi(e) == 64 ? 64 : 128;
}()};

// ---------------------------------------------------------------------------------------
// Weight gradient on the packed row layout: x and dY as the forward and input-gradient
// convolutions already pack them ([group][chunk][2126 rows][64 channels], one padded-grid
// position per row), so no channel-major copy of either is made.  Output row p of group g
// (the centre of its pixel is packed row p + wp + 1) pairs dY there with x rows
// p + dy*wp + dx, all inside the group's 2126 rows, as in the forward kernel.
//
// One workgroup (8 waves): 128 output channels x 64 input channels x 9 taps over the
// k-tiles (64 output rows) of one split.  The dY tile ([64 rows][128 channels]) and the
// x window ([64 + 2wp + 2 rows][64 channels]) sit in LDS in that row-major form and every
// MFMA fragment (8 consecutive rows of one channel) is read with two transposing LDS
// reads (ds_read_tr16_b64); any row offset is aligned, so a tap is a row offset.  Per
// 16-row step a wave reads its dY fragment once and 12 consecutive x rows per kernel row
// (three reads), building dx = 0, 1, 2 from them with alignbit.  Strip halo columns
// (images wider than 36 are packed as strips with one real column on each side) are
// zeroed in the dY tile: those pixels belong to the neighbouring strip.  Either row layout
// (the reference's, or the tight one without zero columns).
// LDS pitch of the dY tile: 160 elements (80 dwords, 16 mod 64) puts the 4 rows x 2
// column halves of a half-wave transposing read on 8 distinct groups of 8 banks (144 put
// two of them on the same banks)
constexpr int kWrA = 128 + 32;
// LDS pitch of the x window: 96 elements (192 bytes, 64 mod 128) keeps the 32 lanes of a
// half-wave transposing read on distinct banks of gfx950's 64 (5.5x fewer conflicts than
// 80 on the largest sweep shape)
constexpr int kWrX = 96;
// x-window vectors per thread for k-tiles of KT rows (8 * (KT + 2*38 + 2) vectors per window)
template <int KT>
constexpr int wr_xv() { return (8 * (KT + 2 * 38 + 2) + 511) / 512; }

struct WgRowsArgs {
  const uint16_t* xp;  // packed x  [groups][ci_chunks][2126][64]
  const uint16_t* dp;  // packed dY [groups][co_chunks][2126][64]
  float* part;         // [splits][co_pad][9][ci_pad]
  float* bpart;        // [splits][co_pad]
  int ci_chunks, co_chunks, ci_pad, co_pad;
  int wp, S, Wg, lead;
  int64_t img, m_total;
  int ktiles, kt_per_split, splits, nco_t, ntiles;
};

typedef short wr_i16x4 __attribute__((ext_vector_type(4)));

// Lane part of a transposing LDS read of a row-major tile: in 16-lane group g = lane / 16
// (columns +16 (g % 2), rows +8 (g / 2)), lane j supplies (row + j / 4, column + 4 (j % 4)),
// and every lane receives 4 consecutive rows of its own column as two dwords.
__device__ inline int wr_lane_off(int pitch, int lane) {
  const int g = lane >> 4, j = lane & 15;
  return (8 * (g >> 1) + (j >> 2)) * pitch + 16 * (g & 1) + 4 * (j & 3);
}

__device__ inline uint2 wr_tr(const uint16_t* p) {
  const wr_i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) wr_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// KT: output rows per k-tile (64 or 128).
template <int KT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void wgrad_rows_kernel(WgRowsArgs a) {
  constexpr int kDv = KT / 32;          // dY vectors per thread
  constexpr int kXv = wr_xv<KT>();      // x-window vectors per thread
  constexpr int kTilesPerGroup = kGroupOutRows / KT;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int xrows = KT + 2 * a.wp + 2;
  // the third read of a kernel row reaches up to 2 rows past the window (values never
  // used): the buffer holds 4 more rows
  const int buf_elems = KT * kWrA + (xrows + 4) * kWrX;
  // blockIdx.x -> (co tile, ci tile, split): a split's channel tiles share one XCD
  const int L = blockIdx.x;
  const int xcd = L % kXcds, kq = L / kXcds;
  const int tile = kq % a.ntiles;
  const int split = (kq / a.ntiles) * kXcds + xcd;
  if (split >= a.splits) return;
  const int co_t = tile % a.nco_t, ci_t = tile / a.nco_t;
  const int co0 = co_t * kTCo, ci0 = ci_t * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int kt0 = split * a.kt_per_split;
  const int kt1 = min(a.ktiles, kt0 + a.kt_per_split);
  const int nxv = xrows * 8;

  f32x16_t acc[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) acc[t] = zero_acc();
  float bsum = 0.0f;
  const bool do_bias = a.bpart && ci_t == 0 && wn == 0;

  // Per-thread load offsets (elements from the k-tile's base), fixed over the k-tiles.
  // dY vector j: row tid / 16 + 32 j, channels (tid % 16) * 8 of the tile's 128; x vector
  // j: window row tid / 8 + 64 j, channels (tid % 8) * 8.  Vector j is vector 0 plus a
  // compile-time offset, so one register of each kind is kept.
  const bool strips = a.S > 1;
  const int d_row0 = tid >> 4;
  const int d_chunk = co0 / 64 + ((tid >> 3) & 1);
  const bool d_chunk_ok = d_chunk < a.co_chunks;
  const int d_off0 = (min(d_chunk, a.co_chunks - 1) * kGroupRows + d_row0 + a.wp + 1) * kKStep + (tid & 7) * 8;
  const int d_rmod0 = d_row0 % a.wp;
  const int x_off0 = (tid >> 3) * kKStep + (tid & 7) * 8;
  const int x_offmax = ((nxv - 1) >> 3) * kKStep + ((nxv - 1) & 7) * 8;

  u32x4_t dreg[kDv];
  u32x4_t xreg[kXv];
  bool dok[kDv];
  // k-tile kt: group kt / kTilesPerGroup, output rows (kt % kTilesPerGroup) * KT of it,
  // i.e. global output rows p = KT kt + row
  auto load = [&](int kt) {
    const int g = kt / kTilesPerGroup, r0 = (kt % kTilesPerGroup) * KT;
    const int64_t rem = a.m_total - int64_t(kt) * KT;  // rows of this tile before the end
    // strip halo columns: p % wp = ((KT kt) % wp + (32 j) % wp (both wave-uniform) +
    // row0 % wp), each term below wp, reduced by two subtractions
    const int base = int((uint32_t(kt) * uint32_t(KT)) % uint32_t(a.wp));
    const uint16_t* db = a.dp + (int64_t(g) * a.co_chunks * kGroupRows + r0) * kKStep;
#pragma unroll
    for (int j = 0; j < kDv; ++j) {
      // branch-free: data column of the centre row p + wp + 1 (row position jc + 1,
      // wrapping to the next row's position 0); a strip's halo columns are masked
      int jc = base + int(uint32_t(32 * j) % uint32_t(a.wp)) + d_rmod0;
      jc -= jc >= a.wp ? a.wp : 0;
      jc -= jc >= a.wp ? a.wp : 0;
      int dj = jc + 1 - a.lead;
      dj = dj == a.wp ? 0 : dj;
      const bool halo = strips && (dj == 0 || dj == a.Wg - 1);
      dok[j] = d_chunk_ok && d_row0 + 32 * j < rem && !halo;
      dreg[j] = *reinterpret_cast<const u32x4_t*>(db + d_off0 + 32 * j * kKStep);
    }
    const uint16_t* xb = a.xp + ((int64_t(g) * a.ci_chunks + ci0 / 64) * kGroupRows + r0) * kKStep;
#pragma unroll
    for (int j = 0; j < kXv; ++j)
      xreg[j] = *reinterpret_cast<const u32x4_t*>(xb + min(x_off0 + 64 * j * kKStep, x_offmax));
  };
  auto store = [&](int buf) {
    uint16_t* as = smem + buf * buf_elems;
    uint16_t* xs = as + KT * kWrA;
#pragma unroll
    for (int j = 0; j < kDv; ++j) {
      const int i = tid + j * 512;
      const u32x4_t z = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(as + (i >> 4) * kWrA + (i & 15) * 8) = dok[j] ? dreg[j] : z;
    }
#pragma unroll
    for (int j = 0; j < kXv; ++j) {
      const int i = tid + j * 512;
      if (i < nxv) *reinterpret_cast<u32x4_t*>(xs + (i >> 3) * kWrX + (i & 7) * 8) = xreg[j];
    }
  };

  // LDS read bases of this lane: dY rows at + q * kWrA, x rows of kernel row dy at
  // + dy * wp * kWrX + q * kWrX (q a compile-time row: an immediate offset)
  const int a_lane = wr_lane_off(kWrA, lane) + wm * 32;
  const int x_lane = KT * kWrA + wr_lane_off(kWrX, lane) + wn * 32;
  const int wrow = a.wp * kWrX;

  if (kt0 < kt1) {
    load(kt0);
    store(0);
  }
  __syncthreads();
  // the k-tile loop, instantiated with and without the bias sums (a wave-uniform choice
  // outside the loop: a branch inside it made every k-step wait for all its LDS reads)
  auto ktiles = [&](auto bias_tag) {
    constexpr bool kBias = decltype(bias_tag)::value;
    for (int kt = kt0; kt < kt1; ++kt) {
      const int cur = (kt - kt0) & 1;
      const bool more = kt + 1 < kt1;
      if (more) load(kt + 1);
      const uint16_t* ab = smem + cur * buf_elems + a_lane;
      const uint16_t* xb0 = smem + cur * buf_elems + x_lane;
      const uint16_t* xbr[3] = {xb0, xb0 + wrow, xb0 + 2 * wrow};
#pragma unroll
      for (int ks = 0; ks < KT / 16; ++ks) {
        const int q = ks * 16;
        const uint2 a0 = wr_tr(ab + q * kWrA), a1 = wr_tr(ab + (q + 4) * kWrA);
        const u32x4_t av = {a0.x, a0.y, a1.x, a1.y};
        if (kBias) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            bsum += __uint_as_float(av[e] << 16) + __uint_as_float(av[e] & 0xFFFF0000u);
        }
        const bf16x8_t af = as_bf16x8(av);
#pragma unroll
        for (int dy = 0; dy < 3; ++dy) {
          const uint16_t* xr = xbr[dy] + q * kWrX;
          const uint2 r0 = wr_tr(xr), r1 = wr_tr(xr + 4 * kWrX);
          const u32x4_t l = {r0.x, r0.y, r1.x, r1.y};
          // dx = 1, 2: the same 12 rows shifted by one and two (reading the dx = 2 operand
          // directly instead measured the same)
          const uint2 r2 = wr_tr(xr + 8 * kWrX);
          u32x4_t s1, s2;
          s1[0] = __builtin_amdgcn_alignbit(r0.y, r0.x, 16);
          s1[1] = __builtin_amdgcn_alignbit(r1.x, r0.y, 16);
          s1[2] = __builtin_amdgcn_alignbit(r1.y, r1.x, 16);
          s1[3] = __builtin_amdgcn_alignbit(r2.x, r1.y, 16);
          s2[0] = r0.y;
          s2[1] = r1.x;
          s2[2] = r1.y;
          s2[3] = r2.x;
          acc[dy * 3 + 0] = mfma_32x32x16(af, as_bf16x8(l), acc[dy * 3 + 0]);
          acc[dy * 3 + 1] = mfma_32x32x16(af, as_bf16x8(s1), acc[dy * 3 + 1]);
          acc[dy * 3 + 2] = mfma_32x32x16(af, as_bf16x8(s2), acc[dy * 3 + 2]);
        }
      }
      if (more) store(cur ^ 1);
      __syncthreads();
    }
  };
  if (do_bias)
    ktiles(std::true_type{});
  else
    ktiles(std::false_type{});

  // partials: part[split][co][tap][ci]; lanes 0..31 write 32 consecutive ci.  Buffer stores
  // from the workgroup's corner (co0, tap 0, ci0): a 32-bit offset per lane and row, the tap
  // as a uniform offset (every store is inside the partials: co < co_pad, ci < ci_pad)
  const int lr = lane & 31;
  {
    // (wave-uniform: read from lane 0, so that the resource is a scalar one)
    const int64_t c64 = (int64_t(split) * a.co_pad * 9 + int64_t(co0) * 9) * a.ci_pad + ci0;
    const int64_t corner = int64_t(uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(c64)))) |
                                   (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(c64 >> 32)))) << 32));
    const int64_t left = (int64_t(a.splits) * a.co_pad * 9 * a.ci_pad - corner) * 4;
    const auto prs = __builtin_amdgcn_make_buffer_rsrc(a.part + corner, 0, clamp_records(left), 0x00020000);
    const int tstride = a.ci_pad * 4;
    int roff[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) roff[i] = ((wm * 32 + mfma_row(i, lane)) * 9 * a.ci_pad + wn * 32 + lr) * 4;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[t][i]), prs, roff[i], t * tstride, 0);
  }
  if (do_bias) {
    // lanes l and l+32 hold the two 8-row halves of channel row l % 32
    const float other = __shfl_down(bsum, 32, 64);
    if (lane < 32) a.bpart[int64_t(split) * a.co_pad + co0 + wm * 32 + lane] = bsum + other;
  }
}

// ---------------------------------------------------------------------------------------
// Weight gradient on the packed row layouts fed by gfx950's 16-byte LDS DMA (buffer_load
// ... lds: a wave's load writes 64 x 16 bytes contiguously at an LDS base, lane L at base +
// 16 L; a lane whose offset is past the buffer range writes zeros).  The workgroup tile,
// waves, split plan and partial layout are wgrad_rows_kernel's (128 output x 64 input
// channels x 9 taps over the k-tiles of one split; eight waves, wave (wm, wn) owning 32 x 32
// channels); the staging differs: k-tiles of 64 output rows go into four LDS buffers three
// k-tiles ahead of their first read, with no register staging, no LDS stores and one
// barrier per k-tile, and fragment reads run one k-step ahead of the MFMAs.  Both tiles
// are unpadded, their 16-byte pieces permuted so that the 4 rows x 64 bytes of a half-wave
// transposing read fall on 64 distinct banks (each lane loads the piece its LDS position
// holds):
//   dY tile [64 rows][16 pieces of 8 channels]: piece c of row r at r * 16 + (c ^ 4 (r & 3));
//   x window [160 rows][8 pieces]: piece c of row r at r * 8 + (c ^ 4 ((r >> 1) & 1)).
// dY pieces past the last channel chunk, rows past the end and a strip's halo columns are
// zeroed (an offset past the range); x rows past the group's 2126 read as zero.
// ---------------------------------------------------------------------------------------
constexpr int kW5Kt = 64;                               // output rows per k-tile
constexpr int kW5Nb = 4;                                // k-tile buffers
constexpr int kW5XRows = 160;                           // window rows per buffer (>= 64 + 78 + 4)
constexpr int kW5Buf = kW5Kt * 128 + kW5XRows * 64;     // elements of one k-tile buffer
constexpr size_t kW5Lds = size_t(kW5Nb) * kW5Buf * 2;   // 144 KiB
// DMA blocks (1 KiB) per k-tile: 16 of dY (4 rows each), 20 of x (8 rows each).  Wave w
// loads dY blocks 2w, 2w + 1 and x blocks 3w .. 3w + 2 (w < 4) or 2w + 4, 2w + 5 (w >= 4):
// 5 or 4 loads per k-tile.
constexpr int kW5LoadsHi = 5, kW5LoadsLo = 4;
struct W5Frags {
  u32x4_t a;      // dY fragment of the wave's 32 output channels
  uint2 x[3][3];  // per kernel row: 12 consecutive rows of the wave's 32 input channels
};

// NW = 4: the same k-tile pipeline with four waves on a 64-output-channel tile (waves
// (wm, wn) in 2 x 2, 32 x 32 channels each): twice the workgroups for a split count and
// half the fp32 partials per workgroup, for layers of up to 64 output channels (no
// half-empty tile) and layers whose grid is small; only the dY tile's first 8 pieces (one
// 64-channel chunk) are loaded, the rest of its LDS rows read as zeros and are never used.
template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void wgrad_rows5_kernel(WgRowsArgs a) {
  static_assert(NW == 8 || NW == 4, "eight or four waves");
  constexpr int kCT = NW == 8 ? kTCo : 64;           // output channels per tile
  constexpr int kDyPer = 16 / NW;                    // dY DMA blocks per wave
  constexpr int kXPer = NW == 8 ? 0 : 5;             // x DMA blocks per wave (four waves)
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  constexpr int kTilesPerGroup = kGroupOutRows / kW5Kt;
  const int L = blockIdx.x;
  const int xcd = L % kXcds, kq = L / kXcds;
  const int tile = kq % a.ntiles;
  const int split = (kq / a.ntiles) * kXcds + xcd;
  if (split >= a.splits) return;
  const int co_t = tile % a.nco_t, ci_t = tile / a.nco_t;
  const int co0 = co_t * kCT, ci0 = ci_t * 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = NW == 8 ? wave & 3 : wave & 1, wn = NW == 8 ? wave >> 2 : wave >> 1;
  const int kt0 = split * a.kt_per_split;
  const int ntl = min(a.ktiles, kt0 + a.kt_per_split) - kt0;

  f32x16_t acc[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) acc[t] = zero_acc();
  float bsum = 0.0f;
  const bool do_bias = a.bpart && ci_t == 0 && wn == 0;

  if (ntl > 0) {
    // DMA plan.  dY block 2 wave + i: k-tile rows 8 wave + 4 i + lane / 16, LDS position
    // lane % 16 holding global piece dq (channel chunk co0 / 64 + dq / 8).
    const bool strips = a.S > 1;
    const int dq = (lane & 15) ^ (4 * (lane >> 4));
    const bool dchunk_ok = (dq >> 3) < kCT / 64 && co0 / 64 + (dq >> 3) < a.co_chunks;
    const int doff0 = (dq >> 3) * kGroupRows * 128 + (dq & 7) * 16;  // bytes, + 128 per row
    int drow[kDyPer], drmod[kDyPer];
#pragma unroll
    for (int i = 0; i < kDyPer; ++i) {
      drow[i] = 4 * kDyPer * wave + 4 * i + (lane >> 4);
      drmod[i] = drow[i] % a.wp;
    }
    const int nrel = min(kCT / 64, a.co_chunks - co0 / 64);
    const int dext = (nrel - 1) * kGroupRows * 128 + kW5Kt * 128;
    // x block xb0 + i: window rows 8 (xb0 + i) + lane / 8, LDS position lane % 8 holding
    // global piece xq (bit 1 of the row is bit 1 of lane / 8)
    const int xb0 = NW == 4 ? kXPer * wave : wave < 4 ? 3 * wave : 2 * wave + 4;
    const int xq = (lane & 7) ^ (4 * ((lane >> 4) & 1));
    const int xoff0 = (8 * xb0 + (lane >> 3)) * 128 + xq * 16;  // bytes, + 1 KiB per block

    // DMA of k-tile tl of the split (clamped to the last: the load count stays static) into
    // buffer tl % kW5Nb: its resources and offsets (plan), then its loads (issue_dy,
    // issue_x), so that the address arithmetic can run before the barrier that frees the
    // buffer and the loads after it
    struct DmaPlan {
      i32x4_t drs, xrs;
      int doff[kDyPer];
      const uint16_t* buf;
    };
    auto plan = [&](int tl) {
      DmaPlan p;
      const int kt = kt0 + min(tl, ntl - 1);
      p.buf = smem + (tl & (kW5Nb - 1)) * kW5Buf;
      const int g = kt / kTilesPerGroup, r0 = (kt % kTilesPerGroup) * kW5Kt;
      const uint16_t* dbase =
          a.dp + ((int64_t(g) * a.co_chunks + co0 / 64) * kGroupRows + r0 + a.wp + 1) * kKStep;
      p.drs = lds_dma_rsrc(dbase, dext);
      const int64_t rem = a.m_total - int64_t(kt) * kW5Kt;  // rows of this k-tile before the end
      const int base = int((uint32_t(kt) * uint32_t(kW5Kt)) % uint32_t(a.wp));
#pragma unroll
      for (int i = 0; i < kDyPer; ++i) {
        // data column of the centre row p + wp + 1 (row position jc + 1, wrapping to the
        // next row's position 0); a strip's halo columns are masked
        int jc = base + drmod[i];
        jc -= jc >= a.wp ? a.wp : 0;
        int dj = jc + 1 - a.lead;
        dj = dj == a.wp ? 0 : dj;
        const bool halo = strips && (dj == 0 || dj == a.Wg - 1);
        const bool ok = dchunk_ok && drow[i] < rem && !halo;
        p.doff[i] = ok ? doff0 + drow[i] * 128 : 0x7FFFFFF0;
      }
      const uint16_t* xbase = a.xp + ((int64_t(g) * a.ci_chunks + ci0 / 64) * kGroupRows + r0) * kKStep;
      p.xrs = lds_dma_rsrc(xbase, (kGroupRows - r0) * 128);
      return p;
    };
    auto issue_dy = [&](const DmaPlan& p) {
#pragma unroll
      for (int i = 0; i < kDyPer; ++i) lds_dma16(p.drs, p.buf + (kDyPer * wave + i) * 512, p.doff[i]);
    };
    auto issue_x = [&](const DmaPlan& p) {
      const uint16_t* xl = p.buf + kW5Kt * 128 + xb0 * 512;
      if constexpr (NW == 4) {
#pragma unroll
        for (int i = 0; i < kXPer; ++i) lds_dma16(p.xrs, xl + i * 512, xoff0 + i * 1024);
      } else {
        lds_dma16(p.xrs, xl, xoff0);
        lds_dma16(p.xrs, xl + 512, xoff0 + 1024);
        if (wave < 4) lds_dma16(p.xrs, xl + 1024, xoff0 + 2048);
      }
    };
    auto load = [&](int tl) {
      const DmaPlan p = plan(tl);
      issue_dy(p);
      issue_x(p);
    };
    // this wave's loads of the oldest k-tile in flight have landed, n k-tiles' may stay
    // in flight
    auto wait_tiles = [&](auto n_tag) {
      constexpr int n = decltype(n_tag)::value;
      if constexpr (NW == 4)
        lds_dma_wait<(kDyPer + kXPer) * n>();
      else if (wave < 4)
        lds_dma_wait<kW5LoadsHi * n>();
      else
        lds_dma_wait<kW5LoadsLo * n>();
    };

    // Lane parts of the transposing reads (wr_lane_off's assignment: in 16-lane group
    // gq = lane / 16, lane j supplies row + 8 (gq / 2) + j / 4, column + 16 (gq % 2) + 4 (j % 4)).
    const int gq = lane >> 4, jq = lane & 15;
    const int rq = 8 * (gq >> 1) + (jq >> 2);
    int x_off[3];
    const int ca = wm * 32 + 16 * (gq & 1) + 4 * (jq & 3);
    const int a_off = rq * 128 + (((ca >> 3) ^ (4 * (rq & 3))) << 3) + (ca & 7);
#pragma unroll
    for (int dy = 0; dy < 3; ++dy) {
      const int c = wn * 32 + 16 * (gq & 1) + 4 * (jq & 3);
      const int r = dy * a.wp + rq;
      x_off[dy] = kW5Kt * 128 + r * 64 + (((c >> 3) ^ (4 * ((r >> 1) & 1))) << 3) + (c & 7);
    }
    // k-step ks of a buffer: rows 16 ks .. +15 (the row bits the permutations use are
    // those of the lane part: 16 ks and 4 q leave bits 0 and 1 of a row alone)
    auto frag_a = [&](W5Frags& f, const uint16_t* buf, int ks) {
      const uint2 lo = wr_tr(buf + a_off + ks * 16 * 128);
      const uint2 hi = wr_tr(buf + a_off + (ks * 16 + 4) * 128);
      f.a = u32x4_t{lo.x, lo.y, hi.x, hi.y};
    };
    auto frag_x = [&](W5Frags& f, const uint16_t* buf, int ks, int dy) {
#pragma unroll
      for (int q = 0; q < 3; ++q) f.x[dy][q] = wr_tr(buf + x_off[dy] + (ks * 16 + 4 * q) * 64);
    };
    auto frags = [&](W5Frags& f, const uint16_t* buf, int ks) {
      frag_a(f, buf, ks);
#pragma unroll
      for (int dy = 0; dy < 3; ++dy) frag_x(f, buf, ks, dy);
    };
    // the three MFMAs of kernel row dy (dx = 0, 1, 2); the bias sums go with dy = 0
    auto mfma_dy = [&](const W5Frags& f, int dy, auto bias_tag) {
      constexpr bool kBias = decltype(bias_tag)::value;
      if (kBias && dy == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          bsum += __uint_as_float(f.a[e] << 16) + __uint_as_float(f.a[e] & 0xFFFF0000u);
      }
      const bf16x8_t af = as_bf16x8(f.a);
      {
        const uint2 r0 = f.x[dy][0], r1 = f.x[dy][1], r2 = f.x[dy][2];
        const u32x4_t l = {r0.x, r0.y, r1.x, r1.y};
        u32x4_t s1, s2;
        s1[0] = __builtin_amdgcn_alignbit(r0.y, r0.x, 16);
        s1[1] = __builtin_amdgcn_alignbit(r1.x, r0.y, 16);
        s1[2] = __builtin_amdgcn_alignbit(r1.y, r1.x, 16);
        s1[3] = __builtin_amdgcn_alignbit(r2.x, r1.y, 16);
        s2[0] = r0.y;
        s2[1] = r1.x;
        s2[2] = r1.y;
        s2[3] = r2.x;
        acc[dy * 3 + 0] = mfma_32x32x16(af, as_bf16x8(l), acc[dy * 3 + 0]);
        acc[dy * 3 + 1] = mfma_32x32x16(af, as_bf16x8(s1), acc[dy * 3 + 1]);
        acc[dy * 3 + 2] = mfma_32x32x16(af, as_bf16x8(s2), acc[dy * 3 + 2]);
      }
    };
    // one k-step (fragments fc) while the next k-step's fragments (fn: buffer nb, k-step
    // nks) are read, in three fenced slices: kernel row dy's reads among its MFMAs
    auto step = [&](W5Frags& fn, const uint16_t* nb, int nks, const W5Frags& fc, auto bias_tag) {
      frag_a(fn, nb, nks);
      frag_x(fn, nb, nks, 0);
      mfma_dy(fc, 0, bias_tag);
      __builtin_amdgcn_sched_barrier(0);
      frag_x(fn, nb, nks, 1);
      mfma_dy(fc, 1, bias_tag);
      __builtin_amdgcn_sched_barrier(0);
      frag_x(fn, nb, nks, 2);
      mfma_dy(fc, 2, bias_tag);
      __builtin_amdgcn_sched_barrier(0);
    };

    // the k-tile loop, instantiated with and without the bias sums (a wave-uniform choice
    // outside the loop)
    auto run = [&](auto bias_tag) {
      W5Frags f0, f1;
#pragma unroll
      for (int t = 0; t < kW5Nb; ++t) load(t);
      wait_tiles(std::integral_constant<int, kW5Nb - 1>{});
      __builtin_amdgcn_s_barrier();
      frags(f0, smem, 0);
      for (int tl = 0; tl < ntl; ++tl) {
        const uint16_t* buf = smem + (tl & (kW5Nb - 1)) * kW5Buf;
        step(f1, buf, 1, f0, bias_tag);
        step(f0, buf, 2, f1, bias_tag);
        step(f1, buf, 3, f0, bias_tag);
        // the address arithmetic of k-tile tl + kW5Nb's DMA, before the barrier
        const DmaPlan p = plan(tl + kW5Nb);
        __builtin_amdgcn_sched_barrier(0);
        // this wave's reads of the buffer are complete and its loads of k-tile tl + 1 have
        // landed (two k-tiles of loads may stay in flight); the barrier publishes every
        // wave's and frees the buffer for k-tile tl + kW5Nb
        lds_reads_wait();
        wait_tiles(std::integral_constant<int, kW5Nb - 2>{});
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // k-step 3 in three fenced slices (one kernel row each), each also issuing part of
        // k-tile tl + 1's first fragments (past the end: never used) and of the DMA into
        // the freed buffer, so that the MFMAs start right after the barrier
        const uint16_t* nbuf = smem + ((tl + 1) & (kW5Nb - 1)) * kW5Buf;
        frag_a(f0, nbuf, 0);
        frag_x(f0, nbuf, 0, 0);
        mfma_dy(f1, 0, bias_tag);
        issue_dy(p);
        __builtin_amdgcn_sched_barrier(0);
        frag_x(f0, nbuf, 0, 1);
        mfma_dy(f1, 1, bias_tag);
        issue_x(p);
        __builtin_amdgcn_sched_barrier(0);
        frag_x(f0, nbuf, 0, 2);
        mfma_dy(f1, 2, bias_tag);
        __builtin_amdgcn_sched_barrier(0);
      }
      // drain the clamped loads issued past the end before the workgroup can exit
      lds_dma_wait<0>();
    };
    if (do_bias)
      run(std::true_type{});
    else
      run(std::false_type{});
  }

  // partials: part[split][co][tap][ci]; lanes 0..31 write 32 consecutive ci.  Buffer stores
  // from the workgroup's corner (co0, tap 0, ci0): a 32-bit offset per lane and row, the tap
  // as a uniform offset (every store is inside the partials: co < co_pad, ci < ci_pad)
  const int lr = lane & 31;
  {
    // (wave-uniform: read from lane 0, so that the resource is a scalar one)
    const int64_t c64 = (int64_t(split) * a.co_pad * 9 + int64_t(co0) * 9) * a.ci_pad + ci0;
    const int64_t corner = int64_t(uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(c64)))) |
                                   (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(c64 >> 32)))) << 32));
    const int64_t left = (int64_t(a.splits) * a.co_pad * 9 * a.ci_pad - corner) * 4;
    const auto prs = __builtin_amdgcn_make_buffer_rsrc(a.part + corner, 0, clamp_records(left), 0x00020000);
    const int tstride = a.ci_pad * 4;
    int roff[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) roff[i] = ((wm * 32 + mfma_row(i, lane)) * 9 * a.ci_pad + wn * 32 + lr) * 4;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[t][i]), prs, roff[i], t * tstride, 0);
  }
  if (do_bias) {
    // lanes l and l+32 hold the two 8-row halves of channel row l % 32
    const float other = __shfl_down(bsum, 32, 64);
    if (lane < 32) a.bpart[int64_t(split) * a.co_pad + co0 + wm * 32 + lane] = bsum + other;
  }
}

// Kernel of the rows weight gradient: 1 register-staged k-tiles (wgrad_rows_kernel), 2
// k-tiles loaded straight into LDS (wgrad_rows5_kernel); XDNA_WGRAD_KERNEL at start-up,
// xdna_conv3x3_set_wgrad_rows_kernel.
// The default, form 2: 2.2 % ahead of form 1 over the sweep's 36 shapes (GPU time per
// shape's fwd + dgrad + wgrad step), 3 % on the largest ones.
constexpr int kWgradRowsDefaultForm = 2;
std::atomic<int> g_wgrad_rows_form{[] {
  const char* e = std::getenv("XDNA_WGRAD_KERNEL");
  const int f = e ? std::atoi(e) : 0;
  return f == 1 || f == 2 ? f : kWgradRowsDefaultForm;
}()};

struct WgRowsPlan {
  ConvGeom geom;
  int form = 1;      // 1: wgrad_rows_kernel, 2: wgrad_rows5_kernel
  int co_tile = 128; // output channels per workgroup tile (form 2: 128 eight waves, 64 four)
  int kt_rows = 64;  // output rows per k-tile
  int ci_chunks = 0, co_chunks = 0, ci_pad = 0, co_pad = 0;
  int ktiles = 0, splits = 0, kt_per = 0;
  size_t part_bytes = 0, bpart_bytes = 0, lds_bytes = 0;
};

// split count of the rows weight gradient: 0 (default) the model below, else forced
// (xdna_conv3x3_set_wgrad_splits, for measurements)
std::atomic<int> g_wgrad_splits{0};
// output-channel tile of the rows weight gradient's form 2: 0 (by layer), 64 or 128
// (xdna_conv3x3_set_wgrad_tile)
std::atomic<int> g_wgrad_tile{0};

WgRowsPlan wgrad_rows_plan(int B, int Cin, int Cout, int H, int W, int layout) {
  WgRowsPlan p;
  p.geom = conv_geom(B, H, W, layout);
  p.ci_chunks = int(ceil_div(Cin, kKStep));
  p.co_chunks = int(ceil_div(Cout, kKStep));
  p.ci_pad = p.ci_chunks * kKStep;
  p.form = g_wgrad_rows_form.load();
  {
    // form 2's tile (xdna_conv3x3_set_wgrad_tile forces one): four waves on 64 output
    // channels for layers of up to 64 output channels and for layers of up to 256 channels
    // each side and 40 GFLOP (measured on the 36 sweep shapes, each tile at its modelled
    // split count: 3-19 % less time there, 1.05-2.5x more on the larger and the
    // 512-channel layers, where one wave per SIMD leaves the latency uncovered); else
    // eight waves on 128
    const int t = g_wgrad_tile.load();
    const double gflop = 2.0 * 9.0 * double(B) * H * W * double(Cin) * double(Cout) * 1e-9;
    const bool small = Cout <= 64 || (Cout <= 256 && Cin <= 256 && gflop <= 40.0);
    p.co_tile = p.form == 2 && (t == 64 || (t == 0 && small)) ? 64 : kTCo;
  }
  p.co_pad = int(ceil_div(Cout, p.co_tile) * p.co_tile);
  p.kt_rows = p.form == 2 ? kW5Kt : g_wgrad_rows_kt.load() == 128 ? 128 : 64;
  p.ktiles = int(ceil_div(p.geom.m_total, p.kt_rows));
  const int64_t tiles = int64_t(p.ci_pad / 64) * (p.co_pad / p.co_tile);
  const int64_t out_elems = int64_t(p.co_pad) * 9 * p.ci_pad;
  // split count: the channel-major path's model (rounds of 256 workgroups x per-CU rate,
  // plus the write and read of the fp32 partials)
  const double flops = 2.0 * 9.0 * double(B) * H * W * double(Cin) * double(Cout);
  // (a single channel tile, the 64-channel layers, splits further: the model's bandwidth
  // doubled there measured up to 12 % faster and no slower elsewhere)
  const double cu_rate = 4.0e12, bw = tiles == 1 ? 10.0e12 : 5.0e12;
  int64_t best = 1;
  double best_t = 1e30;
  const int64_t smax = std::min<int64_t>(p.ktiles, 4096);
  for (int64_t s = 1; s <= smax; s = s < 512 ? s + 1 : s + s / 8) {
    const double rounds = double(ceil_div(tiles * s, 256));
    const double t = rounds * flops / (double(tiles * s) * cu_rate) + 2.0 * double(s) * double(out_elems) * 4.0 / bw;
    if (t < best_t) {
      best_t = t;
      best = s;
    }
  }
  if (g_wgrad_splits.load() > 0) best = std::min<int64_t>(g_wgrad_splits.load(), p.ktiles);
  p.kt_per = int(ceil_div(p.ktiles, best));
  p.splits = int(ceil_div(p.ktiles, p.kt_per));
  p.part_bytes = align256(size_t(p.splits) * out_elems * 4);
  p.bpart_bytes = align256(size_t(p.splits) * p.co_pad * 4);
  p.lds_bytes = p.form == 2 ? kW5Lds
                            : 2 * (size_t(p.kt_rows) * kWrA + size_t(p.kt_rows + 2 * p.geom.st.wp + 2 + 4) * kWrX) * 2;
  return p;
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

size_t xdna_conv3x3_fwd_workspace_bytes(int B, int Cin, int Cout, int H, int W) {
  if (B < 1 || Cin < 1 || Cout < 1 || H < 1 || W < 1) return 0;
  const FwdPlan p = fwd_plan(B, Cin, Cout, H, W);
  return p.packed_bytes + p.wt_bytes;
}

int xdna_conv3x3_fwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* y,
                          int B, int Cin, int Cout, int H, int W, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (!shape_ok("xdna_conv3x3_fwd_bf16", B, Cin, Cout, H, W)) return -1;
  const FwdPlan p = fwd_plan(B, Cin, Cout, H, W);
  if (!workspace || workspace_bytes < p.packed_bytes + p.wt_bytes) {
    set_error("xdna_conv3x3_fwd_bf16: workspace too small");
    return -1;
  }
  uint16_t* xp = static_cast<uint16_t*>(workspace);
  uint16_t* wt = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.packed_bytes);
  if (xdna_hip_memset_async(xp, 0, p.packed_bytes, stream)) return -1;
  if (xdna_conv3x3w_pack_input_strips_range_bf16(x, xp, B, Cin, H, W, p.geom.st.S, p.geom.st.So, 0,
                                                 p.chunks, 0, p.geom.groups, stream))
    return -1;
  if (launch_prep(w, wt, Cout, Cin, p.co_pad, p.chunks, 0, stream)) return -1;
  return launch_rows(xp, wt, bias, y, B, Cin, Cout, H, W, stream);
}

size_t xdna_conv3x3_dgrad_workspace_bytes(int B, int Cin, int Cout, int H, int W) {
  // dgrad is the forward conv of dY (Cout channels) into Cin channels.
  return xdna_conv3x3_fwd_workspace_bytes(B, Cout, Cin, H, W);
}

int xdna_conv3x3_dgrad_bf16(const uint16_t* dy, const uint16_t* w, uint16_t* dx, int B, int Cin,
                            int Cout, int H, int W, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (!shape_ok("xdna_conv3x3_dgrad_bf16", B, Cin, Cout, H, W)) return -1;
  const FwdPlan p = fwd_plan(B, Cout, Cin, H, W);
  if (!workspace || workspace_bytes < p.packed_bytes + p.wt_bytes) {
    set_error("xdna_conv3x3_dgrad_bf16: workspace too small");
    return -1;
  }
  uint16_t* dp = static_cast<uint16_t*>(workspace);
  uint16_t* wt = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.packed_bytes);
  if (xdna_hip_memset_async(dp, 0, p.packed_bytes, stream)) return -1;
  if (xdna_conv3x3w_pack_input_strips_range_bf16(dy, dp, B, Cout, H, W, p.geom.st.S, p.geom.st.So,
                                                 0, p.chunks, 0, p.geom.groups, stream))
    return -1;
  if (launch_prep(w, wt, Cout, Cin, p.co_pad, p.chunks, 1, stream)) return -1;
  return launch_rows(dp, wt, nullptr, dx, B, Cout, Cin, H, W, stream);
}

size_t xdna_conv3x3_wgrad_workspace_bytes(int B, int Cin, int Cout, int H, int W) {
  if (B < 1 || Cin < 1 || Cout < 1 || H < 1 || W < 1) return 0;
  const WgradPlan p = wgrad_plan(B, Cin, Cout, H, W);
  return p.xt_bytes + p.dt_bytes + p.part_bytes + p.bpart_bytes;
}

namespace {
struct WgradBufs {
  uint16_t* xt;
  uint16_t* dt;
  float* part;
  float* bpart;
};

bool wgrad_bufs(const char* what, const WgradPlan& p, void* workspace, size_t workspace_bytes,
                WgradBufs& b) {
  if (p.lds_bytes > kMaxWgradLds || 64 * (p.wlen / 8) > kWgMaxXv * kWgThreads) {
    set_error(std::string(what) + ": image too wide for the LDS window");
    return false;
  }
  const size_t need = p.xt_bytes + p.dt_bytes + p.part_bytes + p.bpart_bytes;
  if (!workspace || workspace_bytes < need) {
    set_error(std::string(what) + ": workspace too small");
    return false;
  }
  char* ws = static_cast<char*>(workspace);
  b.xt = reinterpret_cast<uint16_t*>(ws);
  b.dt = reinterpret_cast<uint16_t*>(ws + p.xt_bytes);
  b.part = reinterpret_cast<float*>(ws + p.xt_bytes + p.dt_bytes);
  b.bpart = reinterpret_cast<float*>(ws + p.xt_bytes + p.dt_bytes + p.part_bytes);
  return true;
}
}  // namespace

int xdna_conv3x3_wgrad_pack_bf16(const uint16_t* x, const uint16_t* dy, int B, int Cin, int Cout,
                                 int H, int W, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (!shape_ok("xdna_conv3x3_wgrad_pack_bf16", B, Cin, Cout, H, W)) return -1;
  const WgradPlan p = wgrad_plan(B, Cin, Cout, H, W);
  WgradBufs bufs;
  if (!wgrad_bufs("xdna_conv3x3_wgrad_pack_bf16", p, workspace, workspace_bytes, bufs)) return -1;
  if (!admit_launch("conv3x3 wgrad pack")) return -1;
  hipStream_t st = as_stream(stream);
  if (pack_cm_launch2(x, bufs.xt, Cin, p.ci_pad, dy, bufs.dt, Cout, p.co_pad, B, H, W, p.cm, st) != 0) return -1;
  return check_launch("conv3x3 wgrad pack");
}

int xdna_conv3x3_wgrad_packed_bf16(uint16_t* gw, uint16_t* gb, int B, int Cin, int Cout, int H,
                                   int W, void* workspace, size_t workspace_bytes, void* stream) {
  if (!shape_ok("xdna_conv3x3_wgrad_packed_bf16", B, Cin, Cout, H, W)) return -1;
  const WgradPlan p = wgrad_plan(B, Cin, Cout, H, W);
  WgradBufs bufs;
  if (!wgrad_bufs("xdna_conv3x3_wgrad_packed_bf16", p, workspace, workspace_bytes, bufs)) return -1;
  if (!admit_launch("conv3x3 wgrad")) return -1;
  hipStream_t st = as_stream(stream);
  WgradArgs a;
  a.xt = bufs.xt;
  a.dt = bufs.dt;
  a.part = bufs.part;
  a.bpart = gb ? bufs.bpart : nullptr;
  a.q = p.cm.q;
  a.wp8 = p.cm.wp8;
  a.ci_pad = p.ci_pad;
  a.co_pad = p.co_pad;
  a.kt_per_split = p.kt_per;
  a.ktiles = int(p.cm.ktiles);
  a.xpitch = p.xpitch;
  a.wlen = p.wlen;
  static bool lds_attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_kernel<4>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess &&
           hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_kernel<6>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess;
  }();
  if (!lds_attr) {
    (void)hipGetLastError();
    set_error("conv3x3 wgrad: cannot raise the dynamic LDS limit");
    return -1;
  }
  a.nco_t = p.co_pad / kTCo;
  a.ntiles = a.nco_t * (p.ci_pad / 64);
  a.splits = p.splits;
  const int64_t nblocks = ceil_div(p.splits, kXcds) * kXcds * int64_t(a.ntiles);
  if (nblocks > int64_t(0x7fffffff)) {
    set_error("conv3x3 wgrad: grid too large");
    return -1;
  }
  const dim3 grid(unsigned(nblocks), 1, 1);
  if (64 * (p.wlen / 8) <= 4 * kWgThreads)
    wgrad_kernel<4><<<grid, kWgThreads, p.lds_bytes, st>>>(a);
  else
    wgrad_kernel<6><<<grid, kWgThreads, p.lds_bytes, st>>>(a);
  launch_wgrad_reduce(bufs.part, bufs.bpart, gw, gb, Cout, Cin, p.co_pad, p.ci_pad, p.splits, st);
  return check_launch("conv3x3 wgrad");
}

int xdna_conv3x3_wgrad_bf16(const uint16_t* x, const uint16_t* dy, uint16_t* gw, uint16_t* gb,
                            int B, int Cin, int Cout, int H, int W, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (xdna_conv3x3_wgrad_pack_bf16(x, dy, B, Cin, Cout, H, W, workspace, workspace_bytes, stream))
    return -1;
  return xdna_conv3x3_wgrad_packed_bf16(gw, gb, B, Cin, Cout, H, W, workspace, workspace_bytes,
                                        stream);
}

size_t xdna_conv3x3_wgrad_rows_workspace_bytes(int B, int Cin, int Cout, int H, int W, int layout) {
  if (B < 1 || Cin < 1 || Cout < 1 || H < 1 || W < 1 || (layout != kLayoutRef && layout != kLayoutTight)) return 0;
  const WgRowsPlan p = wgrad_rows_plan(B, Cin, Cout, H, W, layout);
  return p.part_bytes + p.bpart_bytes;
}

int xdna_conv3x3_wgrad_rows_bf16(const uint16_t* xp, const uint16_t* dp, uint16_t* gw, uint16_t* gb, int B,
                                 int Cin, int Cout, int H, int W, int layout, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!shape_ok("xdna_conv3x3_wgrad_rows_bf16", B, Cin, Cout, H, W)) return -1;
  if (!xp || !dp || !gw || (layout != kLayoutRef && layout != kLayoutTight)) {
    set_error("xdna_conv3x3_wgrad_rows_bf16: null operand or unknown layout");
    return -1;
  }
  const WgRowsPlan p = wgrad_rows_plan(B, Cin, Cout, H, W, layout);
  // the kernel's 32-bit row arithmetic and its strip-column reduction (strips of 21 or
  // more positions)
  if (int64_t(p.ktiles) * p.kt_rows >= (int64_t(1) << 31)) {
    set_error("xdna_conv3x3_wgrad_rows_bf16: shape outside the kernel's range");
    return -1;
  }
  if (!workspace || workspace_bytes < p.part_bytes + p.bpart_bytes) {
    set_error("xdna_conv3x3_wgrad_rows_bf16: workspace too small");
    return -1;
  }
  if (!admit_launch("conv3x3 wgrad rows")) return -1;
  static const bool lds_attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_rows_kernel<64>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_rows_kernel<128>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_rows5_kernel<8>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&wgrad_rows5_kernel<4>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxWgradLds)) == hipSuccess;
  if (!lds_attr || p.lds_bytes > kMaxWgradLds) {
    (void)hipGetLastError();
    set_error("conv3x3 wgrad rows: cannot raise the dynamic LDS limit");
    return -1;
  }
  WgRowsArgs a;
  a.xp = xp;
  a.dp = dp;
  a.part = static_cast<float*>(workspace);
  a.bpart = gb ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.part_bytes) : nullptr;
  a.ci_chunks = p.ci_chunks;
  a.co_chunks = p.co_chunks;
  a.ci_pad = p.ci_pad;
  a.co_pad = p.co_pad;
  a.wp = p.geom.st.wp;
  a.S = p.geom.st.S;
  a.Wg = p.geom.st.Wg;
  a.lead = p.geom.st.lead;
  a.img = p.geom.img;
  a.m_total = p.geom.m_total;
  a.ktiles = p.ktiles;
  a.kt_per_split = p.kt_per;
  a.splits = p.splits;
  a.nco_t = p.co_pad / p.co_tile;
  a.ntiles = a.nco_t * (p.ci_pad / 64);
  const int64_t nblocks = ceil_div(p.splits, kXcds) * kXcds * int64_t(a.ntiles);
  if (nblocks > int64_t(0x7fffffff)) {
    set_error("conv3x3 wgrad rows: grid too large");
    return -1;
  }
  hipStream_t st = as_stream(stream);
  if (p.form == 2 && p.co_tile == 64)
    wgrad_rows5_kernel<4><<<unsigned(nblocks), 256, p.lds_bytes, st>>>(a);
  else if (p.form == 2)
    wgrad_rows5_kernel<8><<<unsigned(nblocks), 512, p.lds_bytes, st>>>(a);
  else if (p.kt_rows == 128)
    wgrad_rows_kernel<128><<<unsigned(nblocks), 512, p.lds_bytes, st>>>(a);
  else
    wgrad_rows_kernel<64><<<unsigned(nblocks), 512, p.lds_bytes, st>>>(a);
  launch_wgrad_reduce(a.part, gb ? a.bpart : nullptr, gw, gb, Cout, Cin, p.co_pad, p.ci_pad, p.splits, st);
  return check_launch("conv3x3 wgrad rows");
}

size_t xdna_conv3x3w_packed_bytes(int B, int C, int H, int W) {
  if (B < 1 || C < 1 || H < 1 || W < 1) return 0;
  return fwd_plan(B, C, 1, H, W).packed_bytes;
}

size_t xdna_conv3x3_prepared_weight_bytes(int cin, int cout) {
  if (cin < 1 || cout < 1) return 0;
  return fwd_plan(1, cin, cout, 1, 1).wt_bytes;
}

int xdna_conv3x3_prepare_weights_bf16(const uint16_t* w, uint16_t* wt, int Cout, int Cin,
                                      int dgrad, void* stream) {
  if (Cout < 1 || Cin < 1) {
    set_error("xdna_conv3x3_prepare_weights_bf16: invalid shape");
    return -1;
  }
  const int cin = dgrad ? Cout : Cin, cout = dgrad ? Cin : Cout;
  const FwdPlan p = fwd_plan(1, cin, cout, 1, 1);
  return launch_prep(w, wt, Cout, Cin, p.co_pad, p.chunks, dgrad ? 1 : 0, stream);
}

int xdna_conv3x3_prepare_weights_both_bf16(const uint16_t* w, uint16_t* wt, uint16_t* wt_dgrad, int Cout,
                                           int Cin, void* stream) {
  if (Cout < 1 || Cin < 1 || !w || !wt || !wt_dgrad) {
    set_error("xdna_conv3x3_prepare_weights_both_bf16: invalid arguments");
    return -1;
  }
  return launch_prep_tiled(w, wt, wt_dgrad, Cout, Cin, stream);
}

int xdna_conv3x3_rows_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias,
                           uint16_t* y, int B, int cin, int cout, int H, int W, void* stream) {
  if (!shape_ok("xdna_conv3x3_rows_bf16", B, cin, cout, H, W)) return -1;
  return launch_rows(xp, wt, bias, y, B, cin, cout, H, W, stream);
}

int xdna_conv3x3_layout_rows_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                  int B, int cin, int cout, int H, int W, int layout, void* stream) {
  if (!shape_ok("xdna_conv3x3_layout_rows_bf16", B, cin, cout, H, W)) return -1;
  if (layout != kLayoutRef && layout != kLayoutTight) {
    set_error("xdna_conv3x3_layout_rows_bf16: unknown layout");
    return -1;
  }
  return launch_rows(xp, wt, bias, y, B, cin, cout, H, W, stream, layout);
}

int xdna_conv3x3_layout_rows_act_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                      int B, int cin, int cout, int H, int W, int layout, int act, void* stream) {
  if (!shape_ok("xdna_conv3x3_layout_rows_act_bf16", B, cin, cout, H, W)) return -1;
  if ((layout != kLayoutRef && layout != kLayoutTight) || act < 0 || act > 1) {
    set_error("xdna_conv3x3_layout_rows_act_bf16: unknown layout or activation");
    return -1;
  }
  return launch_rows(xp, wt, bias, y, B, cin, cout, H, W, stream, layout, act);
}

int xdna_conv3x3_nchw_small_eligible(int B, int cin, int cout, int H, int W) {
  return nchw_small_ok(B, cin, cout, H, W) ? 1 : 0;
}

int xdna_conv3x3_nchw_act_bf16(const uint16_t* x, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int B,
                               int cin, int cout, int H, int W, int act, int s2out, void* stream) {
  if (!shape_ok("xdna_conv3x3_nchw_act_bf16", B, cin, cout, H, W)) return -1;
  if (act < 0 || act > 1 || s2out < 0 || s2out > 1 || !x || !wt || !y) {
    set_error("xdna_conv3x3_nchw_act_bf16: invalid activation, output form or null buffer");
    return -1;
  }
  if (!nchw_small_ok(B, cin, cout, H, W)) {
    set_error("xdna_conv3x3_nchw_act_bf16: not a small-grid conv with W <= 36, cin % 8 == 0 and an input under "
              "2 GiB (xdna_conv3x3_nchw_small_eligible)");
    return -1;
  }
  return launch_rows_nchw(x, wt, bias, y, B, cin, cout, H, W, act, s2out != 0, stream);
}

int xdna_conv3x3_layout_rows_stride2_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                          int B, int cin, int cout, int H, int W, int layout, void* stream) {
  if (!shape_ok("xdna_conv3x3_layout_rows_stride2_bf16", B, cin, cout, H, W)) return -1;
  if (layout != kLayoutRef && layout != kLayoutTight) {
    set_error("xdna_conv3x3_layout_rows_stride2_bf16: unknown layout");
    return -1;
  }
  return launch_rows(xp, wt, bias, y, B, cin, cout, H, W, stream, layout, 0, /*s2out=*/true);
}

int xdna_conv3x3_layout_rows_bfp16_emul_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias,
                                             uint16_t* y, int B, int cin, int cout, int H, int W, int layout, int act,
                                             void* stream) {
  if (!shape_ok("xdna_conv3x3_layout_rows_bfp16_emul_bf16", B, cin, cout, H, W)) return -1;
  if ((layout != kLayoutRef && layout != kLayoutTight) || act < 0 || act > 1) {
    set_error("xdna_conv3x3_layout_rows_bfp16_emul_bf16: unknown layout or activation");
    return -1;
  }
  if ((reinterpret_cast<uintptr_t>(xp) | reinterpret_cast<uintptr_t>(wt)) & 15) {
    set_error("xdna_conv3x3_layout_rows_bfp16_emul_bf16: packed rows and weights must be 16-byte aligned");
    return -1;
  }
  return launch_rows_emul(xp, wt, bias, y, B, cin, cout, H, W, stream, layout, act);
}

int xdna_conv3x3_set_wgrad_rows_kt(int kt_rows) {
  if (kt_rows != 0 && kt_rows != 64 && kt_rows != 128) {
    set_error("xdna_conv3x3_set_wgrad_rows_kt: k-tile rows must be 0 (default), 64 or 128");
    return -1;
  }
  g_wgrad_rows_kt.store(kt_rows == 64 ? 64 : 128);
  return 0;
}

int xdna_conv3x3_set_wgrad_rows_kernel(int form) {
  if (form < 0 || form > 2) {
    set_error("xdna_conv3x3_set_wgrad_rows_kernel: form must be 0 (default), 1 or 2");
    return -1;
  }
  g_wgrad_rows_form.store(form == 0 ? kWgradRowsDefaultForm : form);
  return 0;
}

int xdna_conv3x3_set_rows_variant(int variant) {
  if (variant < 0 || variant > 11) {
    set_error("xdna_conv3x3_set_rows_variant: variant must be 0..11");
    return -1;
  }
  g_rows_variant.store(variant);
  return 0;
}

int xdna_conv3x3_prepare_weights_multi_bf16(int n, const uint16_t* const* w, uint16_t* const* wt,
                                            uint16_t* const* wtd, const int* cout, const int* cin, void* stream) {
  if (n < 0 || (n > 0 && (!w || !wt || !wtd || !cout || !cin))) {
    set_error("xdna_conv3x3_prepare_weights_multi_bf16: invalid arguments");
    return -1;
  }
  for (int i = 0; i < n; ++i)
    if (!w[i] || cout[i] < 1 || cin[i] < 1 || cout[i] > (1 << 20) || cin[i] > (1 << 20)) {
      set_error("xdna_conv3x3_prepare_weights_multi_bf16: invalid weight " + std::to_string(i));
      return -1;
    }
  return launch_prep_multi(n, w, wt, wtd, cout, cin, stream);
}

int xdna_conv3x3_set_wgrad_tile(int co_tile) {
  if (co_tile != 0 && co_tile != 64 && co_tile != 128) {
    set_error("xdna_conv3x3_set_wgrad_tile: 0 (by layer), 64 or 128 output channels");
    return -1;
  }
  g_wgrad_tile.store(co_tile);
  return 0;
}

int xdna_conv3x3_set_wgrad_splits(int splits) {
  if (splits < 0) {
    set_error("xdna_conv3x3_set_wgrad_splits: 0 (the model) or a positive split count");
    return -1;
  }
  g_wgrad_splits.store(splits);
  return 0;
}

int xdna_conv3x3_set_prep_tile(int co) {
  if (co != 0 && co != 8 && co != 32) {
    set_error("xdna_conv3x3_set_prep_tile: the tile must be 0 (by size), 8 or 32");
    return -1;
  }
  g_prep_co.store(co);
  return 0;
}

int xdna_conv3x3_bias_grad_bf16(const uint16_t* dy, uint16_t* gb, int B, int C, int H, int W,
                                void* stream) {
  if (B < 1 || C < 1 || H < 1 || W < 1) {
    set_error("xdna_conv3x3_bias_grad_bf16: invalid shape");
    return -1;
  }
  if (C > 65535 * 4) {
    set_error("xdna_conv3x3_bias_grad_bf16: too many channels");
    return -1;
  }
  if (!admit_launch("xdna_conv3x3_bias_grad_bf16")) return -1;
  // about 1024 workgroups: image groups per channel
  const int P = int(std::min<int64_t>(B, std::max<int64_t>(1, ceil_div(1024, C))));
  const int ipp = int(ceil_div(B, P));
  const int Pn = int(ceil_div(B, ipp));
  float* part = static_cast<float*>(xdna_hip_cache_alloc(size_t(C) * Pn * sizeof(float)));
  if (!part) return -1;
  hipStream_t st = as_stream(stream);
  bias_grad_part_kernel<<<dim3(unsigned(C), unsigned(Pn)), 256, 0, st>>>(dy, part, B, C, int64_t(H) * W, Pn, ipp);
  bias_grad_sum_kernel<<<unsigned(ceil_div(C, 4)), 256, 0, st>>>(part, gb, C, Pn);
  // stream-ordered reuse: the next user of the block runs after the sum
  xdna_hip_cache_free(part);
  return check_launch("xdna_conv3x3_bias_grad_bf16");
}

}  // extern "C"
