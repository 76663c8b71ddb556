// conv3x3w layouts on the device: NCHW bf16 <-> padded-grid row tiles.
//
// Layout (reference spec xdna_train/_designs/conv3x3w_host.py:32-46, 85-140;
// host implementation xdna_train/_native/conv_pack.cpp:632-743):
//   packed input  [groups][chunks][2126][64] bf16.  Virtual image vb = b*S + s,
//   grid row of data column j at image row y is p = (vb*(H+2) + y + 1)*wp + j + 1.
//   Group g holds rows [2048 g, 2048 g + 2126): its last 78 rows duplicate the
//   first 78 of group g+1.  Channels beyond C in the last chunk, border rows and
//   the tail of the last group are never written (the caller zero-fills once).
//   raw output rows [p][128]: output pixel (y, t) of virtual image vb sits at row
//   (vb*(H+2) + y)*wp + first + t, first = 0 (S == 1) or 1 (strips).
// The tight layout (images wider than 36 as strips of up to 36 columns with no zero
// columns: wp = Wg, data column j at row position j) is packed by the same kernels with
// the row position of data column 0 (`lead`) as a parameter.
//
// Both kernels are HBM-bound byte moves.  One thread per packed row (pixel x chunk):
// consecutive threads take consecutive image columns, so each of the (up to) 64
// channel loads of a wave is one contiguous run of NCHW, and each thread writes its
// own 128-byte row with 16-byte stores.  Unpack is the mirror image.
#include "common.h"

#include <atomic>
#include "../../include/xdna_hip.h"

namespace xdna {
namespace {

template <bool kVecStore>
__global__ __launch_bounds__(256) void pack_rows_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int C, int H, int W, int S,
    int So, int Wg, int wp, int lead, int halo_zero, int chunks, int g0, int ng, int v0, int64_t plo,
    int64_t phi, int64_t n_threads) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_threads) return;
  const int j = int(t % Wg);
  t /= Wg;
  const int y = int(t % H);
  t /= H;
  const int chunk = int(t % chunks);
  const int vb = v0 + int(t / chunks);
  const int cc = min(C - chunk * kKStep, kKStep);
  if (cc <= 0) return;
  const int b = vb / S, s = vb % S;
  const int x = (S == 1 ? 0 : s * So - 1) + j;  // source column of data column j
  if (x < 0 || x >= W) return;
  const int64_t p = (int64_t(vb) * (H + 2) + y + 1) * wp + lead + j;
  if (p < plo || p >= phi) return;
  const int64_t g = p / kGroupOutRows;
  const int r = int(p - g * kGroupOutRows);
  const bool main_w = g >= g0 && g < int64_t(g0) + ng;
  const bool halo_w = g > g0 && g <= int64_t(g0) + ng && r + kGroupOutRows < kGroupRows;
  if (!main_w && !halo_w) return;

  uint32_t v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = 0;
  const bool zero = halo_zero && S > 1 && (j == 0 || j == Wg - 1);
  if (!zero) {
    const int64_t plane = int64_t(H) * W;
    const uint16_t* sp = src + ((int64_t(b) * C + chunk * kKStep) * H + y) * W + x;
#pragma unroll
    for (int c = 0; c < kKStep; ++c) {
      if (c < cc) {
        const uint32_t h = sp[c * plane];
        v[c >> 1] |= (c & 1) ? (h << 16) : h;
      }
    }
  }
  uint16_t* rows[2];
  int nrows = 0;
  if (main_w) rows[nrows++] = dst + ((int64_t(g - g0) * chunks + chunk) * kGroupRows + r) * kKStep;
  if (halo_w)
    rows[nrows++] =
        dst + ((int64_t(g - 1 - g0) * chunks + chunk) * kGroupRows + r + kGroupOutRows) * kKStep;
  for (int k = 0; k < nrows; ++k) {
    uint16_t* d = rows[k];
    if (kVecStore && cc == kKStep) {
      uint4* d4 = reinterpret_cast<uint4*>(d);
#pragma unroll
      for (int q = 0; q < 8; ++q) d4[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
#pragma unroll
      for (int c = 0; c < kKStep; ++c)
        if (c < cc) d[c] = uint16_t((c & 1) ? (v[c >> 1] >> 16) : (v[c >> 1] & 0xFFFF));
    }
  }
}

// LDS-staged variant: a workgroup packs R full image rows of one image and one chunk,
// for every strip of those rows.  Phase 1: each item is (source pixel, 8-channel piece);
// consecutive threads take consecutive pixels, so each of the 8 channel loads of a wave
// reads a contiguous run of NCHW, and the 8 values land in LDS as one 16-byte write
// ([pixel][64 channels], see tile_piece).  Phase 2: consecutive threads take consecutive
// 16-byte pieces of packed rows, so a wave store covers 8 whole rows (1 KB contiguous).
constexpr int kLdsPitch = 64;      // elements per staged pixel (unpadded: pieces permuted)

// Element offset of 16-byte piece q (channels 8q .. 8q + 7) of staged pixel pix: pieces sit
// at position q ^ ((pix >> S) & 7) of the pixel's 128 bytes, S = log2 of the pixels per
// phase-1 item.  A 16-lane pass of 16-byte LDS accesses covers 64 banks as 16 slots of 4:
// pixel pix's position lands in slot 8 (pix % 2) + position.  Phase-1 writes (lane t at
// pixel VP t + i, one piece) then use 8 slots (2-way; 16 with VP = 1), where the padded
// 72-element pitch put 16 lanes on 4 slots; phase-2 reads (8 lanes per pixel, pixels
// x and x + 1) use all 16.
template <int S>
__device__ inline int tile_piece(int pix, int q) {
  return pix * kLdsPitch + ((q ^ ((pix >> S) & 7)) << 3);
}
constexpr int kMaxTilePix = 256;   // pixels per workgroup (LDS 32 KiB: four workgroups per CU)

// Writes the 16-byte piece q of packed row p (main copy and, for the first 78 rows of a
// group, the halo copy at the end of the previous group), when p is in [plo, phi).
__device__ inline void put_row_piece(uint16_t* __restrict__ dst, int64_t p, int q, uint4 v,
                                     int chunks, int chunk, int g0, int ng, int64_t plo,
                                     int64_t phi) {
  if (p < plo || p >= phi) return;
  const int64_t g = p / kGroupOutRows;
  const int r = int(p - g * kGroupOutRows);
  if (g >= g0 && g < int64_t(g0) + ng)
    *reinterpret_cast<uint4*>(dst + ((int64_t(g - g0) * chunks + chunk) * kGroupRows + r) * kKStep + q * 8) = v;
  if (g > g0 && g <= int64_t(g0) + ng && r + kGroupOutRows < kGroupRows)
    *reinterpret_cast<uint4*>(dst + ((int64_t(g - 1 - g0) * chunks + chunk) * kGroupRows + r + kGroupOutRows) *
                                        kKStep + q * 8) = v;
}

// kDense = false: only rows of real pixels and only the real channels are written (the
// reference's contract: the caller zero-fills once per shape).  kDense = true: every
// element of groups [g0, g0 + ng) is written, zeros included (border rows and columns,
// padded channels, the rows past the last image), so a buffer needs no fill; workgroups
// from nimg on write the rows past the last image.
// kDil (dense only): the packed image is the H x W spread of src, whose planes are
// ceil(H/2) x ceil(W/2): pixel (y, x) = src[y/2][x/2] at even y and x, 0 elsewhere (the
// gradient of a stride-2 conv on the stride-1 grid).  R is even, so a workgroup's full
// rows [y0, y0 + R) read the source rows [y0/2, y0/2 + R/2) and the LDS tile holds those.
template <int VP, bool kDense, bool kDil = false>
__global__ __launch_bounds__(256) void pack_rows_lds_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int C, int H, int W, int S,
    int So, int Wg, int wp, int lead, int halo_zero, int chunks, int g0, int ng, int b0, int64_t plo,
    int64_t phi, int R, int ybl, int nimg, int64_t tail0) {
  extern __shared__ __attribute__((aligned(16))) uint16_t tile[];
  constexpr int kVpShift = VP == 4 ? 2 : VP == 2 ? 1 : 0;
  int bid = blockIdx.x;
  if (kDense && bid >= nimg) {
    // rows [tail0, phi) hold no image: zeros for every chunk
    const int64_t n = (phi - tail0) * chunks * 8;
    const uint4 z = make_uint4(0, 0, 0, 0);
    for (int64_t i = int64_t(bid - nimg) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x - nimg) * 256) {
      const int q = int(i & 7);
      const int64_t rc = i >> 3;
      const int chunk = int(rc % chunks);
      put_row_piece(dst, tail0 + rc / chunks, q, z, chunks, chunk, g0, ng, plo, phi);
    }
    return;
  }
  const int yb = bid % ybl;
  bid /= ybl;
  const int chunk = bid % chunks;
  const int b = b0 + bid / chunks;
  const int cc = min(C - chunk * kKStep, kKStep);
  if (cc <= 0) return;
  const int y0 = yb * R;
  const int rows = min(R, H - y0);
  // source planes: H x W, or ceil(H/2) x ceil(W/2) spread over H x W (kDil)
  const int Hs = kDil ? (H + 1) >> 1 : H, Ws = kDil ? (W + 1) >> 1 : W;
  const int ys0 = kDil ? y0 >> 1 : y0;
  const int npix = (kDil ? min((rows + 1) >> 1, Hs - ys0) : rows) * Ws;
  const int64_t plane = int64_t(Hs) * Ws;
  const uint16_t* sbase = src + (int64_t(b) * C + chunk * kKStep) * plane + int64_t(ys0) * Ws;
  // phase 1: NCHW rows [y0, y0 + rows) -> tile[pix][c], pix = yy * W + x.  An item is
  // VP consecutive pixels x 16 channels: 16 loads of VP pixels each (one per channel, all
  // issued before the first LDS write), then VP x two 16-byte LDS writes.
  const int nseg16 = (cc + 15) >> 4;
  const int ngrp = (npix + VP - 1) / VP;
  const int nitem = nseg16 * ngrp;
  for (int it = threadIdx.x; it < nitem; it += 256) {
    const int seg = it / ngrp;
    const int pix0 = (it - seg * ngrp) * VP;
    const uint16_t* sp = sbase + int64_t(seg * 16) * plane + pix0;
    uint32_t d[16][(VP + 1) / 2];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool ok = seg * 16 + k < cc;
      if (VP == 4) {
        uint2 t = make_uint2(0, 0);
        if (ok) t = *reinterpret_cast<const uint2*>(sp + k * plane);
        d[k][0] = t.x;
        d[k][1] = t.y;
      } else if (VP == 2) {
        d[k][0] = ok ? *reinterpret_cast<const uint32_t*>(sp + k * plane) : 0u;
      } else {
        d[k][0] = ok ? uint32_t(sp[k * plane]) : 0u;
      }
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      if (pix0 + i < npix) {
        // dword m of pixel i: channel 2m (low half) and channel 2m + 1 (high half)
        uint32_t o[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const uint32_t a = d[2 * m][i >> 1], b = d[2 * m + 1][i >> 1];
          // v_perm_b32 selector: bytes 0-3 come from the second operand, 4-7 from the first
          o[m] = VP == 1 ? (a | (b << 16))
                         : ((i & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)
                                    : __builtin_amdgcn_perm(b, a, 0x05040100u));
        }
        *reinterpret_cast<uint4*>(tile + tile_piece<kVpShift>(pix0 + i, 2 * seg)) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(tile + tile_piece<kVpShift>(pix0 + i, 2 * seg + 1)) = make_uint4(o[4], o[5], o[6], o[7]);
      }
    }
  }
  __syncthreads();

  // phase 2: packed rows of every strip (and the halo copies into the previous group)
  if (kDense) {
    // grid rows y0+1 .. y0+rows (plus the top / bottom border row for the first / last
    // tile), all wp columns, all 64 channels
    const int gy_lo = y0 == 0 ? 0 : y0 + 1;
    const int gy_hi = y0 + rows == H ? H + 2 : y0 + rows + 1;
    const int grows = gy_hi - gy_lo;
    const int nst = S * grows * wp * 8;
    for (int t = threadIdx.x; t < nst; t += 256) {
      const int q = t & 7;
      const int opix = t >> 3;
      const int s = opix / (grows * wp);
      const int rem = opix - s * (grows * wp);
      const int gr = rem / wp, gx = rem - gr * wp;
      const int gy = gy_lo + gr;
      const int j = gx - lead;
      const int x = (S == 1 ? 0 : s * So - 1) + j;
      const bool zero_col = halo_zero && S > 1 && (j == 0 || j == Wg - 1);
      uint4 v = make_uint4(0, 0, 0, 0);
      const bool real = gy >= 1 && gy <= H && j >= 0 && j < Wg && x >= 0 && x < W && !zero_col && q * 8 < cc;
      if (kDil) {
        // image row gy - 1 and column x even: source pixel ((gy - 1) / 2, x / 2)
        if (real && ((gy - 1) & 1) == 0 && (x & 1) == 0)
          v = *reinterpret_cast<const uint4*>(tile + tile_piece<kVpShift>((((gy - 1) >> 1) - ys0) * Ws + (x >> 1), q));
      } else if (real) {
        v = *reinterpret_cast<const uint4*>(tile + tile_piece<kVpShift>((gy - 1 - y0) * W + x, q));
      }
      const int64_t p = ((int64_t(b) * S + s) * (H + 2) + gy) * wp + gx;
      put_row_piece(dst, p, q, v, chunks, chunk, g0, ng, plo, phi);
    }
    return;
  }
  const int nseg = (cc + 7) >> 3;
  const int spix = rows * Wg;  // packed rows per strip
  const int nst = S * spix * nseg;
  for (int t = threadIdx.x; t < nst; t += 256) {
    const int opix = t / nseg;
    const int q = t - opix * nseg;
    const int s = opix / spix;
    const int rem = opix - s * spix;
    const int yy = rem / Wg, j = rem - yy * Wg;
    const int x = (S == 1 ? 0 : s * So - 1) + j;  // source column of data column j
    if (x < 0 || x >= W) continue;                // no source pixel: left as the caller's zero fill
    const int64_t p = ((int64_t(b) * S + s) * (H + 2) + y0 + yy + 1) * wp + lead + j;
    if (p < plo || p >= phi) continue;
    const int64_t g = p / kGroupOutRows;
    const int r = int(p - g * kGroupOutRows);
    const bool main_w = g >= g0 && g < int64_t(g0) + ng;
    const bool halo_w = g > g0 && g <= int64_t(g0) + ng && r + kGroupOutRows < kGroupRows;
    const bool zero = halo_zero && S > 1 && (j == 0 || j == Wg - 1);
    const uint16_t* tp = tile + tile_piece<kVpShift>(yy * W + x, q);
    const bool full = (q + 1) * 8 <= cc;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (!zero) v = *reinterpret_cast<const uint4*>(tp);
    for (int k = 0; k < 2; ++k) {
      if (k == 0 && !main_w) continue;
      if (k == 1 && !halo_w) continue;
      uint16_t* d = k == 0 ? dst + ((int64_t(g - g0) * chunks + chunk) * kGroupRows + r) * kKStep
                           : dst + ((int64_t(g - 1 - g0) * chunks + chunk) * kGroupRows + r +
                                    kGroupOutRows) * kKStep;
      if (full) {
        *reinterpret_cast<uint4*>(d + q * 8) = v;
      } else {
        for (int c = q * 8; c < cc; ++c) d[c] = zero ? uint16_t(0) : tp[c - q * 8];
      }
    }
  }
}

// Zero fill of n 16-byte pieces (a kernel, not a memset, so that graph capture records a
// kernel node).
__global__ __launch_bounds__(256) void zero16_kernel(uint4* __restrict__ dst, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
    dst[i] = make_uint4(0, 0, 0, 0);
}

template <bool kVecLoad>
__global__ __launch_bounds__(256) void unpack_rows_kernel(
    const uint16_t* __restrict__ c, uint16_t* __restrict__ dst, int H, int W, int S, int So,
    int wp, int cout_valid, int C_total, int c_start, int64_t p0, int64_t p1, int v0, int TW,
    int64_t n_threads) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_threads) return;
  const int tc = int(t % TW);
  t /= TW;
  const int y = int(t % H);
  const int vb = v0 + int(t / H);
  const int b = vb / S, s = vb % S;
  const int first = S == 1 ? 0 : 1;
  const int cols = S == 1 ? W : min(So, W - s * So);
  if (tc >= cols) return;
  const int64_t p = (int64_t(vb) * (H + 2) + y) * wp + first + tc;
  if (p < p0 || p >= p1) return;
  const int x = (S == 1 ? 0 : s * So) + tc;
  const uint16_t* row = c + (p - p0) * kRawN;
  const int64_t plane = int64_t(H) * W;
  uint16_t* out = dst + ((int64_t(b) * C_total + c_start) * H + y) * W + x;
  if (kVecLoad) {
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int q = 0; q < kRawN / 8; ++q) {
      if (q * 8 < cout_valid) {
        const uint4 w = r4[q];
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int n = q * 8 + e;
          if (n < cout_valid) out[n * plane] = uint16_t((e & 1) ? (u[e >> 1] >> 16) : (u[e >> 1] & 0xFFFF));
        }
      }
    }
  } else {
    for (int n = 0; n < cout_valid; ++n) out[n * plane] = row[n];
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Image rows per workgroup of the LDS pack: 0 (default) the automatic choice, else forced
// (clamped to the image and the LDS tile); xdna_conv3x3_set_pack_rows, for measurements.
std::atomic<int> g_pack_rows{0};

int pack_launch(const char* what, const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                int S, int So, int halo_zero, int chunks, int g0, int ng, void* stream,
                bool dense = false, int layout = kLayoutRef, bool dil = false) {
  if (B < 0 || C < 0 || H < 0 || W < 0 || chunks < 0 || S < 1 || g0 < 0 || ng < 0 ||
      (S > 1 && So < 1)) {
    set_error(std::string(what) + ": invalid geometry");
    return -1;
  }
  if (B == 0 || C == 0 || H == 0 || W == 0 || chunks == 0 || ng == 0) return 0;
  const bool tight = layout == kLayoutTight && S > 1;
  const int Wg = S == 1 ? W : So + 2;
  const int wp = tight ? Wg : Wg + 2;
  const int lead = tight ? 0 : 1;
  const int64_t Bv = int64_t(B) * S;
  const int64_t img = int64_t(H + 2) * wp;
  const int64_t plo = int64_t(g0) * kGroupOutRows;
  const int64_t phi = int64_t(g0 + ng) * kGroupOutRows + (kGroupRows - kGroupOutRows);
  const int64_t v0 = plo / img;
  const int64_t v1 = std::min<int64_t>((phi - 1) / img + 1, Bv);
  if ((dense || dil) && (!aligned16(dst) || W > kMaxTilePix)) {
    set_error(std::string(what) + ": dense packing needs a 16-byte aligned destination and W <= 256");
    return -1;
  }
  if (dil && !dense) {
    set_error(std::string(what) + ": the spread pack is dense only");
    return -1;
  }
  if (v1 <= v0 && !dense) return 0;
  if (!admit_launch(what)) return -1;
  if (aligned16(dst) && W <= kMaxTilePix) {
    // whole images b0 .. b1-1 cover virtual images v0 .. v1-1; rows outside [plo, phi)
    // are skipped in the kernel
    const int64_t b0 = v1 > v0 ? v0 / S : 0, b1 = v1 > v0 ? ceil_div(v1, S) : 0;
    // tile height by image width, from a sweep of every height on the conv sweep's and the
    // style network's shapes (within 1 % of each shape's best, 5 % less pack time over the
    // sweep than filling the chip with one- or two-row tiles): 2 rows from 64 columns, 3
    // (4 on large grids) from 32, 3 from 16, else 2
    const int64_t row_tasks = (b1 - b0) * chunks * H;
    const int forced = g_pack_rows.load();
    const int by_width = W >= 64 ? 2 : W >= 32 ? (row_tasks >= 4096 ? 4 : 3) : W >= 16 ? 3 : 2;
    int R = std::max(1, std::min({forced > 0 ? forced : by_width, H, kMaxTilePix / W}));
    if (dil) R = std::max(2, R + (R & 1));  // even: a tile's source rows start at y0 / 2
    const int ybl = int(ceil_div(H, R));
    const int64_t nimg = (b1 - b0) * chunks * ybl;
    // dense: rows [tail0, phi) past the last image get workgroups of their own
    const int64_t tail0 = std::max(plo, Bv * img);
    const int64_t ntail = dense && phi > tail0 ? std::min<int64_t>(ceil_div((phi - tail0) * chunks * 8, 256), 1024) : 0;
    const int64_t blocks = nimg + ntail;
    if (blocks == 0) return 0;
    // the tile: R rows of W pixels, or R / 2 source rows of ceil(W/2) (kDil)
    const size_t lds = (dil ? size_t(R / 2) * size_t((W + 1) / 2) : size_t(R) * W) * kLdsPitch * 2;
    // pixels per lane load: every channel run (plane offset + y0 * W) must keep the
    // alignment of the load for every tile row start; the last group of a run is cut
    // short by the tile's pixel count only, and runs are padded in LDS to the group size
    // (kDil: source planes ceil(H/2) x ceil(W/2), R / 2 source rows per tile)
    const int64_t Ws = dil ? (W + 1) / 2 : W;
    const int64_t plane = dil ? int64_t((H + 1) / 2) * Ws : int64_t(H) * W;
    const int64_t tile_src = dil ? int64_t(R / 2) * Ws : int64_t(R) * W;
    const int64_t step = std::gcd<int64_t>(plane, tile_src);  // all run offsets are multiples
    const uintptr_t sa = reinterpret_cast<uintptr_t>(src);
    const int VP = (sa % 8 == 0 && step % 4 == 0 && tile_src % 4 == 0) ? 4
                   : (sa % 4 == 0 && step % 2 == 0 && tile_src % 2 == 0) ? 2 : 1;
    const dim3 grid{unsigned(blocks)};
    hipStream_t st = as_stream(stream);
#define XDNA_PACK_LAUNCH(vp, dn, ...)                                                             \
  pack_rows_lds_kernel<vp, dn, ##__VA_ARGS__><<<grid, 256, lds, st>>>(src, dst, C, H, W, S, So, Wg, wp, lead,  \
                                                      halo_zero, chunks, g0, ng, int(b0), plo, phi, R, ybl,   \
                                                      int(nimg), tail0)
    if (dil) {
      if (VP == 4) XDNA_PACK_LAUNCH(4, true, true);
      else if (VP == 2) XDNA_PACK_LAUNCH(2, true, true);
      else XDNA_PACK_LAUNCH(1, true, true);
    } else if (dense) {
      if (VP == 4) XDNA_PACK_LAUNCH(4, true);
      else if (VP == 2) XDNA_PACK_LAUNCH(2, true);
      else XDNA_PACK_LAUNCH(1, true);
    } else {
      if (VP == 4) XDNA_PACK_LAUNCH(4, false);
      else if (VP == 2) XDNA_PACK_LAUNCH(2, false);
      else XDNA_PACK_LAUNCH(1, false);
    }
#undef XDNA_PACK_LAUNCH
    return check_launch(what);
  }
  const int64_t n = (v1 - v0) * chunks * H * Wg;
  const int threads = 256;
  const int64_t blocks = ceil_div(n, threads);
  if (aligned16(dst))
    pack_rows_kernel<true><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        src, dst, C, H, W, S, So, Wg, wp, lead, halo_zero, chunks, g0, ng, int(v0), plo, phi, n);
  else
    pack_rows_kernel<false><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        src, dst, C, H, W, S, So, Wg, wp, lead, halo_zero, chunks, g0, ng, int(v0), plo, phi, n);
  return check_launch(what);
}

int unpack_launch(const char* what, const uint16_t* c, uint16_t* dst, int B, int H, int W, int S,
                  int So, int cout_valid, int C_total, int c_start, int64_t p0, int64_t p1,
                  void* stream) {
  if (B < 0 || H < 0 || W < 0 || S < 1 || cout_valid < 0 || cout_valid > kRawN ||
      c_start < 0 || c_start + cout_valid > C_total || (S > 1 && So < 1)) {
    set_error(std::string(what) + ": invalid geometry");
    return -1;
  }
  if (B == 0 || H == 0 || W == 0 || cout_valid == 0 || p1 <= p0) return 0;
  const int Wg = S == 1 ? W : So + 2;
  const int wp = Wg + 2;
  const int64_t Bv = int64_t(B) * S;
  const int64_t img = int64_t(H + 2) * wp;
  const int64_t v0 = p0 / img;
  const int64_t v1 = std::min<int64_t>((p1 - 1) / img + 1, Bv);
  if (v1 <= v0) return 0;
  if (!admit_launch(what)) return -1;
  const int TW = S == 1 ? W : So;
  const int64_t n = (v1 - v0) * H * TW;
  const int threads = 256;
  const int64_t blocks = ceil_div(n, threads);
  if (aligned16(c))
    unpack_rows_kernel<true><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        c, dst, H, W, S, So, wp, cout_valid, C_total, c_start, p0, p1, int(v0), TW, n);
  else
    unpack_rows_kernel<false><<<dim3(unsigned(blocks)), threads, 0, as_stream(stream)>>>(
        c, dst, H, W, S, So, wp, cout_valid, C_total, c_start, p0, p1, int(v0), TW, n);
  return check_launch(what);
}

}  // namespace
}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_conv3x3w_pack_input_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                                  int chunks, void* stream) {
  const int64_t m_total = int64_t(B) * (H + 2) * (W + 2);
  const int groups = int(ceil_div(m_total, kGroupOutRows));
  return pack_launch("xdna_conv3x3w_pack_input_bf16", src, dst, B, C, H, W, 1, W, 0, chunks, 0,
                     groups, stream);
}

int xdna_conv3x3w_pack_input_range_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H,
                                        int W, int chunks, int g0, int ng, void* stream) {
  return pack_launch("xdna_conv3x3w_pack_input_range_bf16", src, dst, B, C, H, W, 1, W, 0, chunks,
                     g0, ng, stream);
}

int xdna_conv3x3w_pack_input_strips_range_bf16(const uint16_t* src, uint16_t* dst, int B, int C,
                                               int H, int W, int S, int So, int halo_zero,
                                               int chunks, int g0, int ng, void* stream) {
  return pack_launch("xdna_conv3x3w_pack_input_strips_range_bf16", src, dst, B, C, H, W, S, So,
                     halo_zero, chunks, g0, ng, stream);
}

int xdna_conv3x3w_pack_input_dense_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H,
                                         int W, void* stream) {
  if (B < 1 || C < 1 || H < 1 || W < 1) {
    set_error("xdna_conv3x3w_pack_input_dense_bf16: invalid shape");
    return -1;
  }
  const ConvGeom cg = conv_geom(B, H, W);
  return pack_launch("xdna_conv3x3w_pack_input_dense_bf16", src, dst, B, C, H, W, cg.st.S, cg.st.So, 0,
                     int(ceil_div(C, kKStep)), 0, cg.groups, stream, /*dense=*/true);
}

size_t xdna_conv3x3_layout_packed_bytes(int B, int C, int H, int W, int layout) {
  if (B < 1 || C < 1 || H < 1 || W < 1 || (layout != kLayoutRef && layout != kLayoutTight)) return 0;
  const ConvGeom cg = conv_geom(B, H, W, layout);
  return size_t(cg.groups) * size_t(ceil_div(C, kKStep)) * kGroupRows * kKStep * 2;
}

int xdna_conv3x3_layout_pack_dilate2_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                                          int layout, void* stream) {
  if (B < 1 || C < 1 || H < 1 || W < 1 || (layout != kLayoutRef && layout != kLayoutTight) || !src || !dst) {
    set_error("xdna_conv3x3_layout_pack_dilate2_bf16: invalid arguments");
    return -1;
  }
  if (!aligned16(dst) || W > kMaxTilePix) {
    set_error("xdna_conv3x3_layout_pack_dilate2_bf16: needs a 16-byte aligned destination and W <= 256");
    return -1;
  }
  const ConvGeom cg = conv_geom(B, H, W, layout);
  return pack_launch("xdna_conv3x3_layout_pack_dilate2_bf16", src, dst, B, C, H, W, cg.st.S, cg.st.So, 0,
                     int(ceil_div(C, kKStep)), 0, cg.groups, stream, /*dense=*/true, layout, /*dil=*/true);
}

int xdna_conv3x3_layout_pack_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W, int layout,
                                  void* stream) {
  if (B < 1 || C < 1 || H < 1 || W < 1 || (layout != kLayoutRef && layout != kLayoutTight) || !src || !dst) {
    set_error("xdna_conv3x3_layout_pack_bf16: invalid arguments");
    return -1;
  }
  if (!aligned16(dst)) {
    set_error("xdna_conv3x3_layout_pack_bf16: the destination must be 16-byte aligned");
    return -1;
  }
  const ConvGeom cg = conv_geom(B, H, W, layout);
  const int chunks = int(ceil_div(C, kKStep));
  if (W <= kMaxTilePix)
    return pack_launch("xdna_conv3x3_layout_pack_bf16", src, dst, B, C, H, W, cg.st.S, cg.st.So, 0, chunks, 0,
                       cg.groups, stream, /*dense=*/true, layout);
  // wider rows than the LDS tile: zero fill, then the real pixels
  const int64_t n16 = int64_t(cg.groups) * chunks * kGroupRows * kKStep * 2 / 16;
  if (!admit_launch("xdna_conv3x3_layout_pack_bf16")) return -1;
  zero16_kernel<<<unsigned(std::min<int64_t>(ceil_div(n16, 256), 16384)), 256, 0, as_stream(stream)>>>(
      reinterpret_cast<uint4*>(dst), n16);
  if (check_launch("xdna_conv3x3_layout_pack_bf16")) return -1;
  return pack_launch("xdna_conv3x3_layout_pack_bf16", src, dst, B, C, H, W, cg.st.S, cg.st.So, 0, chunks, 0,
                     cg.groups, stream, /*dense=*/false, layout);
}

int xdna_conv3x3w_unpack_output_bf16(const uint16_t* c, uint16_t* dst, int B, int H, int W,
                                     int cout_valid, int C_total, int c_start, void* stream) {
  const int64_t m_total = int64_t(B) * (H + 2) * (W + 2);
  return unpack_launch("xdna_conv3x3w_unpack_output_bf16", c, dst, B, H, W, 1, W, cout_valid,
                       C_total, c_start, 0, m_total, stream);
}

int xdna_conv3x3w_unpack_output_range_bf16(const uint16_t* c, uint16_t* dst, int B, int H, int W,
                                           int cout_valid, int C_total, int c_start, int p0,
                                           int p1, void* stream) {
  return unpack_launch("xdna_conv3x3w_unpack_output_range_bf16", c, dst, B, H, W, 1, W,
                       cout_valid, C_total, c_start, p0, p1, stream);
}

int xdna_conv3x3w_unpack_output_strips_range_bf16(const uint16_t* c, uint16_t* dst, int B, int H,
                                                  int W, int S, int So, int cout_valid,
                                                  int C_total, int c_start, int p0, int p1,
                                                  void* stream) {
  return unpack_launch("xdna_conv3x3w_unpack_output_strips_range_bf16", c, dst, B, H, W, S, So,
                       cout_valid, C_total, c_start, p0, p1, stream);
}

int xdna_conv3x3w_geometry(int B, int Cin, int H, int W, int64_t* out7) {
  if (B < 1 || Cin < 1 || H < 1 || W < 1) {
    set_error("xdna_conv3x3w_geometry: invalid shape");
    return -1;
  }
  const ConvGeom g = conv_geom(B, H, W);
  out7[0] = g.st.S;
  out7[1] = g.st.So;
  out7[2] = g.st.Wg;
  out7[3] = g.st.wp;
  out7[4] = g.groups;
  out7[5] = ceil_div(Cin, kKStep);
  out7[6] = g.m_total;
  return 0;
}

int xdna_conv3x3_set_pack_rows(int rows) {
  if (rows < 0) {
    set_error("xdna_conv3x3_set_pack_rows: rows must be 0 (automatic) or positive");
    return -1;
  }
  g_pack_rows.store(rows);
  return 0;
}

}  // extern "C"
