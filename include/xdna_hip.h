/*
 * xdna_hip.h -- C ABI of the MI355X (gfx950) training hot path.
 *
 * This is the boundary between the PrivateUse1 "xdna" PyTorch backend (host C++)
 * and the hand-written HIP kernels.  Plain pointers, sizes and a hipStream_t passed
 * as void*; no torch types.  Every pointer argument of a compute entry point is
 * DEVICE memory.  Conventions follow the reference's XRT shim
 * (xdna_train/_vendor/xrt_shim/xrt_shim.h:2-3, 160): an int status (0 = ok,
 * -1 = error) and a thread-local message from xdna_hip_last_error(); pointer
 * returning calls return NULL on error.
 *
 * bf16 tensors are passed as uint16_t bit patterns (round-to-nearest-even when
 * produced from fp32).
 */
#ifndef XDNA_HIP_H
#define XDNA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Errors, poisoning and failure injection                                   */
/* ------------------------------------------------------------------------ */

/* Last error message of the calling thread ("" if none).
 * Replaces shim_last_error (xrt_shim.h:160; xrt_shim.cpp:235-249). */
const char* xdna_hip_last_error(void);

/* 1 once the process is poisoned: a launch or wait failed in a way that may
 * leave device work in flight.  Poisoned processes refuse new launches and
 * leak frees.  Replaces shim_dispatch_poisoned (xrt_shim.cpp:139-151). */
int xdna_hip_poisoned(void);

/* Test hook: the n-th launch from now (n >= 1) fails with an injected error
 * before touching the device; n = 0 disables.  `poison` != 0 also poisons the
 * process at that point (the timeout-without-abort case of
 * xrt_shim.cpp:174-233).  Host-only: nothing is launched. */
int xdna_hip_inject_failure(int64_t nth_launch, int poison);

/* Clears the poisoned flag and the injection counter (tests only). */
int xdna_hip_reset_failure_state(void);

/* Launches issued so far through this library (profiling/tests). */
int64_t xdna_hip_launch_count(void);

/* ------------------------------------------------------------------------ */
/* Device, memory, streams, events  (the shim_* analogue, xrt_shim.h:29-160) */
/* ------------------------------------------------------------------------ */

int xdna_hip_device_count(void);
int xdna_hip_set_device(int device);
int xdna_hip_get_device(int* device);
/* Name, CU count and HBM bytes of the current device. */
int xdna_hip_device_properties(char* name, size_t name_len, int* cu_count,
                               size_t* total_mem, int* gcn_arch);

/* Raw device allocation (no caching).  NULL on failure. */
void* xdna_hip_malloc(size_t bytes);
int xdna_hip_free(void* ptr);

/* Size-binned caching allocator over xdna_hip_malloc (the XdnaBoCache analogue,
 * torch_xdna_device.cpp:205-296).  All work of the library is ordered on the
 * caller's stream, so a released block is reused by later launches in stream
 * order.  Blocks are rounded up to 512 B (small) or 2 MiB (large). */
void* xdna_hip_cache_alloc(size_t bytes);
int xdna_hip_cache_free(void* ptr);
/* Returns every cached (unused) block to the device. */
int xdna_hip_cache_empty(void);
/* stats[0..5] = cached_bytes, allocated_bytes, max_allocated_bytes,
 * fresh_allocations, reuses, frees. */
int xdna_hip_cache_stats(int64_t* stats, int n);

/* Private pools of the cache, for graph capture (the role of PyTorch's graph memory
 * pools; no reference counterpart, the reference has no graph capture).  Between
 * pool_begin(pool) and pool_end() the calling thread's cache_alloc calls are served from
 * `pool` (new hipMalloc calls run with the thread's capture mode relaxed), and blocks of
 * the pool return to it when freed, so they are never handed to other work while a graph
 * that uses them can be replayed.  pool_release(pool) gives the pool's blocks back to
 * the shared pool (call it after the last replay). */
int64_t xdna_hip_cache_pool_create(void);
int xdna_hip_cache_pool_begin(int64_t pool);
int xdna_hip_cache_pool_end(void);
int xdna_hip_cache_pool_release(int64_t pool);

/* out[i] = bf16 rounding of in[i] as every kernel of the library applies it: round to
 * nearest even, NaN -> 0x7FC0 (c10::BFloat16's convention, which the reference's CPU
 * path uses).  A diagnostic that lets tests pin the rounding; no reference counterpart. */
int xdna_round_bf16(const float* in, uint16_t* out, int64_t n, void* stream);

/* The calling thread's current private pool (0: the shared pool). */
int64_t xdna_hip_cache_pool_current(void);

/* 1 if `stream` is capturing a graph, 0 if not, -1 on error.  The backend asks this
 * before using its host-side caches of device buffers, whose contents a captured graph
 * must not depend on. */
int xdna_hip_stream_capturing(void* stream);

int xdna_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                          void* stream); /* kind: 1 H2D, 2 D2H, 3 D2D, 4 default */
int xdna_hip_memset_async(void* dst, int value, size_t bytes, void* stream);

/* Host waits with a deadline (the dispatch deadline of xrt_shim.cpp:57-90, 174-233).
 * Each returns 0 when the work is done, -1 on an error reported by the device or the
 * runtime, and -2 when the deadline passed first: the work may still be running, so the
 * process is poisoned (later launches are refused, frees leak).  The message from
 * xdna_hip_last_error() starts with "deadline:" and names what was waited for.  The
 * deadline is XDNA_WAIT_TIMEOUT_MS (default 30000; 0 = no limit). */
int xdna_hip_stream_synchronize(void* stream);
int xdna_hip_device_synchronize(void);
int xdna_hip_set_wait_timeout_ms(int64_t ms);
int64_t xdna_hip_wait_timeout_ms(void);
/* Longest completed wait of this process, in ms (to size the deadline by measurement;
 * replaces shim_dispatch_max_wait_ms, xrt_shim.h:81). */
double xdna_hip_max_wait_ms(void);
/* Test hook: the n-th host wait from now (n >= 1) reports a timeout at once, without
 * touching the device, and poisons the process; n = 0 disables.  Host-only. */
int xdna_hip_inject_wait_timeout(int64_t nth_wait);

void* xdna_hip_event_create(int timing);
int xdna_hip_event_destroy(void* event);
int xdna_hip_event_record(void* event, void* stream);
/* Bounded like the waits above: 0 done, -1 error, -2 deadline. */
int xdna_hip_event_synchronize(void* event);
/* 1 done, 0 pending, -1 error. */
int xdna_hip_event_query(void* event);
int xdna_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int xdna_hip_stream_wait_event(void* stream, void* event);
/* No counterpart in the reference: a stream of the current device at the default
 * priority, ordered against other streams only by events (the backend's side stream for
 * weight gradients that run beside input gradients inside a captured graph).  NULL on
 * error.  Not destroyed: it lives until the process ends. */
void* xdna_hip_stream_create(void);

/* ------------------------------------------------------------------------ */
/* conv3x3w layouts: NCHW <-> tiled padded-grid rows (bit-exact with the     */
/* reference's host packing).  Device pointers; same arguments and meaning   */
/* as the reference functions named, plus the stream.                        */
/*                                                                          */
/* Packed input: [groups][chunks][2126][64] bf16.  Row p of the padded grid   */
/* of virtual image vb = b*S + s is (vb*(H+2) + y + 1)*wp + j + 1 for data    */
/* column j; group g holds rows [2048 g, 2048 g + 2126).  Only real pixels    */
/* and channels are written: the caller zero-fills dst once per shape.        */
/* ------------------------------------------------------------------------ */

/* Replaces xdna_conv3x3w_pack_input_bf16 (conv_pack.cpp:352-393). */
int xdna_conv3x3w_pack_input_bf16(const uint16_t* src, uint16_t* dst, int B, int C,
                                  int H, int W, int chunks, void* stream);

/* Replaces xdna_conv3x3w_pack_input_range_bf16 (conv_pack.cpp:529-583):
 * groups [g0, g0+ng) written to dst laid out [ng][chunks][2126][64]. */
int xdna_conv3x3w_pack_input_range_bf16(const uint16_t* src, uint16_t* dst, int B, int C,
                                        int H, int W, int chunks, int g0, int ng,
                                        void* stream);

/* Replaces xdna_conv3x3w_pack_input_strips_range_bf16 (conv_pack.cpp:632-700):
 * width tiling into S strips of So output columns (S = 1: plain layout);
 * halo_zero writes zeros in the two strip-halo data columns (dY for dW). */
int xdna_conv3x3w_pack_input_strips_range_bf16(const uint16_t* src, uint16_t* dst, int B,
                                               int C, int H, int W, int S, int So,
                                               int halo_zero, int chunks, int g0, int ng,
                                               void* stream);

/* The whole packed input of xdna_conv3x3w_geometry (all groups and chunks, the strip
 * layout for W > 36) with every element written: the bytes at pixel rows and real
 * channels equal xdna_conv3x3w_pack_input_strips_range_bf16's, every other byte is zero.
 * No reference counterpart: the reference zero-fills a packed buffer once per shape
 * (torch_xdna_device.cpp:1848-1872) and packs real pixels only; this form serves callers
 * that recycle one buffer across shapes or replay captured graphs.  dst must be 16-byte
 * aligned and W <= 256. */
int xdna_conv3x3w_pack_input_dense_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H,
                                        int W, void* stream);

/* BFP16 weight codec (the reference's NPU weight wire format, bit-exact).
 * Replaces xdna_conv3x3w_pack_weights_bfp16 (conv_pack.cpp:398-443; spec
 * conv3x3w_host.py:49-82): OIHW bf16 [Cout][Cin][3][3] -> bfp16ebs8 bytes for output
 * channels [128*n_block, +128), blocks [chunk*9+tap][n/16][k/8][2][8 n][8 k] of 9 bytes
 * (largest biased exponent, then 8 int8 mantissas round(v * 2^(133-e)) clamped to
 * [-128, 127]); channels past Cin / Cout encode as zeros.  Same arguments as the
 * reference plus the stream; dst holds xdna_conv3x3w_weights_bfp16_bytes(chunks) bytes,
 * 16-byte aligned. */
int xdna_conv3x3w_pack_weights_bfp16(const uint16_t* w, uint8_t* dst, int Cout, int Cin, int chunks,
                                     int n_block, void* stream);
/* Replaces xdna_conv3x3w_pack_weights_dx_bfp16 (conv_pack.cpp:474-519): the same bytes
 * for the dX conv's weights w'[ci][co][dy][dx] = w[co][ci][2-dy][2-dx], read from the
 * forward weight w [Cout_fwd][Cin_fwd][3][3]; chunks = ceil(Cout_fwd / 64), n_block over
 * Cin_fwd. */
int xdna_conv3x3w_pack_weights_dx_bfp16(const uint16_t* w, uint8_t* dst, int Cout_fwd, int Cin_fwd,
                                        int chunks, int n_block, void* stream);
/* Bytes of one 128-channel block of BFP16 weights: chunks * 9 * 64 * 128 * 9 / 8
 * (the reference's b_bytes, torch_xdna_device.cpp:2352-2367). */
size_t xdna_conv3x3w_weights_bfp16_bytes(int chunks);
/* No reference counterpart (the reference decodes inside its NPU kernel): 9-byte BFP16
 * blocks -> 8 floats each, v = int8 mantissa * 2^(e - 133); for tests and for
 * reproducing the NPU's weight rounding. */
int xdna_bfp16_decode_f32(const uint8_t* src, float* dst, int64_t nblocks, void* stream);

/* BFP16 emulation of the reference NPU's conv arithmetic (the optional mode its
 * benchmarks/bfp16_training_gate.py:1-20 restates on the CPU; kernel
 * _designs/conv3x3w_kernel.cc:40-51, 105-108, 129-138).
 *
 * xdna_bfp16_quantize8_bf16: every aligned run of 8 bf16 values (nblocks runs, 16 bytes
 * each, 16-byte aligned; src == dst allowed) becomes the values of its bfp16ebs8 block,
 * q * 2^(e_max - 133) with q the codec's mantissa (conv_pack.cpp:398-443: e_max the
 * largest biased exponent, q = clamp(round_half_even(v * 2^(133 - e_max)), -128, 127)),
 * as bf16 bits (exact; -2^128 overflows to -inf).  NaN stays NaN; +-inf saturate to +-inf
 * as the codec's bytes decode.  On the packed rows this is the NPU core's 8-channel
 * conversion of the activations; on the prepared weights, the codec's blocks.
 *
 * xdna_conv3x3_layout_rows_bfp16_emul_bf16: xdna_conv3x3_layout_rows_act_bf16 with that
 * arithmetic: the packed input and the prepared weights quantized (into transient
 * copies), the running sum stored as bf16 after every (chunk, tap), chunks outer and the
 * 9 taps inner as the NPU loops (conv3x3w.py:172-177), the bias added after the last
 * rounding in one more bf16 rounding (torch_xdna_device.cpp:2477-2480).  The forward and
 * input-gradient convs use it (the reference's NPU runs both); weight gradients stay
 * exact. */
int xdna_bfp16_quantize8_bf16(const uint16_t* src, uint16_t* dst, int64_t nblocks, void* stream);
int xdna_conv3x3_layout_rows_bfp16_emul_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias,
                                             uint16_t* y, int B, int cin, int cout, int H, int W, int layout, int act,
                                             void* stream);

/* Replaces xdna_conv3x3w_unpack_output_bf16 (conv_pack.cpp:447-466):
 * [groups*2048][128] bf16 rows -> channel slice [c_start, c_start+cout_valid)
 * of NCHW [B][C_total][H][W] (valid pixels only). */
int xdna_conv3x3w_unpack_output_bf16(const uint16_t* c, uint16_t* dst, int B, int H, int W,
                                     int cout_valid, int C_total, int c_start, void* stream);

/* Replaces xdna_conv3x3w_unpack_output_range_bf16 (conv_pack.cpp:587-616):
 * rows [p0, p1); c points at row p0. */
int xdna_conv3x3w_unpack_output_range_bf16(const uint16_t* c, uint16_t* dst, int B, int H,
                                           int W, int cout_valid, int C_total, int c_start,
                                           int p0, int p1, void* stream);

/* Replaces xdna_conv3x3w_unpack_output_strips_range_bf16 (conv_pack.cpp:706-743). */
int xdna_conv3x3w_unpack_output_strips_range_bf16(const uint16_t* c, uint16_t* dst, int B,
                                                  int H, int W, int S, int So,
                                                  int cout_valid, int C_total, int c_start,
                                                  int p0, int p1, void* stream);

/* ------------------------------------------------------------------------ */
/* 3x3 stride-1 pad-1 convolution (bf16 in/out, fp32 accumulation, one       */
/* rounding).  Replaces the NPU conv3x3w runtime: XdnaConv3x3wRuntime::run    */
/* (torch_xdna_device.cpp:2317-2483), input_grad (:2515-2522) and             */
/* XdnaConv3x3wDwRuntime::compute (:2683-2751).                               */
/* ------------------------------------------------------------------------ */

/* Geometry of the reference plan (torch_xdna_device.cpp:1927-1937, 2112-2157):
 * out[0..6] = strips S, strip_out So, grid_w Wg, wp, groups, chunks(Cin), m_total. */
int xdna_conv3x3w_geometry(int B, int Cin, int H, int W, int64_t* out7);

/* Workspace bytes for the forward (or dgrad, where Cin is dY's channel count)
 * call: packed input + prepared weights. */
size_t xdna_conv3x3_fwd_workspace_bytes(int B, int Cin, int Cout, int H, int W);

/* y[B][Cout][H][W] = conv3x3(x[B][Cin][H][W], w[Cout][Cin][3][3]) (+ bias[Cout]).
 * bias may be NULL.  `workspace` holds the packed input (zero-filled here) and
 * the prepared weights.  A packed copy of x is left at the start of the
 * workspace ([groups][chunks][2126][64]). */
int xdna_conv3x3_fwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                          uint16_t* y, int B, int Cin, int Cout, int H, int W,
                          void* workspace, size_t workspace_bytes, void* stream);

/* dx[B][Cin][H][W] = conv3x3(dy[B][Cout][H][W], flip-swap(w)):
 * w'[ci][co][dy][dx] = w[co][ci][2-dy][2-dx] (conv_pack.cpp:470-473),
 * applied in the weight preparation (no flipped copy of w is made). */
size_t xdna_conv3x3_dgrad_workspace_bytes(int B, int Cin, int Cout, int H, int W);
int xdna_conv3x3_dgrad_bf16(const uint16_t* dy, const uint16_t* w, uint16_t* dx, int B,
                            int Cin, int Cout, int H, int W, void* workspace,
                            size_t workspace_bytes, void* stream);

/* gw[Cout][Cin][3][3] = sum over pixels of dy x shifted(x); gb[Cout] = sum dy
 * (gb may be NULL).  fp32 sums, deterministic two-stage reduction (the same
 * bits on every call), one bf16 rounding. */
size_t xdna_conv3x3_wgrad_workspace_bytes(int B, int Cin, int Cout, int H, int W);
int xdna_conv3x3_wgrad_bf16(const uint16_t* x, const uint16_t* dy, uint16_t* gw,
                            uint16_t* gb, int B, int Cin, int Cout, int H, int W,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Weight gradient (+ bias gradient when gb is not null) from the packed row layouts the
 * forward and input-gradient convs use: xp = x packed in row layout `layout` (Cin
 * channels), dp = dY packed the same way (Cout channels; the input gradient's own packed
 * operand).  No channel-major copy of either is made, and any width works (strips).  Same
 * split-K partials and fixed-order reduce as xdna_conv3x3_wgrad_bf16 (workspace:
 * xdna_conv3x3_wgrad_rows_workspace_bytes, 0 for an invalid shape or layout).  Replaces
 * the same reference stages as xdna_conv3x3_wgrad_bf16 (XdnaConv3x3wDwRuntime::
 * pack_operands / compute, torch_xdna_device.cpp:2660-2751). */
size_t xdna_conv3x3_wgrad_rows_workspace_bytes(int B, int Cin, int Cout, int H, int W, int layout);
/* Output rows per k-tile of xdna_conv3x3_wgrad_rows_bf16: 0 the default (128), 64 or 128.
 * The split-K partition, and with it the fp32 summation order, follows from it; both stay
 * within the conv bar.  Workspace sizes depend on it: query them after setting it.  No
 * reference counterpart (measurements and tests). */
int xdna_conv3x3_set_wgrad_rows_kt(int kt_rows);
/* Kernel of xdna_conv3x3_wgrad_rows_bf16: 0 the default (form 2), 1 k-tiles staged through
 * registers (their rows as set by xdna_conv3x3_set_wgrad_rows_kt), 2 64-row k-tiles loaded
 * straight into LDS four k-tiles deep.  Like the k-tile setter it changes the split-K
 * partition (and the workspace size) within the conv bar.  No reference counterpart
 * (measurements and tests). */
int xdna_conv3x3_set_wgrad_rows_kernel(int form);
int xdna_conv3x3_wgrad_rows_bf16(const uint16_t* xp, const uint16_t* dp, uint16_t* gw, uint16_t* gb, int B,
                                 int Cin, int Cout, int H, int W, int layout, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Bias gradient alone: gb[c] = sum_{b,y,x} dy[b][c][y][x] (fp32 sum, one rounding). */
int xdna_conv3x3_bias_grad_bf16(const uint16_t* dy, uint16_t* gb, int B, int C, int H,
                                int W, void* stream);

/* --- the same convolutions as separate stages (the backend caches packed inputs and
 * prepared weights across calls, like the reference's packed-buffer pool and weight
 * cache, torch_xdna_device.cpp:1819-1914, 2200-2271) --- */

/* Bytes of the packed input [groups][chunks][2126][64] of an NCHW [B][C][H][W]
 * tensor in the strip layout the conv uses. */
size_t xdna_conv3x3w_packed_bytes(int B, int C, int H, int W);

/* Bytes of the prepared weights of a conv with `cin` input / `cout` output channels. */
size_t xdna_conv3x3_prepared_weight_bytes(int cin, int cout);

/* OIHW w[Cout][Cin][3][3] -> prepared A operand.  dgrad = 0: the forward conv
 * (cin = Cin, cout = Cout).  dgrad = 1: the input-gradient conv (cin = Cout,
 * cout = Cin) with the flip+swap map of conv_pack.cpp:470-473. */
int xdna_conv3x3_prepare_weights_bf16(const uint16_t* w, uint16_t* wt, int Cout, int Cin,
                                      int dgrad, void* stream);

/* Both prepared forms of one weight in one launch: wt as xdna_conv3x3_prepare_weights_bf16
 * with dgrad = 0, wt_dgrad as with dgrad = 1 (each sized by
 * xdna_conv3x3_prepared_weight_bytes of its direction).  For trainable weights, whose
 * forward prepares the input gradient's form too.  No reference counterpart. */
int xdna_conv3x3_prepare_weights_both_bf16(const uint16_t* w, uint16_t* wt, uint16_t* wt_dgrad, int Cout,
                                           int Cin, void* stream);

/* y[B][cout][H][W] = conv of the packed input xp (cin channels, strip layout of W)
 * with prepared weights wt (+ bias[cout], may be NULL).  One kernel. */
int xdna_conv3x3_rows_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias,
                           uint16_t* y, int B, int cin, int cout, int H, int W, void* stream);

/* Row layouts of the packed operands.  XDNA_CONV3X3_LAYOUT_REF: the reference's conv3x3w
 * layout above (images wider than 36 as strips of up to 34 columns, each strip row with
 * one neighbour column per side and two zero columns: wp = So + 4).
 * XDNA_CONV3X3_LAYOUT_TIGHT: identical up to 36 columns; wider images as strips of up to
 * 36 columns whose rows hold the strip's columns and one neighbour column per side and
 * nothing else (wp = So + 2, data column j at row position j): the zero columns are never
 * a tap of a real output, and 72 columns take 2 strips of 38 positions instead of 3 of
 * 28.  Same groups of 2126 rows.  The backend's conv ops use the tight layout; no
 * reference counterpart (an internal layout of the same kernels). */
#define XDNA_CONV3X3_LAYOUT_REF 0
#define XDNA_CONV3X3_LAYOUT_TIGHT 1

/* Bytes of the packed input in `layout` (0 for an invalid shape or layout). */
size_t xdna_conv3x3_layout_packed_bytes(int B, int C, int H, int W, int layout);

/* Packs NCHW src into `layout`, writing every element (zeros included: the buffer needs
 * no fill; images wider than 256 are zero-filled by a kernel first).  dst 16-byte aligned.
 * For XDNA_CONV3X3_LAYOUT_REF the result equals xdna_conv3x3w_pack_input_dense_bf16's. */
int xdna_conv3x3_layout_pack_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W, int layout,
                                  void* stream);

/* xdna_conv3x3_rows_bf16 on an input packed in `layout`. */
int xdna_conv3x3_layout_rows_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                  int B, int cin, int cout, int H, int W, int layout, void* stream);

/* General 2-D convolution, bf16 in/out, fp32 accumulation: any kernel size, stride and
 * padding (dilation 1, groups 1), NCHW activations and OIHW weights.  Replaces the
 * reference's CPU route for convolutions outside its 3x3 path
 * (convolution_overrideable_xdna / convolution_backward_overrideable_xdna falling back to
 * aten::convolution on host aliases, torch_xdna_device.cpp:4594-4604, 4862-4874).
 * Output size Ho = (H + 2 ph - KH) / sh + 1 (likewise Wo).  Forward: y [B][Cout][Ho][Wo]
 * (+ bias [Cout] or null).  dgrad: dx [B][Cin][H][W] from dy [B][Cout][Ho][Wo].  wgrad:
 * gw [Cout][Cin][KH][KW] and, when gb is not null, the bias gradient [Cout]; its pixel
 * reduction is split over workgroups and summed in a fixed order (same bits every call).
 * Every tensor below 2^31 elements. */
int xdna_conv2d_fwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* y, int B,
                         int Cin, int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph, int pw,
                         void* stream);
int xdna_conv2d_dgrad_bf16(const uint16_t* dy, const uint16_t* w, uint16_t* dx, int B, int Cin, int Cout,
                           int H, int W, int KH, int KW, int sh, int sw, int ph, int pw, void* stream);
int xdna_conv2d_wgrad_bf16(const uint16_t* x, const uint16_t* dy, uint16_t* gw, uint16_t* gb, int B, int Cin,
                           int Cout, int H, int W, int KH, int KW, int sh, int sw, int ph, int pw,
                           void* stream);

/* Kernel selection of xdna_conv2d_fwd_bf16 / xdna_conv2d_dgrad_bf16, for measurements and
 * tests: 0 automatic (default: at stride 1 with at most 32 output and at least 16 input
 * channels of the direction, and a padded output width up to 128, the direct form, which stages the
 * input rows of 4 output rows in LDS as a zero-padded grid and reads every tap as a row
 * offset; else the gather GEMM), 1 the gather GEMM only.  No reference counterpart. */
int xdna_conv2d_set_variant(int variant);

/* Kernel selection of xdna_conv3x3_rows_bf16 (and the conv calls built on it), for
 * measurements and tests: 0 automatic (default), 1 the main kernel (128 output channels
 * x 64-256 rows per workgroup, weights streamed from L2 per tap), 2 / 3 the small-grid
 * kernel (64 output channels x 64 / 128 rows, whole chunks staged in LDS, split-K when
 * the grid is smaller than the CU count), 4 the wide kernel (256 output channels x 256
 * rows, 8 waves, weights staged in LDS; used for cout > 128 only, else the main kernel),
 * 5 its four-wave form (one wave per SIMD with 128 x 128 wave tiles, fragments
 * software-pipelined; cout > 128 only; the automatic choice for cout >= 256 on large
 * grids), 6 / 7 / 8 four-wave kernels with 128 channels x 256 rows, 128 channels x 512
 * rows and 64 channels x 512 rows per workgroup (any cout), 9 the four-wave kernel with
 * 64 channels x 256 rows and two workgroups per CU (the automatic choice up to 256
 * output channels on all but the smallest grids), 10 / 11 the 128 x 512 and 64 x 256
 * kernels with 16x16x32 MFMAs (10 is the automatic choice where 7 was, 11 where 9 was for
 * 256 output channels on large grids).
 * Results agree to the same tolerance; only the
 * summation grouping differs.  No reference counterpart (a tuning knob, like the
 * reference's XDNA_* performance environment variables).  XDNA_ROWS_VARIANT sets the
 * initial value. */
int xdna_conv3x3_set_rows_variant(int variant);

/* wgrad stage 1: x and dy re-laid out channel-major into the workspace (snapshots:
 * stage 2 reads neither tensor).  Stage 2: the MFMA reduction over pixels and the
 * fixed-order split reduction into gw (and gb when not NULL). */
int xdna_conv3x3_wgrad_pack_bf16(const uint16_t* x, const uint16_t* dy, int B, int Cin,
                                 int Cout, int H, int W, void* workspace,
                                 size_t workspace_bytes, void* stream);
int xdna_conv3x3_wgrad_packed_bf16(uint16_t* gw, uint16_t* gb, int B, int Cin, int Cout,
                                   int H, int W, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* ------------------------------------------------------------------------ */
/* GEMM: replaces mm_xdna / XdnaGemmRuntime::run (torch_xdna_device.cpp:      */
/* 4387-4417, 1358-1457), addmm_out_xdna (:3740-3768) and bmm_out_xdna        */
/* (:3770-3790).                                                              */
/*                                                                          */
/* C[b][m][n] = alpha * sum_k A[b][m][k] B[b][k][n] + beta * bias           */
/* with arbitrary element strides (lda_m, lda_k), (ldb_k, ldb_n), (ldc_m,     */
/* ldc_n) and batch strides; fp32 accumulation, one bf16 rounding.  bias is   */
/* NULL, a [n] row vector (bias_mode 1), an [m][n] matrix with strides        */
/* (bias_sm, bias_sn) (bias_mode 2) or a [m] column vector (bias_mode 3).     */
/* beta == 0 ignores bias (NaNs in it are not propagated), like torch.        */
/* ------------------------------------------------------------------------ */
int xdna_gemm_bf16(const uint16_t* A, const uint16_t* Bm, uint16_t* C, const uint16_t* bias,
                   int batch, int M, int N, int K,
                   int64_t lda_m, int64_t lda_k, int64_t stride_a,
                   int64_t ldb_k, int64_t ldb_n, int64_t stride_b,
                   int64_t ldc_m, int64_t ldc_n, int64_t stride_c,
                   int bias_mode, int64_t bias_sm, int64_t bias_sn,
                   float alpha, float beta, void* stream);

/* Kernel selection of xdna_gemm_bf16, for measurements and tests: 0 automatic (default),
 * 1 the 128 x 128 kernel (any strides, split-K for few long-K tiles), 2 the 256 x 256
 * kernel (8 waves; operands with a unit stride along k or along rows only, else 1 is
 * used), 3 its four-wave form (one wave per SIMD with 128 x 128 wave tiles, software-
 * pipelined, operands staged through registers; also needs K % 8 == 0 and rows % 8 == 0
 * for row-contiguous operands, else 2 or 1), 4 the four-wave kernel with operands loaded
 * straight into LDS (32x32x16 MFMAs; same conditions), 5 that kernel with 16x16x32 MFMAs
 * (the automatic choice on large grids or long K where 3 applies).  No reference
 * counterpart (a tuning knob).
 * XDNA_GEMM_VARIANT sets the initial value. */
int xdna_gemm_set_variant(int variant);

/* 1 (default): under the automatic choice, products with a side or a k of at most 128
 * (and k at most 8192) take the batched small-matrix kernel (64 x 64 tiles, k-tiles of 64
 * with the next one's loads in flight, split-K finished by the fixed-order reduce): the
 * style loss's Gram matrices and their gradients.  0: the other kernels only.  No
 * reference counterpart (a tuning knob).  XDNA_GEMM_SMALL sets the initial value. */
int xdna_gemm_set_small(int on);

/* Image rows per workgroup of the packs that stage rows in LDS: 0 (default) the automatic
 * choice, else this many (clamped to the image and to 256 pixels).  For measurements; no
 * reference counterpart. */
int xdna_conv3x3_set_pack_rows(int rows);

/* Output channels per workgroup of the weight preparation: 0 (default) by the weight's
 * size, else 8 or 32.  For measurements; no reference counterpart. */
int xdna_conv3x3_set_prep_tile(int co);

/* Both prepared forms of n weights in one launch (w[i] OIHW bf16 [cout[i]][cin[i]][3][3];
 * wt[i] / wtd[i] the forward / input-gradient forms as xdna_conv3x3_prepare_weights_both_bf16
 * writes them, either may be NULL).  The backend's fused optimizer step calls it for the
 * conv weights it has just written, so the next forward finds their forms prepared.  No
 * reference counterpart (the reference re-encodes each weight at its next forward,
 * torch_xdna_device.cpp:2208-2271). */
int xdna_conv3x3_prepare_weights_multi_bf16(int n, const uint16_t* const* w, uint16_t* const* wt,
                                            uint16_t* const* wtd, const int* cout, const int* cin, void* stream);

/* Split-K count of the rows weight gradient: 0 (default) its cost model, else this many
 * (at most one per 64-row k-tile).  For measurements; no reference counterpart. */
int xdna_conv3x3_set_wgrad_splits(int splits);
/* Output-channel tile of the rows weight gradient's direct-to-LDS form: 0 (default) by
 * layer (64 channels, four waves, for up to 64 output channels and for layers of up to 256
 * channels each side and 40 GFLOP; else 128, eight waves), or forced to 64 or 128.  For
 * measurements; no reference counterpart. */
int xdna_conv3x3_set_wgrad_tile(int co_tile);

/* No counterpart in the reference: a form of xdna_gemm_bf16 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, kernels and results, bit for bit; it calls no
 * hipMalloc, hipFree or allocating routine.  The split-K fp32 partials, the only device
 * memory the product needs beyond its operands, live in a library-owned device array of
 * XDNA_GEMM_NOALLOC_SCRATCH_BYTES per GPU, held from the first call until the process
 * ends.  A product whose partials need more returns -1 before anything is launched (use
 * xdna_gemm_bf16 for it).  All calls on one GPU share that array, which keeps the last
 * call's contents: calls that can overlap on one GPU (other streams, other threads)
 * race; calls ordered on one stream do not. */
#define XDNA_GEMM_NOALLOC_SCRATCH_BYTES (64u << 20)
int xdna_gemm_bf16_noalloc(const uint16_t* A, const uint16_t* Bm, uint16_t* C, const uint16_t* bias,
                           int batch, int M, int N, int K, int64_t lda_m, int64_t lda_k, int64_t stride_a,
                           int64_t ldb_k, int64_t ldb_n, int64_t stride_b, int64_t ldc_m, int64_t ldc_n,
                           int64_t stride_c, int bias_mode, int64_t bias_sm, int64_t bias_sn, float alpha,
                           float beta, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused Adam / AdamW: replaces torch._fused_adam_ reached through the        */
/* boxed CPU fallback (xdna_cpu_fallback, torch_xdna_device.cpp:5273-5295;    */
/* selected by _prefer_fused_optimizer, device.py:408-436).                   */
/*                                                                          */
/* One pass per element in fp32 opmath; p, m, v (and max_v) stored once in  */
/* their dtype.  dtype: 0 = fp32, 1 = bf16 (p, g, m, v share it).  step is a  */
/* device fp32 scalar per tensor (torch's state_steps, already incremented); */
/* grad_scale / found_inf are optional device fp32 scalars (NULL = absent).  */
/* mode 0 = Adam (L2 weight decay), 1 = AdamW (decoupled).                   */
/* ------------------------------------------------------------------------ */
int xdna_fused_adam(int n_tensors, void* const* params, void* const* grads,
                    void* const* exp_avgs, void* const* exp_avg_sqs,
                    void* const* max_exp_avg_sqs, const float* const* steps,
                    const int64_t* numels, int dtype, double lr, double beta1,
                    double beta2, double weight_decay, double eps, int amsgrad,
                    int maximize, int mode, const float* grad_scale,
                    const float* found_inf, void* stream);

/* The same step with lr a device scalar (lr_dtype 1 = fp32, 2 = fp64), read by the kernel
 * at its value as a double, as torch's CPU kernel reads it (lr.item<double>()): the
 * tensor-lr overloads _fused_adam_.tensor_lr / _fused_adamw_.tensor_lr, which capturable
 * optimizers with a tensor lr call.  No host read of lr, so the step can be captured in
 * a graph.  Same reference counterpart as xdna_fused_adam. */
int xdna_fused_adam_tensor_lr(int n_tensors, void* const* params, void* const* grads,
                              void* const* exp_avgs, void* const* exp_avg_sqs,
                              void* const* max_exp_avg_sqs, const float* const* steps,
                              const int64_t* numels, int dtype, const void* lr, int lr_dtype,
                              double beta1, double beta2, double weight_decay, double eps,
                              int amsgrad, int maximize, int mode, const float* grad_scale,
                              const float* found_inf, void* stream);

/* tensors[i][j] += value (fp32, computed as t + value in fp32) for every element of
 * n_tensors device tensors: torch._foreach_add_(state_steps, 1), which the optimizers
 * call before the fused Adam step (torch/optim/adam.py _fused_adam; the reference runs
 * it on the CPU through its fallback, torch_xdna_device.cpp:5124-5260).  One launch per
 * 64 tensors. */
int xdna_foreach_add_scalar_f32(int n_tensors, float* const* tensors, const int64_t* numels,
                                float value, void* stream);

/* Batch norm of convolutional activations in training mode, any channel length N*L, with
 * the running statistics updated when given: x[N][C][L] bf16, contiguous.  Replaces
 * PyTorch's CPU native_batch_norm / native_batch_norm_backward that the reference reaches
 * through its zero-copy fallback (torch_xdna_device.cpp:5124-5260) for ResNet-style
 * layers.  weight / bias: param_dtype 0 (absent), 1 bf16, 2 fp32; running_mean /
 * running_var: stat_dtype 1 bf16 or 2 fp32 (both NULL: not tracked; stat_dtype 0).  Batch
 * statistics in fp32 from per-range partials combined in a fixed order (the same bits on
 * every call): save_mean, save_invstd = 1 / sqrt(biased var + eps) (fp32 [C]); running
 * stats updated as running = (1 - momentum) * running + momentum * batch, with the
 * unbiased variance.  Backward: dx, dweight, dbias may each be NULL. */
int xdna_batch_norm_train_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                   void* running_mean, void* running_var, int stat_dtype, double momentum,
                                   double eps, uint16_t* y, float* save_mean, float* save_invstd, int64_t N,
                                   int64_t C, int64_t L, void* stream);
int xdna_batch_norm_train_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight, int param_dtype,
                                   const float* save_mean, const float* save_invstd, uint16_t* dx,
                                   void* dweight, void* dbias, int64_t N, int64_t C, int64_t L, void* stream);

/* The same batch norm with its activation fused: y = bf16(act(norm(x))) with act 1 ReLU
 * (v <= 0 -> 0) or 2 LeakyReLU (v > 0 ? v : v * slope), applied in fp32 before the one
 * rounding; act 0 is the plain norm.  The backward takes dy through the activation's
 * gradient from its output y (y <= 0 -> 0 for ReLU, y > 0 ? dy : dy * slope for LeakyReLU)
 * before the norm's sums, so no masked gradient is written.  Replaces the reference's
 * fused BatchNorm2d + ReLU / LeakyReLU region (regions.py:426-461 _BatchNormAct, its CPU
 * kernels region_kernels.cpp:346-457), with the same NaN rule in the backward (ReLU
 * passes the gradient where y is NaN, LeakyReLU scales it). */
int xdna_batch_norm_train_act_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                       void* running_mean, void* running_var, int stat_dtype, double momentum,
                                       double eps, uint16_t* y, float* save_mean, float* save_invstd, int64_t N,
                                       int64_t C, int64_t L, int act, float slope, void* stream);
int xdna_batch_norm_train_act_bwd_bf16(const uint16_t* dy, const uint16_t* x, const uint16_t* y,
                                       const void* weight, int param_dtype, const float* save_mean,
                                       const float* save_invstd, uint16_t* dx, void* dweight, void* dbias,
                                       int64_t N, int64_t C, int64_t L, int act, float slope, void* stream);

/* Batch norm in training mode without running statistics over x[N][C][L] bf16 (the form
 * PyTorch's instance_norm takes: [B, C, H, W] as [1, B*C, H*W]).  Replaces PyTorch's CPU
 * native_batch_norm / native_batch_norm_backward, which the reference reaches through
 * its zero-copy fallback (torch_xdna_device.cpp:5124-5260).  weight / bias: param_dtype
 * 0 (absent: weight 1, bias 0), 1 (bf16), 2 (fp32); save_mean / save_invstd fp32 [C];
 * invstd = 1 / sqrt(biased var + eps).  Backward: dx, dweight, dbias may each be NULL;
 * dweight / dbias are of param_dtype (1 or 2). */
int xdna_batch_norm_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                             uint16_t* y, float* save_mean, float* save_invstd, int64_t N, int64_t C,
                             int64_t L, double eps, void* stream);
int xdna_batch_norm_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight, int param_dtype,
                             const float* save_mean, const float* save_invstd, uint16_t* dx,
                             void* dweight, void* dbias, int64_t N, int64_t C, int64_t L, void* stream);

/* Instance norm over x [B][C][L] (training statistics, no running statistics): each
 * (image, channel) plane normalised on its own, y = (x - mean) * invstd * w[c] + b[c]
 * with C-element parameters (param_dtype 0 none, 1 bf16, 2 fp32); save_mean /
 * save_invstd hold B*C floats.  The backward writes dx (if not null) and, when dweight
 * and dbias are given, the parameter gradients summed over the images in a fixed order.
 * Replaces PyTorch's instance_norm composite on the device (repeat of the parameters,
 * native_batch_norm on [1, B*C, L], and the repeat's backward sums), which the reference
 * runs on its CPU through the fallback (torch_xdna_device.cpp:5124-5260). */
int xdna_instance_norm_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                uint16_t* y, float* save_mean, float* save_invstd, int64_t B, int64_t C,
                                int64_t L, double eps, void* stream);
int xdna_instance_norm_bwd_bf16(const uint16_t* dy, const uint16_t* x, const void* weight, int param_dtype,
                                const float* save_mean, const float* save_invstd, uint16_t* dx, void* dweight,
                                void* dbias, int64_t B, int64_t C, int64_t L, void* stream);

/* Instance norm with its activation fused (act and slope as for the batch norm above):
 * the reference's norm + activation region (regions.py:426-461) widened to InstanceNorm2d,
 * the norm of its style generator's blocks. */
int xdna_instance_norm_act_fwd_bf16(const uint16_t* x, const void* weight, const void* bias, int param_dtype,
                                    uint16_t* y, float* save_mean, float* save_invstd, int64_t B, int64_t C,
                                    int64_t L, double eps, int act, float slope, void* stream);
int xdna_instance_norm_act_bwd_bf16(const uint16_t* dy, const uint16_t* x, const uint16_t* y, const void* weight,
                                    int param_dtype, const float* save_mean, const float* save_invstd,
                                    uint16_t* dx, void* dweight, void* dbias, int64_t B, int64_t C, int64_t L,
                                    int act, float slope, void* stream);

/* Nearest-neighbour upsampling by exactly 2 of `planes` NCHW bf16 planes of H x W (the
 * input size): y[p][oy][ox] = x[p][oy/2][ox/2] into 2H x 2W planes; the backward writes
 * dx[p][iy][ix] = bf16(fp32 sum of the 2x2 block of dy, row-major order).  Buffers
 * 4-byte aligned.  Replaces upsample_nearest2d(_backward) through the zero-copy CPU
 * fallback (torch_xdna_device.cpp:5124-5260). */
int xdna_upsample_nearest2x_bf16(const uint16_t* x, uint16_t* y, int64_t planes, int H, int W, void* stream);
int xdna_upsample_nearest2x_bwd_bf16(const uint16_t* dy, uint16_t* dx, int64_t planes, int H, int W,
                                     void* stream);

/* Stride-2 sampling of `planes` NCHW bf16 planes whose full size is H x W: subsample2
 * writes y[p][oy][ox] = full[p][2oy][2ox] into ceil(H/2) x ceil(W/2) planes; dilate2
 * writes full[p][y][x] = dy[p][y/2][x/2] at even (y, x) and 0 elsewhere.  A 3x3 / stride-2
 * / pad-1 conv is the stride-1 conv subsampled this way, and its input and weight
 * gradients are the stride-1 ones of the dilated gradient.  No reference counterpart (the
 * reference runs strided convs on its CPU through the fallback, torch_xdna_device.cpp:
 * 4524-4606, 4608-4885). */
int xdna_subsample2_bf16(const uint16_t* full, uint16_t* y, int64_t planes, int H, int W, void* stream);
int xdna_dilate2_bf16(const uint16_t* dy, uint16_t* full, int64_t planes, int H, int W, void* stream);

/* The same conv without the sampling passes (the backend's path for 3x3 / stride-2 /
 * pad-1 convs; the reference runs them on its CPU, torch_xdna_device.cpp:4524-4606,
 * 4608-4885):
 * xdna_conv3x3_layout_rows_stride2_bf16: xdna_conv3x3_layout_rows_bf16 of the input
 * packed at its full H x W, storing only the outputs at even (y, x), at (y/2, x/2) of a
 * [B][cout][ceil(H/2)][ceil(W/2)] tensor.
 * xdna_conv3x3_layout_pack_dilate2_bf16: xdna_conv3x3_layout_pack_bf16 of the H x W
 * spread of src ([B][C][ceil(H/2)][ceil(W/2)]: src at even (y, x), 0 elsewhere), without
 * materializing the spread; the input- and weight-gradient convs of the stride-2 conv read
 * this packed gradient.  W <= 256. */
int xdna_conv3x3_layout_rows_stride2_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                          int B, int cin, int cout, int H, int W, int layout, void* stream);
int xdna_conv3x3_layout_pack_dilate2_bf16(const uint16_t* src, uint16_t* dst, int B, int C, int H, int W,
                                          int layout, void* stream);

/* The pack and the conv in one launch for small grids (the reference's pack_input,
 * conv_pack.cpp:632-700, followed by its conv run, torch_xdna_device.cpp:2317-2483, which
 * this pair replaces where no packed copy of the input is needed afterwards):
 * xdna_conv3x3_nchw_act_bf16 is xdna_conv3x3_layout_rows_act_bf16 (s2out = 0) or
 * xdna_conv3x3_layout_rows_stride2_bf16 (s2out = 1, act 0) of the input packed, with the
 * window gathered from the NCHW input x [B][cin][H][W] by the small-grid kernel itself:
 * the same bits as the packed path.  Only where xdna_conv3x3_nchw_small_eligible is 1
 * (W <= 36, cin % 8 == 0, input under 2 GiB, and a grid the small-grid kernel takes);
 * otherwise -1 with an error.  wt is the prepared form of either direction (input gradient:
 * x is dY and cin its channels). */
int xdna_conv3x3_nchw_small_eligible(int B, int cin, int cout, int H, int W);
int xdna_conv3x3_nchw_act_bf16(const uint16_t* x, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int B,
                               int cin, int cout, int H, int W, int act, int s2out, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused training regions: the frozen-feature (perceptual) loss of          */
/* xdna_train/regions.py:1-425 with its host kernels                        */
/* (_native/region_kernels.cpp:51-340) on device memory.  bf16 storage,     */
/* fp32 arithmetic, one rounding per output.  `go` is the loss gradient     */
/* autograd hands in, read on the device: go_dtype 0 none (1), 1 fp32 *,    */
/* 2 bf16 *.                                                                 */
/* ------------------------------------------------------------------------ */

/* xdna_conv3x3_layout_rows_bf16 with an activation in the epilogue, applied to the fp32
 * sum before its rounding: act 0 none, 1 ReLU (PyTorch's: NaN kept, -0 to +0; the result
 * equals relu of the unfused conv output bit for bit).  Replaces the reference region's
 * conv followed by region_relu (regions.py:203-236, region_kernels.cpp:74-92). */
int xdna_conv3x3_layout_rows_act_bf16(const uint16_t* xp, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                      int B, int cin, int cout, int H, int W, int layout, int act, void* stream);

/* 2x2 / stride-2 max-pool of `planes` H x W bf16 planes into floor(H/2) x floor(W/2):
 * PyTorch's rule (the first maximum in row-major window order; a NaN replaces any value).
 * Replaces the pooling half of xdna_region_relu_maxpool2_bf16 (region_kernels.cpp:
 * 149-185), whose ReLU is in the conv epilogue here. */
int xdna_region_maxpool2_bf16(const uint16_t* x, uint16_t* y, int64_t planes, int H, int W, void* stream);

/* Backward of ReLU, max-pool and tap terms in one pass over `planes` H x W planes:
 *   out = (r && r <= 0) ? 0 : bf16(base + extra + scale * go * (ta - tb))
 * base = g, or gp (the gradient of the pooled floor(H/2) x floor(W/2) planes) routed to each
 * window's maximum of px (the pool input; the forward's rule), 0 elsewhere; r, g, gp,
 * extra and ta/tb may each be NULL (g and gp not both).  Replaces region_relu_bwd,
 * region_addtap and region_maxpool2_bwd (region_kernels.cpp:187-340). */
int xdna_region_backward_bf16(const uint16_t* r, const uint16_t* g, const uint16_t* gp, const uint16_t* px,
                              const uint16_t* extra, const uint16_t* ta, const uint16_t* tb, float scale,
                              const void* go, int go_dtype, uint16_t* out, int64_t planes, int H, int W,
                              void* stream);

/* Partial sums per loss term: each call writes xdna_region_loss_parts() floats,
 * scale * (sums of the squared differences over a fixed partition of the elements);
 * xdna_region_loss_finish adds n partials in a fixed order (fp64) into the loss, as an fp32
 * and/or bf16 scalar.  sqdiff: d = a - b (bf16).  gram_sqdiff: d = G / chw - t for bf16
 * Gram matrices G [batch][cc] and fp32 targets t (batch stride t_bstride, 0 to broadcast
 * one).  Replace region_sqdiff_sum (region_kernels.cpp:51-72) without its host
 * round trip. */
int xdna_region_loss_parts(void);
int xdna_region_sqdiff_bf16(const uint16_t* a, const uint16_t* b, int64_t n, float scale, float* part,
                            void* stream);
int xdna_region_gram_sqdiff_bf16(const uint16_t* G, const float* t, int64_t t_bstride, int64_t batch, int64_t cc,
                                 float chw, float scale, float* part, void* stream);
int xdna_region_loss_finish(const float* part, int n, float* out_f32, uint16_t* out_bf16, void* stream);

/* S = bf16(coef * go * (d + d^T) / chw), d = G / chw - t, for batch C x C Gram matrices
 * G = F F^T: the gradient of coef / 2 * sum d^2 with respect to the features F is S F
 * (coef = 2 w / N for w times a mean over N elements).  No reference counterpart (the
 * reference's region has feature taps only). */
int xdna_region_gram_grad_bf16(const uint16_t* G, const float* t, int64_t t_bstride, int64_t batch, int C,
                               float chw, float coef, const void* go, int go_dtype, uint16_t* S, void* stream);

/* ------------------------------------------------------------------------ */
/* Losses of plain training scripts.  The reference runs them on its CPU    */
/* through the zero-copy fallback (torch_xdna_device.cpp:5124-5260).        */
/* dtype / go_dtype: 1 fp32, 2 bf16.  b's element for a's element i is      */
/* b[i % period] (period == n: same shape; a divisor of n: b broadcast over */
/* leading dimensions, as target.expand_as(input)).  reduction: 1 mean,     */
/* 2 sum (PyTorch's enum; 0 none is not served).                            */
/* ------------------------------------------------------------------------ */

/* mse_loss(a, b): the mean (or sum) of (a - b)^2 over n elements into the 0-dim `out` of
 * the operands' dtype.  fp32 partial sums over a fixed partition of the elements, then one
 * workgroup adds them in index order in fp64, so equal inputs give equal bits.  The
 * workspace holds the partials (xdna_mse_loss_workspace_bytes(n)).  Replaces PyTorch's mse_loss
 * (aten::mse_loss, reduced) reached through the fallback. */
size_t xdna_mse_loss_workspace_bytes(int64_t n);
int xdna_mse_loss(const void* a, const void* b, int dtype, int64_t n, int64_t period, int reduction, void* out,
                  void* workspace, size_t workspace_bytes, void* stream);

/* mse_loss_backward: grad[i] = norm * (a[i] - b[i % period]) * go, norm = 2 / n (mean) or
 * 2 (sum), go the incoming gradient (a device scalar of go_dtype), every element of grad
 * written (no fill).  Replaces aten::mse_loss_backward reached through the fallback. */
int xdna_mse_loss_bwd(const void* go, int go_dtype, const void* a, const void* b, int dtype, int64_t n,
                      int64_t period, int reduction, void* grad, void* stream);

/* Column sums of a row-major [R][N] bf16 matrix, out[n] = bf16(fp32 sum over rows), in a
 * fixed order (row slices summed in order, then the slices in order: equal inputs give equal
 * bits).  The bias gradient of a Linear layer (aten::sum over dim 0 of addmm's output
 * gradient), which the reference reaches through its zero-copy CPU fallback
 * (torch_xdna_device.cpp:5124-5260).  The workspace (16-byte aligned) holds the fp32 row
 * slices' partial sums; 0 bytes when one slice suffices. */
size_t xdna_colsum_workspace_bytes(const uint16_t* x, int64_t R, int64_t N);
int xdna_colsum_bf16(const uint16_t* x, uint16_t* out, int64_t R, int64_t N, void* workspace,
                     size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XDNA_HIP_H */
