// Shared declarations of the PrivateUse1 "xdna" backend over HIP device memory.
//
// Layer map (reference torch_xdna_device.cpp): device memory, guard and hooks
// (:131-1318) are device.cpp; the hot operators (:1814-2771, 3740-3790, 4360-4885)
// are ops.cpp; every kernel is reached through the C ABI of include/xdna_hip.h.
#pragma once

#include <ATen/ATen.h>
#include <c10/core/Allocator.h>
#include <torch/library.h>

#include <atomic>
#include <cstdint>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "xdna_hip.h"

namespace xdna_backend {

constexpr c10::DeviceType kXdna = c10::DeviceType::PrivateUse1;

// HIP stream all backend work is ordered on: the current stream of device 0, the same
// one PyTorch-ROCm kernels launched by the fallback use.
void* current_stream();

// Throws c10::Error with the C ABI's last error when rc != 0.
void check_abi(int rc, const char* what);

c10::Allocator* xdna_allocator();

// A new xdna tensor (contiguous).
at::Tensor empty_xdna(at::IntArrayRef size, at::ScalarType dtype,
                      c10::MemoryFormat fmt = c10::MemoryFormat::Contiguous);

// A ROCm ("cuda") tensor aliasing the memory of an xdna tensor (same sizes, strides,
// offset); its storage keeps the xdna storage alive.
at::Tensor cuda_alias(const at::Tensor& t);
// An xdna tensor sharing the memory of a ROCm tensor (its storage keeps the ROCm
// storage alive); the inverse of cuda_alias when t's storage is an alias.
at::Tensor xdna_from_cuda(const at::Tensor& t);

// 0: every op through the generic ROCm fallback; 1: HIP hot path without the HIP weight
// gradient; 2: all HIP paths (default).  Mirrors the reference's npu mode
// (xdna_train/device.py:526-650).
extern std::atomic<int> g_mode;
extern std::atomic<int> g_gconv_mode;
// 3x3 weight gradient: 0 (default) and 2 the rows form, 1 the channel-major form.
extern std::atomic<int> g_wgrad_form;
// 1: captured 3x3 backwards run the rows weight gradient beside the input gradient (opt-in)
extern std::atomic<int> g_wgrad_overlap;
// Row layout of the 3x3 conv operands: 1 (default) tight strips, 0 the reference's layout.
extern std::atomic<int> g_conv_layout;
// 1: the 3x3 / stride-1 forward and input-gradient convs emulate the reference NPU's BFP16
// arithmetic (XDNA_BFP16_EMULATION=1 or set_bfp16_emulation); 0 (default) bf16 x bf16 with
// fp32 sums, the reference's CPU path.
extern std::atomic<int> g_bfp16_emul;

// Write epochs of device allocations (the reference's per-allocation write epoch,
// torch_xdna_device.cpp:493, 576, 620-633, 2222).  Every xdna write path bumps the epoch
// of the allocation it writes: hot-op out= arguments, the arguments the boxed fallback
// writes, copies, resize_ and set_, the fused optimizer steps.  Unlike the version
// counter, this also sees writes through `.data` aliases.  Caches of derived device
// buffers (prepared weights, kept packs) key on it.  Writes made by replaying a captured
// graph run no host code and bump nothing.
uint64_t write_epoch(const at::Tensor& t);
void bump_write_epoch(const at::Tensor& t);

// Tag of the capture the calling thread is in: 0 when the current stream is not
// capturing, else the private pool the captured allocations come from (-1 without one).
// Host caches of device buffers serve only entries made under the same tag, so a graph
// never reads a buffer it does not own.
int64_t capture_tag();

// Per-path counters (the reference's ScopedMappedCpu, torch_xdna_device.cpp:1470-1521).
void count_call(const char* name, int64_t ns);

struct ScopedCount {
  const char* name;
  int64_t t0;
  explicit ScopedCount(const char* n);
  ~ScopedCount();
};

// Hot-path registrations (ops.cpp).
void register_hot_ops(torch::Library& m);
// Autograd-level overrides for the backend (ops.cpp): instance_norm.
void register_autograd_ops(torch::Library& m);

// Drops the cached prepared weight forms (ops.cpp).
void clear_weight_cache();
// A captured graph was replayed: host caches of forms derived from tensors it may have
// written (prepared weights, kept packs) stop serving their older entries (ops.cpp).
void note_graph_replay();
// Drops the packed conv inputs kept for weight gradients (ops.cpp).
void clear_packed_inputs();
// Frozen weights' prepared forms adopted by the captured graph of allocator pool `pool`:
// prepare again those whose weight was written since (before a replay; returns how many),
// or forget them (when the graph is released) (ops.cpp).
int64_t refresh_graph_weights(int64_t pool);
void release_graph_weights(int64_t pool);
// Entries of the prepared-weight and kept-pack caches made under capture tag `tag` (all
// entries for tag < 0): {weights, weight bytes, packs, pack bytes} (ops.cpp).
std::vector<int64_t> cache_stats(int64_t tag);

// Weight-gradient launches so far (ops.cpp).
int64_t dw_jobs();

// Pieces of the fused training regions (ops.cpp): a 3x3 conv with its activation in the
// epilogue (act 0 none, 1 ReLU) and a batched product scaled by alpha.
at::Tensor region_conv3x3(const at::Tensor& x, const at::Tensor& w, const std::optional<at::Tensor>& b, int act);
at::Tensor region_bmm(const at::Tensor& a, const at::Tensor& b, double alpha);
// Training batch / instance norm with a ReLU or LeakyReLU applied before the output's
// rounding, and its backward through the activation's mask (ops.cpp).
std::tuple<at::Tensor, at::Tensor, at::Tensor> region_norm_act_fwd(
    const at::Tensor& x, const at::Tensor& weight, const at::Tensor& bias, const std::optional<at::Tensor>& rm,
    const std::optional<at::Tensor>& rv, double momentum, double eps, int act, double slope, bool instance);
std::tuple<at::Tensor, at::Tensor, at::Tensor> region_norm_act_bwd(
    const at::Tensor& grad, const at::Tensor& x, const at::Tensor& y, const at::Tensor& weight,
    const at::Tensor& mean, const at::Tensor& invstd, int act, double slope, bool instance, bool need_x,
    bool need_params);
// Region kernels on tensors (regions.cpp).
at::Tensor region_maxpool2(const at::Tensor& x);
at::Tensor region_backward(const std::optional<at::Tensor>& r, const std::optional<at::Tensor>& g,
                           const std::optional<at::Tensor>& gp, const std::optional<at::Tensor>& px,
                           const std::optional<at::Tensor>& extra, const std::optional<at::Tensor>& ta,
                           const std::optional<at::Tensor>& tb, double scale, const std::optional<at::Tensor>& go,
                           at::IntArrayRef shape);
int64_t region_loss_parts();
void region_sqdiff(const at::Tensor& a, const at::Tensor& b, double scale, at::Tensor& part, int64_t offset);
void region_gram_sqdiff(const at::Tensor& G, const at::Tensor& t, double chw, double scale, at::Tensor& part,
                        int64_t offset);
std::tuple<at::Tensor, at::Tensor> region_loss_finish(const at::Tensor& part);
at::Tensor region_gram_grad(const at::Tensor& G, const at::Tensor& t, double chw, double coef,
                            const std::optional<at::Tensor>& go);

// Live kernel timing: HIP events around hot-kernel launches on the launch stream,
// with the algorithmic work (FLOP or bytes) of each launch.
struct KernelTimer {
  const char* name;
  double work;
  void* start = nullptr;
  void* stop = nullptr;
  KernelTimer(const char* n, double w);
  ~KernelTimer();
};
void kernel_timing_enable(bool on);
// name -> (launches, total ms, total work); synchronizes the device.
std::vector<std::tuple<std::string, int64_t, double, double>> kernel_timing_report();

}  // namespace xdna_backend
