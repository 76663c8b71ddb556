// Hot-path operators of the xdna backend: 3x3 conv forward / backward, mm / addmm /
// bmm, fused Adam / AdamW.  Every kernel runs through the C ABI (include/xdna_hip.h)
// on PyTorch-ROCm's current HIP stream; shapes outside the hot path go to the generic
// fallback (PyTorch-ROCm kernels on aliases), as the reference sends them to its CPU
// kernels (torch_xdna_device.cpp:4524-4606, 4608-4885, 4360-4417, 3740-3790).
#include "xdna.h"

#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/_fused_adam_native.h>
#include <ATen/ops/instance_norm_native.h>
#include <ATen/ops/max_pool2d_native.h>
#include <torch/csrc/autograd/custom_function.h>
#include <c10/core/impl/LocalDispatchKeySet.h>

#include <algorithm>
#include <array>
#include <deque>
#include <mutex>
#include <optional>
#include <unordered_map>
#include <vector>

namespace xdna_backend {
namespace {

at::Tensor rocm(const at::Tensor& t) {
  return t.defined() && t.device().type() == kXdna ? cuda_alias(t) : t;
}
std::optional<at::Tensor> rocm(const std::optional<at::Tensor>& t) {
  if (!t || !t->defined()) return t;
  return rocm(*t);
}
at::Tensor back(const at::Tensor& t) { return t.defined() && t.is_cuda() ? xdna_from_cuda(t) : t; }

// Dispatch below autograd: the aliases never carry autograd state.
struct BelowAutograd {
  at::AutoDispatchBelowADInplaceOrView guard;
};

at::Tensor alloc_bytes(size_t n) {
  return empty_xdna({int64_t(std::max<size_t>(n, 1))}, at::kByte);
}

// ---------------------------------------------------------------------------------------
// 3x3 conv
// ---------------------------------------------------------------------------------------
bool is_one(c10::SymIntArrayRef v, int64_t x) {
  return v.size() == 2 && v[0] == x && v[1] == x;
}

// The reference's eligibility gate (XdnaConv3x3wRuntime::plan, torch_xdna_device.cpp:
// 2112-2157): bf16, 4-D, 3x3, stride 1, pad 1, dilation 1, groups 1, not transposed.
bool conv_eligible(const at::Tensor& x, const at::Tensor& w, c10::SymIntArrayRef stride,
                   c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation, bool transposed,
                   c10::SymIntArrayRef output_padding, const c10::SymInt& groups) {
  if (g_mode.load() < 1) return false;
  if (x.scalar_type() != at::kBFloat16 || w.scalar_type() != at::kBFloat16) return false;
  if (x.dim() != 4 || w.dim() != 4 || w.size(2) != 3 || w.size(3) != 3) return false;
  if (!is_one(stride, 1) || !is_one(padding, 1) || !is_one(dilation, 1) || transposed) return false;
  if (!is_one(output_padding, 0) || groups != 1) return false;
  if (x.size(0) < 1 || x.size(2) < 1 || x.size(3) < 1 || w.size(0) < 1 || w.size(1) < 1) return false;
  if (x.device().type() != kXdna || w.device().type() != kXdna) return false;
  return true;
}

// 3x3 / stride-2 / pad-1 convs (the style encoder, ResNet's downsampling blocks) run
// through the stride-1 kernels: the forward is the stride-1 conv at every other row and
// column, and both gradients are the stride-1 ones of the gradient spread onto the
// stride-1 grid with zeros (which add nothing to any sum), so the numerics are those of
// the hot path.  4x the MACs of the strided conv, on kernels several times faster than
// MIOpen's on these shapes, and within the conv bar where MIOpen is not.  The reference
// runs them on its CPU through the fallback (torch_xdna_device.cpp:4524-4606, 4608-4885).
// XDNA_CONV_S2=0 sends 3x3 / stride-2 convs to the general kernels instead (their real
// MACs on the gather GEMM), for measurements.
const bool g_conv_s2 = [] {
  const char* e = std::getenv("XDNA_CONV_S2");
  return !(e && std::atoi(e) == 0);
}();

bool conv_s2_eligible(const at::Tensor& x, const at::Tensor& w, c10::SymIntArrayRef stride,
                      c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation, bool transposed,
                      c10::SymIntArrayRef output_padding, const c10::SymInt& groups) {
  if (g_mode.load() < 1 || !g_conv_s2) return false;
  if (x.scalar_type() != at::kBFloat16 || w.scalar_type() != at::kBFloat16) return false;
  if (x.dim() != 4 || w.dim() != 4 || w.size(2) != 3 || w.size(3) != 3) return false;
  if (!is_one(stride, 2) || !is_one(padding, 1) || !is_one(dilation, 1) || transposed) return false;
  if (!is_one(output_padding, 0) || groups != 1) return false;
  if (x.size(0) < 1 || x.size(2) < 1 || x.size(3) < 1 || w.size(0) < 1 || w.size(1) < 1) return false;
  if (x.size(1) != w.size(1)) return false;
  return x.device().type() == kXdna && w.device().type() == kXdna;
}

// Prepared weight forms (forward and input-gradient), keyed by storage, data address,
// offset, shape, strides, version, write epoch, graph-replay generation and direction
// (strides: two views of one storage with the same offset and shape, such as w and
// w.transpose(2, 3), are different weights with one version counter and epoch): the role
// of the reference's weight slots (torch_xdna_device.cpp:2208-2271, keyed on the data
// pointer, version and write epoch).  A weak reference to the storage tells a live tensor
// from a new one at a recycled address; in-place writes through autograd bump the
// version, and every xdna write path (`.data` writes and the fused optimizer steps
// included) bumps the write epoch.  The one writer no host code sees is the replay of a
// captured graph (an optimizer step inside it), so every replay starts a new generation
// and older entries are not served.  Entries carry the capture tag they were made under
// and serve only the same tag: inside a capture the forms are prepared by the graph
// itself, which owns them and sees writes made between replays.
struct PreparedWeights {
  c10::weak_intrusive_ptr<c10::StorageImpl> storage{c10::intrusive_ptr<c10::StorageImpl>()};
  const void* data = nullptr;
  int64_t offset = 0, version = 0, tag = 0;
  uint64_t epoch = 0, generation = 0;
  std::array<int64_t, 4> sizes{}, strides{};
  bool dgrad = false;
  at::Tensor wt;
  uint64_t last_use = 0;
};

struct WeightCache {
  std::mutex mu;
  std::vector<PreparedWeights> entries;
  uint64_t tick = 0;
  size_t bytes = 0;
  static constexpr size_t kMaxEntries = 1024;
  static constexpr size_t kMaxBytes = size_t(4) << 30;
};

std::atomic<uint64_t> g_replay_generation{0};

WeightCache& weight_cache() {
  static auto* c = new WeightCache();
  return *c;
}

}  // namespace

void clear_weight_cache() {
  WeightCache& c = weight_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  c.entries.clear();
  c.bytes = 0;
}

void note_graph_replay() { g_replay_generation.fetch_add(1); }

// Prepared forms that a captured graph reads without preparing them itself.  A capture
// that meets a weight whose form the eager cache holds adopts that form instead of
// recording a preparation: the graph keeps the form (and the weight) alive, and every
// replay first prepares it again, eagerly and on the replay's stream, if the weight was
// written since (version or write epoch), so a replay computes with the weight's current
// value as an eager step would.  Writes the graph itself makes are not seen by host code:
//  * a frozen weight is not written by its graph;
//  * a trainable weight is written by the optimizer step, and where that step is part of
//    the same capture (the fused optimizer's refresh_conv_forms under the capture's tag),
//    the graph records one preparation of every adopted form it wrote right after the
//    step, so each replay leaves the forms of the weights it produced for the next one;
//  * a trainable weight whose adopted forms no captured step refreshes is prepared again
//    before every replay (one launch for all of them).
// The eager cache serves a trainable weight's forms only after the fused optimizer step
// refreshed them (refresh_conv_forms), which an eager warm-up step before the capture does.
namespace {
struct GraphWeight {
  at::Tensor weight, wt;
  bool dgrad = false;
  bool trainable = false;
  bool graph_refreshed = false;  // a captured optimizer step prepares it again after writing
  int64_t version = 0;
  uint64_t epoch = 0;
};

struct GraphWeights {
  std::mutex mu;
  std::unordered_map<int64_t, std::vector<GraphWeight>> by_pool;
};

GraphWeights& graph_weights() {
  static auto* g = new GraphWeights();
  return *g;
}

int64_t weight_version(const at::Tensor& w) {
  return int64_t(w.unsafeGetTensorImpl()->version_counter().current_version());
}

void adopt_graph_weight(int64_t pool, const at::Tensor& w, bool dgrad, const at::Tensor& wt, bool trainable) {
  GraphWeight e;
  e.weight = w;
  e.wt = wt;
  e.dgrad = dgrad;
  e.trainable = trainable;
  e.version = weight_version(w);
  e.epoch = write_epoch(w);
  GraphWeights& g = graph_weights();
  std::lock_guard<std::mutex> lock(g.mu);
  g.by_pool[pool].push_back(std::move(e));
}
}  // namespace

int64_t refresh_graph_weights(int64_t pool) {
  GraphWeights& g = graph_weights();
  std::lock_guard<std::mutex> lock(g.mu);
  auto it = g.by_pool.find(pool);
  if (it == g.by_pool.end()) return 0;
  // every stale form, both forms of one contiguous weight as one job of a single launch
  std::vector<at::Tensor> keep;
  std::vector<const uint16_t*> w;
  std::vector<uint16_t*> wt, wtd;
  std::vector<int> co, ci;
  int64_t n = 0;
  for (GraphWeight& e : it->second) {
    const int64_t ver = weight_version(e.weight);
    const uint64_t ep = write_epoch(e.weight);
    if (ver == e.version && ep == e.epoch && !(e.trainable && !e.graph_refreshed)) continue;
    e.version = ver;
    e.epoch = ep;
    ++n;
    at::Tensor wc = e.weight.contiguous();
    const uint16_t* src = static_cast<const uint16_t*>(wc.const_data_ptr());
    size_t j = 0;
    while (j < w.size() && w[j] != src) ++j;
    if (j == w.size()) {
      keep.push_back(wc);
      w.push_back(src);
      wt.push_back(nullptr);
      wtd.push_back(nullptr);
      co.push_back(int(wc.size(0)));
      ci.push_back(int(wc.size(1)));
    }
    (e.dgrad ? wtd : wt)[j] = static_cast<uint16_t*>(e.wt.data_ptr());
  }
  if (!w.empty())
    check_abi(xdna_conv3x3_prepare_weights_multi_bf16(int(w.size()), w.data(), wt.data(), wtd.data(), co.data(),
                                                      ci.data(), current_stream()),
              "graph weight refresh");
  if (n) count_call("hip_conv3x3.weights_graph_refresh", 0);
  return n;
}

namespace {
// Inside a capture: the adopted forms of the weights a captured optimizer step has just
// written, prepared again by one launch recorded right after the step.
void refresh_captured_forms(int64_t pool, at::TensorList params) {
  GraphWeights& g = graph_weights();
  std::lock_guard<std::mutex> lock(g.mu);
  auto it = g.by_pool.find(pool);
  if (it == g.by_pool.end()) return;
  std::vector<const uint16_t*> w;
  std::vector<uint16_t*> wt, wtd;
  std::vector<int> co, ci;
  std::vector<GraphWeight*> hit;
  for (const auto& p : params) {
    if (!p.defined() || p.dim() != 4 || !p.is_contiguous()) continue;
    std::array<GraphWeight*, 2> fd{nullptr, nullptr};
    for (GraphWeight& e : it->second)
      if (e.trainable && e.weight.const_data_ptr() == p.const_data_ptr() && e.weight.sizes() == p.sizes() &&
          e.weight.strides() == p.strides())
        fd[e.dgrad ? 1 : 0] = &e;
    if (!fd[0] && !fd[1]) continue;
    w.push_back(static_cast<const uint16_t*>(p.const_data_ptr()));
    wt.push_back(fd[0] ? static_cast<uint16_t*>(fd[0]->wt.data_ptr()) : nullptr);
    wtd.push_back(fd[1] ? static_cast<uint16_t*>(fd[1]->wt.data_ptr()) : nullptr);
    co.push_back(int(p.size(0)));
    ci.push_back(int(p.size(1)));
    for (GraphWeight* e : fd)
      if (e) hit.push_back(e);
  }
  if (w.empty()) return;
  check_abi(xdna_conv3x3_prepare_weights_multi_bf16(int(w.size()), w.data(), wt.data(), wtd.data(), co.data(),
                                                    ci.data(), current_stream()),
            "conv weights (captured optimizer step)");
  for (GraphWeight* e : hit) e->graph_refreshed = true;
  count_call("hip_conv3x3.weights_graph_step_refresh", 0);
}
}  // namespace

void purge_capture_entries(int64_t tag);

// Drops everything kept for a captured graph's pool: its adopted frozen weights and the
// prepared weights and kept packs made under its capture tag (never served again, since
// tags are unique pool ids, but holding their device memory until evicted).
void release_graph_weights(int64_t pool) {
  {
    GraphWeights& g = graph_weights();
    std::lock_guard<std::mutex> lock(g.mu);
    g.by_pool.erase(pool);
  }
  if (pool != 0) purge_capture_entries(pool);
}

namespace {

bool weight_cacheable(const at::Tensor& w) { return !w.is_inference() && w.dim() == 4; }

std::array<int64_t, 4> sizes4(const at::Tensor& w) { return {w.size(0), w.size(1), w.size(2), w.size(3)}; }
std::array<int64_t, 4> strides4(const at::Tensor& w) {
  return {w.stride(0), w.stride(1), w.stride(2), w.stride(3)};
}

bool same_weight(const PreparedWeights& e, const at::Tensor& w, bool dgrad, int64_t tag) {
  return e.dgrad == dgrad && e.tag == tag && e.offset == w.storage_offset() && e.data == w.storage().data() &&
         e.sizes == sizes4(w) && e.strides == strides4(w);
}

// The version of an entry that the optimizer step refreshed (refresh_conv_forms): its
// epoch, which every xdna write advances, and its generation decide; the version counter
// moves after the step returns.
constexpr int64_t kAnyVersion = -1;

at::Tensor cached_weights(const at::Tensor& w, bool dgrad, int64_t tag) {
  const uint64_t epoch = write_epoch(w);
  WeightCache& c = weight_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const int64_t ver = int64_t(w.unsafeGetTensorImpl()->version_counter().current_version());
  const uint64_t gen = g_replay_generation.load();
  for (auto& e : c.entries) {
    if (!same_weight(e, w, dgrad, tag) || (e.version != ver && e.version != kAnyVersion) || e.epoch != epoch ||
        e.generation != gen)
      continue;
    auto live = e.storage.lock();
    if (!live || live.get() != w.storage().unsafeGetStorageImpl()) continue;
    e.last_use = ++c.tick;
    return e.wt;
  }
  return at::Tensor();
}

void remember_weights(const at::Tensor& w, bool dgrad, const at::Tensor& wt, int64_t tag) {
  const uint64_t epoch = write_epoch(w);
  WeightCache& c = weight_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const uint64_t gen = g_replay_generation.load();
  // drop entries of dead storages and older generations, and any entry for the same
  // tensor, direction and tag (an older version or epoch)
  const auto stale = [&](const PreparedWeights& e) {
    if (e.storage.expired() || (e.tag == 0 && e.generation != gen)) return true;
    auto live = e.storage.lock();
    return same_weight(e, w, dgrad, tag) && live && live.get() == w.storage().unsafeGetStorageImpl();
  };
  for (auto it = c.entries.begin(); it != c.entries.end();) {
    if (stale(*it)) {
      c.bytes -= size_t(it->wt.nbytes());
      it = c.entries.erase(it);
    } else {
      ++it;
    }
  }
  // then the least recently used ones while over the caps
  while (!c.entries.empty() && (c.entries.size() >= WeightCache::kMaxEntries ||
                                c.bytes + size_t(wt.nbytes()) > WeightCache::kMaxBytes)) {
    auto lru = std::min_element(c.entries.begin(), c.entries.end(),
                                [](const auto& a, const auto& b) { return a.last_use < b.last_use; });
    c.bytes -= size_t(lru->wt.nbytes());
    c.entries.erase(lru);
  }
  PreparedWeights e;
  e.storage = c10::weak_intrusive_ptr<c10::StorageImpl>(w.storage().getWeakStorageImpl());
  e.data = w.storage().data();
  e.offset = w.storage_offset();
  e.version = int64_t(w.unsafeGetTensorImpl()->version_counter().current_version());
  e.epoch = epoch;
  e.generation = gen;
  e.tag = tag;
  e.sizes = sizes4(w);
  e.strides = strides4(w);
  e.dgrad = dgrad;
  e.wt = wt;
  e.last_use = ++c.tick;
  c.bytes += size_t(wt.nbytes());
  c.entries.push_back(std::move(e));
}

// After a fused optimizer step outside graph capture: the conv weights it has just written
// that have eager prepared forms get them made again, all in one launch, into the same
// buffers (stream-ordered after every earlier read of them), and their entries take the
// new epoch; the next forward and input gradient find them instead of preparing each
// weight in a launch of its own.  XDNA_ADAM_PREP=0 turns it off.  Captured steps keep
// preparing in the graph (a replay writes the weights with no host code).
std::atomic<int> g_adam_prep{[] {
  const char* e = std::getenv("XDNA_ADAM_PREP");
  return e && std::atoi(e) == 0 ? 0 : 1;
}()};

void refresh_conv_forms(at::TensorList params) {
  if (!g_adam_prep.load()) return;
  if (const int64_t tag = capture_tag(); tag != 0) {
    refresh_captured_forms(tag, params);
    return;
  }
  WeightCache& c = weight_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const uint64_t gen = g_replay_generation.load();
  std::vector<const uint16_t*> w;
  std::vector<uint16_t*> wt, wtd;
  std::vector<int> co, ci;
  std::vector<std::array<PreparedWeights*, 2>> ent;
  std::vector<uint64_t> epochs;
  for (const auto& p : params) {
    if (!p.defined() || p.scalar_type() != at::kBFloat16 || p.dim() != 4 || p.size(2) != 3 || p.size(3) != 3 ||
        !p.is_contiguous())
      continue;
    std::array<PreparedWeights*, 2> fd{nullptr, nullptr};
    for (auto& e : c.entries) {
      if (!same_weight(e, p, e.dgrad, 0)) continue;  // eager entries of this tensor, either direction
      auto live = e.storage.lock();
      if (!live || live.get() != p.storage().unsafeGetStorageImpl()) continue;
      fd[e.dgrad ? 1 : 0] = &e;
    }
    if (!fd[0] && !fd[1]) continue;
    w.push_back(static_cast<const uint16_t*>(p.const_data_ptr()));
    wt.push_back(fd[0] ? static_cast<uint16_t*>(fd[0]->wt.data_ptr()) : nullptr);
    wtd.push_back(fd[1] ? static_cast<uint16_t*>(fd[1]->wt.data_ptr()) : nullptr);
    co.push_back(int(p.size(0)));
    ci.push_back(int(p.size(1)));
    ent.push_back(fd);
    epochs.push_back(write_epoch(p));
  }
  if (w.empty()) return;
  double bytes = 0.0;
  for (size_t i = 0; i < w.size(); ++i)
    bytes += double(co[i]) * ci[i] * 9.0 * 2.0 * (1.0 + (wt[i] ? 1.0 : 0.0) + (wtd[i] ? 1.0 : 0.0));
  {
    KernelTimer kt("conv3x3_prep", bytes);
    check_abi(xdna_conv3x3_prepare_weights_multi_bf16(int(w.size()), w.data(), wt.data(), wtd.data(), co.data(),
                                                      ci.data(), current_stream()),
              "conv weights (optimizer step)");
  }
  for (size_t i = 0; i < ent.size(); ++i) {
    for (PreparedWeights* e : ent[i]) {
      if (!e) continue;
      e->version = kAnyVersion;
      e->epoch = epochs[i];
      e->generation = gen;
      e->last_use = ++c.tick;
    }
    count_call("hip_conv3x3.weights_refresh", 0);
  }
}

// The packed row layout of an NCHW bf16 tensor ([groups][chunks][2126 rows][64 channels],
// images wider than 36 as strips), as the rows conv kernels and the rows weight gradient
// read it: the tight layout (strips of up to 36 columns without zero columns) unless
// XDNA_CONV_LAYOUT / set_conv_layout asks for the reference's.
at::Tensor pack_rows(const at::Tensor& src, int layout) {
  const int64_t B = src.size(0), cin = src.size(1), H = src.size(2), W = src.size(3);
  at::Tensor x = src.contiguous();
  // The packed input is transient: the pack writes every element (zeros in the borders
  // and padded channels), so a recycled allocation needs no fill.  (The reference keeps a
  // pool of zero-filled buffers per shape, torch_xdna_device.cpp:1848-1872.)
  const size_t pbytes = xdna_conv3x3_layout_packed_bytes(int(B), int(cin), int(H), int(W), layout);
  TORCH_CHECK(pbytes > 0, "xdna conv: invalid packed layout");
  at::Tensor packed = alloc_bytes(pbytes);
  KernelTimer kt("conv3x3w_pack", 2.0 * double(x.numel()) + double(pbytes));
  check_abi(xdna_conv3x3_layout_pack_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                          static_cast<uint16_t*>(packed.data_ptr()), int(B), int(cin), int(H),
                                          int(W), layout, current_stream()),
            "conv pack");
  return packed;
}

// Runs the conv of a packed input (NCHW shape `src`, cin channels) with `w` (forward: w as
// given; dgrad: flip+swap) into a new NCHW tensor of cout channels.
// s1: a stride-1 conv of the model (not the stride-1 form of a stride-2 conv), which the
// BFP16 emulation covers: the reference's NPU takes only stride-1 convs.
// s2out: the forward of a 3x3 / stride-2 / pad-1 conv, storing only the even outputs of
// the stride-1 conv into a ceil(H/2) x ceil(W/2) tensor.
// The prepared form (forward, or input gradient: flip+swap) of conv weight w, from the
// cache or made here.  Both forms are cached (see PreparedWeights).  A trainable weight's
// forward prepares the input gradient's form in the same launch, so the backward of the
// step finds it; the optimizer step then bumps the epoch and the next forward prepares
// both again (or the fused optimizer step prepares them, refresh_conv_forms).
at::Tensor conv_weight_form(const at::Tensor& w, bool dgrad) {
  const int64_t cin = dgrad ? w.size(0) : w.size(1);
  const int64_t cout = dgrad ? w.size(1) : w.size(0);
  at::Tensor wc = w.contiguous();
  void* st = current_stream();
  const int64_t tag = capture_tag();
  const bool cacheable = weight_cacheable(w);
  const bool trainable = w.requires_grad() && !w.is_inference();
  at::Tensor wt = cacheable ? cached_weights(w, dgrad, tag) : at::Tensor();
  if (!wt.defined() && tag > 0 && cacheable && (!trainable || g_adam_prep.load())) {
    // a capture meeting a weight whose eager form is cached: the graph adopts it (kept
    // alive by the graph, prepared again by the captured optimizer step or by replay when
    // the weight was written; see GraphWeight)
    wt = cached_weights(w, dgrad, 0);
    if (wt.defined()) {
      adopt_graph_weight(tag, w, dgrad, wt, trainable);
      remember_weights(w, dgrad, wt, tag);
      count_call("hip_conv3x3.weights_graph", 0);
    }
  }
  // prepare / hit counters (the reference's npu_conv3x3w.weights{,_hit})
  count_call(wt.defined() ? "hip_conv3x3.weights_hit" : "hip_conv3x3.weights", 0);
  if (!wt.defined()) {
    wt = alloc_bytes(xdna_conv3x3_prepared_weight_bytes(int(cin), int(cout)));
    // bytes: the OIHW weight read once, each prepared form written
    KernelTimer kt("conv3x3_prep", double(w.numel()) * 2.0 * (trainable && !dgrad ? 3.0 : 2.0));
    if (trainable && !dgrad) {
      at::Tensor wtd = alloc_bytes(xdna_conv3x3_prepared_weight_bytes(int(cout), int(cin)));
      check_abi(xdna_conv3x3_prepare_weights_both_bf16(static_cast<const uint16_t*>(wc.const_data_ptr()),
                                                       static_cast<uint16_t*>(wt.data_ptr()),
                                                       static_cast<uint16_t*>(wtd.data_ptr()), int(w.size(0)),
                                                       int(w.size(1)), st),
                "conv weights");
      remember_weights(w, true, wtd, tag);
      remember_weights(w, false, wt, tag);
    } else {
      check_abi(xdna_conv3x3_prepare_weights_bf16(static_cast<const uint16_t*>(wc.const_data_ptr()),
                                                  static_cast<uint16_t*>(wt.data_ptr()), int(w.size(0)),
                                                  int(w.size(1)), dgrad ? 1 : 0, st),
                "conv weights");
      if (cacheable) remember_weights(w, dgrad, wt, tag);
    }
  }
  return wt;
}

// Small-grid convs read their NCHW input in place (xdna_conv3x3_nchw_act_bf16: the same
// bits as the pack followed by the packed conv) unless XDNA_CONV_NCHW=0; the BFP16
// emulation keeps its packed path.
std::atomic<int> g_conv_nchw{[] {
  const char* e = std::getenv("XDNA_CONV_NCHW");
  return e && std::atoi(e) == 0 ? 0 : 1;
}()};

bool nchw_route(const at::Tensor& src, int64_t cout, bool s1) {
  if (!g_conv_nchw.load() || (s1 && g_bfp16_emul.load())) return false;
  return xdna_conv3x3_nchw_small_eligible(int(src.size(0)), int(src.size(1)), int(cout), int(src.size(2)),
                                          int(src.size(3))) == 1;
}

// The conv of NCHW src (cin channels) with `w` as hip_conv_packed, for an nchw_route conv.
at::Tensor hip_conv_nchw(const at::Tensor& src_in, const at::Tensor& w, const at::Tensor* bias, bool dgrad,
                         int act = 0, bool s2out = false) {
  const at::Tensor src = src_in.contiguous();
  const int64_t B = src.size(0), cin = src.size(1), H = src.size(2), W = src.size(3);
  const int64_t cout = dgrad ? w.size(1) : w.size(0);
  at::Tensor wt = conv_weight_form(w, dgrad);
  at::Tensor out = s2out ? empty_xdna({B, cout, (H + 1) / 2, (W + 1) / 2}, at::kBFloat16)
                         : empty_xdna({B, cout, H, W}, at::kBFloat16);
  at::Tensor bc;
  if (bias) bc = bias->contiguous();
  const double flops = 2.0 * double(B) * double(H) * double(W) * double(cin) * double(cout) * 9.0;
  KernelTimer kt(s2out ? "conv3x3_rows.s2" : dgrad ? "conv3x3_rows.dgrad" : "conv3x3_rows.fwd", flops);
  count_call("hip_conv3x3.nchw", 0);
  check_abi(xdna_conv3x3_nchw_act_bf16(static_cast<const uint16_t*>(src.const_data_ptr()),
                                       static_cast<const uint16_t*>(wt.const_data_ptr()),
                                       bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr,
                                       static_cast<uint16_t*>(out.data_ptr()), int(B), int(cin), int(cout), int(H),
                                       int(W), act, s2out ? 1 : 0, current_stream()),
            "conv nchw");
  return out;
}

at::Tensor hip_conv_packed(const at::Tensor& packed, int layout, at::IntArrayRef src, const at::Tensor& w,
                           const at::Tensor* bias, bool dgrad, int act = 0, bool s1 = true, bool s2out = false) {
  const int64_t B = src[0], cin = src[1], H = src[2], W = src[3];
  const int64_t cout = dgrad ? w.size(1) : w.size(0);
  void* st = current_stream();
  at::Tensor wt = conv_weight_form(w, dgrad);
  at::Tensor out = s2out ? empty_xdna({B, cout, (H + 1) / 2, (W + 1) / 2}, at::kBFloat16)
                         : empty_xdna({B, cout, H, W}, at::kBFloat16);
  at::Tensor bc;
  if (bias) bc = bias->contiguous();
  const double flops = 2.0 * double(B) * double(H) * double(W) * double(cin) * double(cout) * 9.0;
  if (s2out) {
    KernelTimer kt("conv3x3_rows.s2", flops);
    check_abi(xdna_conv3x3_layout_rows_stride2_bf16(
                  static_cast<const uint16_t*>(packed.const_data_ptr()), static_cast<const uint16_t*>(wt.const_data_ptr()),
                  bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr,
                  static_cast<uint16_t*>(out.data_ptr()), int(B), int(cin), int(cout), int(H), int(W), layout, st),
              "conv rows (stride-2 output)");
    return out;
  }
  if (s1 && g_bfp16_emul.load()) {
    ScopedCount sc(dgrad ? "hip_conv3x3.bfp16_emul.dx.run" : "hip_conv3x3.bfp16_emul.fwd.run");
    check_abi(xdna_conv3x3_layout_rows_bfp16_emul_bf16(
                  static_cast<const uint16_t*>(packed.const_data_ptr()), static_cast<const uint16_t*>(wt.const_data_ptr()),
                  bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr,
                  static_cast<uint16_t*>(out.data_ptr()), int(B), int(cin), int(cout), int(H), int(W), layout, act, st),
              "conv rows (BFP16 emulation)");
    return out;
  }
  KernelTimer kt(dgrad ? "conv3x3_rows.dgrad" : "conv3x3_rows.fwd", flops);
  check_abi(xdna_conv3x3_layout_rows_act_bf16(static_cast<const uint16_t*>(packed.const_data_ptr()),
                                              static_cast<const uint16_t*>(wt.const_data_ptr()),
                                              bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr,
                                              static_cast<uint16_t*>(out.data_ptr()), int(B), int(cin), int(cout),
                                              int(H), int(W), layout, act, st),
            "conv rows");
  return out;
}

at::Tensor hip_conv(const at::Tensor& src, const at::Tensor& w, const at::Tensor* bias, bool dgrad) {
  const int layout = g_conv_layout.load();
  return hip_conv_packed(pack_rows(src, layout), layout, src.sizes(), w, bias, dgrad);
}

// Packed inputs of forward convs kept for the rows weight gradient of the same layer, so
// that the backward does not pack x again.  Keyed by the input's storage, data address,
// offset, sizes, strides, version, write epoch and capture tag (autograd keeps the input
// alive and unchanged until the backward; a pack kept outside a capture is never read
// by a captured backward, nor the reverse); the backward takes its entry out.  Entries
// whose input storage has died are dropped, and the oldest go once the kept bytes pass
// a cap.
struct PackedInput {
  c10::weak_intrusive_ptr<c10::StorageImpl> storage{c10::intrusive_ptr<c10::StorageImpl>()};
  const void* data = nullptr;
  int64_t offset = 0, version = 0, tag = 0;
  uint64_t epoch = 0, generation = 0;
  std::vector<int64_t> sizes, strides;
  int layout = 0;
  at::Tensor packed;
};

struct PackedInputCache {
  std::mutex mu;
  std::deque<PackedInput> entries;
  size_t bytes = 0;
  static constexpr size_t kMaxBytes = size_t(16) << 30;
};

PackedInputCache& packed_input_cache() {
  static auto* c = new PackedInputCache();
  return *c;
}

bool same_input(const PackedInput& e, const at::Tensor& x, int layout, int64_t tag, uint64_t epoch) {
  if (e.layout != layout || e.tag != tag || e.epoch != epoch || e.generation != g_replay_generation.load() ||
      e.data != x.storage().data() ||
      e.offset != x.storage_offset() || e.sizes != x.sizes().vec() || e.strides != x.strides().vec() ||
      e.version != int64_t(x.unsafeGetTensorImpl()->version_counter().current_version()))
    return false;
  auto live = e.storage.lock();
  return live && live.get() == x.storage().unsafeGetStorageImpl();
}

void remember_packed_input(const at::Tensor& x, const at::Tensor& packed, int layout) {
  const int64_t tag = capture_tag();
  const uint64_t epoch = write_epoch(x);
  PackedInputCache& c = packed_input_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  for (auto it = c.entries.begin(); it != c.entries.end();) {
    if (it->storage.expired() || same_input(*it, x, layout, tag, epoch)) {
      c.bytes -= size_t(it->packed.nbytes());
      it = c.entries.erase(it);
    } else {
      ++it;
    }
  }
  PackedInput e;
  e.storage = c10::weak_intrusive_ptr<c10::StorageImpl>(x.storage().getWeakStorageImpl());
  e.data = x.storage().data();
  e.offset = x.storage_offset();
  e.version = int64_t(x.unsafeGetTensorImpl()->version_counter().current_version());
  e.tag = tag;
  e.epoch = epoch;
  e.generation = g_replay_generation.load();
  e.sizes = x.sizes().vec();
  e.strides = x.strides().vec();
  e.layout = layout;
  e.packed = packed;
  c.bytes += size_t(packed.nbytes());
  c.entries.push_back(std::move(e));
  while (c.bytes > PackedInputCache::kMaxBytes && c.entries.size() > 1) {
    c.bytes -= size_t(c.entries.front().packed.nbytes());
    c.entries.pop_front();
  }
}

at::Tensor take_packed_input(const at::Tensor& x, int layout) {
  if (x.is_inference()) return at::Tensor();
  const int64_t tag = capture_tag();
  const uint64_t epoch = write_epoch(x);
  PackedInputCache& c = packed_input_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  for (auto it = c.entries.begin(); it != c.entries.end(); ++it) {
    if (!same_input(*it, x, layout, tag, epoch)) continue;
    at::Tensor p = it->packed;
    c.bytes -= size_t(p.nbytes());
    c.entries.erase(it);
    return p;
  }
  return at::Tensor();
}

}  // namespace

void clear_packed_inputs() {
  PackedInputCache& c = packed_input_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  c.entries.clear();
  c.bytes = 0;
}

std::vector<int64_t> cache_stats(int64_t tag) {
  std::vector<int64_t> out(4, 0);
  {
    WeightCache& c = weight_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    for (const auto& e : c.entries) {
      if (tag >= 0 && e.tag != tag) continue;
      out[0] += 1;
      out[1] += int64_t(e.wt.nbytes());
    }
  }
  PackedInputCache& c = packed_input_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  for (const auto& e : c.entries) {
    if (tag >= 0 && e.tag != tag) continue;
    out[2] += 1;
    out[3] += int64_t(e.packed.nbytes());
  }
  return out;
}

void purge_capture_entries(int64_t tag) {
  {
    WeightCache& c = weight_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    for (auto it = c.entries.begin(); it != c.entries.end();) {
      if (it->tag == tag) {
        c.bytes -= size_t(it->wt.nbytes());
        it = c.entries.erase(it);
      } else {
        ++it;
      }
    }
  }
  PackedInputCache& c = packed_input_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  for (auto it = c.entries.begin(); it != c.entries.end();) {
    if (it->tag == tag) {
      c.bytes -= size_t(it->packed.nbytes());
      it = c.entries.erase(it);
    } else {
      ++it;
    }
  }
}

namespace {

bool wgrad_rows_pick(int64_t Cin, int64_t Cout, int64_t W);
std::atomic<int64_t> g_dw_jobs{0};

// Forward of a 3x3 / stride-1 conv; the packed input is kept when the weight is trainable
// and its gradient takes the rows form (whether or not autograd records this call: a
// caller may run the aten backward itself).  A kept pack whose backward never comes goes
// when its input dies.  Inference tensors keep nothing (they have no version counter).
at::Tensor hip_conv_fwd(const at::Tensor& input, const at::Tensor& weight, const at::Tensor* bias, bool s1 = true,
                        bool s2out = false) {
  const int layout = g_conv_layout.load();
  const bool keep = g_mode.load() >= 2 && weight.requires_grad() && !weight.is_inference() &&
                    !input.is_inference() && wgrad_rows_pick(input.size(1), weight.size(0), input.size(3));
  // no packed copy wanted afterwards: a small grid reads the input in place
  if (!keep && nchw_route(input, weight.size(0), s1)) return hip_conv_nchw(input, weight, bias, false, 0, s2out);
  at::Tensor packed = pack_rows(input, layout);
  if (keep) remember_packed_input(input, packed, layout);
  return hip_conv_packed(packed, layout, input.sizes(), weight, bias, false, 0, s1, s2out);
}

// The spread-and-pack of a stride-2 conv's output gradient: the packed rows of its H x W
// spread (gradient at even (y, x), zeros elsewhere), in one pass.
at::Tensor pack_rows_spread(const at::Tensor& grad_output, int64_t H, int64_t W, int layout) {
  const at::Tensor d = grad_output.contiguous();
  const int64_t B = d.size(0), C = d.size(1);
  if (W > 256) {
    // rows wider than the pack's LDS tile: the spread tensor, then the ordinary pack
    at::Tensor full = empty_xdna({B, C, H, W}, at::kBFloat16);
    check_abi(xdna_dilate2_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                static_cast<uint16_t*>(full.data_ptr()), B * C, int(H), int(W), current_stream()),
              "conv stride-2 dilate");
    return pack_rows(full, layout);
  }
  const size_t pbytes = xdna_conv3x3_layout_packed_bytes(int(B), int(C), int(H), int(W), layout);
  TORCH_CHECK(pbytes > 0, "xdna conv: invalid packed layout");
  at::Tensor packed = alloc_bytes(pbytes);
  KernelTimer kt("conv3x3w_pack", 2.0 * double(d.numel()) + double(pbytes));
  check_abi(xdna_conv3x3_layout_pack_dilate2_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                                  static_cast<uint16_t*>(packed.data_ptr()), int(B), int(C), int(H),
                                                  int(W), layout, current_stream()),
            "conv spread pack");
  return packed;
}

// ---------------------------------------------------------------------------------------
// Other 2-D convolutions (any kernel size, stride and padding; dilation 1, groups 1, bf16):
// the general HIP kernels.  The reference runs these on the CPU (its fallback to
// aten::convolution, torch_xdna_device.cpp:4594-4604, 4862-4874).
// ---------------------------------------------------------------------------------------
bool gconv_eligible(const at::Tensor& x, const at::Tensor& w, c10::SymIntArrayRef stride,
                    c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation, bool transposed,
                    c10::SymIntArrayRef output_padding, const c10::SymInt& groups) {
  if (g_mode.load() < 1) return false;
  if (x.scalar_type() != at::kBFloat16 || w.scalar_type() != at::kBFloat16) return false;
  if (x.dim() != 4 || w.dim() != 4 || x.size(1) != w.size(1)) return false;
  if (stride.size() != 2 || padding.size() != 2 || !is_one(dilation, 1) || transposed) return false;
  if (!is_one(output_padding, 0) || groups != 1) return false;
  if (stride[0] < 1 || stride[1] < 1 || padding[0] < 0 || padding[1] < 0) return false;
  if (x.device().type() != kXdna || w.device().type() != kXdna) return false;
  const int64_t lim = int64_t(1) << 30;
  for (const at::Tensor* t : {&x, &w})
    if (t->numel() >= lim) return false;
  for (int64_t d = 0; d < 4; ++d)
    if (x.size(d) < 1 || w.size(d) < 1) return false;
  const int64_t H = x.size(2), W = x.size(3), KH = w.size(2), KW = w.size(3);
  const int64_t ph = padding[0].expect_int(), pw = padding[1].expect_int();
  if (H + 2 * ph < KH || W + 2 * pw < KW) return false;
  const int64_t Ho = (H + 2 * ph - KH) / stride[0].expect_int() + 1, Wo = (W + 2 * pw - KW) / stride[1].expect_int() + 1;
  return x.size(0) * w.size(0) * Ho * Wo < lim;
}

struct GeomArgs {
  int B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw, Ho, Wo;
};

// Where the general kernels beat MIOpen (measured on the style network's layers, B40
// 36x36): stride-1 layers with 32 or more output channels, forward and weight gradient
// (9x9 3->32: 22 vs 38 us forward), and the forward of stride-1 layers with a few output
// channels and 16 or more inputs, which takes the direct form (9x9 32->3: 28 vs 147 us).
// Strided layers, other input gradients, and the weight gradient of few-output layers
// stay on MIOpen unless mode 2 asks otherwise.
bool gconv_auto(int cout, int sh, int sw) { return cout >= 32 && sh == 1 && sw == 1; }
// 3x3 / stride-1 convs with at most 4 input channels (RGB input layers): the rows path
// pads the input to a 64-channel chunk (16-21x the MACs), so their forward and weight
// gradient take the general kernels (measured on MI355X: ResNet-18's stem B128 3->64 at
// 64x64 forward 80.6 -> 31.0 us, weight gradient 209 -> 133 us; VGG's first layer B40 at
// 36x36 forward 19.2 -> 8.5 us); their input gradient (64 input channels of the gradient
// conv) stays on the rows path, which is faster there.
bool few_input_3x3(const at::Tensor& x, const at::Tensor& w) {
  const int m = g_gconv_mode.load();
  return x.size(1) <= 4 && (m == 2 || (m == 1 && gconv_auto(int(w.size(0)), 1, 1)));
}
bool gconv_auto_fwd(int cin, int cout, int sh, int sw) {
  return gconv_auto(cout, sh, sw) || (cout <= 32 && cin >= 16 && sh == 1 && sw == 1);
}
// The input gradient where the direct form takes it (stride 1, at most 32 input channels
// of the layer and 16 or more outputs: 9x9 3->32 in 29 us); MIOpen's input gradient of
// that layer also misses the 2-ulp bar on some elements.
bool gconv_auto_dgrad(const GeomArgs& g) {
  return g.sh == 1 && g.sw == 1 && g.Cin <= 32 && g.Cout >= 16 && g.ph <= g.KH - 1 && g.pw <= g.KW - 1;
}

GeomArgs gconv_geom(const at::Tensor& x, const at::Tensor& w, c10::SymIntArrayRef stride,
                    c10::SymIntArrayRef padding) {
  GeomArgs g;
  g.B = int(x.size(0)); g.Cin = int(x.size(1)); g.H = int(x.size(2)); g.W = int(x.size(3));
  g.Cout = int(w.size(0)); g.KH = int(w.size(2)); g.KW = int(w.size(3));
  g.sh = int(stride[0].expect_int()); g.sw = int(stride[1].expect_int());
  g.ph = int(padding[0].expect_int()); g.pw = int(padding[1].expect_int());
  g.Ho = (g.H + 2 * g.ph - g.KH) / g.sh + 1;
  g.Wo = (g.W + 2 * g.pw - g.KW) / g.sw + 1;
  return g;
}

at::Tensor hip_gconv_fwd(const at::Tensor& input, const at::Tensor& weight, const at::Tensor* bias,
                         c10::SymIntArrayRef stride, c10::SymIntArrayRef padding) {
  const GeomArgs g = gconv_geom(input, weight, stride, padding);
  at::Tensor x = input.contiguous(), w = weight.contiguous();
  at::Tensor bc;
  if (bias) bc = bias->contiguous();
  at::Tensor y = empty_xdna({g.B, g.Cout, g.Ho, g.Wo}, at::kBFloat16);
  KernelTimer kt("conv2d.fwd", 2.0 * g.B * g.Ho * g.Wo * double(g.Cout) * g.Cin * g.KH * g.KW);
  check_abi(xdna_conv2d_fwd_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                 static_cast<const uint16_t*>(w.const_data_ptr()),
                                 bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr,
                                 static_cast<uint16_t*>(y.data_ptr()), g.B, g.Cin, g.Cout, g.H, g.W, g.KH,
                                 g.KW, g.sh, g.sw, g.ph, g.pw, current_stream()),
            "conv2d forward");
  return y;
}

// ---------------------------------------------------------------------------------------
// 1x1 convolutions (stride 1 or 2, no padding: ResNet's downsampling shortcut) as MFMA
// GEMMs: y[n] = W [Cout x Cin] . x[n] [Cin x HW] for every image (one batched launch with
// the weight broadcast), dx[n] = W^T . dy[n], and dW = dY^T . X over all N*HW pixels as
// one split-K product of channel-major copies.  Stride 2 takes every other pixel of x
// (subsample2) and spreads dx back onto the full grid with zeros (dilate2).  The
// reference runs these on its CPU (torch_xdna_device.cpp:4594-4604, 4862-4874).
// ---------------------------------------------------------------------------------------
bool conv1x1_eligible(const at::Tensor& x, const at::Tensor& w, c10::SymIntArrayRef stride,
                      c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation, bool transposed,
                      c10::SymIntArrayRef output_padding, const c10::SymInt& groups) {
  if (g_mode.load() < 1) return false;
  if (x.scalar_type() != at::kBFloat16 || w.scalar_type() != at::kBFloat16) return false;
  if (x.dim() != 4 || w.dim() != 4 || w.size(2) != 1 || w.size(3) != 1 || x.size(1) != w.size(1)) return false;
  if (!(is_one(stride, 1) || is_one(stride, 2)) || !is_one(padding, 0) || !is_one(dilation, 1) || transposed)
    return false;
  if (!is_one(output_padding, 0) || groups != 1) return false;
  if (x.device().type() != kXdna || w.device().type() != kXdna) return false;
  for (int64_t d = 0; d < 4; ++d)
    if (x.size(d) < 1 || w.size(d) < 1) return false;
  const int64_t lim = int64_t(1) << 30;
  return x.numel() < lim && x.size(0) <= 65535 && x.size(0) * x.size(2) * x.size(3) < lim;
}

// x itself (stride 1) or its stride-2 sample, contiguous
at::Tensor conv1x1_input(const at::Tensor& input, int64_t s) {
  at::Tensor x = input.contiguous();
  if (s == 1) return x;
  const int64_t N = x.size(0), C = x.size(1), H = x.size(2), W = x.size(3);
  at::Tensor xs = empty_xdna({N, C, (H + 1) / 2, (W + 1) / 2}, at::kBFloat16);
  check_abi(xdna_subsample2_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                 static_cast<uint16_t*>(xs.data_ptr()), N * C, int(H), int(W), current_stream()),
            "conv1x1 subsample");
  return xs;
}

at::Tensor hip_conv1x1_fwd(const at::Tensor& input, const at::Tensor& weight, const at::Tensor* bias, int64_t s) {
  const at::Tensor xs = conv1x1_input(input, s);
  const at::Tensor w = weight.contiguous();
  const int64_t N = xs.size(0), Ci = xs.size(1), Ho = xs.size(2), Wo = xs.size(3), Co = w.size(0), P = Ho * Wo;
  at::Tensor y = empty_xdna({N, Co, Ho, Wo}, at::kBFloat16);
  at::Tensor bc;
  if (bias) bc = bias->contiguous();
  KernelTimer kt("conv1x1.fwd", 2.0 * N * P * double(Co) * Ci);
  check_abi(xdna_gemm_bf16(static_cast<const uint16_t*>(w.const_data_ptr()),
                           static_cast<const uint16_t*>(xs.const_data_ptr()), static_cast<uint16_t*>(y.data_ptr()),
                           bias ? static_cast<const uint16_t*>(bc.const_data_ptr()) : nullptr, int(N), int(Co), int(P),
                           int(Ci), Ci, 1, 0, P, 1, Ci * P, P, 1, Co * P, bias ? 3 : 0, 1, 0, 1.0f, 1.0f,
                           current_stream()),
            "conv1x1 forward");
  return y;
}

void hip_conv1x1_bwd(const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight, int64_t s,
                     std::array<bool, 3> mask, at::Tensor& gi, at::Tensor& gw, at::Tensor& gb) {
  const at::Tensor dy = grad_output.contiguous();
  const at::Tensor w = weight.contiguous();
  const int64_t N = input.size(0), Ci = input.size(1), H = input.size(2), W = input.size(3);
  const int64_t Co = w.size(0), Ho = dy.size(2), Wo = dy.size(3), P = Ho * Wo;
  void* st = current_stream();
  if (mask[0]) {
    at::Tensor dxs = empty_xdna({N, Ci, Ho, Wo}, at::kBFloat16);
    KernelTimer kt("conv1x1.dgrad", 2.0 * N * P * double(Co) * Ci);
    check_abi(xdna_gemm_bf16(static_cast<const uint16_t*>(w.const_data_ptr()),
                             static_cast<const uint16_t*>(dy.const_data_ptr()), static_cast<uint16_t*>(dxs.data_ptr()),
                             nullptr, int(N), int(Ci), int(P), int(Co), 1, Ci, 0, P, 1, Co * P, P, 1, Ci * P, 0, 0, 0,
                             1.0f, 0.0f, st),
              "conv1x1 input gradient");
    if (s == 1) {
      gi = dxs;
    } else {
      gi = empty_xdna({N, Ci, H, W}, at::kBFloat16);
      check_abi(xdna_dilate2_bf16(static_cast<const uint16_t*>(dxs.const_data_ptr()),
                                  static_cast<uint16_t*>(gi.data_ptr()), N * Ci, int(H), int(W), st),
                "conv1x1 dilate");
    }
  }
  if (mask[1]) {
    // channel-major copies: dY^T [Co][N*P] and X^T [Ci][N*P], then one product over N*P
    const at::Tensor dyt = dy.permute({1, 0, 2, 3}).contiguous();
    const at::Tensor xst = conv1x1_input(input, s).permute({1, 0, 2, 3}).contiguous();
    const int64_t K = N * P;
    gw = empty_xdna({Co, Ci, 1, 1}, at::kBFloat16);
    KernelTimer kt("conv1x1.wgrad", 2.0 * N * P * double(Co) * Ci);
    check_abi(xdna_gemm_bf16(static_cast<const uint16_t*>(dyt.const_data_ptr()),
                             static_cast<const uint16_t*>(xst.const_data_ptr()), static_cast<uint16_t*>(gw.data_ptr()),
                             nullptr, 1, int(Co), int(Ci), int(K), K, 1, 0, 1, K, 0, Ci, 1, 0, 0, 0, 0, 1.0f, 0.0f, st),
              "conv1x1 weight gradient");
    g_dw_jobs.fetch_add(1);
  }
  if (mask[2]) {
    gb = empty_xdna({Co}, at::kBFloat16);
    check_abi(xdna_conv3x3_bias_grad_bf16(static_cast<const uint16_t*>(dy.const_data_ptr()),
                                          static_cast<uint16_t*>(gb.data_ptr()), int(N), int(Co), int(Ho), int(Wo),
                                          st),
              "conv1x1 bias grad");
  }
}

at::Tensor convolution_overrideable_xdna(const at::Tensor& input, const at::Tensor& weight,
                                         const std::optional<at::Tensor>& bias,
                                         c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                                         c10::SymIntArrayRef dilation, bool transposed,
                                         c10::SymIntArrayRef output_padding, c10::SymInt groups) {
  const bool has_bias = bias && bias->defined();
  if (conv_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
      input.size(1) == weight.size(1) && !few_input_3x3(input, weight) &&
      (!has_bias || (bias->scalar_type() == at::kBFloat16 && bias->dim() == 1 &&
                     bias->size(0) == weight.size(0) && bias->device().type() == kXdna))) {
    ScopedCount sc("hip_conv3x3.fwd.run");
    return hip_conv_fwd(input, weight, has_bias ? &*bias : nullptr);
  }
  if (conv_s2_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
      (!has_bias || (bias->scalar_type() == at::kBFloat16 && bias->dim() == 1 &&
                     bias->size(0) == weight.size(0) && bias->device().type() == kXdna))) {
    ScopedCount sc("hip_conv3x3_s2.fwd.run");
    return hip_conv_fwd(input, weight, has_bias ? &*bias : nullptr, /*s1=*/false, /*s2out=*/true);
  }
  if (conv1x1_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
      (!has_bias || (bias->scalar_type() == at::kBFloat16 && bias->dim() == 1 &&
                     bias->size(0) == weight.size(0) && bias->device().type() == kXdna))) {
    ScopedCount sc("hip_conv1x1.fwd.run");
    return hip_conv1x1_fwd(input, weight, has_bias ? &*bias : nullptr, stride[0].expect_int());
  }
  const int gmode = g_gconv_mode.load();
  if (gmode > 0 &&
      gconv_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
      (gmode == 2 || gconv_auto_fwd(int(weight.size(1)), int(weight.size(0)), int(stride[0].expect_int()),
                                    int(stride[1].expect_int()))) &&
      (!has_bias || (bias->scalar_type() == at::kBFloat16 && bias->dim() == 1 &&
                     bias->size(0) == weight.size(0) && bias->device().type() == kXdna))) {
    ScopedCount sc("hip_conv2d.fwd.run");
    return hip_gconv_fwd(input, weight, has_bias ? &*bias : nullptr, stride, padding);
  }
  ScopedCount sc("aten::convolution.rocm");
  BelowAutograd g;
  return back(at::_ops::convolution::call(rocm(input), rocm(weight), rocm(bias), stride, padding,
                                          dilation, transposed, output_padding, groups));
}

// Weight gradient (+ bias gradient) through the two wgrad stages.  Stage 1 takes
// snapshots of x and dY, so later writes to either cannot change the gradient (the
// reference's deferred-dW contract, run_deferred_dw.py:62-71); stage 2 is ordered
// before every reader of gw by the stream.
void hip_wgrad(const at::Tensor& input, const at::Tensor& dy, at::Tensor& gw, at::Tensor* gb) {
  const int64_t B = input.size(0), Cin = input.size(1), H = input.size(2), W = input.size(3);
  const int64_t Cout = dy.size(1);
  at::Tensor x = input.contiguous();
  at::Tensor d = dy.contiguous();
  void* st = current_stream();
  const size_t wsb = xdna_conv3x3_wgrad_workspace_bytes(int(B), int(Cin), int(Cout), int(H), int(W));
  at::Tensor ws = alloc_bytes(wsb);
  gw = empty_xdna({Cout, Cin, 3, 3}, at::kBFloat16);
  if (gb) *gb = empty_xdna({Cout}, at::kBFloat16);
  check_abi(xdna_conv3x3_wgrad_pack_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                         static_cast<const uint16_t*>(d.const_data_ptr()), int(B),
                                         int(Cin), int(Cout), int(H), int(W), ws.data_ptr(), wsb, st),
            "conv wgrad pack");
  KernelTimer kt("conv3x3_wgrad", 2.0 * double(B) * double(H) * double(W) * double(Cin) * double(Cout) * 9.0);
  check_abi(xdna_conv3x3_wgrad_packed_bf16(static_cast<uint16_t*>(gw.data_ptr()),
                                           gb ? static_cast<uint16_t*>(gb->data_ptr()) : nullptr,
                                           int(B), int(Cin), int(Cout), int(H), int(W), ws.data_ptr(),
                                           wsb, st),
            "conv wgrad");
}

// Weight gradient (+ bias gradient) on the packed row layout: x packed here, dY in the
// packed form its input gradient already read (`dpacked`), so neither is copied
// channel-major.  The packs are snapshots, as in the channel-major form.  Split in two:
// wgrad_rows_prepare makes every buffer the launch uses (x's pack, the workspace, gw, gb),
// wgrad_rows_launch enqueues the kernels on a given stream.
struct WgradRowsJob {
  at::Tensor xpacked, ws;
  size_t wsb = 0;
  int64_t B = 0, Cin = 0, Cout = 0, H = 0, W = 0;
  int layout = 0;
};

WgradRowsJob wgrad_rows_prepare(const at::Tensor& input, int layout, int64_t Cout, at::Tensor& gw, at::Tensor* gb) {
  WgradRowsJob j;
  j.B = input.size(0), j.Cin = input.size(1), j.H = input.size(2), j.W = input.size(3), j.Cout = Cout;
  j.layout = layout;
  j.xpacked = take_packed_input(input, layout);
  if (j.xpacked.defined()) {
    ScopedCount sk("hip_conv3x3.dw_rows.kept_pack");
  } else {
    j.xpacked = pack_rows(input, layout);
  }
  j.wsb = xdna_conv3x3_wgrad_rows_workspace_bytes(int(j.B), int(j.Cin), int(Cout), int(j.H), int(j.W), layout);
  j.ws = alloc_bytes(j.wsb);
  gw = empty_xdna({Cout, j.Cin, 3, 3}, at::kBFloat16);
  if (gb) *gb = empty_xdna({Cout}, at::kBFloat16);
  return j;
}

void wgrad_rows_launch(const WgradRowsJob& j, const at::Tensor& dpacked, at::Tensor& gw, at::Tensor* gb, void* st) {
  check_abi(xdna_conv3x3_wgrad_rows_bf16(static_cast<const uint16_t*>(j.xpacked.const_data_ptr()),
                                         static_cast<const uint16_t*>(dpacked.const_data_ptr()),
                                         static_cast<uint16_t*>(gw.data_ptr()),
                                         gb ? static_cast<uint16_t*>(gb->data_ptr()) : nullptr, int(j.B),
                                         int(j.Cin), int(j.Cout), int(j.H), int(j.W), j.layout, j.ws.data_ptr(),
                                         j.wsb, st),
            "conv wgrad rows");
}

void hip_wgrad_rows(const at::Tensor& input, const at::Tensor& dpacked, int layout, int64_t Cout, at::Tensor& gw,
                    at::Tensor* gb) {
  const WgradRowsJob j = wgrad_rows_prepare(input, layout, Cout, gw, gb);
  KernelTimer kt("conv3x3_wgrad", 2.0 * double(j.B) * double(j.H) * double(j.W) * double(j.Cin) * double(Cout) * 9.0);
  wgrad_rows_launch(j, dpacked, gw, gb, current_stream());
}

// The weight gradient beside the input gradient in captured graphs.  A captured backward of
// a 3x3 layer that needs both forks the weight gradient onto a side stream once dY is
// packed and joins it back after both are enqueued, so in the graph they are parallel
// branches (on small grids each fills a fraction of the CUs).  Every buffer the weight
// gradient uses is made before the fork and released after the join: the caching allocator
// hands a freed block to the next allocation in capture order, which parallel branches do
// not follow, so no block one branch frees may reach the other.  Eager work keeps one
// stream.  Opt-in (XDNA_WGRAD_OVERLAP=1 or set_wgrad_overlap(1); g_wgrad_overlap): on the
// style network's step the graph replays slower with it (436 -> 396 it/s), each fork and
// join costing about 17 us of synchronization between the branches' hardware queues, more
// than the two small kernels gain by sharing the CUs.

struct SideStream {
  void* stream = nullptr;
  void* fork = nullptr;
  void* join = nullptr;
};
std::mutex g_side_mu;
SideStream g_side;

// The side stream and its two events, made outside capture (creating a stream is not a
// call a capture may record): the eager steps that precede a capture make them.
bool side_stream_ready(bool may_create) {
  std::lock_guard<std::mutex> lock(g_side_mu);
  if (g_side.stream) return true;
  if (!may_create) return false;
  void* f = xdna_hip_event_create(0);
  void* j = f ? xdna_hip_event_create(0) : nullptr;
  void* s = j ? xdna_hip_stream_create() : nullptr;
  if (!s) {
    if (f) xdna_hip_event_destroy(f);
    if (j) xdna_hip_event_destroy(j);
    return false;
  }
  g_side = SideStream{s, f, j};
  return true;
}

// Which weight-gradient form a 3x3 layer takes: the rows form (its x operand is the
// forward's kept pack, its dY operand the input gradient's) unless the channel-major form
// is asked for; on the tight layout the rows form measured faster on all 36 sweep shapes
// (6.7 vs 7.8 ms per sweep step, the channel-major copies included).  Images wider than
// 142 exceed the channel-major form's window and always take the rows form.
bool wgrad_rows_pick(int64_t Cin, int64_t Cout, int64_t W) {
  (void)Cin;
  (void)Cout;
  return W > 142 || g_wgrad_form.load() != 1;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> convolution_backward_overrideable_xdna(
    const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight,
    c10::SymIntArrayRef stride, c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation,
    bool transposed, c10::SymIntArrayRef output_padding, c10::SymInt groups,
    std::array<bool, 3> output_mask) {
  at::Tensor gi, gw, gb;
  const bool go_ok = grad_output.scalar_type() == at::kBFloat16 && grad_output.dim() == 4 &&
                     grad_output.device().type() == kXdna && input.size(1) == weight.size(1) &&
                     grad_output.size(1) == weight.size(0) && grad_output.size(0) == input.size(0);
  bool hip = conv_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
             go_ok && grad_output.size(2) == input.size(2) && grad_output.size(3) == input.size(3);
  // stride 2: the stride-1 gradients of the gradient spread onto the stride-1 grid
  // stride 2: the stride-1 gradients of the gradient spread onto the stride-1 grid (its
  // packed rows made in one pass; the spread tensor itself only for the channel-major
  // weight gradient)
  at::Tensor go = grad_output;
  bool strided = false;
  std::vector<int64_t> go_sizes = grad_output.sizes().vec();
  if (!hip && go_ok && conv_s2_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups) &&
      grad_output.size(2) == (input.size(2) + 1) / 2 && grad_output.size(3) == (input.size(3) + 1) / 2) {
    ScopedCount sc("hip_conv3x3_s2.bwd.run");
    go_sizes = {input.size(0), weight.size(0), input.size(2), input.size(3)};
    hip = true;
    strided = true;
  }
  auto mask = output_mask;
  // few input channels: the input gradient here, the weight gradient on the general kernels
  const bool few_in = hip && !strided && few_input_3x3(input, weight);
  const bool dw = hip && mask[1] && g_mode.load() >= 2 && !few_in;
  const bool dw_rows = dw && wgrad_rows_pick(input.size(1), weight.size(0), input.size(3));
  // dY packed once: the input gradient's conv and the rows weight gradient read it
  const int layout = g_conv_layout.load();
  at::Tensor gop;
  // the input gradient alone reads dY: a small grid reads it in place
  const bool dx_nchw = hip && mask[0] && !dw_rows && !strided && nchw_route(go, weight.size(1), true);
  if (hip && ((mask[0] && !dx_nchw) || dw_rows))
    gop = strided ? pack_rows_spread(grad_output, go_sizes[2], go_sizes[3], layout) : pack_rows(go, layout);
  // the rows weight gradient beside the input gradient (captured graphs only)
  const bool both = dw_rows && mask[0];
  const int64_t ctag = both && g_wgrad_overlap.load() ? capture_tag() : 0;
  if (both && ctag == 0 && g_wgrad_overlap.load()) side_stream_ready(true);
  const bool beside = ctag != 0 && side_stream_ready(false);
  WgradRowsJob wjob;
  if (beside) {
    wjob = wgrad_rows_prepare(input, layout, weight.size(0), gw, mask[2] ? &gb : nullptr);
    check_abi(xdna_hip_event_record(g_side.fork, current_stream()), "conv backward fork");
  }
  if (hip && mask[0]) {
    ScopedCount sc("hip_conv3x3.dx.run");
    gi = dx_nchw ? hip_conv_nchw(go, weight, nullptr, true)
                 : hip_conv_packed(gop, layout, go_sizes, weight, nullptr, true, 0, !strided);
    mask[0] = false;
  }
  if (strided && dw && !dw_rows) {
    // the channel-major weight gradient reads the spread gradient as a tensor
    const at::Tensor d = grad_output.contiguous();
    go = empty_xdna(go_sizes, at::kBFloat16);
    check_abi(xdna_dilate2_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                static_cast<uint16_t*>(go.data_ptr()), go_sizes[0] * go_sizes[1], int(go_sizes[2]),
                                int(go_sizes[3]), current_stream()),
              "conv stride-2 dilate");
  }
  if (dw) {
    ScopedCount sc("hip_conv3x3.dw.run");
    if (dw_rows) {
      ScopedCount sr("hip_conv3x3.dw_rows.run");
      if (beside) {
        ScopedCount sb("hip_conv3x3.dw_rows.beside_dx");
        check_abi(xdna_hip_stream_wait_event(g_side.stream, g_side.fork), "conv backward fork");
        wgrad_rows_launch(wjob, gop, gw, mask[2] ? &gb : nullptr, g_side.stream);
        check_abi(xdna_hip_event_record(g_side.join, g_side.stream), "conv backward join");
        check_abi(xdna_hip_stream_wait_event(current_stream(), g_side.join), "conv backward join");
      } else {
        hip_wgrad_rows(input, gop, layout, weight.size(0), gw, mask[2] ? &gb : nullptr);
      }
    } else {
      hip_wgrad(input, go, gw, mask[2] ? &gb : nullptr);
    }
    g_dw_jobs.fetch_add(1);
    mask[1] = false;
    mask[2] = false;
  }
  if (hip && mask[2]) {
    ScopedCount sc("hip_conv3x3.bias_grad.run");
    at::Tensor d = go.contiguous();
    gb = empty_xdna({go.size(1)}, at::kBFloat16);
    check_abi(xdna_conv3x3_bias_grad_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                          static_cast<uint16_t*>(gb.data_ptr()), int(d.size(0)),
                                          int(d.size(1)), int(d.size(2)), int(d.size(3)),
                                          current_stream()),
              "conv bias grad");
    mask[2] = false;
  }
  if (!hip && go_ok && (mask[0] || mask[1] || mask[2]) &&
      conv1x1_eligible(input, weight, stride, padding, dilation, transposed, output_padding, groups)) {
    const int64_t s = stride[0].expect_int();
    TORCH_CHECK(grad_output.size(2) == (input.size(2) + s - 1) / s && grad_output.size(3) == (input.size(3) + s - 1) / s,
                "convolution_backward: grad_output has the wrong spatial size");
    ScopedCount sc("hip_conv1x1.bwd.run");
    std::array<bool, 3> m1 = mask;
    if (g_mode.load() < 2) m1[1] = false;  // mode 1: no HIP weight gradient
    hip_conv1x1_bwd(grad_output, input, weight, s, m1, gi, gw, gb);
    for (int i = 0; i < 3; ++i)
      if (m1[i]) mask[i] = false;
  }
  const int gmode = g_gconv_mode.load();
  const bool ghip = (!hip || few_in) && gmode > 0 &&
                    gconv_eligible(input, weight, stride, padding, dilation, transposed,
                                   output_padding, groups) &&
                    grad_output.scalar_type() == at::kBFloat16 && grad_output.dim() == 4 &&
                    grad_output.device().type() == kXdna && grad_output.size(0) == input.size(0) &&
                    grad_output.size(1) == weight.size(0);
  if (ghip) {
    const GeomArgs g = gconv_geom(input, weight, stride, padding);
    TORCH_CHECK(grad_output.size(2) == g.Ho && grad_output.size(3) == g.Wo,
                "convolution_backward: grad_output has the wrong spatial size");
    at::Tensor d = grad_output.contiguous();
    const double flops = 2.0 * g.B * g.Ho * g.Wo * double(g.Cout) * g.Cin * g.KH * g.KW;
    const bool auto_ok = gconv_auto(g.Cout, g.sh, g.sw);
    if (mask[0] && (gmode == 2 || gconv_auto_dgrad(g))) {
      ScopedCount sc("hip_conv2d.dx.run");
      at::Tensor w = weight.contiguous();
      gi = empty_xdna({g.B, g.Cin, g.H, g.W}, at::kBFloat16);
      KernelTimer kt("conv2d.dgrad", flops);
      check_abi(xdna_conv2d_dgrad_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                       static_cast<const uint16_t*>(w.const_data_ptr()),
                                       static_cast<uint16_t*>(gi.data_ptr()), g.B, g.Cin, g.Cout, g.H, g.W,
                                       g.KH, g.KW, g.sh, g.sw, g.ph, g.pw, current_stream()),
                "conv2d dgrad");
      mask[0] = false;
    }
    if (mask[1] && g_mode.load() >= 2 && (gmode == 2 || auto_ok)) {
      ScopedCount sc("hip_conv2d.dw.run");
      at::Tensor x = input.contiguous();
      gw = empty_xdna({g.Cout, g.Cin, g.KH, g.KW}, at::kBFloat16);
      if (mask[2]) gb = empty_xdna({g.Cout}, at::kBFloat16);
      KernelTimer kt("conv2d.wgrad", flops);
      check_abi(xdna_conv2d_wgrad_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                       static_cast<const uint16_t*>(d.const_data_ptr()),
                                       static_cast<uint16_t*>(gw.data_ptr()),
                                       mask[2] ? static_cast<uint16_t*>(gb.data_ptr()) : nullptr, g.B, g.Cin,
                                       g.Cout, g.H, g.W, g.KH, g.KW, g.sh, g.sw, g.ph, g.pw, current_stream()),
                "conv2d wgrad");
      g_dw_jobs.fetch_add(1);
      mask[1] = false;
      mask[2] = false;
    }
    if (mask[2] && !mask[1]) {
      ScopedCount sc("hip_conv2d.bias_grad.run");
      gb = empty_xdna({g.Cout}, at::kBFloat16);
      check_abi(xdna_conv3x3_bias_grad_bf16(static_cast<const uint16_t*>(d.const_data_ptr()),
                                            static_cast<uint16_t*>(gb.data_ptr()), g.B, g.Cout, g.Ho, g.Wo,
                                            current_stream()),
                "conv2d bias grad");
      mask[2] = false;
    }
  }
  if (mask[0] || mask[1] || mask[2]) {
    ScopedCount sc("aten::convolution_backward.rocm");
    BelowAutograd g;
    std::vector<c10::SymInt> bias_sizes;
    std::optional<c10::SymIntArrayRef> bs;
    if (mask[2]) {
      bias_sizes.push_back(transposed ? weight.sym_size(1) * groups : weight.sym_size(0));
      bs = c10::SymIntArrayRef(bias_sizes);
    }
    auto r = at::_ops::convolution_backward::call(rocm(grad_output), rocm(input), rocm(weight), bs,
                                                  stride, padding, dilation, transposed,
                                                  output_padding, groups, mask);
    if (mask[0]) gi = back(std::get<0>(r));
    if (mask[1]) gw = back(std::get<1>(r));
    if (mask[2]) gb = back(std::get<2>(r));
  }
  return {gi, gw, gb};
}

// ---------------------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------------------
bool gemm_dtype_ok(std::initializer_list<const at::Tensor*> ts) {
  if (g_mode.load() < 1) return false;
  for (const at::Tensor* t : ts)
    if (t->scalar_type() != at::kBFloat16 || t->device().type() != kXdna) return false;
  return true;
}

bool fits_int(const at::Tensor& t) {
  for (int64_t s : t.sizes())
    if (s > (int64_t(1) << 30)) return false;
  return true;
}

// c[b] = alpha * a[b].m[b] + beta * bias  (bias: an [M][N] view, may be broadcast)
void run_gemm(const at::Tensor& a, const at::Tensor& m, at::Tensor& c, const at::Tensor* bias,
              float alpha, float beta) {
  const bool batched = a.dim() == 3;
  const int64_t batch = batched ? a.size(0) : 1;
  const int ia = batched ? 1 : 0;
  const int64_t M = a.size(ia), K = a.size(ia + 1), N = m.size(ia + 1);
  const uint16_t* bp = nullptr;
  int mode = 0;
  int64_t bsm = 0, bsn = 0;
  at::Tensor be;
  if (bias && beta != 0.0f) {
    be = bias->expand({M, N});
    bp = static_cast<const uint16_t*>(be.const_data_ptr());
    bsm = be.stride(0);
    bsn = be.stride(1);
    // a bias broadcast over rows (Linear's [N] vector) or over columns is read once per
    // column / row in the epilogue rather than once per element
    mode = bsm == 0 ? 1 : (bsn == 0 ? 3 : 2);
  }
  KernelTimer kt("gemm", 2.0 * double(batch) * double(M) * double(N) * double(K));
  check_abi(xdna_gemm_bf16(static_cast<const uint16_t*>(a.const_data_ptr()),
                           static_cast<const uint16_t*>(m.const_data_ptr()),
                           static_cast<uint16_t*>(c.data_ptr()), bp, int(batch), int(M), int(N), int(K),
                           a.stride(ia), a.stride(ia + 1), batched ? a.stride(0) : 0, m.stride(ia),
                           m.stride(ia + 1), batched ? m.stride(0) : 0, c.stride(ia), c.stride(ia + 1),
                           batched ? c.stride(0) : 0, mode, bsm, bsn, alpha, beta, current_stream()),
            "gemm");
}

at::Tensor mm_xdna(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2, "mm: expected 2-D tensors");
  TORCH_CHECK(a.size(1) == b.size(0), "mm: mat1 and mat2 shapes cannot be multiplied (",
              a.size(0), "x", a.size(1), " and ", b.size(0), "x", b.size(1), ")");
  if (gemm_dtype_ok({&a, &b}) && fits_int(a) && fits_int(b)) {
    ScopedCount sc("hip_gemm.mm.run");
    at::Tensor c = empty_xdna({a.size(0), b.size(1)}, at::kBFloat16);
    run_gemm(a, b, c, nullptr, 1.0f, 0.0f);
    return c;
  }
  ScopedCount sc("aten::mm.rocm");
  BelowAutograd g;
  return back(at::_ops::mm::call(rocm(a), rocm(b)));
}

// Whether an out= argument can take the product directly: an xdna bf16 tensor (already
// resized to the result's shape) with no internal overlap and no memory shared with any
// operand.  Otherwise the product goes to a new tensor and is copied (the reference's
// prepare_out_xdna / copy, torch_xdna_device.cpp:3500-3524).
// Whether `out` and an operand use the same allocation (conservative: any overlap of
// storages, whatever the strides).
bool shares_memory(const at::Tensor& out, std::initializer_list<const at::Tensor*> operands) {
  if (!out.has_storage() || out.storage().nbytes() == 0) return false;
  for (const at::Tensor* t : operands)
    if (t->defined() && t->has_storage() && t->storage().data() == out.storage().data()) return true;
  return false;
}

bool out_direct_ok(const at::Tensor& out, std::initializer_list<const at::Tensor*> operands) {
  if (out.device().type() != kXdna || out.scalar_type() != at::kBFloat16 || !fits_int(out)) return false;
  if (at::has_internal_overlap(out) != at::MemOverlap::No) return false;
  return !shares_memory(out, operands);
}

at::Tensor& mm_out_xdna(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2, "mm: expected 2-D tensors");
  TORCH_CHECK(a.size(1) == b.size(0), "mm: mat1 and mat2 shapes cannot be multiplied (",
              a.size(0), "x", a.size(1), " and ", b.size(0), "x", b.size(1), ")");
  // operands are checked for shared memory before the resize, which could move it
  if (gemm_dtype_ok({&a, &b}) && fits_int(a) && fits_int(b) && !shares_memory(out, {&a, &b})) {
    at::native::resize_output(out, {a.size(0), b.size(1)});
    if (out_direct_ok(out, {&a, &b})) {
      ScopedCount sc("hip_gemm.mm_out.run");
      run_gemm(a, b, out, nullptr, 1.0f, 0.0f);
      bump_write_epoch(out);
      return out;
    }
  }
  at::Tensor r = mm_xdna(a, b);
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

at::Tensor addmm_xdna(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b,
                      const at::Scalar& beta, const at::Scalar& alpha) {
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2, "addmm: expected 2-D matrices");
  TORCH_CHECK(a.size(1) == b.size(0), "addmm: mat1 and mat2 shapes cannot be multiplied (",
              a.size(0), "x", a.size(1), " and ", b.size(0), "x", b.size(1), ")");
  const int64_t M = a.size(0), N = b.size(1);
  const bool self_ok = self.dim() <= 2 && self.scalar_type() == at::kBFloat16 &&
                       self.device().type() == kXdna && at::is_expandable_to(self.sizes(), {M, N});
  if (gemm_dtype_ok({&a, &b}) && self_ok && fits_int(a) && fits_int(b)) {
    ScopedCount sc("hip_gemm.addmm.run");
    at::Tensor c = empty_xdna({M, N}, at::kBFloat16);
    run_gemm(a, b, c, &self, alpha.to<float>(), beta.to<float>());
    return c;
  }
  ScopedCount sc("aten::addmm.rocm");
  BelowAutograd g;
  return back(at::_ops::addmm::call(rocm(self), rocm(a), rocm(b), beta, alpha));
}

at::Tensor& addmm_out_xdna(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b,
                           const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2, "addmm: expected 2-D matrices");
  TORCH_CHECK(a.size(1) == b.size(0), "addmm: mat1 and mat2 shapes cannot be multiplied (",
              a.size(0), "x", a.size(1), " and ", b.size(0), "x", b.size(1), ")");
  const int64_t M = a.size(0), N = b.size(1);
  const bool self_ok = self.dim() <= 2 && self.scalar_type() == at::kBFloat16 &&
                       self.device().type() == kXdna && at::is_expandable_to(self.sizes(), {M, N});
  // out sharing memory with an operand (self included: out = self is common) takes the
  // copy path; checked before the resize, which could move that memory
  if (gemm_dtype_ok({&a, &b}) && self_ok && fits_int(a) && fits_int(b) && !shares_memory(out, {&a, &b, &self})) {
    at::native::resize_output(out, {M, N});
    if (out_direct_ok(out, {&a, &b, &self})) {
      ScopedCount sc("hip_gemm.addmm_out.run");
      run_gemm(a, b, out, &self, alpha.to<float>(), beta.to<float>());
      bump_write_epoch(out);
      return out;
    }
  }
  at::Tensor r = addmm_xdna(self, a, b, beta, alpha);
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

at::Tensor bmm_xdna(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(a.dim() == 3 && b.dim() == 3, "batch1 and batch2 must be 3D tensors");
  TORCH_CHECK(a.size(0) == b.size(0) && a.size(2) == b.size(1), "bmm: shape mismatch");
  if (gemm_dtype_ok({&a, &b}) && fits_int(a) && fits_int(b) && a.size(0) <= 65535) {
    ScopedCount sc("hip_gemm.bmm.run");
    at::Tensor c = empty_xdna({a.size(0), a.size(1), b.size(2)}, at::kBFloat16);
    run_gemm(a, b, c, nullptr, 1.0f, 0.0f);
    return c;
  }
  ScopedCount sc("aten::bmm.rocm");
  BelowAutograd g;
  return back(at::_ops::bmm::call(rocm(a), rocm(b)));
}

at::Tensor& bmm_out_xdna(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  TORCH_CHECK(a.dim() == 3 && b.dim() == 3, "batch1 and batch2 must be 3D tensors");
  TORCH_CHECK(a.size(0) == b.size(0) && a.size(2) == b.size(1), "bmm: shape mismatch");
  if (gemm_dtype_ok({&a, &b}) && fits_int(a) && fits_int(b) && a.size(0) <= 65535 && !shares_memory(out, {&a, &b})) {
    at::native::resize_output(out, {a.size(0), a.size(1), b.size(2)});
    if (out_direct_ok(out, {&a, &b})) {
      ScopedCount sc("hip_gemm.bmm_out.run");
      run_gemm(a, b, out, nullptr, 1.0f, 0.0f);
      bump_write_epoch(out);
      return out;
    }
  }
  at::Tensor r = bmm_xdna(a, b);
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

// ---------------------------------------------------------------------------------------
// Fused Adam / AdamW (PyTorch's _fused_adam_ schema; the reference runs the CPU kernel
// of this op through its fallback).
// ---------------------------------------------------------------------------------------
bool adam_eligible(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                   at::TensorList mx, at::TensorList steps, bool amsgrad, int& dtype) {
  if (g_mode.load() < 1 || p.empty()) return false;
  const auto st = p[0].scalar_type();
  if (st != at::kBFloat16 && st != at::kFloat) return false;
  dtype = st == at::kBFloat16 ? 1 : 0;
  if (g.size() != p.size() || m.size() != p.size() || v.size() != p.size() ||
      steps.size() != p.size() || (amsgrad && mx.size() != p.size()))
    return false;
  auto ok = [&](const at::Tensor& t, int64_t n) {
    return t.defined() && t.device().type() == kXdna && t.scalar_type() == st && t.is_contiguous() &&
           t.numel() == n;
  };
  for (size_t i = 0; i < p.size(); ++i) {
    const int64_t n = p[i].numel();
    if (!ok(p[i], n) || !ok(g[i], n) || !ok(m[i], n) || !ok(v[i], n)) return false;
    if (amsgrad && !ok(mx[i], n)) return false;
    const at::Tensor& s = steps[i];
    if (s.device().type() != kXdna || s.scalar_type() != at::kFloat || s.numel() != 1) return false;
  }
  return true;
}

std::vector<at::Tensor> rocm_list(at::TensorList l) {
  std::vector<at::Tensor> out;
  out.reserve(l.size());
  for (const auto& t : l) out.push_back(rocm(t));
  return out;
}

// The lists a fused step writes: parameters, moments (max_exp_avg_sqs with amsgrad) and,
// with a grad scale, the unscaled gradients.
void bump_adam_epochs(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                      at::TensorList mx, bool amsgrad, bool grads_written) {
  for (const at::TensorList& l : {p, m, v})
    for (const auto& t : l) bump_write_epoch(t);
  if (amsgrad)
    for (const auto& t : mx) bump_write_epoch(t);
  if (grads_written)
    for (const auto& t : g) bump_write_epoch(t);
}

// lr is a host double, or a device scalar (`lr_t`, the tensor-lr overloads) read by the
// kernel, so no host synchronization happens and the step can be captured.
void fused_adam_common(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                       at::TensorList mx, at::TensorList steps, double lr, const at::Tensor* lr_t,
                       double beta1, double beta2, double wd, double eps, bool amsgrad, bool maximize,
                       const std::optional<at::Tensor>& grad_scale,
                       const std::optional<at::Tensor>& found_inf, bool adamw) {
  int dtype = 1;
  const bool scalars_ok =
      (!grad_scale || (grad_scale->device().type() == kXdna && grad_scale->scalar_type() == at::kFloat)) &&
      (!found_inf || (found_inf->device().type() == kXdna && found_inf->scalar_type() == at::kFloat));
  const bool lr_ok = !lr_t || (lr_t->device().type() == kXdna && lr_t->numel() == 1 &&
                               (lr_t->scalar_type() == at::kFloat || lr_t->scalar_type() == at::kDouble));
  bump_adam_epochs(p, g, m, v, mx, amsgrad, grad_scale.has_value());
  if (scalars_ok && lr_ok && adam_eligible(p, g, m, v, mx, steps, amsgrad, dtype)) {
    ScopedCount sc(adamw ? "hip_adamw.run" : "hip_adam.run");
    const size_t n = p.size();
    std::vector<void*> pp(n), gp(n), mp(n), vp(n), xp(n);
    std::vector<const float*> sp(n);
    std::vector<int64_t> numel(n);
    for (size_t i = 0; i < n; ++i) {
      pp[i] = p[i].data_ptr();
      gp[i] = g[i].data_ptr();
      mp[i] = m[i].data_ptr();
      vp[i] = v[i].data_ptr();
      xp[i] = amsgrad ? mx[i].data_ptr() : nullptr;
      sp[i] = static_cast<const float*>(steps[i].const_data_ptr());
      numel[i] = p[i].numel();
    }
    double bytes = 0.0;
    for (size_t i = 0; i < n; ++i)
      bytes += double(numel[i]) * double(p[i].element_size()) * (amsgrad ? 9.0 : 7.0);
    KernelTimer kt("fused_adam", bytes);
    const float* gsp = grad_scale ? static_cast<const float*>(grad_scale->const_data_ptr()) : nullptr;
    const float* fip = found_inf ? static_cast<const float*>(found_inf->const_data_ptr()) : nullptr;
    if (lr_t)
      check_abi(xdna_fused_adam_tensor_lr(int(n), pp.data(), gp.data(), mp.data(), vp.data(),
                                          amsgrad ? xp.data() : nullptr, sp.data(), numel.data(), dtype,
                                          lr_t->const_data_ptr(), lr_t->scalar_type() == at::kFloat ? 1 : 2,
                                          beta1, beta2, wd, eps, amsgrad ? 1 : 0, maximize ? 1 : 0,
                                          adamw ? 1 : 0, gsp, fip, current_stream()),
                "fused adam (tensor lr)");
    else
      check_abi(xdna_fused_adam(int(n), pp.data(), gp.data(), mp.data(), vp.data(),
                                amsgrad ? xp.data() : nullptr, sp.data(), numel.data(), dtype, lr, beta1,
                                beta2, wd, eps, amsgrad ? 1 : 0, maximize ? 1 : 0, adamw ? 1 : 0, gsp, fip,
                                current_stream()),
                "fused adam");
    refresh_conv_forms(p);
    return;
  }
  ScopedCount sc("aten::_fused_adam_.rocm");
  BelowAutograd guard;
  auto rp = rocm_list(p), rg = rocm_list(g), rm = rocm_list(m), rv = rocm_list(v), rx = rocm_list(mx),
       rs = rocm_list(steps);
  if (lr_t && adamw)
    at::_ops::_fused_adamw__tensor_lr::call(rp, rg, rm, rv, rx, rs, rocm(*lr_t), beta1, beta2, wd, eps, amsgrad,
                                            maximize, rocm(grad_scale), rocm(found_inf));
  else if (lr_t)
    at::_ops::_fused_adam__tensor_lr::call(rp, rg, rm, rv, rx, rs, rocm(*lr_t), beta1, beta2, wd, eps, amsgrad,
                                           maximize, rocm(grad_scale), rocm(found_inf));
  else if (adamw)
    at::_ops::_fused_adamw_::call(rp, rg, rm, rv, rx, rs, lr, beta1, beta2, wd, eps, amsgrad, maximize,
                                  rocm(grad_scale), rocm(found_inf));
  else
    at::_ops::_fused_adam_::call(rp, rg, rm, rv, rx, rs, lr, beta1, beta2, wd, eps, amsgrad, maximize,
                                 rocm(grad_scale), rocm(found_inf));
}

void fused_adam_xdna(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                     at::TensorList mx, at::TensorList steps, double lr, double beta1, double beta2,
                     double wd, double eps, bool amsgrad, bool maximize,
                     const std::optional<at::Tensor>& grad_scale,
                     const std::optional<at::Tensor>& found_inf) {
  fused_adam_common(p, g, m, v, mx, steps, lr, nullptr, beta1, beta2, wd, eps, amsgrad, maximize, grad_scale,
                    found_inf, false);
}

void fused_adamw_xdna(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                      at::TensorList mx, at::TensorList steps, double lr, double beta1, double beta2,
                      double wd, double eps, bool amsgrad, bool maximize,
                      const std::optional<at::Tensor>& grad_scale,
                      const std::optional<at::Tensor>& found_inf) {
  fused_adam_common(p, g, m, v, mx, steps, lr, nullptr, beta1, beta2, wd, eps, amsgrad, maximize, grad_scale,
                    found_inf, true);
}

// torch._foreach_add_(state_steps, 1) before every fused Adam step: one HIP launch for
// the whole list of fp32 xdna tensors; other forms go to PyTorch-ROCm on aliases.
void foreach_add_scalar_xdna(at::TensorList self, const at::Scalar& scalar) {
  for (const auto& t : self) bump_write_epoch(t);
  bool ok = g_mode.load() >= 1 && !scalar.isComplex();
  for (const auto& t : self)
    ok = ok && t.defined() && t.device().type() == kXdna && t.scalar_type() == at::kFloat && t.is_contiguous();
  if (ok) {
    ScopedCount sc("hip_foreach_add.run");
    std::vector<float*> ptrs(self.size());
    std::vector<int64_t> numels(self.size());
    for (size_t i = 0; i < self.size(); ++i) {
      ptrs[i] = self[i].data_ptr<float>();
      numels[i] = self[i].numel();
    }
    check_abi(xdna_foreach_add_scalar_f32(int(self.size()), ptrs.data(), numels.data(), scalar.toFloat(),
                                          current_stream()),
              "foreach add");
    return;
  }
  ScopedCount sc("aten::_foreach_add_.rocm");
  BelowAutograd g;
  at::_ops::_foreach_add__Scalar::call(rocm_list(self), scalar);
}

void fused_adam_tlr_xdna(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                         at::TensorList mx, at::TensorList steps, const at::Tensor& lr, double beta1,
                         double beta2, double wd, double eps, bool amsgrad, bool maximize,
                         const std::optional<at::Tensor>& grad_scale,
                         const std::optional<at::Tensor>& found_inf) {
  fused_adam_common(p, g, m, v, mx, steps, 0.0, &lr, beta1, beta2, wd, eps, amsgrad, maximize, grad_scale,
                    found_inf, false);
}

void fused_adamw_tlr_xdna(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v,
                          at::TensorList mx, at::TensorList steps, const at::Tensor& lr, double beta1,
                          double beta2, double wd, double eps, bool amsgrad, bool maximize,
                          const std::optional<at::Tensor>& grad_scale,
                          const std::optional<at::Tensor>& found_inf) {
  fused_adam_common(p, g, m, v, mx, steps, 0.0, &lr, beta1, beta2, wd, eps, amsgrad, maximize, grad_scale,
                    found_inf, true);
}

struct TimedLaunch {
  std::string name;
  void* start;
  void* stop;
  double work;
};
std::mutex g_kt_mu;
std::atomic<bool> g_kt_on{false};
std::vector<TimedLaunch>& timed() {
  static auto* v = new std::vector<TimedLaunch>();
  return *v;
}
// Events are created when timing is switched on, not per launch: creating two events per
// launch costs the host more than the small launches take on the GPU.  They live until
// the process ends and are reused by the next timing session; launches past the pool's
// end are not timed.
constexpr size_t kTimingEvents = 16384;
std::vector<void*>& event_pool() {
  static auto* v = new std::vector<void*>();
  return *v;
}
size_t g_pool_next = 0;

}  // namespace

KernelTimer::KernelTimer(const char* n, double w) : name(n), work(w) {
  if (!g_kt_on.load(std::memory_order_relaxed)) return;
  {
    std::lock_guard<std::mutex> lock(g_kt_mu);
    if (g_pool_next + 2 > event_pool().size()) return;
    start = event_pool()[g_pool_next];
    stop = event_pool()[g_pool_next + 1];
    g_pool_next += 2;
  }
  xdna_hip_event_record(start, current_stream());
}

KernelTimer::~KernelTimer() {
  if (!start || !stop) return;
  xdna_hip_event_record(stop, current_stream());
  std::lock_guard<std::mutex> lock(g_kt_mu);
  timed().push_back({name, start, stop, work});
}

void kernel_timing_enable(bool on) {
  std::lock_guard<std::mutex> lock(g_kt_mu);
  auto& pool = event_pool();
  while (on && pool.size() < kTimingEvents) {
    void* e = xdna_hip_event_create(1);
    if (!e) break;
    pool.push_back(e);
  }
  timed().clear();
  g_pool_next = 0;
  g_kt_on.store(on);
}

std::vector<std::tuple<std::string, int64_t, double, double>> kernel_timing_report() {
  check_abi(xdna_hip_device_synchronize(), "kernel timing");
  std::map<std::string, std::tuple<int64_t, double, double>> acc;
  std::lock_guard<std::mutex> lock(g_kt_mu);
  for (const auto& t : timed()) {
    float ms = 0.0f;
    if (xdna_hip_event_elapsed_ms(t.start, t.stop, &ms) != 0) continue;
    auto& a = acc[t.name];
    std::get<0>(a) += 1;
    std::get<1>(a) += ms;
    std::get<2>(a) += t.work;
  }
  std::vector<std::tuple<std::string, int64_t, double, double>> out;
  for (const auto& [k, v] : acc) out.emplace_back(k, std::get<0>(v), std::get<1>(v), std::get<2>(v));
  return out;
}

int64_t dw_jobs() { return g_dw_jobs.load(); }

// ---------------------------------------------------------------------------------------
// Batch norm in training mode without running statistics: the form instance_norm takes
// ([B, C, H, W] viewed as [1, B*C, H, W]).  The reference runs it on the CPU through the
// zero-copy fallback (torch_xdna_device.cpp:5124-5260); here one HIP kernel per direction.
// Other forms (running statistics, eval mode, very long channels) use PyTorch-ROCm.
// ---------------------------------------------------------------------------------------
constexpr int64_t kNormMaxPerChannel = 65536;  // one wave per channel up to this many elements

int norm_param_dtype(const std::optional<at::Tensor>& w, const std::optional<at::Tensor>& b) {
  const bool hw = w && w->defined(), hb = b && b->defined();
  if (!hw && !hb) return 0;
  const at::ScalarType t = hw ? w->scalar_type() : b->scalar_type();
  if (hw && hb && w->scalar_type() != b->scalar_type()) return -1;
  return t == at::kBFloat16 ? 1 : t == at::kFloat ? 2 : -1;
}

bool norm_param_ok(const std::optional<at::Tensor>& t, int64_t C) {
  return !t || !t->defined() ||
         (t->dim() == 1 && t->size(0) == C && t->is_contiguous() && t->device().type() == kXdna);
}

bool norm_eligible(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                   const std::optional<at::Tensor>& bias, const std::optional<at::Tensor>& rm,
                   const std::optional<at::Tensor>& rv, bool training) {
  if (g_mode.load() < 1 || !training) return false;
  if ((rm && rm->defined()) || (rv && rv->defined())) return false;
  if (input.scalar_type() != at::kBFloat16 || input.dim() < 2 || input.device().type() != kXdna) return false;
  const int64_t C = input.size(1);
  if (C < 1 || input.numel() == 0 || input.numel() / C > kNormMaxPerChannel) return false;
  return norm_param_dtype(weight, bias) >= 0 && norm_param_ok(weight, C) && norm_param_ok(bias, C);
}

// Training-mode batch norm of conv activations with the spatial kernels (bnorm.hip): any
// channel length, running statistics (bf16 or fp32, both or neither) updated in the same
// launch pair.
int running_stats_dtype(const std::optional<at::Tensor>& rm, const std::optional<at::Tensor>& rv, int64_t C) {
  const bool hm = rm && rm->defined(), hv = rv && rv->defined();
  if (!hm && !hv) return 0;
  if (hm != hv || rm->scalar_type() != rv->scalar_type()) return -1;
  for (const at::Tensor* t : {&*rm, &*rv})
    if (t->dim() != 1 || t->size(0) != C || !t->is_contiguous() || t->device().type() != kXdna) return -1;
  return rm->scalar_type() == at::kBFloat16 ? 1 : rm->scalar_type() == at::kFloat ? 2 : -1;
}

bool bn_train_eligible(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                       const std::optional<at::Tensor>& bias, bool training) {
  if (g_mode.load() < 1 || !training) return false;
  if (input.scalar_type() != at::kBFloat16 || input.dim() < 2 || input.device().type() != kXdna) return false;
  const int64_t C = input.size(1);
  if (C < 1 || input.numel() == 0 || input.size(0) < 1) return false;
  return norm_param_dtype(weight, bias) >= 0 && norm_param_ok(weight, C) && norm_param_ok(bias, C);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_batch_norm_xdna(
    const at::Tensor& input, const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& bias,
    const std::optional<at::Tensor>& running_mean, const std::optional<at::Tensor>& running_var, bool training,
    double momentum, double eps) {
  const int rsd = input.dim() >= 2 ? running_stats_dtype(running_mean, running_var, input.size(1)) : -1;
  if (rsd >= 0 && bn_train_eligible(input, weight, bias, training) &&
      (rsd > 0 || input.numel() / input.size(1) > kNormMaxPerChannel)) {
    ScopedCount sc("hip_batch_norm_train.fwd.run");
    const at::Tensor x = input.contiguous();
    const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
    const int wd = norm_param_dtype(weight, bias);
    at::Tensor y = empty_xdna(x.sizes(), at::kBFloat16);
    at::Tensor mean = empty_xdna({C}, at::kFloat), invstd = empty_xdna({C}, at::kFloat);
    check_abi(xdna_batch_norm_train_fwd_bf16(
                  static_cast<const uint16_t*>(x.const_data_ptr()),
                  weight && weight->defined() ? weight->const_data_ptr() : nullptr,
                  bias && bias->defined() ? bias->const_data_ptr() : nullptr, wd,
                  rsd ? running_mean->data_ptr() : nullptr, rsd ? running_var->data_ptr() : nullptr, rsd, momentum,
                  eps, static_cast<uint16_t*>(y.data_ptr()), mean.data_ptr<float>(), invstd.data_ptr<float>(), N, C,
                  L, current_stream()),
              "batch_norm fwd (training)");
    if (rsd) {
      bump_write_epoch(*running_mean);
      bump_write_epoch(*running_var);
    }
    return {y, mean, invstd};
  }
  if (norm_eligible(input, weight, bias, running_mean, running_var, training)) {
    ScopedCount sc("hip_batch_norm.fwd.run");
    const at::Tensor x = input.contiguous();
    const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
    const int wd = norm_param_dtype(weight, bias);
    at::Tensor y = empty_xdna(x.sizes(), at::kBFloat16);
    at::Tensor mean = empty_xdna({C}, at::kFloat), invstd = empty_xdna({C}, at::kFloat);
    check_abi(xdna_batch_norm_fwd_bf16(
                  static_cast<const uint16_t*>(x.const_data_ptr()),
                  weight && weight->defined() ? weight->const_data_ptr() : nullptr,
                  bias && bias->defined() ? bias->const_data_ptr() : nullptr, wd,
                  static_cast<uint16_t*>(y.data_ptr()), mean.data_ptr<float>(), invstd.data_ptr<float>(), N, C, L,
                  eps, current_stream()),
              "batch_norm fwd");
    return {y, mean, invstd};
  }
  ScopedCount sc("aten::native_batch_norm.rocm");
  BelowAutograd g;
  auto r = at::_ops::native_batch_norm::call(rocm(input), rocm(weight), rocm(bias), rocm(running_mean),
                                             rocm(running_var), training, momentum, eps);
  return {back(std::get<0>(r)), back(std::get<1>(r)), back(std::get<2>(r))};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_batch_norm_backward_xdna(
    const at::Tensor& grad_out, const at::Tensor& input, const std::optional<at::Tensor>& weight,
    const std::optional<at::Tensor>& running_mean, const std::optional<at::Tensor>& running_var,
    const std::optional<at::Tensor>& save_mean, const std::optional<at::Tensor>& save_invstd, bool train,
    double eps, std::array<bool, 3> mask) {
  const bool stats_ok = save_mean && save_mean->defined() && save_invstd && save_invstd->defined() &&
                        save_mean->scalar_type() == at::kFloat && save_invstd->scalar_type() == at::kFloat &&
                        save_mean->is_contiguous() && save_invstd->is_contiguous() &&
                        save_mean->device().type() == kXdna && save_invstd->device().type() == kXdna;
  const bool param_grads_ok = !(mask[1] || mask[2]) || (weight && weight->defined());
  // long channels or running statistics (which the backward does not use): the spatial kernels
  if (stats_ok && param_grads_ok && bn_train_eligible(input, weight, std::nullopt, train) &&
      grad_out.scalar_type() == at::kBFloat16 && grad_out.sizes() == input.sizes() &&
      grad_out.device().type() == kXdna && save_mean->numel() == input.size(1) &&
      save_invstd->numel() == input.size(1) &&
      (input.numel() / input.size(1) > kNormMaxPerChannel || (running_mean && running_mean->defined()))) {
    ScopedCount sc("hip_batch_norm_train.bwd.run");
    const at::Tensor x = input.contiguous(), dy = grad_out.contiguous();
    const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
    const int wd = norm_param_dtype(weight, std::nullopt);
    at::Tensor dx, dw, db;
    if (mask[0]) dx = empty_xdna(x.sizes(), at::kBFloat16);
    const at::ScalarType pt = wd == 2 ? at::kFloat : at::kBFloat16;
    if (mask[1]) dw = empty_xdna({C}, pt);
    if (mask[2]) db = empty_xdna({C}, pt);
    check_abi(xdna_batch_norm_train_bwd_bf16(
                  static_cast<const uint16_t*>(dy.const_data_ptr()), static_cast<const uint16_t*>(x.const_data_ptr()),
                  weight && weight->defined() ? weight->const_data_ptr() : nullptr, wd,
                  save_mean->const_data_ptr<float>(), save_invstd->const_data_ptr<float>(),
                  mask[0] ? static_cast<uint16_t*>(dx.data_ptr()) : nullptr, mask[1] ? dw.data_ptr() : nullptr,
                  mask[2] ? db.data_ptr() : nullptr, N, C, L, current_stream()),
              "batch_norm bwd (training)");
    return {dx, dw, db};
  }
  if (stats_ok && param_grads_ok && norm_eligible(input, weight, std::nullopt, running_mean, running_var, train) &&
      grad_out.scalar_type() == at::kBFloat16 && grad_out.sizes() == input.sizes() &&
      grad_out.device().type() == kXdna && save_mean->numel() == input.size(1) &&
      save_invstd->numel() == input.size(1)) {
    ScopedCount sc("hip_batch_norm.bwd.run");
    const at::Tensor x = input.contiguous(), dy = grad_out.contiguous();
    const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
    const int wd = norm_param_dtype(weight, std::nullopt);
    at::Tensor dx, dw, db;
    if (mask[0]) dx = empty_xdna(x.sizes(), at::kBFloat16);
    const at::ScalarType pt = wd == 2 ? at::kFloat : at::kBFloat16;
    if (mask[1]) dw = empty_xdna({C}, pt);
    if (mask[2]) db = empty_xdna({C}, pt);
    check_abi(xdna_batch_norm_bwd_bf16(
                  static_cast<const uint16_t*>(dy.const_data_ptr()), static_cast<const uint16_t*>(x.const_data_ptr()),
                  weight && weight->defined() ? weight->const_data_ptr() : nullptr, wd,
                  save_mean->const_data_ptr<float>(), save_invstd->const_data_ptr<float>(),
                  mask[0] ? static_cast<uint16_t*>(dx.data_ptr()) : nullptr, mask[1] ? dw.data_ptr() : nullptr,
                  mask[2] ? db.data_ptr() : nullptr, N, C, L, current_stream()),
              "batch_norm bwd");
    return {dx, dw, db};
  }
  ScopedCount sc("aten::native_batch_norm_backward.rocm");
  BelowAutograd g;
  auto r = at::_ops::native_batch_norm_backward::call(rocm(grad_out), rocm(input), rocm(weight),
                                                      rocm(running_mean), rocm(running_var), rocm(save_mean),
                                                      rocm(save_invstd), train, eps, mask);
  return {back(std::get<0>(r)), back(std::get<1>(r)), back(std::get<2>(r))};
}

// ---------------------------------------------------------------------------------------
// instance_norm with training statistics, registered for AutogradPrivateUse1 so that it
// replaces PyTorch's composite (repeat of weight and bias to B*C elements, batch norm on
// [1, B*C, L], and the sums over the images the repeat's backward runs): one kernel
// forward, a kernel plus a parameter-gradient reduce backward.  Other forms (no affine
// parameters or a lone one, running or eval statistics, non-bf16 input) keep the
// composite, whose native_batch_norm calls reach the batch-norm kernels above.
// The reference reaches the same operator through its CPU fallback
// (torch_xdna_device.cpp:5124-5260).
// ---------------------------------------------------------------------------------------
bool instance_norm_eligible(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                            const std::optional<at::Tensor>& bias, const std::optional<at::Tensor>& rm,
                            const std::optional<at::Tensor>& rv, bool use_input_stats) {
  if (g_mode.load() < 1 || !use_input_stats) return false;
  if ((rm && rm->defined()) || (rv && rv->defined())) return false;
  if (input.scalar_type() != at::kBFloat16 || input.dim() < 3 || input.device().type() != kXdna) return false;
  if (input.numel() == 0) return false;
  const int64_t C = input.size(1), L = input.numel() / (input.size(0) * C);
  if (L > kNormMaxPerChannel) return false;
  // affine only: without parameters the composite adds no work around the batch norm
  if (!weight || !weight->defined() || !bias || !bias->defined()) return false;
  if (weight->requires_grad() != bias->requires_grad()) return false;
  return norm_param_dtype(weight, bias) >= 0 && norm_param_ok(weight, C) && norm_param_ok(bias, C);
}

struct InstanceNormFn : public torch::autograd::Function<InstanceNormFn> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& input,
                            const at::Tensor& weight, const at::Tensor& bias, double eps) {
    ScopedCount sc("hip_instance_norm.fwd.run");
    const at::Tensor x = input.contiguous();
    const int64_t B = x.size(0), C = x.size(1), L = x.numel() / (B * C);
    const int wd = norm_param_dtype(weight, bias);
    at::Tensor y = empty_xdna(x.sizes(), at::kBFloat16);
    at::Tensor mean = empty_xdna({B * C}, at::kFloat), invstd = empty_xdna({B * C}, at::kFloat);
    check_abi(xdna_instance_norm_fwd_bf16(
                  static_cast<const uint16_t*>(x.const_data_ptr()), weight.const_data_ptr(), bias.const_data_ptr(),
                  wd, static_cast<uint16_t*>(y.data_ptr()),
                  mean.data_ptr<float>(), invstd.data_ptr<float>(), B, C, L, eps, current_stream()),
              "instance_norm fwd");
    ctx->save_for_backward({x, weight, mean, invstd});
    ctx->saved_data["wd"] = int64_t(wd);
    return y;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor &x = saved[0], &weight = saved[1], &mean = saved[2], &invstd = saved[3];
    const int wd = int(ctx->saved_data["wd"].toInt());
    const bool need_x = ctx->needs_input_grad(0);
    const bool need_p = ctx->needs_input_grad(1) || ctx->needs_input_grad(2);
    at::Tensor dx, dw, db;
    if (!grads[0].defined() || (!need_x && !need_p)) return {dx, dw, db, at::Tensor()};
    ScopedCount sc("hip_instance_norm.bwd.run");
    const int64_t B = x.size(0), C = x.size(1), L = x.numel() / (B * C);
    at::Tensor dy = grads[0].to(at::kBFloat16).contiguous();
    if (need_x) dx = empty_xdna(x.sizes(), at::kBFloat16);
    if (need_p) {
      const at::ScalarType pt = wd == 2 ? at::kFloat : at::kBFloat16;
      dw = empty_xdna({C}, pt);
      db = empty_xdna({C}, pt);
    }
    check_abi(xdna_instance_norm_bwd_bf16(
                  static_cast<const uint16_t*>(dy.const_data_ptr()), static_cast<const uint16_t*>(x.const_data_ptr()),
                  weight.const_data_ptr(), wd, mean.const_data_ptr<float>(),
                  invstd.const_data_ptr<float>(), need_x ? static_cast<uint16_t*>(dx.data_ptr()) : nullptr,
                  need_p ? dw.data_ptr() : nullptr, need_p ? db.data_ptr() : nullptr, B, C, L, current_stream()),
              "instance_norm bwd");
    return {dx, dw, db, at::Tensor()};
  }
};

at::Tensor instance_norm_autograd_xdna(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                                       const std::optional<at::Tensor>& bias,
                                       const std::optional<at::Tensor>& running_mean,
                                       const std::optional<at::Tensor>& running_var, bool use_input_stats,
                                       double momentum, double eps, bool cudnn_enabled) {
  if (instance_norm_eligible(input, weight, bias, running_mean, running_var, use_input_stats)) {
    return InstanceNormFn::apply(input, *weight, *bias, eps);
  }
  return at::native::instance_norm(input, weight, bias, running_mean, running_var, use_input_stats, momentum,
                                   eps, cudnn_enabled);
}

// ---------------------------------------------------------------------------------------
// Nearest 2x upsampling (the style generator's decoder) and its gradient: one HIP kernel
// each for bf16 NCHW-contiguous tensors upsampled by exactly 2 (no scale, or scale 2);
// other forms run PyTorch-ROCm's kernels on aliases.  The reference runs both on its CPU
// through the fallback (torch_xdna_device.cpp:5124-5260).
// ---------------------------------------------------------------------------------------
bool nearest2x_ok(const at::Tensor& t, int64_t oh, int64_t ow, int64_t ih, int64_t iw,
                  std::optional<double> sh, std::optional<double> sw) {
  if (g_mode.load() < 1 || t.scalar_type() != at::kBFloat16 || t.dim() != 4 || t.device().type() != kXdna)
    return false;
  if (oh != 2 * ih || ow != 2 * iw || ih < 1 || iw < 1) return false;
  if ((sh && *sh != 2.0) || (sw && *sw != 2.0)) return false;
  return t.is_contiguous() && (reinterpret_cast<uintptr_t>(t.const_data_ptr()) & 3) == 0;
}

at::Tensor upsample_nearest2d_xdna(const at::Tensor& self, c10::SymIntArrayRef output_size,
                                   std::optional<double> scales_h, std::optional<double> scales_w) {
  if (output_size.size() == 2 && self.dim() == 4 &&
      nearest2x_ok(self, output_size[0].expect_int(), output_size[1].expect_int(), self.size(2), self.size(3),
                   scales_h, scales_w)) {
    ScopedCount sc("hip_upsample_nearest2x.fwd.run");
    const int64_t B = self.size(0), C = self.size(1), H = self.size(2), W = self.size(3);
    at::Tensor y = empty_xdna({B, C, 2 * H, 2 * W}, at::kBFloat16);
    check_abi(xdna_upsample_nearest2x_bf16(static_cast<const uint16_t*>(self.const_data_ptr()),
                                           static_cast<uint16_t*>(y.data_ptr()), B * C, int(H), int(W),
                                           current_stream()),
              "upsample_nearest2d");
    return y;
  }
  ScopedCount sc("aten::upsample_nearest2d.rocm");
  BelowAutograd g;
  return back(at::_ops::upsample_nearest2d::call(rocm(self), output_size, scales_h, scales_w));
}

at::Tensor upsample_nearest2d_backward_xdna(const at::Tensor& grad_output, c10::SymIntArrayRef output_size,
                                            c10::SymIntArrayRef input_size, std::optional<double> scales_h,
                                            std::optional<double> scales_w) {
  if (output_size.size() == 2 && input_size.size() == 4 && grad_output.dim() == 4) {
    const int64_t B = input_size[0].expect_int(), C = input_size[1].expect_int();
    const int64_t H = input_size[2].expect_int(), W = input_size[3].expect_int();
    const int64_t oh = output_size[0].expect_int(), ow = output_size[1].expect_int();
    if (grad_output.size(0) == B && grad_output.size(1) == C && grad_output.size(2) == oh &&
        grad_output.size(3) == ow && nearest2x_ok(grad_output, oh, ow, H, W, scales_h, scales_w)) {
      ScopedCount sc("hip_upsample_nearest2x.bwd.run");
      at::Tensor dx = empty_xdna({B, C, H, W}, at::kBFloat16);
      check_abi(xdna_upsample_nearest2x_bwd_bf16(static_cast<const uint16_t*>(grad_output.const_data_ptr()),
                                                 static_cast<uint16_t*>(dx.data_ptr()), B * C, int(H), int(W),
                                                 current_stream()),
                "upsample_nearest2d_backward");
      return dx;
    }
  }
  ScopedCount sc("aten::upsample_nearest2d_backward.rocm");
  BelowAutograd g;
  return back(at::_ops::upsample_nearest2d_backward::call(rocm(grad_output), output_size, input_size, scales_h,
                                                          scales_w));
}

// ---------------------------------------------------------------------------------------
// Losses and pooling of plain training scripts (the style step's content and Gram style
// terms, VGG's 2x2 pools): one HIP launch each way where PyTorch-ROCm takes two to four
// (fills, indices, separate reductions).  The reference runs all of them on its CPU
// through the fallback (torch_xdna_device.cpp:5124-5260).
// ---------------------------------------------------------------------------------------

// `t`'s row-major element i is the element i % period of the contiguous block at t's data
// pointer when its trailing dimensions are contiguous and its leading ones have stride 0
// (t = block.expand(...)); returns that period, or -1.
int64_t broadcast_period(const at::Tensor& t) {
  int64_t period = 1, k = t.dim();
  while (k > 0 && (t.size(k - 1) == 1 || t.stride(k - 1) == period)) {
    period *= t.size(k - 1);
    --k;
  }
  for (int64_t q = 0; q < k; ++q)
    if (t.size(q) != 1 && t.stride(q) != 0) return -1;
  return period;
}

int loss_dtype(at::ScalarType t) { return t == at::kFloat ? 1 : t == at::kBFloat16 ? 2 : 0; }

bool mse_eligible(const at::Tensor& self, const at::Tensor& target, int64_t reduction) {
  return g_mode.load() >= 1 && (reduction == 1 || reduction == 2) && self.device().type() == kXdna &&
         target.device().type() == kXdna && self.scalar_type() == target.scalar_type() &&
         loss_dtype(self.scalar_type()) != 0 && self.sizes() == target.sizes() && self.numel() > 0;
}

// b operand and its period: target itself when it is a batch-broadcast block, else a copy
std::pair<at::Tensor, int64_t> period_operand(const at::Tensor& target) {
  const int64_t p = broadcast_period(target);
  if (p > 0) return {target, p};
  at::Tensor b = target.contiguous();
  return {b, b.numel()};
}

at::Tensor mse_loss_xdna(const at::Tensor& self, const at::Tensor& target, int64_t reduction) {
  if (mse_eligible(self, target, reduction)) {
    ScopedCount sc("hip_mse_loss.fwd.run");
    const at::Tensor a = self.contiguous();
    const auto [b, period] = period_operand(target);
    const int64_t n = a.numel();
    at::Tensor out = empty_xdna({}, a.scalar_type());
    const size_t wb = xdna_mse_loss_workspace_bytes(n);
    at::Tensor ws = alloc_bytes(wb);
    check_abi(xdna_mse_loss(a.const_data_ptr(), b.const_data_ptr(), loss_dtype(a.scalar_type()), n, period,
                            int(reduction), out.data_ptr(), ws.data_ptr(), wb, current_stream()),
              "mse_loss");
    return out;
  }
  ScopedCount sc("aten::mse_loss.rocm");
  BelowAutograd g;
  return back(at::_ops::mse_loss::call(rocm(self), rocm(target), reduction));
}

at::Tensor mse_loss_backward_xdna(const at::Tensor& grad_output, const at::Tensor& self, const at::Tensor& target,
                                  int64_t reduction) {
  if (mse_eligible(self, target, reduction) && grad_output.numel() == 1 &&
      grad_output.device().type() == kXdna && loss_dtype(grad_output.scalar_type()) != 0) {
    ScopedCount sc("hip_mse_loss.bwd.run");
    const at::Tensor a = self.contiguous();
    const auto [b, period] = period_operand(target);
    const at::Tensor go = grad_output.contiguous();
    at::Tensor grad = empty_xdna(a.sizes(), a.scalar_type());
    check_abi(xdna_mse_loss_bwd(go.const_data_ptr(), loss_dtype(go.scalar_type()), a.const_data_ptr(),
                                b.const_data_ptr(), loss_dtype(a.scalar_type()), a.numel(), period, int(reduction),
                                grad.data_ptr(), current_stream()),
              "mse_loss_backward");
    return grad;
  }
  ScopedCount sc("aten::mse_loss_backward.rocm");
  BelowAutograd g;
  return back(at::_ops::mse_loss_backward::call(rocm(grad_output), rocm(self), rocm(target), reduction));
}

// Sum over the rows of a 2-D bf16 tensor (dim 0, the form autograd's sum_to takes for a
// Linear bias gradient): the fixed-order column sums of xdna_colsum_bf16.  Every other sum
// keeps PyTorch-ROCm's kernel through the aliases.
at::Tensor sum_dim_xdna(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                        std::optional<at::ScalarType> dtype) {
  const bool rows = dim.has_value() && dim->size() == 1 && ((*dim)[0] == 0 || (*dim)[0] == -2);
  if (g_mode.load() >= 1 && rows && self.dim() == 2 && self.scalar_type() == at::kBFloat16 &&
      (!dtype || *dtype == at::kBFloat16) && self.device().type() == kXdna && self.size(0) >= 1 &&
      self.size(1) >= 1) {
    ScopedCount sc("hip_colsum.run");
    const at::Tensor x = self.contiguous();
    const int64_t R = x.size(0), N = x.size(1);
    at::Tensor out = keepdim ? empty_xdna({1, N}, at::kBFloat16) : empty_xdna({N}, at::kBFloat16);
    const uint16_t* xp = static_cast<const uint16_t*>(x.const_data_ptr());
    const size_t wb = xdna_colsum_workspace_bytes(xp, R, N);
    at::Tensor ws = wb ? alloc_bytes(wb) : at::Tensor();
    check_abi(xdna_colsum_bf16(xp, static_cast<uint16_t*>(out.data_ptr()), R, N, wb ? ws.data_ptr() : nullptr, wb,
                               current_stream()),
              "sum over rows");
    return out;
  }
  ScopedCount sc("aten::sum.rocm");
  BelowAutograd g;
  return back(at::_ops::sum_dim_IntList::call(rocm(self), dim, keepdim, dtype));
}

// 2x2 / stride-2 max-pool (floor mode) of bf16 NCHW tensors as its own autograd node: the
// forward writes the pooled values only (no int64 indices), the backward routes each
// window's gradient to the window's maximum recomputed from the saved input (PyTorch's
// rule: the first maximum in row-major order, a NaN wins) and writes every input element,
// so no fill runs first.  Other pools keep PyTorch's composite.
bool pair_of(at::IntArrayRef v, int64_t x) {
  return (v.size() == 1 && v[0] == x) || (v.size() == 2 && v[0] == x && v[1] == x);
}

bool maxpool2_eligible(const at::Tensor& x, at::IntArrayRef kernel, at::IntArrayRef stride,
                       at::IntArrayRef padding, at::IntArrayRef dilation, bool ceil_mode) {
  if (g_mode.load() < 1 || ceil_mode || x.scalar_type() != at::kBFloat16 || x.dim() != 4) return false;
  if (x.device().type() != kXdna || x.size(2) < 2 || x.size(3) < 2 || x.numel() == 0) return false;
  return pair_of(kernel, 2) && (stride.empty() || pair_of(stride, 2)) && pair_of(padding, 0) &&
         pair_of(dilation, 1);
}

struct MaxPool2Fn : public torch::autograd::Function<MaxPool2Fn> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& input) {
    ScopedCount sc("hip_maxpool2.fwd.run");
    const at::Tensor x = input.contiguous();
    at::Tensor y = empty_xdna({x.size(0), x.size(1), x.size(2) / 2, x.size(3) / 2}, at::kBFloat16);
    check_abi(xdna_region_maxpool2_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                        static_cast<uint16_t*>(y.data_ptr()), x.size(0) * x.size(1),
                                        int(x.size(2)), int(x.size(3)), current_stream()),
              "max_pool2d");
    ctx->save_for_backward({x});
    return y;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const at::Tensor x = ctx->get_saved_variables()[0];
    if (!grads[0].defined()) return {at::Tensor()};
    ScopedCount sc("hip_maxpool2.bwd.run");
    const at::Tensor dy = grads[0].to(at::kBFloat16).contiguous();
    at::Tensor dx = empty_xdna(x.sizes(), at::kBFloat16);
    check_abi(xdna_region_backward_bf16(nullptr, nullptr, static_cast<const uint16_t*>(dy.const_data_ptr()),
                                        static_cast<const uint16_t*>(x.const_data_ptr()), nullptr, nullptr, nullptr,
                                        0.0f, nullptr, 0, static_cast<uint16_t*>(dx.data_ptr()),
                                        x.size(0) * x.size(1), int(x.size(2)), int(x.size(3)), current_stream()),
              "max_pool2d backward");
    return {dx};
  }
};

at::Tensor max_pool2d_autograd_xdna(const at::Tensor& self, at::IntArrayRef kernel_size, at::IntArrayRef stride,
                                    at::IntArrayRef padding, at::IntArrayRef dilation, bool ceil_mode) {
  if (maxpool2_eligible(self, kernel_size, stride, padding, dilation, ceil_mode)) return MaxPool2Fn::apply(self);
  return at::native::max_pool2d(self, kernel_size, stride, padding, dilation, ceil_mode);
}

void register_autograd_ops(torch::Library& m) {
  m.impl("instance_norm", TORCH_FN(instance_norm_autograd_xdna));
  m.impl("max_pool2d", TORCH_FN(max_pool2d_autograd_xdna));
}

void register_hot_ops(torch::Library& m) {
  m.impl("convolution_overrideable", TORCH_FN(convolution_overrideable_xdna));
  m.impl("convolution_backward_overrideable", TORCH_FN(convolution_backward_overrideable_xdna));
  m.impl("mm", TORCH_FN(mm_xdna));
  m.impl("mm.out", TORCH_FN(mm_out_xdna));
  m.impl("addmm", TORCH_FN(addmm_xdna));
  m.impl("addmm.out", TORCH_FN(addmm_out_xdna));
  m.impl("bmm", TORCH_FN(bmm_xdna));
  m.impl("bmm.out", TORCH_FN(bmm_out_xdna));
  m.impl("_fused_adam_", TORCH_FN(fused_adam_xdna));
  m.impl("_fused_adamw_", TORCH_FN(fused_adamw_xdna));
  m.impl("_fused_adam_.tensor_lr", TORCH_FN(fused_adam_tlr_xdna));
  m.impl("_fused_adamw_.tensor_lr", TORCH_FN(fused_adamw_tlr_xdna));
  m.impl("_foreach_add_.Scalar", TORCH_FN(foreach_add_scalar_xdna));
  m.impl("native_batch_norm", TORCH_FN(native_batch_norm_xdna));
  m.impl("native_batch_norm_backward", TORCH_FN(native_batch_norm_backward_xdna));
  m.impl("upsample_nearest2d", TORCH_FN(upsample_nearest2d_xdna));
  m.impl("upsample_nearest2d_backward", TORCH_FN(upsample_nearest2d_backward_xdna));
  m.impl("mse_loss", TORCH_FN(mse_loss_xdna));
  m.impl("mse_loss_backward", TORCH_FN(mse_loss_backward_xdna));
  m.impl("sum.dim_IntList", TORCH_FN(sum_dim_xdna));
}

// ---------------------------------------------------------------------------------------
// Convolution and product pieces of the fused regions (regions.cpp, xdna_train/regions.py)
// ---------------------------------------------------------------------------------------

// y = act(conv3x3(x, w) + b) for a 3x3 / stride-1 / pad-1 bf16 conv on the rows kernels,
// the activation applied in the epilogue before the one rounding (act 0 none, 1 ReLU).
// The weight's prepared form is cached as for any conv.
at::Tensor region_conv3x3(const at::Tensor& x, const at::Tensor& w, const std::optional<at::Tensor>& b, int act) {
  TORCH_CHECK(x.dim() == 4 && w.dim() == 4 && w.size(2) == 3 && w.size(3) == 3 && x.size(1) == w.size(1),
              "region conv: expected a 3x3 conv of matching channels");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16 && w.scalar_type() == at::kBFloat16 &&
                  x.device().type() == kXdna && w.device().type() == kXdna,
              "region conv: bf16 xdna tensors expected");
  TORCH_CHECK(act == 0 || act == 1, "region conv: activation must be 0 (none) or 1 (ReLU)");
  const bool has_b = b.has_value() && b->defined();
  if (has_b)
    TORCH_CHECK(b->scalar_type() == at::kBFloat16 && b->dim() == 1 && b->size(0) == w.size(0) &&
                    b->device().type() == kXdna,
                "region conv: bias must be a bf16 xdna vector of the output channels");
  ScopedCount sc(act ? "hip_region.conv_relu.run" : "hip_region.conv.run");
  if (nchw_route(x, w.size(0), true)) return hip_conv_nchw(x, w, has_b ? &*b : nullptr, false, act);
  const int layout = g_conv_layout.load();
  return hip_conv_packed(pack_rows(x, layout), layout, x.sizes(), w, has_b ? &*b : nullptr, false, act);
}

// c[i] = alpha * a[i] . b[i] for batched bf16 operands of any strides (the region's Gram
// products and their gradients).
at::Tensor region_bmm(const at::Tensor& a, const at::Tensor& b, double alpha) {
  TORCH_CHECK(a.dim() == 3 && b.dim() == 3 && a.size(0) == b.size(0) && a.size(2) == b.size(1),
              "region bmm: shape mismatch");
  TORCH_CHECK(gemm_dtype_ok({&a, &b}) && fits_int(a) && fits_int(b) && a.size(0) <= 65535,
              "region bmm: bf16 xdna operands expected");
  ScopedCount sc("hip_region.bmm.run");
  at::Tensor c = empty_xdna({a.size(0), a.size(1), b.size(2)}, at::kBFloat16);
  run_gemm(a, b, c, nullptr, float(alpha), 0.0f);
  return c;
}

// Training norm with its activation (act 1 ReLU, 2 LeakyReLU(slope)) applied before the one
// rounding of the output: batch norm over N*L per channel with the running statistics
// updated when given (bnorm.hip), or instance norm per (image, channel) plane (norm.hip).
// Returns y, save_mean, save_invstd.  The reference's fused BatchNorm + activation
// (region_kernels.cpp:346-457, reached from regions.py:426-461 _BatchNormAct).
std::tuple<at::Tensor, at::Tensor, at::Tensor> region_norm_act_fwd(
    const at::Tensor& x, const at::Tensor& weight, const at::Tensor& bias, const std::optional<at::Tensor>& rm,
    const std::optional<at::Tensor>& rv, double momentum, double eps, int act, double slope, bool instance) {
  TORCH_CHECK(act == 1 || act == 2, "region norm: activation must be 1 (ReLU) or 2 (LeakyReLU)");
  TORCH_CHECK(x.dim() >= 3 && x.scalar_type() == at::kBFloat16 && x.device().type() == kXdna &&
                  x.is_contiguous() && x.numel() > 0,
              "region norm: a non-empty contiguous bf16 xdna input of at least 3 dims expected");
  const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
  const int wd = norm_param_dtype(weight, bias);
  TORCH_CHECK(weight.defined() && bias.defined() && wd > 0 && norm_param_ok(weight, C) && norm_param_ok(bias, C),
              "region norm: affine bf16 or fp32 xdna parameters of the channel count expected");
  const int rsd = running_stats_dtype(rm, rv, C);
  TORCH_CHECK(rsd >= 0 && !(instance && rsd > 0), "region norm: unsupported running statistics");
  TORCH_CHECK(!instance || L <= kNormMaxPerChannel, "region norm: instance planes above ", kNormMaxPerChannel,
              " elements are not supported");
  at::Tensor y = empty_xdna(x.sizes(), at::kBFloat16);
  const int64_t nstat = instance ? N * C : C;
  at::Tensor mean = empty_xdna({nstat}, at::kFloat), invstd = empty_xdna({nstat}, at::kFloat);
  const auto* xp = static_cast<const uint16_t*>(x.const_data_ptr());
  if (instance) {
    ScopedCount sc("hip_region.instance_norm_act.run");
    check_abi(xdna_instance_norm_act_fwd_bf16(xp, weight.const_data_ptr(), bias.const_data_ptr(), wd,
                                              static_cast<uint16_t*>(y.data_ptr()), mean.data_ptr<float>(),
                                              invstd.data_ptr<float>(), N, C, L, eps, act, float(slope),
                                              current_stream()),
              "instance_norm fwd (activation)");
  } else {
    ScopedCount sc("hip_region.batch_norm_act.run");
    check_abi(xdna_batch_norm_train_act_fwd_bf16(
                  xp, weight.const_data_ptr(), bias.const_data_ptr(), wd, rsd ? rm->data_ptr() : nullptr,
                  rsd ? rv->data_ptr() : nullptr, rsd, momentum, eps, static_cast<uint16_t*>(y.data_ptr()),
                  mean.data_ptr<float>(), invstd.data_ptr<float>(), N, C, L, act, float(slope), current_stream()),
              "batch_norm fwd (activation)");
    if (rsd) {
      bump_write_epoch(*rm);
      bump_write_epoch(*rv);
    }
  }
  return {y, mean, invstd};
}

// Backward of region_norm_act_fwd: dy is taken through the activation's gradient (from
// its output y) inside the norm's two passes.  Returns dx (if need_x) and dweight, dbias
// (if need_params) in the parameters' dtype.
std::tuple<at::Tensor, at::Tensor, at::Tensor> region_norm_act_bwd(
    const at::Tensor& grad, const at::Tensor& x, const at::Tensor& y, const at::Tensor& weight,
    const at::Tensor& mean, const at::Tensor& invstd, int act, double slope, bool instance, bool need_x,
    bool need_params) {
  TORCH_CHECK(act == 1 || act == 2, "region norm: activation must be 1 (ReLU) or 2 (LeakyReLU)");
  for (const at::Tensor* t : {&x, &y})
    TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->device().type() == kXdna && t->is_contiguous() &&
                    t->dim() >= 3,
                "region norm: contiguous bf16 xdna input and output expected");
  TORCH_CHECK(y.sizes() == x.sizes() && grad.sizes() == x.sizes() && grad.device().type() == kXdna,
              "region norm: gradient, input and output shapes differ");
  const int64_t N = x.size(0), C = x.size(1), L = x.numel() / (N * C);
  const int wd = norm_param_dtype(weight, std::nullopt);
  TORCH_CHECK(wd > 0 && norm_param_ok(weight, C), "region norm: affine parameters expected");
  const int64_t nstat = instance ? N * C : C;
  for (const at::Tensor* t : {&mean, &invstd})
    TORCH_CHECK(t->scalar_type() == at::kFloat && t->numel() == nstat && t->is_contiguous() &&
                    t->device().type() == kXdna,
                "region norm: saved statistics of the wrong form");
  at::Tensor dx, dw, db;
  if (!need_x && !need_params) return {dx, dw, db};
  const at::Tensor dy = grad.to(at::kBFloat16).contiguous();
  if (need_x) dx = empty_xdna(x.sizes(), at::kBFloat16);
  if (need_params) {
    const at::ScalarType pt = wd == 2 ? at::kFloat : at::kBFloat16;
    dw = empty_xdna({C}, pt);
    db = empty_xdna({C}, pt);
  }
  const auto* dyp = static_cast<const uint16_t*>(dy.const_data_ptr());
  const auto* xp = static_cast<const uint16_t*>(x.const_data_ptr());
  const auto* yp = static_cast<const uint16_t*>(y.const_data_ptr());
  uint16_t* dxp = need_x ? static_cast<uint16_t*>(dx.data_ptr()) : nullptr;
  void* dwp = need_params ? dw.data_ptr() : nullptr;
  void* dbp = need_params ? db.data_ptr() : nullptr;
  if (instance) {
    ScopedCount sc("hip_region.instance_norm_act_bwd.run");
    check_abi(xdna_instance_norm_act_bwd_bf16(dyp, xp, yp, weight.const_data_ptr(), wd, mean.const_data_ptr<float>(),
                                              invstd.const_data_ptr<float>(), dxp, dwp, dbp, N, C, L, act,
                                              float(slope), current_stream()),
              "instance_norm bwd (activation)");
  } else {
    ScopedCount sc("hip_region.batch_norm_act_bwd.run");
    check_abi(xdna_batch_norm_train_act_bwd_bf16(dyp, xp, yp, weight.const_data_ptr(), wd,
                                                 mean.const_data_ptr<float>(), invstd.const_data_ptr<float>(), dxp,
                                                 dwp, dbp, N, C, L, act, float(slope), current_stream()),
              "batch_norm bwd (activation)");
  }
  return {dx, dw, db};
}

}  // namespace xdna_backend
