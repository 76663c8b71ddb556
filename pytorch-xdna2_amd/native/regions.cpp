// Host side of the fused training regions (xdna_train/regions.py): checks and C-ABI calls
// of the region kernels (csrc/region.hip) on tensors.  Mirrors the reference's region
// kernel bindings (torch_xdna_device.cpp:5418-5594, region_kernels.cpp:51-340) for device
// memory: every scalar autograd hands in (the loss gradient) stays on the device.
#include "xdna.h"

namespace xdna_backend {
namespace {

void check_bf16(const at::Tensor& t, const char* what) {
  TORCH_CHECK(t.defined() && t.scalar_type() == at::kBFloat16 && t.device().type() == kXdna && t.is_contiguous(),
              "region: ", what, " must be a contiguous bf16 xdna tensor");
}

const uint16_t* ptr16(const std::optional<at::Tensor>& t) {
  return t.has_value() && t->defined() ? static_cast<const uint16_t*>(t->const_data_ptr()) : nullptr;
}

// the loss gradient autograd passes in: a device scalar (fp32 or bf16), or none
std::pair<const void*, int> go_arg(const std::optional<at::Tensor>& go) {
  if (!go.has_value() || !go->defined()) return {nullptr, 0};
  TORCH_CHECK(go->numel() == 1 && go->device().type() == kXdna &&
                  (go->scalar_type() == at::kFloat || go->scalar_type() == at::kBFloat16),
              "region: the loss gradient must be an fp32 or bf16 xdna scalar");
  return {go->const_data_ptr(), go->scalar_type() == at::kFloat ? 1 : 2};
}

}  // namespace

// 2x2 / stride-2 max-pool of an NCHW bf16 tensor (floor mode, PyTorch's window rule)
at::Tensor region_maxpool2(const at::Tensor& x) {
  check_bf16(x, "pool input");
  TORCH_CHECK(x.dim() == 4, "region maxpool: NCHW input expected");
  at::Tensor y = empty_xdna({x.size(0), x.size(1), x.size(2) / 2, x.size(3) / 2}, at::kBFloat16);
  ScopedCount sc("hip_region.maxpool2.run");
  check_abi(xdna_region_maxpool2_bf16(static_cast<const uint16_t*>(x.const_data_ptr()),
                                      static_cast<uint16_t*>(y.data_ptr()), x.size(0) * x.size(1), int(x.size(2)),
                                      int(x.size(3)), current_stream()),
            "region maxpool");
  return y;
}

// out = (r given and r <= 0) ? 0 : bf16(base + extra + scale * go * (ta - tb)), base = g, or
// gp routed through the max-pool windows of px; any term may be absent.
at::Tensor region_backward(const std::optional<at::Tensor>& r, const std::optional<at::Tensor>& g,
                           const std::optional<at::Tensor>& gp, const std::optional<at::Tensor>& px,
                           const std::optional<at::Tensor>& extra, const std::optional<at::Tensor>& ta,
                           const std::optional<at::Tensor>& tb, double scale, const std::optional<at::Tensor>& go,
                           at::IntArrayRef shape) {
  TORCH_CHECK(shape.size() == 4, "region backward: an NCHW shape expected");
  const int64_t n = shape[0] * shape[1] * shape[2] * shape[3];
  for (const auto* t : {&r, &g, &px, &extra, &ta, &tb})
    if (t->has_value() && (*t)->defined()) {
      check_bf16(**t, "operand");
      TORCH_CHECK((*t)->numel() == n, "region backward: operand of the wrong size");
    }
  if (gp.has_value() && gp->defined()) {
    check_bf16(*gp, "pooled gradient");
    TORCH_CHECK(gp->numel() == shape[0] * shape[1] * (shape[2] / 2) * (shape[3] / 2),
                "region backward: pooled gradient of the wrong size");
  }
  const auto [gop, god] = go_arg(go);
  at::Tensor out = empty_xdna(shape, at::kBFloat16);
  ScopedCount sc("hip_region.backward.run");
  check_abi(xdna_region_backward_bf16(ptr16(r), ptr16(g), ptr16(gp), ptr16(px), ptr16(extra), ptr16(ta), ptr16(tb),
                                      float(scale), gop, god, static_cast<uint16_t*>(out.data_ptr()),
                                      shape[0] * shape[1], int(shape[2]), int(shape[3]), current_stream()),
            "region backward");
  return out;
}

int64_t region_loss_parts() { return xdna_region_loss_parts(); }

// part[offset .. offset + parts) = scale * sums of (a - b)^2 over a fixed partition
void region_sqdiff(const at::Tensor& a, const at::Tensor& b, double scale, at::Tensor& part, int64_t offset) {
  check_bf16(a, "tap");
  check_bf16(b, "target tap");
  TORCH_CHECK(a.numel() == b.numel(), "region sqdiff: size mismatch");
  TORCH_CHECK(part.scalar_type() == at::kFloat && part.device().type() == kXdna && part.is_contiguous() &&
                  offset >= 0 && offset + xdna_region_loss_parts() <= part.numel(),
              "region sqdiff: partial-sum buffer too small");
  ScopedCount sc("hip_region.sqdiff.run");
  check_abi(xdna_region_sqdiff_bf16(static_cast<const uint16_t*>(a.const_data_ptr()),
                                    static_cast<const uint16_t*>(b.const_data_ptr()), a.numel(), float(scale),
                                    part.data_ptr<float>() + offset, current_stream()),
            "region sqdiff");
}

// part[offset ..] = scale * sums of (G / chw - t)^2; G [B][C][C] bf16, t fp32 [1 or B][C][C]
void region_gram_sqdiff(const at::Tensor& G, const at::Tensor& t, double chw, double scale, at::Tensor& part,
                        int64_t offset) {
  check_bf16(G, "Gram matrices");
  TORCH_CHECK(G.dim() == 3 && G.size(1) == G.size(2), "region gram: [B][C][C] Gram matrices expected");
  TORCH_CHECK(t.scalar_type() == at::kFloat && t.device().type() == kXdna && t.is_contiguous() && t.dim() == 3 &&
                  (t.size(0) == 1 || t.size(0) == G.size(0)) && t.size(1) == G.size(1) && t.size(2) == G.size(2),
              "region gram: fp32 target Gram matrices [1 or B][C][C] expected");
  TORCH_CHECK(part.scalar_type() == at::kFloat && part.device().type() == kXdna && part.is_contiguous() &&
                  offset >= 0 && offset + xdna_region_loss_parts() <= part.numel(),
              "region gram: partial-sum buffer too small");
  const int64_t cc = G.size(1) * G.size(2);
  ScopedCount sc("hip_region.gram_sqdiff.run");
  check_abi(xdna_region_gram_sqdiff_bf16(static_cast<const uint16_t*>(G.const_data_ptr()), t.data_ptr<float>(),
                                         t.size(0) == 1 ? 0 : cc, G.size(0), cc, float(chw), float(scale),
                                         part.data_ptr<float>() + offset, current_stream()),
            "region gram sqdiff");
}

// (loss fp32 scalar, loss bf16 scalar) = fixed-order sum of the partials
std::tuple<at::Tensor, at::Tensor> region_loss_finish(const at::Tensor& part) {
  TORCH_CHECK(part.scalar_type() == at::kFloat && part.device().type() == kXdna && part.is_contiguous() &&
                  part.numel() < (int64_t(1) << 30),
              "region finish: fp32 partial sums expected");
  at::Tensor f = empty_xdna({}, at::kFloat);
  at::Tensor h = empty_xdna({}, at::kBFloat16);
  check_abi(xdna_region_loss_finish(part.data_ptr<float>(), int(part.numel()), f.data_ptr<float>(),
                                    static_cast<uint16_t*>(h.data_ptr()), current_stream()),
            "region finish");
  return {f, h};
}

// S = bf16(coef * go * (d + d^T) / chw), d = G / chw - t: the features' gradient is S F
at::Tensor region_gram_grad(const at::Tensor& G, const at::Tensor& t, double chw, double coef,
                            const std::optional<at::Tensor>& go) {
  check_bf16(G, "Gram matrices");
  TORCH_CHECK(G.dim() == 3 && t.dim() == 3 && t.scalar_type() == at::kFloat && t.is_contiguous() &&
                  t.device().type() == kXdna && (t.size(0) == 1 || t.size(0) == G.size(0)) &&
                  t.size(1) == G.size(1) && t.size(2) == G.size(2),
              "region gram grad: shapes");
  const auto [gop, god] = go_arg(go);
  TORCH_CHECK(G.size(1) == G.size(2) && G.size(1) < (int64_t(1) << 20), "region gram grad: square Gram matrices");
  const int64_t cc = G.size(1) * G.size(2);
  at::Tensor S = empty_xdna(G.sizes(), at::kBFloat16);
  ScopedCount sc("hip_region.gram_grad.run");
  check_abi(xdna_region_gram_grad_bf16(static_cast<const uint16_t*>(G.const_data_ptr()), t.data_ptr<float>(),
                                       t.size(0) == 1 ? 0 : cc, G.size(0), int(G.size(1)), float(chw), float(coef),
                                       gop, god, static_cast<uint16_t*>(S.data_ptr()), current_stream()),
            "region gram grad");
  return S;
}

}  // namespace xdna_backend
