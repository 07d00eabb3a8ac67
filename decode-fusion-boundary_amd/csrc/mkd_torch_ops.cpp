// mkd_torch_ops.cpp -- torch operator registration of the decode step
// (libmkd_torch_ops.so). A thin host-only shim over the C ABI of
// libmkd_decode.so: it checks the tensors, fills an MkdStepDesc/MkdSchedule
// from them, launches on the current HIP stream of the cache's device and
// raises (TORCH_CHECK) on a non-zero return code with the library's message.
//
// Counterpart of the reference's torch extension nanovllm_megakernel_C
// (csrc/torch_bindings.cpp:65-184 tg_decode_step, :186-225 tg_zero_regions,
// :227-264 TORCH_LIBRARY registration): same namespace, operators registered on
// the device dispatch key (ROCm's HIP device is torch's "CUDA" key).
// PyTorch-ROCm keeps its HIP devices under torch's "cuda" device type; the
// guard and stream of that arrangement are the *MasqueradingAsCUDA ones.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <optional>

#include "mkd_abi.h"

namespace {

void check_dev(const at::Tensor& t, const char* name, const at::Device& dev) {
  TORCH_CHECK(t.device() == dev, name, " must be on ", dev, " (got ", t.device(), ")");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == MKD_OK, what, " failed (", rc, "): ", mkd_last_error());
}

// One decode step as one persistent launch (mkd_launch_persistent). The caches,
// out_tokens, out_logits and workspace are written; with MKD_FLAG_ADVANCE in
// `flags` so are input_ids and cache_seqlens.
void mkd_decode_step(const at::Tensor& layer_ptrs, const at::Tensor& embed, const at::Tensor& final_norm,
                     const at::Tensor& rope_cos, const at::Tensor& rope_sin, const at::Tensor& k_cache,
                     const at::Tensor& v_cache, const at::Tensor& page_table, const at::Tensor& cache_seqlens,
                     const at::Tensor& row_active, const at::Tensor& input_ids, const at::Tensor& out_tokens,
                     const std::optional<at::Tensor>& out_logits, const at::Tensor& workspace,
                     const at::Tensor& inst, const at::Tensor& num_inst, int64_t grid, int64_t max_inst,
                     int64_t rows, int64_t batch, int64_t num_layers, int64_t lm_slots, int64_t flags,
                     int64_t num_blocks, int64_t block_size) {
  const at::Device dev = k_cache.device();
  TORCH_CHECK(dev.is_cuda(), "k_cache must be a device tensor");
  const struct {
    const at::Tensor* t;
    const char* name;
    at::ScalarType dtype;
  } args[] = {{&layer_ptrs, "layer_ptrs", at::kLong},     {&embed, "embed", at::kBFloat16},
              {&final_norm, "final_norm", at::kBFloat16}, {&rope_cos, "rope_cos", at::kFloat},
              {&rope_sin, "rope_sin", at::kFloat},        {&k_cache, "k_cache", at::kBFloat16},
              {&v_cache, "v_cache", at::kBFloat16},       {&page_table, "page_table", at::kInt},
              {&cache_seqlens, "cache_seqlens", at::kInt}, {&row_active, "row_active", at::kInt},
              {&input_ids, "input_ids", at::kLong},       {&out_tokens, "out_tokens", at::kInt},
              {&workspace, "workspace", at::kByte},       {&inst, "inst", at::kInt},
              {&num_inst, "num_inst", at::kInt}};
  for (const auto& a : args) {
    check_dev(*a.t, a.name, dev);
    TORCH_CHECK(a.t->scalar_type() == a.dtype, a.name, " has dtype ", a.t->scalar_type(), ", expected ", a.dtype);
  }
  TORCH_CHECK(k_cache.dim() == 5 && v_cache.sizes() == k_cache.sizes(),
              "k_cache/v_cache must be [layers, blocks, block_size, kv_heads, head_dim]");
  TORCH_CHECK(k_cache.size(1) == num_blocks && k_cache.size(2) == block_size, "cache geometry mismatch");
  TORCH_CHECK(page_table.dim() == 2 && page_table.size(0) >= rows, "page_table must be [>= rows, pages]");
  TORCH_CHECK(cache_seqlens.numel() >= rows && row_active.numel() >= rows && input_ids.numel() >= rows &&
                  out_tokens.numel() >= rows,
              "per-row tensors must hold at least `rows` entries");
  TORCH_CHECK(inst.numel() >= grid * max_inst * MKD_INST_WORDS && num_inst.numel() >= grid,
              "instruction buffers smaller than grid x max_inst");
  TORCH_CHECK(workspace.numel() >= (int64_t)mkd_workspace_bytes(), "workspace smaller than mkd_workspace_bytes()");
  if (out_logits.has_value()) {
    check_dev(*out_logits, "out_logits", dev);
    TORCH_CHECK(out_logits->scalar_type() == at::kBFloat16 && out_logits->numel() >= rows * MKD_VOCAB,
                "out_logits must be bf16 [rows, vocab]");
  }
  MkdStepDesc d{};
  d.layer_ptrs = reinterpret_cast<const uint64_t*>(layer_ptrs.data_ptr());
  d.embed = reinterpret_cast<const uint16_t*>(embed.data_ptr());
  d.final_norm = reinterpret_cast<const uint16_t*>(final_norm.data_ptr());
  d.rope_cos = rope_cos.data_ptr<float>();
  d.rope_sin = rope_sin.data_ptr<float>();
  d.k_cache = reinterpret_cast<uint16_t*>(k_cache.data_ptr());
  d.v_cache = reinterpret_cast<uint16_t*>(v_cache.data_ptr());
  d.kv_layer_stride = k_cache.stride(0);
  d.num_blocks = (int32_t)num_blocks;
  d.block_size = (int32_t)block_size;
  d.page_table = page_table.data_ptr<int32_t>();
  d.page_stride = (int32_t)page_table.size(1);
  d.cache_seqlens = cache_seqlens.data_ptr<int32_t>();
  d.row_active = row_active.data_ptr<int32_t>();
  d.input_ids = input_ids.data_ptr<int64_t>();
  d.out_tokens = out_tokens.data_ptr<int32_t>();
  d.out_logits = out_logits.has_value() ? reinterpret_cast<uint16_t*>(out_logits->data_ptr()) : nullptr;
  d.workspace = workspace.data_ptr();
  d.workspace_bytes = (uint64_t)workspace.numel();
  d.rows = (int32_t)rows;
  d.batch = (int32_t)batch;
  d.num_layers = (int32_t)num_layers;
  d.lm_slots = (int32_t)lm_slots;
  d.flags = (uint32_t)flags;
  MkdSchedule s{inst.data_ptr<int32_t>(), num_inst.data_ptr<int32_t>(), (int32_t)grid, (int32_t)max_inst};
  c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  check_rc(mkd_launch_persistent(&d, &s, c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream()),
           "mkd_launch_persistent");
}

// Clear the workspace's counters, epoch and tagged words (mkd_reset_counters).
void mkd_reset(const at::Tensor& workspace) {
  TORCH_CHECK(workspace.is_cuda() && workspace.is_contiguous() && workspace.scalar_type() == at::kByte,
              "workspace must be a contiguous uint8 device tensor");
  TORCH_CHECK(workspace.numel() >= (int64_t)mkd_workspace_bytes(), "workspace smaller than mkd_workspace_bytes()");
  MkdStepDesc d{};
  d.workspace = workspace.data_ptr();
  d.workspace_bytes = (uint64_t)workspace.numel();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(workspace.device());
  check_rc(mkd_reset_counters(&d, c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(workspace.device().index()).stream()),
           "mkd_reset_counters");
}

}  // namespace

TORCH_LIBRARY(nanovllm_megakernel_C, m) {
  m.def(
      "mkd_decode_step(Tensor layer_ptrs, Tensor embed, Tensor final_norm, Tensor rope_cos, Tensor rope_sin, "
      "Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor page_table, Tensor(f!) cache_seqlens, Tensor row_active, "
      "Tensor(g!) input_ids, Tensor(c!) out_tokens, Tensor(d!)? out_logits, Tensor(e!) workspace, Tensor inst, "
      "Tensor num_inst, int grid, int max_inst, int rows, int batch, int num_layers, int lm_slots, int flags, "
      "int num_blocks, int block_size) -> ()");
  m.def("mkd_reset_counters(Tensor(a!) workspace) -> ()");
}

TORCH_LIBRARY_IMPL(nanovllm_megakernel_C, CUDA, m) {
  m.impl("mkd_decode_step", &mkd_decode_step);
  m.impl("mkd_reset_counters", &mkd_reset);
}
