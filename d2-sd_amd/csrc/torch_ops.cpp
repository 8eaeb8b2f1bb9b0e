// torch.ops.d2sd.* — torch operators over the C ABI of libd2sd.so
// (include/d2sd.h), for the calls the reference's verify path makes:
//
//   single_prefill_with_kv_cache  flashinfer.single_prefill_with_kv_cache
//                                 (generation/verification.py:145, 159;
//                                  model/cascade_graph.py:54; model/dflash.py:112, 127)
//   merge_state_in_place          flashinfer.merge_state_in_place
//                                 (generation/verification.py:163;
//                                  model/cascade_graph.py:58; model/dflash.py:131)
//   local_attention_merge         the per-row local attention + merge loop that
//                                 CascadeGraphRunner captures (model/cascade_graph.py:52-60)
//   cascade_run / cascade_run_no_alloc
//                                 one cascade verify call of a d2sd_cascade_plan
//                                 (generation/verification.py:127-176 over a token tree)
//
// Each operator checks its tensors, then calls the C entry point on the
// current HIP stream of the tensors' device; there is no other code path.
// Meta kernels give shapes for tracing (torch.compile / fake tensors).  The
// dispatch key named CUDA is where torch registers its GPU (here HIP) device.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>
#include <cstring>

#include "d2sd.h"

namespace {

d2sd_stream_t current_stream() { return (d2sd_stream_t)c10::hip::getCurrentHIPStream().stream(); }

void check(int rc, const char* what) { TORCH_CHECK(rc == D2SD_OK, what, " failed: ", d2sd_last_error()); }

void need_device(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), "d2sd: ", name, " must be a ROCm device tensor");
}

void need_rows(const at::Tensor& t, const char* name, at::ScalarType dt) {
  need_device(t, name);
  TORCH_CHECK(t.scalar_type() == dt, "d2sd: ", name, " must be ", dt, ", got ", t.scalar_type());
  TORCH_CHECK(t.dim() == 3 && t.stride(2) == 1, "d2sd: ", name, " must be 3-D with a contiguous last dimension");
}

const void* ptr_or_null(const c10::optional<at::Tensor>& t) { return t.has_value() ? t->data_ptr() : nullptr; }

// ---- single_prefill_with_kv_cache ----
std::tuple<at::Tensor, at::Tensor> single_prefill(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                  bool causal, c10::string_view kv_layout,
                                                  c10::optional<double> sm_scale, bool lse_base2) {
  need_rows(q, "q", at::kBFloat16);
  need_rows(k, "k", at::kBFloat16);
  need_rows(v, "v", at::kBFloat16);
  TORCH_CHECK(k.sizes() == v.sizes() && k.strides() == v.strides(), "d2sd: k and v must share shape and strides");
  const bool hnd = kv_layout == "HND";
  TORCH_CHECK(hnd || kv_layout == "NHD", "d2sd: kv_layout must be 'NHD' or 'HND'");
  const int64_t qo_len = q.size(0), hq = q.size(1), d = q.size(2);
  const int64_t kv_len = hnd ? k.size(1) : k.size(0), hkv = hnd ? k.size(0) : k.size(1);
  TORCH_CHECK(k.size(2) == d, "d2sd: q and k head_dim differ");
  const int64_t s_n = hnd ? k.stride(1) : k.stride(0), s_h = hnd ? k.stride(0) : k.stride(1);
  const float scale = (float)(sm_scale.has_value() ? *sm_scale : 1.0 / std::sqrt((double)d));
  const c10::DeviceGuard guard(q.device());
  at::Tensor out = at::empty(q.sizes(), q.options());
  at::Tensor lse = at::empty({qo_len, hq}, q.options().dtype(at::kFloat));
  const size_t ws = d2sd_single_prefill_workspace_size((int)qo_len, (int)kv_len, (int)hq, (int)hkv, (int)d, -1);
  at::Tensor work = at::empty({(int64_t)std::max<size_t>(ws, 1)}, q.options().dtype(at::kByte));
  check(d2sd_single_prefill_with_kv_cache(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), s_n,
                                          s_h, out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr<float>(),
                                          (int)qo_len, (int)kv_len, (int)hq, (int)hkv, (int)d, causal ? 1 : 0, -1,
                                          scale, lse_base2 ? 1 : 0, work.data_ptr(), (size_t)work.numel(),
                                          current_stream()),
        "d2sd.single_prefill_with_kv_cache");
  return {out, lse};
}

std::tuple<at::Tensor, at::Tensor> single_prefill_meta(const at::Tensor& q, const at::Tensor&, const at::Tensor&, bool,
                                                       c10::string_view, c10::optional<double>, bool) {
  return {at::empty_like(q), at::empty({q.size(0), q.size(1)}, q.options().dtype(at::kFloat))};
}

// ---- merge_state_in_place ----
void merge_state_in_place(at::Tensor& v, at::Tensor& s, const at::Tensor& v_other, const at::Tensor& s_other,
                          bool lse_base2) {
  need_rows(v, "v", at::kBFloat16);
  need_rows(v_other, "v_other", at::kBFloat16);
  need_device(s, "s");
  need_device(s_other, "s_other");
  TORCH_CHECK(v.sizes() == v_other.sizes(), "d2sd: v and v_other shapes differ");
  TORCH_CHECK(s.scalar_type() == at::kFloat && s_other.scalar_type() == at::kFloat, "d2sd: s, s_other must be float32");
  TORCH_CHECK(s.dim() == 2 && s.size(0) == v.size(0) && s.size(1) == v.size(1) && s_other.sizes() == s.sizes(),
              "d2sd: s / s_other must be [n, heads]");
  TORCH_CHECK(s.stride(1) == 1 && s_other.stride(1) == 1, "d2sd: s / s_other need a contiguous head dimension");
  const c10::DeviceGuard guard(v.device());
  check(d2sd_merge_state_in_place(v.data_ptr(), v.stride(0), v.stride(1), s.data_ptr<float>(), s.stride(0),
                                  v_other.data_ptr(), v_other.stride(0), v_other.stride(1), s_other.data_ptr<float>(),
                                  s_other.stride(0), (int)v.size(0), (int)v.size(1), (int)v.size(2),
                                  lse_base2 ? 1 : 0, current_stream()),
        "d2sd.merge_state_in_place");
}

void merge_state_meta(at::Tensor&, at::Tensor&, const at::Tensor&, const at::Tensor&, bool) {}

// ---- local_attention_merge ----
void local_attention_merge(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, at::Tensor& out,
                           at::Tensor& lse, bool causal, double sm_scale, const c10::optional<at::Tensor>& sinks,
                           bool lse_base2) {
  for (auto* t : {&q, &k, &v, (const at::Tensor*)&out}) {
    need_device(*t, "q/k/v/out");
    TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->dim() == 4 && t->stride(3) == 1,
                "d2sd: q/k/v/out must be bf16 [bsz, Lb, heads, D] with a contiguous head_dim");
  }
  TORCH_CHECK(out.sizes() == q.sizes() && k.sizes() == v.sizes() && k.strides() == v.strides(),
              "d2sd: out must match q, v must match k");
  TORCH_CHECK(lse.scalar_type() == at::kFloat && lse.dim() == 3 && lse.size(0) == q.size(0) &&
                  lse.size(1) == q.size(1) && lse.size(2) == q.size(2) && lse.stride(2) == 1,
              "d2sd: lse must be float32 [bsz, Lb, Hq] with contiguous heads");
  if (sinks.has_value())
    TORCH_CHECK(sinks->scalar_type() == at::kFloat && sinks->numel() == q.size(2) && sinks->is_contiguous(),
                "d2sd: sinks must be a contiguous float32 [Hq]");
  const c10::DeviceGuard guard(q.device());
  check(d2sd_local_attention_merge(q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), v.data_ptr(),
                                   k.stride(0), k.stride(1), k.stride(2), out.data_ptr(), out.stride(0), out.stride(1),
                                   out.stride(2), lse.data_ptr<float>(), lse.stride(0), lse.stride(1), (int)q.size(0),
                                   (int)q.size(1), (int)q.size(2), (int)k.size(2), (int)q.size(3), causal ? 1 : 0,
                                   (float)sm_scale, sinks.has_value() ? sinks->data_ptr<float>() : nullptr,
                                   lse_base2 ? 1 : 0, current_stream()),
        "d2sd.local_attention_merge");
}

void local_attention_merge_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, at::Tensor&, at::Tensor&,
                                bool, double, const c10::optional<at::Tensor>&, bool) {}

// ---- cascade_run ----
// info: the d2sd_cascade_plan_info bytes plan() produced (CPU uint8 tensor);
// prefix: the prefix strides / extent in elements, as run() passes them.
void cascade(bool no_alloc, const at::Tensor& info, const at::Tensor& plan, const at::Tensor& workspace,
             const at::Tensor& q, const at::Tensor& k_suffix, const at::Tensor& v_suffix,
             const c10::optional<at::Tensor>& k_prefix, const c10::optional<at::Tensor>& v_prefix,
             at::IntArrayRef prefix, const c10::optional<at::Tensor>& page_table,
             const c10::optional<at::Tensor>& tree_mask, int64_t mask_mode, int64_t mask_words,
             const c10::optional<at::Tensor>& prefix_len, const c10::optional<at::Tensor>& k_scale,
             const c10::optional<at::Tensor>& v_scale, const c10::optional<at::Tensor>& sinks, double sm_scale,
             bool lse_base2, at::Tensor& out, at::Tensor& lse, const c10::optional<at::Tensor>& k_prefix2,
             const c10::optional<at::Tensor>& v_prefix2, at::IntArrayRef prefix2,
             const c10::optional<at::Tensor>& k2_scale, const c10::optional<at::Tensor>& v2_scale) {
  TORCH_CHECK(info.device().is_cpu() && info.scalar_type() == at::kByte && info.is_contiguous() &&
                  (size_t)info.numel() == sizeof(d2sd_cascade_plan_info),
              "d2sd: info must hold the bytes of a d2sd_cascade_plan_info");
  TORCH_CHECK(prefix.size() == 4, "d2sd: prefix = (stride_tok, stride_head, stride_page, extent)");
  need_rows(q, "q", at::kBFloat16);
  need_rows(k_suffix, "k_suffix", at::kBFloat16);
  need_rows(v_suffix, "v_suffix", at::kBFloat16);
  need_rows(out, "out", at::kBFloat16);
  need_device(plan, "plan");
  need_device(lse, "lse");
  TORCH_CHECK(lse.scalar_type() == at::kFloat && lse.dim() == 2 && lse.stride(1) == 1,
              "d2sd: lse must be float32 [total_q, Hq] with contiguous heads");
  TORCH_CHECK(plan.scalar_type() == at::kInt && plan.is_contiguous(), "d2sd: plan must be a contiguous int32 tensor");
  d2sd_cascade_plan_info pi;
  std::memcpy(&pi, info.data_ptr(), sizeof(pi));
  TORCH_CHECK(plan.numel() >= pi.plan_ints, "d2sd: plan holds fewer entries than info.plan_ints");
  d2sd_cascade_run_args a;
  std::memset(&a, 0, sizeof(a));
  a.plan = plan.data_ptr<int32_t>();
  a.q = q.data_ptr();
  a.q_stride_n = q.stride(0);
  a.q_stride_h = q.stride(1);
  a.k_suffix = k_suffix.data_ptr();
  a.v_suffix = v_suffix.data_ptr();
  a.suffix_stride_n = k_suffix.stride(0);
  a.suffix_stride_h = k_suffix.stride(1);
  a.mask_mode = (int)mask_mode;
  a.mask_words = (int)mask_words;
  a.tree_mask = (const uint64_t*)ptr_or_null(tree_mask);
  a.k_prefix = ptr_or_null(k_prefix);
  a.v_prefix = ptr_or_null(v_prefix);
  a.prefix_stride_tok = prefix[0];
  a.prefix_stride_head = prefix[1];
  a.prefix_stride_page = prefix[2];
  a.prefix_extent = prefix[3];
  a.page_size = pi.page_size;
  a.page_table = (const int32_t*)ptr_or_null(page_table);
  a.prefix_len = (const int32_t*)ptr_or_null(prefix_len);
  a.k_scale = (const float*)ptr_or_null(k_scale);
  a.v_scale = (const float*)ptr_or_null(v_scale);
  a.sinks = (const float*)ptr_or_null(sinks);
  a.out = out.data_ptr();
  a.o_stride_n = out.stride(0);
  a.o_stride_h = out.stride(1);
  a.lse = lse.data_ptr<float>();
  a.lse_stride_n = lse.stride(0);
  a.sm_scale = (float)sm_scale;
  a.lse_base2 = lse_base2 ? 1 : 0;
  if (k_prefix2.has_value()) {
    TORCH_CHECK(prefix2.size() == 3, "d2sd: prefix2 = (stride_tok, stride_head, extent)");
    a.k_prefix2 = k_prefix2->data_ptr();
    a.v_prefix2 = ptr_or_null(v_prefix2);
    a.prefix2_stride_tok = prefix2[0];
    a.prefix2_stride_head = prefix2[1];
    a.prefix2_extent = prefix2[2];
    a.k2_scale = (const float*)ptr_or_null(k2_scale);
    a.v2_scale = (const float*)ptr_or_null(v2_scale);
  }
  if (!no_alloc) {
    need_device(workspace, "workspace");
    a.workspace = workspace.data_ptr();
    a.workspace_bytes = (size_t)workspace.nbytes();
  }
  const c10::DeviceGuard guard(q.device());
  check(no_alloc ? d2sd_cascade_run_noalloc(&pi, &a, current_stream()) : d2sd_cascade_run(&pi, &a, current_stream()),
        no_alloc ? "d2sd.cascade_run_no_alloc" : "d2sd.cascade_run");
}

#define CASCADE_ARGS                                                                                                 \
  const at::Tensor &info, const at::Tensor &plan, const at::Tensor &workspace, const at::Tensor &q,                 \
      const at::Tensor &k_suffix, const at::Tensor &v_suffix, const c10::optional<at::Tensor>&k_prefix,              \
      const c10::optional<at::Tensor>&v_prefix, at::IntArrayRef prefix,                                              \
      const c10::optional<at::Tensor>&page_table, const c10::optional<at::Tensor>&tree_mask, int64_t mask_mode,    \
      int64_t mask_words, const c10::optional<at::Tensor>&prefix_len, const c10::optional<at::Tensor>&k_scale,     \
      const c10::optional<at::Tensor>&v_scale, const c10::optional<at::Tensor>&sinks, double sm_scale,             \
      bool lse_base2, at::Tensor &out, at::Tensor &lse, const c10::optional<at::Tensor>&k_prefix2,               \
      const c10::optional<at::Tensor>&v_prefix2, at::IntArrayRef prefix2, const c10::optional<at::Tensor>&k2_scale, \
      const c10::optional<at::Tensor>&v2_scale
#define CASCADE_PASS                                                                                       \
  info, plan, workspace, q, k_suffix, v_suffix, k_prefix, v_prefix, prefix, page_table, tree_mask, mask_mode, \
      mask_words, prefix_len, k_scale, v_scale, sinks, sm_scale, lse_base2, out, lse, k_prefix2, v_prefix2,   \
      prefix2, k2_scale, v2_scale

void cascade_run(CASCADE_ARGS) { cascade(false, CASCADE_PASS); }
void cascade_run_no_alloc(CASCADE_ARGS) { cascade(true, CASCADE_PASS); }
void cascade_meta(CASCADE_ARGS) {}

}  // namespace

TORCH_LIBRARY(d2sd, m) {
  m.def("single_prefill_with_kv_cache(Tensor q, Tensor k, Tensor v, bool causal=False, str kv_layout=\"NHD\", "
        "float? sm_scale=None, bool lse_base2=False) -> (Tensor, Tensor)");
  m.def("merge_state_in_place(Tensor(a!) v, Tensor(b!) s, Tensor v_other, Tensor s_other, bool lse_base2=False) -> ()");
  m.def("local_attention_merge(Tensor q, Tensor k, Tensor v, Tensor(a!) out, Tensor(b!) lse, bool causal, "
        "float sm_scale, Tensor? sinks=None, bool lse_base2=False) -> ()");
  const char* cascade_schema =
      "(Tensor info, Tensor plan, Tensor workspace, Tensor q, Tensor k_suffix, Tensor v_suffix, Tensor? k_prefix, "
      "Tensor? v_prefix, int[] prefix, Tensor? page_table, Tensor? tree_mask, int mask_mode, int mask_words, "
      "Tensor? prefix_len, Tensor? k_scale, Tensor? v_scale, Tensor? sinks, float sm_scale, bool lse_base2, "
      "Tensor(a!) out, Tensor(b!) lse, Tensor? k_prefix2=None, Tensor? v_prefix2=None, int[] prefix2=[], "
      "Tensor? k2_scale=None, Tensor? v2_scale=None) -> ()";
  m.def((std::string("cascade_run") + cascade_schema).c_str());
  m.def((std::string("cascade_run_no_alloc") + cascade_schema).c_str());
}

TORCH_LIBRARY_IMPL(d2sd, CUDA, m) {
  m.impl("single_prefill_with_kv_cache", &single_prefill);
  m.impl("merge_state_in_place", &merge_state_in_place);
  m.impl("local_attention_merge", &local_attention_merge);
  m.impl("cascade_run", &cascade_run);
  m.impl("cascade_run_no_alloc", &cascade_run_no_alloc);
}

TORCH_LIBRARY_IMPL(d2sd, Meta, m) {
  m.impl("single_prefill_with_kv_cache", &single_prefill_meta);
  m.impl("merge_state_in_place", &merge_state_meta);
  m.impl("local_attention_merge", &local_attention_merge_meta);
  m.impl("cascade_run", &cascade_meta);
  m.impl("cascade_run_no_alloc", &cascade_meta);
}
