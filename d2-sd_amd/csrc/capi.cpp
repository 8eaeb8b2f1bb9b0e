// extern "C" entry points of libd2sd.so (declared in include/d2sd.h).
// Argument validation, work planning and kernel launches; no device memory is
// allocated here except the executable of a captured graph and the cached
// device plans of the single-prefill drop-in (a few tens of KB per shape).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <array>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/d2sd.h"
#include "d2sd_internal.h"
#include "plan.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return D2SD_ERR_HIP;
}

constexpr float kLog2e = 1.4426950408889634f;

int device_num_cus() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lk(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    cache[dev] = n;
  }
  return cache[dev];
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool stride_ok(int64_t s) { return s % 8 == 0; }

int check_heads(int hq, int hkv, int d) {
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return fail(D2SD_ERR_INVALID_ARG, "num_qo_heads must be a positive multiple of num_kv_heads");
  if (d != 64 && d != 128) return fail(D2SD_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  return D2SD_OK;
}

}  // namespace

extern "C" {

static size_t single_cascade_workspace(int qo_len, int kv_len, int num_qo_heads, int num_kv_heads, int head_dim,
                                       int window_left);
static int single_prefill_cascade(const void* q, int64_t q_stride_n, int64_t q_stride_h, const void* k,
                                  const void* v, int64_t kv_stride_n, int64_t kv_stride_h, void* o,
                                  int64_t o_stride_n, int64_t o_stride_h, float* lse, int qo_len, int kv_len,
                                  int num_qo_heads, int num_kv_heads, int head_dim, int causal, float sm_scale,
                                  int lse_base2, void* workspace, size_t workspace_bytes, hipStream_t stream,
                                  bool* used);

static int local_merge_cascade(const void* q, int64_t q_stride_b, int64_t q_stride_n, int64_t q_stride_h,
                               const void* k, const void* v, int64_t kv_stride_b, int64_t kv_stride_n,
                               int64_t kv_stride_h, void* out, int64_t o_stride_b, int64_t o_stride_n,
                               int64_t o_stride_h, float* lse, int64_t lse_stride_b, int64_t lse_stride_n, int bsz,
                               int block_len, int hq, int hkv, int d, int causal, float sm_scale, const float* sinks,
                               int lse_base2, hipStream_t stream, bool* used);

const char* d2sd_last_error(void) { return g_last_error.c_str(); }

const char* d2sd_version(void) { return "d2sd-mi355x 0.1.0 (gfx950)"; }

int d2sd_merge_state_in_place(void* v, int64_t v_stride_n, int64_t v_stride_h, float* s, int64_t s_stride_n,
                              const void* v_other, int64_t vo_stride_n, int64_t vo_stride_h,
                              const float* s_other, int64_t so_stride_n, int seq_len, int num_heads,
                              int head_dim, int lse_base2, d2sd_stream_t stream) {
  g_last_error.clear();
  if (seq_len < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0)
    return fail(D2SD_ERR_INVALID_ARG, "merge_state: bad sizes");
  if (seq_len == 0) return D2SD_OK;
  if (!v || !s || !v_other || !s_other) return fail(D2SD_ERR_INVALID_ARG, "merge_state: null pointer");
  if (!aligned16(v) || !aligned16(v_other) || !stride_ok(v_stride_n) || !stride_ok(v_stride_h) ||
      !stride_ok(vo_stride_n) || !stride_ok(vo_stride_h))
    return fail(D2SD_ERR_INVALID_ARG, "merge_state: v / v_other must be 16-byte aligned with strides % 8 == 0");
  hipError_t e = d2sd::launch_merge_state(v, v_stride_n, v_stride_h, s, s_stride_n, v_other, vo_stride_n,
                                          vo_stride_h, s_other, so_stride_n, seq_len, num_heads, head_dim,
                                          lse_base2, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "merge_state launch");
}

size_t d2sd_single_prefill_workspace_size(int qo_len, int kv_len, int num_qo_heads, int num_kv_heads,
                                          int head_dim, int window_left) {
  if (qo_len <= 0 || kv_len <= 0 || num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  d2sd::ImplicitWork imp{};
  int waves = 0;
  size_t ws = 0;
  d2sd::plan_single(qo_len, kv_len, num_qo_heads, num_kv_heads, head_dim, window_left, device_num_cus(), imp,
                    waves, ws);
  return std::max(ws, single_cascade_workspace(qo_len, kv_len, num_qo_heads, num_kv_heads, head_dim, window_left));
}

int d2sd_single_prefill_with_kv_cache(const void* q, int64_t q_stride_n, int64_t q_stride_h, const void* k,
                                      const void* v, int64_t kv_stride_n, int64_t kv_stride_h, void* o,
                                      int64_t o_stride_n, int64_t o_stride_h, float* lse, int qo_len, int kv_len,
                                      int num_qo_heads, int num_kv_heads, int head_dim, int causal,
                                      int window_left, float sm_scale, int lse_base2, void* workspace,
                                      size_t workspace_bytes, d2sd_stream_t stream) {
  g_last_error.clear();
  if (int rc = check_heads(num_qo_heads, num_kv_heads, head_dim)) return rc;
  if (qo_len < 0 || kv_len < 0) return fail(D2SD_ERR_INVALID_ARG, "single_prefill: negative length");
  if (qo_len == 0) return D2SD_OK;
  if (kv_len == 0) return fail(D2SD_ERR_INVALID_ARG, "single_prefill: kv_len must be > 0");
  if (!q || !k || !v || !o) return fail(D2SD_ERR_INVALID_ARG, "single_prefill: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !stride_ok(q_stride_n) ||
      !stride_ok(q_stride_h) || !stride_ok(kv_stride_n) || !stride_ok(kv_stride_h) || !stride_ok(o_stride_n) ||
      !stride_ok(o_stride_h))
    return fail(D2SD_ERR_INVALID_ARG, "single_prefill: tensors must be 16-byte aligned with strides % 8 == 0");
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale)) return fail(D2SD_ERR_INVALID_ARG, "single_prefill: bad sm_scale");

  // the cascade kernels when the shape maps onto them (see single_prefill_cascade)
  bool used = false;
  if (int rc = single_prefill_cascade(q, q_stride_n, q_stride_h, k, v, kv_stride_n, kv_stride_h, o, o_stride_n,
                                      o_stride_h, lse, qo_len, kv_len, num_qo_heads, num_kv_heads, head_dim,
                                      window_left >= 0 ? -1 : causal, sm_scale, lse_base2, workspace,
                                      workspace_bytes, (hipStream_t)stream, &used))
    return rc;
  if (used) return D2SD_OK;

  d2sd::AttnParams p{};
  int waves = 0;
  size_t ws = 0;
  d2sd::plan_single(qo_len, kv_len, num_qo_heads, num_kv_heads, head_dim, window_left, device_num_cus(), p.imp,
                    waves, ws);
  if (ws > workspace_bytes || (ws > 0 && !workspace))
    return fail(D2SD_ERR_WORKSPACE, "single_prefill: workspace too small (need " + std::to_string(ws) + " bytes)");
  const int rows = 32 * waves;
  const long long slots = (long long)num_kv_heads * p.imp.qtiles * p.imp.splits;
  p.q = q;
  p.q_stride_n = q_stride_n;
  p.q_stride_h = q_stride_h;
  p.o = o;
  p.o_stride_n = o_stride_n;
  p.o_stride_h = o_stride_h;
  p.lse = lse;
  p.lse_stride_n = num_qo_heads;
  p.part_o = workspace;
  p.part_lse = workspace ? (float*)((char*)workspace + slots * rows * head_dim * 2) : nullptr;
  d2sd::KvSource& s0 = p.src[0];
  s0.k = k;
  s0.v = v;
  s0.stride_tok = kv_stride_n;
  s0.stride_head = kv_stride_h;
  s0.mask_mode = causal ? d2sd::MASK_CAUSAL : d2sd::MASK_NONE;
  s0.dtype = d2sd::KV_BF16;
  p.src[1] = s0;
  p.sm_scale = sm_scale;
  p.sm_scale_log2 = sm_scale * kLog2e;
  p.num_kv_heads = num_kv_heads;
  p.group = num_qo_heads / num_kv_heads;
  p.lse_base2 = lse_base2;
  const int nblocks = num_kv_heads * p.imp.qtiles * p.imp.splits;
  hipError_t e = d2sd::launch_attention(p, head_dim, waves, 0, false, false, causal != 0, nblocks,
                                        (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "single_prefill attention launch");
  if (p.imp.splits > 1) {
    e = d2sd::launch_merge(p, head_dim, rows, num_kv_heads * p.imp.qtiles, (hipStream_t)stream);
    if (e != hipSuccess) return fail_hip(e, "single_prefill merge launch");
  }
  return D2SD_OK;
}

int d2sd_local_attention_merge(const void* q, int64_t q_stride_b, int64_t q_stride_n, int64_t q_stride_h,
                               const void* k, const void* v, int64_t kv_stride_b, int64_t kv_stride_n,
                               int64_t kv_stride_h, void* out, int64_t o_stride_b, int64_t o_stride_n,
                               int64_t o_stride_h, float* lse, int64_t lse_stride_b, int64_t lse_stride_n,
                               int bsz, int block_len, int num_qo_heads, int num_kv_heads, int head_dim,
                               int causal, float sm_scale, const float* sinks, int lse_base2,
                               d2sd_stream_t stream) {
  g_last_error.clear();
  if (int rc = check_heads(num_qo_heads, num_kv_heads, head_dim)) return rc;
  if (bsz < 0 || block_len < 0) return fail(D2SD_ERR_INVALID_ARG, "local_attention_merge: negative size");
  if (bsz == 0 || block_len == 0) return D2SD_OK;
  if (!q || !k || !v || !out || !lse) return fail(D2SD_ERR_INVALID_ARG, "local_attention_merge: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !stride_ok(q_stride_b) ||
      !stride_ok(q_stride_n) || !stride_ok(q_stride_h) || !stride_ok(kv_stride_b) || !stride_ok(kv_stride_n) ||
      !stride_ok(kv_stride_h) || !stride_ok(o_stride_b) || !stride_ok(o_stride_n) || !stride_ok(o_stride_h))
    return fail(D2SD_ERR_INVALID_ARG,
                "local_attention_merge: tensors must be 16-byte aligned with strides % 8 == 0");
  // the cascade kernels' suffix items when the batch is laid out row after row
  bool used = false;
  if (int rc = local_merge_cascade(q, q_stride_b, q_stride_n, q_stride_h, k, v, kv_stride_b, kv_stride_n, kv_stride_h,
                                   out, o_stride_b, o_stride_n, o_stride_h, lse, lse_stride_b, lse_stride_n, bsz,
                                   block_len, num_qo_heads, num_kv_heads, head_dim, causal, sm_scale, sinks,
                                   lse_base2, (hipStream_t)stream, &used))
    return rc;
  if (used) return D2SD_OK;

  d2sd::AttnParams p{};
  const int g = num_qo_heads / num_kv_heads;
  const int waves = d2sd::choose_waves(block_len * g);
  const int rows = 32 * waves;
  p.imp.num_reqs = bsz;
  p.imp.qtiles = (block_len * g + rows - 1) / rows;
  p.imp.splits = 1;
  p.imp.chunk_keys = ((block_len + 63) / 64) * 64;
  p.imp.qo_len = block_len;
  p.imp.kv_len = block_len;
  p.imp.kv_begin = 0;
  p.imp.single_mode = d2sd::MODE_INPLACE;
  p.q = q;
  p.q_stride_n = q_stride_n;
  p.q_stride_h = q_stride_h;
  p.q_stride_req = q_stride_b;
  p.o = out;
  p.o_stride_n = o_stride_n;
  p.o_stride_h = o_stride_h;
  p.o_stride_req = o_stride_b;
  p.lse = lse;
  p.lse_stride_n = lse_stride_n;
  p.lse_stride_req = lse_stride_b;
  p.sinks = sinks;
  d2sd::KvSource& s0 = p.src[0];
  s0.k = k;
  s0.v = v;
  s0.stride_tok = kv_stride_n;
  s0.stride_head = kv_stride_h;
  s0.stride_req = kv_stride_b;
  s0.mask_mode = causal ? d2sd::MASK_CAUSAL : d2sd::MASK_NONE;
  s0.dtype = d2sd::KV_BF16;
  p.src[1] = s0;
  p.sm_scale = sm_scale;
  p.sm_scale_log2 = sm_scale * kLog2e;
  p.num_kv_heads = num_kv_heads;
  p.group = g;
  p.lse_base2 = lse_base2;
  const int nblocks = bsz * num_kv_heads * p.imp.qtiles;
  hipError_t e = d2sd::launch_attention(p, head_dim, waves, 0, false, false, causal != 0, nblocks,
                                        (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "local_attention_merge launch");
}

int d2sd_graph_begin_capture(d2sd_stream_t stream) {
  g_last_error.clear();
  if (!stream) return fail(D2SD_ERR_INVALID_ARG, "graph capture needs a non-null stream");
  hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "hipStreamBeginCapture");
}

int d2sd_graph_end_capture(d2sd_stream_t stream, void** graph_exec) {
  g_last_error.clear();
  if (!graph_exec) return fail(D2SD_ERR_INVALID_ARG, "graph_exec is null");
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture((hipStream_t)stream, &graph);
  if (e != hipSuccess) return fail_hip(e, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate");
  *graph_exec = (void*)exec;
  return D2SD_OK;
}

int d2sd_graph_launch(void* graph_exec, d2sd_stream_t stream) {
  g_last_error.clear();
  if (!graph_exec) return fail(D2SD_ERR_INVALID_ARG, "graph_exec is null");
  hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "hipGraphLaunch");
}

int d2sd_graph_destroy(void* graph_exec) {
  g_last_error.clear();
  if (!graph_exec) return D2SD_OK;
  hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph_exec);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "hipGraphExecDestroy");
}

// one_wave: the drop-in runner's in-place plans (local_merge_cascade), whose
// suffix items run as one-wave workgroups of 32 rows (waves_per_block 1,
// which the public entry point does not accept: only the in-place kind has
// that shape)
static int cascade_plan_impl(const d2sd_cascade_plan_desc* desc, int32_t* host_plan, size_t host_plan_ints,
                             d2sd_cascade_plan_info* info, bool one_wave) {
  g_last_error.clear();
  if (!desc || !info) return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: null desc/info");
  if (int rc = check_heads(desc->num_qo_heads, desc->num_kv_heads, desc->head_dim)) return rc;
  if (desc->num_reqs <= 0 || !desc->qo_indptr || !desc->prefix_len)
    return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: need num_reqs > 0, qo_indptr and prefix_len");
  if (desc->kv_dtype != D2SD_KV_BF16 && desc->kv_dtype != D2SD_KV_FP8_E4M3)
    return fail(D2SD_ERR_UNSUPPORTED, "cascade_plan: kv_dtype");
  if (desc->waves_per_block != 0 && desc->waves_per_block != 2 && desc->waves_per_block != 4 &&
      desc->waves_per_block != 8 && !(one_wave && desc->waves_per_block == 1))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: waves_per_block must be 0, 2, 4 or 8");
  if (desc->qo_indptr[0] != 0) return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: qo_indptr[0] must be 0");
  for (int r = 0; r < desc->num_reqs; ++r) {
    if (desc->qo_indptr[r + 1] < desc->qo_indptr[r])
      return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: qo_indptr must be non-decreasing");
    if (desc->prefix_len[r] < 0) return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: negative prefix_len");
  }
  if (desc->page_size < 0 || (desc->page_size & (desc->page_size - 1)))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: page_size must be 0 or a power of two");
  if (desc->page_size > 0) {
    if (!desc->page_indptr) return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: paged prefix needs page_indptr");
    for (int r = 0; r < desc->num_reqs; ++r) {
      const long long need = ((long long)desc->prefix_len[r] + desc->page_size - 1) / desc->page_size;
      if (desc->page_indptr[r + 1] - desc->page_indptr[r] < need)
        return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: page_indptr gives a request fewer pages than prefix_len needs");
    }
  }
  if (desc->prefix_split) {
    if (desc->page_size != 0 || desc->dynamic_prefix)
      return fail(D2SD_ERR_UNSUPPORTED, "cascade_plan: a two-segment prefix needs a contiguous prefix and a static plan");
    for (int r = 0; r < desc->num_reqs; ++r) {
      if (desc->prefix_split[r] < 0 || desc->prefix_split[r] > desc->prefix_len[r])
        return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: prefix_split[r] must lie in [0, prefix_len[r]]");
      if (desc->prefix2_tok_indptr && desc->prefix2_tok_indptr[r] < 0)
        return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: negative prefix2_tok_indptr");
    }
  }
  d2sd::VerifyPlanInput in{};
  in.num_reqs = desc->num_reqs;
  in.qo_indptr = desc->qo_indptr;
  in.prefix_len = desc->prefix_len;
  in.page_indptr = desc->page_indptr;
  in.prefix_tok_indptr = desc->prefix_tok_indptr;
  in.num_qo_heads = desc->num_qo_heads;
  in.num_kv_heads = desc->num_kv_heads;
  in.head_dim = desc->head_dim;
  in.window_left = desc->window_left;
  in.num_cus = desc->num_cus > 0 ? desc->num_cus : device_num_cus();
  in.max_splits = desc->max_splits;
  in.waves = desc->waves_per_block;
  in.page_size = desc->page_size;
  in.prefix_split = desc->prefix_split;
  in.prefix2_tok_indptr = desc->prefix2_tok_indptr;
  if (desc->dynamic_prefix != 0 && desc->dynamic_prefix != 1)
    return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: dynamic_prefix must be 0 or 1");
  if (desc->window_left < -1) return fail(D2SD_ERR_INVALID_ARG, "cascade_plan: window_left must be >= -1");
  d2sd::VerifyPlanOutput out{};
  d2sd::plan_verify(in, out);
  if (desc->page_size > 0) {
    // every paged prefix chunk must fit the kernel's staged page ids (the
    // planner bounds chunks by verify_max_chunk_tiles; this is the check)
    int lg = 0;
    while ((1 << lg) < desc->page_size) ++lg;
    for (const auto& w : out.items) {
      if (w.mode == d2sd::MODE_NOOP || w.src == d2sd::SRC_SUFFIX) continue;
      const long long pages = desc->dynamic_prefix
                                  ? ((long long)w.kv_end - w.kv_begin + 63 + desc->page_size - 2) / desc->page_size + 1
                                  : d2sd::pages_spanned(w.kv_begin, w.kv_end, lg);
      if (pages > d2sd::kMaxStagedPages)
        return fail(D2SD_ERR_UNSUPPORTED, "cascade_plan: a prefix chunk spans " + std::to_string(pages) +
                                              " pages, more than the kernel stages (" +
                                              std::to_string(d2sd::kMaxStagedPages) + ")");
    }
  }
  static_assert(sizeof(d2sd::VerifyItem) == 16 * sizeof(int32_t), "VerifyItem layout");
  static_assert(sizeof(d2sd::VerifyMerge) == 8 * sizeof(int32_t), "VerifyMerge layout");
  std::memset(info, 0, sizeof(*info));
  info->num_items = (int)out.items.size();
  info->num_merges = (int)out.merges.size();
  info->waves_per_block = out.waves;
  info->rows_per_tile = out.rows;
  info->num_slots = out.num_slots;
  info->plan_ints = 16 * info->num_items + 8 * info->num_merges;
  info->workspace_bytes = out.workspace_bytes;
  info->max_splits_used = out.max_splits_used;
  info->num_reqs = desc->num_reqs;
  info->num_qo_heads = desc->num_qo_heads;
  info->num_kv_heads = desc->num_kv_heads;
  info->head_dim = desc->head_dim;
  info->kv_dtype = desc->kv_dtype;
  info->page_size = desc->page_size;
  info->num_groups = out.num_groups;
  info->dynamic_prefix = desc->dynamic_prefix;
  info->window_left = desc->window_left;
  info->fused = out.fused;
  int64_t extent = 0, extent2 = 0;
  for (int r = 0; r < desc->num_reqs; ++r) {
    const int len1 = desc->prefix_split ? desc->prefix_split[r] : desc->prefix_len[r];
    const int len2 = desc->prefix_len[r] - len1;
    if (desc->page_size > 0)
      extent = desc->page_indptr[desc->num_reqs];
    else if (len1 > 0)
      extent = std::max<int64_t>(extent, (int64_t)(desc->prefix_tok_indptr ? desc->prefix_tok_indptr[r] : 0) + len1);
    if (len2 > 0)
      extent2 = std::max<int64_t>(extent2,
                                  (int64_t)(desc->prefix2_tok_indptr ? desc->prefix2_tok_indptr[r] : 0) + len2);
  }
  info->prefix_extent = extent;
  info->prefix2_extent = extent2;
  for (const auto& w : out.items) info->two_segment |= w.mode != d2sd::MODE_NOOP && w.src == d2sd::SRC_PREFIX2;
  int max_q = 0;
  for (int r = 0; r < desc->num_reqs; ++r) max_q = std::max(max_q, desc->qo_indptr[r + 1] - desc->qo_indptr[r]);
  info->max_qo_len = max_q;
  if (host_plan) {
    if (host_plan_ints < (size_t)info->plan_ints)
      return fail(D2SD_ERR_WORKSPACE, "cascade_plan: host_plan too small (need " +
                                          std::to_string(info->plan_ints) + " int32)");
    std::memcpy(host_plan, out.items.data(), out.items.size() * sizeof(d2sd::VerifyItem));
    std::memcpy(host_plan + 16 * out.items.size(), out.merges.data(),
                out.merges.size() * sizeof(d2sd::VerifyMerge));
  }
  return D2SD_OK;
}

int d2sd_cascade_plan(const d2sd_cascade_plan_desc* desc, int32_t* host_plan, size_t host_plan_ints,
                      d2sd_cascade_plan_info* info) {
  return cascade_plan_impl(desc, host_plan, host_plan_ints, info, false);
}

// one_wave: the drop-in runner's in-place plans (one-wave workgroups)
static int build_verify_params(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* a,
                               d2sd::VerifyParams& p, bool one_wave = false) {
  if (!info || !a) return fail(D2SD_ERR_INVALID_ARG, "cascade_run: null info/args");
  const int D = info->head_dim;
  if (int rc = check_heads(info->num_qo_heads, info->num_kv_heads, D)) return rc;
  if ((info->waves_per_block != 2 && info->waves_per_block != 4 && info->waves_per_block != 8 &&
       !(one_wave && info->waves_per_block == 1)) ||
      info->rows_per_tile != d2sd::verify_rows(info->waves_per_block))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: info does not come from d2sd_cascade_plan");
  if (!a->plan || !a->q || !a->k_suffix || !a->v_suffix || !a->out)
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: null pointer");
  if (info->num_slots > 0 && (!a->workspace || a->workspace_bytes < info->workspace_bytes))
    return fail(D2SD_ERR_WORKSPACE, "cascade_run: workspace too small (need " +
                                        std::to_string(info->workspace_bytes) + " bytes)");
  if (!aligned16(a->q) || !aligned16(a->k_suffix) || !aligned16(a->v_suffix) || !aligned16(a->out) ||
      !stride_ok(a->q_stride_n) || !stride_ok(a->q_stride_h) || !stride_ok(a->suffix_stride_n) ||
      !stride_ok(a->suffix_stride_h) || !stride_ok(a->o_stride_n) || !stride_ok(a->o_stride_h))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: tensors must be 16-byte aligned with strides % 8 == 0");
  if (info->workspace_bytes > 0 && !aligned16(a->workspace))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: workspace must be 16-byte aligned");
  const bool has_prefix = a->k_prefix != nullptr;
  // (a two-segment plan whose first segment is empty everywhere reads none of k_prefix)
  if (info->max_splits_used > 0 && !has_prefix && !(info->two_segment && info->prefix_extent == 0))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: the plan has prefix keys but k_prefix is null");
  if (has_prefix) {
    if (info->page_size > 0 ? (a->prefix_extent <= 0 || a->prefix_extent > INT32_MAX)
                            : a->prefix_extent < info->prefix_extent)
      return fail(D2SD_ERR_INVALID_ARG, info->page_size > 0
                                            ? "cascade_run: prefix_extent must be the pool's page count"
                                            : "cascade_run: k_prefix holds fewer tokens than the plan reads (need " +
                                                  std::to_string(info->prefix_extent) + ")");
    if (info->dynamic_prefix && !a->prefix_len)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: a dynamic-prefix plan needs the device prefix_len array");
    const int esz = info->kv_dtype == D2SD_KV_FP8_E4M3 ? 1 : 2;
    auto ok = [&](int64_t st) { return (st * esz) % 16 == 0; };
    if (!a->v_prefix || !aligned16(a->k_prefix) || !aligned16(a->v_prefix) || !ok(a->prefix_stride_tok) ||
        !ok(a->prefix_stride_head) || (info->page_size > 0 && !ok(a->prefix_stride_page)))
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: prefix K/V must be 16-byte aligned with 16-byte strides");
    if (a->page_size != info->page_size)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: page_size differs from the planned one");
    if (info->page_size > 0 && !a->page_table)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: paged prefix needs page_table");
  }
  if (a->mask_mode != D2SD_MASK_NONE && a->mask_mode != D2SD_MASK_CAUSAL && a->mask_mode != D2SD_MASK_TREE)
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: mask_mode");
  if (a->mask_mode == D2SD_MASK_TREE && (!a->tree_mask || a->mask_words <= 0))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: tree mask needs tree_mask and mask_words");
  if (a->mask_mode == D2SD_MASK_TREE && (long long)a->mask_words * 64 < info->max_qo_len)
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: mask_words (" + std::to_string(a->mask_words) +
                                          ") must cover the widest request's " + std::to_string(info->max_qo_len) +
                                          " nodes (" + std::to_string((info->max_qo_len + 63) / 64) + " words)");
  if (info->kv_dtype == D2SD_KV_FP8_E4M3 && has_prefix && (!a->k_scale || !a->v_scale))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: fp8 prefix needs k_scale and v_scale");
  if (info->two_segment) {
    const int esz = info->kv_dtype == D2SD_KV_FP8_E4M3 ? 1 : 2;
    if (info->page_size != 0 || info->dynamic_prefix)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: info does not come from d2sd_cascade_plan");
    if (!a->k_prefix2 || !a->v_prefix2)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: the plan reads a second prefix segment; k_prefix2 / v_prefix2 are null");
    if (!aligned16(a->k_prefix2) || !aligned16(a->v_prefix2) || (a->prefix2_stride_tok * esz) % 16 != 0 ||
        (a->prefix2_stride_head * esz) % 16 != 0)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: second prefix segment must be 16-byte aligned with 16-byte strides");
    if (a->prefix2_extent < info->prefix2_extent)
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: k_prefix2 holds fewer tokens than the plan reads (need " +
                                            std::to_string(info->prefix2_extent) + ")");
    if (info->kv_dtype == D2SD_KV_FP8_E4M3 && (!a->k2_scale || !a->v2_scale))
      return fail(D2SD_ERR_INVALID_ARG, "cascade_run: fp8 second prefix segment needs k2_scale and v2_scale");
  }
  if (!(a->sm_scale > 0.f) || !std::isfinite(a->sm_scale))
    return fail(D2SD_ERR_INVALID_ARG, "cascade_run: bad sm_scale");

  p = d2sd::VerifyParams{};
  p.q = a->q;
  p.q_stride_n = a->q_stride_n;
  p.q_stride_h = a->q_stride_h;
  p.o = a->out;
  p.o_stride_n = a->o_stride_n;
  p.o_stride_h = a->o_stride_h;
  p.lse = a->lse;
  p.lse_stride_n = a->lse_stride_n;
  const long long rows = info->rows_per_tile;
  p.part_o = a->workspace;
  p.part_lse = a->workspace ? (float*)((char*)a->workspace + (long long)info->num_slots * rows * D * 2) : nullptr;
  p.items = (const d2sd::VerifyItem*)a->plan;
  p.merges = (const d2sd::VerifyMerge*)(a->plan + 16 * (long long)info->num_items);
  p.prefix_len = info->dynamic_prefix ? a->prefix_len : nullptr;
  p.window_left = info->window_left;
  p.sinks = a->sinks;
  p.tree_mask = (const unsigned long long*)a->tree_mask;
  d2sd::VerifySource& pre = p.pre;
  pre.k = a->k_prefix;
  pre.v = a->v_prefix;
  pre.stride_tok = a->prefix_stride_tok;
  pre.stride_head = a->prefix_stride_head;
  pre.stride_page = a->prefix_stride_page;
  pre.page_table = info->page_size > 0 ? a->page_table : nullptr;
  pre.k_scale = a->k_scale;
  pre.v_scale = a->v_scale;
  int lg = 0;
  while (info->page_size > 0 && (1 << lg) < info->page_size) ++lg;
  pre.log2_page = lg;
  pre.fp8 = info->kv_dtype == D2SD_KV_FP8_E4M3;
  pre.num_pages = info->page_size > 0 ? (int)a->prefix_extent : 0;
  if (info->two_segment) {
    d2sd::VerifySource& pre2 = p.pre2;
    pre2.k = a->k_prefix2;
    pre2.v = a->v_prefix2;
    pre2.stride_tok = a->prefix2_stride_tok;
    pre2.stride_head = a->prefix2_stride_head;
    pre2.k_scale = a->k2_scale;
    pre2.v_scale = a->v2_scale;
    pre2.fp8 = pre.fp8;
  }
  d2sd::VerifySource& suf = p.suf;
  suf.k = a->k_suffix;
  suf.v = a->v_suffix;
  suf.stride_tok = a->suffix_stride_n;
  suf.stride_head = a->suffix_stride_h;
  p.sm_scale = a->sm_scale;
  p.sm_scale_log2 = a->sm_scale * kLog2e;
  p.group = info->num_qo_heads / info->num_kv_heads;
  p.mask_mode = a->mask_mode;
  p.mask_words = a->mask_words;
  p.lse_base2 = a->lse_base2;
  p.num_merges = info->num_merges;
  return D2SD_OK;
}

// ---------------------------------------------------------------------------
// single_prefill_with_kv_cache on the cascade kernels.  With qo_len <= kv_len
// and no window, a single prefill is a one-request cascade: the first
// kv_len - qo_len keys are a contiguous prefix every query sees, the last
// qo_len keys the suffix level, fully visible (non-causal) or a chain
// (causal: query i sees suffix keys 0..i, FlashInfer's bottom-right
// alignment).  The plan is a dynamic-prefix plan for the largest prefix of a
// 512-key bucket of the prefix length kv_len - qo_len, cached per (device,
// qo_len, bucket, heads, head_dim), and the kernel takes the current prefix
// length as an argument, so a cache that grows step by step reuses one plan
// per bucket.  Without a prefix (qo_len == kv_len, e.g. a row's local causal
// attention) the plan has suffix items only, which write the output in one
// launch.  The first call of a shape plans and uploads (hipMalloc and a copy
// on a library-owned stream, see upload_single_plan); when the caller's
// stream is being captured, past kSinglePlanCap cached shapes, or for shapes
// the cascade form does not cover, the caller falls back to the
// single-source kernels.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSingleBucket = 512;
constexpr size_t kSinglePlanCap = 512;

struct SinglePlan {
  d2sd_cascade_plan_info info;
  int32_t* plan_dev;
};

std::mutex g_single_mu;
std::map<std::array<int, 6>, SinglePlan> g_single_plans;      // uploaded plans
std::map<std::array<int, 6>, size_t> g_single_workspace;     // workspace sizes (host planning only)

bool single_cascade_applies(int qo_len, int kv_len, int window_left) {
  return window_left < 0 && qo_len > 0 && qo_len <= kv_len && kv_len <= INT32_MAX - kSingleBucket;
}

// Plans the cascade form on the host; false if it does not apply.
// The planned prefix of a single prefill: kv_len - qo_len rounded up to the bucket.
int single_bucket(int qo_len, int kv_len) {
  const int pre = kv_len - qo_len;
  return (pre + kSingleBucket - 1) / kSingleBucket * kSingleBucket;
}

bool single_cascade_plan(int qo_len, int kv_len, int hq, int hkv, int d, d2sd_cascade_plan_info* info,
                         std::vector<int32_t>* host) {
  const int bucket = single_bucket(qo_len, kv_len);
  int32_t qo_indptr[2] = {0, qo_len}, prefix_len[1] = {bucket}, tok0[1] = {0};
  d2sd_cascade_plan_desc desc{};
  desc.num_reqs = 1;
  desc.qo_indptr = qo_indptr;
  desc.prefix_len = prefix_len;
  desc.prefix_tok_indptr = tok0;
  desc.num_qo_heads = hq;
  desc.num_kv_heads = hkv;
  desc.head_dim = d;
  desc.window_left = -1;
  desc.kv_dtype = D2SD_KV_BF16;
  desc.page_size = 0;
  desc.dynamic_prefix = bucket > 0 ? 1 : 0;
  const std::string saved = g_last_error;
  bool ok = d2sd_cascade_plan(&desc, nullptr, 0, info) == D2SD_OK;
  if (ok && host) {
    host->assign((size_t)info->plan_ints, 0);
    ok = d2sd_cascade_plan(&desc, host->data(), host->size(), info) == D2SD_OK;
  }
  g_last_error = saved;
  return ok;
}

// Device copy of a single-prefill plan (kept until the process ends).  The
// upload may run while a stream of any thread is being captured: this thread
// switches to relaxed capture mode for the allocation, so that it neither
// fails nor invalidates another thread's global-mode capture, and the copy
// goes through a library-owned non-blocking stream, never the legacy null
// stream, which would synchronise with (and so break) a capturing stream.
// *dev stays null (and the caller falls back to the single-source kernels)
// when the allocation fails.
int upload_single_plan(const std::vector<int32_t>& host, int32_t** dev) {
  *dev = nullptr;
  static std::vector<hipStream_t> streams;  // one per device, under g_single_mu
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    (void)hipGetLastError();
    return D2SD_OK;
  }
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) {
    (void)hipGetLastError();
    return D2SD_OK;
  }
  int rc = D2SD_OK;
  int32_t* p = nullptr;
  if ((int)streams.size() <= device) streams.resize(device + 1, nullptr);
  if (!streams[device] && hipStreamCreateWithFlags(&streams[device], hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    streams[device] = nullptr;
  } else if (hipMalloc((void**)&p, host.size() * sizeof(int32_t)) != hipSuccess) {
    (void)hipGetLastError();
    p = nullptr;
  } else {
    hipError_t e = hipMemcpyAsync(p, host.data(), host.size() * sizeof(int32_t), hipMemcpyHostToDevice,
                                  streams[device]);
    if (e == hipSuccess) e = hipStreamSynchronize(streams[device]);
    if (e != hipSuccess) {
      (void)hipFree(p);
      p = nullptr;
      rc = fail_hip(e, "single_prefill: plan upload");
    }
  }
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  *dev = p;
  return rc;
}

}  // namespace

static size_t single_cascade_workspace(int qo_len, int kv_len, int hq, int hkv, int d, int window_left) {
  if (!single_cascade_applies(qo_len, kv_len, window_left)) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) (void)hipGetLastError();
  const int bucket = single_bucket(qo_len, kv_len);
  const std::array<int, 6> key = {dev, qo_len, bucket, hq, hkv, d};
  std::lock_guard<std::mutex> lk(g_single_mu);
  auto it = g_single_workspace.find(key);
  if (it != g_single_workspace.end()) return it->second;
  d2sd_cascade_plan_info info{};
  const size_t ws = single_cascade_plan(qo_len, kv_len, hq, hkv, d, &info, nullptr) ? info.workspace_bytes : 0;
  if (g_single_workspace.size() < 4 * kSinglePlanCap) g_single_workspace.emplace(key, ws);
  return ws;
}

static int single_prefill_cascade(const void* q, int64_t q_stride_n, int64_t q_stride_h, const void* k,
                                  const void* v, int64_t kv_stride_n, int64_t kv_stride_h, void* o,
                                  int64_t o_stride_n, int64_t o_stride_h, float* lse, int qo_len, int kv_len,
                                  int hq, int hkv, int d, int causal, float sm_scale, int lse_base2,
                                  void* workspace, size_t workspace_bytes, hipStream_t stream, bool* used) {
  *used = false;
  if (causal < 0 || !single_cascade_applies(qo_len, kv_len, -1)) return D2SD_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return D2SD_OK;
  }
  const int bucket = single_bucket(qo_len, kv_len);
  const std::array<int, 6> key = {dev, qo_len, bucket, hq, hkv, d};
  SinglePlan sp{};
  {
    std::lock_guard<std::mutex> lk(g_single_mu);
    auto it = g_single_plans.find(key);
    if (it != g_single_plans.end()) {
      sp = it->second;
    } else {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return D2SD_OK;
      }
      if (cs != hipStreamCaptureStatusNone || g_single_plans.size() >= kSinglePlanCap) return D2SD_OK;
      std::vector<int32_t> host;
      if (!single_cascade_plan(qo_len, kv_len, hq, hkv, d, &sp.info, &host)) return D2SD_OK;
      if (int rc = upload_single_plan(host, &sp.plan_dev)) return rc;
      if (!sp.plan_dev) return D2SD_OK;
      g_single_plans.emplace(key, sp);
    }
  }
  if (sp.info.workspace_bytes > workspace_bytes || (sp.info.workspace_bytes > 0 && !workspace))
    return fail(D2SD_ERR_WORKSPACE, "single_prefill: workspace too small (need " +
                                        std::to_string(sp.info.workspace_bytes) + " bytes)");
  const int L = kv_len - qo_len;
  d2sd_cascade_run_args a{};
  a.plan = sp.plan_dev;
  a.q = q;
  a.q_stride_n = q_stride_n;
  a.q_stride_h = q_stride_h;
  a.k_suffix = (const char*)k + (size_t)L * (size_t)kv_stride_n * 2;
  a.v_suffix = (const char*)v + (size_t)L * (size_t)kv_stride_n * 2;
  a.suffix_stride_n = kv_stride_n;
  a.suffix_stride_h = kv_stride_h;
  a.mask_mode = causal ? D2SD_MASK_CAUSAL : D2SD_MASK_NONE;
  const bool has_prefix = sp.info.dynamic_prefix != 0;
  a.k_prefix = has_prefix ? k : nullptr;
  a.v_prefix = has_prefix ? v : nullptr;
  a.prefix_stride_tok = kv_stride_n;
  a.prefix_stride_head = kv_stride_h;
  // the planned extent is the bucket's; the kernels read only the first L keys
  a.prefix_extent = sp.info.prefix_extent;
  a.prefix_len = sp.plan_dev;  // (a dynamic plan needs the field; the value below is used instead)
  a.out = o;
  a.o_stride_n = o_stride_n;
  a.o_stride_h = o_stride_h;
  a.lse = lse;
  a.lse_stride_n = hq;
  a.sm_scale = sm_scale;
  a.lse_base2 = lse_base2;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  d2sd::VerifyParams p{};
  if (int rc = build_verify_params(&sp.info, &a, p)) return rc;
  p.prefix_len = nullptr;
  p.prefix_len_set = has_prefix ? 1 : 0;
  p.prefix_len_value = L;
  hipError_t e = d2sd::launch_verify_attention(p, d, sp.info.waves_per_block, false, false,
                                               sp.info.fused ? d2sd::KIND_FUSED : d2sd::KIND_SPLIT,
                                               sp.info.num_items, stream);
  if (e != hipSuccess) return fail_hip(e, "single_prefill attention launch");
  if (sp.info.num_merges > 0) {
    e = d2sd::launch_verify_merge(p, d, sp.info.rows_per_tile, sp.info.num_merges, stream);
    if (e != hipSuccess) return fail_hip(e, "single_prefill merge launch");
  }
  *used = true;
  return D2SD_OK;
}

// ---------------------------------------------------------------------------
// local_attention_merge on the cascade kernels.  With every tensor laid out
// row after row (batch stride = block_len x token stride), the bsz rows are
// requests without a prefix whose suffix level is the row's own block
// (causal or not): one suffix item per (row, kv head, q-tile), merged in
// place into out / lse (MODE_INPLACE, the KIND_INPLACE kernel).  The plan is
// cached per (device, bsz, block_len, heads, head_dim) and uploaded by the
// first call of a shape (as single_prefill's; a call whose stream is being
// captured, or past kSinglePlanCap shapes, takes the single-source kernel).
// ---------------------------------------------------------------------------
namespace {
std::map<std::array<int, 6>, SinglePlan> g_local_plans;  // under g_single_mu
}

static int local_merge_cascade(const void* q, int64_t q_stride_b, int64_t q_stride_n, int64_t q_stride_h,
                               const void* k, const void* v, int64_t kv_stride_b, int64_t kv_stride_n,
                               int64_t kv_stride_h, void* out, int64_t o_stride_b, int64_t o_stride_n,
                               int64_t o_stride_h, float* lse, int64_t lse_stride_b, int64_t lse_stride_n, int bsz,
                               int block_len, int hq, int hkv, int d, int causal, float sm_scale, const float* sinks,
                               int lse_base2, hipStream_t stream, bool* used) {
  *used = false;
  const int64_t L = block_len;
  if (q_stride_b != L * q_stride_n || kv_stride_b != L * kv_stride_n || o_stride_b != L * o_stride_n ||
      lse_stride_b != L * lse_stride_n || (int64_t)bsz * L > INT32_MAX / 2)
    return D2SD_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return D2SD_OK;
  }
  const std::array<int, 6> key = {dev, bsz, block_len, hq, hkv, d};
  SinglePlan sp{};
  {
    std::lock_guard<std::mutex> lk(g_single_mu);
    auto it = g_local_plans.find(key);
    if (it != g_local_plans.end()) {
      sp = it->second;
    } else {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return D2SD_OK;
      }
      if (cs != hipStreamCaptureStatusNone || g_local_plans.size() >= kSinglePlanCap) return D2SD_OK;
      std::vector<int32_t> qo(bsz + 1), pl(bsz, 0);
      for (int r = 0; r <= bsz; ++r) qo[r] = r * block_len;
      d2sd_cascade_plan_desc desc{};
      desc.num_reqs = bsz;
      desc.qo_indptr = qo.data();
      desc.prefix_len = pl.data();
      desc.num_qo_heads = hq;
      desc.num_kv_heads = hkv;
      desc.head_dim = d;
      desc.window_left = -1;
      desc.kv_dtype = D2SD_KV_BF16;
      // one-wave workgroups of 32 rows: four times the workgroups of a
      // 128-row tile, each loading a quarter of the stored output and Q
      desc.waves_per_block = 1;
      const std::string saved = g_last_error;
      std::vector<int32_t> host;
      bool ok = cascade_plan_impl(&desc, nullptr, 0, &sp.info, true) == D2SD_OK;
      if (ok) {
        host.assign((size_t)sp.info.plan_ints, 0);
        ok = cascade_plan_impl(&desc, host.data(), host.size(), &sp.info, true) == D2SD_OK;
      }
      g_last_error = saved;
      if (!ok || sp.info.num_merges != 0 || sp.info.num_slots != 0) return D2SD_OK;
      // every item is a suffix item writing the output: merge in place instead
      for (int i = 0; i < sp.info.num_items; ++i) {
        d2sd::VerifyItem* w = (d2sd::VerifyItem*)(host.data() + 16 * (size_t)i);
        if (w->mode == d2sd::MODE_FINAL) w->mode = d2sd::MODE_INPLACE;
      }
      if (int rc = upload_single_plan(host, &sp.plan_dev)) return rc;
      if (!sp.plan_dev) return D2SD_OK;
      g_local_plans.emplace(key, sp);
    }
  }
  d2sd_cascade_run_args a{};
  a.plan = sp.plan_dev;
  a.q = q;
  a.q_stride_n = q_stride_n;
  a.q_stride_h = q_stride_h;
  a.k_suffix = k;
  a.v_suffix = v;
  a.suffix_stride_n = kv_stride_n;
  a.suffix_stride_h = kv_stride_h;
  a.mask_mode = causal ? D2SD_MASK_CAUSAL : D2SD_MASK_NONE;
  a.out = out;
  a.o_stride_n = o_stride_n;
  a.o_stride_h = o_stride_h;
  a.lse = lse;
  a.lse_stride_n = lse_stride_n;
  a.sm_scale = sm_scale;
  a.sinks = sinks;
  a.lse_base2 = lse_base2;
  d2sd::VerifyParams p{};
  if (int rc = build_verify_params(&sp.info, &a, p, true)) return rc;
  hipError_t e = d2sd::launch_verify_attention(p, d, sp.info.waves_per_block, false, false, d2sd::KIND_INPLACE,
                                               sp.info.num_items, stream);
  if (e != hipSuccess) return fail_hip(e, "local_attention_merge launch");
  *used = true;
  return D2SD_OK;
}

int d2sd_cascade_attention(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* a,
                           d2sd_stream_t stream) {
  g_last_error.clear();
  d2sd::VerifyParams p{};
  if (int rc = build_verify_params(info, a, p)) return rc;
  hipError_t e = d2sd::launch_verify_attention(p, info->head_dim, info->waves_per_block, info->page_size > 0,
                                               info->kv_dtype == D2SD_KV_FP8_E4M3,
                                               info->two_segment ? d2sd::KIND_SEGMENTS
                                               : info->fused     ? d2sd::KIND_FUSED
                                                                 : d2sd::KIND_SPLIT,
                                               info->num_items,
                                               (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "cascade attention launch");
}

int d2sd_cascade_merge(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  d2sd::VerifyParams p{};
  if (int rc = build_verify_params(info, a, p)) return rc;
  hipError_t e = d2sd::launch_verify_merge(p, info->head_dim, info->rows_per_tile, info->num_merges,
                                           (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "cascade merge launch");
}

int d2sd_cascade_run(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* a, d2sd_stream_t stream) {
  if (int rc = d2sd_cascade_attention(info, a, stream)) return rc;
  return d2sd_cascade_merge(info, a, stream);
}

size_t d2sd_cascade_scratch_bytes(void) { return (size_t)d2sd::kVerifyScratchBytes; }

int d2sd_cascade_run_noalloc(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* a,
                             d2sd_stream_t stream) {
  g_last_error.clear();
  if (!info || !a) return fail(D2SD_ERR_INVALID_ARG, "cascade_run_noalloc: null info/args");
  if (info->workspace_bytes > d2sd::kVerifyScratchBytes)
    return fail(D2SD_ERR_WORKSPACE, "cascade_run_noalloc: the plan needs " + std::to_string(info->workspace_bytes) +
                                        " bytes of partial states, more than the library's " +
                                        std::to_string(d2sd::kVerifyScratchBytes) + "-byte workspace");
  void* ws = nullptr;
  if (hipError_t e = d2sd::verify_scratch(&ws)) return fail_hip(e, "cascade_run_noalloc: workspace lookup");
  d2sd_cascade_run_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = (size_t)d2sd::kVerifyScratchBytes;
  if (int rc = d2sd_cascade_attention(info, &b, stream)) return rc;
  return d2sd_cascade_merge(info, &b, stream);
}

// Candidate-tree build (replaces generation/d3_generator.py:116-180).
int d2sd_d3_tree_build(const d2sd_d3_tree_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  if (!a) return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: null args");
  if (a->block_size < 2 || a->block_size > 65 || a->block_size_2 < a->block_size || a->topk < 1)
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: need 2 <= block_size <= 65, block_size_2 >= block_size, topk >= 1");
  if (a->conf_dtype != D2SD_DTYPE_BF16 && a->conf_dtype != D2SD_DTYPE_F32)
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: conf_dtype must be D2SD_DTYPE_BF16 or D2SD_DTYPE_F32");
  const int k = std::min(a->topk, a->block_size - 1);
  const long long worst = (long long)a->block_size_2 + (long long)k * (a->block_size_2 - 1);
  if (a->capacity < worst || a->capacity > (1 << 24))
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: capacity must hold the largest tree (" + std::to_string(worst) +
                                          " nodes)");
  if (a->rows_cap < k + 1 || a->rows_cap > d2sd::kTreeMaxRows)
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: rows_cap must be in [min(topk, block_size - 1) + 1, 65]");
  if ((long long)a->mask_words * 64 < a->capacity)
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: mask_words too small for capacity");
  if (!a->conf || !a->num_nodes || !a->parents || !a->node_index || !a->tree_mask)
    return fail(D2SD_ERR_INVALID_ARG, "d3_tree_build: null pointer");
  d2sd::TreeBuildParams p{};
  p.conf = a->conf;
  p.conf_bf16 = a->conf_dtype == D2SD_DTYPE_BF16 ? 1 : 0;
  p.block_size = a->block_size;
  p.block_size_2 = a->block_size_2;
  p.topk = a->topk;
  p.capacity = a->capacity;
  p.rows_cap = a->rows_cap;
  p.mask_words = a->mask_words;
  p.num_nodes = a->num_nodes;
  p.num_rows = a->num_rows;
  p.parents = a->parents;
  p.node_index = a->node_index;
  p.tree_mask = (unsigned long long*)a->tree_mask;
  p.shared = a->shared;
  p.rates = a->rates;
  hipError_t e = d2sd::launch_d3_tree_build(p, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "d3_tree_build launch");
}

// QK RMSNorm + RoPE (replaces generation/verification.py:113-123).
int d2sd_qk_norm_rope(const d2sd_qk_norm_rope_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  if (!a) return fail(D2SD_ERR_INVALID_ARG, "qk_norm_rope: null args");
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(D2SD_ERR_UNSUPPORTED, "qk_norm_rope: head_dim must be 64, 128 or 256");
  if (a->num_tokens < 0 || a->num_qo_heads < 0 || a->num_kv_heads < 0)
    return fail(D2SD_ERR_INVALID_ARG, "qk_norm_rope: negative count");
  if ((a->num_qo_heads > 0 && !a->q) || (a->num_kv_heads > 0 && !a->k))
    return fail(D2SD_ERR_INVALID_ARG, "qk_norm_rope: null q or k");
  if ((a->cos == nullptr) != (a->sin == nullptr))
    return fail(D2SD_ERR_INVALID_ARG, "qk_norm_rope: cos and sin go together");
  if (!(a->eps >= 0.f)) return fail(D2SD_ERR_INVALID_ARG, "qk_norm_rope: eps must be >= 0");
  d2sd::QkRopeParams p{};
  p.q = a->q;
  p.k = a->k;
  p.q_stride_n = a->q_stride_n;
  p.q_stride_h = a->q_stride_h;
  p.k_stride_n = a->k_stride_n;
  p.k_stride_h = a->k_stride_h;
  p.q_norm = a->q_norm;
  p.k_norm = a->k_norm;
  p.cos = a->cos;
  p.sin = a->sin;
  p.cs_stride = a->cs_stride;
  p.eps = a->eps;
  p.num_tokens = a->num_tokens;
  p.num_qo_heads = a->num_qo_heads;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.half_cos = a->half_cos ? 1 : 0;
  hipError_t e = d2sd::launch_qk_norm_rope(p, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "qk_norm_rope launch");
}

// Greedy acceptance walk (replaces generation/d3_generator.py:204-225 at temperature 0).
size_t d2sd_greedy_accept_workspace_size(int num_nodes, int vocab) {
  if (num_nodes <= 0 || vocab <= 0) return 0;
  int chunks = 1, chunk_len = 8;
  d2sd::greedy_accept_chunks(num_nodes, vocab, chunks, chunk_len);
  return (size_t)num_nodes * chunks * sizeof(unsigned long long);
}

namespace {

// Checks the walk's arguments and fills its parameters (sampling fields zero).
int walk_params(const d2sd_greedy_accept_args* a, d2sd::AcceptParams& p) {
  if (!a) return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: null args");
  if (a->num_rows < 1 || a->num_rows > 64)
    return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: num_rows must be in [1, 64]");
  if (a->row_len < 1 || a->num_nodes < 1 || a->vocab < 1)
    return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: row_len, num_nodes and vocab must be positive");
  if (a->num_nodes > d2sd::kAcceptMaxNodes || a->num_rows * a->row_len > d2sd::kAcceptMaxCells)
    return fail(D2SD_ERR_UNSUPPORTED, "greedy_accept: at most 4096 nodes and 2048 row positions");
  if (a->logits_dtype != D2SD_DTYPE_BF16 && a->logits_dtype != D2SD_DTYPE_F32)
    return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: logits_dtype must be D2SD_DTYPE_BF16 or D2SD_DTYPE_F32");
  if (a->logits_stride < a->vocab)
    return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: logits_stride must be >= vocab");
  if (!a->logits || !a->node_index || !a->draft_ids || !a->accept_ids || !a->accept_nodes || !a->result ||
      !a->workspace)
    return fail(D2SD_ERR_INVALID_ARG, "greedy_accept: null pointer");
  if (a->workspace_bytes < d2sd_greedy_accept_workspace_size(a->num_nodes, a->vocab))
    return fail(D2SD_ERR_WORKSPACE, "greedy_accept: workspace too small (need " +
                                        std::to_string(d2sd_greedy_accept_workspace_size(a->num_nodes, a->vocab)) +
                                        " bytes)");
  p = d2sd::AcceptParams{};
  p.logits = a->logits;
  p.logits_stride = a->logits_stride;
  p.node_index = a->node_index;
  p.draft_ids = (const long long*)a->draft_ids;
  p.accept_ids = (long long*)a->accept_ids;
  p.accept_nodes = a->accept_nodes;
  p.result = a->result;
  p.keys = (unsigned long long*)a->workspace;
  p.num_rows = a->num_rows;
  p.row_len = a->row_len;
  p.num_nodes = a->num_nodes;
  p.vocab = a->vocab;
  d2sd::greedy_accept_chunks(a->num_nodes, a->vocab, p.chunks, p.chunk_len);
  return D2SD_OK;
}

}  // namespace

int d2sd_greedy_accept(const d2sd_greedy_accept_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  d2sd::AcceptParams p;
  if (int rc = walk_params(a, p)) return rc;
  hipError_t e = d2sd::launch_greedy_accept(p, a->logits_dtype == D2SD_DTYPE_BF16, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "greedy_accept launch");
}

// The walk at any temperature (generation/d3_generator.py:204-225 with
// model/utils.py:28-37).
int d2sd_sample_accept(const d2sd_sample_accept_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  if (!a) return fail(D2SD_ERR_INVALID_ARG, "sample_accept: null args");
  if (!(a->temperature >= 0.f) || !std::isfinite(a->temperature))
    return fail(D2SD_ERR_INVALID_ARG, "sample_accept: temperature must be finite and >= 0");
  d2sd::AcceptParams p;
  if (int rc = walk_params(&a->walk, p)) return rc;
  p.node_tokens = (long long*)a->node_tokens;
  if (a->temperature >= 1e-5f) {
    if (!a->rng_step) return fail(D2SD_ERR_INVALID_ARG, "sample_accept: rng_step is required when sampling");
    p.inv_temperature = 1.f / a->temperature;
    p.seed_lo = (unsigned)(a->seed & 0xFFFFFFFFull);
    p.seed_hi = (unsigned)(a->seed >> 32);
    p.rng_step = (long long*)a->rng_step;
  }
  hipError_t e = d2sd::launch_greedy_accept(p, a->walk.logits_dtype == D2SD_DTYPE_BF16, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "sample_accept launch");
}

// Accepted-branch KV commit (replaces generation/d3_generator.py:227-232).
int d2sd_paged_kv_append(const d2sd_kv_append_args* a, d2sd_stream_t stream) {
  g_last_error.clear();
  if (!a) return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: null args");
  if (a->num_accepted < 0 || a->num_layers < 0 || a->prefix_len < 0)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: negative count");
  if (a->num_accepted == 0 || a->num_layers == 0) return D2SD_OK;
  if (a->num_kv_heads <= 0 || a->head_dim <= 0 || a->head_dim % 8 != 0)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: head_dim must be a positive multiple of 8");
  if (a->page_size <= 0 || (a->page_size & (a->page_size - 1)) != 0)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: page_size must be a power of two");
  if (a->num_rows <= 0 || a->pool_pages <= 0)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: num_rows and pool_pages must be positive");
  if (!a->node_ids || !a->page_table || !a->k_new || !a->v_new || !a->k_pool || !a->v_pool)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: null pointer");
  const int64_t strides[5] = {a->new_stride_n, a->new_stride_h, a->pool_stride_page, a->pool_stride_head,
                              a->pool_stride_tok};
  for (int64_t st : strides)
    if (st <= 0 || st % 8 != 0)
      return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: strides must be positive multiples of 8 elements");
  if ((int64_t)a->prefix_len + a->num_accepted > (int64_t)INT32_MAX)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: cache position overflows int32");
  if (!a->prefix_len_dev &&
      ((int64_t)a->prefix_len + a->num_accepted + a->page_size - 1) / a->page_size > (int64_t)a->page_table_len)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: page_table does not cover prefix_len + num_accepted");
  if (a->page_table_len <= 0) return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: empty page_table");
  if (a->advance_prefix && !a->prefix_len_dev)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: advance_prefix needs prefix_len_dev");
  if (a->pool_dtype != D2SD_KV_BF16 && a->pool_dtype != D2SD_KV_FP8_E4M3)
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: pool_dtype must be D2SD_KV_BF16 or D2SD_KV_FP8_E4M3");
  if (a->pool_dtype == D2SD_KV_FP8_E4M3 && (!a->k_scale || !a->v_scale))
    return fail(D2SD_ERR_INVALID_ARG, "paged_kv_append: fp8 pools need k_scale and v_scale");
  d2sd::KvAppendParams p{};
  p.node_ids = a->node_ids;
  p.page_table = a->page_table;
  p.k_new = a->k_new;
  p.v_new = a->v_new;
  p.k_pool = a->k_pool;
  p.v_pool = a->v_pool;
  p.new_stride_n = a->new_stride_n;
  p.new_stride_h = a->new_stride_h;
  p.pool_stride_page = a->pool_stride_page;
  p.pool_stride_head = a->pool_stride_head;
  p.pool_stride_tok = a->pool_stride_tok;
  p.num_layers = a->num_layers;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  int lg = 0;
  while ((1 << lg) < a->page_size) ++lg;
  p.log2_page = lg;
  p.prefix_len = a->prefix_len;
  p.num_accepted = a->num_accepted;
  p.num_rows = a->num_rows;
  p.pool_pages = a->pool_pages;
  p.num_accepted_dev = a->num_accepted_dev;
  p.prefix_len_dev = a->prefix_len_dev;
  p.page_table_len = a->page_table_len;
  p.pool_dtype = a->pool_dtype == D2SD_KV_FP8_E4M3 ? d2sd::KV_FP8 : d2sd::KV_BF16;
  p.k_scale = a->k_scale;
  p.v_scale = a->v_scale;
  hipError_t e = d2sd::launch_kv_append(p, a->advance_prefix != 0, (hipStream_t)stream);
  return e == hipSuccess ? D2SD_OK : fail_hip(e, "paged_kv_append launch");
}

}  // extern "C"
