/*
 * d2sd.h — C ABI of the MI355X (gfx950) cascade tree-verification attention
 * library `libd2sd.so`.
 *
 * Every entry point takes raw device pointers, element strides (int64, in
 * units of elements, not bytes), plain sizes and a hipStream_t, and returns
 * 0 (D2SD_OK) or a non-zero status; d2sd_last_error() then holds a message.
 * Scratch space is caller-provided (d2sd_cascade_run_noalloc uses a
 * library-owned array instead).  Device memory is allocated in two places
 * only: d2sd_graph_end_capture (the graph executable) and the first
 * d2sd_single_prefill_with_kv_cache call of each shape, which plans and
 * uploads that shape's work list once (hipMalloc plus a synchronous copy on a
 * library-owned stream, in relaxed capture mode so that a capture running on
 * another thread is not disturbed; kept until the process ends, at most 512
 * shapes).  When the caller's stream is being captured that first call takes
 * the single-source kernels instead, which allocate nothing.  The other launch
 * entry points never synchronise the host, so they may be captured into a
 * hipGraph.
 *
 * Tensor conventions (all bf16 = bfloat16, lse = float32):
 *   q   : [qo_len, num_qo_heads, head_dim]      (NHD; head_dim contiguous)
 *   k,v : [kv_len, num_kv_heads, head_dim]      (NHD), or any layout
 *         expressible with (stride_tok, stride_head) — e.g. the
 *         [num_kv_heads, kv_len, head_dim] DynamicCache layout (HND)
 *   o   : like q
 *   lse : [qo_len, num_qo_heads], natural log unless lse_base2 != 0
 * Query head h reads kv head h / (num_qo_heads / num_kv_heads)  (GQA).
 * head_dim must be 64 or 128; pointers must be 16-byte aligned and every
 * stride a multiple of 8 elements.
 */
#ifndef D2SD_H_
#define D2SD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* d2sd_stream_t; /* == hipStream_t */

#define D2SD_OK 0
#define D2SD_ERR_INVALID_ARG 1
#define D2SD_ERR_UNSUPPORTED 2
#define D2SD_ERR_WORKSPACE 3
#define D2SD_ERR_HIP 4

#define D2SD_KV_BF16 0
#define D2SD_KV_FP8_E4M3 1 /* OCP e4m3fn bytes, dequantised with per-kv-head fp32 scales */

#define D2SD_MASK_NONE 0
#define D2SD_MASK_CAUSAL 1 /* key j visible to query i iff j <= i + (kv_len - qo_len) */
#define D2SD_MASK_TREE 2   /* ancestor bitmask, see d2sd_cascade_run_args */

/* Message for the last failed call on this thread ("" if none). */
const char* d2sd_last_error(void);
/* Library version string. */
const char* d2sd_version(void);

/* ------------------------------------------------------------------------
 * merge_state_in_place
 * Replaces flashinfer.merge_state_in_place(v, s, v_other, s_other) as called
 * at generation/verification.py:163-165, model/cascade_graph.py:58-60 and
 * model/dflash.py:131-133.
 *   s' = logaddexp(s, s_other);  v' = v*e^(s-s') + v_other*e^(s_other-s')
 * v: [seq_len, num_heads, head_dim] bf16 (updated), s: [seq_len, num_heads]
 * fp32 (updated).  An operand with lse = -inf contributes nothing.
 * ---------------------------------------------------------------------- */
int d2sd_merge_state_in_place(void* v, int64_t v_stride_n, int64_t v_stride_h,
                              float* s, int64_t s_stride_n,
                              const void* v_other, int64_t vo_stride_n, int64_t vo_stride_h,
                              const float* s_other, int64_t so_stride_n,
                              int seq_len, int num_heads, int head_dim, int lse_base2,
                              d2sd_stream_t stream);

/* ------------------------------------------------------------------------
 * single_prefill_with_kv_cache
 * Replaces flashinfer.single_prefill_with_kv_cache(q, k, v, causal=...,
 * return_lse=True, sm_scale=...) as called at generation/verification.py:145
 * (shared prefix, causal=False), verification.py:159 (per-branch local,
 * causal=True), model/cascade_graph.py:54 and model/dflash.py:112,127.
 * window_left >= 0 keeps only the last window_left keys for every query
 * (the prefix truncation rule of generation/verification.py:133-135);
 * -1 disables it.  lse may be NULL.  The workspace (device memory, at least
 * d2sd_single_prefill_workspace_size() bytes) holds split-KV partials.
 * With window_left < 0 and 0 < qo_len <= kv_len the call runs as a
 * one-request cascade (the first kv_len - qo_len keys a shared prefix, the
 * last qo_len keys the suffix level, fully visible or causal): the first
 * call of a (device, qo_len, 512-key bucket of kv_len - qo_len, heads,
 * head_dim) shape plans it and uploads the plan to device memory the library
 * keeps until the process ends (at most 512 shapes); a first call under
 * stream capture, later shapes and other calls use the single-source kernel.
 * ---------------------------------------------------------------------- */
size_t d2sd_single_prefill_workspace_size(int qo_len, int kv_len, int num_qo_heads,
                                          int num_kv_heads, int head_dim, int window_left);
int d2sd_single_prefill_with_kv_cache(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                      const void* k, const void* v,
                                      int64_t kv_stride_n, int64_t kv_stride_h,
                                      void* o, int64_t o_stride_n, int64_t o_stride_h,
                                      float* lse, int qo_len, int kv_len, int num_qo_heads,
                                      int num_kv_heads, int head_dim, int causal,
                                      int window_left, float sm_scale, int lse_base2,
                                      void* workspace, size_t workspace_bytes,
                                      d2sd_stream_t stream);

/* ------------------------------------------------------------------------
 * local_attention_merge
 * One launch for the whole per-row loop that CascadeGraphRunner captures
 * (model/cascade_graph.py:52-60): for every row i < bsz,
 *   (o_l, lse_l) = attention(q[i], k[i], v[i], causal)   (block_len x block_len)
 *   merge_state_in_place(out[i], lse[i], o_l, lse_l)
 * q/out: [bsz, block_len, num_qo_heads, head_dim]; k/v: [bsz, block_len,
 * num_kv_heads, head_dim]; lse: [bsz, block_len, num_qo_heads] fp32.
 * sinks (nullable, [num_qo_heads] fp32) additionally applies the GPT-OSS
 * rescale out *= sigmoid(lse - sink) of generation/verification.py:173-176
 * after the merge (lse itself keeps the merged value).
 * ---------------------------------------------------------------------- */
int d2sd_local_attention_merge(const void* q, int64_t q_stride_b, int64_t q_stride_n,
                               int64_t q_stride_h, const void* k, const void* v,
                               int64_t kv_stride_b, int64_t kv_stride_n, int64_t kv_stride_h,
                               void* out, int64_t o_stride_b, int64_t o_stride_n,
                               int64_t o_stride_h, float* lse, int64_t lse_stride_b,
                               int64_t lse_stride_n, int bsz, int block_len, int num_qo_heads,
                               int num_kv_heads, int head_dim, int causal, float sm_scale,
                               const float* sinks, int lse_base2, d2sd_stream_t stream);

/* ------------------------------------------------------------------------
 * hipGraph capture / replay owned by the library.
 * Replaces torch.cuda.CUDAGraph capture (model/cascade_graph.py:67-71) and
 * replay (cascade_graph.py:107).  Capture runs on `stream` (which must not
 * be the null stream) in thread-local capture mode.
 * ---------------------------------------------------------------------- */
int d2sd_graph_begin_capture(d2sd_stream_t stream);
int d2sd_graph_end_capture(d2sd_stream_t stream, void** graph_exec);
int d2sd_graph_launch(void* graph_exec, d2sd_stream_t stream);
int d2sd_graph_destroy(void* graph_exec);

/* ------------------------------------------------------------------------
 * Cascade verify attention: plan() / run().
 * No reference counterpart calls a plan(); this pair is the single-call form
 * of generation/verification.py:127-176 (prefix fetch + window, shared-prefix
 * attention, per-branch attention, merge, GPT-OSS sink) over a token TREE of
 * unique candidate nodes instead of bsz duplicated rows, for a batch of
 * requests.
 *
 * Request r owns query/suffix tokens [qo_indptr[r], qo_indptr[r+1]) of q,
 * k_suffix, v_suffix, out and lse, and a prefix of prefix_len[r] keys.
 * Suffix key j is visible to suffix query i of request r iff bit j of
 *   tree_mask[(qo_indptr[r] + i) * mask_words + j / 64]
 * is set (bit (j % 64), little-endian 64-bit words).  mask_mode may instead
 * be D2SD_MASK_CAUSAL (chain: key j visible iff j <= i) or D2SD_MASK_NONE (all
 * suffix keys visible, the non-causal DTA-draft case of
 * model/dflash.py:127-130).
 *
 * The prefix is either contiguous (page_size == 0): key t of request r at
 *   k_prefix + (prefix_tok_indptr[r] + t)*prefix_stride_tok + h*prefix_stride_head
 * (prefix_tok_indptr may be NULL: all requests then start at token 0), or
 * paged (page_size a power of two): key t at
 *   k_prefix + page_table[page_indptr[r] + t/page_size]*prefix_stride_page
 *            + (t % page_size)*prefix_stride_tok + h*prefix_stride_head.
 * window_left >= 0 keeps the last window_left prefix keys (all queries).
 *
 * Two-segment prefix (prefix_split != NULL; contiguous first segment, static
 * plans): the prefix of request r is the concatenation
 *   [keys 0 .. prefix_split[r]) of k_prefix as above
 *   | keys 0 .. prefix_len[r] - prefix_split[r]) of k_prefix2,
 * key u of the second segment at
 *   k_prefix2 + (prefix2_tok_indptr[r] + u)*prefix2_stride_tok + h*prefix2_stride_head
 * (prefix2_tok_indptr may be NULL: 0).  This is the DTA draft's shared level
 * [draft cache | projected target context] (model/dflash.py:103-106) read in
 * place instead of concatenated; the window applies to the concatenation.
 *
 * plan() bakes every per-request offset into a work list the caller uploads;
 * run() is the attention launch (prefix key chunks and suffix trees, each
 * writing a partial state to the workspace, or the output directly when a
 * request has no prefix) and a merge launch (log-sum-exp merge + sink into
 * out / lse).
 * run() allocates nothing and never synchronises the host, so it may be
 * captured into a hipGraph; the device plan, page_table contents and tensors
 * may change between replays as long as the plan's shape does not.
 *
 * Growing prefixes (dynamic_prefix = 1): plan() then takes prefix_len[r] as
 * the largest prefix request r will have, and run() reads the current length
 * of each request from the device array args.prefix_len (clamped to
 * [0, planned length]), so one captured graph replays while the cache grows
 * step by step (the page table must hold the pages of the current length).
 * The planned key chunks are scaled to the current span (each boundary
 * b -> floor(b * span / planned_span) rounded down to 64 keys, the last at the
 * span's end), so every workgroup keeps its share of the work at any length.
 *
 * Paged page ids are clamped below args.prefix_extent (the pool's page
 * count): an id outside the pool reads a wrong page but never memory outside
 * the pool.  Q, K and V must be NaN-free (the kernels are built without NaN
 * semantics); the result of a NaN input is undefined but stays in bounds.
 * ---------------------------------------------------------------------- */
typedef struct {
  int num_reqs;
  const int32_t* qo_indptr;         /* host, [num_reqs + 1] */
  const int32_t* prefix_len;        /* host, [num_reqs] */
  const int32_t* page_indptr;       /* host, [num_reqs + 1]; required when page_size > 0 */
  const int32_t* prefix_tok_indptr; /* host, [num_reqs]; contiguous prefix, nullable */
  int num_qo_heads;
  int num_kv_heads;
  int head_dim;
  int window_left;     /* -1: full prefix */
  int kv_dtype;        /* D2SD_KV_* of the prefix cache */
  int page_size;       /* 0: contiguous prefix; else the pool's page size */
  int num_cus;         /* 0: query the device */
  int max_splits;      /* 0: default cap */
  int waves_per_block; /* 0 = choose; 2 (64-row waves, 128-row tiles), 4 (32-row
                          waves, 128-row tiles) or 8 (32-row waves, 256-row tiles) */
  int dynamic_prefix;  /* 1: prefix_len is each request's largest prefix; run()
                          reads the current lengths from args.prefix_len */
  const int32_t* prefix_split;       /* host [num_reqs], nullable: two-segment
                                        prefix, 0 <= prefix_split[r] <= prefix_len[r]
                                        (page_size 0, dynamic_prefix 0) */
  const int32_t* prefix2_tok_indptr; /* host [num_reqs], nullable: token of the
                                        second segment's key 0 of request r */
} d2sd_cascade_plan_desc;

typedef struct {
  int num_items;        /* workgroups of the attention launch */
  int num_merges;       /* groups merged by the merge launch */
  int waves_per_block;
  int rows_per_tile;    /* packed (query, head) rows per workgroup and partial slot */
  int num_slots;        /* partial slots in the workspace */
  int plan_ints;        /* int32 entries written to host_plan */
  size_t workspace_bytes;
  int max_splits_used;  /* prefix key chunks of the most-split request */
  int num_reqs;
  int num_qo_heads;
  int num_kv_heads;
  int head_dim;
  int kv_dtype;
  int page_size;
  int num_groups;         /* (request, kv head, q-tile) groups */
  int dynamic_prefix;     /* the plan's dynamic_prefix */
  int window_left;        /* the plan's window_left */
  int64_t prefix_extent;  /* contiguous prefix: tokens k_prefix must hold
                             (max_r prefix_tok_indptr[r] + prefix_len[r]);
                             paged: page_table entries the plan reads */
  int max_qo_len;         /* nodes of the widest request: a tree mask needs
                             mask_words >= ceil(max_qo_len / 64) */
  int fused;              /* 1: no request's prefix is split; each workgroup
                             reads its rows' prefix and then their suffix tree
                             and writes out / lse (run() is one launch, no
                             workspace) */
  int two_segment;        /* 1: the plan reads keys of a second prefix segment
                             (run() then needs k_prefix2 / v_prefix2) */
  int64_t prefix2_extent; /* tokens k_prefix2 must hold
                             (max_r prefix2_tok_indptr[r] + prefix_len[r] - prefix_split[r]) */
} d2sd_cascade_plan_info;

/* Fills host_plan (capacity host_plan_ints int32) with the work list; the
 * caller copies these plan_ints int32 values to device memory and passes that
 * pointer to d2sd_cascade_run.  Pass host_plan = NULL to only fill info. */
int d2sd_cascade_plan(const d2sd_cascade_plan_desc* desc, int32_t* host_plan,
                      size_t host_plan_ints, d2sd_cascade_plan_info* info);

typedef struct {
  const int32_t* plan;      /* device copy of the host plan */
  const void* q;            /* [total_q, Hq, D] bf16 */
  int64_t q_stride_n, q_stride_h;
  const void* k_suffix;     /* [total_q, Hkv, D] bf16 */
  const void* v_suffix;
  int64_t suffix_stride_n, suffix_stride_h;
  int mask_mode;            /* D2SD_MASK_* for the suffix level */
  int mask_words;           /* 64-bit words per tree-mask row (>= ceil(info.max_qo_len / 64)) */
  const uint64_t* tree_mask;
  const void* k_prefix;     /* bf16 or fp8 bytes; NULL when no request has a prefix */
  const void* v_prefix;
  int64_t prefix_stride_tok, prefix_stride_head, prefix_stride_page;
  int page_size;            /* must equal the planned page size */
  const int32_t* page_table;/* device (paged) */
  int64_t prefix_extent;    /* contiguous: tokens in k_prefix (>= info.prefix_extent);
                               paged: pages in the pool */
  const int32_t* prefix_len;/* device [num_reqs]: current prefix lengths
                               (dynamic plans; ignored otherwise) */
  const float* k_scale;     /* fp8: [Hkv] */
  const float* v_scale;
  const float* sinks;       /* nullable, [Hq] */
  void* out;                /* [total_q, Hq, D] bf16 */
  int64_t o_stride_n, o_stride_h;
  float* lse;               /* nullable, [total_q, Hq] */
  int64_t lse_stride_n;
  float sm_scale;
  int lse_base2;
  void* workspace;          /* >= info.workspace_bytes */
  size_t workspace_bytes;
  const void* k_prefix2;    /* second prefix segment (info.two_segment): contiguous,
                               the prefix's dtype; NULL otherwise */
  const void* v_prefix2;
  int64_t prefix2_stride_tok, prefix2_stride_head;
  int64_t prefix2_extent;   /* tokens in k_prefix2 (>= info.prefix2_extent) */
  const float* k2_scale;    /* fp8: [Hkv] scales of the second segment */
  const float* v2_scale;
} d2sd_cascade_run_args;

/* run = attention launch then merge launch; both halves are also exported. */
int d2sd_cascade_run(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* args,
                     d2sd_stream_t stream);
int d2sd_cascade_attention(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* args,
                           d2sd_stream_t stream);
int d2sd_cascade_merge(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* args,
                       d2sd_stream_t stream);

/* d2sd_cascade_run without a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * partial states live in a library-owned device array of
 * d2sd_cascade_scratch_bytes() bytes (32 MiB) per GPU, kept until the process
 * ends; args.workspace / workspace_bytes are ignored, and a plan whose
 * info.workspace_bytes exceeds the array is rejected (D2SD_ERR_WORKSPACE).
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other threads) race.  Nothing in it needs clearing: each
 * partial state is written by its producer before the merge reads it.
 * The first call on a device looks the array's address up; later calls make
 * no runtime call besides the two launches. */
size_t d2sd_cascade_scratch_bytes(void);
int d2sd_cascade_run_noalloc(const d2sd_cascade_plan_info* info, const d2sd_cascade_run_args* args,
                             d2sd_stream_t stream);

/* ----------------------------------------------------------------------
 * Accepted-branch KV commit into the paged prefix cache.
 * Replaces generation/d3_generator.py:227-232: per layer
 *   layer.keys = torch.cat([layer.keys, k_win], dim=2)   (values alike),
 * k_win = the accepted row's first acceptance_length new keys, which copies
 * the whole cache every step.  Here token i of the accepted branch (row
 * node_ids[i] of every layer's k_new / v_new) is written to cache position
 * prefix_len + i: page page_table[(prefix_len + i) / page_size], slot
 * (prefix_len + i) % page_size, for all layers in one launch.  The page
 * table must already hold the pages for prefix_len + num_accepted tokens.
 * With prefix_len_dev the length lives on the device and may advance there,
 * so one captured commit replays step after step.
 * Node ids outside [0, num_rows) and page ids outside [0, pool_pages) are
 * skipped (nothing written).  Pools are bf16, or (pool_dtype =
 * D2SD_KV_FP8_E4M3) e4m3fn bytes holding value / scale[kv head], the format
 * d2sd_cascade_run reads: each new bf16 value x is stored as
 * e4m3fn(clamp(x / scale, -448, 448)), the quotient correctly rounded in fp32
 * and the byte rounded to nearest even (torch's float8_e4m3fn cast after the
 * clamp).  Strides in elements must be multiples of 8, new rows 16-byte and
 * pool rows 16-byte (bf16) or 8-byte (fp8) aligned.  No allocation, no host
 * synchronisation (capturable).
 * ---------------------------------------------------------------------- */
typedef struct {
  int num_layers;
  int num_kv_heads;
  int head_dim;              /* multiple of 8 */
  int page_size;             /* power of two */
  int prefix_len;            /* tokens already cached */
  int num_accepted;          /* tokens appended */
  int num_rows;              /* rows of each k_new / v_new */
  int pool_pages;            /* pages of each pool */
  int page_table_len;        /* entries of page_table; must cover prefix_len + num_accepted */
  const int32_t* node_ids;   /* device [num_accepted] */
  const int32_t* page_table; /* device, the request's pages */
  const uint64_t* k_new;     /* device [num_layers]: addresses of bf16 [rows, Hkv, D] */
  const uint64_t* v_new;
  const uint64_t* k_pool;    /* device [num_layers]: addresses of the bf16 page pools */
  const uint64_t* v_pool;
  int64_t new_stride_n, new_stride_h;                         /* elements */
  int64_t pool_stride_page, pool_stride_head, pool_stride_tok; /* elements */
  const int32_t* num_accepted_dev; /* nullable: device count read by the kernel
                                      (e.g. d2sd_greedy_accept's result[0]),
                                      clamped to [0, num_accepted] */
  int32_t* prefix_len_dev;   /* nullable: the cache length is read here instead of
                                prefix_len (e.g. a dynamic cascade plan's
                                prefix_len array); tokens whose page index
                                reaches page_table_len are skipped */
  int advance_prefix;        /* with prefix_len_dev: a second launch then adds the
                                accepted count to *prefix_len_dev */
  int pool_dtype;            /* D2SD_KV_BF16 (0) or D2SD_KV_FP8_E4M3 */
  const uint64_t* k_scale;   /* fp8 pools: device [num_layers] addresses of fp32 [num_kv_heads] */
  const uint64_t* v_scale;
} d2sd_kv_append_args;

int d2sd_paged_kv_append(const d2sd_kv_append_args* args, d2sd_stream_t stream);

/* ----------------------------------------------------------------------
 * Candidate-tree build of one D2SD step on the device.
 * Replaces generation/d3_generator.py:116-180 up to the rows it verifies:
 * rejection rates from the draft confidences (rates[0] = 1 - c0,
 * rates[k] = cumprod(c)[k-1] * (1 - c_k), with torch's arithmetic for the
 * confidences' dtype), the top-k boundaries (torch.topk + sorted + .tolist()
 * at :123-125; equal rates ranked by index), and the rows: the DFlash row
 * (with its continuation when block_size_2 > block_size, else last) and per
 * boundary pl a row sharing its first pl + 1 tokens.  Outputs the token tree
 * of those rows in fixed capacity: unique nodes (row-major order of first
 * appearance), node_index [rows_cap, block_size_2], parents [capacity]
 * (-1 = root) and the ancestor mask [capacity, mask_words] in the layout
 * d2sd_cascade_run reads (bit j of row i: node j is i or an ancestor of i).
 * Nodes past num_nodes are roots seeing only themselves; rows past num_rows
 * repeat the DFlash row.  One single-wave launch, no host synchronisation.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* conf;     /* device [block_size - 1], dtype conf_dtype */
  int conf_dtype;       /* D2SD_DTYPE_BF16 or D2SD_DTYPE_F32 */
  int block_size;       /* DFlash block (2..65) */
  int block_size_2;     /* >= block_size */
  int topk;             /* >= 1 */
  int capacity;         /* >= block_size_2 + min(topk, block_size - 1) * (block_size_2 - 1) */
  int rows_cap;         /* >= min(topk, block_size - 1) + 1, <= 65 */
  int mask_words;       /* >= ceil(capacity / 64) */
  int32_t* num_nodes;   /* device [1] */
  int32_t* num_rows;    /* device [1], nullable */
  int32_t* parents;     /* device [capacity] */
  int32_t* node_index;  /* device [rows_cap, block_size_2] */
  uint64_t* tree_mask;  /* device [capacity, mask_words] */
  int32_t* shared;      /* device [rows_cap], nullable: tokens each row shares with the DFlash row */
  float* rates;         /* device [block_size - 1], nullable */
} d2sd_d3_tree_args;

int d2sd_d3_tree_build(const d2sd_d3_tree_args* args, d2sd_stream_t stream);

/* ----------------------------------------------------------------------
 * Per-head RMSNorm of the new queries and keys, then rotary embedding, in
 * place, one launch.  Replaces generation/verification.py:113-123 (Qwen3:
 * attn.q_norm / k_norm + _apply_rotary_pos_emb_qwen3; GPT-OSS: RoPE only)
 * and its transposes: q [tokens, Hq, D] and k [tokens, Hkv, D] stay
 * token-major (the layout d2sd_cascade_run reads).  Numerics follow the
 * reference's bf16 ops step for step:
 *   y = bf16(w * bf16(x / sqrt(mean(x^2) + eps)))      (when w is given)
 *   out = bf16(bf16(y * cos) + bf16(rotate_half(y) * sin))  (when cos is given)
 * cos / sin: bf16 [tokens, D] (Qwen3, halves equal) or [tokens, D / 2]
 * (GPT-OSS; half_cos = 1), the rotary table at each token's position.
 * head_dim 64, 128 or 256, contiguous.
 * ---------------------------------------------------------------------- */
typedef struct {
  void* q;
  void* k;
  int64_t q_stride_n, q_stride_h, k_stride_n, k_stride_h; /* elements */
  const void* q_norm;   /* bf16 [D] or NULL (no norm) */
  const void* k_norm;
  const void* cos;      /* bf16 or NULL (no rotation) */
  const void* sin;
  int64_t cs_stride;    /* elements between tokens of cos / sin */
  float eps;
  int num_tokens;
  int num_qo_heads;
  int num_kv_heads;
  int head_dim;
  int half_cos;
} d2sd_qk_norm_rope_args;

int d2sd_qk_norm_rope(const d2sd_qk_norm_rope_args* args, d2sd_stream_t stream);

/* ----------------------------------------------------------------------
 * Greedy acceptance walk of the verify tree, on the device.
 * Replaces generation/d3_generator.py:204-225 at temperature 0 (greedy
 * sampling is torch.argmax, model/utils.py:28-33, first index on ties):
 * with every row valid, step a takes the first valid row vb, accepts the
 * argmax of the logits of its node node_index[vb][a], and keeps the rows
 * whose draft token at position a + 1 equals it; the walk ends when no row
 * is valid or after row_len tokens.  Writes accept_ids[0..n) (token ids),
 * accept_nodes[0..n) (their nodes, the rows of the step's suffix K/V that
 * the KV commit appends), result[0] = n (acceptance_length) and result[1] =
 * the final valid row (valid_block).  Logits of every node are read once
 * (HBM bound); no host synchronisation.  A node id outside [0, num_nodes)
 * ends the walk.  Logits must be NaN-free.
 * ---------------------------------------------------------------------- */
#define D2SD_DTYPE_BF16 0
#define D2SD_DTYPE_F32 1
typedef struct {
  int num_rows;               /* candidate rows (bsz), <= 64 */
  int row_len;                /* positions per row (block_size_2); num_rows * row_len <= 2048 */
  int num_nodes;              /* rows of logits, <= 4096 */
  int vocab;
  int logits_dtype;           /* D2SD_DTYPE_* */
  const void* logits;         /* device [num_nodes, vocab], row stride logits_stride elements */
  int64_t logits_stride;
  const int32_t* node_index;  /* device [num_rows, row_len] */
  const int64_t* draft_ids;   /* device [num_rows, row_len]: the rows' draft tokens (block_output_ids) */
  int64_t* accept_ids;        /* device out [row_len] */
  int32_t* accept_nodes;      /* device out [row_len] */
  int32_t* result;            /* device out [2]: acceptance_length, valid_block */
  void* workspace;            /* device, d2sd_greedy_accept_workspace_size bytes */
  size_t workspace_bytes;
} d2sd_greedy_accept_args;

size_t d2sd_greedy_accept_workspace_size(int num_nodes, int vocab);
int d2sd_greedy_accept(const d2sd_greedy_accept_args* args, d2sd_stream_t stream);

/* ----------------------------------------------------------------------
 * The same walk at any temperature (generation/d3_generator.py:204-225 with
 * sample(logit, temperature), model/utils.py:28-37).  temperature < 1e-5 is
 * the greedy walk above (the reference's own threshold) and leaves
 * *rng_step alone.  Otherwise each accepted token is drawn from
 * softmax(logits / temperature): logits / temperature is computed as torch
 * does on the GPU (logits times the fp32 reciprocal, rounded to the logits
 * dtype) and the draw is torch.multinomial's exponential race,
 * argmax_v p_v / E_v, E_v ~ Exp(1), taken in log space.  E_v = -ln(u_v), u_v
 * from Philox4x32-10 with counter (v / 4, node, *rng_step) and key seed, so
 * the draws are a pure function of (logits, seed, *rng_step); the call
 * reads *rng_step and then advances it by one, so consecutive calls, and
 * replays of a captured call, draw independently.  The random stream is not
 * torch's: a sampled walk matches the reference in distribution, not token
 * for token.  node_tokens (nullable) receives every node's token (argmax at
 * temperature 0).  Workspace: d2sd_greedy_accept_workspace_size bytes.
 * ---------------------------------------------------------------------- */
typedef struct {
  d2sd_greedy_accept_args walk;
  float temperature;          /* >= 0, finite */
  uint64_t seed;
  int64_t* rng_step;          /* device [1]: step counter; required when temperature >= 1e-5 */
  int64_t* node_tokens;       /* device out [num_nodes], nullable */
} d2sd_sample_accept_args;

int d2sd_sample_accept(const d2sd_sample_accept_args* args, d2sd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* D2SD_H_ */
