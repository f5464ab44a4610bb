/*
 * dsa_mli.h — C ABI of libdsa_mli.so, the MI355X (gfx950) DeepSeek Sparse
 * Attention decode hot path: lightning-indexer scan over a paged fp8 key
 * cache, exact top-k select, split-K sparse MLA over the fp8 656-byte latent
 * pool, and the Multi-layer Indexer (MLI) lag schedule as one captured
 * hipGraph of fused per-layer launches (attention and indexer workgroups in
 * one grid).
 *
 * Conventions (every entry point):
 *   - plain device pointers and sizes; no torch types;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream);
 *   - the call only enqueues work; it never allocates device memory and
 *     never synchronises; caller owns every output and scratch buffer;
 *   - return 0 (DSA_OK) on success, a negative DSA_ERR_* code when an
 *     argument violates the contract (nothing is launched then), and
 *     DSA_ERR_HIP when the HIP launch itself failed;
 *     dsa_last_error() returns a message for the calling thread;
 *   - per-row context lengths are read from device memory (`seq_lens`), so a
 *     captured launch replays correctly as contexts grow;
 *   - work goes to the calling thread's current device; the library's own
 *     per-device state (kernel LDS attributes, CU counts, the static array of
 *     the allocation-free entry point) is set up on a device's first call.
 *
 * Data layouts in HBM (shared by all entry points):
 *   index-K page  : 8448 bytes = [64 keys x 128 B e4m3][64 x fp32 key scale]
 *                   token g of row b lives in page page_table[b*pt_stride + g/64],
 *                   slot g%64.
 *   latent KV row : 656 bytes = [512 e4m3][4 fp32 scales, one per 128 dims]
 *                   [64 bf16 rope]; the row of token g of row b is KV slot
 *                   page_table[b*pt_stride + g/64]*64 + g%64.
 *   e4m3          : OCP float8 e4m3fn (bias 7, max 448, 0x7f/0xff = NaN).
 */
#ifndef DSA_MLI_H
#define DSA_MLI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_OK 0
#define DSA_ERR_INVALID_ARG (-1)  /* null pointer, bad size or stride */
#define DSA_ERR_UNSUPPORTED (-2)  /* shape outside the compiled kernels */
#define DSA_ERR_HIP (-3)          /* hipLaunch / hipGraph call failed */

#define DSA_PAGE_TOKENS 64
#define DSA_INDEX_DIM 128
#define DSA_INDEX_PAGE_BYTES 8448 /* 64*128 + 64*4 */
#define DSA_LATENT_DIM 512
#define DSA_ROPE_DIM 64
#define DSA_QK_DIM 576
#define DSA_LATENT_ROW_BYTES 656  /* 512 + 4*4 + 64*2 */
#define DSA_TOPK_MAX_CTX 262144   /* longest row the top-k select accepts */

/* dsa_topk flags */
#define DSA_TOPK_POSITION_ORDER 0 /* selected indices ascending, pads last */
#define DSA_TOPK_SORTED 1         /* score descending, ties lower index first */

/* Message for the last failing call on this host thread ("" if none). */
const char* dsa_last_error(void);

/* Library version string. */
const char* dsa_version(void);

/* sizeof(dsa_layer_args) as the library was built: a caller compares it with
 * its own sizeof to detect a header mismatch (0.3 appended `dense`). */
size_t dsa_layer_args_bytes(void);

/*
 * Count of in-launch group waits that expired on the current device since
 * the library was loaded (or since the last call with reset != 0); reset != 0
 * zeroes it after reading.  Returns -1 if the count cannot be read.
 * Synchronous (waits for the device's queued work to read the counter).
 *
 * The cooperative top-k select and the split-K merge hand data between
 * workgroups of ONE launch through bounded spin waits.  They rely on every
 * workgroup of a group being resident at once: workgroups are dispatched in
 * index order and each group is smaller than the device, so this holds when
 * the launch has the device to itself or shares it only with kernels that
 * finish without waiting on it.  A wait that expires (about a second) is
 * counted here and the launch goes on, so a launch that broke the
 * assumption returns instead of hanging the device -- but its results are
 * wrong.  A caller that cannot rule out such sharing checks that this count
 * stays 0.  No counterpart in the reference, whose waits are unbounded
 * (K:1093-1095, K:2219-2224).
 */
int dsa_sync_timeouts(int reset);

/*
 * The same expiries per buffer, asynchronously: every wait that expires also
 * adds 1 to a status word of its group in the caller's buffers -- one per
 * top-k scratch row (the row's select) and one per (row, 16-head group) of
 * a sparse-MLA workspace (the split merge).  This enqueues ONE small kernel
 * on `stream` that writes into *status (a device int32) the sum of the
 * words of the first B_scan rows of topk_scratch (slab_stride as it was
 * allocated with) and of the B_attn*(H/16) groups of workspace, and zeroes
 * them when clear != 0.  Either buffer may be NULL.  It never synchronises
 * and may be captured in a graph (after the launches it covers), so a
 * caller can check each step's launches when it next reads *status: 0 means
 * every in-launch wait of those buffers was satisfied.
 * No counterpart in the reference (its waits are unbounded).
 */
int dsa_sync_status(const void* topk_scratch, int B_scan, int slab_stride,
                    const void* workspace, int B_attn, int H, int32_t* status,
                    int clear, void* stream);

/*
 * (1) Lightning-indexer scan.
 *   scores[b, g] = kscale[g] * sum_h w[b,h] * ReLU( sum_d q[b,h,d] * k[g,d] )
 * for g < seq_lens[b]; scores[b, g] = -inf for seq_lens[b] <= g < slab_stride.
 *   q_fp8      [B, Hidx, 128] e4m3 (the per-head query scale is folded into w)
 *   w          [B, Hidx] fp32
 *   index_k    [num_pages, 8448] bytes
 *   page_table [B, pt_stride] int32 physical page ids (ids outside
 *              [0, num_pages) score -inf instead of being read)
 *   seq_lens   [B] int32 (clamped to min(pt_stride*64, slab_stride))
 *   scores     [B, slab_stride] fp32
 * Hidx must be 16, 32, 48 or 64.
 * Replaces: reference kernels/cuda_fused_sparse_splitk.py hp_indexer_block
 * (K:1677-2157) reached through launch_fused_sparse_splitk_paged
 * (K:2770) with with_select=1, and ref_indexer_logits_fp8 (K:2990-2992);
 * CPU semantics attention_core.py:27-49 (indexer_logits).
 */
int dsa_indexer_scan(const void* q_fp8, const float* w, const void* index_k,
                     int64_t num_pages, const int32_t* page_table,
                     const int32_t* seq_lens, float* scores, int B, int Hidx,
                     int pt_stride, int slab_stride, void* stream);

/*
 * (2) Exact top-k select over each row's first seq_lens[b] scores.
 * Order of selection: score descending, ties -> lower index first; NaN
 * ranks above +inf and -0.0 equals +0.0.  Selected entries whose score is
 * not finite become `pad_value`, as do the slots beyond seq_lens[b] when the
 * row is shorter than topk.
 *   flags = DSA_TOPK_POSITION_ORDER: out[b] = selected finite indices in
 *           ascending index order, then pads;
 *   flags = DSA_TOPK_SORTED: out[b] in selection order (torch.topk order
 *           with the lower-index tie rule), non-finite entries -> pad in place.
 * page_table != NULL: each emitted position g is replaced by its KV slot
 * page_table[b*pt_stride + g/64]*64 + g%64 (position order only).
 *   scores  [B, slab_stride] fp32;  out_idx [B, topk] int32
 *   scratch dsa_topk_scratch_bytes(B, slab_stride) bytes, zero-filled once
 *           before the first call; every call leaves it ready for the next
 *           (counters re-armed, barrier flags consistent), so calls chain and
 *           graph replays need no memset; zeroing it again between calls is
 *           harmless.  Two calls that overlap in time must not share a
 *           scratch buffer.
 * DSA_TOPK_POSITION_ORDER runs as ONE launch: the workgroups of a row each
 * load a slice of its scores and select together (the decode layer's
 * cooperative select); DSA_TOPK_SORTED runs as two launches (histogram,
 * then per-slice filter and a sorting finalize).
 * Requires topk <= 8192 (<= 4096 with DSA_TOPK_SORTED) and
 * slab_stride <= DSA_TOPK_MAX_CTX.
 * Replaces: reference attention_core.py:66-91 (select_topk), and on the GPU
 * tl_topk (tilelang_dsa/topk_selector.py:355-386) and the in-kernel exact
 * select with hp_page_to_slot (K:1097-1144, K:1248-1310).
 */
size_t dsa_topk_scratch_bytes(int B, int slab_stride);
int dsa_topk(const float* scores, const int32_t* seq_lens,
             const int32_t* page_table, int pt_stride, void* scratch,
             int32_t* out_idx, int B, int slab_stride, int topk, int flags,
             int32_t pad_value, void* stream);

/*
 * (3) Split-K sparse MLA decode over the fp8 latent pool.
 *   out[b,h,:] = sum_j softmax_j(sm_scale * q[b,h,:] . kv_j) * kv_j[:512]
 * over the j in idx[b, :topk] with 0 <= idx < kv_rows (others are masked);
 * kv_j = dequant(row idx[b,j]) = bf16_rn(f32(e4m3) * scale[d/128]) for d<512,
 * rope bf16 for d>=512.  A row with no valid index gives 0.  Indices are
 * expected distinct (a repeated slot is counted once per occurrence).
 *   q         [B, H, 576] bf16;     kv_pool [kv_rows, 656] bytes
 *   idx       [B, topk] int32 KV slots
 *   workspace dsa_sparse_mla_workspace_bytes(B, H, nsplit) bytes: split
 *             partials plus one barrier per (row, head group) through which
 *             the splits merge together; zero-fill it once before the first
 *             call, every call leaves the barriers ready for the next.
 *             Calls that overlap in time must not share it.
 *   out       [B, H, 512] bf16
 * H must be a multiple of 16; 1 <= nsplit <= 128 (nsplit=0: automatic, and
 * a workspace sized with nsplit=0 fits any nsplit).
 * Replaces: hp_attention_block + combine (K:1312-1666, K:996-1045) and
 * ref_sparse_mla (K:2950-2966); CPU semantics attention_core.py:94-146.
 */
size_t dsa_sparse_mla_workspace_bytes(int B, int H, int nsplit);
int dsa_sparse_mla_decode(const void* q_bf16, const void* kv_pool,
                          int64_t kv_rows, const int32_t* idx, void* workspace,
                          void* out_bf16, int B, int H, int topk, int nsplit,
                          float sm_scale, void* stream);

/*
 * (3a) Dense MLA decode: the attention of (3) over every token of each row,
 * keys 0..seq_lens[b]-1 at KV slots page_table[b*pt_stride + j/64]*64 + j%64
 * (seq_lens clamped to pt_stride*64).  workspace:
 * dsa_sparse_mla_workspace_bytes(B, H, nsplit), as for (3); nsplit = 0:
 * one split per 64 keys of the page table's capacity, at most 128.
 * Replaces: dense_mla_core (attention_core.py:142-160), the full-attention
 * layers and the DENSE cold start of DSAModel.forward (model.py:51-59,
 * 104-114).
 */
int dsa_dense_mla_decode(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                         const int32_t* page_table, int pt_stride, const int32_t* seq_lens,
                         void* workspace, void* out_bf16, int B, int H, int nsplit,
                         float sm_scale, void* stream);

/*
 * (3b) The same sparse MLA decode with no workspace argument and no
 * allocation: the split partials and the per-(row, head group) barriers live
 * in a static device array of the library (one copy per device, about 19 MB,
 * held until the process ends), for callers that cannot allocate (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limits: B*H/16 <= 512 and B*(H/16)*nsplit*32896 bytes of partials
 * <= 16 MiB (nsplit after nsplit = 0 is resolved); a call beyond them returns
 * DSA_ERR_UNSUPPORTED without launching.  Results equal (3)'s at the same
 * nsplit, bit for bit.  Every call on a device shares that device's array:
 * calls that overlap in time on one device (two streams, two threads) race
 * and give wrong results.
 * No counterpart in the reference; added for callers that cannot allocate.
 */
int dsa_sparse_mla_decode_noalloc(const void* q_bf16, const void* kv_pool,
                                  int64_t kv_rows, const int32_t* idx,
                                  void* out_bf16, int B, int H, int topk,
                                  int nsplit, float sm_scale, void* stream);

/*
 * (4) One DSA decode layer on one stream:
 *   indexer scan -> top-k (position order, KV-slot output into next_idx),
 *   and attention over attend_idx (the lagged set: the attention and the
 *   scan then share ONE launch; from B = 8 rows the scan launch carries
 *   the attention on about a quarter of the CUs when the rows' capacity is
 *   large next to B * topk, and the select follows; else scan, select and
 *   attention are three launches in that order), or over this layer's own
 *   fresh selection when attend_idx == NULL (baseline DSA: scan, select,
 *   then attention).
 * scores [B, slab_stride] fp32 scratch; next_idx [B, topk] int32.
 * Replaces: DSALayer.fused_attention_and_indices (dsa_layer.py:173-192)
 * for one decode row per request.
 */
typedef struct dsa_layer_args {
  /* indexer operands (NULL q_fp8: this layer runs no indexer) */
  const void* q_fp8;        /* [B, Hidx, 128] e4m3 */
  const float* w;           /* [B, Hidx] */
  const void* index_k;      /* [num_idx_pages, 8448] */
  int64_t num_idx_pages;
  float* scores;            /* [B, slab_stride] scratch */
  void* topk_scratch;       /* dsa_topk_scratch_bytes(B, slab_stride), zeroed once */
  int32_t* next_idx;        /* [B, topk] out: KV slots, -1 pad */
  /* attention operands (NULL q_bf16: this layer runs no attention) */
  const void* q_bf16;       /* [B, H, 576] */
  const void* kv_pool;      /* [kv_rows, 656] */
  int64_t kv_rows;
  const int32_t* attend_idx;/* [B, topk] KV slots; NULL = see (4) / (5) */
  void* workspace;          /* dsa_sparse_mla_workspace_bytes(B,H,nsplit), zeroed once */
  void* out_bf16;           /* [B, H, 512] */
  /* shared */
  const int32_t* page_table;/* [B, pt_stride] */
  const int32_t* seq_lens;  /* [B] */
  int B, Hidx, H, topk, nsplit, pt_stride, slab_stride;
  float sm_scale;
  /* 1: the attention is dense over each row's first seq_lens[b] tokens
   * (attend_idx ignored) -- a full-attention layer, or the DENSE cold start
   * of layer 0; 0: sparse over attend_idx / the schedule's selection */
  int dense;
} dsa_layer_args;
/* nsplit = 0: automatic.  The attention launched alone takes one split per
 * 64 selected keys, at most one workgroup per CU over the batch's (row, head
 * group)s; the attention of a layer launch that also scans (the lagged case)
 * takes the same, capped so its workgroups hold about a quarter of the CUs
 * (in a launch shared with the scan).  The split count is part of the
 * arithmetic: outputs at different split counts agree to rounding, not
 * bitwise. */

int dsa_decode_layer(const dsa_layer_args* args, void* stream);

/*
 * (5) MLI lag schedule over a stack of layers, eagerly or as one hipGraph.
 * Layer i attends the selection of the most recent earlier layer that runs
 * an indexer (its attend_idx when given; layer 0 must be given one, unless
 * it is dense), or densely when its `dense` flag is set, and
 * layer i's indexer scan runs in the SAME launch as layer i's attention
 * (role-decoupled workgroups; from B = 8 rows the scan launch carries the
 * attention and the select follows, or the three run as separate launches),
 * followed by layer i's
 * top-k select, which layer i+1 attends.  A layer whose q_fp8 is NULL runs no indexer (IndexCache
 * reuse); one whose q_bf16 is NULL runs no attention.  Everything is on one
 * stream: the overlap of indexer and attention is inside each launch.
 * Replaces: DSAModel.forward LAGGED_FUSED (model.py:109-136) and the serving
 * side-stream fork/join (sglang overlay patch P:1774-1833, P:2942-2997).
 */
typedef struct dsa_mli_graph dsa_mli_graph;
int dsa_mli_graph_create(const dsa_layer_args* layers, int num_layers,
                         void* capture_stream, dsa_mli_graph** out_graph);
int dsa_mli_graph_launch(dsa_mli_graph* graph, void* stream);
int dsa_mli_graph_destroy(dsa_mli_graph* graph);
int dsa_mli_run_eager(const dsa_layer_args* layers, int num_layers,
                      void* stream);

/*
 * (5b) The same schedule at lag depth k (1 <= k <= 64; k = 1 is the entries
 * above).  Number the layers that run an indexer R_0, R_1, ... in order.  A
 * layer whose attend_idx is NULL attends:
 *   k == 1: the fresh selection of the most recent earlier R (as above);
 *   k >= 2: for R_n with n >= k, R_{n-k}'s fresh selection; otherwise (R_n
 *           with n < k, and every reuse layer) the set the previous layer
 *           attended.  Reuse layers thus copy their producer's attended set.
 * Give layer 0 its own next_idx as attend_idx for the reference's cold start
 * (layer 0 attends its own fresh selection; then R_n attends R_{n-k}).
 * Every selection is written by an earlier launch on the same stream, so no
 * event joins are needed; depth changes which buffer each layer reads, not
 * the launches.
 * Replaces: the depth-k deferred-indexer FIFO (hh_lag_queue_push /
 * hh_lag_queue_join_oldest, P:1835-1904) and _hh_lag_refresh_dispatch_depth
 * (P:3020-3100), configured by index_reuse_lag_depth (P:4388-4431).
 */
int dsa_mli_graph_create_depth(const dsa_layer_args* layers, int num_layers, int lag_depth,
                               void* capture_stream, dsa_mli_graph** out_graph);
int dsa_mli_run_eager_depth(const dsa_layer_args* layers, int num_layers, int lag_depth,
                            void* stream);

/*
 * (6) Decode-step operand preparation: the fp8 quantizers and paged appends
 * whose outputs (4) consumes.  Rule, per 128-element row (the reference
 * harness's quantize_e4m3_rowwise, K:2969-2974):
 *   scale = max(amax, 1e-6) / 448,  code = e4m3_rne(clamp(x / scale, +-448)).
 *
 * Indexer query: q [B, Hidx, 128] bf16, w [B, Hidx] fp32 ->
 *   q_fp8 [B, Hidx, 128] e4m3, w_fold [B, Hidx] = w * scale (per head).
 * Replaces: the serving act_quant of the indexer query and the q-scale fold
 * (sglang overlay P:338, P:343; transformer.py:1139-1144), harness
 * K:2981-2985.
 */
int dsa_quantize_index_query(const void* q_bf16, const float* w, void* q_fp8, float* w_fold, int B,
                             int Hidx, void* stream);

/*
 * Index-K append: keys k [n, 128] bf16 of tokens (rows[i], pos[i]) -> their
 * codes at slot pos%64 of page page_table[rows[i]*pt_stride + pos/64] and the
 * fp32 scale in that page's scale tail.  A token whose page entry is outside
 * [0, num_pages) is skipped.
 * Replaces: _store_index_k_cache (sglang overlay P:339-342).
 */
int dsa_append_index_keys(const void* k_bf16, const int32_t* rows, const int32_t* pos, int n,
                          const int32_t* page_table, int pt_stride, void* index_k, int64_t num_pages,
                          void* stream);

/*
 * Latent append: latent [n, 576] bf16 (512 latent | 64 rope) -> 656-byte rows
 * at KV slots slots[i]: 512 e4m3 codes quantized per 128-dim group, the four
 * fp32 group scales, the 64 rope values as bf16 (the layout of (3)).  A slot
 * outside [0, kv_rows) is skipped.
 * Replaces: SGLang v0.5.16's fp8 KV-cache quantizer, which the reference's
 * kernels read back (dequant K:1181-1197; dequantize_k_cache P:789).
 */
int dsa_append_latent_rows(const void* latent_bf16, const int32_t* slots, int n, void* kv_pool, int64_t kv_rows,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MLI_H */
