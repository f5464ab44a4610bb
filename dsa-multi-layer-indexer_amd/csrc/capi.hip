// C ABI of libdsa_mli.so: argument contracts, the decode-layer composite and
// the MLI schedule (eager and captured as one hipGraph).
//
// Contract checks mirror the reference launcher's TORCH_CHECKs
// (kernels/cuda_fused_sparse_splitk.py K:2399-2611) as negative return codes;
// nothing is launched when a check fails.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "dsa_common.h"
#include "dsa_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return DSA_OK;
  return fail(DSA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define DSA_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return fail(code, __VA_ARGS__); \
  } while (0)

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_scan(const void* q_fp8, const float* w, const void* index_k, int64_t num_pages,
               const int32_t* page_table, const int32_t* seq_lens, const float* scores, int B,
               int Hidx, int pt_stride, int slab_stride) {
  DSA_REQUIRE(q_fp8 && w && index_k && page_table && seq_lens && scores, DSA_ERR_INVALID_ARG,
              "dsa_indexer_scan: null pointer argument");
  DSA_REQUIRE(B >= 1, DSA_ERR_INVALID_ARG, "dsa_indexer_scan: B must be >= 1 (got %d)", B);
  DSA_REQUIRE(B <= 65535, DSA_ERR_UNSUPPORTED, "dsa_indexer_scan: B must be <= 65535");
  DSA_REQUIRE(Hidx >= 16 && Hidx <= 64 && Hidx % 16 == 0, DSA_ERR_UNSUPPORTED,
              "dsa_indexer_scan: index_n_heads must be 16, 32, 48 or 64 (got %d)", Hidx);
  DSA_REQUIRE(num_pages >= 1, DSA_ERR_INVALID_ARG, "dsa_indexer_scan: num_pages must be >= 1");
  DSA_REQUIRE(pt_stride >= 1, DSA_ERR_INVALID_ARG, "dsa_indexer_scan: pt_stride must be >= 1");
  DSA_REQUIRE(slab_stride >= 1, DSA_ERR_INVALID_ARG, "dsa_indexer_scan: slab_stride must be >= 1");
  DSA_REQUIRE(aligned16(q_fp8) && aligned16(index_k), DSA_ERR_INVALID_ARG,
              "dsa_indexer_scan: q_fp8 and index_k must be 16-byte aligned");
  return DSA_OK;
}

int check_topk(const float* scores, const int32_t* seq_lens, const int32_t* page_table,
               int pt_stride, const void* scratch, const int32_t* out_idx, int B,
               int slab_stride, int topk, int flags) {
  DSA_REQUIRE(scores && seq_lens && out_idx && scratch, DSA_ERR_INVALID_ARG,
              "dsa_topk: null pointer argument");
  DSA_REQUIRE(aligned16(scratch), DSA_ERR_INVALID_ARG, "dsa_topk: scratch must be 16-byte aligned");
  DSA_REQUIRE(B >= 1 && B <= 65535, DSA_ERR_INVALID_ARG, "dsa_topk: B must be in [1, 65535] (got %d)", B);
  DSA_REQUIRE(topk >= 1, DSA_ERR_INVALID_ARG, "dsa_topk: topk must be >= 1 (got %d)", topk);
  DSA_REQUIRE(flags == DSA_TOPK_POSITION_ORDER || flags == DSA_TOPK_SORTED, DSA_ERR_INVALID_ARG,
              "dsa_topk: unknown flags %d", flags);
  DSA_REQUIRE(topk <= (flags == DSA_TOPK_SORTED ? 4096 : 8192), DSA_ERR_UNSUPPORTED,
              "dsa_topk: topk %d above the supported maximum", topk);
  DSA_REQUIRE(slab_stride >= 1 && slab_stride <= DSA_TOPK_MAX_CTX, DSA_ERR_UNSUPPORTED,
              "dsa_topk: slab_stride must be in [1, %d] (got %d)", DSA_TOPK_MAX_CTX, slab_stride);
  DSA_REQUIRE(page_table == nullptr || flags == DSA_TOPK_POSITION_ORDER, DSA_ERR_INVALID_ARG,
              "dsa_topk: page-table slot mapping requires DSA_TOPK_POSITION_ORDER");
  DSA_REQUIRE(page_table == nullptr || (int64_t)pt_stride * DSA_PAGE_TOKENS >= slab_stride,
              DSA_ERR_INVALID_ARG, "dsa_topk: page table must cover slab_stride (pt_stride*64 >= slab_stride)");
  return DSA_OK;
}

int check_mla(const void* q_bf16, const void* kv_pool, int64_t kv_rows, const int32_t* idx,
              const void* workspace, const void* out_bf16, int B, int H, int topk, int nsplit,
              bool idx_required = true, bool ws_required = true) {
  DSA_REQUIRE(q_bf16 && kv_pool && (idx || !idx_required) && (workspace || !ws_required) && out_bf16,
              DSA_ERR_INVALID_ARG, "dsa_sparse_mla_decode: null pointer argument");
  DSA_REQUIRE(B >= 1 && B <= 65535, DSA_ERR_INVALID_ARG, "dsa_sparse_mla_decode: bad B %d", B);
  DSA_REQUIRE(H >= 16 && H % 16 == 0 && H <= 16 * 64, DSA_ERR_UNSUPPORTED,
              "dsa_sparse_mla_decode: H must be a positive multiple of 16 (got %d)", H);
  DSA_REQUIRE(topk >= 1, DSA_ERR_INVALID_ARG, "dsa_sparse_mla_decode: topk must be >= 1");
  DSA_REQUIRE(nsplit >= 0 && nsplit <= 128, DSA_ERR_UNSUPPORTED,
              "dsa_sparse_mla_decode: nsplit must be in [0, 128] (got %d)", nsplit);
  DSA_REQUIRE(kv_rows >= 1, DSA_ERR_INVALID_ARG, "dsa_sparse_mla_decode: kv_rows must be >= 1");
  DSA_REQUIRE(aligned16(q_bf16) && aligned16(kv_pool) && (aligned16(workspace) || !ws_required) &&
                  ((uintptr_t)out_bf16 & 7) == 0,
              DSA_ERR_INVALID_ARG, "dsa_sparse_mla_decode: q/kv_pool/workspace must be 16-byte aligned");
  return DSA_OK;
}

int resolve_nsplit(int nsplit, int topk, int B, int H) {
  return nsplit > 0 ? nsplit : dsa::attn_auto_nsplit(topk, B, H);
}

// in_schedule: attend_idx == NULL is resolved by the MLI schedule (the most
// recent earlier selection) instead of meaning "this layer's own selection".
int check_layer(const dsa_layer_args* a, bool in_schedule = false) {
  DSA_REQUIRE(a != nullptr, DSA_ERR_INVALID_ARG, "dsa_layer_args is null");
  DSA_REQUIRE(a->dense == 0 || a->dense == 1, DSA_ERR_INVALID_ARG, "dsa_layer_args.dense must be 0 or 1");
  int rc;
  if (a->q_fp8) {
    rc = check_scan(a->q_fp8, a->w, a->index_k, a->num_idx_pages, a->page_table, a->seq_lens,
                    a->scores, a->B, a->Hidx, a->pt_stride, a->slab_stride);
    if (rc) return rc;
    rc = check_topk(a->scores, a->seq_lens, a->page_table, a->pt_stride, a->topk_scratch,
                    a->next_idx, a->B, a->slab_stride, a->topk, DSA_TOPK_POSITION_ORDER);
    if (rc) return rc;
  }
  if (a->q_bf16 && a->dense) {
    DSA_REQUIRE(a->page_table && a->seq_lens && a->pt_stride >= 1, DSA_ERR_INVALID_ARG,
                "dsa_decode_layer: dense attention needs page_table, pt_stride and seq_lens");
    DSA_REQUIRE((int64_t)a->pt_stride * DSA_PAGE_TOKENS <= (int64_t)1 << 30, DSA_ERR_UNSUPPORTED,
                "dsa_decode_layer: dense attention over pt_stride*64 keys must be <= 2^30");
    rc = check_mla(a->q_bf16, a->kv_pool, a->kv_rows, nullptr, a->workspace, a->out_bf16, a->B, a->H,
                   a->pt_stride * DSA_PAGE_TOKENS, a->nsplit, /*idx_required=*/false);
    if (rc) return rc;
  } else if (a->q_bf16) {
    const int32_t* att = a->attend_idx ? a->attend_idx : a->next_idx;
    DSA_REQUIRE(in_schedule || a->attend_idx || a->q_fp8, DSA_ERR_INVALID_ARG,
                "dsa_decode_layer: attention needs attend_idx or an indexer");
    rc = check_mla(a->q_bf16, a->kv_pool, a->kv_rows, att, a->workspace, a->out_bf16, a->B, a->H,
                   a->topk, a->nsplit, /*idx_required=*/!in_schedule);
    if (rc) return rc;
  }
  return DSA_OK;
}

dsa::AttnArgs attn_args(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                        const int32_t* idx, void* workspace, void* out_bf16, int B, int H,
                        int topk, int nsplit, float sm_scale) {
  dsa::AttnArgs A{};
  A.q = (const uint16_t*)q_bf16;
  A.pool = (const uint8_t*)kv_pool;
  A.kv_rows = (long)kv_rows;
  A.idx = idx;
  A.out = (uint16_t*)out_bf16;
  A.H = H;
  A.topk = topk;
  A.nsplit = resolve_nsplit(nsplit, topk, B, H);
  A.sm_log2 = sm_scale * 1.4426950408889634f;
  dsa::attn_bind_workspace(A, workspace, B);
  return A;
}

// Dense attention over each row's first seq_lens[b] tokens (their KV slots
// through the page table); the split count covers the page table's capacity.
dsa::AttnArgs dense_attn_args(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                              const int32_t* page_table, int pt_stride, const int32_t* seq_lens,
                              void* workspace, void* out_bf16, int B, int H, int nsplit, float sm_scale) {
  dsa::AttnArgs A = attn_args(q_bf16, kv_pool, kv_rows, nullptr, workspace, out_bf16, B, H,
                              pt_stride * DSA_PAGE_TOKENS, nsplit, sm_scale);
  A.dense_pt = page_table;
  A.dense_lens = seq_lens;
  A.dense_pt_stride = pt_stride;
  return A;
}

dsa::ScanArgs scan_args(const void* q_fp8, const float* w, const void* index_k, int64_t num_pages,
                        const int32_t* page_table, const int32_t* seq_lens, float* scores,
                        int Hidx, int pt_stride, int slab_stride, void* topk_scratch,
                        int32_t* next_idx = nullptr, int topk = 0) {
  dsa::ScanArgs S{};
  S.q8 = (const uint8_t*)q_fp8;
  S.w = w;
  S.pages = (const uint8_t*)index_k;
  S.num_pages = (long)num_pages;
  S.page_table = page_table;
  S.seq_lens = seq_lens;
  S.scores = scores;
  S.hist = (uint32_t*)topk_scratch;
  S.hist_row_words = dsa::topk_row_words(slab_stride);
  S.next_idx = next_idx;
  S.topk = topk;
  S.pt_stride = pt_stride;
  S.slab_stride = slab_stride;
  S.Hidx = Hidx;
  return S;
}

// Rows from which a layer's indexer runs as two launches (scan, then select
// beside the attention) instead of one: the fused launch pins one workgroup
// per CU for the whole scan, which large batches cannot afford.
constexpr int kSplitLaunchRows = 8;

// One layer on one stream.  attend: the selection its attention reads
// (nullptr: no attention); with_indexer: scan + select into next_idx, both
// in the decode launch (the row's last scan workgroup selects).  When the
// attention reads this layer's own fresh selection, it is a second launch.
int enqueue_layer(const dsa_layer_args* a, const int32_t* attend, bool with_indexer,
                  hipStream_t s) {
  dsa::AttnArgs A{};
  dsa::ScanArgs S{};
  const bool dense = a->dense != 0;
  const bool attention = a->q_bf16 != nullptr && (attend != nullptr || dense);
  // one launch, both roles (the attention does not read this layer's selection)
  const bool shared = attention && with_indexer && (dense || attend != a->next_idx);
  const int att_keys = dense ? a->pt_stride * DSA_PAGE_TOKENS : a->topk;
  const auto make_attn = [&](int nsplit) {
    return dense ? dense_attn_args(a->q_bf16, a->kv_pool, a->kv_rows, a->page_table, a->pt_stride, a->seq_lens,
                                   a->workspace, a->out_bf16, a->B, a->H, nsplit, a->sm_scale)
                 : attn_args(a->q_bf16, a->kv_pool, a->kv_rows, attend, a->workspace, a->out_bf16, a->B, a->H,
                             a->topk, nsplit, a->sm_scale);
  };
  if (attention)
    A = make_attn(a->nsplit > 0 ? a->nsplit : (shared ? dsa::attn_fused_nsplit(att_keys, a->B, a->H) : 0));
  if (with_indexer)
    S = scan_args(a->q_fp8, a->w, a->index_k, a->num_idx_pages, a->page_table, a->seq_lens,
                  a->scores, a->Hidx, a->pt_stride, a->slab_stride, a->topk_scratch, a->next_idx,
                  a->topk);
  const bool own = attention && with_indexer && !dense && attend == a->next_idx;
  int rc;
  if (with_indexer && a->B >= kSplitLaunchRows) {
    // large batches: a plain scan launch writes the scores, a select launch
    // loads them; the attention runs in the scan launch (below) or alone
    // after the select at its own split count
    dsa::ScanArgs P = S;
    P.next_idx = nullptr;
    P.hist = nullptr;
    // the attention over a set this layer does not produce (sparse) rides
    // in the scan launch, on the CUs beside the scan: its gather then
    // shares the scan's time instead of following the select.  About a
    // quarter of the CUs for it (measured at 8, 16, 32 and 64 rows: 64
    // attention workgroups beat 32 and 96-128; C4 with 2 splits per row
    // 108 against 120 us per layer with the attention launched after the
    // select), and only when the scan is long next to the attention's share
    // of keys (the row capacity stands in for the lengths, which are on the
    // device): 32 rows of 2K-16K tokens ran 77 against 67 us with it.
    const long att_groups = (long)a->B * (a->H / dsa::kHeadGroup);
    const long quarter = dsa::device_cu_count() / 4;
    const int ride_splits = (int)std::min(8L, std::max(1L, quarter / std::max(1L, att_groups)));
    const long cap_tokens = (long)a->B * std::min((long)a->slab_stride, (long)a->pt_stride * DSA_PAGE_TOKENS);
    const bool ride = attention && !own && !dense && a->nsplit <= 0 && dsa::flat_scan_on() &&
                      dsa::flat_scan_fits(P, a->B) && att_groups * ride_splits <= quarter &&
                      cap_tokens >= 20L * att_groups * a->topk;
    if (ride) {
      A = make_attn(ride_splits);
      rc = hip_status(dsa::launch_flat_scan(&A, a->B, P, a->B, s), "indexer scan + attention launch");
    } else {
      rc = hip_status(dsa::launch_decode_main(nullptr, 0, &P, a->B, s), "indexer scan launch");
    }
    if (rc) return rc;
    S.from_scores = 1;
    rc = hip_status(dsa::launch_decode_main(nullptr, 0, &S, a->B, s), "top-k select launch");
    if (rc || !attention || ride) return rc;
    if (a->nsplit <= 0) A = make_attn(0);
    return hip_status(dsa::launch_decode_main(&A, a->B, nullptr, 0, s), "attention launch");
  }
  rc = hip_status(dsa::launch_decode_main(attention && !own ? &A : nullptr, a->B, with_indexer ? &S : nullptr,
                                          a->B, s),
                  "decode main launch");
  if (rc) return rc;
  if (own) rc = hip_status(dsa::launch_decode_main(&A, a->B, nullptr, 0, s), "attention launch");
  return rc;
}

// The MLI schedule on one stream: layer i = ONE launch running attention(i)
// over a lagged selection side by side with indexer-scan(i) + top-k(i).
// Which selection a layer attends when its attend_idx is NULL (lag depth k,
// producers R_0, R_1, ... numbered in layer order):
//   k == 1: the fresh selection of the most recent earlier producer
//           (P:2942-2997); reuse layers carry that fresh set forward;
//   k >= 2: producer R_n attends R_{n-k}'s fresh selection once n >= k and the
//           incoming carry before that; every layer carries out the set it
//           attended, so reuse layers copy their producer's attended set
//           (P:1835-1904, P:3020-3100).
// A layer with attend_idx set attends it, and carries it out unless k == 1
// and the layer is a producer.
constexpr int kMaxLagDepth = 64;

template <class F>
int walk_mli(const dsa_layer_args* layers, int n, int depth, F&& on_layer) {
  const int32_t* fresh[kMaxLagDepth];  // ring of the last `depth` producers' selections
  long produced = 0;
  const int32_t* carried = nullptr;
  for (int i = 0; i < n; ++i) {
    const dsa_layer_args* a = &layers[i];
    const bool producer = a->q_fp8 != nullptr;
    const int32_t* lagged = (producer && depth >= 2 && produced >= depth) ? fresh[produced % depth] : carried;
    // a dense layer attends no selection
    const int32_t* att = a->dense ? nullptr : (a->attend_idx ? a->attend_idx : lagged);
    const int rc = on_layer(i, a, att);
    if (rc) return rc;
    carried = att;
    if (producer) {
      fresh[produced % depth] = a->next_idx;  // the slot just read holds R_{n-k}
      ++produced;
      if (depth == 1) carried = a->next_idx;
    }
  }
  return DSA_OK;
}

int check_depth(int depth) {
  DSA_REQUIRE(depth >= 1 && depth <= kMaxLagDepth, DSA_ERR_INVALID_ARG, "mli: lag depth %d outside [1, %d]",
              depth, kMaxLagDepth);
  return DSA_OK;
}

int enqueue_mli(const dsa_layer_args* layers, int n, int depth, hipStream_t s) {
  return walk_mli(layers, n, depth, [&](int i, const dsa_layer_args* a, const int32_t* att) {
    if (a->q_bf16 && !a->dense && !att) return fail(DSA_ERR_INVALID_ARG, "mli layer %d: no selection to attend", i);
    return enqueue_layer(a, a->q_bf16 ? att : nullptr, a->q_fp8 != nullptr, s);
  });
}

int check_mli(const dsa_layer_args* layers, int n, int depth) {
  DSA_REQUIRE(layers && n >= 1, DSA_ERR_INVALID_ARG, "mli: need at least one layer");
  int rc = check_depth(depth);
  if (rc) return rc;
  return walk_mli(layers, n, depth, [&](int i, const dsa_layer_args* a, const int32_t* att) {
    const int lrc = check_layer(a, true);
    if (lrc) return lrc;
    if (a->dense && depth != 1)
      return fail(DSA_ERR_UNSUPPORTED, "mli layer %d: dense attention layers need lag depth 1", i);
    if (a->q_bf16 && !a->dense && !att)
      return fail(DSA_ERR_INVALID_ARG, "mli layer %d: attend_idx is NULL and no earlier selection to attend", i);
    return DSA_OK;
  });
}

}  // namespace

// ---- allocation-free sparse MLA: the split workspace in a static device
// array.  Layout: kNoAllocGroups group barriers at fixed offsets (so a call of
// one shape never writes partials over the barriers another shape uses; the
// array is zero at load, and every launch leaves its barriers re-armed),
// then the split partials of the current call.  One copy per device; calls
// that overlap in time on one device race on it. ----
constexpr int kNoAllocGroups = 512;  // (row, head group) pairs per call
constexpr size_t kNoAllocSyncBytes = (size_t)kNoAllocGroups * dsa::kSyncWords * sizeof(uint32_t);
constexpr size_t kNoAllocPartialBytes = (size_t)16 << 20;
constexpr size_t kNoAllocScratchBytes = kNoAllocSyncBytes + kNoAllocPartialBytes;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kNoAllocMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device (with that device current).  The array's name in host code is only
// a host-side handle; kernels must be given this address.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  DSA_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, DSA_ERR_UNSUPPORTED, "device %d beyond %d", dev,
              kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DSA_OK;
}

}  // namespace

struct dsa_mli_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

extern "C" {

const char* dsa_last_error(void) { return g_err; }

const char* dsa_version(void) { return "dsa_mli 0.4.0 gfx950"; }

size_t dsa_layer_args_bytes(void) { return sizeof(dsa_layer_args); }

int dsa_sync_timeouts(int reset) { return dsa::group_wait_timeouts(reset); }

int dsa_sync_status(const void* topk_scratch, int B_scan, int slab_stride, const void* workspace, int B_attn,
                    int H, int32_t* status, int clear, void* stream) {
  DSA_REQUIRE(status, DSA_ERR_INVALID_ARG, "dsa_sync_status: null status pointer");
  DSA_REQUIRE(!topk_scratch || (B_scan >= 1 && slab_stride >= 1 && slab_stride <= DSA_TOPK_MAX_CTX),
              DSA_ERR_INVALID_ARG, "dsa_sync_status: bad top-k scratch shape (B_scan %d, slab_stride %d)", B_scan,
              slab_stride);
  DSA_REQUIRE(!workspace || (B_attn >= 1 && H >= 16 && H % 16 == 0), DSA_ERR_INVALID_ARG,
              "dsa_sync_status: bad workspace shape (B_attn %d, H %d)", B_attn, H);
  return hip_status(dsa::launch_sync_status(const_cast<void*>(topk_scratch), B_scan, slab_stride,
                                            const_cast<void*>(workspace), workspace ? B_attn * (H / 16) : 0,
                                            status, clear ? 1 : 0, (hipStream_t)stream),
                    "sync status launch");
}

int dsa_indexer_scan(const void* q_fp8, const float* w, const void* index_k, int64_t num_pages,
                     const int32_t* page_table, const int32_t* seq_lens, float* scores, int B,
                     int Hidx, int pt_stride, int slab_stride, void* stream) {
  int rc = check_scan(q_fp8, w, index_k, num_pages, page_table, seq_lens, scores, B, Hidx,
                      pt_stride, slab_stride);
  if (rc) return rc;
  dsa::ScanArgs S = scan_args(q_fp8, w, index_k, num_pages, page_table, seq_lens, scores, Hidx,
                              pt_stride, slab_stride, nullptr);
  return hip_status(dsa::launch_decode_main(nullptr, 0, &S, B, (hipStream_t)stream),
                    "indexer scan launch");
}

size_t dsa_topk_scratch_bytes(int B, int slab_stride) {
  if (B < 1 || slab_stride < 1 || slab_stride > DSA_TOPK_MAX_CTX) return 0;
  return dsa::topk_scratch_bytes(B, slab_stride);
}

int dsa_topk(const float* scores, const int32_t* seq_lens, const int32_t* page_table,
             int pt_stride, void* scratch, int32_t* out_idx, int B, int slab_stride, int topk,
             int flags, int32_t pad_value, void* stream) {
  int rc = check_topk(scores, seq_lens, page_table, pt_stride, scratch, out_idx, B, slab_stride,
                      topk, flags);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (flags == DSA_TOPK_POSITION_ORDER) {
    // position order: one launch of the decode kernel's select over the given
    // scores (its workgroups split each row and select together).  The
    // select only reads the scores (the score-loading role stores none), so
    // the caller's const buffer is passed through ScanArgs unchanged.
    dsa::ScanArgs S = scan_args(nullptr, nullptr, nullptr, 0, page_table, seq_lens,
                                const_cast<float*>(scores), 16,
                                page_table ? pt_stride : (slab_stride + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS,
                                slab_stride, scratch, out_idx, topk);
    S.from_scores = 1;
    S.standalone = 1;
    S.pad = pad_value;
    return hip_status(dsa::launch_decode_main(nullptr, 0, &S, B, s), "top-k launch");
  }
  rc = hip_status(dsa::launch_topk_hist(scores, seq_lens, scratch, B, slab_stride, topk, s),
                  "top-k histogram launch");
  if (rc) return rc;
  return hip_status(dsa::launch_topk_select(scores, seq_lens, page_table, pt_stride, scratch,
                                            out_idx, B, slab_stride, topk,
                                            flags == DSA_TOPK_SORTED, pad_value, s),
                    "top-k select launch");
}

size_t dsa_sparse_mla_workspace_bytes(int B, int H, int nsplit) {
  if (B < 1 || B > 65535 || H < 16 || H % 16 || H > 16 * 64 || nsplit < 0 || nsplit > 128) return 0;
  return dsa::attn_workspace_bytes(B, H, nsplit > 0 ? nsplit : 128);
}

int dsa_sparse_mla_decode(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                          const int32_t* idx, void* workspace, void* out_bf16, int B, int H,
                          int topk, int nsplit, float sm_scale, void* stream) {
  int rc = check_mla(q_bf16, kv_pool, kv_rows, idx, workspace, out_bf16, B, H, topk, nsplit);
  if (rc) return rc;
  dsa::AttnArgs A = attn_args(q_bf16, kv_pool, kv_rows, idx, workspace, out_bf16, B, H, topk,
                              nsplit, sm_scale);
  return hip_status(dsa::launch_decode_main(&A, B, nullptr, 0, (hipStream_t)stream),
                    "sparse MLA launch");
}

int dsa_dense_mla_decode(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                         const int32_t* page_table, int pt_stride, const int32_t* seq_lens,
                         void* workspace, void* out_bf16, int B, int H, int nsplit, float sm_scale,
                         void* stream) {
  DSA_REQUIRE(page_table && seq_lens && pt_stride >= 1, DSA_ERR_INVALID_ARG,
              "dsa_dense_mla_decode: page_table, seq_lens and pt_stride >= 1 are required");
  DSA_REQUIRE((int64_t)pt_stride * DSA_PAGE_TOKENS <= (int64_t)1 << 30, DSA_ERR_UNSUPPORTED,
              "dsa_dense_mla_decode: pt_stride too large");
  int rc = check_mla(q_bf16, kv_pool, kv_rows, nullptr, workspace, out_bf16, B, H, pt_stride * DSA_PAGE_TOKENS,
                     nsplit, /*idx_required=*/false);
  if (rc) return rc;
  dsa::AttnArgs A = dense_attn_args(q_bf16, kv_pool, kv_rows, page_table, pt_stride, seq_lens, workspace,
                                    out_bf16, B, H, nsplit, sm_scale);
  return hip_status(dsa::launch_decode_main(&A, B, nullptr, 0, (hipStream_t)stream), "dense MLA launch");
}

int dsa_sparse_mla_decode_noalloc(const void* q_bf16, const void* kv_pool, int64_t kv_rows,
                                  const int32_t* idx, void* out_bf16, int B, int H, int topk, int nsplit,
                                  float sm_scale, void* stream) {
  int rc = check_mla(q_bf16, kv_pool, kv_rows, idx, nullptr, out_bf16, B, H, topk, nsplit, true,
                     /*ws_required=*/false);
  if (rc) return rc;
  const int groups = B * (H / 16);
  const int ns = resolve_nsplit(nsplit, topk, B, H);
  const size_t part = dsa::attn_workspace_bytes(B, H, ns) - (size_t)groups * dsa::kSyncWords * sizeof(uint32_t);
  DSA_REQUIRE(groups <= kNoAllocGroups, DSA_ERR_UNSUPPORTED,
              "dsa_sparse_mla_decode_noalloc: B*H/16 = %d above the static limit %d", groups, kNoAllocGroups);
  DSA_REQUIRE(part <= kNoAllocPartialBytes, DSA_ERR_UNSUPPORTED,
              "dsa_sparse_mla_decode_noalloc: %zu partial bytes (B=%d, H=%d, nsplit=%d) above the static %zu",
              part, B, H, ns, kNoAllocPartialBytes);
  void* base = nullptr;
  rc = scratch_ptr(&base);
  if (rc) return rc;
  dsa::AttnArgs A = attn_args(q_bf16, kv_pool, kv_rows, idx, base, out_bf16, B, H, topk, ns, sm_scale);
  // barriers stay at their fixed offsets; the partials follow all of them
  A.sync = reinterpret_cast<uint32_t*>(base);
  A.part_o = reinterpret_cast<float*>(static_cast<unsigned char*>(base) + kNoAllocSyncBytes);
  A.part_ml = A.part_o + (size_t)groups * ns * 16 * DSA_LATENT_DIM;
  return hip_status(dsa::launch_decode_main(&A, B, nullptr, 0, (hipStream_t)stream),
                    "sparse MLA (no-alloc) launch");
}

int dsa_decode_layer(const dsa_layer_args* args, void* stream) {
  int rc = check_layer(args);
  if (rc) return rc;
  const int32_t* att = args->attend_idx ? args->attend_idx : args->next_idx;
  return enqueue_layer(args, args->q_bf16 ? att : nullptr, args->q_fp8 != nullptr,
                       (hipStream_t)stream);
}

int dsa_mli_run_eager_depth(const dsa_layer_args* layers, int num_layers, int lag_depth, void* stream) {
  int rc = check_mli(layers, num_layers, lag_depth);
  if (rc) return rc;
  return enqueue_mli(layers, num_layers, lag_depth, (hipStream_t)stream);
}

int dsa_mli_run_eager(const dsa_layer_args* layers, int num_layers, void* stream) {
  return dsa_mli_run_eager_depth(layers, num_layers, 1, stream);
}

int dsa_mli_graph_create_depth(const dsa_layer_args* layers, int num_layers, int lag_depth,
                               void* capture_stream, dsa_mli_graph** out_graph) {
  DSA_REQUIRE(out_graph, DSA_ERR_INVALID_ARG, "dsa_mli_graph_create: out_graph is null");
  *out_graph = nullptr;
  int rc = check_mli(layers, num_layers, lag_depth);
  if (rc) return rc;
  DSA_REQUIRE(capture_stream, DSA_ERR_INVALID_ARG,
              "dsa_mli_graph_create: capture_stream must be a non-null stream");
  hipStream_t s = (hipStream_t)capture_stream;
  dsa_mli_graph* g = new dsa_mli_graph();
  rc = hip_status(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  if (!rc) {
    const int erc = enqueue_mli(layers, num_layers, lag_depth, s);
    const int crc = hip_status(hipStreamEndCapture(s, &g->graph), "hipStreamEndCapture");
    rc = erc ? erc : crc;
    if (!rc) rc = hip_status(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0),
                             "hipGraphInstantiate");
  }
  if (rc) {
    dsa_mli_graph_destroy(g);
    return rc;
  }
  *out_graph = g;
  return DSA_OK;
}

int dsa_mli_graph_create(const dsa_layer_args* layers, int num_layers, void* capture_stream,
                         dsa_mli_graph** out_graph) {
  return dsa_mli_graph_create_depth(layers, num_layers, 1, capture_stream, out_graph);
}

int dsa_mli_graph_launch(dsa_mli_graph* graph, void* stream) {
  DSA_REQUIRE(graph && graph->exec, DSA_ERR_INVALID_ARG, "dsa_mli_graph_launch: invalid graph");
  return hip_status(hipGraphLaunch(graph->exec, (hipStream_t)stream), "hipGraphLaunch");
}

int dsa_mli_graph_destroy(dsa_mli_graph* graph) {
  if (!graph) return DSA_OK;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
  return DSA_OK;
}

// Internal (not in the public header): phase timestamps.  on=1 clears and
// enables, on=0 disables; read copies n words (n <= 512*16) of the table.
int dsa_internal_debug(int on) {
  DSA_REQUIRE(!on || dsa::kPhaseStamps, DSA_ERR_INVALID_ARG,
              "dsa_internal_debug: library built without -DDSA_PHASE_STAMPS");
  const int v = on ? 1 : 0;
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(dsa::g_dbg_on), &v, sizeof(v));
  if (e == hipSuccess && on) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(dsa::g_dbg));
    if (e == hipSuccess) e = hipMemset(p, 0, sizeof(unsigned long long) * dsa::kDbgBlocks * dsa::kDbgPhases);
  }
  return hip_status(e, "debug enable");
}

int dsa_internal_debug_read(unsigned long long* host, int n) {
  n = std::max(0, std::min(n, dsa::kDbgBlocks * dsa::kDbgPhases));
  return hip_status(hipMemcpyFromSymbol(host, HIP_SYMBOL(dsa::g_dbg), n * sizeof(unsigned long long)),
                    "debug read");
}

// Internal (not in the public header): selects the fp8 MFMA form of the scan.
int dsa_internal_set_scan_variant(int v) {
  dsa::set_scan_variant(v);
  return DSA_OK;
}

int dsa_quantize_index_query(const void* q_bf16, const float* w, void* q_fp8, float* w_fold, int B,
                             int Hidx, void* stream) {
  DSA_REQUIRE(q_bf16 && w && q_fp8 && w_fold, DSA_ERR_INVALID_ARG,
              "dsa_quantize_index_query: null pointer");
  DSA_REQUIRE(B >= 1 && Hidx >= 1, DSA_ERR_INVALID_ARG,
              "dsa_quantize_index_query: B and Hidx must be >= 1 (got %d, %d)", B, Hidx);
  return hip_status(dsa::launch_quant_query(q_bf16, w, q_fp8, w_fold, (long)B * Hidx, (hipStream_t)stream),
                    "quantize index query");
}

int dsa_append_index_keys(const void* k_bf16, const int32_t* rows, const int32_t* pos, int n,
                          const int32_t* page_table, int pt_stride, void* index_k, int64_t num_pages,
                          void* stream) {
  DSA_REQUIRE(n >= 0, DSA_ERR_INVALID_ARG, "dsa_append_index_keys: n must be >= 0 (got %d)", n);
  if (n == 0) return DSA_OK;
  DSA_REQUIRE(k_bf16 && rows && pos && page_table && index_k, DSA_ERR_INVALID_ARG,
              "dsa_append_index_keys: null pointer");
  DSA_REQUIRE(pt_stride >= 1 && num_pages >= 1, DSA_ERR_INVALID_ARG,
              "dsa_append_index_keys: pt_stride and num_pages must be >= 1");
  return hip_status(dsa::launch_append_keys(k_bf16, rows, pos, n, page_table, pt_stride, index_k, (long)num_pages,
                                            (hipStream_t)stream),
                    "append index keys");
}

int dsa_append_latent_rows(const void* latent_bf16, const int32_t* slots, int n, void* kv_pool, int64_t kv_rows,
                           void* stream) {
  DSA_REQUIRE(n >= 0, DSA_ERR_INVALID_ARG, "dsa_append_latent_rows: n must be >= 0 (got %d)", n);
  if (n == 0) return DSA_OK;
  DSA_REQUIRE(latent_bf16 && slots && kv_pool, DSA_ERR_INVALID_ARG, "dsa_append_latent_rows: null pointer");
  DSA_REQUIRE(kv_rows >= 1, DSA_ERR_INVALID_ARG, "dsa_append_latent_rows: kv_rows must be >= 1");
  return hip_status(dsa::launch_append_latent(latent_bf16, slots, n, kv_pool, (long)kv_rows, (hipStream_t)stream),
                    "append latent rows");
}

}  // extern "C"
// Internal: choose the cooperative (1, default) or single-workgroup (0)
// select inside the decode launch; read (and optionally reset) the count of
// group waits that expired.
extern "C" int dsa_internal_set_coop_select(int on) {
  dsa::set_coop_select(on);
  return DSA_OK;
}
extern "C" int dsa_internal_group_wait_timeouts(int reset) { return dsa::group_wait_timeouts(reset); }
// Internal: plain scans of >= 2 rows as one index space over all rows (1,
// default) or per row (0).
extern "C" int dsa_internal_set_flat_scan(int on) {
  dsa::set_flat_scan(on);
  return DSA_OK;
}
// Internal test hook: polls before an in-launch wait gives up (n < 0: the
// default, about a second).  n = 0 makes every wait that is not already
// satisfied give up at once, so tests can check expiry reporting without a
// kernel that waits for long.
extern "C" int dsa_internal_set_spin_limit(int n) {
  dsa::set_spin_limit(n);
  return DSA_OK;
}
extern "C" int dsa_internal_set_scan_blocks_cap(int n) {
  dsa::set_scan_blocks_cap(n);
  return DSA_OK;
}
