// Host-side launch interface between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dsa {

constexpr int kHeadGroup = 16;  // attention heads per head group (one MFMA row block)
constexpr int kFlatRows = 1024;   // rows the flat plain scan takes

// Split-K sparse MLA over the fp8 latent pool (attention role).
struct AttnArgs {
  const uint16_t* q;     // [B, H, 576] bf16
  const uint8_t* pool;   // [kv_rows, 656]
  long kv_rows;
  const int* idx;        // [B, topk] KV slots
  float* part_o;         // [B, H/16, nsplit, 16, 512]
  float* part_ml;        // [B, H/16, nsplit, 16, 2]
  uint32_t* sync;        // [B, H/16] group barriers of the splits, zero before first use
  uint16_t* out;         // [B, H, 512] bf16
  int H, topk, nsplit;
  float sm_log2;         // sm_scale * log2(e)
  // dense attention (idx unused): key j of row b is token j, at KV slot
  // dense_pt[b, j/64]*64 + j%64, for j < dense_lens[b]; topk = the keys a
  // row may hold (dense_pt_stride * 64)
  const int* dense_pt;   // [B, dense_pt_stride] or nullptr
  const int* dense_lens; // [B]
  int dense_pt_stride;
};

// Lightning-indexer scan over the paged fp8 index-K cache (scan role).
struct ScanArgs {
  const uint8_t* q8;     // [B, Hidx, 128] e4m3
  const float* w;        // [B, Hidx]
  const uint8_t* pages;  // [num_pages, 8448]
  long num_pages;
  const int* page_table; // [B, pt_stride]
  const int* seq_lens;   // [B]
  float* scores;         // [B, slab_stride]
  uint32_t* hist;        // top-k scratch rows (nullptr: no histogram)
  long hist_row_words;
  int* next_idx;         // [B, topk]: when set, the row's last scan workgroup
                         // runs the whole top-k select (KV-slot output, -1 pad)
  int topk;
  int pt_stride, slab_stride, Hidx;
  int blocks_per_row;    // filled by the launcher
  int coop;              // filled by the launcher: the row's scan workgroups
                         // select together (group barriers)
  int rows;              // filled by the launcher: B
  int balance;           // filled by the launcher: workgroups per row by length
  int max_nb;            // filled by the launcher: cap on one row's workgroups
  int target;            // filled by the launcher: workgroups to plan for
  int from_scores;       // the select reads the slab instead of scoring keys
  int standalone;        // with from_scores: the top-k op alone (pad below;
                         // page_table may be null: positions are emitted)
  int pad;               // standalone: value of the unused output entries
  int pub_stride;        // filled by the launcher: cooperative-select list
  int pub_target;        // stride and target (0: computed per row)
};

// One grid with n attention blocks (A != nullptr, rows B_att) and scan blocks
// (S != nullptr, rows B_scan).
hipError_t launch_decode_main(const AttnArgs* A, int B_att, const ScanArgs* S, int B_scan,
                              hipStream_t s);
void set_scan_variant(int v);
void set_coop_select(int on);
void set_flat_scan(int on);
void set_scan_blocks_cap(int n);
int group_wait_timeouts(int reset);
void set_spin_limit(int n);  // < 0: the default
// Sum of the expired-wait status words of B_scan top-k scratch rows and
// `groups` attention barrier areas (B * H/16) into *out (device int).
hipError_t launch_sync_status(void* topk_scratch, int B_scan, int slab, void* workspace, int groups, int* out,
                              int clear, hipStream_t s);
// Plain scan of 2..1024 rows as one index space (scan_flat.hip); with A,
// the attention of B_att rows in the same grid (A->nsplit splits per row
// and head group).
hipError_t launch_flat_scan(const AttnArgs* A, int B_att, const ScanArgs& S, int B, hipStream_t s);
bool flat_scan_fits(const ScanArgs& S, int B);
bool flat_scan_on();
int device_cu_count();
int attn_auto_nsplit(int topk, int B, int H);
int attn_fused_nsplit(int topk, int B, int H);
size_t attn_workspace_bytes(int B, int H, int nsplit);
void attn_bind_workspace(AttnArgs& A, void* ws, int B);

// Top-k: histogram (standalone) + select (filter, last arriver finalizes).
size_t topk_scratch_bytes(int B, int slab);
size_t row_select_lds_bytes();
long topk_row_words(int slab);
hipError_t launch_topk_hist(const float* scores, const int* seq_lens, void* scratch, int B,
                            int slab, int K, hipStream_t s);
hipError_t launch_topk_select(const float* scores, const int* seq_lens, const int* page_table,
                              int pt_stride, void* scratch, int* out, int B, int slab, int K,
                              int sorted, int pad, hipStream_t s);

// Decode-step operand preparation (quant.hip).
hipError_t launch_quant_query(const void* q_bf16, const float* w, void* codes, float* w_out, long rows,
                              hipStream_t s);
hipError_t launch_append_keys(const void* k_bf16, const int* rows, const int* pos, int n, const int* page_table,
                              int pt_stride, void* pages, long num_pages, hipStream_t s);
hipError_t launch_append_latent(const void* lat_bf16, const int* slots, int n, void* pool, long kv_rows,
                                hipStream_t s);

}  // namespace dsa
