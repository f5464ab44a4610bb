// Exact top-k select over rows of fp32 scores (gfx950).
//
// Ranking: rank_key() order (score descending, -0.0 == +0.0, NaN above +inf);
// ties at the threshold go to the lower index.  That is the reference's
// select_topk (attention_core.py:66-91: torch.topk + non-finite -> sentinel)
// with its unspecified tie order pinned to "lower index wins", computed with
// the radix-select structure of the GPU selectors (tilelang_dsa/
// topk_selector.py:36-194; in-kernel exact select K:1097-1129, K:1248-1310).
//
// Two launches (the histogram is fused into the indexer scan on the decode
// path, leaving one), so a 128K-196K row is read by many CUs:
//   (A) histogram: workgroups over 4096-score slices build an LDS histogram
//       of the 12 high key bits and add its non-zero bins to the row's
//       global histogram (the scan role of the main decode launch does the
//       same for the scores it produces);
//   (B) select: every slice workgroup derives the same threshold bin T1 from
//       the global histogram, writes the row's "key bin > T1" membership
//       bitmap with wave ballots (one owner per word, no atomics), and
//       appends the bin-T1 keys to a candidate list; the LAST slice
//       workgroup of the row to arrive (arrival counter, no waiting) then
//       finalizes: two 10-bit refinements over the candidates give the exact
//       threshold key t*; candidates above t* and the lowest-index keys equal
//       to t* join the bitmap; prefix popcounts emit the result.  If the
//       candidate list overflowed, the finalize refines by re-reading the row
//       (exact either way).
// Every ordering decision is a bitmap prefix count: the output is
// deterministic.  The per-row scratch (histogram + counters) must be zero
// before the first call; the finalize clears it again, so calls chain and
// replay in graphs without a memset.
#include <algorithm>

#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

__device__ int g_dbg_on = 0;
__device__ unsigned long long g_dbg[kDbgBlocks * kDbgPhases];
__device__ int g_group_wait_timeouts = 0;
__device__ int g_group_spin_max = kGroupSpinMax;

constexpr int kNB1 = 4096;      // first digit: key bits [31:20]
constexpr int kNB2 = 1024;      // refinements: bits [19:10], [9:0]
constexpr int kCandCap = 4096;  // bin-T1 candidates kept per row
constexpr int kMaxWords = DSA_TOPK_MAX_CTX / 32;
constexpr int kSliceThreads = 256;
constexpr int kSlice = 4096;    // scores per slice workgroup (16 per thread)

// per-row scratch layout (uint32 words)
constexpr int kHistOff = 0;
constexpr int kCntOff = kNB1;       // bin-T1 candidate count
constexpr int kArrOff = kNB1 + 1;   // select workgroups arrived
// cooperative select inside the decode launch (decode_main.hip): per-row
// group barriers live after the candidates; per-workgroup counts in the
// bitmap area, candidates (keys, then positions) in the candidate area
constexpr int kBmOff = kNB1 + 64;

__host__ __device__ inline long bitmap_words(int slab) { return ((long)slab + 2047) / 2048 * 64; }
// group-barrier area (after the candidates): per barrier, kSyncGroups
// arrival counters, one top counter and 8 release flags, each in its own
// 256-byte line
constexpr int kSyncGroups = 16;
constexpr int kSyncFlags = 8;
constexpr int kSyncLine = 64;  // words
constexpr int kSyncWords = (kSyncGroups + 1 + kSyncFlags) * kSyncLine;
constexpr int kNumSync = 4;  // slots 0 and 3: the list barrier (group_barrier_rep)
static_assert(kSyncGroups == kGroupSyncGroups && kSyncFlags == kGroupSyncFlags && kSyncLine == kGroupSyncLine,
              "group-barrier layout");
__host__ __device__ inline long row_sync_off(int slab) { return kBmOff + bitmap_words(slab) + 2L * kCandCap; }
// published local top keys of the cooperative select (decode_main.hip):
// kPubHdrWords of per-workgroup headers, then kPubWords of key lists
constexpr int kPubWords = 16384;
constexpr int kPubHdrWords = 4 * 256;
__host__ __device__ inline long row_pub_off(int slab) { return row_sync_off(slab) + (long)kNumSync * kSyncWords; }
__host__ __device__ inline long row_scratch_words(int slab) {
  return row_pub_off(slab) + kPubHdrWords + kPubWords;
}

// Exclusive prefix sum over the block (thread order); *total gets the sum.
// wave_tmp holds one word per wave.
// TRAIL = false drops the closing barrier: the caller then guarantees a
// block barrier before wave_tmp is written again.
template <bool TRAIL = true>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tmp, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const uint32_t inc = wave_scan_incl(v);
  if (lane == kWave - 1) wave_tmp[wv] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < nwaves; ++i) {
    const uint32_t x = wave_tmp[i];
    before += (i < wv) ? x : 0u;
    tot += x;
  }
  if constexpr (TRAIL) __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Largest bin T with sum_{b >= T} hist[b] >= need (need >= 1 and the total
// >= need).  Writes T to res[0] and the count strictly above T to res[1].
__device__ __forceinline__ void find_threshold(const uint32_t* hist, int nbins, uint32_t need, uint32_t* wave_tmp,
                               uint32_t* res) {
  const int per = nbins / (int)blockDim.x;
  const int hi = nbins - (int)threadIdx.x * per;  // this thread: bins [hi-per, hi)
  uint32_t local = 0;
  for (int i = 1; i <= per; ++i) local += hist[hi - i];
  uint32_t total;
  uint32_t acc = block_exclusive_scan(local, wave_tmp, &total);
  for (int i = 1; i <= per; ++i) {
    const uint32_t h = hist[hi - i];
    if (acc < need && acc + h >= need) {
      res[0] = (uint32_t)(hi - i);
      res[1] = acc;
    }
    acc += h;
  }
  __syncthreads();
}

// find_threshold for a compile-time NBINS / NT (>= 1 bin per thread),
// every loop unrolled so the LDS reads are in flight together; also writes
// the histogram's total to res[2] (res: 3 words).
template <int NBINS, int NT>
__device__ __forceinline__ void find_threshold_fixed(const uint32_t* hist, uint32_t need, uint32_t* wave_tmp,
                                                     uint32_t* res) {
  constexpr int kPer = NBINS / NT;
  static_assert(kPer >= 1 && NBINS % NT == 0, "bins per thread");
  const int hi = NBINS - (int)threadIdx.x * kPer;
  uint32_t h[kPer];
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    h[i] = hist[hi - 1 - i];
    local += h[i];
  }
  uint32_t total;
  uint32_t acc = block_exclusive_scan(local, wave_tmp, &total);
  if (threadIdx.x == 0) res[2] = total;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (acc < need && acc + h[i] >= need) {
      res[0] = (uint32_t)(hi - 1 - i);
      res[1] = acc;
    }
    acc += h[i];
  }
  __syncthreads();
}

// dst[0..n) = src[0..n) for n 32-bit words, with every load of the block
// issued before any LDS store (PER uint4 per thread covers n <= PER*4*blockDim).
// Both pointers 16-byte aligned; the tail (n % 4) is copied word by word.
// DEV: device-scope loads (data published in this launch by other workgroups).
template <int PER, bool DEV = false>
__device__ __forceinline__ void copy_words_to_lds(uint32_t* dst, const uint32_t* src, int n) {
  const int t = threadIdx.x, nt = blockDim.x;
  const int n4 = n >> 2;
  const __amdgpu_buffer_rsrc_t rsrc = dev_rsrc(src, (uint32_t)n * 4u);
  uint4 r[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = t + j * nt;
    if (i < n4) r[j] = DEV ? load_dev16(rsrc, 16u * i) : reinterpret_cast<const uint4*>(src)[i];
  }
  uint32_t tail = 0;
  const int ti = (n4 << 2) + t;
  if (ti < n) tail = DEV ? load_dev4(rsrc, 4u * ti) : src[ti];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = t + j * nt;
    if (i < n4) reinterpret_cast<uint4*>(dst)[i] = r[j];
  }
  if (ti < n) dst[ti] = tail;
}

__device__ __forceinline__ int row_len(const int* seq_lens, int row, int slab) {
  return max(0, min(seq_lens[row], slab));
}

// ---------------------------------------------------------------- (A)
__global__ __launch_bounds__(kSliceThreads) void topk_hist_kernel(
    const float* __restrict__ scores, const int* __restrict__ seq_lens,
    uint32_t* __restrict__ scratch, int slab, int K) {
  __shared__ uint32_t hist[kNB1];
  const int row = blockIdx.y;
  const int len = row_len(seq_lens, row, slab);
  const int p0 = blockIdx.x * kSlice;
  if (len <= K || p0 >= len) return;
  const int t = threadIdx.x;
  for (int i = t; i < kNB1; i += kSliceThreads) hist[i] = 0u;
  __syncthreads();
  const float* s = scores + (long)row * slab;
  constexpr int kPer = kSlice / kSliceThreads;
  float v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = p0 + t + j * kSliceThreads;
    v[j] = (i < len) ? s[i] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (p0 + t + j * kSliceThreads < len) atomicAdd(&hist[rank_key(v[j]) >> 20], 1u);
  __syncthreads();
  uint32_t* g = scratch + (long)row * row_scratch_words(slab) + kHistOff;
  for (int i = t; i < kNB1; i += kSliceThreads)
    if (hist[i]) atomicAdd(&g[i], hist[i]);
}

// ---------------------------------------------------------------- (B)
// Filter one 4096-score slice (len > K, p0 < len).  hist/wave_tmp/res/woff
// are LDS of the calling workgroup.
__device__ __forceinline__ void filter_slice(const float* __restrict__ s, int len, int p0, uint32_t* rs, int slab,
                             int K, int keep_nonfinite, uint32_t* hist, uint32_t* wave_tmp,
                             uint32_t* res, uint32_t* woff) {
  const int t = threadIdx.x;
  const int dbk = blockIdx.y * gridDim.x + blockIdx.x;
  copy_words_to_lds<kNB1 / 4 / kSliceThreads>(hist, rs + kHistOff, kNB1);
  __syncthreads();
  dbg_stamp(dbk, 1);
  find_threshold(hist, kNB1, (uint32_t)K, wave_tmp, res);
  const uint32_t T1 = res[0];
  dbg_stamp(dbk, 2);

  uint32_t* bm = rs + kBmOff;
  uint32_t* cand = rs + kBmOff + bitmap_words(slab);
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  constexpr int kIters = kSlice / kSliceThreads;
  float v[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int i = p0 + wv * kWave + it * kSliceThreads + lane;
    v[it] = (i < len) ? s[i] : 0.f;
  }
  // pass 1: ballots; bitmap words; per-wave candidate counts
  uint64_t eqm[kIters];
  uint32_t wcount = 0;
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int base = p0 + wv * kWave + it * kSliceThreads;
    const int i = base + lane;
    const bool valid = i < len;
    const uint32_t k = valid ? rank_key(v[it]) : 0u;
    const uint32_t bin = k >> 20;
    const uint64_t gt = __ballot(valid && bin > T1 && (keep_nonfinite || key_is_finite(k)));
    eqm[it] = __ballot(valid && bin == T1);
    wcount += (uint32_t)__popcll(eqm[it]);
    if (lane == 0 && base < len) {
      store_dev(&bm[base >> 5], (uint32_t)gt);
      store_dev(&bm[(base >> 5) + 1], (uint32_t)(gt >> 32));
    }
  }
  dbg_stamp(dbk, 3);
  // one global reservation per workgroup for its bin-T1 candidates
  if (lane == 0) woff[wv] = wcount;
  __syncthreads();
  if (t == 0) {
    uint32_t tot = 0;
    for (int w = 0; w < kSliceThreads / kWave; ++w) { const uint32_t c = woff[w]; woff[w] = tot; tot += c; }
    woff[kSliceThreads / kWave] = tot ? atomicAdd(&rs[kCntOff], tot) : 0u;
  }
  __syncthreads();
  if (wcount) {
    uint32_t slot0 = woff[kSliceThreads / kWave] + woff[wv];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if ((eqm[it] >> lane) & 1ull) {
        const uint32_t slot = slot0 + (uint32_t)__popcll(eqm[it] & lt_mask);
        if (slot < (uint32_t)kCandCap) {
          store_dev(&cand[2 * slot], rank_key(v[it]));
          store_dev(&cand[2 * slot + 1], (uint32_t)(p0 + wv * kWave + it * kSliceThreads + lane));
        }
      }
      slot0 += (uint32_t)__popcll(eqm[it]);
    }
  }
}


// Exact threshold key among the bin-T1 candidates ck[0..nc): two 10-bit
// refinements (key bits [19:10], then [9:0]) of the `need1` keys still to
// select.  tstar = the K-th ranked key, need3 = how many keys equal to it
// are selected.  hist (>= kNB2 words of LDS) must be zero on entry and is
// left dirty.
__device__ __forceinline__ void refine_candidates(const uint32_t* ck, int nc, uint32_t T1, uint32_t need1,
                                                  uint32_t* hist, uint32_t* wave_tmp, uint32_t* res,
                                                  uint32_t& tstar, uint32_t& need3) {
  const int t = threadIdx.x, nthr = blockDim.x;
  for (int j = t; j < nc; j += nthr) atomicAdd(&hist[(ck[j] >> 10) & 1023u], 1u);
  __syncthreads();
  find_threshold(hist, kNB2, need1, wave_tmp, res);
  const uint32_t T2 = res[0];
  const uint32_t need2 = need1 - res[1];
  __syncthreads();
  for (int i = t; i < kNB2; i += nthr) hist[i] = 0u;
  __syncthreads();
  const uint32_t pre2 = (T1 << 10) | T2;
  for (int j = t; j < nc; j += nthr) {
    const uint32_t k = ck[j];
    if ((k >> 10) == pre2) atomicAdd(&hist[k & 1023u], 1u);
  }
  __syncthreads();
  find_threshold(hist, kNB2, need2, wave_tmp, res);
  tstar = (pre2 << 10) | res[0];
  need3 = need2 - res[1];
}

// ---------------------------------------------------------------- (C)
// Per-row resolution in one workgroup of any size (256 in the select
// kernel, 512 when the decode launch's last scan workgroup of a row runs it).
struct FinShared {
  uint32_t sel[kMaxWords];
  uint32_t tie[kMaxWords];
  uint32_t cand_key[kCandCap];
  int cand_idx[kCandCap];
  uint32_t hist[kNB1];
  int pt[kMaxWords / 2];  // page-table row (DSA_TOPK_MAX_CTX / 64 pages)
  uint32_t wave_tmp[16];
  uint32_t res[4];
  uint32_t woff[kSliceThreads / kWave + 1];
  uint32_t ncand;
  uint32_t last;
};

__device__ __forceinline__ void set_bit(uint32_t* bm, int i) {
  atomicOr(&bm[i >> 5], 1u << (i & 31));
}

// sel |= the `need` lowest-index set bits of tie.
__device__ __forceinline__ void take_lowest_ties(FinShared& sh, int nw, uint32_t need) {
  const int t = threadIdx.x, nthr = blockDim.x;
  const int per = (nw + nthr - 1) / nthr;
  const int w0 = min(nw, t * per), w1 = min(nw, w0 + per);
  uint32_t local = 0;
  for (int i = w0; i < w1; ++i) local += __popc(sh.tie[i]);
  uint32_t total;
  uint32_t pre = block_exclusive_scan(local, sh.wave_tmp, &total);
  for (int i = w0; i < w1 && pre < need; ++i) {
    uint32_t word = sh.tie[i];
    const uint32_t cnt = __popc(word);
    if (pre + cnt > need) {
      uint32_t keep = 0;
      for (uint32_t k = pre; k < need; ++k) {
        const uint32_t low = word & (0u - word);
        keep |= low;
        word ^= low;
      }
      word = keep;
    }
    sh.sel[i] |= word;
    pre += cnt;
  }
  __syncthreads();
}

// One pass over the row's scores building, in LDS, the "bin > T1" bitmap
// (finite scores only unless keep) and the bin-T1 candidate list.  Each
// wave reads 64 consecutive scores per load (256 coalesced bytes) so one
// ballot is two bitmap words; lane j keeps the ballot of iteration j and
// the wave stores its kPassJ ballots with one write per lane.  Candidates are
// rare (about one score in a hundred): each lane flags its own in a 64-bit
// mask, a wave prefix sum places them, one LDS atomic per wave reserves
// the space.
constexpr int kPassJ = 32;  // <= kWave: ballot j is kept by lane j

__device__ __forceinline__ void pass_load(float (&v)[kPassJ], __amdgpu_buffer_rsrc_t rsrc, int wbase,
                                          int lane) {
#pragma unroll
  for (int j = 0; j < kPassJ; ++j) v[j] = __uint_as_float(load_dev4(rsrc, 4u * (wbase + j * kWave + lane)));
}

__device__ __forceinline__ void pass_batch(FinShared& sh, const float (&v)[kPassJ], int wbase, int len,
                                           uint32_t T1, bool keep, bool collect, int lane) {
  uint64_t mine = 0, candm = 0;
#pragma unroll
  for (int j = 0; j < kPassJ; ++j) {
    const int p = wbase + j * kWave + lane;
    const uint32_t k = rank_key(v[j]);
    const uint32_t bin = k >> 20;
    const bool in = p < len;
    const uint64_t gt = __ballot(in && bin > T1 && (keep || key_is_finite(k)));
    mine = (lane == j) ? gt : mine;
    candm |= (uint64_t)(in && bin == T1) << j;
  }
  const int wpos = wbase + lane * kWave;  // iteration `lane`'s first position
  if (lane < kPassJ && wpos < len)
    *reinterpret_cast<uint2*>(&sh.sel[wpos >> 5]) = make_uint2((uint32_t)mine, (uint32_t)(mine >> 32));
  if (!collect || !__ballot(candm != 0)) return;
  const uint32_t c = (uint32_t)__popcll(candm);
  uint32_t incl = c;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t n = __shfl_up(incl, o);
    if (lane >= o) incl += n;
  }
  const uint32_t total = __shfl(incl, kWave - 1);
  uint32_t base = 0;
  if (lane == 0) base = atomicAdd(&sh.ncand, total);
  uint32_t slot = __shfl(base, 0) + incl - c;
#pragma unroll
  for (int j = 0; j < kPassJ; ++j) {
    if ((candm >> j) & 1ull) {
      if (slot < (uint32_t)kCandCap) {
        sh.cand_key[slot] = rank_key(v[j]);
        sh.cand_idx[slot] = wbase + j * kWave + lane;
      }
      ++slot;
    }
  }
}

__device__ __forceinline__ void pass_over_scores(FinShared& sh, const float* __restrict__ s, int len,
                                                 int slab, uint32_t T1, bool keep, bool collect) {
  const int t = threadIdx.x, nthr = blockDim.x;
  const int lane = t & (kWave - 1), wv = t / kWave, nwv = nthr / kWave;
  // the scores were published in this launch: device-scope loads; the
  // resource spans the row's first slab floats (loads past it return 0)
  const __amdgpu_buffer_rsrc_t rsrc = dev_rsrc(s, (uint32_t)slab * 4u);
  const int per_batch = nwv * kPassJ * kWave;
  const int woff = wv * kPassJ * kWave;
  for (int b0 = 0; b0 + woff < len; b0 += per_batch) {
    float v[kPassJ];
    pass_load(v, rsrc, b0 + woff, lane);
    pass_batch(sh, v, b0 + woff, len, T1, keep, collect, lane);
  }
}

// keep_nonfinite = 0 (position order): sel holds only finite selections --
// selected non-finite scores become pads; 1 (sorted): sel holds every
// selected index and non-finite ones turn into pads where they sort.
// fused = true: the bitmap and candidates come from a pass over the scores
// here; false: from the select kernel's slice workgroups (scratch).
__device__ __forceinline__ void finalize_row(FinShared& sh, const float* __restrict__ s, int len,
                             const int* __restrict__ pt_row, int pt_stride, uint32_t* rs,
                             int* __restrict__ o, int slab, int K, int sorted, int pad, bool fused) {
  const int t = threadIdx.x, nthr = blockDim.x;
  const int nw = (len + 31) >> 5;
  const bool keep = sorted != 0;
  const bool map_slots = pt_row != nullptr;
  if (map_slots) {  // the row may be unaligned: plain batched loads
    const int npt = min(pt_stride, (len + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS);
    constexpr int kPer = kMaxWords / 2 / kSliceThreads;
    int v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = t + j * nthr;
      v[j] = (i < npt) ? pt_row[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (t + j * nthr < npt) sh.pt[t + j * nthr] = v[j];
  }

  if (len <= K) {
    // everything is selected; position order drops the non-finite scores
    for (int i = t; i < nw; i += nthr) {
      float v[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) v[j] = (i * 32 + j < len) ? s[i * 32 + j] : 0.f;
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (i * 32 + j < len && (keep || key_is_finite(rank_key(v[j])))) word |= 1u << j;
      sh.sel[i] = word;
    }
    __syncthreads();
  } else {
    const uint32_t* bm = rs + kBmOff;
    const uint32_t* cand = rs + kBmOff + bitmap_words(slab);
    if (!fused) copy_words_to_lds<kMaxWords / 4 / kSliceThreads, true>(sh.sel, bm, nw);
    copy_words_to_lds<kNB1 / 4 / kSliceThreads, true>(sh.hist, rs + kHistOff, kNB1);
    for (int i = t; i < nw; i += nthr) sh.tie[i] = 0u;
    if (t == 0) sh.ncand = 0u;
    __syncthreads();
    find_threshold(sh.hist, kNB1, (uint32_t)K, sh.wave_tmp, sh.res);
    const uint32_t T1 = sh.res[0];
    const uint32_t need1 = (uint32_t)K - sh.res[1];
    const uint32_t in_bin = sh.hist[T1];
    dbg_stamp(blockIdx.y * gridDim.x + blockIdx.x, 12);
    __syncthreads();
    for (int i = t; i < kNB2; i += nthr) sh.hist[i] = 0u;
    if (fused) pass_over_scores(sh, s, len, slab, T1, keep, in_bin <= (uint32_t)kCandCap);
    __syncthreads();
    if (fused) dbg_stamp(blockIdx.y * gridDim.x + blockIdx.x, 6);
    if (fused && in_bin > (uint32_t)kCandCap) dbg_stamp(blockIdx.y * gridDim.x + blockIdx.x, 7);

    uint32_t tstar, need3;
    if (in_bin <= (uint32_t)kCandCap) {
      const int nc = (int)in_bin;
      if (!fused) {  // (key, idx) pairs, device scope, all loads in flight
        constexpr int kPer = kCandCap / kSliceThreads;
        const __amdgpu_buffer_rsrc_t crs = dev_rsrc(cand, 8u * kCandCap);
        uint2 v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int i = t + j * nthr;
          if (i < nc) v[j] = make_uint2(load_dev4(crs, 8u * i), load_dev4(crs, 8u * i + 4u));
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int i = t + j * nthr;
          if (i < nc) { sh.cand_key[i] = v[j].x; sh.cand_idx[i] = (int)v[j].y; }
        }
        __syncthreads();
      }
      refine_candidates(sh.cand_key, nc, T1, need1, sh.hist, sh.wave_tmp, sh.res, tstar, need3);
      for (int j = t; j < nc; j += nthr) {
        const uint32_t k = sh.cand_key[j];
        if (k > tstar) {
          if (keep || key_is_finite(k)) set_bit(sh.sel, sh.cand_idx[j]);
        } else if (k == tstar) {
          set_bit(sh.tie, sh.cand_idx[j]);
        }
      }
      __syncthreads();
    } else {
      // candidate list overflowed: refine by re-reading the row
      for (int i = t; i < len; i += nthr) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 20) == T1) atomicAdd(&sh.hist[(k >> 10) & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need1, sh.wave_tmp, sh.res);
      const uint32_t T2 = sh.res[0];
      const uint32_t need2 = need1 - sh.res[1];
      __syncthreads();
      for (int i = t; i < kNB2; i += nthr) sh.hist[i] = 0u;
      __syncthreads();
      const uint32_t pre2 = (T1 << 10) | T2;
      for (int i = t; i < len; i += nthr) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 10) == pre2) atomicAdd(&sh.hist[k & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need2, sh.wave_tmp, sh.res);
      tstar = (pre2 << 10) | sh.res[0];
      need3 = need2 - sh.res[1];
      for (int i = t; i < len; i += nthr) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 20) != T1) continue;
        if (k > tstar) {
          if (keep || key_is_finite(k)) set_bit(sh.sel, i);
        } else if (k == tstar) {
          set_bit(sh.tie, i);
        }
      }
      __syncthreads();
    }
    // the ties all carry key t*: in position order they are pads if t* is not finite
    dbg_stamp(blockIdx.y * gridDim.x + blockIdx.x, 13);
    if constexpr (kPhaseStamps)
      if (fused && t == 0 && g_dbg_on && blockIdx.x < kDbgBlocks) g_dbg[blockIdx.x * kDbgPhases + 11] = in_bin;
    if (keep || key_is_finite(tstar)) take_lowest_ties(sh, nw, need3);
  }
  // re-arm the row's histogram and candidate count for the next call (the
  // fused scan adds to the histogram even for rows of <= K scores)
  __syncthreads();
  for (int i = t; i < kNB1; i += nthr) rs[kHistOff + i] = 0u;
  if (t == 0) rs[kCntOff] = 0u;

  dbg_stamp(blockIdx.y * gridDim.x + blockIdx.x, 14);
  // ---- emit ----
  const int per = (nw + nthr - 1) / nthr;
  const int w0 = min(nw, t * per), w1 = min(nw, w0 + per);
  uint32_t local = 0;
  for (int i = w0; i < w1; ++i) local += __popc(sh.sel[i]);
  uint32_t nsel;
  uint32_t pos = block_exclusive_scan(local, sh.wave_tmp, &nsel);
  if (!sorted) {
    for (int i = w0; i < w1; ++i) {
      uint32_t word = sh.sel[i];
      while (word) {
        const int b = __ffs(word) - 1;
        word &= word - 1;
        const int g = i * 32 + b;
        o[min(pos++, (uint32_t)K - 1u)] = map_slots ? (sh.pt[g >> 6] * DSA_PAGE_TOKENS + (g & 63)) : g;  // < K by construction
      }
    }
    for (int j = (int)nsel + t; j < K; j += nthr) o[j] = pad;
    return;
  }

  // sorted: gather (key, idx) of the selection, bitonic sort (key desc, idx asc)
  for (int i = w0; i < w1; ++i) {
    uint32_t word = sh.sel[i];
    while (word) {
      const int b = __ffs(word) - 1;
      word &= word - 1;
      sh.cand_idx[pos++] = i * 32 + b;
    }
  }
  __syncthreads();
  for (int j = t; j < (int)nsel; j += nthr) sh.cand_key[j] = rank_key(s[sh.cand_idx[j]]);
  int P = 1;
  while (P < (int)nsel) P <<= 1;
  for (int j = (int)nsel + t; j < P; j += nthr) {
    sh.cand_key[j] = 0u;  // below every real key (-inf is 0x007fffff)
    sh.cand_idx[j] = 0x7fffffff;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = t; i < P; i += nthr) {
        const int p = i ^ j;
        if (p > i) {
          const uint32_t ka = sh.cand_key[i], kb = sh.cand_key[p];
          const int ia = sh.cand_idx[i], ib = sh.cand_idx[p];
          const bool a_first = (ka > kb) || (ka == kb && ia < ib);
          const bool up = ((i & k) == 0);
          if (up ? !a_first : a_first) {
            sh.cand_key[i] = kb; sh.cand_key[p] = ka;
            sh.cand_idx[i] = ib; sh.cand_idx[p] = ia;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int j = t; j < K; j += nthr) {
    int v = pad;
    if (j < (int)nsel && key_is_finite(sh.cand_key[j])) v = sh.cand_idx[j];
    o[j] = v;
  }
}

__global__ __launch_bounds__(kSliceThreads) void topk_select_kernel(
    const float* __restrict__ scores, const int* __restrict__ seq_lens,
    const int* __restrict__ page_table, int pt_stride, uint32_t* __restrict__ scratch,
    int* __restrict__ out, int slab, int K, int sorted, int pad) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  FinShared& sh = *reinterpret_cast<FinShared*>(smem_raw);
  const int row = blockIdx.y;
  const int t = threadIdx.x;
  const float* s = scores + (long)row * slab;
  uint32_t* rs = scratch + (long)row * row_scratch_words(slab);
  const int len = row_len(seq_lens, row, slab);
  const int p0 = blockIdx.x * kSlice;
  const int dbk = blockIdx.y * gridDim.x + blockIdx.x;
  dbg_stamp(dbk, 8);
  if (len > K && p0 < len)
    filter_slice(s, len, p0, rs, slab, K, sorted, sh.hist, sh.wave_tmp, sh.res, sh.woff);
  dbg_stamp(dbk, 9);
  // arrival: the row's last slice workgroup finalizes (the bitmap and the
  // candidates went out with device-scope stores; wait for them, then count)
  wait_mem();
  __syncthreads();
  if (t == 0) {
    const uint32_t prev = atomicAdd(&rs[kArrOff], 1u);
    sh.last = (prev == gridDim.x - 1u) ? 1u : 0u;
  }
  __syncthreads();
  dbg_stamp(dbk, 10);
  if (!sh.last) return;
  if (t == 0) rs[kArrOff] = 0u;
  dbg_stamp(dbk, 11);
  finalize_row(sh, s, len, page_table ? page_table + (long)row * pt_stride : nullptr, pt_stride, rs,
               out + (long)row * K, slab, K, sorted, pad, /*fused=*/false);
  dbg_stamp(dbk, 15);
}

size_t row_select_lds_bytes() { return sizeof(FinShared); }

size_t topk_scratch_bytes(int B, int slab) {
  return (size_t)B * row_scratch_words(slab) * sizeof(uint32_t);
}

long topk_row_words(int slab) { return row_scratch_words(slab); }

hipError_t launch_topk_hist(const float* scores, const int* seq_lens, void* scratch, int B,
                            int slab, int K, hipStream_t s) {
  const dim3 slices((slab + kSlice - 1) / kSlice, B);
  hipLaunchKernelGGL(topk_hist_kernel, slices, dim3(kSliceThreads), 0, s, scores, seq_lens,
                     reinterpret_cast<uint32_t*>(scratch), slab, K);
  return hipGetLastError();
}

hipError_t launch_topk_select(const float* scores, const int* seq_lens, const int* page_table,
                              int pt_stride, void* scratch, int* out, int B, int slab, int K,
                              int sorted, int pad, hipStream_t s) {
  static PerDeviceOnce attr;
  const hipError_t e = attr.run([] {
    return hipFuncSetAttribute((const void*)topk_select_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)sizeof(FinShared));
  });
  if (e != hipSuccess) return e;
  const dim3 slices((slab + kSlice - 1) / kSlice, B);
  hipLaunchKernelGGL(topk_select_kernel, slices, dim3(kSliceThreads), sizeof(FinShared), s, scores,
                     seq_lens, page_table, pt_stride, reinterpret_cast<uint32_t*>(scratch), out,
                     slab, K, sorted, pad);
  return hipGetLastError();
}

}  // namespace dsa
