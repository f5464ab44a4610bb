// Exact top-k select over rows of fp32 scores (gfx950).
//
// Ranking: rank_key() order (score descending, -0.0 == +0.0, NaN above +inf);
// ties at the threshold go to the lower index.  That is the reference's
// select_topk (attention_core.py:66-91: torch.topk + non-finite -> sentinel)
// with its unspecified tie order pinned to "lower index wins", computed with
// the radix-select structure of the GPU selectors (tilelang_dsa/
// topk_selector.py:36-194; in-kernel exact select K:1097-1129, K:1248-1310).
//
// Three launches, so a 128K-196K row is read by many CUs instead of one:
//   (A) histogram: workgroups over 4096-score slices build an LDS histogram
//       of the 12 high key bits and add its non-zero bins to the row's
//       global histogram;
//   (B) filter: every slice workgroup derives the same threshold bin T1 from
//       the global histogram, writes the row's "key bin > T1" membership
//       bitmap with wave ballots (one owner per word, no atomics), and
//       appends the bin-T1 keys to a candidate list;
//   (C) finalize, one workgroup per row: two 10-bit refinements over the
//       candidates give the exact threshold key t*; candidates above t* and
//       the lowest-index keys equal to t* join the bitmap; prefix popcounts
//       emit the result.  If the candidate list overflowed, (C) refines by
//       re-reading the row (exact either way).
// Every ordering decision is a bitmap prefix count: the output is
// deterministic.  The per-row scratch (histogram + counter) must be zero
// before the first call; (C) clears it again, so calls chain and replay
// in graphs without a memset.
#include <algorithm>

#include "dsa_common.h"

namespace dsa {

constexpr int kNB1 = 4096;      // first digit: key bits [31:20]
constexpr int kNB2 = 1024;      // refinements: bits [19:10], [9:0]
constexpr int kCandCap = 4096;  // bin-T1 candidates kept per row
constexpr int kMaxWords = DSA_TOPK_MAX_CTX / 32;
constexpr int kSliceThreads = 256;
constexpr int kSlice = 4096;    // scores per slice workgroup (16 per thread)
constexpr int kFinThreads = 1024;

// per-row scratch layout (uint32 words)
constexpr int kHistOff = 0;
constexpr int kCntOff = kNB1;
constexpr int kBmOff = kNB1 + 64;

__host__ __device__ inline long bitmap_words(int slab) { return ((long)slab + 2047) / 2048 * 64; }
__host__ __device__ inline long row_scratch_words(int slab) {
  return kBmOff + bitmap_words(slab) + 2L * kCandCap;
}

// Exclusive prefix sum over the block (thread order); *total gets the sum.
// wave_tmp holds one word per wave.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tmp, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  uint32_t inc = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t n = __shfl_up(inc, o);
    if (lane >= o) inc += n;
  }
  if (lane == kWave - 1) wave_tmp[wv] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < nwaves; ++i) {
    const uint32_t x = wave_tmp[i];
    before += (i < wv) ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Largest bin T with sum_{b >= T} hist[b] >= need (need >= 1 and the total
// >= need).  Writes T to res[0] and the count strictly above T to res[1].
__device__ void find_threshold(const uint32_t* hist, int nbins, uint32_t need, uint32_t* wave_tmp,
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
  const int p1 = min(len, p0 + kSlice);
  for (int i = p0 + t; i < p1; i += kSliceThreads) atomicAdd(&hist[rank_key(s[i]) >> 20], 1u);
  __syncthreads();
  uint32_t* g = scratch + (long)row * row_scratch_words(slab) + kHistOff;
  for (int i = t; i < kNB1; i += kSliceThreads)
    if (hist[i]) atomicAdd(&g[i], hist[i]);
}

// ---------------------------------------------------------------- (B)
__global__ __launch_bounds__(kSliceThreads) void topk_filter_kernel(
    const float* __restrict__ scores, const int* __restrict__ seq_lens,
    uint32_t* __restrict__ scratch, int slab, int K) {
  __shared__ uint32_t hist[kNB1];
  __shared__ uint32_t wave_tmp[kSliceThreads / kWave];
  __shared__ uint32_t res[2];
  const int row = blockIdx.y;
  const int len = row_len(seq_lens, row, slab);
  const int p0 = blockIdx.x * kSlice;
  if (len <= K || p0 >= len) return;
  const int t = threadIdx.x;
  uint32_t* rs = scratch + (long)row * row_scratch_words(slab);
  for (int i = t; i < kNB1; i += kSliceThreads) hist[i] = rs[kHistOff + i];
  __syncthreads();
  find_threshold(hist, kNB1, (uint32_t)K, wave_tmp, res);
  const uint32_t T1 = res[0];

  const float* s = scores + (long)row * slab;
  uint32_t* bm = rs + kBmOff;
  uint32_t* cand = rs + kBmOff + bitmap_words(slab);
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = p0 + wv * kWave; base < min(len, p0 + kSlice); base += kSliceThreads) {
    const int i = base + lane;
    const bool valid = i < len;
    const uint32_t k = valid ? rank_key(s[i]) : 0u;
    const uint32_t bin = k >> 20;
    const uint64_t gt = __ballot(valid && bin > T1);
    const uint64_t eq = __ballot(valid && bin == T1);
    if (lane == 0) {
      bm[base >> 5] = (uint32_t)gt;
      bm[(base >> 5) + 1] = (uint32_t)(gt >> 32);
    }
    if (eq) {
      uint32_t off = 0;
      if (lane == 0) off = atomicAdd(&rs[kCntOff], (uint32_t)__popcll(eq));
      off = __shfl(off, 0);
      if (valid && bin == T1) {
        const uint32_t slot = off + (uint32_t)__popcll(eq & lt_mask);
        if (slot < (uint32_t)kCandCap) {
          cand[2 * slot] = k;
          cand[2 * slot + 1] = (uint32_t)i;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- (C)
struct FinShared {
  uint32_t sel[kMaxWords];
  uint32_t tie[kMaxWords];
  uint32_t cand_key[kCandCap];
  int cand_idx[kCandCap];
  uint32_t hist[kNB1];
  uint32_t wave_tmp[kFinThreads / kWave];
  uint32_t res[2];
};

__device__ __forceinline__ void set_bit(uint32_t* bm, int i) {
  atomicOr(&bm[i >> 5], 1u << (i & 31));
}

// sel |= the `need` lowest-index set bits of tie.
__device__ void take_lowest_ties(FinShared& sh, int nw, uint32_t need) {
  const int t = threadIdx.x;
  const int per = (nw + kFinThreads - 1) / kFinThreads;
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

__global__ __launch_bounds__(kFinThreads) void topk_finalize_kernel(
    const float* __restrict__ scores, const int* __restrict__ seq_lens,
    const int* __restrict__ page_table, int pt_stride, uint32_t* __restrict__ scratch,
    int* __restrict__ out, int slab, int K, int sorted, int pad) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  FinShared& sh = *reinterpret_cast<FinShared*>(smem_raw);
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const float* s = scores + (long)row * slab;
  int* o = out + (long)row * K;
  uint32_t* rs = scratch + (long)row * row_scratch_words(slab);
  const int len = row_len(seq_lens, row, slab);
  const int nw = (len + 31) >> 5;

  if (len <= K) {
    for (int i = t; i < nw; i += kFinThreads) {
      const int rem = len - i * 32;
      sh.sel[i] = rem >= 32 ? 0xffffffffu : ((1u << rem) - 1u);
    }
    __syncthreads();
  } else {
    const uint32_t* bm = rs + kBmOff;
    const uint32_t* cand = rs + kBmOff + bitmap_words(slab);
    for (int i = t; i < nw; i += kFinThreads) { sh.sel[i] = bm[i]; sh.tie[i] = 0u; }
    for (int i = t; i < kNB1; i += kFinThreads) sh.hist[i] = rs[kHistOff + i];
    __syncthreads();
    find_threshold(sh.hist, kNB1, (uint32_t)K, sh.wave_tmp, sh.res);
    const uint32_t T1 = sh.res[0];
    const uint32_t need1 = (uint32_t)K - sh.res[1];
    const uint32_t in_bin = sh.hist[T1];
    __syncthreads();
    for (int i = t; i < kNB2; i += kFinThreads) sh.hist[i] = 0u;
    __syncthreads();

    uint32_t tstar, need3;
    if (in_bin <= (uint32_t)kCandCap) {
      const int nc = (int)in_bin;
      for (int j = t; j < nc; j += kFinThreads) {
        sh.cand_key[j] = cand[2 * j];
        sh.cand_idx[j] = (int)cand[2 * j + 1];
      }
      __syncthreads();
      for (int j = t; j < nc; j += kFinThreads) atomicAdd(&sh.hist[(sh.cand_key[j] >> 10) & 1023u], 1u);
      __syncthreads();
      find_threshold(sh.hist, kNB2, need1, sh.wave_tmp, sh.res);
      const uint32_t T2 = sh.res[0];
      const uint32_t need2 = need1 - sh.res[1];
      __syncthreads();
      for (int i = t; i < kNB2; i += kFinThreads) sh.hist[i] = 0u;
      __syncthreads();
      const uint32_t pre2 = (T1 << 10) | T2;
      for (int j = t; j < nc; j += kFinThreads) {
        const uint32_t k = sh.cand_key[j];
        if ((k >> 10) == pre2) atomicAdd(&sh.hist[k & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need2, sh.wave_tmp, sh.res);
      tstar = (pre2 << 10) | sh.res[0];
      need3 = need2 - sh.res[1];
      for (int j = t; j < nc; j += kFinThreads) {
        const uint32_t k = sh.cand_key[j];
        if (k > tstar) set_bit(sh.sel, sh.cand_idx[j]);
        else if (k == tstar) set_bit(sh.tie, sh.cand_idx[j]);
      }
      __syncthreads();
    } else {
      // candidate list overflowed: refine by re-reading the row
      for (int i = t; i < len; i += kFinThreads) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 20) == T1) atomicAdd(&sh.hist[(k >> 10) & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need1, sh.wave_tmp, sh.res);
      const uint32_t T2 = sh.res[0];
      const uint32_t need2 = need1 - sh.res[1];
      __syncthreads();
      for (int i = t; i < kNB2; i += kFinThreads) sh.hist[i] = 0u;
      __syncthreads();
      const uint32_t pre2 = (T1 << 10) | T2;
      for (int i = t; i < len; i += kFinThreads) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 10) == pre2) atomicAdd(&sh.hist[k & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need2, sh.wave_tmp, sh.res);
      tstar = (pre2 << 10) | sh.res[0];
      need3 = need2 - sh.res[1];
      for (int i = t; i < len; i += kFinThreads) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 20) != T1) continue;
        if (k > tstar) set_bit(sh.sel, i);
        else if (k == tstar) set_bit(sh.tie, i);
      }
      __syncthreads();
    }
    take_lowest_ties(sh, nw, need3);
    // re-arm the row's scratch for the next call
    for (int i = t; i < kNB1; i += kFinThreads) rs[kHistOff + i] = 0u;
    if (t == 0) rs[kCntOff] = 0u;
  }

  // ---- emit ----
  const int per = (nw + kFinThreads - 1) / kFinThreads;
  const int w0 = min(nw, t * per), w1 = min(nw, w0 + per);
  const int* pt_row = page_table ? page_table + (long)row * pt_stride : nullptr;
  if (!sorted) {
    // drop non-finite selections (they become pads), then ascending emit
    for (int i = w0; i < w1; ++i) {
      uint32_t word = sh.sel[i], keep = word;
      while (word) {
        const int b = __ffs(word) - 1;
        word &= word - 1;
        if (!key_is_finite(rank_key(s[i * 32 + b]))) keep &= ~(1u << b);
      }
      sh.sel[i] = keep;
    }
    uint32_t local = 0;
    for (int i = w0; i < w1; ++i) local += __popc(sh.sel[i]);
    uint32_t nsel;
    uint32_t pos = block_exclusive_scan(local, sh.wave_tmp, &nsel);
    for (int i = w0; i < w1; ++i) {
      uint32_t word = sh.sel[i];
      while (word) {
        const int b = __ffs(word) - 1;
        word &= word - 1;
        const int g = i * 32 + b;
        o[pos++] = pt_row ? (pt_row[g >> 6] * DSA_PAGE_TOKENS + (g & 63)) : g;
      }
    }
    for (int j = (int)nsel + t; j < K; j += kFinThreads) o[j] = pad;
    return;
  }

  // sorted: gather (key, idx) of the selection, bitonic sort (key desc, idx asc)
  uint32_t local = 0;
  for (int i = w0; i < w1; ++i) local += __popc(sh.sel[i]);
  uint32_t nsel;
  uint32_t pos = block_exclusive_scan(local, sh.wave_tmp, &nsel);
  for (int i = w0; i < w1; ++i) {
    uint32_t word = sh.sel[i];
    while (word) {
      const int b = __ffs(word) - 1;
      word &= word - 1;
      const int g = i * 32 + b;
      sh.cand_key[pos] = rank_key(s[g]);
      sh.cand_idx[pos] = g;
      ++pos;
    }
  }
  int P = 1;
  while (P < (int)nsel) P <<= 1;
  for (int j = (int)nsel + t; j < P; j += kFinThreads) {
    sh.cand_key[j] = 0u;  // below every real key (-inf is 0x007fffff)
    sh.cand_idx[j] = 0x7fffffff;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = t; i < P; i += kFinThreads) {
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
  for (int j = t; j < K; j += kFinThreads) {
    int v = pad;
    if (j < (int)nsel && key_is_finite(sh.cand_key[j])) v = sh.cand_idx[j];
    o[j] = v;
  }
}

size_t topk_scratch_bytes(int B, int slab) {
  return (size_t)B * row_scratch_words(slab) * sizeof(uint32_t);
}

hipError_t launch_topk(const float* scores, const int* seq_lens, const int* page_table,
                       int pt_stride, void* scratch, int* out, int B, int slab, int K, int sorted,
                       int pad, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)topk_finalize_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)sizeof(FinShared));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  uint32_t* sc = reinterpret_cast<uint32_t*>(scratch);
  const dim3 slices((slab + kSlice - 1) / kSlice, B);
  hipLaunchKernelGGL(topk_hist_kernel, slices, dim3(kSliceThreads), 0, s, scores, seq_lens, sc,
                     slab, K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(topk_filter_kernel, slices, dim3(kSliceThreads), 0, s, scores, seq_lens, sc,
                     slab, K);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(topk_finalize_kernel, dim3(B), dim3(kFinThreads), sizeof(FinShared), s,
                     scores, seq_lens, page_table, pt_stride, sc, out, slab, K, sorted, pad);
  return hipGetLastError();
}

}  // namespace dsa
