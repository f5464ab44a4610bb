// Exact top-k select over a row of fp32 scores (gfx950), one 1024-thread
// workgroup per row.
//
// Ranking: rank_key() order (score descending, -0.0 == +0.0, NaN above +inf);
// ties at the threshold go to the lower index.  That is the reference's
// select_topk (attention_core.py:66-91: torch.topk + non-finite -> sentinel)
// with its unspecified tie order pinned to "lower index wins", and the
// radix-select structure of the GPU selectors (tilelang_dsa/topk_selector.py
// 36-194, K:1097-1129, K:1248-1310): a 12-bit histogram over the high key
// bits finds the threshold bin, two 10-bit refinements over the bin's
// candidates find the exact threshold key t*, every key > t* is selected and
// the lowest-index keys == t* fill the rest.
//
// Membership is kept as two LDS bitmaps over the row (selected / tied), so
// the tie rule and the position-ordered emit are prefix popcounts, with no
// ordering atomics anywhere: the output is deterministic.  Bin candidates go
// to LDS when the threshold bin holds <= kCandCap keys; otherwise the
// refinement re-reads the row (exact either way).
#include <algorithm>

#include "dsa_common.h"

namespace dsa {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / kWave;
constexpr int kNB1 = 4096;   // first digit: key bits [31:20]
constexpr int kNB2 = 1024;   // second / third digits: bits [19:10], [9:0]
constexpr int kCandCap = 4096;
constexpr int kMaxWords = DSA_TOPK_MAX_CTX / 32;
constexpr int kSortMax = 4096;

struct TopkShared {
  uint32_t hist[kNB1];
  uint32_t sel[kMaxWords];
  uint32_t tie[kMaxWords];
  uint32_t cand_key[kCandCap];
  int cand_idx[kCandCap];
  uint32_t wave_tmp[kTkWaves];
  uint32_t misc[8];
};

// Exclusive prefix sum over the block (thread order); *total gets the sum.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tmp, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  uint32_t inc = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t n = __shfl_up(inc, o);
    if (lane >= o) inc += n;
  }
  if (lane == kWave - 1) wave_tmp[wv] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kTkWaves; ++i) {
    const uint32_t x = wave_tmp[i];
    before += (i < wv) ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + inc - v;
}

// Largest bin T with sum_{b >= T} hist[b] >= need (need >= 1, and the total
// is >= need).  Writes T to misc[0] and the count strictly above T to misc[1].
__device__ void find_threshold(const uint32_t* hist, int nbins, uint32_t need, TopkShared& sh) {
  const int per = nbins / kTkThreads;  // 4 or 1
  const int t = threadIdx.x;
  // thread t owns bins [hi - per, hi), counted from the top
  const int hi = nbins - t * per;
  uint32_t local = 0;
  for (int i = 1; i <= per; ++i) local += hist[hi - i];
  uint32_t total;
  const uint32_t above = block_exclusive_scan(local, sh.wave_tmp, &total);
  uint32_t acc = above;
  for (int i = 1; i <= per; ++i) {
    const uint32_t h = hist[hi - i];
    if (acc < need && acc + h >= need) {
      sh.misc[0] = (uint32_t)(hi - i);
      sh.misc[1] = acc;
    }
    acc += h;
  }
  __syncthreads();
}

__device__ __forceinline__ void set_bit(uint32_t* bm, int i) {
  atomicOr(&bm[i >> 5], 1u << (i & 31));
}

// sel |= the `need` lowest-index set bits of tie.
__device__ void take_lowest_ties(TopkShared& sh, int nw, uint32_t need) {
  const int t = threadIdx.x;
  const int per = (nw + kTkThreads - 1) / kTkThreads;
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

__global__ __launch_bounds__(kTkThreads) void topk_kernel(
    const float* __restrict__ scores, const int* __restrict__ seq_lens,
    const int* __restrict__ page_table, int pt_stride, int* __restrict__ out, int slab_stride,
    int K, int sorted, int pad) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  TopkShared& sh = *reinterpret_cast<TopkShared*>(smem_raw);
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const float* s = scores + (long)row * slab_stride;
  int* o = out + (long)row * K;
  const int len = max(0, min(seq_lens[row], slab_stride));
  const int nw = (len + 31) >> 5;

  for (int i = t; i < nw; i += kTkThreads) { sh.sel[i] = 0u; sh.tie[i] = 0u; }
  for (int i = t; i < kNB1; i += kTkThreads) sh.hist[i] = 0u;
  if (t < 8) sh.misc[t] = 0u;
  __syncthreads();

  if (len <= K) {
    for (int i = t; i < nw; i += kTkThreads) {
      const int rem = len - i * 32;
      sh.sel[i] = rem >= 32 ? 0xffffffffu : ((1u << rem) - 1u);
    }
    __syncthreads();
  } else {
    for (int i = t; i < len; i += kTkThreads) atomicAdd(&sh.hist[rank_key(s[i]) >> 20], 1u);
    __syncthreads();
    find_threshold(sh.hist, kNB1, (uint32_t)K, sh);
    const uint32_t T1 = sh.misc[0];
    const uint32_t need1 = (uint32_t)K - sh.misc[1];
    const uint32_t in_bin = sh.hist[T1];
    __syncthreads();
    for (int i = t; i < kNB1; i += kTkThreads) sh.hist[i] = 0u;
    if (t == 0) sh.misc[2] = 0u;
    __syncthreads();

    uint32_t tstar, need3;
    if (in_bin <= (uint32_t)kCandCap) {
      // keys above the bin are selected now; the bin's keys become candidates
      for (int i = t; i < len; i += kTkThreads) {
        const uint32_t k = rank_key(s[i]);
        const uint32_t b = k >> 20;
        if (b > T1) {
          set_bit(sh.sel, i);
        } else if (b == T1) {
          const uint32_t slot = atomicAdd(&sh.misc[2], 1u);
          sh.cand_key[slot] = k;
          sh.cand_idx[slot] = i;
        }
      }
      __syncthreads();
      const int nc = (int)sh.misc[2];
      for (int j = t; j < nc; j += kTkThreads) atomicAdd(&sh.hist[(sh.cand_key[j] >> 10) & 1023u], 1u);
      __syncthreads();
      find_threshold(sh.hist, kNB2, need1, sh);
      const uint32_t T2 = sh.misc[0];
      const uint32_t need2 = need1 - sh.misc[1];
      __syncthreads();
      for (int i = t; i < kNB2; i += kTkThreads) sh.hist[i] = 0u;
      __syncthreads();
      const uint32_t pre2 = (T1 << 10) | T2;
      for (int j = t; j < nc; j += kTkThreads) {
        const uint32_t k = sh.cand_key[j];
        if ((k >> 10) == pre2) atomicAdd(&sh.hist[k & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need2, sh);
      tstar = (pre2 << 10) | sh.misc[0];
      need3 = need2 - sh.misc[1];
      for (int j = t; j < nc; j += kTkThreads) {
        const uint32_t k = sh.cand_key[j];
        if (k > tstar) set_bit(sh.sel, sh.cand_idx[j]);
        else if (k == tstar) set_bit(sh.tie, sh.cand_idx[j]);
      }
      __syncthreads();
    } else {
      // threshold bin too large for LDS: refine by re-reading the row
      for (int i = t; i < len; i += kTkThreads) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 20) == T1) atomicAdd(&sh.hist[(k >> 10) & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need1, sh);
      const uint32_t T2 = sh.misc[0];
      const uint32_t need2 = need1 - sh.misc[1];
      __syncthreads();
      for (int i = t; i < kNB2; i += kTkThreads) sh.hist[i] = 0u;
      __syncthreads();
      const uint32_t pre2 = (T1 << 10) | T2;
      for (int i = t; i < len; i += kTkThreads) {
        const uint32_t k = rank_key(s[i]);
        if ((k >> 10) == pre2) atomicAdd(&sh.hist[k & 1023u], 1u);
      }
      __syncthreads();
      find_threshold(sh.hist, kNB2, need2, sh);
      tstar = (pre2 << 10) | sh.misc[0];
      need3 = need2 - sh.misc[1];
      for (int i = t; i < len; i += kTkThreads) {
        const uint32_t k = rank_key(s[i]);
        if (k > tstar) set_bit(sh.sel, i);
        else if (k == tstar) set_bit(sh.tie, i);
      }
      __syncthreads();
    }
    take_lowest_ties(sh, nw, need3);
  }

  // ---- emit ----
  const int per = (nw + kTkThreads - 1) / kTkThreads;
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
    for (int j = (int)nsel + t; j < K; j += kTkThreads) o[j] = pad;
    return;
  }

  // sorted: gather (key, idx), bitonic sort by (key desc, idx asc)
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
  for (int j = (int)nsel + t; j < P; j += kTkThreads) {
    sh.cand_key[j] = 0u;  // below every real key (-inf is 0x007fffff)
    sh.cand_idx[j] = 0x7fffffff;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = t; i < P; i += kTkThreads) {
        const int p = i ^ j;
        if (p > i) {
          const uint32_t ka = sh.cand_key[i], kb = sh.cand_key[p];
          const int ia = sh.cand_idx[i], ib = sh.cand_idx[p];
          // "a first" in the final order
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
  for (int j = t; j < K; j += kTkThreads) {
    int v = pad;
    if (j < (int)nsel && key_is_finite(sh.cand_key[j])) v = sh.cand_idx[j];
    o[j] = v;
  }
}

size_t topk_shared_bytes() { return sizeof(TopkShared); }

hipError_t launch_topk(const float* scores, const int* seq_lens, const int* page_table,
                       int pt_stride, int* out, int B, int slab_stride, int K, int sorted,
                       int pad, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)topk_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)sizeof(TopkShared));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(topk_kernel, dim3(B), dim3(kTkThreads), sizeof(TopkShared), s, scores,
                     seq_lens, page_table, pt_stride, out, slab_stride, K, sorted, pad);
  return hipGetLastError();
}

}  // namespace dsa
