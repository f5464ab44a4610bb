// Plain indexer scan over every row's chunks as ONE index space (gfx950).
//
// The plain scan (scores only: no histogram, no select; the first launch of
// a large-batch layer and dsa_indexer_scan) computes, per token g of row b
// (reference hp_indexer_block K:1677-2157, fp8 semantics K:2990-2992):
//   score[b,g] = kscale[g] * sum_h w[b,h] * ReLU(q[b,h,:] . k[g,:]),
// -inf for g in [len_b, slab_stride).  The arithmetic per 4-chunk group is
// the decode launch's scan role (scan_block), in the same order, so the
// scores are the same bits.
//
// Work layout.  Row b's positions are cut into batches of 64 tokens (one
// index-K page, 4 chunks of 16 keys; the last batch of a row is partly
// past len_b).  The batches of all rows, row after row, form one index
// space; workgroup w (512 threads, one per CU: its LDS) takes the w-th
// equal share of it, and its 8 waves take the batches of that share one at
// a time from an LDS counter, each keeping its next batch's loads in flight
// while it scores the current one.  Measured on the per-row form (two
// 8-wave workgroups per CU, each over a fixed range of one row): on every
// CU the workgroup dispatched first ended ~15 us before the second (C4:
// medians 55 and 70.6 us; the SIMDs issue for the older waves first, and a
// 16-wave form of this kernel without the second buffer showed waves 12-15
// taking 2 batches to waves 0-3's 16).  Here a slower wave takes fewer
// batches, the waves of a workgroup end within ~0.3 us, and the
// workgroups' shares are equal to within one batch.
//
// The workgroup prefetches its batches' page entries into LDS; a wave
// reloads its query operand and head weights from memory when its next
// batch is in another row (takes increase, so each wave meets each row of
// its share at most once).  The -inf tails [64 * batches_b, slab) are one
// more index space, also cut in equal shares, written after the scores.

namespace dsa {

constexpr int kFlatThreads = 512;
constexpr int kFlatWaves = kFlatThreads / kWave;
constexpr int kFlatMaxRows = kFlatScanMaxRows;  // rows whose prefixes a workgroup holds
constexpr int kFlatMaxPages = 4096;  // batches (page entries) of one share
constexpr int kFlatBufBatches = 256;  // shares of at most this many batches stage their scores in LDS

struct FlatShared {
  int bpre[kFlatMaxRows + 1];  // row b's batches: [bpre[b], bpre[b + 1])
  int tpre[kFlatMaxRows + 1];  // row b's tail positions in the tail space
  int lens[kFlatMaxRows];
  int pts[kFlatMaxPages];      // page entry of each batch of the share
  uint32_t wsum[2][kFlatWaves];
  uint32_t next;               // next batch of the share to take
  float sbuf[kFlatBufBatches * DSA_PAGE_TOKENS];  // the share's scores, written out at the end
};

static_assert(sizeof(FlatShared) <= 160 * 1024, "the flat scan's LDS fits one CU");
static size_t lds_flat_max() { return std::max(sizeof(FlatShared), sizeof(AttnShared)); }

// largest r in [0, n) with pre[r] <= v (pre[0] == 0 <= v)
__device__ __forceinline__ int flat_row_of(const int* pre, int n, int v) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= v) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// ATTN: workgroups [0, n_att) run the attention role (A.nsplit splits per
// (row, head group), merged as in the decode launch) over a selection this
// launch does not produce, beside the scan on the other CUs (one workgroup
// per CU each: the LDS), so that the attention's gather and the scan's
// stream share the launch instead of following each other.  Attention
// workgroups come first in the grid, so a (row, head group)'s splits are
// resident together (their merge waits for each other); the scan's never
// wait.
template <int NHG, int VARIANT, bool ATTN>
__global__ void __launch_bounds__(kFlatThreads) flat_scan_kernel(const AttnArgs A, int n_att, const ScanArgs S,
                                                                 int B) {
  constexpr int kHeads = NHG * 16;
  extern __shared__ __align__(16) unsigned char smem[];
  if constexpr (ATTN) {
    if ((int)blockIdx.x < n_att) {
      dbg_begin();
      const int nhg = A.H / kHG;
      const int bid = blockIdx.x;
      attention_block<false>(A, bid / (A.nsplit * nhg), (bid / A.nsplit) % nhg, bid % A.nsplit, smem);
      dbg_flush(blockIdx.x);
      return;
    }
  }
  FlatShared& fs = *reinterpret_cast<FlatShared*>(smem);
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  const int kr = lane & 15, kc = lane >> 4;
  const int cap = min(S.slab_stride, S.pt_stride * DSA_PAGE_TOKENS);
  if constexpr (kPhaseStamps) {
    dbg_begin();
    __syncthreads();
  }
  dbg_stamp(0, 0);
  dbg_hw_ids();

  // ---- prefixes over the rows: batches and -inf tail positions; thread
  // t takes rows [kRowsPer * t, kRowsPer * t + kRowsPer) ----
  {
    constexpr int kRowsPer = kFlatMaxRows / kFlatThreads;
    static_assert(kRowsPer * kFlatThreads == kFlatMaxRows, "rows per thread");
    int nbat[kRowsPer], ntail[kRowsPer];
    uint32_t sb = 0, st = 0;
#pragma unroll
    for (int k = 0; k < kRowsPer; ++k) {
      const int row = kRowsPer * t + k;
      int len = 0;
      nbat[k] = ntail[k] = 0;
      if (row < B) {
        len = max(0, min(S.seq_lens[row], cap));
        nbat[k] = (len + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS;
        ntail[k] = S.slab_stride - min(nbat[k] * DSA_PAGE_TOKENS, S.slab_stride);
        fs.lens[row] = len;
      }
      sb += (uint32_t)nbat[k];
      st += (uint32_t)ntail[k];
    }
    const uint32_t ib = wave_scan_incl<0>(sb), it = wave_scan_incl<0>(st);
    if (lane == kWave - 1) {
      fs.wsum[0][wv] = ib;
      fs.wsum[1][wv] = it;
    }
    if (t == 0) {
      fs.bpre[0] = 0;
      fs.tpre[0] = 0;
      fs.next = 0u;
    }
    __syncthreads();
    uint32_t ob = ib - sb, ot = it - st;  // exclusive: the rows before this thread's
#pragma unroll
    for (int w2 = 0; w2 < kFlatWaves; ++w2) {
      ob += w2 < wv ? fs.wsum[0][w2] : 0u;
      ot += w2 < wv ? fs.wsum[1][w2] : 0u;
    }
#pragma unroll
    for (int k = 0; k < kRowsPer; ++k) {
      const int row = kRowsPer * t + k;
      ob += (uint32_t)nbat[k];
      ot += (uint32_t)ntail[k];
      if (row < B) {
        fs.bpre[row + 1] = (int)ob;
        fs.tpre[row + 1] = (int)ot;
      }
    }
    __syncthreads();
  }
  const int nwg = (int)gridDim.x - n_att, w = (int)blockIdx.x - n_att;
  const int NB = fs.bpre[B], NT = fs.tpre[B];
  const int b0 = (int)((long)NB * w / nwg), nr = (int)((long)NB * (w + 1) / nwg) - b0;

  // ---- the share's page entries (a row at a time: consecutive batches) ----
  if (nr > 0) {
    int r = flat_row_of(fs.bpre, B, b0);
    for (int i = t; i < nr; i += kFlatThreads) {
      const int b = b0 + i;
      while (fs.bpre[r + 1] <= b) ++r;
      fs.pts[i] = S.page_table[(long)r * S.pt_stride + (b - fs.bpre[r])];
    }
  }
  __syncthreads();
  dbg_stamp(0, 1);
  // Scores interleaved with the key stream as 256-byte stores cost C4's
  // scan ~13% (79 against 69 us with the stores left out; non-temporal
  // stores: the same 79): a share that fits the LDS buffer keeps its scores
  // there and writes them out at the end as 16-byte stores of contiguous
  // runs (C4's scan 79.0 -> 74.6 us).  Those end-of-launch stores, and the
  // -inf tails after them, are non-temporal: written as ordinary stores
  // they sat dirty in the L2s, whose write-back the launch's end then
  // waited for (C4's scan 75.6 -> 72.0 us, its layer ~109 -> ~104 us).
  const bool staged = nr <= kFlatBufBatches;
  // rows start on 16-byte boundaries: the staged runs go out as 16-byte stores
  const bool vec = S.slab_stride % 4 == 0 && ((uintptr_t)S.scores & 15) == 0;

  // ---- the waves take the share's batches; each wave keeps the next
  // batch's loads in flight while it scores the current one ----
  const auto take = [&]() -> int {
    uint32_t i = 0;
    if (lane == 0) i = atomicAdd(&fs.next, 1u);
    return __builtin_amdgcn_readfirstlane((int)i);
  };
  struct Batch {
    uint4 kv[4][2];
    float ksc;
    int i, r, c0;
    bool pok;
  };
  int rrow = nr > 0 ? flat_row_of(fs.bpre, B, b0) : 0;  // row of the last batch issued (takes increase)
  // issue batch i's loads: 8 key loads (4 chunks) and the lane's key scale
  const auto issue = [&](int i, Batch& x) {
    const int b = b0 + i;
    while (fs.bpre[rrow + 1] <= b) ++rrow;  // uniform
    x.i = i;
    x.r = rrow;
    x.c0 = (b - fs.bpre[rrow]) * 4;  // the batch's first chunk in the row
    const int nck = (fs.lens[rrow] + kChunkKeys - 1) / kChunkKeys;
    const int pg = __builtin_amdgcn_readfirstlane(fs.pts[i]);
    x.pok = pg >= 0 && (long)pg < S.num_pages;
    // one resource over the page (empty for an invalid page: its loads
    // return 0); a chunk past the row's last reads past the resource
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(S.pages) + (x.pok ? (long)pg * DSA_INDEX_PAGE_BYTES : 0L), (short)0,
        x.pok ? DSA_INDEX_PAGE_BYTES : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = x.c0 + j < nck ? j * (kChunkKeys * DSA_INDEX_DIM) + kr * DSA_INDEX_DIM + kc * 32
                                     : DSA_INDEX_PAGE_BYTES;
      x.kv[j][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      x.kv[j][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0));
    }
    // lane (j, kr): key kr's scale of chunk j
    x.ksc = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rs, DSA_PAGE_TOKENS * DSA_INDEX_DIM + 4 * lane, 0, 0));
  };
  int qrow = -1;
  v8i qa[NHG];
  float wr[NHG][4];
  int nbatch = 0;
  // score batch x: the scan role's group arithmetic (scan_block), in the
  // same order -- ReLU*w summed over each lane's heads per chunk, then the
  // 4 chunks transpose-reduced by lane swaps so that lane (j, kr) holds key
  // kr of chunk j
  const auto score = [&](const Batch& x) {
    ++nbatch;
    if (x.r != qrow) {  // uniform: the query operand and weights of row x.r
      const uint8_t* qs = S.q8 + (long)x.r * kHeads * DSA_INDEX_DIM;
#pragma unroll
      for (int hg = 0; hg < NHG; ++hg) {
        const uint4* p = reinterpret_cast<const uint4*>(qs + (hg * 16 + kr) * DSA_INDEX_DIM + kc * 32);
        const uint4 a = p[0], bq = p[1];
        qa[hg] = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)bq.x, (int)bq.y, (int)bq.z, (int)bq.w};
        const float4 w4 = *reinterpret_cast<const float4*>(S.w + (long)x.r * kHeads + hg * 16 + 4 * kc);
        wr[hg][0] = w4.x;
        wr[hg][1] = w4.y;
        wr[hg][2] = w4.z;
        wr[hg][3] = w4.w;
      }
      qrow = x.r;
    }
    const int len = fs.lens[x.r];
    const int nck = (len + kChunkKeys - 1) / kChunkKeys;
    float a[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v8i kb = v8i{(int)x.kv[j][0].x, (int)x.kv[j][0].y, (int)x.kv[j][0].z, (int)x.kv[j][0].w,
                         (int)x.kv[j][1].x, (int)x.kv[j][1].y, (int)x.kv[j][1].z, (int)x.kv[j][1].w};
      a[j] = 0.f;
      if (x.c0 + j >= nck) continue;  // uniform: past the row's chunks
#pragma unroll
      for (int hg = 0; hg < NHG; ++hg) {
        const v4f d = qk_fp8<VARIANT>(qa[hg], kb);
#pragma unroll
        for (int q = 0; q < 4; ++q) a[j] += wr[hg][q] * __int_as_float(max(__float_as_int(d[q]), 0));
      }
    }
    const auto add32 = [](float u, float v) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(v), false, false);
      return __uint_as_float(p[0]) + __uint_as_float(p[1]);
    };
    const float xs = add32(a[0], a[2]);
    const float ys = add32(a[1], a[3]);
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(xs), __float_as_uint(ys), false, false);
    const float acc = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const int g = (x.c0 + kc) * kChunkKeys + kr;  // == the batch's first position + lane
    const float v = (x.pok && g < len) ? acc * x.ksc : -INFINITY;
    if (staged) fs.sbuf[x.i * DSA_PAGE_TOKENS + lane] = v;
    else if (g < S.slab_stride) S.scores[(long)x.r * S.slab_stride + g] = v;
  };
  // ping-pong over two batches' registers
  Batch X0, X1;
  int i = take();
  if (i < nr) issue(i, X0);
  while (i < nr) {
    const int j = take();
    if (j < nr) issue(j, X1);
    score(X0);
    if (j >= nr) break;
    i = take();
    if (i < nr) issue(i, X0);
    score(X1);
  }

  // ---- the staged scores, a row's run at a time ----
  if (staged && nr > 0) {
    __syncthreads();
    dbg_stamp(0, 2);
    for (int r = flat_row_of(fs.bpre, B, b0); r < B && fs.bpre[r] < b0 + nr; ++r) {
      const int bs = max(b0, fs.bpre[r]), be = min(b0 + nr, fs.bpre[r + 1]);
      const int p0 = (bs - fs.bpre[r]) * DSA_PAGE_TOKENS;
      const int p1 = min((be - fs.bpre[r]) * DSA_PAGE_TOKENS, S.slab_stride);
      const float* src = fs.sbuf + (bs - b0) * DSA_PAGE_TOKENS - p0;
      float* dst = S.scores + (long)r * S.slab_stride;
      if (vec) {  // 16-byte stores (p0, p1 and the row start are multiples of 4)
        for (int p = p0 + 4 * t; p < p1; p += 4 * kFlatThreads)
          __builtin_nontemporal_store(*reinterpret_cast<const v4f*>(src + p), reinterpret_cast<v4f*>(dst + p));
      } else {
        for (int p = p0 + t; p < p1; p += kFlatThreads) __builtin_nontemporal_store(src[p], dst + p);
      }
    }
  }

  dbg_stamp(0, 3);
  // ---- this workgroup's share of the -inf tails ----
  {
    const int t0 = (int)((long)NT * w / nwg), t1 = (int)((long)NT * (w + 1) / nwg);
    if (t0 < t1) {
      for (int r = flat_row_of(fs.tpre, B, t0); r < B && fs.tpre[r] < t1; ++r) {
        const int s0 = max(t0, fs.tpre[r]), s1 = min(t1, fs.tpre[r + 1]);
        const int base = min((fs.bpre[r + 1] - fs.bpre[r]) * DSA_PAGE_TOKENS, S.slab_stride) - fs.tpre[r];
        float* srow = S.scores + (long)r * S.slab_stride + base;
        for (int p = s0 + t; p < s1; p += kFlatThreads) __builtin_nontemporal_store(-INFINITY, srow + p);
      }
    }
  }
  dbg_stamp(0, 4);
  dbg_stamp_lane0(16 + wv);
  dbg_value_lane0(32 + wv, (unsigned long long)nbatch);
  dbg_flush(blockIdx.x);
}

template <int NHG, bool ATTN>
static hipError_t launch_flat(dim3 grid, size_t lds, hipStream_t s, const AttnArgs& A, int n_att, const ScanArgs& S,
                              int B) {
  static PerDeviceOnce attr;
  const hipError_t e = attr.run([] {
    hipError_t r = hipFuncSetAttribute((const void*)flat_scan_kernel<NHG, 0, ATTN>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_flat_max());
    if (r == hipSuccess)
      r = hipFuncSetAttribute((const void*)flat_scan_kernel<NHG, 1, ATTN>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_flat_max());
    return r;
  });
  if (e != hipSuccess) return e;
  if (g_scan_variant == 0)
    hipLaunchKernelGGL((flat_scan_kernel<NHG, 0, ATTN>), grid, dim3(kFlatThreads), lds, s, A, n_att, S, B);
  else
    hipLaunchKernelGGL((flat_scan_kernel<NHG, 1, ATTN>), grid, dim3(kFlatThreads), lds, s, A, n_att, S, B);
  return hipGetLastError();
}

// Whether B rows fit the flat scan's index spaces (batches and tail
// positions counted in 32-bit ints, row prefixes held in LDS).
bool flat_scan_fits(const ScanArgs& S, int B) {
  const long cap = std::min((long)S.slab_stride, (long)S.pt_stride * DSA_PAGE_TOKENS);
  const long max_batches = (long)B * ((cap + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS);
  return B >= 1 && B <= kFlatMaxRows && max_batches < (1L << 31) && (long)B * S.slab_stride < (1L << 31);
}

// Plain scan launch: one 512-thread workgroup per CU the attention leaves
// (more when a share would exceed the LDS page table); with A, the
// attention of B_att rows (A->nsplit splits per row and head group) in the
// same grid first.
hipError_t launch_flat_scan(const AttnArgs* A, int B_att, const ScanArgs& S, int B, hipStream_t s) {
  if (!flat_scan_fits(S, B)) return hipErrorInvalidValue;
  const long cap = std::min((long)S.slab_stride, (long)S.pt_stride * DSA_PAGE_TOKENS);
  const long max_batches = (long)B * ((cap + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS);
  const int n_att = A ? B_att * (A->H / kHG) * A->nsplit : 0;
  const int nwg = (int)std::max<long>(std::max(device_cus() - n_att, device_cus() / 2),
                                      (max_batches + kFlatMaxPages - 1) / kFlatMaxPages);
  const dim3 grid(n_att + nwg);
  const size_t lds = A ? lds_flat_max() : sizeof(FlatShared);
  const AttnArgs a = A ? *A : AttnArgs{};
  switch (S.Hidx / 16) {
    case 1: return A ? launch_flat<1, true>(grid, lds, s, a, n_att, S, B) : launch_flat<1, false>(grid, lds, s, a, 0, S, B);
    case 2: return A ? launch_flat<2, true>(grid, lds, s, a, n_att, S, B) : launch_flat<2, false>(grid, lds, s, a, 0, S, B);
    case 3: return A ? launch_flat<3, true>(grid, lds, s, a, n_att, S, B) : launch_flat<3, false>(grid, lds, s, a, 0, S, B);
    default: return A ? launch_flat<4, true>(grid, lds, s, a, n_att, S, B) : launch_flat<4, false>(grid, lds, s, a, 0, S, B);
  }
}

}  // namespace dsa
