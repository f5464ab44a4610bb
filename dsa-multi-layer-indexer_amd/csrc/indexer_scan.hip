// Lightning-indexer scan over the paged fp8 index-K cache (gfx950).
//
//   score[b, g] = kscale[g] * sum_h w[b,h] * ReLU(q[b,h,:] . k[g,:])
//
// Semantics follow the reference's fp8 indexer: ReLU before the positive
// per-key scale, the per-head query scale folded into w
// (kernels/cuda_fused_sparse_splitk.py K:2977-2992, hp_indexer_block
// K:1677-2157; inference/modeling/kernels.py:285-312).
//
// MI355X mapping.  The work is an HBM stream of 8448-byte pages (132 B per
// key).  A wavefront owns 16-key chunks (2 KB contiguous inside a page) and
// contracts each against the resident query with one
// v_mfma_f32_16x16x128_f8f6f4 per 16 heads: the A operand is the query
// (rows = heads), B is the key chunk (columns = keys), so a whole 128-d dot
// product is one instruction and no fp8 byte passes through LDS.  Every lane
// loads 32 contiguous bytes of one key straight into its B-operand registers;
// A and B use the same lane->k assignment, so the contraction is over
// matching bytes whatever order the hardware walks k in.  The 16x16 result
// leaves each lane with one key and 4 heads: ReLU * w is summed in-lane over
// the heads it holds and across the 4 lane groups with two xor shuffles.
// Each wave keeps kScanBatch chunks (8 KB) of loads in flight.
#include <algorithm>

#include "dsa_common.h"

namespace dsa {

constexpr int kScanThreads = 256;
constexpr int kScanWaves = kScanThreads / kWave;
constexpr int kScanBatch = 4;  // 16-key chunks per wave with loads in flight
constexpr int kChunkKeys = 16;


template <int NHG, int VARIANT>
__device__ __forceinline__ v4f qk_fp8(const v8i& qa, const v8i& kb) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (VARIANT == 0) {
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa, kb, acc, 0, 0, 0, 0, 0, 0);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      long a = ((long)(uint32_t)qa[2 * j]) | ((long)(uint32_t)qa[2 * j + 1] << 32);
      long b = ((long)(uint32_t)kb[2 * j]) | ((long)(uint32_t)kb[2 * j + 1] << 32);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, acc, 0, 0, 0);
    }
  }
  return acc;
}

template <int NHG, int VARIANT>
__global__ __launch_bounds__(kScanThreads) void indexer_scan_kernel(
    const uint8_t* __restrict__ q8, const float* __restrict__ w,
    const uint8_t* __restrict__ pages, long num_pages,
    const int* __restrict__ page_table, const int* __restrict__ seq_lens,
    float* __restrict__ scores, int pt_stride, int slab_stride) {
  constexpr int kHeads = NHG * 16;
  __shared__ __align__(16) uint8_t qs[kHeads * DSA_INDEX_DIM];
  __shared__ float ws[kHeads];

  const int row = blockIdx.y;
  const int t = threadIdx.x;
  {
    const uint4* src = reinterpret_cast<const uint4*>(q8 + (long)row * kHeads * DSA_INDEX_DIM);
    for (int i = t; i < kHeads * DSA_INDEX_DIM / 16; i += kScanThreads)
      reinterpret_cast<uint4*>(qs)[i] = src[i];
    if (t < kHeads) ws[t] = w[(long)row * kHeads + t];
  }

  const int cap = min(slab_stride, pt_stride * DSA_PAGE_TOKENS);
  const int len = max(0, min(seq_lens[row], cap));
  const int nchunks = (len + kChunkKeys - 1) / kChunkKeys;
  const int nb = gridDim.x, bid = blockIdx.x;
  const int c0 = (int)((long)nchunks * bid / nb);
  const int c1 = (int)((long)nchunks * (bid + 1) / nb);
  float* srow = scores + (long)row * slab_stride;

  // Slab tail past the last scored chunk -> -inf, spread over the row's blocks.
  {
    const long tail0 = (long)nchunks * kChunkKeys;
    const long tail = (long)slab_stride - tail0;
    if (tail > 0) {
      const long p0 = tail0 + tail * bid / nb, p1 = tail0 + tail * (bid + 1) / nb;
      for (long p = p0 + t; p < p1; p += kScanThreads) srow[p] = -INFINITY;
    }
  }
  __syncthreads();

  const int lane = t & (kWave - 1);
  const int wv = wave_id();
  const int kr = lane & 15;  // key (B column) / head (A row) of this lane
  const int kc = lane >> 4;  // 32-byte k chunk of this lane

  v8i qa[NHG];
  float wr[NHG][4];
#pragma unroll
  for (int hg = 0; hg < NHG; ++hg) {
    const uint4* p = reinterpret_cast<const uint4*>(qs + (hg * 16 + kr) * DSA_INDEX_DIM + kc * 32);
    const uint4 a = p[0], b = p[1];
    qa[hg] = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) wr[hg][r] = ws[hg * 16 + 4 * kc + r];
  }

  // Waves take contiguous sub-ranges of the block's chunks.
  const int n = c1 - c0;
  const int w0 = c0 + (int)((long)n * wv / kScanWaves);
  const int w1 = c0 + (int)((long)n * (wv + 1) / kScanWaves);
  const int* pt_row = page_table + (long)row * pt_stride;

  for (int cb = w0; cb < w1; cb += kScanBatch) {
    uint4 kv[kScanBatch][2];
    float ksc[kScanBatch];
    bool ok[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      const int c = cb + i;
      ok[i] = false;
      kv[i][0] = kv[i][1] = make_uint4(0, 0, 0, 0);
      ksc[i] = 0.f;
      if (c < w1) {
        const int page = pt_row[c >> 2];
        if (page >= 0 && (long)page < num_pages) {
          ok[i] = true;
          const uint8_t* base = pages + (long)page * DSA_INDEX_PAGE_BYTES;
          const uint4* kp = reinterpret_cast<const uint4*>(
              base + (c & 3) * (kChunkKeys * DSA_INDEX_DIM) + kr * DSA_INDEX_DIM + kc * 32);
          kv[i][0] = kp[0];
          kv[i][1] = kp[1];
          ksc[i] = reinterpret_cast<const float*>(base + DSA_PAGE_TOKENS * DSA_INDEX_DIM)[(c & 3) * kChunkKeys + kr];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      const int c = cb + i;
      if (c >= w1) break;
      float acc = 0.f;
      if (ok[i]) {
        const v8i kb = v8i{(int)kv[i][0].x, (int)kv[i][0].y, (int)kv[i][0].z, (int)kv[i][0].w,
                           (int)kv[i][1].x, (int)kv[i][1].y, (int)kv[i][1].z, (int)kv[i][1].w};
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
          const v4f d = qk_fp8<NHG, VARIANT>(qa[hg], kb);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc += wr[hg][r] * fmaxf(d[r], 0.f);
        }
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
      }
      const int g = c * kChunkKeys + kr;
      if (lane < 16 && g < slab_stride) srow[g] = (ok[i] && g < len) ? acc * ksc[i] : -INFINITY;
    }
  }
}

template <int NHG, int VARIANT>
static hipError_t launch_scan_t(dim3 grid, hipStream_t s, const uint8_t* q8, const float* w,
                                const uint8_t* pages, long num_pages, const int* pt,
                                const int* seq_lens, float* scores, int pt_stride, int slab_stride) {
  hipLaunchKernelGGL((indexer_scan_kernel<NHG, VARIANT>), grid, dim3(kScanThreads), 0, s, q8, w,
                     pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
  return hipGetLastError();
}

static int g_host_scan_variant = 0;

void set_scan_variant(int v) { g_host_scan_variant = v ? 1 : 0; }

int scan_blocks_per_row(int B, int pt_stride, int slab_stride) {
  // ~512 blocks of 4 waves in total (2 per CU), never more than one block
  // per 4 chunks of the row's capacity.
  const long cap = std::min((long)slab_stride, (long)pt_stride * DSA_PAGE_TOKENS);
  const long cap_chunks = (cap + kChunkKeys - 1) / kChunkKeys;
  long per_row = (512 + B - 1) / B;
  per_row = std::min(per_row, std::max(1L, cap_chunks / kScanWaves));
  return (int)std::max(1L, per_row);
}

hipError_t launch_indexer_scan(const uint8_t* q8, const float* w, const uint8_t* pages,
                               long num_pages, const int* pt, const int* seq_lens, float* scores,
                               int B, int Hidx, int pt_stride, int slab_stride, hipStream_t s) {
  const dim3 grid(scan_blocks_per_row(B, pt_stride, slab_stride), B);
  const int nhg = Hidx / 16;
  if (g_host_scan_variant == 0) {
    switch (nhg) {
      case 1: return launch_scan_t<1, 0>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
      case 2: return launch_scan_t<2, 0>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
      case 3: return launch_scan_t<3, 0>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
      default: return launch_scan_t<4, 0>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
    }
  }
  switch (nhg) {
    case 1: return launch_scan_t<1, 1>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
    case 2: return launch_scan_t<2, 1>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
    case 3: return launch_scan_t<3, 1>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
    default: return launch_scan_t<4, 1>(grid, s, q8, w, pages, num_pages, pt, seq_lens, scores, pt_stride, slab_stride);
  }
}

}  // namespace dsa
