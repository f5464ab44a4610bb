// Split-K sparse MLA decode over the fp8 656-byte latent pool (gfx950).
//
//   out[b,h,:] = sum_j softmax_j(sm * q[b,h,:] . kv_j) * kv_j[:512]
//
// kv_j is the dequantised latent row of KV slot idx[b,j]:
// bf16_rn(f32(e4m3) * scale[d/128]) for the 512 latent dims and the stored
// bf16 rope for the last 64 (reference hp_dequant4 K:1181-1197, gather
// K:1355-1395; CPU semantics attention_core.py:94-146, ref_sparse_mla
// K:2950-2966).  The value is the first 512 dims of the same row.
//
// MI355X mapping.  Workgroup (split, head-group, row) of 4 waves handles
// 64-key tiles of its slice of idx[b, :topk].  Each wave owns 16 keys; lane
// (kr, kc) gathers key kr's bytes [128kc, 128kc+128) + scale kc + rope
// [16kc, 16kc+16) straight from HBM into registers (4 lanes per 656-byte row,
// each reading a contiguous run), dequantises them and feeds them as the B
// operand of v_mfma_f32_16x16x32_bf16 with the 16 heads as A, so QK needs no
// LDS staging.  Q and K use the same lane->k assignment (kc selects which
// 8-element piece of the 576 dims a lane carries at each of 18 steps), so the
// contraction is exact over the 576 dims.  The value tile goes to LDS
// transposed ([dim][key]) for the PV MFMA, softmax runs in the exp2 domain,
// and each split writes (O, m, l) partials that a second kernel merges with
// log-sum-exp weights (combine_kernel K:996-1045).
#include <algorithm>

#include "dsa_common.h"

namespace dsa {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kTile = 16 * kAttnWaves;  // 64 keys per tile
constexpr int kVtLd = kTile + 8;        // Vt row stride (bf16 elements)
constexpr int kPLd = kTile + 8;         // P row stride (bf16 elements)
constexpr int kHeadsPerGroup = 16;

__device__ __forceinline__ v4f mfma_bf16(const uint4& a, const uint4& b, v4f c) {
  v8bf av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
}

// 16 e4m3 (one uint4) * scale -> 16 bf16 (two uint4: elements 0-7, 8-15)
__device__ __forceinline__ void dequant16(const uint4& v, float sc, uint4& lo, uint4& hi) {
  float f[16];
  e4m3x4_to_f32(v.x, f + 0);
  e4m3x4_to_f32(v.y, f + 4);
  e4m3x4_to_f32(v.z, f + 8);
  e4m3x4_to_f32(v.w, f + 12);
  lo.x = pack_bf16x2(f[0] * sc, f[1] * sc);
  lo.y = pack_bf16x2(f[2] * sc, f[3] * sc);
  lo.z = pack_bf16x2(f[4] * sc, f[5] * sc);
  lo.w = pack_bf16x2(f[6] * sc, f[7] * sc);
  hi.x = pack_bf16x2(f[8] * sc, f[9] * sc);
  hi.y = pack_bf16x2(f[10] * sc, f[11] * sc);
  hi.z = pack_bf16x2(f[12] * sc, f[13] * sc);
  hi.w = pack_bf16x2(f[14] * sc, f[15] * sc);
}

struct AttnShared {
  uint16_t vt[DSA_LATENT_DIM * kVtLd];      // value tile, [dim][key]
  float s[kHeadsPerGroup * kTile];           // scores (log2 domain)
  uint16_t p[kHeadsPerGroup * kPLd];         // probabilities, bf16
  float m[kHeadsPerGroup], l[kHeadsPerGroup], alpha[kHeadsPerGroup];
};

__global__ __launch_bounds__(kAttnThreads) void sparse_mla_split_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ pool, long kv_rows,
    const int* __restrict__ idx, float* __restrict__ part_o, float* __restrict__ part_ml,
    int H, int topk, int nsplit, float sm_log2) {
  __shared__ AttnShared sh;
  const int sp = blockIdx.x, hg = blockIdx.y, b = blockIdx.z;
  const int nhg = gridDim.y;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = wave_id();
  const int kr = lane & 15, kc = lane >> 4;

  const int kps = (topk + nsplit - 1) / nsplit;
  const int k0 = min(topk, sp * kps), k1 = min(topk, k0 + kps);

  // Q (A operand): steps 0..15 -> dims 128kc + 8s, steps 16,17 -> 512 + 16kc + 8(s-16)
  uint4 qa[18];
  {
    const uint16_t* qrow = q + ((long)b * H + hg * kHeadsPerGroup + kr) * DSA_QK_DIM;
#pragma unroll
    for (int s = 0; s < 16; ++s) qa[s] = *reinterpret_cast<const uint4*>(qrow + 128 * kc + 8 * s);
#pragma unroll
    for (int s = 0; s < 2; ++s)
      qa[16 + s] = *reinterpret_cast<const uint4*>(qrow + DSA_LATENT_DIM + 16 * kc + 8 * s);
  }
  if (t < kHeadsPerGroup) { sh.m[t] = -INFINITY; sh.l[t] = 0.f; }

  v4f o[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) o[nt] = v4f{0.f, 0.f, 0.f, 0.f};

  const int* idx_row = idx + (long)b * topk;
  for (int tile0 = k0; tile0 < k1; tile0 += kTile) {
    const int j = tile0 + 16 * wv + kr;
    const int slot = (j < k1) ? idx_row[j] : -1;
    const bool valid = slot >= 0 && (long)slot < kv_rows;
    const uint8_t* rowp = pool + (valid ? (long)slot : 0L) * DSA_LATENT_ROW_BYTES;
    uint4 nope[8], rope[2];
    float sc = 0.f;
    if (valid) {
      const uint4* np = reinterpret_cast<const uint4*>(rowp + 128 * kc);
#pragma unroll
      for (int i = 0; i < 8; ++i) nope[i] = np[i];
      sc = reinterpret_cast<const float*>(rowp + DSA_LATENT_DIM)[kc];
      const uint4* rp = reinterpret_cast<const uint4*>(rowp + DSA_LATENT_DIM + 16 + 32 * kc);
      rope[0] = rp[0];
      rope[1] = rp[1];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) nope[i] = make_uint4(0, 0, 0, 0);
      rope[0] = rope[1] = make_uint4(0, 0, 0, 0);
    }

    // dequantise + QK
    uint4 kb[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) dequant16(nope[i], sc, kb[2 * i], kb[2 * i + 1]);
    v4f sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s) sacc = mfma_bf16(qa[s], kb[s], sacc);
    sacc = mfma_bf16(qa[16], rope[0], sacc);
    sacc = mfma_bf16(qa[17], rope[1], sacc);

    // lane holds key (16wv + kr), heads 4kc + r
    const int kl = 16 * wv + kr;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sh.s[(4 * kc + r) * kTile + kl] = valid ? sacc[r] * sm_log2 : -INFINITY;
    // value tile, transposed: vt[d][kl] for d in [128kc, 128kc+128)
    {
      uint16_t* vcol = sh.vt + (128 * kc) * kVtLd + kl;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const uint4 v = kb[s];
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vcol[(8 * s + 2 * e) * kVtLd] = (uint16_t)(w4[e] & 0xffffu);
          vcol[(8 * s + 2 * e + 1) * kVtLd] = (uint16_t)(w4[e] >> 16);
        }
      }
    }
    __syncthreads();

    // online softmax: thread t -> head t/16, keys 4*(t%16) .. +4
    {
      const int h = t >> 4, q4 = (t & 15) * 4;
      float sv[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) { sv[i] = sh.s[h * kTile + q4 + i]; tmax = fmaxf(tmax, sv[i]); }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off));
      const float m_old = sh.m[h];
      const float m_new = fmaxf(m_old, tmax);
      const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_old - m_new);
      float psum = 0.f;
      uint32_t pw[2];
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float p0 = (sv[i] == -INFINITY) ? 0.f : exp2f(sv[i] - m_new);
        const float p1 = (sv[i + 1] == -INFINITY) ? 0.f : exp2f(sv[i + 1] - m_new);
        psum += p0 + p1;
        pw[i >> 1] = pack_bf16x2(p0, p1);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) psum += __shfl_xor(psum, off);
      uint32_t* prow = reinterpret_cast<uint32_t*>(sh.p + h * kPLd + q4);
      prow[0] = pw[0];
      prow[1] = pw[1];
      __syncthreads();
      if ((t & 15) == 0) {
        sh.m[h] = m_new;
        sh.l[h] = sh.l[h] * alpha + psum;
        sh.alpha[h] = alpha;
      }
    }
    __syncthreads();

    // PV: O[16 heads x 512] += P[16 x 64] V[64 x 512]; wave owns cols [128wv, +128)
    float a4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a4[r] = sh.alpha[4 * kc + r];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[nt][r] *= a4[r];
#pragma unroll
    for (int ks = 0; ks < kTile / 32; ++ks) {
      const uint4 pa = *reinterpret_cast<const uint4*>(sh.p + kr * kPLd + 32 * ks + 8 * kc);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const int col = 128 * wv + 16 * nt + kr;
        const uint4 vb = *reinterpret_cast<const uint4*>(sh.vt + col * kVtLd + 32 * ks + 8 * kc);
        o[nt] = mfma_bf16(pa, vb, o[nt]);
      }
    }
    __syncthreads();
  }

  // partials: O [16][512] (unnormalised), (m, l) per head (log2 domain)
  const long pblk = ((long)b * nhg + hg) * nsplit + sp;
  float* po = part_o + pblk * (kHeadsPerGroup * DSA_LATENT_DIM);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      po[(4 * kc + r) * DSA_LATENT_DIM + 128 * wv + 16 * nt + kr] = o[nt][r];
  if (t < kHeadsPerGroup) {
    part_ml[pblk * (2 * kHeadsPerGroup) + 2 * t] = sh.m[t];
    part_ml[pblk * (2 * kHeadsPerGroup) + 2 * t + 1] = sh.l[t];
  }
}

constexpr int kCombCols = 16;                               // output dims per block
constexpr int kCombThreads = kHeadsPerGroup * kCombCols / 4;  // one float4 per thread
constexpr int kMaxSplit = 128;

// Log-sum-exp merge of the split partials (reference combine_kernel
// K:996-1045): m* = max m_s, L = sum l_s 2^(m_s-m*), out = sum O_s 2^(m_s-m*) / L.
// Splits with m = -inf contribute nothing; a row with no valid key gives 0.
// Block (column slice, head group, row): 16 heads x 16 dims, so the merge
// of a b=1 row spreads over 32 workgroups.
__global__ __launch_bounds__(kCombThreads) void sparse_mla_combine_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    uint16_t* __restrict__ out, int H, int nsplit) {
  __shared__ float wgt[kMaxSplit * kHeadsPerGroup];
  const int cb = blockIdx.x, hg = blockIdx.y, b = blockIdx.z, nhg = gridDim.y;
  const int t = threadIdx.x;
  const long pblk0 = ((long)b * nhg + hg) * nsplit;
  if (t < kHeadsPerGroup) {
    const float* ml = part_ml + pblk0 * 2 * kHeadsPerGroup + 2 * t;
    float mx = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, ml[sp * 2 * kHeadsPerGroup]);
    float L = 0.f;
    if (mx != -INFINITY)
      for (int sp = 0; sp < nsplit; ++sp) {
        const float ms = ml[sp * 2 * kHeadsPerGroup];
        if (ms != -INFINITY) L += ml[sp * 2 * kHeadsPerGroup + 1] * exp2f(ms - mx);
      }
    const float inv = (mx != -INFINITY && L > 0.f) ? 1.f / L : 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float ms = ml[sp * 2 * kHeadsPerGroup];
      wgt[sp * kHeadsPerGroup + t] = (ms != -INFINITY) ? exp2f(ms - mx) * inv : 0.f;
    }
  }
  __syncthreads();
  const int h = t / (kCombCols / 4);
  const int d = cb * kCombCols + (t % (kCombCols / 4)) * 4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const float* po = part_o + pblk0 * (kHeadsPerGroup * DSA_LATENT_DIM) + h * DSA_LATENT_DIM + d;
  for (int sp = 0; sp < nsplit; ++sp) {
    const float wt = wgt[sp * kHeadsPerGroup + h];
    if (wt != 0.f) {
      const float4 x = *reinterpret_cast<const float4*>(po + (long)sp * (kHeadsPerGroup * DSA_LATENT_DIM));
      acc.x += x.x * wt; acc.y += x.y * wt; acc.z += x.z * wt; acc.w += x.w * wt;
    }
  }
  uint2 pk;
  pk.x = pack_bf16x2(acc.x, acc.y);
  pk.y = pack_bf16x2(acc.z, acc.w);
  *reinterpret_cast<uint2*>(out + ((long)b * H + hg * kHeadsPerGroup + h) * DSA_LATENT_DIM + d) = pk;
}

int sparse_mla_auto_nsplit(int topk) {
  return std::max(1, std::min(kMaxSplit, (topk + kTile - 1) / kTile));
}

size_t sparse_mla_workspace_bytes(int B, int H, int nsplit) {
  const size_t blocks = (size_t)B * (H / kHeadsPerGroup) * nsplit;
  return blocks * kHeadsPerGroup * (DSA_LATENT_DIM + 2) * sizeof(float);
}

hipError_t launch_sparse_mla(const uint16_t* q, const uint8_t* pool, long kv_rows,
                             const int* idx, void* workspace, uint16_t* out, int B, int H,
                             int topk, int nsplit, float sm_scale, hipStream_t s) {
  const int nhg = H / kHeadsPerGroup;
  float* part_o = reinterpret_cast<float*>(workspace);
  float* part_ml = part_o + (size_t)B * nhg * nsplit * kHeadsPerGroup * DSA_LATENT_DIM;
  const float sm_log2 = sm_scale * 1.4426950408889634f;
  hipLaunchKernelGGL(sparse_mla_split_kernel, dim3(nsplit, nhg, B), dim3(kAttnThreads), 0, s, q,
                     pool, kv_rows, idx, part_o, part_ml, H, topk, nsplit, sm_log2);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sparse_mla_combine_kernel, dim3(DSA_LATENT_DIM / kCombCols, nhg, B),
                     dim3(kCombThreads), 0, s, part_o, part_ml, out, H, nsplit);
  return hipGetLastError();
}

}  // namespace dsa
