// The decode layer's main launch (gfx950): sparse-MLA attention workgroups
// and lightning-indexer scan workgroups in ONE grid.
//
// Roles by blockIdx.x (role-decoupled workgroups, as the reference's HIDE
// kernel does, K:1047-1070):
//   [0, n_att)         attention: (row, head group, split) of split-K sparse
//                      MLA; the splits of a (row, head group) pass a group
//                      barrier, then each merges (log-sum-exp) a 1/nsplit
//                      slice of the outputs;
//   [n_att, +n_scan)   indexer scan: (row, slice) of the row's 16-key
//                      chunks; the row's scan workgroups then select its
//                      top-k together (coop_select: each publishes a short
//                      list of its top keys, and after one barrier every
//                      workgroup finds the exact threshold from the lists
//                      and writes its own selected positions), while the
//                      attention workgroups are still busy.
// Under the MLI lag, layer L's attention (over layer L-1's selection) and
// layer L's indexer scan are independent, so one grid runs both and the
// scan's HBM stream hides under the attention's gather latency.  Measured on
// MI355X: two HIP streams, or one hipGraph with two branches, did not run
// these concurrently (the host dispatches one node at a time), while one
// grid does by construction.
//
// Attention (reference hp_attention_block K:1312-1598, combine K:996-1045,
// CPU semantics attention_core.py:94-146):
//   out[b,h,:] = sum_j softmax_j(sm * q[b,h,:] . kv_j) * kv_j[:512],
//   kv_j = bf16_rn(f32(e4m3) * scale[d/128]) | bf16 rope (K:1181-1197).
// A workgroup (8 waves) takes 128-key tiles of its split.  Lane (kr, kc) of
// wave w gathers key 16w+kr's bytes [128kc, +128) + scale kc + rope
// [16kc, +16) straight into registers (4 lanes per 656-byte row, each a
// contiguous run), dequantises them and feeds them as the B operand of
// v_mfma_f32_16x16x32_bf16 with the 16 heads as A; Q and K use the same
// lane->k assignment, so the 576-dim contraction needs no LDS staging.
// The value tile is written to LDS transposed ([dim][key]) for the PV MFMA;
// softmax runs in the exp2 domain.
//
// Scan (reference hp_indexer_block K:1677-2157, fp8 semantics K:2990-2992):
//   score[b,g] = kscale[g] * sum_h w[b,h] * ReLU(q[b,h,:] . k[g,:]).
// A wave owns 16-key chunks (2 KB contiguous in an 8448-byte page); one
// v_mfma_f32_16x16x128_f8f6f4 per 16 heads contracts the whole 128-d dot
// product (A = query heads, B = key chunk, loaded straight from HBM into
// registers with the same lane->k assignment as A).  Each lane ends with one
// key x 4 heads: ReLU*w summed in-lane, then across lane groups with two xor
// shuffles.  Several chunks per wave have loads in flight (scan_batch).
#include <algorithm>

#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

constexpr int kMainThreads = 512;
constexpr int kMainWaves = kMainThreads / kWave;  // 8

// ======================================================================
// attention role
// ======================================================================
constexpr int kTile = 16 * kMainWaves;  // 128 keys per tile
constexpr int kVLd = DSA_LATENT_DIM + 16;  // value tile row stride (bf16): 264 dwords, 8 mod 64 banks
constexpr int kPLd = kTile + 8;         // probability row stride (bf16)
constexpr int kHG = kHeadGroup;         // heads per group
constexpr int kMaxSplit = 128;
constexpr int kAutoSplitKeys = 64;  // selected keys per split by default

struct AttnShared {
  uint16_t vt[kTile * kVLd];             // value tile [key][dim], row-major
  float s[kHG * kTile];                  // scores, log2 domain
  uint16_t p[kHG * kPLd];                // probabilities, bf16
  float m[kHG], l[kHG], alpha[kHG];
};
static_assert(kMaxSplit * 3 * kHG * sizeof(float) + kMainThreads * 16 <= sizeof(AttnShared::vt), "merge scratch");

__device__ __forceinline__ v4f mfma_bf16(const uint4& a, const uint4& b, v4f c) {
  v8bf av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
}

// 16 e4m3 (one uint4) * scale -> 16 bf16 (two uint4: elements 0-7, 8-15),
// bf16_rn(f32(e4m3) * scale) exactly.
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

typedef short v4s __attribute__((ext_vector_type(4)));

// B operand of the PV MFMA (k = 32 keys, n = 16 dims) from the row-major
// value tile with two ds_read_b64_tr_b16.  Within each 16-lane group that
// instruction hands lane i element (i & 3) of the 8-byte word addressed by
// lane 4j + (i >> 2), as element j.  So lane (a, g) of k-group g addresses
// key 8g + (a >> 2) (+4 for the second read), dims col0 + 4(a & 3): lane n
// then holds V[8g + 0..7][col0 + n], k-slots 8g..8g+7 -- the same k-slot ->
// key map the probabilities' A operand uses (P[h][32ks + 8g + e]).
__device__ __forceinline__ uint4 load_v_operand(const uint16_t* vt, int key0, int col0, int lane) {
  const int a = lane & 15, g = lane >> 4;
  const uint16_t* p = vt + (key0 + 8 * g + (a >> 2)) * kVLd + col0 + 4 * (a & 3);
  typedef v4s __attribute__((address_space(3)))* lds_v4s;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(p));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(p + 4 * kVLd));
  uint4 r;
  __builtin_memcpy(&r.x, &lo, 8);
  __builtin_memcpy(&r.z, &hi, 8);
  return r;
}

// STAGE_Q: the query block is loaded once per workgroup and staged in LDS
// (attention-only launches); otherwise each key wave loads its operand from
// memory (the fused launch: measured 0.13 us per C3 layer faster that way,
// while an attention-only launch is 0.3 us faster staged).
template <bool STAGE_Q>
__device__ __forceinline__ void attention_block(const AttnArgs& A, int b, int hg, int sp, unsigned char* smem) {
  AttnShared& sh = *reinterpret_cast<AttnShared*>(smem);
  const int nhg = A.H / kHG, nsplit = A.nsplit;
  const int dbk = blockIdx.x;
  dbg_stamp(dbk, 0);
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = wave_id();
  const int kr = lane & 15, kc = lane >> 4;
  // the barrier's flag value, read now and used at the barrier (the load's
  // latency hides under the gather)
  const uint32_t sense = (t == 0) ? group_sense(A.sync + ((long)b * nhg + hg) * kSyncWords, sp) : 0u;
  const int kps = (A.topk + nsplit - 1) / nsplit;
  const int k0 = min(A.topk, sp * kps), k1 = min(A.topk, k0 + kps);
  // the KV slot of key j of the row: the selection's entry, or (dense) the
  // slot of token j through the page table (-1 at or past the row's length)
  const int* idx_row = A.idx + (long)b * A.topk;
  const int* dpt_row = A.dense_pt + (long)b * A.dense_pt_stride;
  const int dlen = A.dense_pt ? max(0, min(A.dense_lens[b], A.topk)) : 0;
  const auto key_slot = [&](int j) {
    if (j >= k1) return -1;
    if (!A.dense_pt) return idx_row[j];
    return j < dlen ? dpt_row[j >> 6] * DSA_PAGE_TOKENS + (j & (DSA_PAGE_TOKENS - 1)) : -1;
  };

  // STAGE_Q: the query block (16 heads x 576 bf16, 18 KB) is loaded once per
  // workgroup, coalesced (thread t: uint4s t, t + 512, ...), and staged in
  // LDS for the key waves' operand reads (each wave loading its own copy
  // would read it 4-8 times through the vector L1).  Issued first: the key
  // rows wait for their slots anyway.
  constexpr int kQVec = kHG * DSA_QK_DIM / 8, kQRowVec = DSA_QK_DIM / 8;
  uint4 qv[(kQVec + kMainThreads - 1) / kMainThreads];
  if constexpr (STAGE_Q) {
    const uint4* qsrc = reinterpret_cast<const uint4*>(A.q + ((long)b * A.H + hg * kHG) * DSA_QK_DIM);
#pragma unroll
    for (int j = 0; j < (kQVec + kMainThreads - 1) / kMainThreads; ++j) {
      const int u = t + j * kMainThreads;
      qv[j] = u < kQVec ? qsrc[u] : make_uint4(0, 0, 0, 0);
    }
  }
  // the first two tiles' slots (the gathers depend on them)
  const int slot0 = key_slot(k0 + 16 * wv + kr);
  int slot_next = key_slot(k0 + kTile + 16 * wv + kr);
  // staged now, so the query registers are free before the rows are loaded
  // (the unstaged form loads each wave's operand after the rows, below)
  constexpr int kQLd = DSA_QK_DIM + 8;
  static_assert(kHG * kQLd <= kTile * kVLd, "the query stages in the value tile");
  if constexpr (STAGE_Q) {
#pragma unroll
    for (int j = 0; j < (kQVec + kMainThreads - 1) / kMainThreads; ++j) {
      const int u = t + j * kMainThreads;
      if (u < kQVec)
        *reinterpret_cast<uint4*>(sh.vt + (u / kQRowVec) * kQLd + (u % kQRowVec) * 8) = qv[j];
    }
  }
  // This lane's bytes of one key row (zeros for an invalid slot).  Step i
  // of a row's 512 latent bytes: lane (kr, kc) reads bytes 64i + 16kc ..
  // + 16 of key kr, so each load instruction reads 64 contiguous bytes of
  // each of its 16 rows (a load whose 64 lanes touch 64 different cache
  // lines is bound by the vector L1's line lookups, not by memory).  The
  // dot product is over all dims, so the query takes the same dim order.
  struct RowRegs {
    uint4 nope[8], rope[2];
    float4 sc;  // the row's 4 scales (one per 128 dims)
    bool valid;
  };
  const auto load_row = [&](int slot, RowRegs& r) {
    r.valid = slot >= 0 && (long)slot < A.kv_rows;
    r.sc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r.valid) {
      const uint8_t* rowp = A.pool + (long)slot * DSA_LATENT_ROW_BYTES;
#pragma unroll
      for (int i = 0; i < 8; ++i) r.nope[i] = *reinterpret_cast<const uint4*>(rowp + 64 * i + 16 * kc);
      r.sc = *reinterpret_cast<const float4*>(rowp + DSA_LATENT_DIM);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        r.rope[s2] = *reinterpret_cast<const uint4*>(rowp + DSA_LATENT_DIM + 16 + 64 * s2 + 16 * kc);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) r.nope[i] = make_uint4(0, 0, 0, 0);
      r.rope[0] = r.rope[1] = make_uint4(0, 0, 0, 0);
    }
  };
  RowRegs cur;
  load_row(slot0, cur);

  // Q (A operand) in the keys' dim order: steps 2i, 2i + 1 -> dims 64i +
  // 16kc + 0..7, + 8..15; steps 16 + s -> rope dims 32s + 8kc + 0..7, read
  // from the staged block (rows kQLd bf16 apart: 292 dwords, so the 16 heads
  // of a read fall in distinct bank groups).  A wave with no keys in its
  // split (short splits) reads none.  The staging area is the value tile's,
  // which the tile loop writes after the barrier below.
  if constexpr (STAGE_Q) __syncthreads();
  uint4 qa[18];
  if (16 * wv < k1 - k0) {
    const uint16_t* qrow = STAGE_Q ? sh.vt + kr * kQLd : A.q + ((long)b * A.H + hg * kHG + kr) * DSA_QK_DIM;
#pragma unroll
    for (int s = 0; s < 16; ++s) qa[s] = *reinterpret_cast<const uint4*>(qrow + 64 * (s >> 1) + 16 * kc + 8 * (s & 1));
#pragma unroll
    for (int s = 0; s < 2; ++s)
      qa[16 + s] = *reinterpret_cast<const uint4*>(qrow + DSA_LATENT_DIM + 32 * s + 8 * kc);
  } else {
#pragma unroll
    for (int s = 0; s < 18; ++s) qa[s] = make_uint4(0, 0, 0, 0);
  }
  if constexpr (STAGE_Q) __syncthreads();  // every wave has its operand before the value tile is written
  if (t < kHG) { sh.m[t] = -INFINITY; sh.l[t] = 0.f; }

  v4f o[4];  // wave owns output dims [64 wv, 64 wv + 64): 4 n-tiles
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) o[nt] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int tile0 = k0; tile0 < k1; tile0 += kTile) {
    // the next tile's gather is in flight while this tile is computed
    const bool more = tile0 + kTile < k1;  // uniform
    RowRegs nxt;
    if (more) {
      load_row(slot_next, nxt);
      const int jn = tile0 + 2 * kTile + 16 * wv + kr;  // the slot after it, early
      slot_next = key_slot(jn);
    }
    const bool valid = cur.valid;
    const uint4* nope = cur.nope;
    const uint4* rope = cur.rope;
    const float sc4[4] = {cur.sc.x, cur.sc.y, cur.sc.z, cur.sc.w};

    // dequantise -> QK MFMA + row-major value tile (16-byte stores).  The
    // dequant is VALU-bound and a SIMD runs two waves, so a wave with no key
    // in this tile skips it (zeroing its value rows when the PV k-steps in
    // use cover them); the PV below skips k-steps past the tile's keys.
    const int nk = k1 - tile0;                        // keys in this tile
    const int nks = min(kTile / 32, (nk + 31) >> 5);  // PV k-steps in use
    const int kl = 16 * wv + kr;
    uint4* vrow = reinterpret_cast<uint4*>(sh.vt + kl * kVLd + 16 * kc);
    v4f sacc = {0.f, 0.f, 0.f, 0.f};
    if (16 * wv < nk) {  // uniform
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint4 lo, hi;
        dequant16(nope[i], sc4[i >> 1], lo, hi);
        sacc = mfma_bf16(qa[2 * i], lo, sacc);
        sacc = mfma_bf16(qa[2 * i + 1], hi, sacc);
        vrow[8 * i] = lo;  // dims 64i + 16kc ..
        vrow[8 * i + 1] = hi;
      }
      sacc = mfma_bf16(qa[16], rope[0], sacc);
      sacc = mfma_bf16(qa[17], rope[1], sacc);
    } else if (16 * wv < 32 * nks) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vrow[8 * i] = vrow[8 * i + 1] = make_uint4(0, 0, 0, 0);
    }
    dbg_stamp(dbk, 1);
    // lane holds key kl (column), heads 4kc + r (rows)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sh.s[(4 * kc + r) * kTile + kl] = valid ? sacc[r] * A.sm_log2 : -INFINITY;
    __syncthreads();
    dbg_stamp(dbk, 6);

    // online softmax: thread t -> head t/32, keys 4*(t%32) .. +4
    {
      const int h = t >> 5, q4 = (t & 31) * 4;
      float sv[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) { sv[i] = sh.s[h * kTile + q4 + i]; tmax = fmaxf(tmax, sv[i]); }
      tmax = half_wave_reduce<2>(tmax);
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
      psum = half_wave_reduce<0>(psum);
      uint32_t* prow = reinterpret_cast<uint32_t*>(sh.p + h * kPLd + q4);
      prow[0] = pw[0];
      prow[1] = pw[1];
      __syncthreads();
      if ((t & 31) == 0) {
        sh.m[h] = m_new;
        sh.l[h] = sh.l[h] * alpha + psum;
        sh.alpha[h] = alpha;
      }
    }
    __syncthreads();
    dbg_stamp(dbk, 2);

    // PV: O[16 x 512] += P[16 x 128] V[128 x 512]
    float a4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a4[r] = sh.alpha[4 * kc + r];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[nt][r] *= a4[r];
#pragma unroll
    for (int ks = 0; ks < kTile / 32; ++ks) {
      if (ks >= nks) break;  // uniform: no keys past here
      const uint4 pa = *reinterpret_cast<const uint4*>(sh.p + kr * kPLd + 32 * ks + 8 * kc);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint4 vb = load_v_operand(sh.vt, 32 * ks, 64 * wv + 16 * nt, lane);
        o[nt] = mfma_bf16(pa, vb, o[nt]);
      }
    }
    __syncthreads();
    if (more) cur = nxt;
  }

  dbg_stamp(dbk, 3);
  // partials: O (unnormalised) in the MFMA's output layout, [512 dims][16
  // heads]: lane (kr, kc) of n-tile nt holds heads 4kc .. 4kc + 3 of dim
  // 64wv + 16nt + kr, one 16-byte store, so each wave store writes 1 KB
  // contiguous (16 dims x 16 heads; per-element stores of a [head][dim]
  // layout took ~0.8 us to issue).  (m, l) per head, log2 domain.
  const long pblk0 = ((long)b * nhg + hg) * nsplit;
  const long pblk = pblk0 + sp;
  {
    const __amdgpu_buffer_rsrc_t pw = dev_rsrc(A.part_o + pblk * (kHG * DSA_LATENT_DIM), kHG * DSA_LATENT_DIM * 4u);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      store_dev16(pw, 4u * (uint32_t)((64 * wv + 16 * nt + kr) * kHG + 4 * kc),
                  make_float4(o[nt][0], o[nt][1], o[nt][2], o[nt][3]));
  }
  if (t < kHG) {
    store_dev(&A.part_ml[pblk * (2 * kHG) + 2 * t], sh.m[t]);
    store_dev(&A.part_ml[pblk * (2 * kHG) + 2 * t + 1], sh.l[t]);
  }

  // every split of (row, head group) waits for the others' partials, then
  // merges a 1/nsplit slice of the 16 x 512 outputs
  group_barrier(A.sync + ((long)b * nhg + hg) * kSyncWords, sp, nsplit, sense);
  dbg_stamp(dbk, 4);

  // log-sum-exp merge (reference combine_kernel K:996-1045):
  // m* = max m_s, L = sum l_s 2^(m_s - m*), out = sum O_s 2^(m_s - m*) / L,
  // the splits summed in a fixed order (deterministic output).
  // float4 units of the group's outputs: unit v = heads 4(v & 3) .. + 3 of
  // dim v >> 2 (the partials' layout)
  constexpr int kVec = kHG * DSA_LATENT_DIM / 4;
  float* mls = reinterpret_cast<float*>(sh.vt);
  float* wgt = mls + kMaxSplit * 2 * kHG;
  float4* red = reinterpret_cast<float4*>(wgt + kMaxSplit * kHG);
  const float* pbase = A.part_o + pblk0 * (kHG * DSA_LATENT_DIM);
  const __amdgpu_buffer_rsrc_t prs = dev_rsrc(pbase, (uint32_t)nsplit * kHG * DSA_LATENT_DIM * 4u);
  const __amdgpu_buffer_rsrc_t mrs = dev_rsrc(A.part_ml + pblk0 * 2 * kHG, nsplit * 2 * kHG * 4u);
  const int v_lo = (int)((long)kVec * sp / nsplit), nv = (int)((long)kVec * (sp + 1) / nsplit) - v_lo;
  const int span = min(nv, kMainThreads);  // outputs per round
  int G = 1;                               // thread groups over the splits
  while (2 * G * span <= kMainThreads && 2 * G <= nsplit) G *= 2;
  const int spg = (nsplit + G - 1) / G;
  const int g = t / span;
  constexpr int kLd = 8;                   // partial loads in flight per thread
  float4 x[kLd];
  // loads past s1 read 0: they are issued at the resource's end, so every
  // load is issued unconditionally and the compiler can wait for the
  // earlier (m, l) loads alone (a conditional load in between made it wait
  // for all of them, these partials included)
  const uint32_t p_end = 16u * (uint32_t)(nsplit * kVec);
  auto load_x = [&](int v, int s0, int s1) {
#pragma unroll
    for (int i = 0; i < kLd; ++i)
      x[i] = __builtin_bit_cast(float4, load_dev16(prs, s0 + i < s1 ? 16u * ((s0 + i) * kVec + v) : p_end));
  };
  {  // the splits' (m, l) first (nsplit*32 floats, <= 8 per thread), then this
     // thread's partials: the merge weights are computed while those arrive
    constexpr int kPer = kMaxSplit * 2 * kHG / kMainThreads;
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {  // rounds past the splits' pairs are skipped (uniform)
      const int i = t + j * kMainThreads;
      v[j] = j * kMainThreads < nsplit * 2 * kHG
                 ? __uint_as_float(load_dev4(mrs, i < nsplit * 2 * kHG ? 4u * i : 0xfffffffcu))
                 : 0.f;
    }
    const bool act = g < G && t - g * span < nv;
    load_x(v_lo + t - g * span, act ? g * spg : 0, act ? min(nsplit, (g + 1) * spg) : 0);
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (t + j * kMainThreads < nsplit * 2 * kHG) mls[t + j * kMainThreads] = v[j];
  }
  __syncthreads();
  dbg_stamp(dbk, 8);
  if (t < kHG * 16) {
    // one 16-lane DPP row per head; lane i of the row takes the splits
    // i, i + 16, ... (<= kMaxSplit / 16 each)
    const int h = t >> 4, i = t & 15;
    constexpr int kPerLane = kMaxSplit / 16;
    float ms[kPerLane], ls[kPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int s2 = i + 16 * j;
      const float2 ml = s2 < nsplit ? *reinterpret_cast<const float2*>(&mls[s2 * 2 * kHG + 2 * h])
                                    : make_float2(-INFINITY, 0.f);
      ms[j] = ml.x;
      ls[j] = ml.y;
      mx = fmaxf(mx, ms[j]);
    }
    mx = row16_reduce<2>(mx);
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      ms[j] = ms[j] != -INFINITY ? exp2f(ms[j] - mx) : 0.f;  // the split's factor
      L += ls[j] * ms[j];
    }
    L = row16_reduce<0>(L);
    const float inv = (mx != -INFINITY && L > 0.f) ? 1.f / L : 0.f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int s2 = i + 16 * j;
      if (s2 < nsplit) wgt[s2 * kHG + h] = ms[j] * inv;
    }
  }
  __syncthreads();
  dbg_stamp(dbk, 5);
  for (int r0 = 0; r0 < nv; r0 += span) {
    const int vi = r0 + t - g * span;
    const bool active = g < G && vi < nv;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) {
      const int v = v_lo + vi;
      const int h0 = 4 * (v & 3);
      const int s0 = g * spg, s1 = min(nsplit, s0 + spg);
      for (int sb = s0; sb < s1; sb += kLd) {
        if (r0 != 0 || sb != s0) load_x(v, sb, s1);
#pragma unroll
        for (int i = 0; i < kLd; ++i) {
          const float4 wt = (sb + i < s1) ? *reinterpret_cast<const float4*>(&wgt[(sb + i) * kHG + h0])
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
          acc.x += x[i].x * wt.x; acc.y += x[i].y * wt.y;
          acc.z += x[i].z * wt.z; acc.w += x[i].w * wt.w;
        }
      }
    }
    if (G > 1) {
      if (active) red[t] = acc;
      __syncthreads();
      if (g == 0 && active)
        for (int k = 1; k < G; ++k) {
          const float4 y = red[k * span + t];
          acc.x += y.x; acc.y += y.y; acc.z += y.z; acc.w += y.w;
        }
      __syncthreads();
    }
    if (g == 0 && active) {
      const int v = v_lo + vi;
      const uint32_t p01 = pack_bf16x2(acc.x, acc.y), p23 = pack_bf16x2(acc.z, acc.w);
      uint16_t* op = A.out + ((long)b * A.H + hg * kHG + 4 * (v & 3)) * DSA_LATENT_DIM + (v >> 2);
      op[0] = (uint16_t)p01;
      op[DSA_LATENT_DIM] = (uint16_t)(p01 >> 16);
      op[2 * DSA_LATENT_DIM] = (uint16_t)p23;
      op[3 * DSA_LATENT_DIM] = (uint16_t)(p23 >> 16);
    }
  }
  dbg_stamp(dbk, 7);
}

// ======================================================================
// indexer-scan role
// ======================================================================
constexpr int kChunkKeys = 16;
// chunks per wave with loads in flight: 8 when the scan workgroup owns its
// CU (the select's LDS); 4 in a plain scan, where two workgroups share a CU
template <bool SELECT>
constexpr int scan_batch() { return SELECT ? 8 : 4; }
constexpr int kHistBins = 4096;

constexpr int kScanMaxPages = 4100;  // page-table entries a workgroup prefetches
// Histogram area: 4096 fine bins, 32 spill bins (branch-free updates),
// then 64 coarse bins (coarse c = fine bins [64c, 64c + 64)) and their 32
// spill bins.
// Union histogram of the published-list select: 2048 bins in 64 groups of
// 32, each group padded to 36 words so that lanes summing one group each
// read distinct LDS banks.
constexpr int kUnionBins = 2048;
constexpr int kUnionGroup = 32, kUnionStride = 36, kUnionWords = kWave * kUnionStride;
__device__ __forceinline__ uint32_t union_slot(uint32_t b) { return b + (b / kUnionGroup) * (kUnionStride - kUnionGroup); }
constexpr int kCoarseOff = kHistBins + 64;
constexpr int kCoarseSpillOff = kCoarseOff + 64;
constexpr int kHistWords = kCoarseSpillOff + 32;
static_assert(kHistWords % 4 == 0, "the histogram area is cleared in uint4s");
static_assert(kUnionWords + kWave <= kHistWords, "the union histogram and its per-lane spill words fit the histogram area");
struct ScanShared {
  uint8_t qs[64 * DSA_INDEX_DIM];
  float ws[64];
  alignas(16) uint32_t hist[kHistWords];
  int pts[kScanMaxPages];
};

// Cooperative select: the scan workgroup keeps the rank keys of its own
// positions and takes part in the row's selection.
constexpr int kCoopKeys = 16384;     // positions per workgroup
constexpr int kCoopMaxBlocks = 256;  // workgroups per row
constexpr int kPubHdr = 4;           // list header: count, bound key, finite count, max key
constexpr int kCoopCand = 1024;      // threshold-bin candidates resolved by rank counting
constexpr int kEmitRegs = 8;         // emit: entries per thread read into registers at once
struct CoopShared {
  ScanShared scan;
  alignas(16) uint32_t keys[kCoopKeys];
  uint16_t lpos[kPubWords];  // the published entries: own position index
  uint32_t wave_tmp[4 * kMainWaves];
  uint32_t res[4];
  uint32_t misc[4];
  uint32_t sense[kNumSync];
  alignas(16) uint32_t ck[kCoopCand];  // threshold-bin candidates: key, union entry index
  uint32_t ce[kCoopCand];
  uint32_t wstat[2 * kMainWaves];  // per wave, from the scan: finite keys, largest key
  uint32_t pred[2 * kMainWaves];   // per wave: union counts of pass 2
};

static_assert(sizeof(CoopShared) <= 160 * 1024, "the cooperative select's LDS must fit one CU");
static_assert(kCoopKeys <= 65536, "own positions are stored as 16-bit indices");

// Keys a workgroup's list aims to hold: twice its expected share of the K
// selected keys plus 8.  The list's capacity (a multiple of 4, within the
// area) adds half a share, so that the threshold bin often fits whole (else
// it is split by sub-bins); every workgroup loads every list after the
// barrier, so capacity costs load time.
// A list too short for its workgroup only costs the fallback to the
// single-workgroup select.
__host__ __device__ inline int pub_target(int nb, int K) { return 2 * (int)(((uint32_t)K + nb - 1) / (uint32_t)nb) + 8; }
__host__ __device__ inline int pub_stride(int nb, int K) {
  const int want = pub_target(nb, K) + (int)((((uint32_t)K + nb - 1) / (uint32_t)nb + 1) / 2);
  return min((want + 3) & ~3, (int)((uint32_t)kPubWords / (uint32_t)nb) & ~3);
}

// A list bound that lists nothing; a row whose bound it is goes to the
// single-workgroup select (it cannot hold K keys >= the bound).
constexpr uint32_t kNoKeys = 0xffffffffu;
__device__ __forceinline__ uint32_t next_bin_key(uint32_t bin) { return bin >= 4095u ? kNoKeys : (bin + 1u) << 20; }

// ---- wave-level steps of the published-list select: every wave of the
// workgroup computes the same result, so no block barrier is needed ----

// The largest fine bin T with #(keys in bins >= T) >= need, over the 4096
// fine bins and their 64 coarse sums: two DPP scans (coarse, then the 64
// fine bins of the chosen coarse bin).  need >= 1; when the histogram holds
// fewer than need keys only `total` is set.
struct BinThreshold {
  uint32_t bin, above, cnt, total;  // above: keys in bins > bin; cnt: keys in bin
};
__device__ __forceinline__ BinThreshold wave_threshold(const uint32_t* hist, uint32_t need) {
  const int lane = threadIdx.x & (kWave - 1);
  BinThreshold r{0u, 0u, 0u, 0u};
  const uint32_t c = hist[kCoarseOff + kWave - 1 - lane];  // lane 0: the top coarse bin
  const uint32_t pc = wave_scan_incl<0>(c);                 // keys in coarse bins >= 63 - lane
  r.total = (uint32_t)__builtin_amdgcn_readlane((int)pc, kWave - 1);
  if (r.total < need) return r;
  const int l1 = __builtin_ctzll(__ballot(pc >= need));
  const uint32_t cbin = (uint32_t)(kWave - 1 - l1);
  const uint32_t above_c = (uint32_t)__builtin_amdgcn_readlane((int)(pc - c), l1);
  const uint32_t f = hist[cbin * kWave + kWave - 1 - lane];
  const uint32_t pf = wave_scan_incl<0>(f) + above_c;
  const int l2 = __builtin_ctzll(__ballot(pf >= need));
  r.bin = cbin * kWave + (uint32_t)(kWave - 1 - l2);
  r.cnt = (uint32_t)__builtin_amdgcn_readlane((int)f, l2);
  r.above = (uint32_t)__builtin_amdgcn_readlane((int)pf, l2) - r.cnt;
  return r;
}

// The same over a histogram of kWave groups of PER bins (PER = 32 or 64),
// group g at word STRIDE * g, without coarse sums: lane l first sums group
// 63 - l.
template <int PER, int STRIDE>
__device__ __forceinline__ BinThreshold wave_threshold_sum(const uint32_t* hist, uint32_t need) {
  static_assert((PER == 32 || PER == 64) && STRIDE % 4 == 0 && STRIDE >= PER, "group layout");
  const int lane = threadIdx.x & (kWave - 1);
  BinThreshold r{0u, 0u, 0u, 0u};
  const uint4* p = reinterpret_cast<const uint4*>(hist + STRIDE * (kWave - 1 - lane));
  uint32_t c = 0;
#pragma unroll
  for (int q = 0; q < PER / 4; ++q) {
    const uint4 v = p[q];
    c += v.x + v.y + v.z + v.w;
  }
  const uint32_t pc = wave_scan_incl<0>(c);
  r.total = (uint32_t)__builtin_amdgcn_readlane((int)pc, kWave - 1);
  if (r.total < need) return r;
  const int l1 = __builtin_ctzll(__ballot(pc >= need));
  const uint32_t grp = (uint32_t)(kWave - 1 - l1);
  const uint32_t above_c = (uint32_t)__builtin_amdgcn_readlane((int)(pc - c), l1);
  const uint32_t f = lane < PER ? hist[grp * STRIDE + PER - 1 - lane] : 0u;
  const uint32_t pf = wave_scan_incl<0>(f) + above_c;
  const int l2 = __builtin_ctzll(__ballot(lane < PER && pf >= need));
  r.bin = grp * PER + (uint32_t)(PER - 1 - l2);
  r.cnt = (uint32_t)__builtin_amdgcn_readlane((int)f, l2);
  r.above = (uint32_t)__builtin_amdgcn_readlane((int)pf, l2) - r.cnt;
  return r;
}

// this lane's rank among the set lanes of a wave mask
__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Workgroup i's share [part(n, i, nb), part(n, i + 1, nb)) of n items, in
// 32-bit unsigned arithmetic (a 64-bit division is ~100 instructions, and
// every instruction on this serial path costs ~2 ns): n * nb < 2^32, which
// the launcher checks.
__device__ __forceinline__ int part(int n, int i, int nb) {
  return (int)(((uint32_t)n * (uint32_t)i) / (uint32_t)nb);
}

// Cooperative radix select, the published-list select's fallback when the
// lists cannot decide (the row's top keys are packed into the positions of
// a few workgroups, e.g. a recent-token window, or many equal scores).  The
// row's workgroups still hold their own keys in LDS; together they find the
// exact K-th key t* with three radix digits (key bits 31-20, 19-8, 7-0, the
// digit structure of tilelang_dsa/topk_selector.py:36-194):
//   each workgroup histograms the digit of its own keys that match the
//   prefix so far, adds its non-zero bins to the row's global histogram of
//   the pass (device-scope atomics), meets the others at a barrier, loads
//   the summed histogram and takes the threshold bin (every workgroup reads
//   the same sums, so all agree);
// then every workgroup publishes its counts of finite keys above t* and of
// keys equal to t*, and after one more barrier takes the counts of the
// workgroups before it (its output offset).  Global areas of the row: the
// pass-0 histogram in the standalone select's histogram (zero between
// calls: cleared again here once read), passes 1 and 2 in its candidate
// area (cleared here before use), the counts in its bitmap area (the
// launcher keeps nb <= its words), the barrier counters in the otherwise
// unused barrier areas 1 and 2: one set per launch parity (the list
// barrier's sense), the other set is re-zeroed by every launch's list
// barrier, so each launch starts from zero without a counter of its own.
// Four barriers, no re-read of scores.
struct RadixSel {
  uint32_t tstar, need3, sel_before, ties_before, sel_above;
  uint32_t own_gt, own_eq;  // this workgroup's finite keys above t*, keys equal to t*
};
// A reusable barrier of the row's nb workgroups on monotonic counters (no
// re-zeroing between uses): member bid arrives on group counter bid % 8; a
// group's last arrival (its counter reaching use * group size) adds itself,
// without waiting, to 8 replicated top counters, and each member polls the
// replica of its XCD (bid % 8) until use * groups have arrived.  So no line
// is both hit by many atomics and polled by many workgroups.  Lines (64
// words each) of `ctr`: 0-7 group counters, 8-15 top replicas.  The wait is
// bounded like the group barriers'.
constexpr int kRadixGroups = 8;
__host__ __device__ inline long radix_sync_off(int slab, uint32_t set) {
  return row_sync_off(slab) + (1L + (long)set) * kSyncWords;
}
static_assert(2 * kRadixGroups <= kGroupSyncGroups + 1 + kGroupSyncFlags && kNumSync >= 4,
              "the radix barrier's counter sets fit barrier areas 1 and 2");
__device__ __forceinline__ void counter_barrier(uint32_t* ctr, int bid, int nb, uint32_t use, uint32_t* status) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int g = bid % kRadixGroups;
    const uint32_t ng = (uint32_t)((nb - 1 - g) / kRadixGroups + 1);
    const uint32_t ngroups = (uint32_t)min(nb, kRadixGroups);
    if (__hip_atomic_fetch_add(&ctr[g * kGroupSyncLine], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        use * ng - 1u)
      for (int r = 0; r < kRadixGroups; ++r)
        __hip_atomic_fetch_add(&ctr[(kRadixGroups + r) * kGroupSyncLine], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t* top = &ctr[(kRadixGroups + bid % kRadixGroups) * kGroupSyncLine];
    const int lim = g_group_spin_max;
    for (int i = 0; __hip_atomic_load(top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < use * ngroups; ++i) {
      if (i == lim) {
        wait_expired(status);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}
__device__ __forceinline__ RadixSel coop_radix(CoopShared& cs, uint32_t* rs, int slab, int bid, int nb, int nown,
                                               uint32_t K, uint32_t set) {
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  uint32_t* hist = cs.scan.hist;  // the union histogram is dead: 4096 words
  uint32_t* g0 = rs + kHistOff;
  uint32_t* g12 = rs + kBmOff + bitmap_words(slab);  // 2 x 4096 words
  uint32_t* cnts = rs + kBmOff;
  uint32_t* ctr = rs + radix_sync_off(slab, set);
  uint32_t* status = rs + row_sync_off(slab) + kSyncStatusWord;  // the row's, as for the list barrier
  // A lower bound on t* from the list headers: workgroup b holds count_b
  // keys >= its list bound lo_b, so if the workgroups whose bound lies in
  // 12-bit bins >= TB hold >= K such keys together, t* >= TB's lower edge,
  // and pass 0 need only count keys in bins >= TB (exact counts there are
  // all the threshold search reads).  This spares most workgroups most of
  // their pass-0 atomics, which contend on the same bins of the row.
  uint32_t tb = 0;
  {
    for (int i = t; i < kHistWords / 4; i += kMainThreads) reinterpret_cast<uint4*>(hist)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    if (t < nb) {
      const uint4 h = load_dev16(dev_rsrc(rs + row_pub_off(slab), 16u * (uint32_t)nb), 16u * (uint32_t)t);
      if (h.x > 0u && h.y != kNoKeys) {  // count, bound
        atomicAdd(&hist[h.y >> 20], h.x);
        atomicAdd(&hist[kCoarseOff + (h.y >> 26)], h.x);
      }
    }
    __syncthreads();
    const BinThreshold th = wave_threshold(hist, K);
    tb = th.total >= K ? th.bin : 0u;
  }
  uint32_t prefix = 0, need = K;
  uint32_t uses = 0;  // barriers passed (the counters' targets grow by one use each)
#pragma unroll 1
  for (int p = 0; p < 3; ++p) {
    const int shift = p == 0 ? 20 : (p == 1 ? 8 : 0);
    const int bits = p == 2 ? 8 : 12;
    for (int i = t; i < kHistBins / 4; i += kMainThreads) reinterpret_cast<uint4*>(hist)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    for (int i = t; i < nown; i += kMainThreads) {
      const uint32_t k = cs.keys[i];
      if (p == 0 ? (k >> 20) >= tb : (k >> (p == 1 ? 20 : 8)) == prefix)
        atomicAdd(&hist[(k >> shift) & ((1u << bits) - 1u)], 1u);
    }
    __syncthreads();
    dbg_stamp(blockIdx.x, 35 + 4 * p);
    uint32_t* g = p == 0 ? g0 : g12 + (p - 1) * kHistBins;
#pragma unroll
    for (int j = 0; j < kHistBins / kMainThreads; ++j) {
      const int i = t + j * kMainThreads;
      const uint32_t v = hist[i];
      if (v) __hip_atomic_fetch_add(&g[i], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (p == 0)  // passes 1 and 2 start from zero: cleared before anyone adds to them
      for (int i = part(2 * kHistBins, bid, nb) + t; i < part(2 * kHistBins, bid + 1, nb); i += kMainThreads)
        store_dev(&g12[i], 0u);
    counter_barrier(ctr, bid, nb, ++uses, status);
    dbg_stamp(blockIdx.x, 32 + 4 * p);
    {
      // thread t: bins 8t .. 8t + 7; eight threads sum a coarse bin of 64
      static_assert(kHistBins == 8 * kMainThreads, "eight bins per thread");
      const __amdgpu_buffer_rsrc_t r = dev_rsrc(g, 4u * kHistBins);
      const uint4 a = load_dev16(r, 32u * (uint32_t)t), b = load_dev16(r, 32u * (uint32_t)t + 16u);
      reinterpret_cast<uint4*>(hist)[2 * t] = a;
      reinterpret_cast<uint4*>(hist)[2 * t + 1] = b;
      uint32_t v = a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w;
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      if ((t & 7) == 0) hist[kCoarseOff + (t >> 3)] = v;
    }
    __syncthreads();
    dbg_stamp(blockIdx.x, 33 + 4 * p);
    // the row holds >= need keys with this prefix, so the bin exists
    const BinThreshold th = wave_threshold(hist, need);
    prefix = (prefix << bits) | th.bin;
    need -= th.above;
    dbg_stamp(blockIdx.x, 34 + 4 * p);
    __syncthreads();  // hist is cleared next
    // the whole bin is taken: every key >= its lower edge is selected, the
    // rest is not, so t* = edge - 1 with no ties to take (every workgroup
    // sees the same sums and stops alike).  The edge is > 0: the lowest bin
    // of a pass cannot hold the row's last K keys of more than K.
    const uint32_t edge = prefix << shift;
    if (th.cnt == need && edge > 0u) {
      prefix = edge - 1u;
      need = 0u;
      break;
    }
  }
  RadixSel r{prefix, need, 0u, 0u, 0u, 0u, 0u};
  uint32_t gt = 0, eq = 0;
  for (int i = t; i < nown; i += kMainThreads) {
    const uint32_t k = cs.keys[i];
    gt += (k > prefix && key_is_finite(k)) ? 1u : 0u;
    eq += (need && k == prefix) ? 1u : 0u;
  }
  const uint4 c = block_reduce4<0, 0, 0, 0>(make_uint4(gt, eq, 0u, 0u), cs.wave_tmp);
  r.own_gt = c.x;
  r.own_eq = c.y;
  static_assert(kCoopKeys < 65536, "packed per-workgroup counts");
  if (t == 0) store_dev(&cnts[bid], c.x | c.y << 16);
  dbg_stamp(blockIdx.x, 44);
  counter_barrier(ctr, bid, nb, ++uses, status);
  dbg_stamp(blockIdx.x, 45);
  {
    // every wave reduces all counts itself (lane l: workgroups l, l + 64, ...)
    const __amdgpu_buffer_rsrc_t cr = dev_rsrc(cnts, 4u * (uint32_t)nb);
    uint32_t sb = 0, tb = 0, sa = 0;
#pragma unroll
    for (int k = 0; k < kCoopMaxBlocks / kWave; ++k) {
      const int j = lane + k * kWave;
      const uint32_t w = load_dev4(cr, 4u * (uint32_t)j);  // 0 past nb
      sb += j < bid ? (w & 0xffffu) : 0u;
      tb += j < bid ? (w >> 16) : 0u;
      sa += w & 0xffffu;
    }
    r.sel_before = wave_reduce<0>(sb);
    r.ties_before = wave_reduce<0>(tb);
    r.sel_above = wave_reduce<0>(sa);
  }
  dbg_stamp(blockIdx.x, 46);
  // every workgroup has read the pass-0 histogram: clear this one's share
  for (int i = part(kHistBins, bid, nb) + t; i < part(kHistBins, bid + 1, nb); i += kMainThreads) store_dev(&g0[i], 0u);
  dbg_stamp(blockIdx.x, 47);
  return r;
}

// Published-list form of the cooperative select (the default).  Each scan
// workgroup of the row publishes every own key >= its bound lo_b (at most P
// keys, the list's capacity; lo_b = 0 when it holds at most P), zero-padded,
// in its stride of the row's list area, and a header {count, lo_b, finite
// count, max key} (the padding is below every real key: the smallest, -inf,
// is 0x007fffff).  lo_b is the lower edge of the 12-bit bin holding the
// workgroup's M-th key when that whole bin fits, else the exact smallest key
// value with at most P own keys at or above it.
// After ONE group barrier every workgroup reads all lists and, from them
// alone, finds the exact K-th key t* of their union and the ties to take.
// The union holds every key >= t* of the row when it holds at least K keys
// >= L = the largest bound (then t* >= L); the workgroups check that (they
// all see the same lists, so they agree) and otherwise run the cooperative
// radix select over the keys they hold (coop_radix) for t* and the offsets.
// From the lists, the offsets follow from the lists of the workgroups
// before this one.  Each workgroup then writes its own selected positions
// (KV slots) in position order.
// Expects, from the scan: the own keys in cs.keys (position order), their
// fine and coarse histograms, and cs.wstat.
// pts: this workgroup's page-table entries from page pg0 on (in LDS) when
// pts_lds, else the row's page table is read from memory.
// NU: uint4s of the union each thread holds (thread t: t, t + 512, ...);
// past the union they read as 0, below every bound, so every per-entry loop
// runs NU times without a guard.
template <bool TOPK, int NU>
__device__ __forceinline__ void coop_select(CoopShared& cs, unsigned char* smem, const ScanArgs& S, int bid,
                                            int nb, int len, int p_lo, int p_hi, uint32_t* rs,
                                            const float* srow, const int* pt_row, int* o, const int* pts,
                                            int pg0, bool pts_lds) {
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = wave_id();
  const int K = S.topk;
  const bool all = len <= K;
  const int nown = max(0, p_hi - p_lo);
  // list stride and target: from the launcher when every row has the same
  // workgroup count (two divisions fewer on this path), else per row
  const int P = S.pub_stride ? S.pub_stride : pub_stride(nb, K);
  const uint32_t M = (uint32_t)min(S.pub_stride ? S.pub_target : pub_target(nb, K), P);
  uint32_t* ghdr = rs + row_pub_off(S.slab_stride);  // [nb][kPubHdr]
  uint32_t* gpub = ghdr + kPubHdrWords;              // [nb][P] keys, zero-padded
  uint32_t* sync = rs + row_sync_off(S.slab_stride);
  const int dbk = blockIdx.x;

  uint32_t fin_own = 0, kmax_own = 0;  // reduced per wave by the scan
#pragma unroll
  for (int w = 0; w < kMainWaves; ++w) {
    fin_own += cs.wstat[2 * w];
    kmax_own = max(kmax_own, cs.wstat[2 * w + 1]);
  }

  // ---- own bound lo_b and the list's count ----
  uint32_t lo_b = 0, cnt = 0;
  if (all) {
    lo_b = kNoKeys;  // nothing to publish but the finite count
  } else if ((uint32_t)nown <= (uint32_t)P) {
    cnt = (uint32_t)nown;  // every own key
  } else {
    const BinThreshold th = wave_threshold(cs.scan.hist, M);
    if (th.above + th.cnt <= (uint32_t)P) {
      lo_b = th.bin << 20;  // the whole bin fits
      cnt = th.above + th.cnt;
    } else if (th.cnt > 256u) {
      lo_b = next_bin_key(th.bin);
      cnt = th.above;
    } else {
      // the bin split by the next 8 key bits: the bound is the lowest
      // sub-bin edge with #{own >= edge} <= P (each wave the same).  Every
      // own key >= the edge is listed, as the list requires.
      uint32_t* sub = cs.ck;  // 256 counters; the candidates come later
      if (t < 256) sub[t] = 0u;
      __syncthreads();
      // four keys' loads in flight before their counts
      for (int i = t; i < nown; i += 4 * kMainThreads) {
        uint32_t kk[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) kk[u] = i + u * kMainThreads < nown ? cs.keys[i + u * kMainThreads] : 0u;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i + u * kMainThreads < nown && (kk[u] >> 20) == th.bin) atomicAdd(&sub[(kk[u] >> 12) & 255u], 1u);
      }
      __syncthreads();
      // lane l: sub-bins 255-4l .. 252-4l, top down
      const uint4 v = reinterpret_cast<const uint4*>(sub)[kWave - 1 - lane];
      const uint32_t a0 = v.w, a1 = v.z, a2 = v.y, a3 = v.x;
      const uint32_t lt = a0 + a1 + a2 + a3;
      const uint32_t c0 = wave_scan_incl<0>(lt) - lt + a0, c1 = c0 + a1, c2 = c1 + a2, c3 = c2 + a3;
      const uint32_t room = (uint32_t)P - th.above;
      const uint32_t n_ok = wave_reduce<0>((c0 <= room ? 1u : 0u) + (c1 <= room ? 1u : 0u) +
                                           (c2 <= room ? 1u : 0u) + (c3 <= room ? 1u : 0u));
      const uint32_t got = wave_reduce<2>(c3 <= room ? c3 : (c2 <= room ? c2 : (c1 <= room ? c1 : (c0 <= room ? c0 : 0u))));
      // no sub-bin fits (ties at its top): start above the bin
      lo_b = n_ok ? (th.bin << 20) | ((256u - n_ok) << 12) : next_bin_key(th.bin);
      cnt = th.above + got;
    }
  }

  dbg_stamp(dbk, 25);
  dbg_value(dbk, 27, all ? 9ull : ((uint32_t)nown <= (uint32_t)P ? 3ull : (lo_b == 0u ? 4ull : ((lo_b & 0xfffffu) ? 2ull : 0ull))));
  // ---- publish in position order; the entries' positions stay in LDS
  // (lpos) for the emit, then zero padding, header
  uint16_t* lpos = cs.lpos;  // a list holds <= kPubWords entries
  {
    uint32_t* mine = gpub + (long)bid * P;
    if (!all && lo_b != kNoKeys && nown <= 4 * kMainThreads) {
      // a few positions per thread: thread t takes contiguous positions and
      // one block scan gives it its slots
      const int per = (nown + kMainThreads - 1) / kMainThreads;
      const int i0 = min(nown, t * per), i1 = min(nown, i0 + per);
      uint32_t c = 0;
      for (int i = i0; i < i1; ++i) c += cs.keys[i] >= lo_b ? 1u : 0u;
      uint32_t tot;
      // no closing barrier: wave_tmp is next written after the group barrier
      uint32_t off = block_exclusive_scan<false>(c, cs.wave_tmp, &tot);  // tot == cnt
      dbg_stamp(dbk, 26);
      for (int i = i0; i < i1; ++i) {
        const uint32_t k = cs.keys[i];
        if (k >= lo_b) {
          const uint32_t slot = min(off++, (uint32_t)P - 1u);  // < cnt <= P by construction
          lpos[slot] = (uint16_t)i;
          store_dev(&mine[slot], k);
        }
      }
    } else if (!all && lo_b != kNoKeys) {
      // many positions: wave w takes the contiguous positions [w * seg,
      // (w + 1) * seg) in steps of 256 (lane l: positions 4l .. 4l + 3 of
      // the step, one 16-byte LDS read; every step's read issued at once),
      // orders its entries by lane within a step (a wave scan) and places
      // them after those of the waves before it.  (Thread-contiguous runs of
      // this length cost one dependent LDS round trip per position.)
      constexpr int kStep = 4 * kWave, kSteps = kCoopKeys / (kMainWaves * kStep);
      static_assert(kSteps * kMainWaves * kStep == kCoopKeys, "publish steps cover the own keys");
      const int seg = (nown + kMainWaves * kStep - 1) / (kMainWaves * kStep) * kStep;
      const int w0 = min(nown, wv * seg), w1 = min(nown, w0 + seg);  // wave-uniform
      const uint4* k4 = reinterpret_cast<const uint4*>(cs.keys);
      uint4 kv[kSteps];
      uint32_t sel[kSteps];  // bit e: position 4 * lane + e of the step is listed
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        const int i = w0 + st * kStep + 4 * lane;
        kv[st] = k4[(i < kCoopKeys ? i : 0) >> 2];  // in bounds; masked below
      }
      uint32_t c = 0;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        const int i = w0 + st * kStep + 4 * lane;
        const uint32_t w4[4] = {kv[st].x, kv[st].y, kv[st].z, kv[st].w};
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) m |= (i + e < w1 && w4[e] >= lo_b) ? 1u << e : 0u;
        sel[st] = m;
        c += (uint32_t)__popc(m);
      }
      c = wave_reduce<0>(c);
      // no closing barrier: wave_tmp is next written after the group barrier
      if (lane == 0) cs.wave_tmp[wv] = c;
      __syncthreads();
      uint32_t off = 0;
#pragma unroll
      for (int w = 0; w < kMainWaves; ++w) off += w < wv ? cs.wave_tmp[w] : 0u;
      dbg_stamp(dbk, 26);
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        if (w0 + st * kStep >= w1) break;  // uniform
        const uint32_t n = (uint32_t)__popc(sel[st]);
        const uint32_t incl = wave_scan_incl<0>(n);
        uint32_t slot = off + incl - n;
        const int i = w0 + st * kStep + 4 * lane;
        const uint32_t w4[4] = {kv[st].x, kv[st].y, kv[st].z, kv[st].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (sel[st] & (1u << e)) {
            const uint32_t sl = min(slot++, (uint32_t)P - 1u);  // < cnt <= P by construction
            lpos[sl] = (uint16_t)(i + e);
            store_dev(&mine[sl], w4[e]);
          }
        off += (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
      }
    }
    if (!all)
      for (int i = (int)cnt + t; i < P; i += kMainThreads) store_dev(&mine[i], 0u);
    if (t < kPubHdr) {
      const uint32_t v = t == 0 ? cnt : (t == 1 ? lo_b : (t == 2 ? fin_own : (cnt ? kmax_own : 0u)));
      store_dev(&ghdr[bid * kPubHdr + t], v);
    }
  }
  dbg_stamp(dbk, 8);
  group_arrive_rep(sync, sync + 3 * kSyncWords, bid, nb, cs.sense[0]);
  // while the other workgroups arrive: clear what the union steps count
  // (the scan's histogram is no longer needed)
  static_assert(kUnionWords % 4 == 0 && kUnionWords <= 8 * kMainThreads, "union histogram clear");
  for (int i = t; i < kUnionWords / 4; i += kMainThreads)
    reinterpret_cast<uint4*>(cs.scan.hist)[i] = make_uint4(0, 0, 0, 0);
  if (t < kWave) cs.ck[t] = 0u;  // candidates past the count read as 0
  if (t == 0) cs.misc[1] = 0u;
  // a list of at most one wave's entries is emitted by wave 0 (below): its
  // lane l takes entry l, whose key and output slot are read now
  const auto slot_of = [&](int p) {  // a position, or its KV slot when there is a page table
    if (TOPK && !pt_row) return p;
    return (pts_lds ? pts[(p >> 6) - pg0] : pt_row[p >> 6]) * DSA_PAGE_TOKENS + (p & (DSA_PAGE_TOKENS - 1));
  };
  const bool wave_emit = !all && cnt <= (uint32_t)kWave;
  uint32_t em_key = 0;
  int em_slot = 0;
  if (wave_emit && wv == 0 && lane < (int)cnt) {
    const int i = (int)lpos[lane];
    em_key = cs.keys[i];
    em_slot = slot_of(p_lo + i);
  }
  group_wait_rep(sync, sync + 3 * kSyncWords, bid, nb, cs.sense[0], rs + radix_sync_off(S.slab_stride, (cs.sense[0] & 1u) ^ 1u),
                 2 * kRadixGroups);
  dbg_stamp(dbk, 9);

  // ---- every workgroup: all lists into registers (one batch of
  // device-scope loads; thread t holds uint4s t, t + 512, ... of the area);
  // every wave loads all headers (lane l: l, l + 64, ...) and reduces them
  // itself, so no block step is needed ----
  const int nent = all ? 0 : nb * P;
  constexpr int kU = NU;
  static_assert(NU * 4 * kMainThreads <= kPubWords, "union registers");
  static_assert(kCoopMaxBlocks <= 4 * kWave, "headers: 4 per lane");
  uint4 u[kU];
  uint32_t h0 = 0, h1 = 0;
  {
    const __amdgpu_buffer_rsrc_t r = dev_rsrc(gpub, 4u * (uint32_t)nent);
    const __amdgpu_buffer_rsrc_t hr = dev_rsrc(ghdr, 16u * (uint32_t)nb);
    uint4 h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = load_dev16(hr, 16u * (uint32_t)(lane + k * kWave));  // 0 past nb
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int i = t + j * kMainThreads;
      u[j] = load_dev16(r, 16u * i);  // 0 past the end of the resource
    }
    // all: (finite keys of the lists before this one, of all lists);
    // else: (largest bound, largest key)
    uint32_t a = 0, b = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = lane + k * kWave;
      a = all ? a + (j < bid ? h[k].z : 0u) : max(a, h[k].y);
      b = all ? b + h[k].z : max(b, h[k].w);
    }
    h0 = all ? wave_reduce<0>(a) : wave_reduce<2>(a);
    h1 = all ? wave_reduce<0>(b) : wave_reduce<2>(b);
  }
  dbg_stamp(dbk, 10);
  // f(word, union index) over this thread's words (zeros past the end: below
  // every bound)
  const auto for_mine = [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const uint32_t e = 4u * (uint32_t)(t + j * kMainThreads);
      f(u[j].x, e);
      f(u[j].y, e + 1u);
      f(u[j].z, e + 2u);
      f(u[j].w, e + 3u);
    }
  };

  uint32_t tstar = 0, need3 = 0;
  bool radix = false;  // t* from the cooperative radix select: every own key is a candidate
  uint32_t radix_own = 0;  // then: this workgroup's selected keys
  // sel_before = selected above t* before this workgroup, ties_before = ties
  // before it, sel_above = all selected above t*; all: finite counts
  uint32_t sel_before = 0, ties_before = 0, sel_above = 0;
  const uint32_t mine0 = (uint32_t)(bid * P);
  if (all) {
    sel_before = h0;
    sel_above = h1;
  } else {
    // t* must be >= L = the largest list bound for the lists to hold every
    // key >= t*; keys below L never matter.
    const uint32_t lo = max(h0, kKeyNegInf), hi = h1;
    bool ok = hi >= lo;
    uint32_t T1 = 0, above = 0, nbin = 0;
    int sh = 0;
    if (ok) {
      // a bit window over [lo, hi], anchored at lo: bin (w - lo) >> sh,
      // (hi - lo) >> sh < kUnionBins (the finer the bins, the fewer keys
      // share the threshold bin)
      {
        const uint32_t d = hi - lo;
        sh = d < (uint32_t)kUnionBins ? 0 : 32 - __builtin_clz(d) - 11;
      }
      static_assert(kUnionBins == 2048, "the window shift keeps 11 bits");
      uint32_t* hist = cs.scan.hist;
      // branch-free: keys below lo land in spill bins past the histogram
      // (a spill word per lane: the lanes' atomics never collide)
      const uint32_t spill = kUnionWords + (uint32_t)(t & (kWave - 1));
      for_mine([&](uint32_t w, uint32_t) { atomicAdd(&hist[w >= lo ? union_slot((w - lo) >> sh) : spill], 1u); });
      __syncthreads();
      dbg_stamp(dbk, 12);
      const BinThreshold th = wave_threshold_sum<kUnionGroup, kUnionStride>(hist, (uint32_t)K);
      ok = th.total >= (uint32_t)K;  // the union holds at least K keys >= lo
      T1 = th.bin;                   // == (t* - lo) >> sh
      above = th.above;
      nbin = th.cnt;
    }
    dbg_stamp(dbk, 4);
    if (!ok) {
      // the lists cannot decide (every workgroup sees the same lists, so
      // all of them come here): the cooperative radix select over the keys
      // the workgroups hold
      const RadixSel rr = coop_radix(cs, rs, S.slab_stride, bid, nb, nown, (uint32_t)K, cs.sense[0] & 1u);
      tstar = rr.tstar;
      need3 = rr.need3;
      sel_before = rr.sel_before;
      ties_before = rr.ties_before;
      sel_above = rr.sel_above;
      radix_own = rr.own_gt + (key_is_finite(tstar) ? min(rr.own_eq, need3 - min(ties_before, need3)) : 0u);
      radix = true;
    } else {
    // pass 2: finite keys above T1's bin are selected: count them (and
    // those of the lists before this one; a list is a whole number of
    // uint4s); T1's bin -> candidates.  Edges: bin > T1 <=> w > top, and
    // bin == T1 <=> bot <= w <= top.
    const uint64_t top64 = (uint64_t)lo + (((uint64_t)T1 + 1u) << sh) - 1u;
    const uint32_t top = top64 > 0xffffffffull ? 0xffffffffu : (uint32_t)top64;
    const uint32_t bot = lo + (T1 << sh);
    uint32_t ax = 0, az = 0, cmask = 0;
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const bool before = 4u * (uint32_t)(t + j * kMainThreads) < mine0;
      const uint32_t w4[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
      uint32_t gj = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        gj += (w4[c] > top && w4[c] < kKeyPosInf) ? 1u : 0u;
        cmask |= (w4[c] >= bot && w4[c] <= top) ? (1u << (4 * j + c)) : 0u;
      }
      az += gj;
      ax += before ? gj : 0u;
    }
    dbg_stamp(dbk, 13);
    if (__ballot(cmask != 0)) {  // rare: most waves hold no candidate
      for (uint32_t m = cmask; m; m &= m - 1u) {
        const int b = __builtin_ctz(m);
        const int j = b >> 2, c = b & 3;
        const uint32_t e = 4u * (uint32_t)(t + j * kMainThreads) + (uint32_t)c;
        uint32_t w = 0;
#pragma unroll
        for (int jj = 0; jj < kU; ++jj)
          if (jj == j) w = c == 0 ? u[jj].x : (c == 1 ? u[jj].y : (c == 2 ? u[jj].z : u[jj].w));
        const uint32_t slot = atomicAdd(&cs.misc[1], 1u);
        if (slot < (uint32_t)kCoopCand) {
          cs.ck[slot] = w;
          cs.ce[slot] = e;
        }
      }
    }
    dbg_stamp(dbk, 6);
    // both counts in one reduction: each is at most the union's size
    // (<= kPubWords < 2^16)
    static_assert(kPubWords < 65536, "packed union counts");
    const uint32_t axz = wave_reduce<0>(ax | az << 16);
    if (lane == 0) cs.pred[wv] = axz;
    __syncthreads();
    dbg_stamp(dbk, 7);
#pragma unroll
    for (int w = 0; w < kMainWaves; ++w) {
      const uint32_t v = cs.pred[w];
      sel_before += v & 0xffffu;
      sel_above += v >> 16;
    }
    const uint32_t nc = nbin;                   // == the candidates collected
    // (value slot 27 holds the bound path)
    const uint32_t need = (uint32_t)K - above;  // 1 <= need <= nc
    if (nc <= (uint32_t)kWave) {
      // each wave: exact t* by rank counting (the candidate c with
      // #{> c} < need <= #{>= c}) and the candidates' share of the offsets
      const bool in = lane < (int)nc;
      const uint32_t c = in ? cs.ck[lane] : 0u;
      const uint32_t e = in ? cs.ce[lane] : 0u;
      uint32_t gtc = 0, gec = 0;
      const uint4* c4 = reinterpret_cast<const uint4*>(cs.ck);  // zero past nc: below every candidate
      const int nq = ((int)nc + 3) >> 2;
#pragma unroll 4
      for (int q = 0; q < nq; ++q) {
        const uint4 x = c4[q];
        gtc += (x.x > c ? 1u : 0u) + (x.y > c ? 1u : 0u) + (x.z > c ? 1u : 0u) + (x.w > c ? 1u : 0u);
        gec += (x.x >= c ? 1u : 0u) + (x.y >= c ? 1u : 0u) + (x.z >= c ? 1u : 0u) + (x.w >= c ? 1u : 0u);
      }
      const int l = __builtin_ctzll(__ballot(in && gtc < need && need <= gec));
      tstar = (uint32_t)__builtin_amdgcn_readlane((int)c, l);
      need3 = need - (uint32_t)__builtin_amdgcn_readlane((int)gtc, l);
      const bool g = in && c > tstar && key_is_finite(c);
      const bool tie = in && c == tstar;
      const bool before = e < mine0;
      sel_before += (uint32_t)__popcll(__ballot(g && before));
      ties_before = (uint32_t)__popcll(__ballot(tie && before));
      sel_above += (uint32_t)__popcll(__ballot(g));
    } else {
      if (nc <= (uint32_t)kCoopCand) {
        // rank counting in 16-byte broadcast reads: pad the last uint4 with
        // 0 (below every candidate)
        if (t < 3 && nc + (uint32_t)t < (uint32_t)kCoopCand) cs.ck[nc + t] = 0u;
        __syncthreads();
        const uint4* c4 = reinterpret_cast<const uint4*>(cs.ck);
        const int nq = ((int)nc + 3) >> 2;
        for (uint32_t j = t; j < nc; j += kMainThreads) {
          const uint32_t c = cs.ck[j];
          uint32_t gtc = 0, gec = 0;
#pragma unroll 4
          for (int q = 0; q < nq; ++q) {
            const uint4 x = c4[q];
            gtc += (x.x > c ? 1u : 0u) + (x.y > c ? 1u : 0u) + (x.z > c ? 1u : 0u) + (x.w > c ? 1u : 0u);
            gec += (x.x >= c ? 1u : 0u) + (x.y >= c ? 1u : 0u) + (x.z >= c ? 1u : 0u) + (x.w >= c ? 1u : 0u);
          }
          if (gtc < need && need <= gec) {
            cs.res[0] = c;
            cs.res[1] = need - gtc;
          }
        }
        __syncthreads();
        tstar = cs.res[0];
        need3 = cs.res[1];
      } else {
        // many keys share T1's bin: refine its low sh bits, <= 10 per level
        uint32_t* hist = cs.scan.hist;
        uint32_t prefix = T1, nd = need;
        int s2 = sh;
        while (s2 > 0) {
          const int sub = min(10, s2);
          s2 -= sub;
          for (int i = t; i < kNB2; i += kMainThreads) hist[i] = 0u;
          __syncthreads();
          const int hs = s2 + sub;
          for_mine([&](uint32_t w, uint32_t) {
            if (w >= lo && ((w - lo) >> hs) == prefix) atomicAdd(&hist[((w - lo) >> s2) & ((1u << sub) - 1u)], 1u);
          });
          __syncthreads();
          find_threshold_fixed<kNB2, kMainThreads>(hist, nd, cs.wave_tmp, cs.res);
          prefix = (prefix << sub) | cs.res[0];
          nd -= cs.res[1];
        }
        tstar = lo + prefix;
        need3 = nd;
      }
      // the bin-T1 keys' share (keys above the bin were counted in pass 2)
      uint4 acc = make_uint4(0, 0, 0, 0);
      const auto count = [&](uint32_t w, uint32_t e) {
        const bool g = w > tstar && key_is_finite(w);
        const bool before = e < mine0;
        acc.x += (g && before) ? 1u : 0u;
        acc.y += (w == tstar && before) ? 1u : 0u;
        acc.z += g ? 1u : 0u;
      };
      if (nc <= (uint32_t)kCoopCand) {
        for (uint32_t j = t; j < nc; j += kMainThreads) count(cs.ck[j], cs.ce[j]);
      } else {
        for_mine([&](uint32_t w, uint32_t e) {
          if (w >= lo && ((w - lo) >> sh) == T1) count(w, e);
        });
      }
      const uint4 r = block_reduce4<0, 0, 0, 0>(acc, cs.wave_tmp);
      sel_before += r.x;
      ties_before = r.y;
      sel_above += r.z;
    }
    }  // the lists decide
    dbg_stamp(dbk, 15);
  }
  const bool tfin = !all && key_is_finite(tstar);
  const uint32_t base = sel_before + (tfin ? min(ties_before, need3) : 0u);
  const uint32_t nsel = sel_above + (tfin ? need3 : 0u);
  dbg_stamp(dbk, 14);

  // ---- emit own selections in position order.  Every selected key is in
  // this workgroup's list (it is >= t* >= every list bound), which holds the
  // entries in position order: thread t takes contiguous entries.  A row of
  // <= K tokens publishes nothing and takes every finite key instead. ----
  const bool walk_own = all || radix;  // the entries are all own keys, not the list
  const int n_e = walk_own ? nown : (int)cnt;
  if (wave_emit && !radix) {
    // a list of at most one wave's entries: wave 0 emits it, ranks by ballot
    if (wv == 0) {
      const bool in = lane < n_e;
      const uint32_t k = em_key;
      const uint64_t below = (1ull << lane) - 1ull;
      const bool tie = in && tfin && k == tstar;
      const uint32_t tr = ties_before + (uint32_t)__popcll(__ballot(tie) & below);
      const bool sel = in && key_is_finite(k) && (k > tstar || (tie && tr < need3));
      const uint32_t pos = base + (uint32_t)__popcll(__ballot(sel) & below);
      if (sel) o[min(pos, (uint32_t)K - 1u)] = em_slot;  // < K by construction
    }
    if (bid == nb - 1)
      for (int j = (int)nsel + t; j < K; j += kMainThreads) o[j] = TOPK ? S.pad : -1;
    dbg_stamp(dbk, 11);
    return;
  }
  if (radix && radix_own == 0u) {  // nothing of this workgroup's is selected
    if (bid == nb - 1)
      for (int j = (int)nsel + t; j < K; j += kMainThreads) o[j] = TOPK ? S.pad : -1;
    return;
  }
  const int per = (n_e + kMainThreads - 1) / kMainThreads;
  const int e0 = min(n_e, t * per), e1 = min(n_e, e0 + per);
  const auto entry = [&](int e) { return walk_own ? e : (int)lpos[e]; };  // -> own position index
  // The thread's entries in blocks of kEmitRegs, every LDS read of a block
  // issued unconditionally (so all are in flight together); past e1 an
  // entry reads key 0 (below every key: never selected, never a tie).
  const int e_last = max(e1 - 1, 0);
  const auto load_blk = [&](int eb, int (&ii)[kEmitRegs], uint32_t (&kk)[kEmitRegs]) {
#pragma unroll
    for (int j = 0; j < kEmitRegs; ++j) ii[j] = min(entry(min(eb + j, e_last)), kCoopKeys - 1);
#pragma unroll
    for (int j = 0; j < kEmitRegs; ++j) {
      const uint32_t k = cs.keys[ii[j]];
      kk[j] = eb + j < e1 ? k : 0u;
    }
  };
  // output slots of a block, read unconditionally (page entries of the
  // workgroup's own pages; a position clamped into the row), so that the
  // stores after them need not wait for one another
  const auto slots_blk = [&](const int (&ii)[kEmitRegs], int (&sl)[kEmitRegs]) {
    if (TOPK && !pt_row) {
#pragma unroll
      for (int j = 0; j < kEmitRegs; ++j) sl[j] = p_lo + ii[j];
    } else if (pts_lds) {
#pragma unroll
      for (int j = 0; j < kEmitRegs; ++j) {
        const int p = p_lo + ii[j];
        sl[j] = pts[min((p >> 6) - pg0, kScanMaxPages - 1)] * DSA_PAGE_TOKENS + (p & (DSA_PAGE_TOKENS - 1));
      }
    } else {
#pragma unroll
      for (int j = 0; j < kEmitRegs; ++j) {
        const int p = min(p_lo + ii[j], S.pt_stride * DSA_PAGE_TOKENS - 1);
        sl[j] = pt_row[p >> 6] * DSA_PAGE_TOKENS + (p & (DSA_PAGE_TOKENS - 1));
      }
    }
  };
  // tr: the rank among the row's ties at t* of the next tie seen
  const auto is_sel = [&](uint32_t k, uint32_t& tr) {
    const bool tie = tfin && k == tstar;
    const bool sel = key_is_finite(k) && (all || k > tstar || (tie && tr < need3));
    tr += tie ? 1u : 0u;
    return sel;
  };
  // pass 1: the thread's keys above t* and ties at t*; ONE block scan of
  // both (packed: each count < 2^16) gives the output position: the keys
  // above t* before this thread plus the ties selected before it (ties are
  // taken in rank order, the first need3 of the row)
  int ii[kEmitRegs], sl[kEmitRegs];
  uint32_t kk[kEmitRegs];
#pragma unroll
  for (int j = 0; j < kEmitRegs; ++j) ii[j] = 0, kk[j] = 0u;
  uint32_t ngt = 0, nt = 0;
  for (int eb = e0; eb < e1; eb += kEmitRegs) {
    load_blk(eb, ii, kk);
#pragma unroll
    for (int j = 0; j < kEmitRegs; ++j) {
      ngt += (key_is_finite(kk[j]) && (all || kk[j] > tstar)) ? 1u : 0u;
      nt += (tfin && kk[j] == tstar) ? 1u : 0u;
    }
  }
  const bool one = per <= kEmitRegs;  // uniform: the block is still in registers
  if (one && e0 < e1) slots_blk(ii, sl);
  dbg_stamp(dbk, 32);
  static_assert(kCoopKeys < 65536, "packed emit counts");
  uint32_t tot;
  const uint32_t pk = block_exclusive_scan(ngt | nt << 16, cs.wave_tmp, &tot);
  dbg_stamp(dbk, 34);
  uint32_t tr = ties_before + (pk >> 16);
  uint32_t pos = sel_before + (pk & 0xffffu) + (tfin ? min(tr, need3) : 0u);
  if (one) {
#pragma unroll
    for (int j = 0; j < kEmitRegs; ++j)
      if (is_sel(kk[j], tr)) o[min(pos++, (uint32_t)K - 1u)] = sl[j];  // < K by construction
  } else {
    for (int eb = e0; eb < e1; eb += kEmitRegs) {
      load_blk(eb, ii, kk);
      slots_blk(ii, sl);
#pragma unroll
      for (int j = 0; j < kEmitRegs; ++j)
        if (is_sel(kk[j], tr)) o[min(pos++, (uint32_t)K - 1u)] = sl[j];  // < K by construction
    }
  }
  dbg_stamp(dbk, 35);
  if (bid == nb - 1)
    for (int j = (int)nsel + t; j < K; j += kMainThreads) o[j] = TOPK ? S.pad : -1;
  dbg_stamp(dbk, 11);
}

template <int VARIANT>
__device__ __forceinline__ v4f qk_fp8(const v8i& qa, const v8i& kb) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (VARIANT == 0) {
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa, kb, acc, 0, 0, 0, 0, 0, 0);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long a = ((long)(uint32_t)qa[2 * j]) | ((long)(uint32_t)qa[2 * j + 1] << 32);
      const long bb = ((long)(uint32_t)kb[2 * j]) | ((long)(uint32_t)kb[2 * j + 1] << 32);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, bb, acc, 0, 0, 0);
    }
  }
  return acc;
}

// The single-workgroup select of one row over its scores in memory: the
// cooperative select's fallback (its lists could not decide, e.g. many equal
// scores) and the select of rows the cooperative one does not take.  Exact
// top-K by rank key, ties to the lower position, the same rule as
// coop_select: t* by three radix passes over the row's keys (bits 31-21,
// 20-10, 9-0; an LDS histogram each), then one pass in position order that
// writes every finite key above t* and the lowest-position ties at t* (KV
// slots through the page table; positions when TOPK has none), pads after.
// It reads the row four times; compact on purpose (it shares the kernel's
// registers with the common path).
constexpr int kRowSelWords = 2048 + 4 * 8 + 4;  // LDS words select_row uses
template <bool TOPK>
__device__ __forceinline__ void select_row(unsigned char* smem, const float* srow, int len, const int* pt_row,
                                           int* o, int K, int pad) {
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem);
  uint32_t* wtmp = hist + 2048;
  uint32_t* res = wtmp + 4 * 8;
  const int t = threadIdx.x;
  constexpr int kT = kMainThreads, kB = 8;  // loads in flight per thread
  const __amdgpu_buffer_rsrc_t sr = dev_rsrc(srow, 4u * (uint32_t)max(len, 0));
  uint32_t tstar = 0, need = 0;  // need: ties at t* to take
  if (len > K) {
    need = (uint32_t)K;
    uint32_t prefix = 0;
    for (int p = 0; p < 3; ++p) {
      const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0), bits = p == 2 ? 10 : 11;
      for (int i = t; i < 2048; i += kT) hist[i] = 0u;
      __syncthreads();
      for (int i0 = 0; i0 < len; i0 += kB * kT) {
        uint32_t k[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int i = i0 + j * kT + t;
          k[j] = rank_key(__uint_as_float(load_dev4(sr, i < len ? 4u * (uint32_t)i : 0xfffffffcu)));
        }
#pragma unroll
        for (int j = 0; j < kB; ++j)
          if (i0 + j * kT + t < len && (p == 0 || (k[j] >> (sh + bits)) == prefix))
            atomicAdd(&hist[(k[j] >> sh) & ((1u << bits) - 1u)], 1u);
      }
      __syncthreads();
      find_threshold(hist, 1 << bits, need, wtmp, res);
      prefix = (prefix << bits) | res[0];
      need -= res[1];
      __syncthreads();
    }
    tstar = prefix;
  }
  // position order: thread t takes positions [i0 + kB t, +kB) of each round
  uint32_t run_sel = 0, run_tie = 0;
  for (int i0 = 0; i0 < len; i0 += kB * kT) {
    uint32_t k[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int i = i0 + kB * t + j;
      k[j] = rank_key(__uint_as_float(load_dev4(sr, i < len ? 4u * (uint32_t)i : 0xfffffffcu)));
    }
    uint32_t nt = 0;
#pragma unroll
    for (int j = 0; j < kB; ++j) nt += (len > K && i0 + kB * t + j < len && k[j] == tstar) ? 1u : 0u;
    uint32_t tie_tot;
    uint32_t tr = run_tie + block_exclusive_scan(nt, wtmp, &tie_tot);
    uint32_t ns = 0;
    bool sel[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const bool in = i0 + kB * t + j < len;
      const bool tie = len > K && in && k[j] == tstar;
      sel[j] = in && key_is_finite(k[j]) && (len <= K || k[j] > tstar || (tie && tr < need));
      tr += tie ? 1u : 0u;
      ns += sel[j] ? 1u : 0u;
    }
    uint32_t sel_tot;
    uint32_t pos = run_sel + block_exclusive_scan(ns, wtmp, &sel_tot);
#pragma unroll
    for (int j = 0; j < kB; ++j)
      if (sel[j]) {
        const int i = i0 + kB * t + j;
        o[min(pos++, (uint32_t)K - 1u)] =
            (TOPK && !pt_row) ? i : pt_row[i >> 6] * DSA_PAGE_TOKENS + (i & (DSA_PAGE_TOKENS - 1));
      }
    run_sel += sel_tot;
    run_tie += tie_tot;
  }
  for (int j = (int)run_sel + t; j < K; j += kT) o[j] = pad;
}


// FROM_SCORES: the row's scores are already in the slab (a plain scan
// launch wrote them); the workgroup loads its positions' scores instead of
// scoring the keys, then selects as usual.
// LISTS: the cooperative select's union registers, 4 or 8 uint4s per thread
// when the launch fixes one size for every row, 0 for both (chosen per row)
template <int NHG, int VARIANT, bool SELECT, bool FROM_SCORES = false, bool TOPK = false, int LISTS = 0>
__device__ __forceinline__ void scan_block(const ScanArgs& S, int row, int bid, int nb, unsigned char* smem) {
  constexpr int kHeads = NHG * 16;
  ScanShared& sh = *reinterpret_cast<ScanShared*>(smem);
  const int t = threadIdx.x;
  const bool with_hist = S.hist != nullptr;
  const int dbk = blockIdx.x;
  dbg_stamp(dbk, 0);
  dbg_hw_ids();
  const int cap = min(S.slab_stride, S.pt_stride * DSA_PAGE_TOKENS);
  // TOPK (the standalone top-k over given scores): no page table means the
  // output is positions
  const int* pt_row = (TOPK && !S.page_table) ? nullptr : S.page_table + (long)row * S.pt_stride;
  const bool has_pt = !TOPK || pt_row != nullptr;
  // The page-table entries of this workgroup's chunks are prefetched with the
  // query, speculating that the row is full (len == cap, the usual decode
  // case) so the prefetch need not wait for seq_lens; a shorter row reloads.
  const int ncap = (cap + kChunkKeys - 1) / kChunkKeys;
  const int sc0 = part(ncap, bid, nb), sc1 = part(ncap, bid + 1, nb);
  const int spg0 = sc0 >> 2;
  const int snpg = (sc1 > sc0) ? ((sc1 - 1) >> 2) - spg0 + 1 : 0;
  // the row barriers' flag values (flipped once per use), loaded first and
  // stored to LDS in this prologue: held in a register until the select, the
  // load made the scan's end wait for every load and store the scan issued
  // (the wait counter counts in issue order, stores included)
  uint32_t sense = 0;
  if (S.coop && t < kNumSync)
    sense = group_sense(S.hist + (long)row * S.hist_row_words + row_sync_off(S.slab_stride) + t * kSyncWords,
                        bid);
  constexpr int kQ = FROM_SCORES ? 0 : kHeads * DSA_INDEX_DIM / 16;  // uint4 of the query block
  const uint4* qsrc = reinterpret_cast<const uint4*>(S.q8 + (long)row * kHeads * DSA_INDEX_DIM);
  uint4 qv = make_uint4(0, 0, 0, 0);
  if (t < kQ) qv = qsrc[t];
  const float wv0 = (!FROM_SCORES && t < kHeads) ? S.w[(long)row * kHeads + t] : 0.f;
  const int spv = (has_pt && snpg <= kMainThreads && t < snpg) ? pt_row[spg0 + t] : 0;
  dbg_stamp(dbk, 28);
  const int len = max(0, min(S.seq_lens[row], cap));
  const int nchunks = (len + kChunkKeys - 1) / kChunkKeys;
  const int c0 = part(nchunks, bid, nb);
  const int c1 = part(nchunks, bid + 1, nb);
  const int pg0 = c0 >> 2;
  const int npg = (c1 > c0) ? ((c1 - 1) >> 2) - pg0 + 1 : 0;
  const bool pts_lds = has_pt && npg <= kScanMaxPages;
  {
    const bool spec_ok = nchunks == ncap && snpg <= kMainThreads;  // then pg0, npg == spg0, snpg
    dbg_stamp(dbk, 29);
    if (t < kQ) reinterpret_cast<uint4*>(sh.qs)[t] = qv;
    dbg_stamp(dbk, 30);
    for (int i = t + kMainThreads; i < kQ; i += kMainThreads) reinterpret_cast<uint4*>(sh.qs)[i] = qsrc[i];
    if (!FROM_SCORES && t < kHeads) sh.ws[t] = wv0;
    if (pts_lds) {
      if (spec_ok) {
        if (t < npg) sh.pts[t] = spv;
      } else {
        for (int i = t; i < npg; i += kMainThreads) sh.pts[i] = pt_row[pg0 + i];
      }
    }
    if (with_hist)
      for (int i = t; i < kHistWords / 4; i += kMainThreads) reinterpret_cast<uint4*>(sh.hist)[i] = make_uint4(0, 0, 0, 0);
    if (S.coop && t < kNumSync) reinterpret_cast<CoopShared*>(smem)->sense[t] = sense;
  }
  float* srow = S.scores + (long)row * S.slab_stride;
  if constexpr (!FROM_SCORES) {  // slab tail past the last scored chunk -> -inf, over the row's blocks
    const long tail0 = (long)nchunks * kChunkKeys;
    const long tail = (long)S.slab_stride - tail0;
    if (tail > 0) {
      const long p0 = tail0 + tail * bid / nb, p1 = tail0 + tail * (bid + 1) / nb;
      for (long p = p0 + t; p < p1; p += kMainThreads) {
        if (S.next_idx) store_dev(&srow[p], -INFINITY);
        else srow[p] = -INFINITY;
      }
    }
  }
  dbg_stamp(dbk, 31);
  __syncthreads();

  dbg_stamp(dbk, 1);
  const int lane = t & (kWave - 1);
  const int wv = wave_id();
  const int kr = lane & 15, kc = lane >> 4;
  uint32_t kmax = 0, nfin = 0;  // own keys (cooperative select)
  if constexpr (FROM_SCORES) {
    // this workgroup's positions [c0*16, min(c1*16, len)), 8 coalesced
    // loads in flight per thread
    const int q_lo = c0 * kChunkKeys, q_n = max(0, min(c1 * kChunkKeys, len) - q_lo);
    const float* src = srow + q_lo;
    constexpr int kB = 8;
    for (int i0 = t; i0 < q_n; i0 += kB * kMainThreads) {
      float v[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int i = i0 + j * kMainThreads;
        v[j] = i < q_n ? src[i] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int i = i0 + j * kMainThreads;
        if (i < q_n) {
          const uint32_t key = rank_key(v[j]);
          atomicAdd(&sh.hist[key >> 20], 1u);
          if (SELECT && S.coop) {  // the coarse bins are summed after the loop
            reinterpret_cast<CoopShared*>(smem)->keys[i] = key;
            kmax = max(kmax, key);
            nfin += key_is_finite(key) ? 1u : 0u;
          }
        }
      }
    }
  } else {
  v8i qa[NHG];
  float wr[NHG][4];
#pragma unroll
  for (int hg = 0; hg < NHG; ++hg) {
    const uint4* p = reinterpret_cast<const uint4*>(sh.qs + (hg * 16 + kr) * DSA_INDEX_DIM + kc * 32);
    const uint4 a = p[0], bq = p[1];
    qa[hg] = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)bq.x, (int)bq.y, (int)bq.z, (int)bq.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) wr[hg][r] = sh.ws[hg * 16 + 4 * kc + r];
  }

  const int n = c1 - c0;
  const int w0 = c0 + (int)((uint32_t)(n * wv) / kMainWaves);
  const int w1 = c0 + (int)((uint32_t)(n * (wv + 1)) / kMainWaves);
  constexpr int kScanBatch = scan_batch<SELECT>();
  // One batch of chunks per step, every load issued before any is used.
  // Branch-free: each chunk reads through a buffer resource over its page
  // (an empty one for a chunk past w1 or an invalid page, so its loads
  // return 0 without a memory access), and the page entries come from LDS,
  // so the compiler can wait for each chunk's loads alone.  PT_LDS false
  // (a workgroup with more pages than the LDS table holds; the launcher
  // sizes workgroups so that this does not happen) reads the page table
  // from memory instead.
  const auto run_chunks = [&](auto pt_lds) {
    constexpr bool kPtLds = decltype(pt_lds)::value;
    for (int cb = w0; cb < w1; cb += kScanBatch) {
      uint4 kv[kScanBatch][2];
      int pgs[kScanBatch];  // the chunk's page, -1 when it has none (uniform)
#pragma unroll
      for (int i = 0; i < kScanBatch; ++i) {
        const int c = min(cb + i, w1 - 1);
        const int pg = __builtin_amdgcn_readfirstlane(kPtLds ? sh.pts[(c >> 2) - pg0] : pt_row[c >> 2]);
        const bool ok = cb + i < w1 && pg >= 0 && (long)pg < S.num_pages;
        pgs[i] = ok ? pg : -1;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(S.pages) + (ok ? (long)pg * DSA_INDEX_PAGE_BYTES : 0L), (short)0,
            ok ? DSA_INDEX_PAGE_BYTES : 0, 0x00020000);
        const int off = (c & 3) * (kChunkKeys * DSA_INDEX_DIM) + kr * DSA_INDEX_DIM + kc * 32;
        kv[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
        kv[i][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0));
      }
      // the key scales in the layout of the reduced scores: lane (j, kr) of
      // group q loads key kr's scale of chunk 4q + j (one load per group;
      // 0 for a chunk without a page)
      float ksl[kScanBatch / 4];
#pragma unroll
      for (int q = 0; q < kScanBatch / 4; ++q) {
        const int pl = kc == 0 ? pgs[4 * q] : (kc == 1 ? pgs[4 * q + 1] : (kc == 2 ? pgs[4 * q + 2] : pgs[4 * q + 3]));
        const int cl = cb + 4 * q + kc;
        const float* sp = reinterpret_cast<const float*>(S.pages + (long)max(pl, 0) * DSA_INDEX_PAGE_BYTES +
                                                         DSA_PAGE_TOKENS * DSA_INDEX_DIM) +
                          (cl & 3) * kChunkKeys + kr;
        ksl[q] = pl >= 0 ? *sp : 0.f;
      }
      // Groups of 4 chunks: each lane sums ReLU*w over its 16 heads of
      // every chunk, then two rounds of lane swaps transpose-reduce the
      // four 16-lane groups so that lane (j, kr) ends with key kr of chunk
      // 4q + j -- the same additions in the same order as reducing each
      // chunk into lanes 0-15 (+ lane i+32, then + lane i+16), with 3 swaps
      // and 3 adds per 4 chunks, and the per-key tail below runs once per
      // group on all 64 lanes.
      static_assert(kScanBatch % 4 == 0, "chunks are reduced in groups of 4");
#pragma unroll
      for (int q = 0; q < kScanBatch / 4; ++q) {
        if (cb + 4 * q >= w1) break;  // uniform
        float a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 4 * q + j;
          const v8i kb = v8i{(int)kv[i][0].x, (int)kv[i][0].y, (int)kv[i][0].z, (int)kv[i][0].w,
                             (int)kv[i][1].x, (int)kv[i][1].y, (int)kv[i][1].z, (int)kv[i][1].w};
          a[j] = 0.f;  // an invalid chunk's zero keys give 0
          if (cb + i >= w1) continue;  // uniform: past the wave's chunks
#pragma unroll
          for (int hg = 0; hg < NHG; ++hg) {
            const v4f d = qk_fp8<VARIANT>(qa[hg], kb);
#pragma unroll
            // ReLU as one integer max on the bits (a negative float, -0
            // included, is a negative integer): fmaxf adds a NaN-quieting
            // max before each, and the MFMA of finite fp8 values is finite
            for (int r = 0; r < 4; ++r)
              a[j] += wr[hg][r] * __int_as_float(max(__float_as_int(d[r]), 0));
          }
        }
        // permlane32_swap(x, y) -> {[x.lo, y.lo], [x.hi, y.hi]} (32-lane
        // halves); permlane16_swap(x, y) -> {[x.r0, y.r0, x.r2, y.r2],
        // [x.r1, y.r1, x.r3, y.r3]} (16-lane rows)
        const auto add32 = [](float x, float y) {
          const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
          return __uint_as_float(r[0]) + __uint_as_float(r[1]);
        };
        const float x = add32(a[0], a[2]);  // lanes 0-31: chunk 0; 32-63: chunk 2
        const float y = add32(a[1], a[3]);  // chunks 1, 3
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        const float acc = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
        const int c = cb + 4 * q + kc;  // this lane's chunk
        const bool okj = (kc == 0 ? pgs[4 * q] : (kc == 1 ? pgs[4 * q + 1] : (kc == 2 ? pgs[4 * q + 2] : pgs[4 * q + 3]))) >= 0;
        const int g = c * kChunkKeys + kr;
        if (c < w1 && g < S.slab_stride) {
          const float v = (okj && g < len) ? acc * ksl[q] : -INFINITY;
          // device-scope stores when the row's last workgroup reads them back
          if (S.next_idx) store_dev(&srow[g], v);
          else srow[g] = v;
          if (with_hist && g < len) {
            const uint32_t key = rank_key(v);
            atomicAdd(&sh.hist[key >> 20], 1u);
            if (SELECT && S.coop) {
              reinterpret_cast<CoopShared*>(smem)->keys[g - c0 * kChunkKeys] = key;
              atomicAdd(&sh.hist[kCoarseOff + (key >> 26)], 1u);
              kmax = max(kmax, key);
              nfin += key_is_finite(key) ? 1u : 0u;
            }
          }
        }
      }
    }
  };
  if (pts_lds)
    run_chunks(std::true_type{});
  else
    run_chunks(std::false_type{});
  }  // !FROM_SCORES
  dbg_stamp(dbk, 2);
  dbg_stamp_lane0(16 + wave_id());
  if (!with_hist) return;
  if constexpr (SELECT) {
    if (S.coop) {
      CoopShared& cs = *reinterpret_cast<CoopShared*>(smem);
      kmax = wave_reduce<2>(kmax);
      nfin = wave_reduce<0>(nfin);
      if (lane == 0) {
        cs.wstat[2 * wv] = nfin;
        cs.wstat[2 * wv + 1] = kmax;
      }
    }
  }
  __syncthreads();
  if constexpr (FROM_SCORES && SELECT) {
    if (S.coop) {  // coarse bin c = the 64 fine bins [64c, 64c + 64): 8 threads per bin
      const uint4* f4 = reinterpret_cast<const uint4*>(sh.hist + 8 * t);
      const uint4 a = f4[0], b = f4[1];
      uint32_t v = a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w;
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      if ((t & 7) == 0) sh.hist[kCoarseOff + (t >> 3)] = v;
      __syncthreads();
    }
  }
  dbg_stamp(dbk, 6);
  uint32_t* rs = S.hist + (long)row * S.hist_row_words;
  dbg_stamp(dbk, 3);
  if constexpr (!SELECT) return;
  if (!S.next_idx) return;
  if (S.coop) {
    // the union's uint4s per thread: 4 (up to 8192 entries, C3's 224 lists)
    // or 8.  A launch whose rows all have one size carries only that form
    // (the other, unused, made the kernel's code larger; LISTS == 4 with a
    // row of wider lists, which the launcher does not send, takes the
    // single-workgroup select)
    CoopShared& cs = *reinterpret_cast<CoopShared*>(smem);
    int* o = S.next_idx + (long)row * S.topk;
    const int p_hi = min(c1 * kChunkKeys, len);
    const bool narrow = nb * pub_stride(nb, S.topk) <= 4 * 4 * kMainThreads;
    if constexpr (LISTS == 4) {
      if (narrow) {
        coop_select<TOPK, 4>(cs, smem, S, bid, nb, len, c0 * kChunkKeys, p_hi, rs, srow, pt_row, o, sh.pts, pg0,
                             pts_lds);
        return;
      }
      // (not sent by the launcher) too many list entries for this form: the
      // single-workgroup select below
    } else if constexpr (LISTS == 8) {
      coop_select<TOPK, 8>(cs, smem, S, bid, nb, len, c0 * kChunkKeys, p_hi, rs, srow, pt_row, o, sh.pts, pg0,
                           pts_lds);
      return;
    } else {
      if (narrow)
        coop_select<TOPK, 4>(cs, smem, S, bid, nb, len, c0 * kChunkKeys, p_hi, rs, srow, pt_row, o, sh.pts, pg0,
                             pts_lds);
      else
        coop_select<TOPK, 8>(cs, smem, S, bid, nb, len, c0 * kChunkKeys, p_hi, rs, srow, pt_row, o, sh.pts, pg0,
                             pts_lds);
      return;
    }
  }
  // arrival: wait for this slice's device-scope score stores, then count;
  // the row's last slice selects
  wait_mem();
  __syncthreads();
  __shared__ uint32_t last;
  if (t == 0) last = (atomicAdd(&rs[kArrOff], 1u) == (uint32_t)nb - 1u) ? 1u : 0u;
  __syncthreads();
  if (!last) return;
  if (t == 0) rs[kArrOff] = 0u;
  dbg_stamp(dbk, 4);
  __syncthreads();  // the scan's LDS is dead now
  select_row<TOPK>(smem, srow, len, pt_row, S.next_idx + (long)row * S.topk, S.topk, TOPK ? S.pad : -1);
  dbg_stamp(dbk, 5);
}

// ======================================================================
// the fused launch
// ======================================================================
// ROLES: bit 0 attention workgroups, bit 1 scan workgroups, bit 2 the scan
// workgroups also select.  Each role set is its own instantiation, so a
// launch pays only for the registers of the roles it runs (a scan-only
// launch keeps several workgroups per CU resident).
// kRolePlan: scan workgroups per row by length (ragged batches), a separate
// instantiation so that batch-1 launches carry none of its code
// kRoleFromScores: the select loads the scores a plain scan launch wrote
// kRoleTopk: with kRoleFromScores, the standalone top-k (caller's pad value;
//   positions when there is no page table)
// kRoleWide: the select's lists of every row need 8 union uint4s per thread
// (otherwise 4; planned launches choose per row)
constexpr int kRoleAttn = 1, kRoleScan = 2, kRoleSelect = 4, kRolePlan = 8, kRoleFromScores = 16,
              kRoleTopk = 32, kRoleWide = 64;

// Workgroups per row by length (ragged batches of <= 64 rows): every row
// gets the workgroups its keys and page entries need (the cooperative
// select holds <= kCoopKeys keys per workgroup, the LDS page table <=
// kScanMaxPages - 2 pages), and the rest of the launch's nscan workgroups in
// proportion to its length, so that every workgroup streams about the same
// number of keys; a row's workgroups stay contiguous in block index.  Each
// wave computes the same plan from seq_lens (lane r: row r), no barrier.
// Only max(S.target, what the rows need) workgroups are planned; returns
// (row, index within the row, the row's workgroups), row -1 for a workgroup
// no row needs (it exits at once).
__device__ __forceinline__ int3 plan_row(const ScanArgs& S, int bid, int nscan) {
  const int lane = threadIdx.x & (kWave - 1);
  const bool in = lane < S.rows;
  const long cap = min((long)S.slab_stride, (long)S.pt_stride * DSA_PAGE_TOKENS);
  const uint32_t len = in ? (uint32_t)max(0L, min((long)S.seq_lens[lane], cap)) : 0u;
  uint32_t need = 0;
  if (in) {
    const uint32_t pages = (len + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS;
    need = max(1u, (pages + kScanMaxPages - 3) / (kScanMaxPages - 2));
    if (S.coop) need = max(need, (len + kCoopKeys - 1) / kCoopKeys);
  }
  const uint32_t total = wave_reduce<0>(len);
  // the workgroups to use: the launcher's target (one per free CU when the
  // select pins a workgroup to its CU), at least what the rows need
  const int needed = (int)wave_reduce<0>(need);
  const uint32_t spare = (uint32_t)max(0, min(nscan, max(S.target, needed)) - needed);
  uint32_t extra = 0;
  if (in) extra = total ? (uint32_t)(((uint64_t)spare * len) / total) : spare / (uint32_t)S.rows;
  const uint32_t rem = spare - wave_reduce<0>(extra);  // < rows
  extra += (in && (uint32_t)lane < rem) ? 1u : 0u;
  const uint32_t n = in ? min(need + extra, (uint32_t)S.max_nb) : 0u;
  const uint32_t incl = wave_scan_incl<0>(n);
  const uint64_t m = __ballot(in && incl > (uint32_t)bid);
  if (!m) return make_int3(-1, 0, 0);
  const int r = __builtin_ctzll(m);
  const int excl = __builtin_amdgcn_readlane((int)(incl - n), r);
  return make_int3(r, bid - excl, __builtin_amdgcn_readlane((int)n, r));
}

template <int NHG, int VARIANT, int ROLES>
__global__ __launch_bounds__(kMainThreads, (ROLES & ~kRolePlan) == kRoleScan ? 4 : 1) void decode_main_kernel(AttnArgs A, int n_att,
                                                                                             ScanArgs S) {
  extern __shared__ __align__(16) unsigned char smem[];
  int bid = blockIdx.x;
  dbg_begin();
  if constexpr ((ROLES & kRoleAttn) != 0) {
    if (bid < n_att) {
      const int nhg = A.H / kHG;
      const int sp = bid % A.nsplit;
      const int hg = (bid / A.nsplit) % nhg;
      const int b = bid / (A.nsplit * nhg);
      attention_block<ROLES == kRoleAttn>(A, b, hg, sp, smem);
      dbg_flush(blockIdx.x);
      return;
    }
  }
  if constexpr ((ROLES & kRoleScan) != 0) {
    bid -= n_att;
    int row = bid / S.blocks_per_row, nb = S.blocks_per_row;
    bid -= row * nb;
    if constexpr ((ROLES & kRolePlan) != 0) {
      const int3 slot = plan_row(S, blockIdx.x - n_att, (int)gridDim.x - n_att);
      if (slot.x < 0) return;  // a spare workgroup: no row needs it
      row = slot.x;
      bid = slot.y;
      nb = slot.z;
    }
    constexpr int kLists = (ROLES & kRolePlan) ? 0 : ((ROLES & kRoleWide) ? 8 : 4);
    scan_block<NHG, VARIANT, (ROLES & kRoleSelect) != 0, (ROLES & kRoleFromScores) != 0, (ROLES & kRoleTopk) != 0,
               kLists>(S, row, bid, nb, smem);
    dbg_flush(blockIdx.x);
  }
}

// ---------------------------------------------------------------- host side
static int g_scan_variant = 0;
void set_scan_variant(int v) { g_scan_variant = v ? 1 : 0; }
static int g_coop_select = 1;
void set_coop_select(int on) { g_coop_select = on ? 1 : 0; }
int group_wait_timeouts(int reset) {
  int v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_group_wait_timeouts), sizeof(int)) != hipSuccess) return -1;
  if (reset) {
    const int z = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_group_wait_timeouts), &z, sizeof(int)) != hipSuccess) return -1;
  }
  return v;
}

void set_spin_limit(int n) {
  const int v = n < 0 ? kGroupSpinMax : n;
  (void)hipMemcpyToSymbol(HIP_SYMBOL(g_group_spin_max), &v, sizeof(int));
}

// Sum of the status words (expired waits) of nrows top-k scratch rows and
// ngroups attention barrier areas into *out, optionally re-zeroed.  One
// workgroup; the words are read with device-scope loads.
constexpr int kStatusThreads = 256;
__global__ __launch_bounds__(kStatusThreads) void sync_status_kernel(uint32_t* scr, int nrows, long row_words,
                                                                     long row_off, uint32_t* ws, int ngroups,
                                                                     int* out, int clear) {
  __shared__ uint32_t part[kStatusThreads / kWave];
  const int t = threadIdx.x;
  uint32_t v = 0;
  for (int i = t; i < nrows; i += kStatusThreads) {
    uint32_t* p = scr + (long)i * row_words + row_off;
    v += __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (clear) store_dev(p, 0u);
  }
  for (int i = t; i < ngroups; i += kStatusThreads) {
    uint32_t* p = ws + (long)i * kSyncWords + kSyncStatusWord;
    v += __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (clear) store_dev(p, 0u);
  }
  v = wave_reduce<0>(v);
  if ((t & (kWave - 1)) == 0) part[t / kWave] = v;
  __syncthreads();
  if (t == 0) {
    uint32_t tot = 0;
    for (int w = 0; w < kStatusThreads / kWave; ++w) tot += part[w];
    out[0] = (int)min(tot, 0x7fffffffu);
  }
}

hipError_t launch_sync_status(void* topk_scratch, int B_scan, int slab, void* workspace, int groups, int* out,
                              int clear, hipStream_t s) {
  hipLaunchKernelGGL(sync_status_kernel, dim3(1), dim3(kStatusThreads), 0, s, static_cast<uint32_t*>(topk_scratch),
                     topk_scratch ? B_scan : 0, row_scratch_words(slab), row_sync_off(slab) + kSyncStatusWord,
                     static_cast<uint32_t*>(workspace), workspace ? groups : 0, out, clear);
  return hipGetLastError();
}

static int device_cus();
int device_cu_count() { return device_cus(); }
// the current device's CU count (devices 0-63 cached)
static int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const bool keep = dev >= 0 && dev < 64;
  int cus = keep ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (!cus) {
    hipDeviceProp_t prop;
    cus = hipGetDeviceProperties(&prop, dev) == hipSuccess ? prop.multiProcessorCount : 256;
    if (keep) cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// One split per 64 selected keys (half a tile: more workgroups gather at
// once, which the latency-bound gather needs; at top-2048, b = 1: 16.3 ->
// 14.9 us per attention-only layer), at most one round of workgroups.
int attn_auto_nsplit(int topk, int B, int H) {
  const int groups = std::max(1, B * (H / kHG));
  const int cap = std::min(kMaxSplit, std::max(1, device_cus() / groups));
  return std::max(1, std::min(cap, (topk + kAutoSplitKeys - 1) / kAutoSplitKeys));
}

// Splits when the attention shares the launch with indexer scans: the
// default count, but the attention workgroups together take at most about a
// quarter of the CUs, so the scans keep the rest (at b = 1: 32 splits of 64
// keys beside 224 scan workgroups).
int attn_fused_nsplit(int topk, int B, int H) {
  const int groups = std::max(1, B * (H / kHG));
  return std::max(1, std::min(attn_auto_nsplit(topk, B, H), device_cus() / 4 / groups));
}

// [one group barrier per (row, head group) | partials o | partials (m, l)]:
// the barriers sit at offsets that do not depend on nsplit, so launches with
// different split counts can share one workspace (sized for the largest).
size_t attn_workspace_bytes(int B, int H, int nsplit) {
  const size_t blocks = (size_t)B * (H / kHG) * nsplit;
  const size_t sync = (size_t)B * (H / kHG) * kSyncWords;
  return (sync + blocks * kHG * (DSA_LATENT_DIM + 2)) * sizeof(float);
}

void attn_bind_workspace(AttnArgs& A, void* ws, int B) {
  const size_t blocks = (size_t)B * (A.H / kHG) * A.nsplit;
  A.sync = reinterpret_cast<uint32_t*>(ws);
  A.part_o = reinterpret_cast<float*>(A.sync + (size_t)B * (A.H / kHG) * kSyncWords);
  A.part_ml = A.part_o + blocks * kHG * DSA_LATENT_DIM;
}

static int g_scan_blocks_cap = 0;  // internal: cap on scan workgroups per launch (0 = none)
void set_scan_blocks_cap(int n) { g_scan_blocks_cap = std::max(0, n); }

int scan_blocks_per_row(int B, int pt_stride, int slab_stride, int att_blocks, bool big_lds) {
  const long cap = std::min((long)slab_stride, (long)pt_stride * DSA_PAGE_TOKENS);
  const long cap_chunks = (cap + kChunkKeys - 1) / kChunkKeys;
  const int cus = device_cus();
  // when the launch's LDS (attention tile or the select) pins one block per
  // CU, fill the CUs the attention leaves; a plain scan: two blocks per CU
  long target = big_lds ? std::max<long>(cus - att_blocks, cus / 2) : 2L * cus;
  if (g_scan_blocks_cap > 0) target = std::min<long>(target, g_scan_blocks_cap);
  long per_row = (target + B - 1) / B;
  per_row = std::min(per_row, std::max(1L, cap_chunks / kMainWaves));
  // each workgroup's page-table entries must fit the LDS table
  const long cap_pages = (cap + DSA_PAGE_TOKENS - 1) / DSA_PAGE_TOKENS;
  per_row = std::max(per_row, (cap_pages + kScanMaxPages - 3) / (kScanMaxPages - 2));
  return (int)std::max(1L, per_row);
}

template <int NHG, int VARIANT, int ROLES>
static hipError_t launch_k(dim3 grid, size_t lds, size_t lds_max, hipStream_t s, const AttnArgs& A,
                           int n_att, const ScanArgs& S) {
  static PerDeviceOnce attr;
  const hipError_t e = attr.run([lds_max] {
    return hipFuncSetAttribute((const void*)decode_main_kernel<NHG, VARIANT, ROLES>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
  });
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_main_kernel<NHG, VARIANT, ROLES>), grid, dim3(kMainThreads), lds, s, A, n_att, S);
  return hipGetLastError();
}

template <int NHG, int PLAN>
static hipError_t launch_nhg_p(dim3 grid, size_t lds, size_t lds_max, hipStream_t s, const AttnArgs& A,
                               int n_att, const ScanArgs& S) {
  const bool att = n_att > 0;
  if (S.from_scores) {
    if (S.standalone) return launch_k<1, 0, kRoleScan | kRoleSelect | kRoleFromScores | kRoleTopk | PLAN>(
        grid, lds, lds_max, s, A, n_att, S);
    if (!att) return launch_k<NHG, 0, kRoleScan | kRoleSelect | kRoleFromScores | PLAN>(grid, lds, lds_max, s, A, n_att, S);
    return launch_k<NHG, 0, kRoleAttn | kRoleScan | kRoleSelect | kRoleFromScores | PLAN>(grid, lds, lds_max, s, A,
                                                                                         n_att, S);
  }
  if (!att && !S.next_idx)  // plain scan: the only role with the alternative MFMA form
    return g_scan_variant == 0 ? launch_k<NHG, 0, kRoleScan | (PLAN & kRolePlan)>(grid, lds, lds_max, s, A, n_att, S)
                               : launch_k<NHG, 1, kRoleScan | (PLAN & kRolePlan)>(grid, lds, lds_max, s, A, n_att, S);
  if (!att) return launch_k<NHG, 0, kRoleScan | kRoleSelect | PLAN>(grid, lds, lds_max, s, A, n_att, S);
  return launch_k<NHG, 0, kRoleAttn | kRoleScan | kRoleSelect | PLAN>(grid, lds, lds_max, s, A, n_att, S);
}

template <int NHG>
static hipError_t launch_nhg(dim3 grid, size_t lds, size_t lds_max, hipStream_t s, const AttnArgs& A,
                             int n_att, const ScanArgs& S) {
  const bool scan = S.blocks_per_row > 0 && grid.x > (unsigned)n_att;
  if (!scan) return launch_k<4, 0, kRoleAttn>(grid, lds, lds_max, s, A, n_att, S);
  if (S.balance) return launch_nhg_p<NHG, kRolePlan>(grid, lds, lds_max, s, A, n_att, S);
  // one workgroup count for every row: the select's union size is fixed
  const bool wide = S.next_idx && S.coop &&
                    (long)S.blocks_per_row * pub_stride(S.blocks_per_row, S.topk) > 4L * 4 * kMainThreads;
  return wide ? launch_nhg_p<NHG, kRoleWide>(grid, lds, lds_max, s, A, n_att, S)
              : launch_nhg_p<NHG, 0>(grid, lds, lds_max, s, A, n_att, S);
}

// the plain scan as one index space over every row (scan_flat.hip)
hipError_t launch_flat_scan(const AttnArgs* A, int B_att, const ScanArgs& S, int B, hipStream_t s);
constexpr int kFlatScanMaxRows = kFlatRows;
static int g_flat_scan = 1;  // internal switch: plain scans of >= 2 rows through launch_flat_scan
void set_flat_scan(int on) { g_flat_scan = on ? 1 : 0; }
bool flat_scan_on() { return g_flat_scan != 0; }

hipError_t launch_decode_main(const AttnArgs* A, int B_att, const ScanArgs* S, int B_scan,
                              hipStream_t s) {
#ifndef DSA_FLAT_MIN_ROWS
#define DSA_FLAT_MIN_ROWS 2
#endif
  if (!A && S && !S->next_idx && !S->hist && g_flat_scan && B_scan >= DSA_FLAT_MIN_ROWS && flat_scan_fits(*S, B_scan))
    return launch_flat_scan(nullptr, 0, *S, B_scan, s);
  const size_t lds_attn = sizeof(AttnShared);
  const size_t lds_coop = std::max(sizeof(CoopShared), (size_t)kRowSelWords * 4);
  const size_t lds_max = std::max(lds_attn, lds_coop);
  AttnArgs a{};
  ScanArgs sc{};
  int n_att = 0, n_scan = 0;
  if (A) {
    a = *A;
    n_att = B_att * (a.H / kHG) * a.nsplit;
  }
  const bool select = S && S->next_idx;
  if (S) {
    sc = *S;
    sc.blocks_per_row = scan_blocks_per_row(B_scan, sc.pt_stride, sc.slab_stride, n_att,
                                            n_att > 0 || select);
    sc.coop = 0;
    if (select && g_coop_select) {
      // cooperative select: the row's workgroups wait for each other, so
      // they must all be resident at once.  Workgroups are dispatched in
      // index order, round-robin over the XCDs, and attention workgroups
      // never wait: a row of at most (CUs - one per XCD) workgroups always
      // becomes fully resident.  Each workgroup keeps its keys in LDS.
      const long cap = std::min((long)sc.slab_stride, (long)sc.pt_stride * DSA_PAGE_TOKENS);
      const long cap_chunks = (cap + kChunkKeys - 1) / kChunkKeys;
      const long min_nb = (cap_chunks + kCoopKeys / kChunkKeys - 1) / (kCoopKeys / kChunkKeys);
      const long max_nb = std::min<long>(kCoopMaxBlocks, device_cus() - 8);
      const long bw = bitmap_words(sc.slab_stride);
      long nb = std::max<long>(std::min<long>(sc.blocks_per_row, max_nb), min_nb);
      if (nb <= max_nb && nb <= bw) {
        sc.blocks_per_row = (int)nb;
        sc.coop = 1;
      }
    }
    n_scan = B_scan * sc.blocks_per_row;
    // ragged batches: workgroups per row by length (the grid stays B x nb)
    sc.rows = B_scan;
    sc.balance = B_scan > 1 && B_scan <= kWave;
    sc.max_nb = sc.coop ? (int)std::min<long>(kCoopMaxBlocks, device_cus() - 8) : n_scan;
    // one workgroup count for every row: the select's list sizing is fixed
    sc.pub_stride = sc.coop && !sc.balance ? pub_stride(sc.blocks_per_row, sc.topk) : 0;
    sc.pub_target = sc.coop && !sc.balance ? pub_target(sc.blocks_per_row, sc.topk) : 0;
    // the workgroups split a row's chunks in 32-bit arithmetic (part())
    const long cap_chunks =
        (std::min((long)sc.slab_stride, (long)sc.pt_stride * DSA_PAGE_TOKENS) + kChunkKeys - 1) / kChunkKeys;
    if ((cap_chunks + 1) * (long)std::max(sc.max_nb, sc.blocks_per_row) >= (1L << 32)) return hipErrorInvalidValue;
    // one round of workgroups: when the launch's LDS pins one workgroup per
    // CU, the CUs the attention leaves (spare workgroups exit at once)
    const bool big_lds = n_att > 0 || select;
    sc.target = big_lds ? std::max(device_cus() - n_att, device_cus() / 2) : n_scan;
  }
  if (n_att + n_scan == 0) return hipSuccess;
  size_t lds = sizeof(ScanShared);
  if (n_att) lds = std::max(lds, lds_attn);
  if (select) lds = std::max(lds, sc.coop ? lds_coop : (size_t)kRowSelWords * 4);
  const dim3 grid(n_att + n_scan);
  switch (S ? sc.Hidx / 16 : 4) {
    case 1: return launch_nhg<1>(grid, lds, lds_max, s, a, n_att, sc);
    case 2: return launch_nhg<2>(grid, lds, lds_max, s, a, n_att, sc);
    case 3: return launch_nhg<3>(grid, lds, lds_max, s, a, n_att, sc);
    default: return launch_nhg<4>(grid, lds, lds_max, s, a, n_att, sc);
  }
}

}  // namespace dsa
