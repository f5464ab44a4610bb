// Decode-step operand preparation on gfx950: the fp8 quantizers that feed
// the scan and the attention, and the paged appends of one step's keys.
//
// Quantization rule (the reference harness's quantize_e4m3_rowwise,
// K:2969-2974, also the build's fixtures): per 128-element row,
//   scale = max(amax, 1e-6) / 448,  code = e4m3_rne(clamp(x / scale, +-448)),
// with x / scale an IEEE fp32 division and the OCP e4m3fn round to nearest
// even done in software (no dependence on a hardware conversion's modes).
//   - indexer query: one row per (token, head); the scale folds into the
//     head weight, w' = w * scale (K:2984-2985; serving act_quant P:338);
//   - index key: one row per token into the paged cache, 128 codes at slot
//     (g % 64) of page page_table[row, g / 64] and its scale in the page's
//     scale tail (K:540-546, K:2428; serving _store_index_k_cache P:339-342);
//   - latent row: 512 latent values as four 128-element rows (codes + four
//     fp32 scales) and 64 bf16 rope values, packed into the 656-byte row at
//     the token's KV slot (K:1114, K:1355-1395; SGLang's fp8 KV layout).
// One wave per 128-element row: lane l holds elements 2l, 2l+1; the row's
// amax is a DPP max over the wave.
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

constexpr int kQuantThreads = 256;  // 4 waves, one row each

// OCP e4m3fn code of x, |x| <= 448, round to nearest even; exact.
__device__ __forceinline__ uint32_t e4m3_rne(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0.015625f) {  // below 2^-6: multiples of 2^-9 (8 -> 0x08, the smallest normal)
    code = (uint32_t)__builtin_rintf(a * 512.f);
  } else {
    const uint32_t b = __float_as_uint(a);
    const uint32_t r = (b + 0x7ffffu + ((b >> 20) & 1u)) >> 20;  // 8-bit exponent | 3-bit mantissa
    code = r - ((127u - 7u) << 3);
  }
  return sign | code;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// amax of a 128-element row held two per lane, every lane gets it
__device__ __forceinline__ float row_amax(float x0, float x1) {
  const uint32_t m = __float_as_uint(fmaxf(fabsf(x0), fabsf(x1)));  // non-negative: bits order as values
  return __uint_as_float(wave_reduce<2>(m));
}

__device__ __forceinline__ float quant_scale(float amax) { return fmaxf(amax, 1e-6f) / 448.f; }

__device__ __forceinline__ uint32_t quant_pair(float x0, float x1, float scale) {
  const float a = fminf(fmaxf(x0 / scale, -448.f), 448.f);
  const float b = fminf(fmaxf(x1 / scale, -448.f), 448.f);
  return e4m3_rne(a) | (e4m3_rne(b) << 8);
}

// q [rows, 128] bf16 -> codes [rows, 128], w_out[row] = w[row] * scale
__global__ __launch_bounds__(kQuantThreads) void quant_query_kernel(const uint32_t* __restrict__ q, const float* w,
                                                                     uint16_t* codes, float* w_out, long rows) {
  const long row = (long)blockIdx.x * (kQuantThreads / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= rows) return;  // whole waves exit together
  const uint32_t pr = q[row * 64 + lane];
  const float x0 = bf16_to_f32(pr & 0xffffu), x1 = bf16_to_f32(pr >> 16);
  const float scale = quant_scale(row_amax(x0, x1));
  codes[row * 64 + lane] = (uint16_t)quant_pair(x0, x1, scale);
  if (lane == 0) w_out[row] = w[row] * scale;
}

// keys [n, 128] bf16 of (row[i], pos[i]) -> the paged index cache
__global__ __launch_bounds__(kQuantThreads) void append_keys_kernel(const uint32_t* __restrict__ k, const int* rows,
                                                                     const int* pos, int n, const int* page_table,
                                                                     int pt_stride, uint8_t* pages, long num_pages) {
  const int i = blockIdx.x * (kQuantThreads / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (i >= n) return;
  const int r = rows[i], g = pos[i];
  const int page = (g >= 0 && g / DSA_PAGE_TOKENS < pt_stride) ? page_table[(long)r * pt_stride + g / DSA_PAGE_TOKENS]
                                                                  : -1;
  const uint32_t pr = k[(long)i * 64 + lane];
  const float x0 = bf16_to_f32(pr & 0xffffu), x1 = bf16_to_f32(pr >> 16);
  const float scale = quant_scale(row_amax(x0, x1));
  if (page < 0 || page >= num_pages) return;  // no page for this token: nothing stored
  uint8_t* base = pages + (long)page * DSA_INDEX_PAGE_BYTES;
  const int slot = g % DSA_PAGE_TOKENS;
  reinterpret_cast<uint16_t*>(base + slot * DSA_INDEX_DIM)[lane] = (uint16_t)quant_pair(x0, x1, scale);
  if (lane == 0) reinterpret_cast<float*>(base + DSA_PAGE_TOKENS * DSA_INDEX_DIM)[slot] = scale;
}

// latent [n, 576] bf16 -> 656-byte rows at KV slots slot[i]
__global__ __launch_bounds__(kQuantThreads) void append_latent_kernel(const uint16_t* __restrict__ lat,
                                                                       const int* slots, int n, uint8_t* pool,
                                                                       long kv_rows) {
  const int i = blockIdx.x * (kQuantThreads / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (i >= n) return;
  const long slot = slots[i];
  const uint16_t* src = lat + (long)i * DSA_QK_DIM;
  uint8_t* dst = pool + slot * DSA_LATENT_ROW_BYTES;
  const bool ok = slot >= 0 && slot < kv_rows;
  float sc[4];
  uint32_t codes[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {  // the four 128-dim groups, one after another
    const uint32_t pr = reinterpret_cast<const uint32_t*>(src + grp * 128)[lane];
    const float x0 = bf16_to_f32(pr & 0xffffu), x1 = bf16_to_f32(pr >> 16);
    sc[grp] = quant_scale(row_amax(x0, x1));
    codes[grp] = quant_pair(x0, x1, sc[grp]);
  }
  if (!ok) return;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) reinterpret_cast<uint16_t*>(dst + grp * 128)[lane] = (uint16_t)codes[grp];
  if (lane < 4) reinterpret_cast<float*>(dst + DSA_LATENT_DIM)[lane] = sc[lane];
  if (lane < 32)  // 64 bf16 rope values, 4 bytes per lane
    reinterpret_cast<uint32_t*>(dst + DSA_LATENT_DIM + 16)[lane] =
        reinterpret_cast<const uint32_t*>(src + DSA_LATENT_DIM)[lane];
}

static dim3 quant_grid(long rows) { return dim3((unsigned)((rows + kQuantThreads / kWave - 1) / (kQuantThreads / kWave))); }

hipError_t launch_quant_query(const void* q_bf16, const float* w, void* codes, float* w_out, long rows,
                              hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(quant_query_kernel, quant_grid(rows), dim3(kQuantThreads), 0, s,
                     reinterpret_cast<const uint32_t*>(q_bf16), w, reinterpret_cast<uint16_t*>(codes), w_out, rows);
  return hipGetLastError();
}

hipError_t launch_append_keys(const void* k_bf16, const int* rows, const int* pos, int n, const int* page_table,
                              int pt_stride, void* pages, long num_pages, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(append_keys_kernel, quant_grid(n), dim3(kQuantThreads), 0, s,
                     reinterpret_cast<const uint32_t*>(k_bf16), rows, pos, n, page_table, pt_stride,
                     reinterpret_cast<uint8_t*>(pages), num_pages);
  return hipGetLastError();
}

hipError_t launch_append_latent(const void* lat_bf16, const int* slots, int n, void* pool, long kv_rows,
                                hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(append_latent_kernel, quant_grid(n), dim3(kQuantThreads), 0, s,
                     reinterpret_cast<const uint16_t*>(lat_bf16), slots, n, reinterpret_cast<uint8_t*>(pool),
                     kv_rows);
  return hipGetLastError();
}

}  // namespace dsa
