// Shared device helpers for the gfx950 DSA decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "dsa_mli.h"

namespace dsa {

// Host side: a set-up step (a kernel's LDS attribute) that must run once per
// device, on the first launch with that device current.  Devices 0-63 are
// remembered; any other device runs the step on every launch.
struct PerDeviceOnce {
  std::atomic<uint64_t> done{0};
  template <class F>
  hipError_t run(F&& step) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uint64_t bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0ull;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    const hipError_t e = step();
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return e;
  }
};

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Order-preserving map fp32 -> u32 used by every ranking in this library:
// larger key == ranks higher.  -0.0 is folded onto +0.0 and every NaN onto
// the top key, so the order is total and matches the comparison the
// reference's select makes (torch.topk treats NaN as largest, -0.0 == +0.0).
// Same transform as the reference's hp_exact_key (K:1132-1135) apart from the
// canonicalisation of NaN and -0.0.
__device__ __forceinline__ uint32_t rank_key(float x) {
  uint32_t b = __float_as_uint(x);
  if (x != x) return 0xffffffffu;
  if ((b & 0x7fffffffu) == 0u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// -inf maps to this key, +inf to 0xff800000; NaN to 0xffffffff.
constexpr uint32_t kKeyNegInf = 0x007fffffu;
constexpr uint32_t kKeyPosInf = 0xff800000u;
__device__ __forceinline__ bool key_is_finite(uint32_t k) {
  return k > kKeyNegInf && k < kKeyPosInf;
}

// Two fp32 -> packed bf16 (lo in bits 0-15), round to nearest even: one
// gfx950 v_cvt_pk_bf16_f32 (the default round mode is nearest even; the
// inputs here are finite).
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){lo, hi}, v2bf));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Four OCP e4m3 (one 32-bit word, byte i = element i) -> fp32, exact.
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* o) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  o[0] = lo[0];
  o[1] = lo[1];
  o[2] = hi[0];
  o[3] = hi[1];
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

// ---- wave-wide scans and reductions on DPP (row shifts + row broadcasts,
// no LDS round trip; lanes whose source is outside the row keep `ident`) ----
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t ident) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, CTRL, ROW_MASK, 0xf, false);
}
// OP: 0 = sum, 1 = min, 2 = max (unsigned)
template <int OP>
__device__ __forceinline__ uint32_t u32_op(uint32_t a, uint32_t b) {
  return OP == 0 ? a + b : (OP == 1 ? (a < b ? a : b) : (a > b ? a : b));
}
template <int OP>
constexpr uint32_t u32_ident() { return OP == 1 ? 0xffffffffu : 0u; }
// inclusive scan over the wave's 64 lanes (lane order)
template <int OP = 0>
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
  constexpr uint32_t id = u32_ident<OP>();
  v = u32_op<OP>(v, dpp_u32<0x111, 0xf>(v, id));  // row_shr:1
  v = u32_op<OP>(v, dpp_u32<0x112, 0xf>(v, id));  // row_shr:2
  v = u32_op<OP>(v, dpp_u32<0x114, 0xf>(v, id));  // row_shr:4
  v = u32_op<OP>(v, dpp_u32<0x118, 0xf>(v, id));  // row_shr:8
  v = u32_op<OP>(v, dpp_u32<0x142, 0xa>(v, id));  // row_bcast:15 -> rows 1, 3
  v = u32_op<OP>(v, dpp_u32<0x143, 0xc>(v, id));  // row_bcast:31 -> rows 2, 3
  return v;
}
// reduction over the wave, the same value in every lane
template <int OP = 0>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_scan_incl<OP>(v), 63);
}

// Reductions over each half-wave (lanes 0-31 and 32-63, e.g. one softmax row
// per half): every lane gets its half's result.  OP: 0 = sum, 2 = max.
template <int OP>
__device__ __forceinline__ float half_wave_reduce(float v) {
  const float id = OP == 2 ? -INFINITY : 0.f;
  auto op = [](float a, float b) { return OP == 2 ? fmaxf(a, b) : a + b; };
  auto sh = [&](auto ctrl, auto rows, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(id), __float_as_int(x), decltype(ctrl)::value,
                                                      decltype(rows)::value, 0xf, false));
  };
  using C1 = std::integral_constant<int, 0x111>;
  using C2 = std::integral_constant<int, 0x112>;
  using C4 = std::integral_constant<int, 0x114>;
  using C8 = std::integral_constant<int, 0x118>;
  using B15 = std::integral_constant<int, 0x142>;
  using All = std::integral_constant<int, 0xf>;
  using Odd = std::integral_constant<int, 0xa>;
  v = op(v, sh(C1{}, All{}, v));
  v = op(v, sh(C2{}, All{}, v));
  v = op(v, sh(C4{}, All{}, v));
  v = op(v, sh(C8{}, All{}, v));
  v = op(v, sh(B15{}, Odd{}, v));  // rows 1, 3 += rows 0, 2 (their lane 15)
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return (threadIdx.x & 32) ? hi : lo;
}

// Reduction over each 16-lane DPP row (OP: 0 = sum, 2 = max), every lane
// of the row gets the result: an inclusive scan by row shifts leaves it in
// the row's lane 15, which a bpermute hands to the row.  All lanes active.
template <int OP>
__device__ __forceinline__ float row16_reduce(float v) {
  const float id = OP == 2 ? -INFINITY : 0.f;
  auto op = [](float a, float b) { return OP == 2 ? fmaxf(a, b) : a + b; };
  auto shr = [&](auto ctrl, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(id), __float_as_int(x), decltype(ctrl)::value,
                                                      0xf, 0xf, false));
  };
  v = op(v, shr(std::integral_constant<int, 0x111>{}, v));  // row_shr:1
  v = op(v, shr(std::integral_constant<int, 0x112>{}, v));  // row_shr:2
  v = op(v, shr(std::integral_constant<int, 0x114>{}, v));  // row_shr:4
  v = op(v, shr(std::integral_constant<int, 0x118>{}, v));  // row_shr:8 -> lane 15 holds the row's result
  const int src = (int)((threadIdx.x & ~15u) | 15u) & (kWave - 1);
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Phase timestamps for profiling, compiled in only with -DDSA_PHASE_STAMPS
// (each stamp reads the enable flag from memory and waits for it, which
// would put a memory round trip on the critical path of every phase):
// thread 0 of workgroup `blk` records the 100 MHz constant clock at phase
// `ph`; the internal dsa_internal_debug entry point clears the table.
// Counterpart of the reference's hp_dbg stamps (K:1076-1091).
constexpr int kDbgBlocks = 512;
constexpr int kDbgPhases = 48;
extern __device__ int g_dbg_on;
extern __device__ unsigned long long g_dbg[kDbgBlocks * kDbgPhases];
#ifdef DSA_PHASE_STAMPS
// Profiling builds record into LDS (no memory traffic, so a stamp does not
// delay the launch's own waits for its loads and stores) and copy the
// workgroup's stamps to g_dbg once, at its end (dbg_flush).
constexpr bool kPhaseStamps = true;
__shared__ unsigned long long s_dbg_marks[kDbgPhases];
__device__ __forceinline__ void dbg_begin() {
  if (threadIdx.x < kDbgPhases) s_dbg_marks[threadIdx.x] = 0ull;
}
__device__ __forceinline__ void dbg_stamp(int, int ph) {
  if (threadIdx.x == 0) s_dbg_marks[ph] = __builtin_amdgcn_s_memrealtime();
}
// Same, recorded by lane 0 of wave `w` instead of thread 0.
__device__ __forceinline__ void dbg_stamp_wave(int, int ph, int w) {
  if (threadIdx.x == (unsigned)(w * kWave)) s_dbg_marks[ph] = __builtin_amdgcn_s_memrealtime();
}
// Same, recorded by lane 0 of every wave that calls it.
__device__ __forceinline__ void dbg_stamp_lane0(int ph) {
  if ((threadIdx.x & (kWave - 1)) == 0) s_dbg_marks[ph] = __builtin_amdgcn_s_memrealtime();
}
// a value instead of a time (the probe reads it from the same table)
__device__ __forceinline__ void dbg_value(int, int ph, unsigned long long v) {
  if (threadIdx.x == 0) s_dbg_marks[ph] = v;
}
// a value recorded by lane 0 of every wave that calls it
__device__ __forceinline__ void dbg_value_lane0(int ph, unsigned long long v) {
  if ((threadIdx.x & (kWave - 1)) == 0) s_dbg_marks[ph] = v;
}
// the workgroup's XCD (XCC_ID) and hardware id (HW_ID: CU, SIMD, shader
// engine) into slots 40 and 41
__device__ __forceinline__ void dbg_hw_ids() {
  if (threadIdx.x == 0) {
    s_dbg_marks[40] = (unsigned)__builtin_amdgcn_s_getreg((3 << 11) | 20);   // XCC_ID[3:0]
    s_dbg_marks[41] = (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID
  }
}
// every thread of the workgroup calls it once, at the end
__device__ __forceinline__ void dbg_flush(int blk) {
  __syncthreads();
  if (threadIdx.x < kDbgPhases && blk < kDbgBlocks) g_dbg[blk * kDbgPhases + threadIdx.x] = s_dbg_marks[threadIdx.x];
}
#else
constexpr bool kPhaseStamps = false;
__device__ __forceinline__ void dbg_begin() {}
__device__ __forceinline__ void dbg_flush(int) {}
__device__ __forceinline__ void dbg_value(int, int, unsigned long long) {}
__device__ __forceinline__ void dbg_hw_ids() {}
__device__ __forceinline__ void dbg_value_lane0(int, unsigned long long) {}
__device__ __forceinline__ void dbg_stamp(int, int) {}
__device__ __forceinline__ void dbg_stamp_wave(int, int, int) {}
__device__ __forceinline__ void dbg_stamp_lane0(int) {}
#endif

// ---- device-coherent publication between workgroups of one launch ----
// Data a workgroup hands to the "last arriving" workgroup of its group is
// written with device-scope stores (global_store ... sc1: coherent across
// all XCDs' L2s by themselves), the writer waits for its stores to complete
// (s_waitcnt), then increments an arrival counter with a device-scope
// atomic.  The last arriver reads the data with device-scope loads
// (buffer_load ... sc1).  This is the release/acquire the AMDGPU memory
// model implements for agent-scope atomics, without the whole-L2 writeback
// and invalidate (buffer_wbl2 / buffer_inv) that a fence would add per
// workgroup.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until every memory operation this thread issued has completed
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

constexpr int kCpolSc1 = 16;  // buffer-load cache policy: device scope
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at byte offset off (0 beyond the resource's size), device scope
__device__ __forceinline__ uint4 load_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1));
}
// 16-byte device-scope store at byte offset off (dropped beyond the size)
__device__ __forceinline__ void store_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, off, 0, kCpolSc1);
}
__device__ __forceinline__ uint32_t load_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCpolSc1);
}

// Sense-reversing group barrier between co-resident workgroups of one
// launch.  sync: kGroupSyncGroups arrival counters, a top counter and
// kGroupSyncFlags release flags, one 256-byte line each (zero before first
// use).  Every member publishes (device-scope stores, waited for) and
// arrives on its group's counter (member bid -> group bid % 16, so each line
// sees few atomics); the last of a group arrives on the top counter; the
// last of all re-zeroes the counters and flips the flags.  A group of at
// most kGroupFlatMax members arrives on counter 0 alone.  The others spin
// on the flag of their XCD (bid % 8), reading it with device-scope loads.
// `sense` is the flags' value before this barrier (read at launch start;
// the flags flip once per use).  The wait is bounded (about a second): on
// expiry it counts in g_group_wait_timeouts and goes on, so a launch that
// breaks the co-residency assumption returns (with wrong results, and the
// counter says so) instead of hanging the device.
extern __device__ int g_group_wait_timeouts;
constexpr int kGroupSpinMax = 1 << 20;
// polls before a wait gives up (kGroupSpinMax; lowered only by the library's
// internal test hook, so that tests can make every wait give up at once)
extern __device__ int g_group_spin_max;
// The status word of a group: word 1 of line 0 of its barrier area (no
// barrier uses it).  Each wait of the group's members that expires adds 1
// there as well as to the process-wide count, so the caller can tell which
// buffers (which launch's rows and head groups) were affected.
constexpr int kSyncStatusWord = 1;
__device__ __forceinline__ void wait_expired(uint32_t* status) {
  atomicAdd(&g_group_wait_timeouts, 1);
  atomicAdd(status, 1u);
}
constexpr int kGroupSyncGroups = 16, kGroupSyncFlags = 8, kGroupSyncLine = 64;
constexpr int kGroupFlatMax = 32;  // groups up to this size use one arrival counter
__device__ __forceinline__ uint32_t group_sense(const uint32_t* sync, int bid) {
  return __hip_atomic_load(&sync[(kGroupSyncGroups + 1 + (bid & (kGroupSyncFlags - 1))) * kGroupSyncLine],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A group barrier with one atomic round trip on the last arrival's path,
// in two halves (group_arrive_rep, group_wait_rep).
// Members arrive on kRepGroups group counters; a group's last arrival adds
// itself, without waiting for the result, to kRepTops replicated top
// counters, and every member polls the replica of its XCD until all groups
// are in.  Two counter sets alternate by launch (`sense`, the flags of
// `sync` read at launch start), so nothing is re-zeroed while a member may
// still read it: after passing, workgroup 0 clears the other set (the next
// launch's) and flips the flags.  Layout: set s's group counters on lines
// 8s..8s+7 of `sync`, its top replicas on lines 8s..8s+7 of `tops` (a second
// barrier area), the flags where group_barrier keeps them.
constexpr int kRepGroups = 8, kRepTops = 8;
static_assert(2 * kRepGroups <= kGroupSyncGroups && 2 * kRepTops <= kGroupSyncGroups + 1,
              "two counter sets fit a barrier area");
// Arrival half: publishes (waits for this workgroup's stores) and arrives.
// The caller may do work that needs no other workgroup's data, then calls
// group_wait_rep with the same arguments.
__device__ __forceinline__ void group_arrive_rep(uint32_t* sync, uint32_t* tops, int bid, int nb,
                                                 uint32_t sense) {
  const uint32_t set = sense & 1u;
  wait_mem();
  dbg_stamp(0, 23);
  __syncthreads();
  dbg_stamp(0, 24);
  if (threadIdx.x == 0) {
    const int g = bid % kRepGroups;
    const uint32_t ng = (uint32_t)((nb - 1 - g) / kRepGroups + 1);
    if (atomicAdd(&sync[(set * kRepGroups + g) * kGroupSyncLine], 1u) == ng - 1u)
      for (int r = 0; r < kRepTops; ++r)
        __hip_atomic_fetch_add(&tops[(set * kRepTops + r) * kGroupSyncLine], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  }
}
// Wait half: returns (to every thread) once all nb members have arrived.
// Workgroup 0 also zeroes `nclr` lines of `clr` (another structure's next
// counter set) with the next set's counters.
__device__ __forceinline__ void group_wait_rep(uint32_t* sync, uint32_t* tops, int bid, int nb, uint32_t sense,
                                               uint32_t* clr = nullptr, int nclr = 0) {
  const uint32_t set = sense & 1u;
  if (threadIdx.x == 0) {
    const uint32_t ngroups = (uint32_t)min(nb, kRepGroups);
    const uint32_t* top = &tops[(set * kRepTops + bid % kRepTops) * kGroupSyncLine];
    const int lim = g_group_spin_max;
    for (int i = 0; __hip_atomic_load(top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < ngroups; ++i) {
      if (i == lim) {
        wait_expired(&sync[kSyncStatusWord]);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  if (bid == 0) {
    const int t = threadIdx.x;
    if (t < kRepGroups) store_dev(&sync[((set ^ 1u) * kRepGroups + t) * kGroupSyncLine], 0u);
    else if (t < kRepGroups + kRepTops)
      store_dev(&tops[((set ^ 1u) * kRepTops + (t - kRepGroups)) * kGroupSyncLine], 0u);
    else if (t < kRepGroups + kRepTops + kGroupSyncFlags)
      store_dev(&sync[(kGroupSyncGroups + 1 + (t - kRepGroups - kRepTops)) * kGroupSyncLine], sense ^ 1u);
    else if (t < kRepGroups + kRepTops + kGroupSyncFlags + nclr)
      store_dev(&clr[(t - kRepGroups - kRepTops - kGroupSyncFlags) * kGroupSyncLine], 0u);
  }
}

__device__ __forceinline__ void group_barrier(uint32_t* sync, int bid, int nb, uint32_t sense) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    // a small group arrives on one counter (one atomic round trip); a large
    // one on kGroupSyncGroups counters, whose last arrivals meet on a top one
    const int ngrp = nb <= kGroupFlatMax ? 1 : kGroupSyncGroups;
    const int g = bid % ngrp;
    const uint32_t ng = (uint32_t)((nb - 1 - g) / ngrp + 1);
    bool last = false;
    if (atomicAdd(&sync[g * kGroupSyncLine], 1u) == ng - 1u) {
      const uint32_t ngroups = (uint32_t)min(nb, ngrp);
      last = ngrp == 1 || atomicAdd(&sync[kGroupSyncGroups * kGroupSyncLine], 1u) == ngroups - 1u;
    }
    if (last) {
      // re-zero the counters for the next launch (each barrier is used once
      // per launch, and the launch boundary orders these stores before the
      // next launch's arrivals, so the flags need not wait for them)
      for (int i = 0; i <= kGroupSyncGroups; ++i) store_dev(&sync[i * kGroupSyncLine], 0u);
      for (int f = 0; f < kGroupSyncFlags; ++f)
        store_dev(&sync[(kGroupSyncGroups + 1 + f) * kGroupSyncLine], sense ^ 1u);
    } else {
      const int lim = g_group_spin_max;
      for (int i = 0; group_sense(sync, bid) == sense; ++i) {
        if (i == lim) {
          wait_expired(&sync[kSyncStatusWord]);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
  }
  __syncthreads();
}

// Exclusive prefix count of a per-thread flag in thread order; *total gets
// the block's count.  wave_tmp: one word per wave.
__device__ __forceinline__ uint32_t block_flag_scan(bool f, uint32_t* wave_tmp, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave, nw = blockDim.x / kWave;
  const uint64_t m = __ballot(f);
  const uint32_t in_wave = (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) wave_tmp[wv] = (uint32_t)__popcll(m);
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    const uint32_t x = wave_tmp[i];
    before += (i < wv) ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + in_wave;
}

// Block-wide reduction of four per-thread values; OPn: 0 = sum, 1 = min,
// 2 = max.  wave_tmp: 4 words per wave.
template <int OP>
__device__ __forceinline__ uint32_t red_op(uint32_t a, uint32_t b) {
  return OP == 0 ? a + b : (OP == 1 ? min(a, b) : max(a, b));
}
template <int OP0, int OP1, int OP2, int OP3>
__device__ __forceinline__ uint4 block_reduce4(uint4 v, uint32_t* wave_tmp) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave, nw = blockDim.x / kWave;
  v.x = wave_scan_incl<OP0>(v.x);
  v.y = wave_scan_incl<OP1>(v.y);
  v.z = wave_scan_incl<OP2>(v.z);
  v.w = wave_scan_incl<OP3>(v.w);
  if (lane == kWave - 1) *reinterpret_cast<uint4*>(&wave_tmp[4 * wv]) = v;
  __syncthreads();
  uint4 r = *reinterpret_cast<const uint4*>(&wave_tmp[0]);
  for (int i = 1; i < nw; ++i) {
    const uint4 x = *reinterpret_cast<const uint4*>(&wave_tmp[4 * i]);
    r.x = red_op<OP0>(r.x, x.x);
    r.y = red_op<OP1>(r.y, x.y);
    r.z = red_op<OP2>(r.z, x.z);
    r.w = red_op<OP3>(r.w, x.w);
  }
  __syncthreads();
  return r;
}


}  // namespace dsa
