// Shared device and host helpers of libbcm_event_scan (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <type_traits>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "bcm_event_scan.h"

namespace bcm {

constexpr int kWave = 64;
// Sequence steps per restore / gather tile (one 64-bit mask per tile).
constexpr int kTile = 64;

// ---------------------------------------------------------------- errors
// Defined in abi.hip; thread-local so concurrent callers do not clobber it.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* fn);
// The restore backward's fix-up pass (restore.hip): closes the runs that
// cross tiles from the per-(tile, channel) head / tail / last-event arrays.
int restore_bwd_fix(int64_t nT, int64_t n_rows, const float* head, const float* tail, const int32_t* tend,
                    float* dy, int64_t n_events, hipStream_t stream, const char* fn);
// Zero fill with a kernel (abi.hip).
int zero_bytes(void* ptr, int64_t bytes, hipStream_t s, const char* fn);

inline int64_t bitmask_words(int64_t L) { return ((L + 1023) / 1024) * 32; }
inline int64_t tile_count(int64_t L) { return (L + kTile - 1) / kTile; }
inline hipStream_t hs(bcm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// Compute units of the current device.
inline int device_cus() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
  return v;
}
// LDS bytes one workgroup may use on the current device (static + dynamic).
inline int max_lds_bytes() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) return 65536;
  return v;
}

// ---------------------------------------------------------------- dtypes
using bf16 = __hip_bfloat16;
using f16 = __half;

template <typename T> __device__ __forceinline__ float to_f(T v);
template <> __device__ __forceinline__ float to_f<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f<uint8_t>(uint8_t v) { return (float)v; }
template <> __device__ __forceinline__ float to_f<f16>(f16 v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f<bf16>(bf16 v) { return __bfloat162float(v); }

template <typename T> __device__ __forceinline__ T from_f(float v);
template <> __device__ __forceinline__ float from_f<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f<f16>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float v) { return __float2bfloat16(v); }

inline size_t dtype_size(int dt) { return dt == BCM_F32 ? 4 : (dt == BCM_U8 ? 1 : 2); }
inline bool dtype_ok(int dt) { return dt == BCM_F32 || dt == BCM_F16 || dt == BCM_BF16; }

// Calls fn(T{}) with the C++ type of a dtype code.
template <typename F> inline void dispatch_dtype(int dt, F&& fn) {
  if (dt == BCM_F32) fn(float{});
  else if (dt == BCM_F16) fn(f16{});
  else fn(bf16{});
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// MI355X has 8 XCDs, each with its own L2; workgroup i of a launch runs on
// XCD i % 8. xcd_block() maps the hardware block id to a logical one so that
// every XCD works through a contiguous range of logical blocks: data that
// neighbouring logical blocks share is then fetched into one L2, not eight.
// A bijection on [0, nblk) for any nblk.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_block(int bid, int nblk) {
  const int per = nblk / kXcds, rem = nblk % kXcds;
  const int x = bid % kXcds, i = bid / kXcds;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

// Orders LDS traffic between the lanes of one wave (no block barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_sum(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

// Inclusive prefix max over the 64 lanes.
__device__ __forceinline__ int wave_incl_max(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v = max(v, o);
  }
  return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v |= __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, kWave));
  return v;
}

// Sum over aligned groups of G lanes (result in every lane of the group).
template <int G> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, G);
  return v;
}

// 64-bit event mask of one 64-step tile (bitmask words 2j and 2j+1).
__device__ __forceinline__ uint64_t tile_mask(const uint32_t* row, int64_t j) {
  const uint2 w = *reinterpret_cast<const uint2*>(row + 2 * j);
  return (uint64_t)w.x | ((uint64_t)w.y << 32);
}

// ------------------------------------------------------ buffer resources
// A raw buffer resource over [base, base + bytes). Lanes whose byte offset
// is out of range read 0 and their stores are dropped by the hardware, which
// gives branch-free predication (no exec-mask branches, no waits).
constexpr uint32_t kBufOOB = 0x80000000u;
constexpr int kBufFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes > 0x7fffffffll ? 0x7fffffff : (int32_t)(bytes < 0 ? 0 : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, kBufFlags);
}

// Cache policy of a buffer access. kStream marks data read or written once
// (the dense [B, L, D] / [B, D, L] streams): non-temporal, so written lines are
// not kept dirty in the last-level cache, where their later write-back would
// compete with the next kernel's traffic, and read lines do not displace the
// event arrays that one kernel hands to the next.
constexpr int kKeep = 0;
constexpr int kStream = 2;  // nt

template <typename T, int POL = kKeep>
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL));
  } else if constexpr (std::is_same<T, bf16>::value) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL) << 16);
  } else {
    const unsigned short b = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL);
    return __half2float(*reinterpret_cast<const f16*>(&b));
  }
}

__device__ __forceinline__ int32_t buf_load_i32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

template <int POL = kKeep> __device__ __forceinline__ void buf_store_f32(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, POL);
}
// Store v converted to T (round to nearest even for the 16-bit types).
template <typename T, int POL = kKeep>
__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  if constexpr (sizeof(T) == 4) {
    buf_store_f32<POL>(r, off, v);
  } else {
    const T h = from_f<T>(v);
    unsigned short b;
    __builtin_memcpy(&b, &h, 2);
    __builtin_amdgcn_raw_buffer_store_b16(b, r, off, 0, POL);
  }
}

// Non-temporal (streaming) plain loads and stores of raw bits.
template <typename V> __device__ __forceinline__ V ld_stream(const V* p) { return __builtin_nontemporal_load(p); }
template <typename V> __device__ __forceinline__ void st_stream(V v, V* p) { __builtin_nontemporal_store(v, p); }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// One element of T read with streaming policy (its raw bits).
template <typename T> __device__ __forceinline__ T ld_stream_elem(const T* p) {
  using U = typename std::conditional<sizeof(T) == 4, uint32_t,
                                      typename std::conditional<sizeof(T) == 2, unsigned short, uint8_t>::type>::type;
  const U b = ld_stream(reinterpret_cast<const U*>(p));
  T h;
  __builtin_memcpy(&h, &b, sizeof(T));
  return h;
}

// The value itself, hidden from common-subexpression elimination and
// loop-invariant code motion: offsets derived from it are recomputed where
// they are used instead of being kept live in registers.
template <typename V> __device__ __forceinline__ V opaque(V v) {
  asm volatile("" : "+v"(v));
  return v;
}

// DPP lane permutations inside rows of 16 lanes (VALU, no LDS round trip).
template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- lane 7-i inside each 8 lanes

// Max over the 64 lanes with DPP row steps and four lane reads (no LDS).
__device__ __forceinline__ int wave_max_dpp(int v) {
  v = max(v, (int)dpp<kDppXor1>((uint32_t)v));
  v = max(v, (int)dpp<kDppXor2>((uint32_t)v));
  v = max(v, (int)dpp<kDppHalfMirror>((uint32_t)v));
  v = max(v, (int)dpp<0x140>((uint32_t)v));  // row_mirror: every lane holds its row's max
  const int a = max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16));
  const int b = max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48));
  return max(a, b);
}

// Inclusive prefix sum over the 64 lanes: DPP row scans, then the row
// totals (lanes 15, 31, 47) read as scalars. No LDS round trips.
__device__ __forceinline__ int wave_incl_sum_dpp(int v) {
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1, zero fill
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
  const int t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31);
  const int t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane_id() >> 4;
  return v + (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
}

// exp2 of a clamped exponent: the decay of the reference scan
// (selective_scan_common.h:45-52 clamps Δ·A·log2e to [-126, 126]).
__device__ __forceinline__ float decay(float e) {
  return __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(e, -126.0f, 126.0f));
}

}  // namespace bcm
