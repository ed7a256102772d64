// Constants and device helpers shared by the depthwise scan kernels
// (scan.hip: lane groups over items; scan_sl.hip: lanes over states).
#pragma once
#include "bcm_common.hpp"

namespace bcm {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kScanThreads = 512;   // workgroup size bound (8 waves)
template <int G, bool BWD> constexpr int kScanThreadsG = kScanThreads;
constexpr int kTabK = 64;           // gaps k = 1..kTabK (at least) come from the decay table
constexpr int kTabStride = kTabK + 1;  // entry 0 = 1.0: the decay of a padding item
constexpr int kTabMaxN = 64;        // the table is used when dstate <= kTabMaxN
constexpr int kTabElems = kTabMaxN * 129;  // its static LDS array (33 KB)
// Longest gap in the table for dstate N: kTabElems / N entries per row, at
// most 257 (gaps up to 128 at N = 64, 256 at N <= 32), so sparse streams
// stay on it.
__host__ __device__ constexpr int tab_gaps(int N) { return (kTabElems / N < 257 ? kTabElems / N : 257) - 1; }
constexpr int kSchedBlock = 8;      // items per scheduling block in the backward's long passes
constexpr int kXChunk = 2048;       // events per saved-state chunk of x (selective_scan.cpp:795)
constexpr int kFixSlots = 4;        // backward: item slots with a long gap that the table path fixes up
constexpr int kFixMinR = 16;        // ... in shapes of at least this many items per lane (the fix-up's
                                    // registers would cost R = 8 its fourth wave per SIMD)

// Decay of an item from the table: `tb` is the item's byte offset in a table
// row, `row` the state's row base in bytes (wave-uniform), so each read costs
// one address add.
__device__ __forceinline__ float tab(const float* sT, uint32_t row, uint32_t tb) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(sT) + (row + tb));
}

// Decay table of workgroup d: T[s][0] = 1 (padding), T[s][k] = the decay of
// gap k (same expression and rounding as the per-event path), rows of
// tab_gaps(N) + 1 entries. nthr: the workgroup's threads.
__device__ __forceinline__ void build_decay_table(float* sT, const bcm_scan_args& a, int d, float dti, float dta,
                                                  int nthr) {
  const int N = a.dstate;
  const int tstr = tab_gaps(N) + 1;
  for (int i = threadIdx.x; i < N * tstr; i += nthr) {
    const int s = i / tstr, q = i - s * tstr;
    sT[i] = q == 0 ? 1.0f : decay(fmaf(dti, (float)(q - 1), dta) * (a.A[(int64_t)d * N + s] * kLog2e));
  }
}

// Barrier after the LDS set-up, then: true if some decay exponent of
// workgroup d can be positive (A > 0 or Δ < 0); lane products are then
// multiplied out exactly. Every thread reads the N values of A·log2e from
// LDS (same sign as A), so the kernel needs no static LDS for a vote.
__device__ __forceinline__ bool exact_products(const float* sAl, int N, float dti, float dta) {
  __syncthreads();
  bool f = dti < 0.0f || dta < 0.0f;
  for (int s = 0; s < N; ++s) f |= sAl[s] > 0.0f;
  return f;
}

// Length order of model channel d's channels (ch = d + b·dim, b < n_per_d),
// used when channels span several passes: ord[rank] = b, longest first,
// ties by b. keys is LDS scratch of n_per_d ints, dead after the return.
// nthr: the workgroup's threads.
constexpr int kSortMax = 256;  // most channels per model channel that are ranked
__device__ __forceinline__ void rank_channels(const bcm_scan_args& a, int d, int n_per_d, int* keys, int* ord,
                                              int nthr) {
  for (int i = threadIdx.x; i < n_per_d; i += nthr) {
    const int64_t ch = (int64_t)d + (int64_t)i * a.dim;
    keys[i] = a.cu_seqlens[ch + 1] - a.cu_seqlens[ch];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_per_d; i += nthr) {
    const int ki = keys[i];
    int r = 0;
    for (int q = 0; q < n_per_d; ++q) {
      const int kq = keys[q];
      r += (kq > ki) | ((kq == ki) & (q < i));
    }
    ord[r] = i;
  }
  __syncthreads();
}

// Value i of model channel d's parameter-gradient block (dA[d, :],
// dW_B[d, :], dW_C[d, :], ddt_idle[d], ddt_active[d], dD[d]).
__device__ __forceinline__ void store_param_grad(const bcm_scan_args& a, int d, int N, int i, float v) {
  if (i < N) a.dA[(int64_t)d * N + i] = v;
  else if (i < 2 * N) a.dW_B[(int64_t)d * N + (i - N)] = v;
  else if (i < 3 * N) a.dW_C[(int64_t)d * N + (i - 2 * N)] = v;
  else if (i == 3 * N) a.ddt_idle[d] = v;
  else if (i == 3 * N + 1) a.ddt_active[d] = v;
  else if (a.dD) a.dD[d] = v;
}

// A channel of n events longer than the caller's max_seqlen: its saved
// states (x, chunk_g) have fewer rows than its passes need. Flagged in the
// caller's status word (a plain vector store; several lanes may write it).
__device__ __forceinline__ void report_seqlen(const bcm_scan_args& a, int n) {
  if (n > a.max_seqlen && a.status) a.status[0] = BCM_SCAN_SEQLEN_EXCEEDED;
}

// Dense gradient rows of the fused gather backward (bcm_scan_bwd_rows): the
// extraction's event index of every channel row and the [NC, L] output.
struct ScanRows {
  const uint32_t* bitmask;  // channel ch reads mask row ch / mrd (words W)
  int64_t mrd, W;
  const int32_t* ts;        // [NC, nT + 1] absolute index of each tile's first event
  int64_t nT, L;
  void* dx;                 // [NC, L] of T
};

// ---- state-lane kernels (scan_sl.hip) for dstate 16: lane = (channel, state)
constexpr int kSLN = 16;     // dstate they serve
constexpr int kSLPass = 32;  // events per pass (one state per lane): chunk_g rows, the backward's unit of work
// Events per pass of the state-lane kernels for a dstate they serve.
int sl_pass_len(int dstate);
// True when the state-lane kernels run this scan (forward and backward
// alike, so that chunk_g has the passes the backward expects).
bool sl_applies(const bcm_scan_args& a);
// The process-wide family setting (BCM_SCAN_AUTO / _LANES / _ITEMS).
int scan_family();
// Workgroups per model channel the state-lane kernels use for these arguments.
int sl_split(const bcm_scan_args& a);
int sl_launch_fwd(const bcm_scan_args& a, hipStream_t s, const char* fn);
int sl_launch_bwd(const bcm_scan_args& a, hipStream_t s, const char* fn, const ScanRows* rw);
// Sums S workgroups' parameter-gradient partials (k_scan_param_reduce, scan.hip).
int sl_param_reduce(const bcm_scan_args& a, int S, hipStream_t s, const char* fn);
// True when sl_launch_bwd writes the dense rows of rw itself.
bool sl_rows_fusable(const bcm_scan_args& a, const bcm_scan_rows& r);

}  // namespace bcm
