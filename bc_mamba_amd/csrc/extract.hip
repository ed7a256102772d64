// Stage 1: event extraction, expansion and the event gather (fwd / bwd).
//
// Reference behaviour: csrc/extract/extract_events_cuda.cu
//   count_base_kernel :192-208, DeviceScan :361-372, fill_base_kernel
//   :226-312, build_logical_cu_kernel :449-467, expand_events_direct_kernel
//   :482-509, gather_events_fwd2_kernel :629-642, scatter_events_bwd2 :649-662.
//
// MI355X design: one wave per membrane row. The count pass reads the
// membrane once with 16-byte loads and packs the threshold bits into a
// bitmask (1 bit per step, 1/32 of an fp32 membrane); the fill pass reads
// only that bitmask, turns each lane's 32-step word into events with popcount
// and a wave prefix sum, stages the segment's event times in LDS and writes
// ch / t / k (and, fused, the gathered x values and the tile table) with
// coalesced stores.
#include "bcm_common.hpp"

#include <type_traits>

namespace bcm {

// ------------------------------------------------------------------ count
// Sum and maximum of the block's row counts (one value per wave, uniform in
// the wave) to bsum[blockIdx] / bmax[blockIdx]. Every wave of the block
// calls it once (rows past the end with 0).
// Threads per block of the count and fill launches: kernels use the constant,
// not blockDim (whose load from the launch's implicit arguments would come
// first, one more round trip before any work).
constexpr int kExBlock = 256;

__device__ __forceinline__ void block_totals(int cnt, int32_t* bsum, int32_t* bmax) {
  __shared__ int s_c[4];
  if (lane_id() == 0) s_c[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int sm = 0, mx = 0;
    for (int w = 0; w < kExBlock / kWave; ++w) {
      sm += s_c[w];
      mx = max(mx, s_c[w]);
    }
    bsum[blockIdx.x] = sm;
    bmax[blockIdx.x] = mx;
  }
}

// One wave per row. A batch of up to 8 groups (8 x 16 bytes per lane) is
// loaded before any of it is used, so a row of 2048 fp32 steps is one round
// trip to memory.
// BLK: each block also writes its rows' event sum and maximum row count to
// bsum[blk] / bmax[blk] (one barrier, no atomics), which the fill pass turns
// into row offsets itself (no separate offsets scan).
template <typename T, bool VEC, bool BLK>
__global__ __launch_bounds__(256) void k_count(const T* __restrict__ x, int64_t n_rows, int64_t L, float thr,
                                               uint32_t* __restrict__ bitmask, int64_t W,
                                               int32_t* __restrict__ counts, int32_t* __restrict__ bsum,
                                               int32_t* __restrict__ bmax) {
  constexpr int PER = 16 / sizeof(T);  // steps per lane per group
  constexpr int GS = kWave * PER;      // steps per group
  constexpr int LPW = 32 / PER;        // lanes per 32-bit word
  constexpr int WPG = GS / 32;         // words per group
  constexpr int BATCH = 8;
  // the arguments of the first loads come in the first batch of argument
  // loads (one wait), not on demand one batch later
  asm volatile("" ::"s"(x), "s"(L), "s"(n_rows), "s"(thr), "s"(bitmask), "s"(W));
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (kExBlock / kWave) + threadIdx.x / kWave;
  // the row's bits and event count (0 for a row past the end)
  auto count_row = [&]() {
    const T* xr = x + row * L;
    uint32_t* br = bitmask + row * W;
    int cnt = 0;
    const int64_t ng = (L + GS - 1) / GS;
    for (int64_t g0 = 0; g0 < ng; g0 += BATCH) {
      uint32_t bits[BATCH];
      if (VEC && (g0 + BATCH) * GS <= L) {
        uint4 raw[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const u32x4 t = ld_stream(reinterpret_cast<const u32x4*>(xr + (g0 + i) * GS + lane * PER));
          __builtin_memcpy(&raw[i], &t, 16);
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const T* v = reinterpret_cast<const T*>(&raw[i]);
          bits[i] = 0;
#pragma unroll
          for (int e = 0; e < PER; ++e) bits[i] |= (uint32_t)(to_f(v[e]) > thr) << e;
        }
      } else {  // tail batch: full groups still use 16-byte loads
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const int64_t t0 = (g0 + i) * GS + (int64_t)lane * PER;
          bits[i] = 0;
          if (VEC && t0 + PER <= L) {
            const u32x4 raw = ld_stream(reinterpret_cast<const u32x4*>(xr + t0));
            const T* v = reinterpret_cast<const T*>(&raw);
#pragma unroll
            for (int e = 0; e < PER; ++e) bits[i] |= (uint32_t)(to_f(v[e]) > thr) << e;
          } else {
#pragma unroll
            for (int e = 0; e < PER; ++e)
              if (t0 + e < L) bits[i] |= (uint32_t)(to_f(xr[t0 + e]) > thr) << e;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        if (g0 + i < ng) {
          cnt += __popc(bits[i]);
          // pack the lanes' PER-bit pieces of one 32-step word (DPP, no LDS)
          uint32_t w = bits[i] << (PER * (lane % LPW));
          if constexpr (LPW >= 2) w |= dpp<kDppXor1>(w);
          if constexpr (LPW >= 4) w |= dpp<kDppXor2>(w);
          if constexpr (LPW >= 8) w |= dpp<kDppHalfMirror>(w);
          if (lane % LPW == 0) br[(g0 + i) * WPG + lane / LPW] = w;
        }
      }
    }
    return wave_sum(cnt);
  };
  const int cnt = row < n_rows ? count_row() : 0;
  if (row < n_rows && lane == 0) counts[row] = cnt;
  if constexpr (BLK) block_totals(cnt, bsum, bmax);  // every wave, one barrier
}

// ------------------------------------------------- spikes straight to bits
// The straight-through spike head (SpikeSamplerSurrogate mode "ste",
// e_model.py:233-254: s = (p >= thr) + p - p, evaluated left to right) on
// p [B, L, Dm], writing the event bitmask of the rows (b, d) directly: no
// transposed copy of s and no count pass over it. One wave per (b, 64
// channels, 64-step tile): lane d reads p[b, l, d] for the tile's 64 steps
// (each a coalesced 256-byte row of the wave), packs the 64 bits of its row
// into one mask word pair and, when s is requested, writes s in p's layout.
// Bits past L stay 0; the padding words of a row are not written.
template <typename T>
__global__ __launch_bounds__(256) void k_spike_bits(const T* __restrict__ p, int64_t B, int64_t L, int64_t Dm,
                                                    float thr, uint32_t* __restrict__ bitmask, int64_t W,
                                                    T* __restrict__ s_out) {
  const int lane = lane_id();
  const int64_t nT = (L + kTile - 1) / kTile, nG = (Dm + kWave - 1) / kWave;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (gw >= B * nG * nT) return;
  const int64_t j = gw % nT, g = (gw / nT) % nG, b = gw / (nT * nG);
  const int64_t d = g * kWave + lane;
  if (d >= Dm) return;
  const int64_t t0 = j * kTile;
  const int n = (int)(L - t0 < kTile ? L - t0 : kTile);
  const T* pr = p + (b * L + t0) * Dm + d;
  thr = to_f(from_f<T>(thr));  // torch compares in p's dtype
  float v[kTile];
#pragma unroll
  for (int l = 0; l < kTile; ++l) v[l] = l < n ? to_f(pr[(int64_t)l * Dm]) : 0.0f;  // all 64 loads in flight
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int l = 0; l < kTile; ++l) {
    const bool hit = l < n && v[l] >= thr;
    if (l < 32) lo |= (uint32_t)hit << l;
    else hi |= (uint32_t)hit << (l - 32);
  }
  *reinterpret_cast<uint2*>(bitmask + (b * Dm + d) * W + 2 * j) = make_uint2(lo, hi);
  if (s_out) {
    T* sr = s_out + (b * L + t0) * Dm + d;
#pragma unroll
    for (int l = 0; l < kTile; ++l) {
      if (l < n) {
        // the STE value rounded as torch rounds it: the hard spike in p's
        // dtype, plus p, minus p
        const float h = to_f(from_f<T>(v[l] >= thr ? 1.0f : 0.0f));
        const float a = to_f(from_f<T>(h + v[l]));
        sr[(int64_t)l * Dm] = from_f<T>(a - v[l]);
      }
    }
  }
}

// Counts and block totals (as k_count with BLK) from a finished bitmask:
// one wave per row.
__global__ __launch_bounds__(256) void k_count_bits(const uint32_t* __restrict__ bitmask, int64_t n_rows, int64_t L,
                                                    int64_t W, int32_t* __restrict__ counts,
                                                    int32_t* __restrict__ bsum, int32_t* __restrict__ bmax) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  int cnt = 0;
  if (row < n_rows) {
    const int64_t nw = (L + 31) / 32;
    for (int64_t w = lane; w < nw; w += kWave) cnt += __popc(bitmask[row * W + w]);
    cnt = wave_sum(cnt);
    if (lane == 0) counts[row] = cnt;
  }
  block_totals(cnt, bsum, bmax);
}

// ------------------------------------------------------------------- scan
// One block: exclusive offsets of the per-row counts, total and maximum.
// cu[0] = 0, cu[i+1] = counts[0] + ... + counts[i]; meta = (total, max).
// One workgroup: 8 counts per thread (two 16-byte loads), DPP wave scans,
// one barrier per 8192 counts.
// maxsrc != NULL: meta's maximum is taken over maxsrc[0..n) instead of the
// counts (the block maxima when the counts are block sums).
template <bool VEC>
__global__ __launch_bounds__(1024) void k_scan_counts(const int32_t* __restrict__ counts, int64_t n,
                                                      int32_t* __restrict__ cu, int32_t* __restrict__ meta,
                                                      const int32_t* __restrict__ maxsrc) {
  constexpr int ITEMS = 8;
  __shared__ int s_wsum[2][16];
  __shared__ int s_wmax[16];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int nw = blockDim.x / kWave;
  int carry = 0, mx = 0, par = 0;
  for (int64_t base = 0; base < n; base += (int64_t)blockDim.x * ITEMS, par ^= 1) {
    const int64_t i0 = base + (int64_t)tid * ITEMS;
    int v[ITEMS];
    if (VEC && i0 + ITEMS <= n) {
      const int4 a = *reinterpret_cast<const int4*>(counts + i0);
      const int4 b = *reinterpret_cast<const int4*>(counts + i0 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) v[i] = i0 + i < n ? counts[i0 + i] : 0;
    }
    int sum = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      sum += v[i];
      mx = max(mx, maxsrc ? (i0 + i < n ? maxsrc[i0 + i] : 0) : v[i]);
    }
    const int incl = wave_incl_sum_dpp(sum);
    if (lane == kWave - 1) s_wsum[par][wave] = incl;  // double-buffered: one barrier per pass
    __syncthreads();
    int woff = 0, total = 0;
    for (int w = 0; w < nw; ++w) {
      const int x = s_wsum[par][w];
      woff += w < wave ? x : 0;
      total += x;
    }
    int run = carry + woff + incl - sum;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      run += v[i];
      if (i0 + i < n) cu[i0 + i + 1] = run;
    }
    carry += total;
  }
  mx = wave_max_dpp(mx);
  if (lane == 0) s_wmax[wave] = mx;
  __syncthreads();
  if (tid == 0) {
    int m = 0;
    for (int w = 0; w < nw; ++w) m = max(m, s_wmax[w]);
    cu[0] = 0;
    // (total, max) in one 64-bit system-scope store: written through to
    // memory, so a host polling pinned memory sees both values at once,
    // before the kernel ends and without an event
    const uint64_t packed = (uint64_t)(uint32_t)carry | ((uint64_t)(uint32_t)m << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(meta), packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// ------------------------------------------------------------------- fill
constexpr int kFillSeg = 64 * 32;  // steps per segment (one word per lane)

// The depthwise causal conv + SiLU evaluated at the events (fill with
// KM > 0): row lc of the conv input is x + (lc / dim) * sb + (lc % dim) * sd.
struct ConvAt {
  const float* w;     // [dim, K]
  const float* bias;  // [dim] or NULL
  int K, dim, silu;
  int64_t sb, sd;     // element strides of the batch and channel index
};

// silu(bias + sum_k w[k] x[t-(K-1)+k]) at step t of row xr, x = 0 before
// t = 0: the expression and order of bcm_causal_conv1d_fwd, so the value
// (after rounding to T) is the one the dense conv writes at (row, t).
template <typename T, int KM>
__device__ __forceinline__ T conv_at(const T* __restrict__ xr, int t, const float* wk, float b0, int K, bool silu) {
  float xv[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) {  // the taps' loads in flight together
    const int tt = t - (K - 1) + k;
    xv[k] = (k < K && tt >= 0) ? to_f(xr[tt]) : 0.0f;  // cached: an event's taps share lines
  }
  float pre = b0;
#pragma unroll
  for (int k = 0; k < KM; ++k)
    if (k < K) pre = fmaf(wk[k], xv[k], pre);
  return from_f<T>(silu ? pre / (1.0f + __expf(-pre)) : pre);
}

// BLK: the row offsets come from the count pass's block sums (bsum/bmax,
// one per 4 rows) and the counts of the block's rows before each row; the
// fill writes cu_seqlens itself. With bpre == NULL (few blocks) each block
// adds up the sums of the blocks before it, and block 0 also writes meta =
// (E, max count) (one 64-bit store written through to memory, so a host may
// poll it while the fill runs); that is quadratic in the block count, so
// for many blocks a one-workgroup scan of the block sums runs first
// (k_scan_counts over bsum: bpre[i] = sum of the blocks before block i, and
// meta) and each block reads its offset from bpre.
// KM = 0: x_ev gathers x at the events; KM = 4 (width exactly 4) or 8 (any
// width <= 8): x_ev is the conv + SiLU of x (ConvAt) at the events.
template <typename T, bool GATHER, bool TILES, bool BLK, int KM = 0>
__global__ __launch_bounds__(256) void k_fill(const uint32_t* __restrict__ bitmask, int64_t W,
                                              const int32_t* __restrict__ base_cu, int64_t n_rows, int64_t L,
                                              int expand, const T* __restrict__ x, int32_t* __restrict__ ch_ids,
                                              int32_t* __restrict__ t_steps, int32_t* __restrict__ k_flat,
                                              T* __restrict__ x_ev, int32_t* __restrict__ tile_start, int64_t nT,
                                              int32_t* __restrict__ head_flags, const int32_t* __restrict__ counts,
                                              const int32_t* __restrict__ bsum, const int32_t* __restrict__ bmax,
                                              const int32_t* __restrict__ bpre, int32_t* __restrict__ meta,
                                              int32_t* __restrict__ cu_out, const ConvAt cv) {
  static_assert(KM == 0 || GATHER, "the conv form writes x_ev");
  // the arguments of the first loads come in the first batch of argument
  // loads (one wait), not on demand batch after batch
  asm volatile("" ::"s"(bitmask), "s"(W), "s"(n_rows), "s"(L), "s"(counts), "s"(bsum));
  __shared__ int32_t s_t[4][kFillSeg];
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int64_t c = (int64_t)blockIdx.x * 4 + wave;
  // the first segment's bitmask word does not depend on the offsets: its
  // load is in flight while they are worked out
  const bool live = c < n_rows;
  const int64_t nwords = (L + 31) / 32;
  const uint32_t* br = bitmask + (live ? c : 0) * W;
  // unconditional (a clamped index, the value selected where it is used), so
  // that no wait for it comes before the offsets' loads are issued
  const uint32_t word_raw = br[lane < nwords ? lane : 0];
  const bool word_ok = live && lane < nwords;
  int32_t cu0, n;
  if constexpr (BLK) {
    __shared__ int s_part[4][2];
    const int64_t r0 = (int64_t)blockIdx.x * 4;
    int cb[4];  // the block's row counts (clamped loads issued together, then selected)
#pragma unroll
    for (int q = 0; q < 4; ++q) cb[q] = counts[r0 + q < n_rows ? r0 + q : n_rows - 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) cb[q] = r0 + q < n_rows ? cb[q] : 0;
    const int64_t nblk = (n_rows + 3) / 4;
    const bool first = blockIdx.x == 0 && bpre == nullptr;
    int sm = 0, mx = 0;  // blocks before this one (all blocks for block 0's totals)
    const int64_t lim = bpre ? 0 : (first ? nblk : (int64_t)blockIdx.x);
    for (int64_t i0 = 0; i0 < lim; i0 += 8 * kExBlock) {  // 8 independent loads per thread in flight
      int vs[8], vm[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int64_t i = i0 + q * kExBlock + threadIdx.x;
        vs[q] = i < lim ? bsum[i] : 0;
        vm[q] = (first && i < lim) ? bmax[i] : 0;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        sm += vs[q];
        mx = max(mx, vm[q]);
      }
    }
    sm = wave_sum(sm);
    mx = wave_max(mx);
    if (lane == 0) {
      s_part[wave][0] = sm;
      s_part[wave][1] = mx;
    }
    __syncthreads();
    int before = 0, total_max = 0;
    for (int w = 0; w < 4; ++w) {
      before += s_part[w][0];
      total_max = max(total_max, s_part[w][1]);
    }
    if (bpre) before = bpre[blockIdx.x];
    if (first && threadIdx.x == 0) {
      const uint64_t packed = (uint64_t)(uint32_t)before | ((uint64_t)(uint32_t)total_max << 32);
      __hip_atomic_store(reinterpret_cast<uint64_t*>(meta), packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (first) before = 0;
    if (!live) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) before += q < wave ? cb[q] : 0;
    cu0 = before;
    n = cb[wave];
    for (int r = lane; r < expand; r += kWave) cu_out[c * expand + r] = cu0 * expand + r * n;
    if (c == n_rows - 1 && lane == 0) cu_out[n_rows * expand] = (cu0 + n) * expand;
  } else {
    if (!live) return;
    cu0 = base_cu[c];
    n = base_cu[c + 1] - cu0;
  }
  if (TILES && lane == 0) {
    for (int r = 0; r < expand; ++r)
      tile_start[(c * expand + r) * (nT + 1) + nT] = cu0 * expand + r * n + n;
  }
  if (n <= 0 && !TILES) return;
  int32_t* st = s_t[wave];
  int prev_t = -1;
  int off = 0;
  for (int64_t w0 = 0; w0 < nwords; w0 += kWave) {
    const int64_t w = w0 + lane;
    const uint32_t word = w0 == 0 ? (word_ok ? word_raw : 0u) : (w < nwords ? br[w] : 0u);
    const int pc = __popc(word);
    const int incl = wave_incl_sum(pc);
    const int excl = incl - pc;
    const int seg_cnt = __shfl(incl, kWave - 1, kWave);
    const int last_t = word ? (int)(32 * w + 31 - __clz((int)word)) : -1;
    const int seg_last = wave_max(last_t);
    if (TILES && (w % 2 == 0) && (w / 2 < nT)) {
      for (int r = 0; r < expand; ++r)
        tile_start[(c * expand + r) * (nT + 1) + w / 2] = cu0 * expand + r * n + off + excl;
    }
    uint32_t ww = word;
    int pos = excl;
    while (ww) {
      const int b = __ffs((int)ww) - 1;
      ww &= ww - 1;
      st[pos++] = (int)(32 * w + b);
    }
    wave_sync();
    // write-out in batches of FB events per lane: the gathers of a batch are
    // in flight together and the index stores never wait on them. 8 for the
    // plain gather (a row's ~300 events in one batch at 15 % density: 22.9 ->
    // 21.0 us at config 1); 4 for the conv form, whose 4 taps per event
    // already fill the queue (8 there: 39 -> 48 us at config 4)
    constexpr int FB = KM > 0 ? 4 : 8;
    for (int r = 0; r < expand; ++r) {
      const int64_t lc = c * expand + r;
      const int64_t obase = (int64_t)cu0 * expand + (int64_t)r * n + off;
      // conv form: the channel's taps and input row (wave-uniform)
      constexpr int KW = KM > 0 ? KM : 1;
      float wk[KW];
      float b0 = 0.0f;
      const T* xr = x + lc * L;
      if constexpr (KM > 0) {
        const int dch = (int)(lc % cv.dim);
#pragma unroll
        for (int k = 0; k < KM; ++k) wk[k] = k < cv.K ? cv.w[(int64_t)dch * cv.K + k] : 0.0f;
        b0 = cv.bias ? cv.bias[dch] : 0.0f;
        xr = x + (lc / cv.dim) * cv.sb + (int64_t)dch * cv.sd;
      }
      for (int i0 = 0; i0 < seg_cnt; i0 += FB * kWave) {
        int tv[FB];
        T xv[FB];
#pragma unroll
        for (int q = 0; q < FB; ++q) {
          const int i = i0 + q * kWave + lane;
          tv[q] = i < seg_cnt ? st[i] : 0;
          if constexpr (KM > 0) xv[q] = conv_at<T, KM>(xr, tv[q], wk, b0, KM == 4 ? 4 : cv.K, cv.silu != 0);
          else if (GATHER) xv[q] = ld_stream_elem(xr + tv[q]);
        }
#pragma unroll
        for (int q = 0; q < FB; ++q) {
          const int i = i0 + q * kWave + lane;
          if (i < seg_cnt) {
            const int tp = i > 0 ? st[i - 1] : prev_t;
            if (ch_ids) ch_ids[obase + i] = (int32_t)lc;
            if (t_steps) t_steps[obase + i] = tv[q];
            k_flat[obase + i] = tp < 0 ? tv[q] + 1 : tv[q] - tp;
            if (head_flags) head_flags[obase + i] = tp < 0 ? 1 : 0;
          }
        }
        if (GATHER) {
#pragma unroll
          for (int q = 0; q < FB; ++q) {
            const int i = i0 + q * kWave + lane;
            if (i < seg_cnt) x_ev[obase + i] = xv[q];
          }
        }
      }
    }
    wave_sync();
    prev_t = max(prev_t, seg_last);
    off += seg_cnt;
  }
}

// ----------------------------------------------------------------- expand
__global__ __launch_bounds__(256) void k_expand_cu(const int32_t* __restrict__ base_cu, int64_t n_rows, int expand,
                                                   int32_t* __restrict__ cu) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c > n_rows) return;
  if (c < n_rows) {
    const int32_t s = base_cu[c];
    const int32_t cnt = base_cu[c + 1] - s;
    for (int r = 0; r < expand; ++r) cu[c * expand + r] = s * expand + r * cnt;
  } else {
    cu[n_rows * expand] = base_cu[n_rows] * expand;
  }
}

__global__ __launch_bounds__(256) void k_expand_events(const int32_t* __restrict__ bch, const int32_t* __restrict__ bt,
                                                       const int32_t* __restrict__ bk,
                                                       const int32_t* __restrict__ base_cu, int64_t n_rows,
                                                       int64_t E_base, int expand, int32_t* __restrict__ ch,
                                                       int32_t* __restrict__ t, int32_t* __restrict__ k) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E_base) return;
  const int32_t c = bch[i];
  if (c < 0 || c >= n_rows) return;
  const int32_t s = base_cu[c];
  const int32_t cnt = base_cu[c + 1] - s;
  const int64_t off = i - s;
  if (off < 0 || off >= cnt) return;
  const int32_t tv = bt[i], kv = bk[i];
  for (int r = 0; r < expand; ++r) {
    const int64_t pos = (int64_t)s * expand + (int64_t)r * cnt + off;
    ch[pos] = c * expand + r;
    t[pos] = tv;
    k[pos] = kv;
  }
}

__global__ __launch_bounds__(1024) void k_seqlen_max(const int32_t* __restrict__ cu, int64_t n,
                                                     int32_t* __restrict__ out) {
  __shared__ int s_m[16];
  int m = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = max(m, cu[i + 1] - cu[i]);
  m = wave_max(m);
  if (lane_id() == 0) s_m[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    int r = 0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) r = max(r, s_m[w]);
    out[0] = r;
  }
}

// ----------------------------------------------------------------- gather
template <typename T>
__global__ __launch_bounds__(256) void k_gather_fwd(const T* __restrict__ x, int64_t n_rows, int64_t L,
                                                    const int32_t* __restrict__ ch, const int32_t* __restrict__ t,
                                                    int64_t E, T* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int32_t c = ch[e], s = t[e];
  const bool ok = c >= 0 && c < n_rows && s >= 0 && s < L;
  out[e] = ok ? x[(int64_t)c * L + s] : from_f<T>(0.0f);
}

template <typename T>
__global__ __launch_bounds__(256) void k_scatter(const T* __restrict__ g, const int32_t* __restrict__ ch,
                                                 const int32_t* __restrict__ t, int64_t E, int64_t n_rows, int64_t L,
                                                 T* __restrict__ dx) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int32_t c = ch[e], s = t[e];
  if (c >= 0 && c < n_rows && s >= 0 && s < L) dx[(int64_t)c * L + s] = g[e];
}

// Row-wise gather backward for time-sorted events: dx[row, t] = g[e] at the
// row's events, 0 elsewhere. One wave per row, in windows of kGatherWin
// steps: the window's event values (contiguous in g) are staged in LDS with
// coalesced loads, then each lane writes 4 consecutive steps per 256-step
// segment (one 16-byte store per lane, whole 1 KB rows per instruction),
// taking its events' positions from the tile masks and the tile table.
constexpr int kGatherWin = 2048;  // steps per window (32 tiles)

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_gather_bwd_rows(const T* __restrict__ g, const uint32_t* __restrict__ bitmask,
                                                         int64_t W, int64_t mrd,
                                                         const int32_t* __restrict__ tile_start, int64_t nT,
                                                         int64_t n_rows, int64_t L, T* __restrict__ dx) {
  __shared__ float s_g[4][kGatherWin];
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= n_rows) return;
  const int32_t* ts = tile_start + row * (nT + 1);
  const uint32_t* br = bitmask + (row / mrd) * W;
  float* sg = s_g[wave];
  T* dr = dx + row * L;
  constexpr int SEGS = kGatherWin / 256;
  for (int64_t w0 = 0; w0 < L; w0 += kGatherWin) {
    const int64_t j0 = w0 / kTile;
    const int64_t j1 = j0 + kGatherWin / kTile < nT ? j0 + kGatherWin / kTile : nT;
    const int32_t e0 = ts[j0];
    const int n = ts[j1] - e0;  // events in the window, <= kGatherWin
    const __amdgpu_buffer_rsrc_t rg = buf_rsrc(g + e0, (int64_t)n * (int64_t)sizeof(T));
    // tile table entries and masks of the lane's segments, and the window's
    // values, all in flight together
    int32_t te[SEGS];
    uint64_t tm[SEGS];
#pragma unroll
    for (int k = 0; k < SEGS; ++k) {
      const int64_t t = w0 + 256 * k + 4 * lane;
      const int64_t j = (t < L ? t : L - 1) / kTile;
      te[k] = ts[j];
      tm[k] = tile_mask(br, j);
    }
    for (int q = 0; q * kWave < n; ++q) {
      const int i = q * kWave + lane;
      const float v = buf_load<T>(rg, (uint32_t)i * (uint32_t)sizeof(T));
      if (i < n && i < kGatherWin) sg[i] = v;
    }
    wave_sync();
#pragma unroll
    for (int k = 0; k < SEGS; ++k) {
      const int64_t t0 = w0 + 256 * k + 4 * lane;
      if (t0 >= L) break;
      const int off = (int)(t0 % kTile);
      const uint64_t m = tm[k];
      int e = te[k] - e0 + __popcll(m & ((1ull << off) - 1ull));
      const uint32_t nib = (uint32_t)(m >> off) & 0xFu;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool bit = (nib >> i) & 1u;
        const float x = sg[bit ? e : 0];
        v[i] = bit ? x : 0.0f;
        e += bit ? 1 : 0;
      }
      if (VEC && t0 + 4 <= L) {
        T o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = from_f<T>(v[i]);
        if constexpr (sizeof(T) == 4) st_stream(*reinterpret_cast<u32x4*>(o), reinterpret_cast<u32x4*>(dr + t0));
        else st_stream(*reinterpret_cast<u32x2*>(o), reinterpret_cast<u32x2*>(dr + t0));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t0 + i < L) dr[t0 + i] = from_f<T>(v[i]);
      }
    }
    wave_sync();  // the staging area is refilled by the next window
  }
}

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Above this many 4-row blocks the fill reads its row offsets from a scan of
// the block sums instead of summing them per block (block i reads i values:
// ~2 M L2 reads at 2048 blocks, ~8 M at 4096, quadratic beyond).
constexpr int64_t kFillSelfScanBlocks = 4096;

// The prefix of the block sums (bpre = block_sums + 2 * nblk) and meta, when
// the fill does not derive them itself; returns bpre or NULL.
static const int32_t* block_prefix(const int32_t* block_sums, int64_t nblk, int32_t* meta, hipStream_t s) {
  if (nblk <= kFillSelfScanBlocks) return nullptr;
  int32_t* bpre = const_cast<int32_t*>(block_sums) + 2 * nblk;
  hipLaunchKernelGGL(k_scan_counts<false>, dim3(1), dim3(1024), 0, s, block_sums, nblk, bpre, meta,
                     block_sums + nblk);
  return bpre;
}

static unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace bcm

using namespace bcm;

extern "C" {

int bcm_extract_count(const void* membrane, int dtype, int64_t n_rows, int64_t L, float threshold,
                      uint32_t* bitmask, int32_t* counts, bcm_stream_t stream) {
  const char* fn = "bcm_extract_count";
  if (!dtype_ok(dtype) && dtype != BCM_U8) return set_error(BCM_EINVAL, "%s: membrane must be fp32, fp16, bf16 or u8", fn);
  if (n_rows < 0 || L < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  if (n_rows == 0) return BCM_OK;
  if (L == 0) return zero_bytes(counts, n_rows * 4, hs(stream), fn);
  if (!membrane || !bitmask || !counts) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_rows * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_rows * L must fit in int32", fn);
  const int64_t W = bitmask_words(L);
  const bool vec = aligned(membrane, 16) && ((L * (int64_t)dtype_size(dtype)) % 16 == 0);
  const dim3 grid(blocks_for(n_rows, 4)), block(256);
  auto go = [&](auto tag) {
    using T = decltype(tag);
    const T* x = static_cast<const T*>(membrane);
    if (vec)
      hipLaunchKernelGGL((k_count<T, true, false>), grid, block, 0, hs(stream), x, n_rows, L, threshold, bitmask, W,
                         counts, nullptr, nullptr);
    else
      hipLaunchKernelGGL((k_count<T, false, false>), grid, block, 0, hs(stream), x, n_rows, L, threshold, bitmask, W,
                         counts, nullptr, nullptr);
  };
  if (dtype == BCM_U8) go(uint8_t{});
  else dispatch_dtype(dtype, go);
  return check_launch(fn);
}

int bcm_extract_scan(const int32_t* counts, int64_t n_rows, int32_t* cu_seqlens, int32_t* meta,
                     bcm_stream_t stream) {
  const char* fn = "bcm_extract_scan";
  if (n_rows < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  if (!cu_seqlens || !meta || (n_rows > 0 && !counts)) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (!aligned(meta, 8)) return set_error(BCM_EINVAL, "%s: meta must be 8-byte aligned", fn);
  if (aligned(counts, 16))
    hipLaunchKernelGGL(k_scan_counts<true>, dim3(1), dim3(1024), 0, hs(stream), counts, n_rows, cu_seqlens, meta,
                       nullptr);
  else
    hipLaunchKernelGGL(k_scan_counts<false>, dim3(1), dim3(1024), 0, hs(stream), counts, n_rows, cu_seqlens, meta,
                       nullptr);
  return check_launch(fn);
}

int bcm_extract_fill(const uint32_t* bitmask, const int32_t* base_cu, int64_t n_rows, int64_t L, int64_t expand,
                     const void* x, int x_dtype, int32_t* ch_ids, int32_t* t_steps, int32_t* k_flat, void* x_events,
                     int32_t* tile_start, int32_t* head_flags, bcm_stream_t stream) {
  const char* fn = "bcm_extract_fill";
  if (n_rows < 0 || L < 0 || expand < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (n_rows == 0 || L == 0) return BCM_OK;
  if (!bitmask || !base_cu) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if ((x == nullptr) != (x_events == nullptr))
    return set_error(BCM_EINVAL, "%s: x and x_events must both be given or both be NULL", fn);
  if (x && !dtype_ok(x_dtype)) return set_error(BCM_EINVAL, "%s: x must be fp32, fp16 or bf16", fn);
  if (n_rows * expand * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: rows * expand * L must fit in int32", fn);
  if (tile_start && !aligned(bitmask, 8)) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L);
  const dim3 grid(blocks_for(n_rows, 4)), block(256);
  const int ex = (int)expand;
  auto launch = [&](auto tag, auto gather, auto tiles) {
    using T = decltype(tag);
    constexpr bool G = decltype(gather)::value;
    constexpr bool TT = decltype(tiles)::value;
    hipLaunchKernelGGL((k_fill<T, G, TT, false>), grid, block, 0, hs(stream), bitmask, W, base_cu, n_rows, L, ex,
                       static_cast<const T*>(x), ch_ids, t_steps, k_flat, static_cast<T*>(x_events), tile_start, nT,
                       head_flags, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, ConvAt{});
  };
  using Y = std::true_type;
  using N = std::false_type;
  if (!k_flat) return set_error(BCM_EINVAL, "%s: null output pointer", fn);
  if (x) {
    dispatch_dtype(x_dtype, [&](auto tag) {
      if (tile_start) launch(tag, Y{}, Y{});
      else launch(tag, Y{}, N{});
    });
  } else {
    if (tile_start) launch(float{}, N{}, Y{});
    else launch(float{}, N{}, N{});
  }
  return check_launch(fn);
}

// block_sums layout: [nblk] sums, [nblk] maxima, [nblk + 1] exclusive
// prefix of the sums (written only when the fill scans them first).
int64_t bcm_extract_block_sums_bytes(int64_t n_rows) { return n_rows < 0 ? 0 : 4 * (3 * ((n_rows + 3) / 4) + 1); }

int bcm_extract_count_blocks(const void* membrane, int dtype, int64_t n_rows, int64_t L, float threshold,
                             uint32_t* bitmask, int32_t* counts, int32_t* block_sums, bcm_stream_t stream) {
  const char* fn = "bcm_extract_count_blocks";
  if (!dtype_ok(dtype) && dtype != BCM_U8) return set_error(BCM_EINVAL, "%s: membrane must be fp32, fp16, bf16 or u8", fn);
  if (n_rows < 1 || L < 1) return set_error(BCM_EINVAL, "%s: n_rows and L must be positive", fn);
  if (!membrane || !bitmask || !counts || !block_sums) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_rows * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_rows * L must fit in int32", fn);
  const int64_t W = bitmask_words(L), nblk = (n_rows + 3) / 4;
  const bool vec = aligned(membrane, 16) && ((L * (int64_t)dtype_size(dtype)) % 16 == 0);
  const dim3 grid((unsigned)nblk), block(256);
  auto go = [&](auto tag) {
    using T = decltype(tag);
    const T* x = static_cast<const T*>(membrane);
    if (vec)
      hipLaunchKernelGGL((k_count<T, true, true>), grid, block, 0, hs(stream), x, n_rows, L, threshold, bitmask, W,
                         counts, block_sums, block_sums + nblk);
    else
      hipLaunchKernelGGL((k_count<T, false, true>), grid, block, 0, hs(stream), x, n_rows, L, threshold, bitmask, W,
                         counts, block_sums, block_sums + nblk);
  };
  if (dtype == BCM_U8) go(uint8_t{});
  else dispatch_dtype(dtype, go);
  return check_launch(fn);
}

int bcm_extract_fill_blocks(const uint32_t* bitmask, const int32_t* counts, const int32_t* block_sums,
                            int32_t* meta, int64_t n_rows, int64_t L, int64_t expand, const void* x, int x_dtype,
                            int32_t* cu_seqlens, int32_t* ch_ids, int32_t* t_steps, int32_t* k_flat,
                            void* x_events, int32_t* tile_start, bcm_stream_t stream) {
  const char* fn = "bcm_extract_fill_blocks";
  if (n_rows < 1 || L < 1 || expand < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (!bitmask || !counts || !block_sums || !meta || !cu_seqlens || !k_flat)
    return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (!aligned(meta, 8)) return set_error(BCM_EINVAL, "%s: meta must be 8-byte aligned", fn);
  if ((x == nullptr) != (x_events == nullptr))
    return set_error(BCM_EINVAL, "%s: x and x_events must both be given or both be NULL", fn);
  if (x && !dtype_ok(x_dtype)) return set_error(BCM_EINVAL, "%s: x must be fp32, fp16 or bf16", fn);
  if (n_rows * expand * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: rows * expand * L must fit in int32", fn);
  if (tile_start && !aligned(bitmask, 8)) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L), nblk = (n_rows + 3) / 4;
  const dim3 grid((unsigned)nblk), block(256);
  const int ex = (int)expand;
  const int32_t* bpre = block_prefix(block_sums, nblk, meta, hs(stream));
  auto launch = [&](auto tag, auto gather, auto tiles) {
    using T = decltype(tag);
    constexpr bool G = decltype(gather)::value;
    constexpr bool TT = decltype(tiles)::value;
    hipLaunchKernelGGL((k_fill<T, G, TT, true>), grid, block, 0, hs(stream), bitmask, W, nullptr, n_rows, L, ex,
                       static_cast<const T*>(x), ch_ids, t_steps, k_flat, static_cast<T*>(x_events), tile_start, nT,
                       nullptr, counts, block_sums, block_sums + nblk, bpre, meta, cu_seqlens, ConvAt{});
  };
  using Y = std::true_type;
  using N = std::false_type;
  if (x) {
    dispatch_dtype(x_dtype, [&](auto tag) {
      if (tile_start) launch(tag, Y{}, Y{});
      else launch(tag, Y{}, N{});
    });
  } else {
    if (tile_start) launch(float{}, N{}, Y{});
    else launch(float{}, N{}, N{});
  }
  return check_launch(fn);
}

int bcm_extract_fill_blocks_conv(const uint32_t* bitmask, const int32_t* counts, const int32_t* block_sums,
                                 int32_t* meta, int64_t n_rows, int64_t L, int64_t expand, const void* x, int x_dtype,
                                 int64_t x_batch_stride, int64_t x_dim_stride, int64_t dim, const float* weight,
                                 const float* bias, int K, int silu, int32_t* cu_seqlens, int32_t* ch_ids,
                                 int32_t* t_steps, int32_t* k_flat, void* x_events, int32_t* tile_start,
                                 bcm_stream_t stream) {
  const char* fn = "bcm_extract_fill_blocks_conv";
  if (n_rows < 1 || L < 1 || expand < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (!bitmask || !counts || !block_sums || !meta || !cu_seqlens || !k_flat || !x || !x_events || !weight)
    return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (!aligned(meta, 8)) return set_error(BCM_EINVAL, "%s: meta must be 8-byte aligned", fn);
  if (!dtype_ok(x_dtype)) return set_error(BCM_EINVAL, "%s: x must be fp32, fp16 or bf16", fn);
  if (K < 1 || K > 8) return set_error(BCM_EINVAL, "%s: kernel width must be in [1, 8]", fn);
  if (dim < 1 || (n_rows * expand) % dim != 0 || dim > INT32_MAX)
    return set_error(BCM_EINVAL, "%s: n_rows * expand must be a multiple of dim", fn);
  if (x_batch_stride < 0 || x_dim_stride < 0) return set_error(BCM_EINVAL, "%s: negative stride", fn);
  if (n_rows * expand * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: rows * expand * L must fit in int32", fn);
  if (tile_start && !aligned(bitmask, 8)) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L), nblk = (n_rows + 3) / 4;
  const dim3 grid((unsigned)nblk), block(256);
  const int ex = (int)expand;
  const ConvAt cv{weight, bias, K, (int)dim, silu, x_batch_stride, x_dim_stride};
  const int32_t* bpre = block_prefix(block_sums, nblk, meta, hs(stream));
  dispatch_dtype(x_dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto tiles, auto km) {
      constexpr bool TT = decltype(tiles)::value;
      constexpr int KM = decltype(km)::value;
      hipLaunchKernelGGL((k_fill<T, true, TT, true, KM>), grid, block, 0, hs(stream), bitmask, W, nullptr, n_rows, L,
                         ex, static_cast<const T*>(x), ch_ids, t_steps, k_flat, static_cast<T*>(x_events), tile_start,
                         nT, nullptr, counts, block_sums, block_sums + nblk, bpre, meta, cu_seqlens, cv);
    };
    using K4 = std::integral_constant<int, 4>;
    using K8 = std::integral_constant<int, 8>;
    if (tile_start) {
      if (K == 4) go(std::true_type{}, K4{});
      else go(std::true_type{}, K8{});
    } else {
      if (K == 4) go(std::false_type{}, K4{});
      else go(std::false_type{}, K8{});
    }
  });
  return check_launch(fn);
}

int bcm_spike_bits(const void* p, int dtype, int64_t B, int64_t L, int64_t Dm, float threshold, uint32_t* bitmask,
                   void* s_out, bcm_stream_t stream) {
  const char* fn = "bcm_spike_bits";
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: p must be fp32, fp16 or bf16", fn);
  if (B < 0 || L < 0 || Dm < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  if (B == 0 || L == 0 || Dm == 0) return BCM_OK;
  if (!p || !bitmask) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (!aligned(bitmask, 8)) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  if (B * L * Dm > INT32_MAX) return set_error(BCM_EINVAL, "%s: B * L * Dm must fit in int32", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (Dm + kWave - 1) / kWave;
  const dim3 grid(blocks_for(B * nG * nT, 4)), block(256);
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL((k_spike_bits<T>), grid, block, 0, hs(stream), static_cast<const T*>(p), B, L, Dm, threshold,
                       bitmask, W, static_cast<T*>(s_out));
  });
  return check_launch(fn);
}

int bcm_extract_count_bits(const uint32_t* bitmask, int64_t n_rows, int64_t L, int32_t* counts, int32_t* block_sums,
                           bcm_stream_t stream) {
  const char* fn = "bcm_extract_count_bits";
  if (n_rows < 1 || L < 1) return set_error(BCM_EINVAL, "%s: n_rows and L must be positive", fn);
  if (!bitmask || !counts || !block_sums) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_rows * L > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_rows * L must fit in int32", fn);
  const int64_t nblk = (n_rows + 3) / 4;
  hipLaunchKernelGGL(k_count_bits, dim3((unsigned)nblk), dim3(256), 0, hs(stream), bitmask, n_rows, L,
                     bitmask_words(L), counts, block_sums, block_sums + nblk);
  return check_launch(fn);
}

int bcm_expand_events(const int32_t* base_ch, const int32_t* base_t, const int32_t* base_k, const int32_t* base_cu,
                      int64_t n_rows, int64_t E_base, int64_t expand, int32_t* ch_ids, int32_t* t_steps,
                      int32_t* k_flat, int32_t* cu_seqlens, bcm_stream_t stream) {
  const char* fn = "bcm_expand_events";
  if (n_rows < 0 || E_base < 0 || expand < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (!base_cu || !cu_seqlens) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if ((n_rows + 1) * expand > INT32_MAX || E_base * expand > INT32_MAX)
    return set_error(BCM_EINVAL, "%s: expanded sizes must fit in int32", fn);
  hipLaunchKernelGGL(k_expand_cu, dim3(blocks_for(n_rows + 1, 256)), dim3(256), 0, hs(stream), base_cu, n_rows,
                     (int)expand, cu_seqlens);
  int rc = check_launch(fn);
  if (rc || E_base == 0) return rc;
  if (!base_ch || !base_t || !base_k || !ch_ids || !t_steps || !k_flat)
    return set_error(BCM_EINVAL, "%s: null pointer", fn);
  hipLaunchKernelGGL(k_expand_events, dim3(blocks_for(E_base, 256)), dim3(256), 0, hs(stream), base_ch, base_t,
                     base_k, base_cu, n_rows, E_base, (int)expand, ch_ids, t_steps, k_flat);
  return check_launch(fn);
}

int bcm_seqlen_max(const int32_t* cu_seqlens, int64_t n, int32_t* out, bcm_stream_t stream) {
  const char* fn = "bcm_seqlen_max";
  if (n < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  if (!out || (n > 0 && !cu_seqlens)) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  hipLaunchKernelGGL(k_seqlen_max, dim3(1), dim3(1024), 0, hs(stream), cu_seqlens, n, out);
  return check_launch(fn);
}

int bcm_gather_fwd(const void* x, int dtype, int64_t n_rows, int64_t L, const int32_t* ch_ids,
                   const int32_t* t_steps, int64_t E, void* out, bcm_stream_t stream) {
  const char* fn = "bcm_gather_fwd";
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: x must be fp32, fp16 or bf16", fn);
  if (E < 0 || n_rows < 0 || L < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  if (E == 0) return BCM_OK;
  if (!x || !ch_ids || !t_steps || !out) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(k_gather_fwd<T>, dim3(blocks_for(E, 256)), dim3(256), 0, hs(stream),
                       static_cast<const T*>(x), n_rows, L, ch_ids, t_steps, E, static_cast<T*>(out));
  });
  return check_launch(fn);
}

int bcm_gather_bwd(const void* g, int dtype, const int32_t* ch_ids, const int32_t* t_steps, int64_t E,
                   int64_t n_rows, int64_t L, void* dx, bcm_stream_t stream) {
  const char* fn = "bcm_gather_bwd";
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: grad must be fp32, fp16 or bf16", fn);
  if (E < 0 || n_rows < 0 || L < 0) return set_error(BCM_EINVAL, "%s: negative size", fn);
  int rc = zero_bytes(dx, n_rows * L * (int64_t)dtype_size(dtype), hs(stream), fn);
  if (rc || E == 0) return rc;
  if (!g || !ch_ids || !t_steps) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(k_scatter<T>, dim3(blocks_for(E, 256)), dim3(256), 0, hs(stream), static_cast<const T*>(g),
                       ch_ids, t_steps, E, n_rows, L, static_cast<T*>(dx));
  });
  return check_launch(fn);
}

int bcm_gather_bwd_rows(const void* g, int dtype, const uint32_t* bitmask, int64_t mask_row_div,
                        const int32_t* tile_start, int64_t n_rows, int64_t L, void* dx, bcm_stream_t stream) {
  const char* fn = "bcm_gather_bwd_rows";
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: grad must be fp32, fp16 or bf16", fn);
  if (n_rows < 0 || L < 0 || mask_row_div < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (n_rows == 0 || L == 0) return BCM_OK;
  if (!bitmask || !tile_start || !dx) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (!aligned(bitmask, 8)) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L);
  const size_t es = dtype_size(dtype);
  const bool vec = aligned(dx, 4 * es) && ((L * (int64_t)es) % (4 * es) == 0);
  const dim3 grid(blocks_for(n_rows, 4)), block(256);
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (vec)
      hipLaunchKernelGGL((k_gather_bwd_rows<T, true>), grid, block, 0, hs(stream), static_cast<const T*>(g), bitmask,
                         W, mask_row_div, tile_start, nT, n_rows, L, static_cast<T*>(dx));
    else
      hipLaunchKernelGGL((k_gather_bwd_rows<T, false>), grid, block, 0, hs(stream), static_cast<const T*>(g),
                         bitmask, W, mask_row_div, tile_start, nT, n_rows, L, static_cast<T*>(dx));
  });
  return check_launch(fn);
}

}  // extern "C"
