// Stage 3: causal zero-order-hold restore (r_nodecay), forward and backward.
//
// Reference behaviour: csrc/r_nodecay/restore_dense_fwd_kernel.cuh:38-114
// (out[b,t,d] = y of the last event at or before t, 0 before the first),
// restore_dense_bwd_kernel.cuh:42-112 (dy[e] = sum of dout over the steps
// that event e owns), restore_dense.cpp:43-202 (shapes, dtypes, fp32 dy).
//
// MI355X design: one wave per (batch b, 64 consecutive channels d, 64-step
// tile). Lane = channel, so every step of the sweep is one coalesced
// 64-channel row of the (B, L, D) tensor. The tile's event positions come
// from the 64-bit tile mask of the event bitmask and the first event index
// from the tile table, so all value loads are independent (no search, no
// serial pointer chasing). Each kernel runs in branch-free phases (all loads,
// register work, back-to-back stores) so no store waits on another. The
// backward uses no atomics on dy: runs inside a tile are written by the tile
// pass, runs that cross a tile edge by a small fix-up pass (bcm_restore_bwd)
// or, in one kernel, by a look-back over the preceding tiles' published
// partials (bcm_restore_bwd_chained); each event exactly once
// (deterministic, no zero-fill of dy).
#include "bcm_common.hpp"

#include <mutex>

namespace bcm {

template <bool USE_LDS>
__global__ __launch_bounds__(64) void k_build_index(const int32_t* __restrict__ t_steps,
                                                    const int32_t* __restrict__ cu, int64_t L, int64_t W, int64_t nT,
                                                    uint32_t* __restrict__ bitmask, int32_t* __restrict__ tile_start,
                                                    float* __restrict__ zero_f32, int64_t n_zero) {
  extern __shared__ uint32_t s_bits[];
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  uint32_t* gb = bitmask + row * W;
  uint32_t* bits = USE_LDS ? s_bits : gb;
  for (int64_t i = lane; i < W; i += kWave) bits[i] = 0u;
  __syncthreads();
  if (zero_f32) {  // row r zeroes its share [r*n_zero/rows, (r+1)*n_zero/rows)
    const int64_t rows = gridDim.x;
    const int64_t z0 = row * n_zero / rows, z1 = (row + 1) * n_zero / rows;
    for (int64_t i = z0 + lane; i < z1; i += kWave) zero_f32[i] = 0.0f;
  }
  const int32_t s = cu[row], e = cu[row + 1];
  for (int64_t i = s + lane; i < e; i += kWave) {
    const int32_t t = t_steps[i];
    if (t >= 0 && t < L) atomicOr(&bits[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  if (USE_LDS)
    for (int64_t i = lane; i < W; i += kWave) gb[i] = s_bits[i];
  int carry = 0;
  for (int64_t j0 = 0; j0 < nT; j0 += kWave) {
    const int64_t j = j0 + lane;
    const int pc = j < nT ? __popc(bits[2 * j]) + __popc(bits[2 * j + 1]) : 0;
    const int incl = wave_incl_sum(pc);
    if (j < nT) tile_start[row * (nT + 1) + j] = s + carry + incl - pc;
    carry += __shfl(incl, kWave - 1, kWave);
  }
  if (lane == 0) tile_start[row * (nT + 1) + nT] = s + carry;
}

struct TileWave {
  int b, j, g, dd, ch;
  bool ok;        // lane maps to a channel (dd < dim)
  int e_base;     // first event index of the wave's 64 channels
};

// wave id -> (b, tile j, channel group g); g varies fastest so neighbouring
// waves write neighbouring 256-byte pieces of the same (b, t) rows, and the
// XCD remap keeps consecutive tiles of a channel (which share event-value
// lines and index rows) in one L2. Lanes
// past `dim` are clamped to the group's last channel (addresses stay valid)
// and flagged !ok.
// nPos: positions along time per (b, g); nT: tiles per row of the tile table.
// The tile kernels run 256-thread blocks, (waves + 3) / 4 of them: the wave id
// comes from these constants and the `waves` argument, not from the launch's
// implicit arguments (whose loads would come first, one round trip each).
constexpr int kTileWaves = 4;  // waves per block
__device__ __forceinline__ int tile_wave_id(int waves) {
  return xcd_block(blockIdx.x, (waves + kTileWaves - 1) / kTileWaves) * kTileWaves + (int)(threadIdx.x / kWave);
}

__device__ __forceinline__ TileWave tile_wave(int nPos, int nG, int dim, const int32_t* tile_start, int nT,
                                              int waves) {
  TileWave w;
  // wave-uniform by construction; readfirstlane lets the compiler keep it (and
  // the buffer descriptors built from it) in SGPRs
  const int wid = __builtin_amdgcn_readfirstlane(tile_wave_id(waves));
  w.g = wid % nG;
  const int bj = wid / nG;
  w.j = bj % nPos;
  w.b = bj / nPos;
  const int d = w.g * kWave + lane_id();
  w.ok = d < dim;
  w.dd = w.ok ? d : dim - 1;
  w.ch = w.b * dim + w.dd;
  w.e_base = tile_start[(int64_t)(w.b * dim + w.g * kWave) * (nT + 1)];
  return w;
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_restore_fwd(const TI* __restrict__ y, int64_t n_events,
                                                     const uint32_t* __restrict__ bitmask, int64_t W, int64_t mrd,
                                                     const int32_t* __restrict__ tile_start, int nT, int nG,
                                                     int waves, int dim, int64_t L, int64_t out_elems,
                                                     TO* __restrict__ out) {
  // the arguments of the first loads come in the first batch of argument
  // loads (one wait), not on demand one batch later
  asm volatile("" ::"s"(tile_start), "s"(bitmask), "s"(y), "s"(W), "s"(mrd), "s"(L), "s"(out_elems));
  if (tile_wave_id(waves) >= waves) return;
  const TileWave w = tile_wave(nT, nG, dim, tile_start, nT, waves);
  const int32_t* ts = tile_start + (int64_t)w.ch * (nT + 1);
  const int32_t cu0 = ts[0], elo = ts[w.j];
  const uint64_t m = w.ok ? tile_mask(bitmask + (w.ch / mrd) * W, w.j) : 0ull;
  const int e_base = __builtin_amdgcn_readfirstlane(w.e_base);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y + e_base, (n_events - e_base) * (int64_t)sizeof(TI));
  // the value held before the tile (its previous event's), then the tile's
  // event values, one load per step with out-of-range offsets for steps
  // without an event (no branches, all loads independent), in the order the
  // stores below use them, so that the first stores wait for the first
  // loads only (the empty asm on val, after the loads are issued, keeps the
  // compiler from folding the first select into a predicated reload of
  // val's register issued last; it waits for val's load alone)
  float val = buf_load<TI>(ry, elo > cu0 ? (uint32_t)(elo - 1 - e_base) * (uint32_t)sizeof(TI) : kBufOOB);
  float v[kTile];
  uint32_t idx = (uint32_t)(elo - e_base);
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    const uint32_t bit = (uint32_t)(m >> s) & 1u;
    v[s] = buf_load<TI>(ry, bit ? idx * (uint32_t)sizeof(TI) : kBufOOB);
    idx += bit;
  }
  asm volatile("" : "+v"(val));
  // One straight-line pass for every tile (v[] stays in registers): lanes
  // past dim and steps past L get an out-of-range offset, so their stores
  // are dropped by the buffer unit instead of branched around.
  const int64_t t0 = (int64_t)w.j * kTile;
  const int steps = (int)(L - t0 < kTile ? L - t0 : kTile);
  const int64_t obase = ((int64_t)w.b * L + t0) * dim + (int64_t)w.g * kWave;
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out + obase, (out_elems - obase) * (int64_t)sizeof(TO));
  const uint32_t lane_off = w.ok ? (uint32_t)lane_id() * (uint32_t)sizeof(TO) : kBufOOB;
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(TO);
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    val = ((m >> s) & 1ull) ? v[s] : val;
    buf_store<TO, kStream>(ro, s < steps ? lane_off + (uint32_t)s * row_bytes : kBufOOB, val);
  }
}

// Restore forward for 16-bit outputs with two channels per lane (dim even):
// one wave per (b, 128 consecutive channels, 64-step tile), so each store
// instruction writes a whole 256-byte run of a (b, t) row (two packed
// 16-bit values per lane), as the one-channel form does for fp32, whose
// 16-bit stores filled only half of that (config 2, bf16: restore forward
// at 2.5 TB/s). Loads as in k_restore_fwd, per channel of the lane; with
// TI == TO the values travel as raw 16-bit words.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_restore_fwd_pair(const TI* __restrict__ y, int64_t n_events,
                                                          const uint32_t* __restrict__ bitmask, int64_t W,
                                                          int64_t mrd, const int32_t* __restrict__ tile_start,
                                                          int nT, int nG, int waves, int dim, int64_t L,
                                                          int64_t out_elems, TO* __restrict__ out) {
  static_assert(sizeof(TO) == 2, "16-bit outputs");
  constexpr bool RAW = std::is_same<TI, TO>::value;
  asm volatile("" ::"s"(tile_start), "s"(bitmask), "s"(y), "s"(W), "s"(mrd), "s"(L), "s"(out_elems));
  if (tile_wave_id(waves) >= waves) return;
  const int wid = __builtin_amdgcn_readfirstlane(tile_wave_id(waves));
  const int g = wid % nG, bj = wid / nG;
  const int j = bj % nT, b = bj / nT;
  const int lane = lane_id();
  const int d = g * 2 * kWave + 2 * lane;
  const bool ok = d < dim;  // dim is even: both channels of the lane exist or neither
  const int64_t ch = (int64_t)b * dim + (ok ? d : dim - 2);
  const int32_t* ts0 = tile_start + ch * (nT + 1);
  const int32_t* ts1 = ts0 + (nT + 1);
  const int32_t c0 = ts0[0], lo0 = ts0[j], c1 = ts1[0], lo1 = ts1[j];
  const uint64_t m0 = ok ? tile_mask(bitmask + (ch / mrd) * W, j) : 0ull;
  const uint64_t m1 = ok ? tile_mask(bitmask + ((ch + 1) / mrd) * W, j) : 0ull;
  const int e_base = __builtin_amdgcn_readfirstlane(tile_start[((int64_t)b * dim + g * 2 * kWave) * (nT + 1)]);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y + e_base, (n_events - e_base) * (int64_t)sizeof(TI));
  auto ld = [&](uint32_t off) -> uint32_t {  // raw 16-bit word, or the fp32 value's bits
    if constexpr (RAW) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ry, off, 0, 0);
    else return __float_as_uint(buf_load<TI>(ry, off));
  };
  // the values held before the tile, then the tile's event values, in the
  // order the stores use them (out-of-range offsets where a step has none)
  uint32_t val0 = ld(ok && lo0 > c0 ? (uint32_t)(lo0 - 1 - e_base) * (uint32_t)sizeof(TI) : kBufOOB);
  uint32_t val1 = ld(ok && lo1 > c1 ? (uint32_t)(lo1 - 1 - e_base) * (uint32_t)sizeof(TI) : kBufOOB);
  uint32_t v0[kTile], v1[kTile];
  uint32_t i0 = (uint32_t)(lo0 - e_base), i1 = (uint32_t)(lo1 - e_base);
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    const uint32_t b0 = (uint32_t)(m0 >> s) & 1u, b1 = (uint32_t)(m1 >> s) & 1u;
    v0[s] = ld(b0 ? i0 * (uint32_t)sizeof(TI) : kBufOOB);
    v1[s] = ld(b1 ? i1 * (uint32_t)sizeof(TI) : kBufOOB);
    i0 += b0;
    i1 += b1;
  }
  asm volatile("" : "+v"(val0), "+v"(val1));
  const int64_t t0 = (int64_t)j * kTile;
  const int steps = (int)(L - t0 < kTile ? L - t0 : kTile);
  const int64_t obase = ((int64_t)b * L + t0) * dim + (int64_t)g * 2 * kWave;
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out + obase, (out_elems - obase) * 2);
  const uint32_t lane_off = ok ? (uint32_t)lane * 4u : kBufOOB;
  const uint32_t row_bytes = (uint32_t)dim * 2u;
  auto bits16 = [&](uint32_t v) -> uint32_t {
    if constexpr (RAW) return v;
    else {
      const TO h = from_f<TO>(__uint_as_float(v));
      unsigned short u;
      __builtin_memcpy(&u, &h, 2);
      return u;
    }
  };
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    val0 = ((m0 >> s) & 1ull) ? v0[s] : val0;
    val1 = ((m1 >> s) & 1ull) ? v1[s] : val1;
    __builtin_amdgcn_raw_buffer_store_b32(bits16(val0) | (bits16(val1) << 16), ro,
                                          s < steps ? lane_off + (uint32_t)s * row_bytes : kBufOOB, 0, kStream);
  }
}

// Restore backward, tile pass. Runs that start and end inside the tile are
// final; the partial runs at the tile edges (head: before the first event;
// tail: from the last event to the tile end) go to per-tile side arrays
// [nT][n_rows] for the fix-up pass, with the tile's end event index (-1 for
// a tile without events). At each event a lane stages the run that
// the event closes in LDS (value and destination, one 8-byte write at the
// lane's next slot; slots from a wave prefix sum of the per-lane event
// counts). A lane's first slot holds its head, which is read back and whose
// destination is then marked out of range. The staged runs are written out
// with consecutive lanes on consecutive slots: a channel's runs are
// consecutive dy entries, so each store instruction covers a few contiguous
// pieces instead of up to 64 scattered words. Waves with more events than
// the staging area store the runs directly.
constexpr int kBwdStage = 1024;    // staged runs per wave (about 680 at 15% density)
constexpr uint32_t kNoDst = kBufOOB / 4;  // destination whose byte offset is out of range

template <typename TI>
__global__ __launch_bounds__(256, 4) void k_restore_bwd_tiles(const TI* __restrict__ dout, int64_t n_events,
                                                              const uint32_t* __restrict__ bitmask, int64_t W,
                                                              int64_t mrd, const int32_t* __restrict__ tile_start,
                                                              int nT, int nG, int waves, int dim, int64_t L,
                                                              int64_t n_rows, float* __restrict__ dy,
                                                              float* __restrict__ head, float* __restrict__ tail,
                                                              int32_t* __restrict__ tend) {
  __shared__ uint2 s_run[4][kBwdStage];  // (value bits, destination)
  // the arguments of the first loads come in the first batch of argument
  // loads (one wait), not on demand one batch later
  asm volatile("" ::"s"(tile_start), "s"(bitmask), "s"(dout), "s"(W), "s"(mrd), "s"(L), "s"(n_rows));
  if (tile_wave_id(waves) >= waves) return;
  const TileWave w = tile_wave(nT, nG, dim, tile_start, nT, waves);
  const int wave = threadIdx.x / kWave, lane = lane_id();
  // dout rows of the tile; steps past L and lanes past dim read 0
  const int64_t t0 = (int64_t)w.j * kTile;
  const int steps = (int)(L - t0 < kTile ? L - t0 : kTile);
  const int64_t gbase = ((int64_t)w.b * L + t0) * dim + (int64_t)w.g * kWave;
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(dout + gbase, (n_rows * L - gbase) * (int64_t)sizeof(TI));
  const uint32_t lane_off = w.ok ? (uint32_t)lane * (uint32_t)sizeof(TI) : kBufOOB;
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(TI);
  // the tile's first event index and mask before its rows, so that the
  // sweep below starts when the first rows are in (in-order load counts)
  const int32_t elo = tile_start[(int64_t)w.ch * (nT + 1) + w.j];
  const uint64_t m = w.ok ? tile_mask(bitmask + (w.ch / mrd) * W, w.j) : 0ull;
  float gv[kTile];
#pragma unroll
  for (int s = 0; s < kTile; ++s) gv[s] = buf_load<TI, kStream>(rg, s < steps ? lane_off + (uint32_t)s * row_bytes : kBufOOB);
  const int e_base = __builtin_amdgcn_readfirstlane(w.e_base);
  const __amdgpu_buffer_rsrc_t rdy = buf_rsrc(dy + e_base, (n_events - e_base) * 4);
  const int nev = __popcll(m);
  const int incl = wave_incl_sum_dpp(nev);
  const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
  // sum: the open run; hsum: the steps before the tile's first event (the
  // whole tile when it has none)
  float sum = 0.0f, hsum;
  if (total <= kBwdStage) {  // wave-uniform
    uint2* sr = s_run[wave];
    const int pre = incl - nev;
    uint32_t slot = (uint32_t)pre;
    uint32_t dst = (uint32_t)(elo - e_base) - 1u;  // event whose run the next event closes
#pragma unroll
    for (int s = 0; s < kTile; ++s) {
      const bool bit = (m >> s) & 1ull;
      if (bit) {
        sr[slot] = make_uint2(__float_as_uint(sum), dst);
        ++slot;
        ++dst;
      }
      sum = (bit ? 0.0f : sum) + gv[s];
    }
    hsum = sum;
    if (nev) {  // the first slot is the head: read it back, drop its store
      hsum = __uint_as_float(sr[pre].x);
      sr[pre].y = kNoDst;
    }
    wave_sync();
    for (int k = 0; k < total; k += kWave) {
      const int i = k + lane;
      const uint2 v = sr[i < total ? i : 0];
      buf_store_f32(rdy, i < total ? v.y * 4u : kBufOOB, __uint_as_float(v.x));
    }
  } else {
    uint32_t r = 0;  // events seen so far in the tile
    const uint32_t ebase = (uint32_t)(elo - e_base);
    const int first = m ? __builtin_ctzll(m) : kTile;  // step of the tile's first event
    hsum = 0.0f;
#pragma unroll
    for (int s = 0; s < kTile; ++s) {
      const uint32_t bit = (uint32_t)(m >> s) & 1u;
      // the run of event (elo + r - 1) closes here when r >= 1
      buf_store_f32(rdy, (bit && r) ? (ebase + r - 1) * 4u : kBufOOB, sum);
      r += bit;
      sum = (bit ? 0.0f : sum) + gv[s];
      hsum += s < first ? gv[s] : 0.0f;
    }
  }
  if (w.ok) {
    const int64_t o = (int64_t)w.j * n_rows + w.ch;
    head[o] = hsum;
    tail[o] = sum;
    tend[o] = nev ? elo + nev : -1;
  }
}

// Restore backward, fix-up pass: the run of the last event of tile j is its
// tail partial plus the head partials of the following tiles up to and
// including the next tile that holds an event. One lane per (tile, channel);
// every read is coalesced ([nT][n_rows] side arrays), only the dy store is
// scattered.
__global__ __launch_bounds__(256) void k_restore_bwd_fix(int64_t nT, int64_t n_rows, const float* __restrict__ head,
                                                         const float* __restrict__ tail,
                                                         const int32_t* __restrict__ tend, float* __restrict__ dy,
                                                         int64_t n_events) {
  // the arguments come in one batch of argument loads
  asm volatile("" ::"s"(nT), "s"(n_rows), "s"(head), "s"(tail), "s"(tend), "s"(dy), "s"(n_events));
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256-thread blocks
  const int64_t n = nT * n_rows;
  if (i >= n) return;
  // the tile's entries and the next tile's (where the run usually ends) in
  // one round trip
  const int64_t q1 = i + n_rows;
  const int64_t q1c = q1 < n ? q1 : i;
  const int32_t e_end = tend[i], e1 = tend[q1c];
  const float tl = tail[i], h1 = head[q1c];
  asm volatile("" ::"v"(tl), "v"(h1), "v"(e1));  // all four loads before the branch below: one wait
  // no event in the tile (its head belongs to an earlier tile's owner); an
  // index outside dy (a workspace the tile pass did not fill) is never stored
  if (e_end <= 0 || e_end > n_events) return;
  float acc = tl;
  if (q1 < n) {
    acc += h1;
    if (e1 < 0) {
      for (int64_t q = q1 + n_rows; q < n; q += n_rows) {
        acc += head[q];
        if (tend[q] >= 0) break;
      }
    }
  }
  dy[e_end - 1] = acc;
}

// Restore backward in one pass: the tile pass above, with the runs that
// cross tile edges closed by decoupled look-back instead of a fix-up pass.
//
// Sync area (64-bit words, zero before the first call, zero again after
// every call): word 0 reserved, word 1 a status word (nonzero: a look-back
// wait gave up), then one slot per (tile j, channel) at 2 + j * n_rows + ch.
//  * Waves take wave ids in the tile kernels' order (channel group fastest,
//    then tile, then batch), so tile j - 1 of a channel has a smaller id than
//    tile j. The host launches the ids in ranges of at most 4 blocks per CU,
//    which fit the device at once (launch bounds of 4 blocks, 32 KB of LDS
//    each): a wave waits only on smaller ids, of its own launch (resident
//    with it, whatever order the hardware dispatches workgroups in) or of an
//    earlier one (complete), so every wait ends.
//  * A tile publishes, per channel, the partial it hands on: the run open
//    at its end (status 2, the tile holds an event) or its whole sum
//    (status 1, no event), as one 64-bit word (status << 32 | value). It
//    publishes where an event lies at or before the tile and the tile is
//    not the last, i.e. where some later tile will read the slot.
//  * A tile whose first event has an earlier event in the channel closes
//    that event's run: its head (the steps before its first event) plus the
//    slots of the tiles before it, walked back to the nearest one with
//    status 2. The last tile closes the channel's last run the same way
//    when it holds no event (its whole sum plus the walk), else from its
//    own open run. A tile clears each slot it reads. Every published slot
//    is read by exactly one tile (the channel's next tile with an event,
//    else its last tile), so after the launch every slot is zero again.
//  * A run closed at a tile's first event goes to dy[first event - 1],
//    beside the tile's other runs in the same staged stores; only the
//    channel's last run is a separate store.
constexpr uint32_t kChainSpin = 1u << 20;  // polls before a wait gives up (about a second; never reached
                                           // when every wave of a launch can be resident)
constexpr int64_t kSyncHead = 2;           // sync words before the slots
constexpr int kChainBlocksPerCu = 4;       // the kernel's launch bounds: 4 blocks of 256 fit a CU
constexpr int kChainBatch = 4;             // slots a look-back round reads after its first

// TO: dy's type (fp32, or u's 16-bit type: the cast the reference's
// autograd applies before the scan backward, rounded the same way).
template <typename TI, typename TO>
__global__ __launch_bounds__(256, kChainBlocksPerCu) void k_restore_bwd_chain(
    const TI* __restrict__ dout, int64_t n_events, const uint32_t* __restrict__ bitmask, int64_t W, int64_t mrd,
    const int32_t* __restrict__ tile_start, int nT, int nG, int waves, int wid0, int nblk, int dim, int64_t L,
    int64_t n_rows, TO* __restrict__ dy, uint64_t* __restrict__ sync) {
  constexpr uint32_t SO = sizeof(TO);
  __shared__ uint2 s_run[4][kBwdStage];  // (value bits, destination)
  asm volatile("" ::"s"(tile_start), "s"(bitmask), "s"(dout), "s"(W), "s"(mrd), "s"(L), "s"(n_rows), "s"(sync));
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int wid = __builtin_amdgcn_readfirstlane(wid0 + xcd_block(blockIdx.x, nblk) * kTileWaves + wave);
  if (wid >= waves) return;
  TileWave w;
  w.g = wid % nG;
  w.j = (wid / nG) % nT;
  w.b = wid / nG / nT;
  {
    const int d = w.g * kWave + lane;
    w.ok = d < dim;
    w.dd = w.ok ? d : dim - 1;
    w.ch = w.b * dim + w.dd;
  }
  const int32_t* ts = tile_start + (int64_t)w.ch * (nT + 1);
  const int e_base = __builtin_amdgcn_readfirstlane(tile_start[(int64_t)(w.b * dim + w.g * kWave) * (nT + 1)]);
  const int64_t t0 = (int64_t)w.j * kTile;
  const int steps = (int)(L - t0 < kTile ? L - t0 : kTile);
  const int64_t gbase = ((int64_t)w.b * L + t0) * dim + (int64_t)w.g * kWave;
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(dout + gbase, (n_rows * L - gbase) * (int64_t)sizeof(TI));
  const uint32_t lane_off = w.ok ? (uint32_t)lane * (uint32_t)sizeof(TI) : kBufOOB;
  const uint32_t row_bytes = (uint32_t)dim * (uint32_t)sizeof(TI);
  const int32_t elo = ts[w.j], ts0 = ts[0], tsN = ts[nT];
  const uint64_t m = w.ok ? tile_mask(bitmask + (w.ch / mrd) * W, w.j) : 0ull;
  float gv[kTile];
#pragma unroll
  for (int s = 0; s < kTile; ++s) gv[s] = buf_load<TI, kStream>(rg, s < steps ? lane_off + (uint32_t)s * row_bytes : kBufOOB);
  const __amdgpu_buffer_rsrc_t rdy = buf_rsrc(dy + e_base, (n_events - e_base) * (int64_t)SO);
  const int nev = __popcll(m);
  const int incl = wave_incl_sum_dpp(nev);
  const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
  const bool staged = total <= kBwdStage;  // wave-uniform
  uint2* sr = s_run[wave];
  const int pre = incl - nev;
  float sum = 0.0f, hsum = 0.0f;
  if (staged) {
    uint32_t slot = (uint32_t)pre;
    uint32_t dst = (uint32_t)(elo - e_base) - 1u;  // event whose run the next event closes
#pragma unroll
    for (int s = 0; s < kTile; ++s) {
      const bool bit = (m >> s) & 1ull;
      if (bit) {
        sr[slot] = make_uint2(__float_as_uint(sum), dst);
        ++slot;
        ++dst;
      }
      sum = (bit ? 0.0f : sum) + gv[s];
    }
    hsum = nev ? __uint_as_float(sr[pre].x) : sum;
  } else {
    uint32_t r = 0;  // events seen so far in the tile
    const uint32_t ebase = (uint32_t)(elo - e_base);
    const int first = m ? __builtin_ctzll(m) : kTile;  // step of the tile's first event
#pragma unroll
    for (int s = 0; s < kTile; ++s) {
      const uint32_t bit = (uint32_t)(m >> s) & 1u;
      // the run of event (elo + r - 1) closes here when r >= 1
      buf_store<TO>(rdy, (bit && r) ? (ebase + r - 1) * SO : kBufOOB, sum);
      r += bit;
      sum = (bit ? 0.0f : sum) + gv[s];
      hsum += s < first ? gv[s] : 0.0f;
    }
  }
  // publish the partial this tile hands on, then close the run that ends
  // at the tile's first event (or, in the last tile, the channel's last run)
  uint64_t* slots = sync + kSyncHead;
  const int32_t enext = elo + nev;  // first event at or after tile j + 1
  if (w.ok && w.j < nT - 1 && enext > ts0)
    __hip_atomic_store(&slots[(int64_t)w.j * n_rows + w.ch],
                       ((uint64_t)(nev ? 2u : 1u) << 32) | (uint64_t)__float_as_uint(sum), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const bool last = w.ok && w.j == nT - 1 && tsN > ts0;  // the channel's last run ends in this tile
  const bool head = w.ok && nev > 0 && elo > ts0;        // the run open at the tile's start ends here
  const bool need = head || (last && nev == 0);
  float carry = nev ? hsum : sum;
  bool open = need;
  int jj = w.j - 1;
  // the walk reads one slot a round trip, four once it has met a tile
  // without events (long silences: fewer serial round trips)
  int nq = 1;
  bool wide = false;
  for (uint32_t it = 0; __builtin_amdgcn_ballot_w64(open); ++it) {
    bool idle = false;
    if (open) {
      if (jj < 0 || it >= kChainSpin) {  // cannot happen with consistent inputs; recorded, never hangs
        __hip_atomic_store(reinterpret_cast<uint32_t*>(sync + 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        open = false;
      } else {
        uint64_t v[kChainBatch];
#pragma unroll
        for (int q = 0; q < kChainBatch; ++q)
          v[q] = (q < nq && jj - q >= 0)
                     ? __hip_atomic_load(&slots[(int64_t)(jj - q) * n_rows + w.ch], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT)
                     : 0ull;
        // take the slots in order up to the first unpublished one or the
        // first with status 2
#pragma unroll
        for (int q = 0; q < kChainBatch; ++q) {
          if (open && !idle && q < nq) {
            if (v[q]) {
              __hip_atomic_store(&slots[(int64_t)jj * n_rows + w.ch], (uint64_t)0, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
              carry += __uint_as_float((uint32_t)v[q]);
              if ((uint32_t)(v[q] >> 32) == 2u) {
                open = false;
              } else {
                --jj;
                wide = true;
              }
            } else {
              idle = jj >= 0;  // not yet published (jj < 0 is caught above on the next round)
            }
          }
        }
        nq = wide ? kChainBatch : 1;
      }
    }
    if (__builtin_amdgcn_ballot_w64(idle)) __builtin_amdgcn_s_sleep(1);
  }
  if (staged) {
    if (nev) sr[pre] = make_uint2(__float_as_uint(carry), head ? (uint32_t)(elo - e_base) - 1u : kNoDst);
    wave_sync();
    for (int k = 0; k < total; k += kWave) {
      const int i = k + lane;
      const uint2 v = sr[i < total ? i : 0];
      buf_store<TO>(rdy, i < total ? v.y * SO : kBufOOB, __uint_as_float(v.x));
    }
  } else {
    buf_store<TO>(rdy, head ? ((uint32_t)(elo - e_base) - 1u) * SO : kBufOOB, carry);
  }
  // the channel's last run: the tile's open run, or (no event in the tile)
  // the walked-back sum
  if (last) buf_store<TO>(rdy, (uint32_t)(tsN - 1 - e_base) * SO, nev ? sum : carry);
}

static unsigned nblk(int64_t waves) { return (unsigned)((waves + 3) / 4); }

// Scratch of the allocation-free restore backward (bcm_restore_bwd_noalloc):
// the per-tile head / tail partials and tile end indices, 3 words per
// (channel, tile), for up to BCM_RESTORE_BWD_NOALLOC_MAX_TILES of them
// (8 MiB per device, held until the process ends). Each device holds its own
// copy; host code uses the address that hipGetSymbolAddress gives for the
// current device, never the array's name.
constexpr int64_t kScratchWords = 3ll * BCM_RESTORE_BWD_NOALLOC_MAX_TILES;
static __device__ __align__(256) float scratch[kScratchWords];

// Device address of `scratch` on the current device, resolved once per
// device (first call on it) and cached.
static int scratch_ptr(float** out, const char* fn) {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDev] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
    return set_error(BCM_EHIP, "%s: no current HIP device", fn);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(BCM_EHIP, "%s: hipGetSymbolAddress(scratch) failed: %s", fn, hipGetErrorString(e));
    ptrs[dev] = p;
  }
  *out = static_cast<float*>(ptrs[dev]);
  return BCM_OK;
}

static int check_restore(const char* fn, const uint32_t* bitmask, int64_t mrd, const int32_t* tile_start,
                         int64_t n_rows, int64_t dim, int64_t L) {
  if (n_rows < 0 || dim < 1 || L < 1 || mrd < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (n_rows % dim != 0) return set_error(BCM_EINVAL, "%s: n_channels (B*D) must be divisible by dim", fn);
  if (n_rows > 0 && (!bitmask || !tile_start)) return set_error(BCM_EINVAL, "%s: null event index", fn);
  if ((reinterpret_cast<uintptr_t>(bitmask) & 7) != 0) return set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  return BCM_OK;
}

}  // namespace bcm

using namespace bcm;

extern "C" {

int bcm_build_event_index(const int32_t* t_steps, const int32_t* cu_seqlens, int64_t n_rows, int64_t L,
                          uint32_t* bitmask, int32_t* tile_start, float* zero_f32, int64_t n_zero,
                          bcm_stream_t stream) {
  const char* fn = "bcm_build_event_index";
  if (n_rows < 0 || L < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (n_zero < 0) return set_error(BCM_EINVAL, "%s: negative n_zero", fn);
  if (n_rows == 0) return zero_f32 ? zero_bytes(zero_f32, n_zero * 4, hs(stream), fn) : BCM_OK;
  if (!t_steps || !cu_seqlens || !bitmask || !tile_start) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L);
  const int64_t lds = W * 4;
  if (lds <= 65536)
    hipLaunchKernelGGL(k_build_index<true>, dim3((unsigned)n_rows), dim3(64), (size_t)lds, hs(stream), t_steps,
                       cu_seqlens, L, W, nT, bitmask, tile_start, zero_f32, n_zero);
  else
    hipLaunchKernelGGL(k_build_index<false>, dim3((unsigned)n_rows), dim3(64), 0, hs(stream), t_steps, cu_seqlens,
                       L, W, nT, bitmask, tile_start, zero_f32, n_zero);
  return check_launch(fn);
}

int bcm_restore_fwd(const void* y, int y_dtype, int64_t n_events, const uint32_t* bitmask, int64_t mask_row_div,
                    const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, void* out, int out_dtype,
                    bcm_stream_t stream) {
  const char* fn = "bcm_restore_fwd";
  if (!dtype_ok(y_dtype)) return set_error(BCM_EINVAL, "%s: y_flat must be fp32, fp16, or bf16", fn);
  if (!dtype_ok(out_dtype)) return set_error(BCM_EINVAL, "%s: out_dtype must be fp32, fp16, or bf16", fn);
  if (y_dtype != BCM_F32 && out_dtype != y_dtype)
    return set_error(BCM_EINVAL, "%s: %s input only supports %s output", fn, y_dtype == BCM_F16 ? "fp16" : "bf16",
                     y_dtype == BCM_F16 ? "fp16" : "bf16");
  int rc = check_restore(fn, bitmask, mask_row_div, tile_start, n_rows, dim, L);
  if (rc) return rc;
  if (n_rows == 0) return BCM_OK;
  if (!out) return set_error(BCM_EINVAL, "%s: null output", fn);
  if (n_events < 0 || (n_events > 0 && !y)) return set_error(BCM_EINVAL, "%s: invalid y", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (dim + kWave - 1) / kWave;
  const int64_t waves = (n_rows / dim) * nT * nG;
  // per-lane 32-bit buffer offsets span 64 rows of dim elements
  if (waves > INT32_MAX / 2 || dim > (1 << 22)) return set_error(BCM_EINVAL, "%s: problem too large", fn);
  auto go = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    if constexpr (sizeof(TO) == 2) {
      // two channels per lane: whole 256-byte row runs per store (dim even;
      // 4-byte aligned stores)
      if (dim % 2 == 0 && reinterpret_cast<uintptr_t>(out) % 4 == 0) {
        const int64_t nG2 = (dim + 2 * kWave - 1) / (2 * kWave), waves2 = (n_rows / dim) * nT * nG2;
        hipLaunchKernelGGL((k_restore_fwd_pair<TI, TO>), dim3(nblk(waves2)), dim3(256), 0, hs(stream),
                           static_cast<const TI*>(y), n_events, bitmask, W, mask_row_div, tile_start, (int)nT,
                           (int)nG2, (int)waves2, (int)dim, L, n_rows * L, static_cast<TO*>(out));
        return;
      }
    }
    hipLaunchKernelGGL((k_restore_fwd<TI, TO>), dim3(nblk(waves)), dim3(256), 0, hs(stream),
                       static_cast<const TI*>(y), n_events, bitmask, W, mask_row_div, tile_start, (int)nT, (int)nG,
                       (int)waves, (int)dim, L, n_rows * L, static_cast<TO*>(out));
  };
  if (y_dtype == BCM_F32) dispatch_dtype(out_dtype, [&](auto to) { go(float{}, to); });
  else if (y_dtype == BCM_F16) go(f16{}, f16{});
  else go(bf16{}, bf16{});
  return check_launch(fn);
}

int64_t bcm_restore_bwd_workspace_bytes(int64_t n_rows, int64_t L) {
  return (n_rows < 0 || L < 1) ? 0 : 3 * 4 * n_rows * tile_count(L);
}

}  // extern "C"

namespace bcm {

int restore_bwd_fix(int64_t nT, int64_t n_rows, const float* head, const float* tail, const int32_t* tend,
                    float* dy, int64_t n_events, hipStream_t stream, const char* fn) {
  hipLaunchKernelGGL(k_restore_bwd_fix, dim3((unsigned)((nT * n_rows + 255) / 256)), dim3(256), 0, stream, nT,
                     n_rows, head, tail, tend, dy, n_events);
  return check_launch(fn);
}

// Checks shared by both restore backward entry points (0: go on; 1: done,
// nothing to launch; negative: error code negated).
static int restore_bwd_checks(const char* fn, const void* dout, int dtype, const uint32_t* bitmask,
                              int64_t mask_row_div, const int32_t* tile_start, int64_t n_rows, int64_t dim,
                              int64_t L, const float* dy, int64_t n_events) {
  if (!dtype_ok(dtype)) return -set_error(BCM_EINVAL, "%s: dout must be fp32/fp16/bf16", fn);
  const int rc = check_restore(fn, bitmask, mask_row_div, tile_start, n_rows, dim, L);
  if (rc) return -rc;
  if (n_rows == 0) return 1;
  if (!dout || (n_events > 0 && !dy) || n_events < 0) return -set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_events * 4 > INT32_MAX) return -set_error(BCM_EINVAL, "%s: dy must be below 2 GiB", fn);
  return 0;
}

// Tile pass and fix-up pass with the side arrays in `workspace` (3 words
// per (channel, tile), fully written by the tile pass before the fix-up
// reads them).
static int restore_bwd_run(const char* fn, const void* dout, int dtype, const uint32_t* bitmask,
                           int64_t mask_row_div, const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L,
                           float* dy, int64_t n_events, float* workspace, hipStream_t stream) {
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (dim + kWave - 1) / kWave;
  float* head = workspace;
  float* tail = head + nT * n_rows;
  int32_t* tend = reinterpret_cast<int32_t*>(tail + nT * n_rows);
  const int64_t waves = (n_rows / dim) * nT * nG;
  if (waves > INT32_MAX / 2 || dim > (1 << 22)) return set_error(BCM_EINVAL, "%s: problem too large", fn);
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(k_restore_bwd_tiles<T>, dim3(nblk(waves)), dim3(256), 0, stream,
                       static_cast<const T*>(dout), n_events, bitmask, W, mask_row_div, tile_start, (int)nT,
                       (int)nG, (int)waves, (int)dim, L, n_rows, dy, head, tail, tend);
  });
  const int rc = check_launch(fn);
  if (rc) return rc;
  return restore_bwd_fix(nT, n_rows, head, tail, tend, dy, n_events, stream, fn);
}

}  // namespace bcm

extern "C" {

int bcm_restore_bwd(const void* dout, int dtype, const uint32_t* bitmask, int64_t mask_row_div,
                    const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, float* dy, int64_t n_events,
                    void* workspace, int64_t workspace_bytes, bcm_stream_t stream) {
  const char* fn = "bcm_restore_bwd";
  const int c = restore_bwd_checks(fn, dout, dtype, bitmask, mask_row_div, tile_start, n_rows, dim, L, dy, n_events);
  if (c) return c > 0 ? BCM_OK : -c;
  if (!workspace || workspace_bytes < bcm_restore_bwd_workspace_bytes(n_rows, L))
    return set_error(BCM_EINVAL, "%s: workspace of %lld bytes required", fn,
                     (long long)bcm_restore_bwd_workspace_bytes(n_rows, L));
  return restore_bwd_run(fn, dout, dtype, bitmask, mask_row_div, tile_start, n_rows, dim, L, dy, n_events,
                         static_cast<float*>(workspace), hs(stream));
}

int bcm_restore_bwd_noalloc(const void* dout, int dtype, const uint32_t* bitmask, int64_t mask_row_div,
                            const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, float* dy,
                            int64_t n_events, bcm_stream_t stream) {
  const char* fn = "bcm_restore_bwd_noalloc";
  const int c = restore_bwd_checks(fn, dout, dtype, bitmask, mask_row_div, tile_start, n_rows, dim, L, dy, n_events);
  if (c) return c > 0 ? BCM_OK : -c;
  if (n_rows * tile_count(L) > BCM_RESTORE_BWD_NOALLOC_MAX_TILES)
    return set_error(BCM_EINVAL, "%s: n_rows * ceil(L / 64) = %lld exceeds the scratch limit of %lld", fn,
                     (long long)(n_rows * tile_count(L)), (long long)BCM_RESTORE_BWD_NOALLOC_MAX_TILES);
  float* ws = nullptr;
  const int rc = scratch_ptr(&ws, fn);
  if (rc) return rc;
  return restore_bwd_run(fn, dout, dtype, bitmask, mask_row_div, tile_start, n_rows, dim, L, dy, n_events, ws,
                         hs(stream));
}

int64_t bcm_restore_bwd_sync_bytes(int64_t n_rows, int64_t L) {
  return (n_rows < 0 || L < 1) ? 0 : 8 * (kSyncHead + n_rows * tile_count(L));
}

int bcm_restore_bwd_chained(const void* dout, int dtype, const uint32_t* bitmask, int64_t mask_row_div,
                            const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, void* dy,
                            int dy_dtype, int64_t n_events, void* sync, int64_t sync_bytes, bcm_stream_t stream) {
  const char* fn = "bcm_restore_bwd_chained";
  if (dy_dtype != BCM_F32 && dy_dtype != dtype)
    return set_error(BCM_EINVAL, "%s: dy must be fp32 or dout's dtype", fn);
  const int c = restore_bwd_checks(fn, dout, dtype, bitmask, mask_row_div, tile_start, n_rows, dim, L,
                                   static_cast<const float*>(dy), n_events);
  if (c) return c > 0 ? BCM_OK : -c;
  if (!sync || (reinterpret_cast<uintptr_t>(sync) & 7) != 0 || sync_bytes < bcm_restore_bwd_sync_bytes(n_rows, L))
    return set_error(BCM_EINVAL, "%s: an 8-byte aligned sync area of %lld bytes required", fn,
                     (long long)bcm_restore_bwd_sync_bytes(n_rows, L));
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (dim + kWave - 1) / kWave;
  const int64_t waves = (n_rows / dim) * nT * nG;
  if (waves > INT32_MAX / 2 || dim > (1 << 22)) return set_error(BCM_EINVAL, "%s: problem too large", fn);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    return set_error(BCM_EHIP, "%s: cannot read the device's compute-unit count", fn);
  // launches of at most kChainBlocksPerCu blocks per CU, in wave-id order
  const int64_t per_launch = (int64_t)cus * kChainBlocksPerCu * kTileWaves;
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto otag) {
      using TO = decltype(otag);
      for (int64_t w0 = 0; w0 < waves; w0 += per_launch) {
        const int64_t n = std::min(per_launch, waves - w0);
        const int nb = (int)nblk(n);
        hipLaunchKernelGGL((k_restore_bwd_chain<T, TO>), dim3(nb), dim3(256), 0, hs(stream),
                           static_cast<const T*>(dout), n_events, bitmask, W, mask_row_div, tile_start, (int)nT,
                           (int)nG, (int)waves, (int)w0, nb, (int)dim, L, n_rows, static_cast<TO*>(dy),
                           static_cast<uint64_t*>(sync));
      }
    };
    if (dy_dtype == BCM_F32) go(float{});
    else go(T{});
  });
  return check_launch(fn);
}

}  // extern "C"
