// Stage 3 fused with the block's output projection: zero-order-hold restore
// -> out_proj, forward and backward, without the dense restore output.
//
// Reference behaviour: e_model.py:499-504 (y_dense = restore_dense_fn(...);
// out = self.out_proj(y_dense)), i.e. out[b, t, :] = W z[b, t, :] + bias with
// z[b, t, d] = y of channel (b, d)'s last event at or before t (0 before its
// first; restore_dense_fwd_kernel.cuh:38-114) and W [d_model, D] the
// nn.Linear weight. Backward: dW = sum over (b, t) of dOut[b, t, :] (x)
// z[b, t, :], dz = dOut W, and dy[e] = sum of dz over the steps event e owns
// (restore_dense_bwd_kernel.cuh:42-112).
//
// MI355X design: z [B, L, D] and dz never exist in HBM. The products run on
// the matrix cores at their fp32 rate (v_mfma_f32_32x32x2_f32), on 64 x 64
// output tiles of 4 waves (32 x 32 each). The contraction index of MFMA step
// s pairs the two lane halves h as k = 16 h + s, so each lane's operand run
// is 16 consecutive elements of one row (or of one channel's steps).
//  - forward: per (b, 64-step tile j, 64 output columns), z is generated 32
//    channels at a time into LDS from the event index (one tile-mask
//    popcount and one gather per element, no search), double-buffered
//    against the MFMAs; W fragments come from L2.
//  - dy: the dz tile [64 steps x 64 channels] = dOut tile W[:, channels] is
//    staged once in LDS; one wave then runs the restore backward's sweep
//    over it (runs closed inside the tile go to dy; head, tail and last
//    event to the fix-up arrays) and the restore backward's fix-up pass
//    closes the runs that cross tiles. No atomics.
//  - dW: per (64 rows of W, 64 channels, one sequence segment of up to
//    1024 steps) a partial dOut^T z, with z generated per lane from the
//    event index (16 consecutive steps of one channel per MFMA operand run),
//    then a fixed-order sum of the partials (deterministic).
// fp32 throughout: the MFMA products are exact and accumulate in fp32, as
// the reference's fp32 GEMM does (in another order).
#include "bcm_common.hpp"

namespace bcm {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPT = 64;          // output tile edge
constexpr int kKC = 32;          // contraction chunk (16 MFMA steps)
constexpr int kRS = kKC + 4;     // LDS row stride of an operand chunk (16-byte rows, conflict-free 16-byte reads)
constexpr int kDS = kPT + 1;     // LDS row stride of a dz tile
constexpr int kSeg = 512;        // sequence steps per dW partial (1600 items at a config-4 layer)
static_assert(kSeg % 64 == 0, "a dW segment starts a 64-step tile");

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of the 32 x 32 MFMA result held in register r of lane half h (the
// column is the lane index mod 32).
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// z of one channel at step s (0..63) of a tile: the value of the last event
// at or before s. m: the tile's event mask, tsj: index of the channel's first
// event at or after the tile start, first: index of the channel's first
// event (earlier indices belong to other channels: z = 0).
__device__ __forceinline__ uint32_t zoh_off(uint64_t m, int s, int32_t tsj, int32_t first, bool ok) {
  const int32_t idx = tsj + (int32_t)__popcll(m << (63 - s)) - 1;
  return (ok && idx >= first) ? (uint32_t)idx * 4u : kBufOOB;
}

// ---------------------------------------------------------------- forward
// Item (b, j, nb): out rows t0 = 64 j .. t0 + 63 of sequence b, columns
// n0 = 64 nb .. n0 + 63. Wave w: rows 32 (w & 1), columns 32 (w >> 1).
// The tile's index words of every channel (mask, first event at or after
// the tile, first event of the channel) are staged in LDS once. Per
// 32-channel chunk both operands are staged in LDS, rows of 36 floats
// (double-buffered, one barrier per chunk): the W rows from coalesced row
// loads, and z with lane = step, so each gather instruction reads one
// channel's events of the tile (one or two cache lines). MFMA operand runs
// are read 4 at a time (16-byte LDS reads, conflict-free at this stride).
__global__ __launch_bounds__(256) void k_restore_proj_fwd(const float* __restrict__ y, int64_t n_events,
                                                          const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                          int64_t mrd, const int32_t* __restrict__ tile_start,
                                                          int nT, int dim, int L, const float* __restrict__ weight,
                                                          const float* __restrict__ bias, int dm, int nNB,
                                                          float* __restrict__ out) {
  extern __shared__ float4 s_dyn[];
  float* sZ = reinterpret_cast<float*>(s_dyn);  // [2][64][kRS]: z chunk [step][channel]
  float* sW = sZ + 2 * kPT * kRS;               // [2][64][kRS]: W chunk [row][channel]
  uint4* sIdx = reinterpret_cast<uint4*>(sW + 2 * kPT * kRS);  // [dim]: mask lo, mask hi, tsj, first
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int nb = item % nNB, bj = item / nNB;
  const int j = bj % nT, b = bj / nT;
  const int t0 = j * kTile, n0 = nb * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rb = 32 * (w & 1), cb = 32 * (w >> 1);
  const int li = lane & 31, h = lane >> 5;
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y, n_events * 4);
  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(weight, (int64_t)dm * dim * 4);
  for (int d = tid; d < dim; d += blockDim.x) {
    const int64_t ch = (int64_t)b * dim + d;
    const uint64_t m = tile_mask(bitmask + (ch / mrd) * Wd, j);
    const int32_t* ts = tile_start + ch * (nT + 1);
    sIdx[d] = make_uint4((uint32_t)m, (uint32_t)(m >> 32), (uint32_t)ts[j], (uint32_t)ts[0]);
  }
  __syncthreads();
  // z: wave w stages channels 8w .. 8w + 7 of the chunk, lane = step
  float zr[8];
  auto gen = [&](int c) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int d = c * kKC + 8 * w + q;  // wave-uniform
      const bool ok = d < dim;
      const uint4 ix = sIdx[ok ? d : 0];
      const uint64_t m = (uint64_t)ix.x | ((uint64_t)ix.y << 32);
      zr[q] = buf_load<float>(ry, zoh_off(m, lane, (int32_t)ix.z, (int32_t)ix.w, ok));
    }
  };
  // W: row (tid >> 3) + 32 i of the column tile, channels 4 (tid & 7) .. + 3
  float4 wr[2];
  const int wc = 4 * (tid & 7), wrow = tid >> 3;
  auto wload = [&](int c) {
    const int k = c * kKC + wc;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int n = n0 + wrow + 32 * i;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = buf_load<float>(rw, (n < dm && k + e < dim) ? (uint32_t)(n * dim + k + e) * 4u : kBufOOB);
      wr[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
  };
  const int nK = (dim + kKC - 1) / kKC;
  f32x16 acc = {};
  gen(0);
  wload(0);
  for (int c = 0; c < nK; ++c) {
    float* zb = sZ + (c & 1) * kPT * kRS;
    float* wb = sW + (c & 1) * kPT * kRS;
    *reinterpret_cast<float4*>(zb + lane * kRS + 8 * w) = make_float4(zr[0], zr[1], zr[2], zr[3]);
    *reinterpret_cast<float4*>(zb + lane * kRS + 8 * w + 4) = make_float4(zr[4], zr[5], zr[6], zr[7]);
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<float4*>(wb + (wrow + 32 * i) * kRS + wc) = wr[i];
    __syncthreads();  // chunk c staged; every wave is done with chunk c - 1's buffers
    if (c + 1 < nK) {  // the next chunk's loads fly under this chunk's MFMAs
      gen(c + 1);
      wload(c + 1);
    }
    const float4* za = reinterpret_cast<const float4*>(zb + (rb + li) * kRS + 16 * h);
    const float4* wa = reinterpret_cast<const float4*>(wb + (cb + li) * kRS + 16 * h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 a = za[v], bq = wa[v];
      acc = mfma32(a.x, bq.x, acc);
      acc = mfma32(a.y, bq.y, acc);
      acc = mfma32(a.z, bq.z, acc);
      acc = mfma32(a.w, bq.w, acc);
    }
  }
  // out[b, t0 + row, n]: lanes 0-31 and 32-63 each store a 128-byte row piece
  const int n = n0 + cb + li;
  const int64_t obase = ((int64_t)b * L + t0) * dm;
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out + obase, ((int64_t)(L - t0) * dm) * 4);
  const float bv = (bias && n < dm) ? bias[n] : 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = rb + acc_row(r, h);
    const bool ok = n < dm && t0 + row < L;
    buf_store_f32(ro, ok ? (uint32_t)(row * dm + n) * 4u : kBufOOB, acc[r] + bv);
  }
}

// ------------------------------------------------------------- dy (dz pass)
// Item (b, j, db): dz rows t0 .. t0 + 63, channels d0 = 64 db .. + 63. Per
// 32-row chunk of W: the dOut tile columns [step][k] from coalesced row
// loads, and W [k][channel] transposed into [channel][k] on its way to LDS,
// so both MFMA operand runs are 16-byte LDS reads (double-buffered, one
// barrier per chunk).
__global__ __launch_bounds__(256) void k_restore_proj_dy(const float* __restrict__ dout, int64_t n_events,
                                                         const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                         int64_t mrd, const int32_t* __restrict__ tile_start,
                                                         int nT, int dim, int L, int64_t n_rows,
                                                         const float* __restrict__ weight, int dm, int nDB,
                                                         float* __restrict__ dy, float* __restrict__ head,
                                                         float* __restrict__ tail, int32_t* __restrict__ tend) {
  __shared__ float4 s_ab[2 * 2 * kPT * kRS / 4];
  float* sA = reinterpret_cast<float*>(s_ab);  // [2][64][kRS]: dOut chunk [step][k]
  float* sB = sA + 2 * kPT * kRS;              // [2][64][kRS]: W chunk [channel][k]
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int db = item % nDB, bj = item / nDB;
  const int j = bj % nT, b = bj / nT;
  const int t0 = j * kTile, d0 = db * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rb = 32 * (w & 1), cb = 32 * (w >> 1);
  const int li = lane & 31, h = lane >> 5;
  const int64_t gbase = ((int64_t)b * L + t0) * dm;
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(dout + gbase, ((int64_t)(L - t0) * dm) * 4);
  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(weight, (int64_t)dm * dim * 4);
  // dOut: step (tid >> 3) + 32 i, columns 4 (tid & 7) .. + 3 of the chunk;
  // W: row (tid >> 6) + 4 i of the chunk, channel tid & 63
  const int ac = 4 * (tid & 7), ar = tid >> 3, bc = tid & 63, br = tid >> 6;
  float4 av[2];
  float bv[8];
  auto load = [&](int c) {
    const int k = c * kKC + ac;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = ar + 32 * i;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = buf_load<float>(rg, (t0 + row < L && k + e < dm) ? (uint32_t)(row * dm + k + e) * 4u : kBufOOB);
      av[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
    const int d = d0 + bc;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kr = c * kKC + br + 4 * i;
      bv[i] = buf_load<float>(rw, (kr < dm && d < dim) ? (uint32_t)(kr * dim + d) * 4u : kBufOOB);
    }
  };
  const int nK = (dm + kKC - 1) / kKC;
  f32x16 acc = {};
  load(0);
  for (int c = 0; c < nK; ++c) {
    float* ab = sA + (c & 1) * kPT * kRS;
    float* bb = sB + (c & 1) * kPT * kRS;
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<float4*>(ab + (ar + 32 * i) * kRS + ac) = av[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) bb[bc * kRS + br + 4 * i] = bv[i];
    __syncthreads();
    if (c + 1 < nK) load(c + 1);
    const float4* aa = reinterpret_cast<const float4*>(ab + (rb + li) * kRS + 16 * h);
    const float4* ba = reinterpret_cast<const float4*>(bb + (cb + li) * kRS + 16 * h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 a = aa[v], bq = ba[v];
      acc = mfma32(a.x, bq.x, acc);
      acc = mfma32(a.y, bq.y, acc);
      acc = mfma32(a.z, bq.z, acc);
      acc = mfma32(a.w, bq.w, acc);
    }
  }
  // dz tile [64 steps][64 channels] in LDS (over the operand buffers)
  __syncthreads();
  float* sD = sA;
  static_assert(4 * kPT * kRS >= kPT * kDS, "dz tile fits the operand buffers");
#pragma unroll
  for (int r = 0; r < 16; ++r) sD[(rb + acc_row(r, h)) * kDS + cb + li] = acc[r];
  __syncthreads();
  if (w != 0) return;
  // one wave: lane = channel d0 + lane, the restore backward's sweep over
  // the tile's 64 steps (rows past L hold 0 and have no event bits)
  const int dd = d0 + lane;
  const bool ok = dd < dim;
  const int64_t ch = (int64_t)b * dim + (ok ? dd : dim - 1);
  const uint64_t m = ok ? tile_mask(bitmask + (ch / mrd) * Wd, j) : 0ull;
  const int32_t elo = tile_start[ch * (nT + 1) + j];
  const __amdgpu_buffer_rsrc_t rdy = buf_rsrc(dy, n_events * 4);
  const int first = m ? __builtin_ctzll(m) : kTile;
  uint32_t r = 0;  // events seen so far in the tile
  float sum = 0.0f, hsum = 0.0f;
  for (int s = 0; s < kTile; ++s) {
    const float gv = sD[s * kDS + lane];
    const uint32_t bit = (uint32_t)(m >> s) & 1u;
    // the run of event elo + r - 1 closes here when r >= 1
    buf_store_f32(rdy, (bit && r) ? (uint32_t)(elo + (int32_t)r - 1) * 4u : kBufOOB, sum);
    r += bit;
    sum = (bit ? 0.0f : sum) + gv;
    hsum += s < first ? gv : 0.0f;
  }
  if (ok) {
    const int64_t o = (int64_t)j * n_rows + ch;
    head[o] = hsum;
    tail[o] = sum;
    tend[o] = r ? elo + (int32_t)r : -1;
  }
}

// ------------------------------------------------- dy, LDS-DMA form
// The dy product with both operands brought in by LDS DMA (gfx950's
// global_load_lds_dwordx4: 16 bytes per lane straight into LDS, no register
// staging), two stages in flight; for d_model % 32 == 0 and dim % 64 == 0
// (the items then never straddle the contraction or channel ends).
// Item (b, jj, db): dz rows t0 = 128 jj .. t0 + 127 (two 64-step tiles),
// channels d0 = 64 db .. + 63. Wave w: steps 64 (w & 1) .. + 63 (two 32-row
// MFMA blocks sharing one W fragment), channels 32 (w >> 1) .. + 31.
typedef __attribute__((address_space(3))) void* lds_vptr;
__device__ __forceinline__ uint32_t lds_off(const void* p) { return (uint32_t)(size_t)(lds_vptr)p; }
// 16 bytes per lane from gptr into LDS at the wave-uniform byte offset off +
// 16 * lane. The compiler does not track these loads: the kernel waits for
// them (vmcnt) before the barrier that hands the stage to the other waves.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t off) {
  const uint32_t o = __builtin_amdgcn_readfirstlane(off);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(o) : "memory", "m0");
}
__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// 16-byte slot of a 128-byte LDS row: rows 2i and 2i+1 keep their slots,
// the 8 row pairs rotate them, so 16 consecutive rows reading the same slot
// hit 16 different bank groups
__device__ __forceinline__ int qswz(int row) { return (row >> 1) & 7; }
constexpr int kDyT = 128;  // dz rows (steps) per item of the DMA form

__global__ __launch_bounds__(256) void k_restore_proj_dy_dma(const float* __restrict__ dout, int64_t n_events,
                                                             const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                             int64_t mrd, const int32_t* __restrict__ tile_start,
                                                             int nT, int dim, int L, int64_t n_rows,
                                                             const float* __restrict__ weight, int dm, int nDB,
                                                             float* __restrict__ dy, float* __restrict__ head,
                                                             float* __restrict__ tail, int32_t* __restrict__ tend) {
  extern __shared__ float4 s_dyn[];
  float* sA = reinterpret_cast<float*>(s_dyn);  // [2][128][32]: dOut rows, slots swizzled
  float* sB = sA + 2 * kDyT * kKC;              // [2][32][64]: W rows of the item's channels
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int nJJ = (nT + 1) / 2;
  const int db = item % nDB, bj = item / nDB;
  const int jj = bj % nJJ, b = bj / nJJ;
  const int t0 = jj * kDyT, d0 = db * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int li = lane & 31, h = lane >> 5;
  const int rb = 64 * (w & 1), cb = 32 * (w >> 1);
  const float* gb = dout + (int64_t)b * L * dm;
  auto issue = [&](int c, int st) {
    // dOut: 16 wave loads of 8 rows each (4 per wave); rows past L read row
    // L - 1 (their dz is not used)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int blk = 4 * w + i;
      const int row = blk * 8 + (lane >> 3);
      const int q = (lane & 7) ^ qswz(row);
      const int t = min(t0 + row, L - 1);
      lds_dma16(gb + (int64_t)t * dm + c * kKC + 4 * q, lds_off(sA + st * kDyT * kKC + blk * 256));
    }
    // W: 8 wave loads of 4 rows of 64 channels (2 per wave)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int blk = 2 * w + i;
      const int kr = blk * 4 + (lane >> 4);
      lds_dma16(weight + (int64_t)(c * kKC + kr) * dim + d0 + 4 * (lane & 15),
                lds_off(sB + st * kKC * kPT + blk * 256));
    }
  };
  const int nK = dm / kKC;
  f32x16 acc0 = {}, acc1 = {};
  issue(0, 0);
  for (int c = 0; c < nK; ++c) {
    wait_vmcnt0();    // this wave's part of stage c has landed
    __syncthreads();  // everyone's has, and every wave is done with stage c - 1
    if (c + 1 < nK) issue(c + 1, (c + 1) & 1);
    const float* ab = sA + (c & 1) * kDyT * kKC;
    const float* bb = sB + (c & 1) * kKC * kPT;
    const float4* a0 = reinterpret_cast<const float4*>(ab + (rb + li) * kKC);
    const float4* a1 = reinterpret_cast<const float4*>(ab + (rb + 32 + li) * kKC);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 p0 = a0[(4 * h + v) ^ qswz(rb + li)], p1 = a1[(4 * h + v) ^ qswz(rb + 32 + li)];
      const float* bk = bb + (16 * h + 4 * v) * kPT + cb + li;
      acc0 = mfma32(p0.x, bk[0], acc0);
      acc1 = mfma32(p1.x, bk[0], acc1);
      acc0 = mfma32(p0.y, bk[kPT], acc0);
      acc1 = mfma32(p1.y, bk[kPT], acc1);
      acc0 = mfma32(p0.z, bk[2 * kPT], acc0);
      acc1 = mfma32(p1.z, bk[2 * kPT], acc1);
      acc0 = mfma32(p0.w, bk[3 * kPT], acc0);
      acc1 = mfma32(p1.w, bk[3 * kPT], acc1);
    }
  }
  // dz tile [128 steps][64 channels] in LDS over the operand stages
  __syncthreads();
  float* sD = sA;
  static_assert(2 * kDyT * kKC + 2 * kKC * kPT >= kDyT * kDS, "dz tile fits the operand stages");
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    sD[(rb + acc_row(r, h)) * kDS + cb + li] = acc0[r];
    sD[(rb + 32 + acc_row(r, h)) * kDS + cb + li] = acc1[r];
  }
  __syncthreads();
  // waves 0 and 1: the restore backward's sweep over tile 2 jj + w, lane =
  // channel d0 + lane (rows past L count as 0 and hold no event bits)
  const int j = 2 * jj + w;
  if (w > 1 || j >= nT) return;
  const int64_t ch = (int64_t)b * dim + d0 + lane;
  const uint64_t m = tile_mask(bitmask + (ch / mrd) * Wd, j);
  const int32_t elo = tile_start[ch * (nT + 1) + j];
  const __amdgpu_buffer_rsrc_t rdy = buf_rsrc(dy, n_events * 4);
  const int first = m ? __builtin_ctzll(m) : kTile;
  const int steps = min(kTile, L - j * kTile);
  uint32_t r = 0;
  float sum = 0.0f, hsum = 0.0f;
  for (int s = 0; s < kTile; ++s) {
    const float gv = s < steps ? sD[(64 * w + s) * kDS + lane] : 0.0f;
    const uint32_t bit = (uint32_t)(m >> s) & 1u;
    buf_store_f32(rdy, (bit && r) ? (uint32_t)(elo + (int32_t)r - 1) * 4u : kBufOOB, sum);
    r += bit;
    sum = (bit ? 0.0f : sum) + gv;
    hsum += s < first ? gv : 0.0f;
  }
  const int64_t o = (int64_t)j * n_rows + ch;
  head[o] = hsum;
  tail[o] = sum;
  tend[o] = r ? elo + (int32_t)r : -1;
}

// --------------------------------------------- forward, LDS-DMA form
// The forward with W brought in by LDS DMA and z generated into LDS, for
// dim % 32 == 0 and d_model % 64 == 0. Item (b, jj, nb): out rows t0 = 128 jj
// .. + 127 (two 64-step tiles), columns n0 = 64 nb .. + 63. Wave w: steps
// 64 (w & 1) .. + 63 (two 32-row MFMA blocks sharing one W fragment),
// columns 32 (w >> 1) .. + 31. Both operands sit in 128-byte LDS rows with
// their 16-byte slots rotated per row pair (qswz), read 4 values at a time.
// z of chunk c: wave w generates tile 2 jj + (w & 1), channels 16 (w >> 1)
// .. + 15 of the chunk, lane = step (each gather reads one channel's events
// of the tile); the tiles' index words are staged once per item.
__global__ __launch_bounds__(256) void k_restore_proj_fwd_dma(const float* __restrict__ y, int64_t n_events,
                                                              const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                              int64_t mrd, const int32_t* __restrict__ tile_start,
                                                              int nT, int dim, int L,
                                                              const float* __restrict__ weight,
                                                              const float* __restrict__ bias, int dm, int nNB,
                                                              float* __restrict__ out) {
  extern __shared__ float4 s_dyn[];
  float* sZ = reinterpret_cast<float*>(s_dyn);                // [2][128][32]: z rows (steps)
  float* sW = sZ + 2 * kDyT * kKC;                            // [2][64][32]: W rows (columns of out)
  uint4* sIdx = reinterpret_cast<uint4*>(sW + 2 * kPT * kKC);  // [2][dim]: mask lo, hi, tsj, first
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int nJJ = (nT + 1) / 2;
  const int nb = item % nNB, bj = item / nNB;
  const int jj = bj % nJJ, b = bj / nJJ;
  const int t0 = jj * kDyT, n0 = nb * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int li = lane & 31, h = lane >> 5;
  const int rb = 64 * (w & 1), cb = 32 * (w >> 1);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y, n_events * 4);
  for (int i = tid; i < 2 * dim; i += blockDim.x) {
    const int th = i / dim, d = i - th * dim;
    const int j = min(2 * jj + th, nT - 1);  // a second tile past the end repeats the last (rows not stored)
    const int64_t ch = (int64_t)b * dim + d;
    const uint64_t m = tile_mask(bitmask + (ch / mrd) * Wd, j);
    const int32_t* ts = tile_start + ch * (nT + 1);
    sIdx[i] = make_uint4((uint32_t)m, (uint32_t)(m >> 32), (uint32_t)ts[j], (uint32_t)ts[0]);
  }
  __syncthreads();
  const int th = w & 1, zc = 16 * (w >> 1);
  float zr[16];
  auto gen = [&](int c) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const uint4 ix = sIdx[th * dim + c * kKC + zc + q];  // wave-uniform: an LDS broadcast
      const uint64_t m = (uint64_t)ix.x | ((uint64_t)ix.y << 32);
      zr[q] = buf_load<float>(ry, zoh_off(m, lane, (int32_t)ix.z, (int32_t)ix.w, true));
    }
  };
  auto issue_w = [&](int c, int st) {  // 8 wave loads of 8 W rows (2 per wave)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int blk = 2 * w + i;
      const int row = blk * 8 + (lane >> 3);
      const int q = (lane & 7) ^ qswz(row);
      lds_dma16(weight + (int64_t)(n0 + row) * dim + c * kKC + 4 * q, lds_off(sW + st * kPT * kKC + blk * 256));
    }
  };
  const int nK = dim / kKC;
  f32x16 acc0 = {}, acc1 = {};
  issue_w(0, 0);
  gen(0);
  const int zrow = 64 * th + lane;
  for (int c = 0; c < nK; ++c) {
    float* zb = sZ + (c & 1) * kDyT * kKC;
    float4* zrw = reinterpret_cast<float4*>(zb + zrow * kKC);
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      zrw[((zc >> 2) + qq) ^ qswz(zrow)] = make_float4(zr[4 * qq], zr[4 * qq + 1], zr[4 * qq + 2], zr[4 * qq + 3]);
    wait_vmcnt0();    // this wave's W rows of chunk c have landed
    __syncthreads();  // z and W of chunk c are staged; every wave is done with chunk c - 1
    if (c + 1 < nK) {
      issue_w(c + 1, (c + 1) & 1);
      gen(c + 1);
    }
    const float* wb = sW + (c & 1) * kPT * kKC;
    const float4* a0 = reinterpret_cast<const float4*>(zb + (rb + li) * kKC);
    const float4* a1 = reinterpret_cast<const float4*>(zb + (rb + 32 + li) * kKC);
    const float4* bw = reinterpret_cast<const float4*>(wb + (cb + li) * kKC);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 p0 = a0[(4 * h + v) ^ qswz(rb + li)], p1 = a1[(4 * h + v) ^ qswz(rb + 32 + li)];
      const float4 q = bw[(4 * h + v) ^ qswz(cb + li)];
      acc0 = mfma32(p0.x, q.x, acc0);
      acc1 = mfma32(p1.x, q.x, acc1);
      acc0 = mfma32(p0.y, q.y, acc0);
      acc1 = mfma32(p1.y, q.y, acc1);
      acc0 = mfma32(p0.z, q.z, acc0);
      acc1 = mfma32(p1.z, q.z, acc1);
      acc0 = mfma32(p0.w, q.w, acc0);
      acc1 = mfma32(p1.w, q.w, acc1);
    }
  }
  const int n = n0 + cb + li;
  const int64_t obase = ((int64_t)b * L + t0) * dm;
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out + obase, ((int64_t)(L - t0) * dm) * 4);
  const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int r0 = rb + acc_row(r, h), r1 = r0 + 32;
    buf_store_f32(ro, t0 + r0 < L ? (uint32_t)(r0 * dm + n) * 4u : kBufOOB, acc0[r] + bv);
    buf_store_f32(ro, t0 + r1 < L ? (uint32_t)(r1 * dm + n) * 4u : kBufOOB, acc1[r] + bv);
  }
}

// ----------------------------------------------------------- dW partials
// Item (p = b * nSeg + seg, nb, db): rows n0 = 128 nb .. of dW, channels
// d0 = 64 db .., the steps of segment seg of sequence b in 32-step chunks.
// Wave w: W rows 32 w, all 64 channels in two accumulators (two
// independent MFMA chains per wave, 32 MFMAs per chunk). Per chunk, dOut
// (transposed to [row of W][step] on its way to LDS) and z ([channel][step],
// lane = step: each gather reads one channel's events, two channels per
// instruction) are staged in LDS, so both operand runs (along the steps)
// are 16-byte LDS reads; z is gathered once per 128 rows of W.
constexpr int kPTW = 128;  // rows of W per dW item
__global__ __launch_bounds__(256) void k_restore_proj_dw(const float* __restrict__ dout,
                                                         const float* __restrict__ y, int64_t n_events,
                                                         const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                         int64_t mrd, const int32_t* __restrict__ tile_start,
                                                         int nT, int dim, int L, int dm, int nNB, int nDB,
                                                         int nSeg, float* __restrict__ part) {
  __shared__ float4 s_ab[2 * (kPTW + kPT) * kRS / 4];
  float* sA = reinterpret_cast<float*>(s_ab);  // [2][128][kRS]: dOut chunk [row of W][step]
  float* sZ = sA + 2 * kPTW * kRS;             // [2][64][kRS]: z chunk [channel][step]
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int db = item % nDB, r1 = item / nDB;
  const int nb = r1 % nNB, p = r1 / nNB;
  const int seg = p % nSeg, b = p / nSeg;
  const int n0 = nb * kPTW, d0 = db * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rb = 32 * w;
  const int li = lane & 31, h = lane >> 5;
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(dout + (int64_t)b * L * dm, (int64_t)L * dm * 4);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y, n_events * 4);
  // dOut: step (tid >> 6) + 4 i of the chunk, rows n0 + (tid & 63) and + 64
  const int an = tid & 63, at = tid >> 6;
  // z: lane step li, channels d0 + 32 h + 8 w + q
  int32_t zfirst[8];
  const int32_t* zts[8];
  const uint32_t* zmrow[8];
  bool zok[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int d = d0 + 32 * h + 8 * w + q;
    zok[q] = d < dim;
    const int64_t ch = (int64_t)b * dim + (zok[q] ? d : dim - 1);
    zmrow[q] = bitmask + (ch / mrd) * Wd;
    zts[q] = tile_start + ch * (nT + 1);
    zfirst[q] = zts[q][0];
  }
  // the index words (tile mask, first event at or after the tile) of the
  // current 64-step tile and of the next one, fetched a tile ahead, so a
  // chunk's gathers of y wait for no index load of their own (the next
  // tile's row is clamped at the last tile: in range, unused)
  uint64_t mcur[8], mnxt[8];
  int32_t tcur[8], tnxt[8];
  auto index_words = [&](int jt) {
    const int jc = min(jt, nT - 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      mnxt[q] = zok[q] ? tile_mask(zmrow[q], jc) : 0ull;
      tnxt[q] = zts[q][jc];
    }
  };
  float ar_[16], zr[8];
  auto load = [&](int t0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = t0 + at + 4 * (i & 7), n = n0 + an + 64 * (i >> 3);
      ar_[i] = buf_load<float>(rg, (t < L && n < dm) ? (uint32_t)(t * dm + n) * 4u : kBufOOB);
    }
    const int jt = t0 >> 6, so = (t0 & 63) + li;  // the chunk's 32 steps lie in tile jt
    if ((t0 & 63) == 0) {  // the first chunk of tile jt: its words are in, the next tile's go out
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        mcur[q] = mnxt[q];
        tcur[q] = tnxt[q];
      }
      index_words(jt + 1);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) zr[q] = buf_load<float>(ry, zoh_off(mcur[q], so, tcur[q], zfirst[q], zok[q]));
  };
  const int tb = seg * kSeg, te = min(L, tb + kSeg);
  f32x16 acc0 = {}, acc1 = {};
  index_words(tb >> 6);  // a segment starts a tile (kSeg % 64 == 0)
  load(tb);
  for (int t0 = tb, c = 0; t0 < te; t0 += kKC, ++c) {
    float* ab = sA + (c & 1) * kPTW * kRS;
    float* zb = sZ + (c & 1) * kPT * kRS;
#pragma unroll
    for (int i = 0; i < 16; ++i) ab[(an + 64 * (i >> 3)) * kRS + at + 4 * (i & 7)] = ar_[i];
#pragma unroll
    for (int q = 0; q < 8; ++q) zb[(32 * h + 8 * w + q) * kRS + li] = zr[q];
    __syncthreads();
    if (t0 + kKC < te) load(t0 + kKC);
    const float4* aa = reinterpret_cast<const float4*>(ab + (rb + li) * kRS + 16 * h);
    const float4* za0 = reinterpret_cast<const float4*>(zb + li * kRS + 16 * h);
    const float4* za1 = reinterpret_cast<const float4*>(zb + (32 + li) * kRS + 16 * h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 a = aa[v], b0 = za0[v], b1 = za1[v];
      acc0 = mfma32(a.x, b0.x, acc0);
      acc1 = mfma32(a.x, b1.x, acc1);
      acc0 = mfma32(a.y, b0.y, acc0);
      acc1 = mfma32(a.y, b1.y, acc1);
      acc0 = mfma32(a.z, b0.z, acc0);
      acc1 = mfma32(a.z, b1.z, acc1);
      acc0 = mfma32(a.w, b0.w, acc0);
      acc1 = mfma32(a.w, b1.w, acc1);
    }
  }
  float* pp = part + (int64_t)p * dm * dim;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int nr = n0 + rb + acc_row(r, h);
    if (nr < dm && d0 + li < dim) pp[(int64_t)nr * dim + d0 + li] = acc0[r];
    if (nr < dm && d0 + 32 + li < dim) pp[(int64_t)nr * dim + d0 + 32 + li] = acc1[r];
  }
}

// dW by LDS DMA (d_model % 128 == 0, L % 32 == 0: every DMA row is a
// whole 512-byte run of one step of dOut inside the sequence). The
// transposed product dW^T[d][n] = sum_t z[t][d] dOut[t][n]: z is the MFMA A
// operand ([channel][step] in LDS, 16-byte reads along the steps, as
// above) and dOut the B operand in its own [step][n] layout, brought into
// LDS by global_load_lds_dwordx4 (no register staging, no transposing
// stores), one 4-byte read per MFMA step. Item (p, nb, db): n0 = 128 nb,
// d0 = 64 db; wave w: n block 32 w, channel blocks 0 and 1 (two chains).
// A chunk's 32 dOut rows sit in row pairs of kDwPair floats (two 512-byte
// rows and 16 bytes of padding): the lane halves read rows 16 apart, 8 row
// pairs = 2080 floats apart, on opposite halves of the 64 banks. The
// partials are laid out [p][d][n] (lanes write consecutive n).
constexpr int kDwPair = 2 * kPTW + 4;  // floats per dOut row pair in LDS
__global__ __launch_bounds__(256) void k_restore_proj_dw_dma(const float* __restrict__ dout,
                                                             const float* __restrict__ y, int64_t n_events,
                                                             const uint32_t* __restrict__ bitmask, int64_t Wd,
                                                             int64_t mrd, const int32_t* __restrict__ tile_start,
                                                             int nT, int dim, int L, int dm, int nNB, int nDB,
                                                             int nSeg, float* __restrict__ part) {
  __shared__ float4 s_dw[(2 * (kKC / 2) * kDwPair + 2 * kPT * kRS) / 4];
  float* sB = reinterpret_cast<float*>(s_dw);    // [2][16 row pairs][kDwPair]: dOut chunk [step][n]
  float* sZ = sB + 2 * (kKC / 2) * kDwPair;      // [2][64][kRS]: z chunk [channel][step]
  const int item = xcd_block(blockIdx.x, gridDim.x);
  const int db = item % nDB, r1 = item / nDB;
  const int nb = r1 % nNB, p = r1 / nNB;
  const int seg = p % nSeg, b = p / nSeg;
  const int n0 = nb * kPTW, d0 = db * kPT;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int li = lane & 31, h = lane >> 5;
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y, n_events * 4);
  // z: lane step li, channels d0 + 32 h + 8 w + q
  int32_t zfirst[8];
  const int32_t* zts[8];
  const uint32_t* zmrow[8];
  bool zok[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int d = d0 + 32 * h + 8 * w + q;
    zok[q] = d < dim;
    const int64_t ch = (int64_t)b * dim + (zok[q] ? d : dim - 1);
    zmrow[q] = bitmask + (ch / mrd) * Wd;
    zts[q] = tile_start + ch * (nT + 1);
    zfirst[q] = zts[q][0];
  }
  uint64_t mcur[8], mnxt[8];
  int32_t tcur[8], tnxt[8];
  auto index_words = [&](int jt) {  // a tile ahead, as in k_restore_proj_dw
    const int jc = min(jt, nT - 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      mnxt[q] = zok[q] ? tile_mask(zmrow[q], jc) : 0ull;
      tnxt[q] = zts[q][jc];
    }
  };
  float zr[8];
  auto gather = [&](int t0) {
    const int jt = t0 >> 6, so = (t0 & 63) + li;
    if ((t0 & 63) == 0) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        mcur[q] = mnxt[q];
        tcur[q] = tnxt[q];
      }
      index_words(jt + 1);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) zr[q] = buf_load<float>(ry, zoh_off(mcur[q], so, tcur[q], zfirst[q], zok[q]));
  };
  // wave w brings row pairs 4 w .. 4 w + 3 of the chunk: lane l takes 16
  // bytes of row 2 pp + (l >> 5) at n0 + 4 (l & 31)
  const float* gd = dout + (int64_t)b * L * dm + n0 + 4 * li;
  auto dma = [&](int t0, int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pp = 4 * w + i;
      lds_dma16(gd + (int64_t)(t0 + 2 * pp + h) * dm, lds_off(sB + (st * (kKC / 2) + pp) * kDwPair));
    }
  };
  const int tb = seg * kSeg, te = min(L, tb + kSeg);
  f32x16 acc0 = {}, acc1 = {};
  index_words(tb >> 6);
  dma(tb, 0);
  gather(tb);
  for (int t0 = tb, c = 0; t0 < te; t0 += kKC, ++c) {
    const int st = c & 1;
    float* zb = sZ + st * kPT * kRS;
#pragma unroll
    for (int q = 0; q < 8; ++q) zb[(32 * h + 8 * w + q) * kRS + li] = zr[q];
    wait_vmcnt0();  // this wave's dOut rows of chunk c have landed
    __syncthreads();
    if (t0 + kKC < te) {
      dma(t0 + kKC, st ^ 1);
      gather(t0 + kKC);
    }
    const float* bl = sB + st * (kKC / 2) * kDwPair + h * 8 * kDwPair + 32 * w + li;
    const float4* za0 = reinterpret_cast<const float4*>(zb + li * kRS + 16 * h);
    const float4* za1 = reinterpret_cast<const float4*>(zb + (32 + li) * kRS + 16 * h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 a0 = za0[v], a1 = za1[v];
      const float a0v[4] = {a0.x, a0.y, a0.z, a0.w}, a1v[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sidx = 4 * v + e;  // MFMA step: steps 16 h + sidx of the chunk
        const float bv = bl[(sidx >> 1) * kDwPair + (sidx & 1) * kPTW];
        acc0 = mfma32(a0v[e], bv, acc0);
        acc1 = mfma32(a1v[e], bv, acc1);
      }
    }
  }
  float* pp = part + (int64_t)p * dm * dim;
  const int n = n0 + 32 * w + li;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int dr = d0 + acc_row(r, h);
    if (dr < dim) pp[(int64_t)dr * dm + n] = acc0[r];
    if (dr + 32 < dim) pp[(int64_t)(dr + 32) * dm + n] = acc1[r];
  }
}

// dW = sum of the partials in partial order.
// dmajor: partials laid out [p][d][n] (the DMA form); the thread of partial
// element i (consecutive i: coalesced reads) writes dW[n][d].
__global__ __launch_bounds__(256) void k_restore_proj_dw_sum(const float* __restrict__ part, int64_t n_parts,
                                                             int64_t count, int dm, int dim, int dmajor,
                                                             float* __restrict__ dw) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float v = 0.0f;
  int64_t q = 0;
  for (; q + 4 <= n_parts; q += 4) {  // 4 loads in flight, summed in order
    const float a0 = part[q * count + i], a1 = part[(q + 1) * count + i];
    const float a2 = part[(q + 2) * count + i], a3 = part[(q + 3) * count + i];
    v = (((v + a0) + a1) + a2) + a3;
  }
  for (; q < n_parts; ++q) v += part[q * count + i];
  dw[dmajor ? (i % dm) * dim + i / dm : i] = v;
}

struct ProjShape {
  int64_t W, nT, nNB, nNBW, nDB, nSeg, n_parts;
};

static ProjShape proj_shape(int64_t n_rows, int64_t dim, int64_t L, int64_t dm) {
  ProjShape s;
  s.W = bitmask_words(L);
  s.nT = tile_count(L);
  s.nNB = (dm + kPT - 1) / kPT;
  s.nNBW = (dm + kPTW - 1) / kPTW;
  s.nDB = (dim + kPT - 1) / kPT;
  s.nSeg = (L + kSeg - 1) / kSeg;
  s.n_parts = (n_rows / dim) * s.nSeg;
  return s;
}

static int check_proj(const char* fn, const uint32_t* bitmask, int64_t mrd, const int32_t* tile_start,
                      int64_t n_rows, int64_t dim, int64_t L, const float* weight, int64_t dm, int64_t n_events) {
  if (n_rows < 0 || dim < 1 || L < 1 || mrd < 1 || dm < 1) return set_error(BCM_EINVAL, "%s: invalid sizes", fn);
  if (n_rows % dim) return set_error(BCM_EINVAL, "%s: n_rows must be a multiple of dim", fn);
  if (n_rows && (!bitmask || !tile_start || !weight)) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_events < 0 || n_events * 4 > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_events out of range", fn);
  // 32-bit buffer offsets: one W, one sequence of dout / out
  if (dm * dim * 4 > INT32_MAX || L * dm * 4 > INT32_MAX || n_rows / dim * tile_count(L) * ((dm + kPT - 1) / kPT) >
                                                                 INT32_MAX / 2)
    return set_error(BCM_EINVAL, "%s: problem too large", fn);
  return BCM_OK;
}

}  // namespace bcm

using namespace bcm;

extern "C" {

int bcm_restore_proj_fwd(const float* y, int64_t n_events, const uint32_t* bitmask, int64_t mask_row_div,
                         const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, const float* weight,
                         const float* bias, int64_t d_model, float* out, bcm_stream_t stream) {
  const char* fn = "bcm_restore_proj_fwd";
  int rc = check_proj(fn, bitmask, mask_row_div, tile_start, n_rows, dim, L, weight, d_model, n_events);
  if (rc) return rc;
  if (n_rows == 0) return BCM_OK;
  if (!out || (n_events > 0 && !y)) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  const ProjShape s = proj_shape(n_rows, dim, L, d_model);
  // the LDS-DMA form wants whole 32-channel chunks, whole 64-column blocks
  // and 16-byte aligned W rows; its per-channel index words take 32 bytes
  // of LDS per channel, so wide layers (dim above ~3.5k on a 160 KB part)
  // take the register-staged form, which needs 16
  const size_t lds_dma = (size_t)(2 * kDyT * kKC + 2 * kPT * kKC) * 4 + (size_t)dim * 32;
  const bool dma = dim % kKC == 0 && d_model % kPT == 0 && (reinterpret_cast<uintptr_t>(weight) & 15) == 0 &&
                   (int64_t)lds_dma <= max_lds_bytes();
  if (dma) {
    const int64_t items = (n_rows / dim) * ((s.nT + 1) / 2) * s.nNB;
    const size_t lds = lds_dma;
    hipLaunchKernelGGL(k_restore_proj_fwd_dma, dim3((unsigned)items), dim3(256), lds, hs(stream), y, n_events, bitmask,
                       s.W, mask_row_div, tile_start, (int)s.nT, (int)dim, (int)L, weight, bias, (int)d_model,
                       (int)s.nNB, out);
    return check_launch(fn);
  }
  const int64_t items = (n_rows / dim) * s.nT * s.nNB;
  const size_t lds = (size_t)(4 * kPT * kRS) * 4 + (size_t)dim * 16;  // operand buffers + per-channel index words
  if ((int64_t)lds > max_lds_bytes())
    return set_error(BCM_EINVAL, "%s: dim %lld needs %lld bytes of LDS", fn, (long long)dim, (long long)lds);
  hipLaunchKernelGGL(k_restore_proj_fwd, dim3((unsigned)items), dim3(256), lds, hs(stream), y, n_events, bitmask, s.W,
                     mask_row_div, tile_start, (int)s.nT, (int)dim, (int)L, weight, bias, (int)d_model, (int)s.nNB,
                     out);
  return check_launch(fn);
}

int64_t bcm_restore_proj_bwd_workspace_bytes(int64_t n_rows, int64_t dim, int64_t L, int64_t d_model) {
  if (n_rows < 0 || dim < 1 || L < 1 || d_model < 1) return 0;
  const ProjShape s = proj_shape(n_rows, dim, L, d_model);
  return 3 * 4 * n_rows * s.nT + 4 * s.n_parts * d_model * dim;
}

int bcm_restore_proj_bwd(const float* dout, const float* y, int64_t n_events, const uint32_t* bitmask,
                         int64_t mask_row_div, const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L,
                         const float* weight, int64_t d_model, float* dy, float* dweight, void* workspace,
                         int64_t workspace_bytes, bcm_stream_t stream) {
  const char* fn = "bcm_restore_proj_bwd";
  int rc = check_proj(fn, bitmask, mask_row_div, tile_start, n_rows, dim, L, weight, d_model, n_events);
  if (rc) return rc;
  if (!dout && n_rows) return set_error(BCM_EINVAL, "%s: null dout", fn);
  if (dweight && n_events > 0 && !y) return set_error(BCM_EINVAL, "%s: dweight needs y", fn);
  const ProjShape s = proj_shape(n_rows, dim, L, d_model);
  // the fix-up arrays always, the weight gradient's partials only with dweight
  const int64_t need = 3 * 4 * n_rows * s.nT + (dweight ? 4 * s.n_parts * d_model * dim : 0);
  if (!workspace || workspace_bytes < need)
    return set_error(BCM_EINVAL, "%s: workspace of %lld bytes required", fn, (long long)need);
  const hipStream_t st = hs(stream);
  const int64_t B = n_rows / dim;
  if (B * s.nT * s.nDB > INT32_MAX / 2 || s.n_parts * s.nNB * s.nDB > INT32_MAX / 2)
    return set_error(BCM_EINVAL, "%s: problem too large", fn);
  float* head = static_cast<float*>(workspace);
  float* tail = head + s.nT * n_rows;
  int32_t* tend = reinterpret_cast<int32_t*>(tail + s.nT * n_rows);
  float* part = reinterpret_cast<float*>(tend + s.nT * n_rows);
  if (dy && n_events > 0) {
    // the LDS-DMA form wants whole 32-row chunks of W, whole 64-channel
    // blocks and 16-byte aligned rows
    const bool dma = d_model % kKC == 0 && dim % kPT == 0 && (reinterpret_cast<uintptr_t>(dout) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(weight) & 15) == 0;
    if (dma) {
      const int64_t nJJ = (s.nT + 1) / 2;
      const size_t lds = (size_t)(2 * kDyT * kKC + 2 * kKC * kPT) * 4;
      hipLaunchKernelGGL(k_restore_proj_dy_dma, dim3((unsigned)(B * nJJ * s.nDB)), dim3(256), lds, st, dout,
                         n_events, bitmask, s.W, mask_row_div, tile_start, (int)s.nT, (int)dim, (int)L, n_rows,
                         weight, (int)d_model, (int)s.nDB, dy, head, tail, tend);
    } else {
      hipLaunchKernelGGL(k_restore_proj_dy, dim3((unsigned)(B * s.nT * s.nDB)), dim3(256), 0, st, dout, n_events,
                         bitmask, s.W, mask_row_div, tile_start, (int)s.nT, (int)dim, (int)L, n_rows, weight,
                         (int)d_model, (int)s.nDB, dy, head, tail, tend);
    }
    if ((rc = check_launch(fn))) return rc;
    if ((rc = restore_bwd_fix(s.nT, n_rows, head, tail, tend, dy, n_events, st, fn))) return rc;
  }
  if (dweight) {  // no tokens (n_parts = 0): the sum writes dW = 0
    // the LDS-DMA form where every dOut row it brings is a whole 512-byte
    // run inside the sequence
    const bool dma = d_model % kPTW == 0 && L % kKC == 0;
    const dim3 grid((unsigned)(s.n_parts * s.nNBW * s.nDB));
    if (s.n_parts > 0 && dma)
      hipLaunchKernelGGL(k_restore_proj_dw_dma, grid, dim3(256), 0, st, dout, y, n_events, bitmask, s.W,
                         mask_row_div, tile_start, (int)s.nT, (int)dim, (int)L, (int)d_model, (int)s.nNBW,
                         (int)s.nDB, (int)s.nSeg, part);
    else if (s.n_parts > 0)
      hipLaunchKernelGGL(k_restore_proj_dw, grid, dim3(256), 0, st, dout, y, n_events, bitmask, s.W, mask_row_div,
                         tile_start, (int)s.nT, (int)dim, (int)L, (int)d_model, (int)s.nNBW, (int)s.nDB,
                         (int)s.nSeg, part);
    if ((rc = check_launch(fn))) return rc;
    const int64_t count = d_model * dim;
    hipLaunchKernelGGL(k_restore_proj_dw_sum, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, part,
                       s.n_parts, count, (int)d_model, (int)dim, dma ? 1 : 0, dweight);
    if ((rc = check_launch(fn))) return rc;
  }
  return BCM_OK;
}

}  // extern "C"
