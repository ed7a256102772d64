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
// serial pointer chasing) and there are no per-position atomics: the
// backward writes runs that end inside the tile with plain stores and only
// the two tile-crossing partial runs per lane with fp32 atomics.
#include "bcm_common.hpp"

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
  int64_t b, j, ch, dd;
  bool ok;
};

// wave id -> (b, tile j, channel group g); g varies fastest so neighbouring
// waves write neighbouring 256-byte pieces of the same (b, t) rows.
__device__ __forceinline__ TileWave tile_wave(int64_t n_rows, int64_t dim, int64_t nT, int64_t nG) {
  TileWave w;
  const int64_t wid = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int64_t Bn = n_rows / dim;
  w.ok = wid < Bn * nT * nG;
  const int64_t g = wid % nG, bj = wid / nG;
  w.j = bj % nT;
  w.b = bj / nT;
  w.dd = g * kWave + lane_id();
  w.ok = w.ok && w.dd < dim;
  w.ch = w.b * dim + w.dd;
  return w;
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_restore_fwd(const TI* __restrict__ y, const uint32_t* __restrict__ bitmask,
                                                     int64_t W, int64_t mrd, const int32_t* __restrict__ tile_start,
                                                     int64_t nT, int64_t n_rows, int64_t dim, int64_t L, int64_t nG,
                                                     TO* __restrict__ out) {
  const TileWave w = tile_wave(n_rows, dim, nT, nG);
  if (!w.ok) return;
  const int32_t* ts = tile_start + w.ch * (nT + 1);
  const int32_t cu0 = ts[0], elo = ts[w.j];
  const uint64_t m = tile_mask(bitmask + (w.ch / mrd) * W, w.j);
  float val = elo > cu0 ? to_f(y[elo - 1]) : 0.0f;
  const int64_t t0 = w.j * kTile;
  const int steps = (int)((L - t0) < kTile ? (L - t0) : kTile);
  float v[kTile];
  int idx = elo - 1;
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    if ((m >> s) & 1ull) {
      ++idx;
      v[s] = to_f(y[idx]);
    }
  }
  TO* o = out + (w.b * L + t0) * dim + w.dd;
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    if (s < steps) {
      if ((m >> s) & 1ull) val = v[s];
      o[(int64_t)s * dim] = from_f<TO>(val);
    }
  }
}

template <typename TI>
__global__ __launch_bounds__(256) void k_restore_bwd(const TI* __restrict__ dout, const uint32_t* __restrict__ bitmask,
                                                     int64_t W, int64_t mrd, const int32_t* __restrict__ tile_start,
                                                     int64_t nT, int64_t n_rows, int64_t dim, int64_t L, int64_t nG,
                                                     float* __restrict__ dy) {
  const TileWave w = tile_wave(n_rows, dim, nT, nG);
  if (!w.ok) return;
  const int32_t* ts = tile_start + w.ch * (nT + 1);
  const int32_t cu0 = ts[0], elo = ts[w.j];
  const uint64_t m = tile_mask(bitmask + (w.ch / mrd) * W, w.j);
  const int64_t t0 = w.j * kTile;
  const int steps = (int)((L - t0) < kTile ? (L - t0) : kTile);
  const TI* g = dout + (w.b * L + t0) * dim + w.dd;
  float gv[kTile];
#pragma unroll
  for (int s = 0; s < kTile; ++s) gv[s] = s < steps ? to_f(g[(int64_t)s * dim]) : 0.0f;
  float sum = 0.0f;
  int idx = elo - 1;
  bool head = true;  // the open run started before this tile
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    if ((m >> s) & 1ull) {
      if (head) {
        if (idx >= cu0) unsafeAtomicAdd(dy + idx, sum);
        head = false;
      } else {
        dy[idx] = sum;  // run started and ended inside this tile
      }
      ++idx;
      sum = 0.0f;
    }
    sum += gv[s];
  }
  if (idx >= cu0) unsafeAtomicAdd(dy + idx, sum);
}

static unsigned nblk(int64_t waves) { return (unsigned)((waves + 3) / 4); }

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

int bcm_restore_fwd(const void* y, int y_dtype, const uint32_t* bitmask, int64_t mask_row_div,
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
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (dim + kWave - 1) / kWave;
  const int64_t waves = (n_rows / dim) * nT * nG;
  auto go = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    hipLaunchKernelGGL((k_restore_fwd<TI, TO>), dim3(nblk(waves)), dim3(256), 0, hs(stream),
                       static_cast<const TI*>(y), bitmask, W, mask_row_div, tile_start, nT, n_rows, dim, L, nG,
                       static_cast<TO*>(out));
  };
  if (y_dtype == BCM_F32) dispatch_dtype(out_dtype, [&](auto to) { go(float{}, to); });
  else if (y_dtype == BCM_F16) go(f16{}, f16{});
  else go(bf16{}, bf16{});
  return check_launch(fn);
}

int bcm_restore_bwd(const void* dout, int dtype, const uint32_t* bitmask, int64_t mask_row_div,
                    const int32_t* tile_start, int64_t n_rows, int64_t dim, int64_t L, float* dy,
                    bcm_stream_t stream) {
  const char* fn = "bcm_restore_bwd";
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: dout must be fp32/fp16/bf16", fn);
  int rc = check_restore(fn, bitmask, mask_row_div, tile_start, n_rows, dim, L);
  if (rc) return rc;
  if (n_rows == 0) return BCM_OK;
  if (!dout || !dy) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  const int64_t W = bitmask_words(L), nT = tile_count(L), nG = (dim + kWave - 1) / kWave;
  const int64_t waves = (n_rows / dim) * nT * nG;
  dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(k_restore_bwd<T>, dim3(nblk(waves)), dim3(256), 0, hs(stream), static_cast<const T*>(dout),
                       bitmask, W, mask_row_div, tile_start, nT, n_rows, dim, L, nG, dy);
  });
  return check_launch(fn);
}

}  // extern "C"
