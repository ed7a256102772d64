// Causal depthwise conv1d + SiLU, the producer of x_conv (the values the
// event gather reads), forward and backward.
//
// Reference behaviour: e_model.py:442-451 (x = silu(conv1d(x)[..., :L]),
// nn.Conv1d(groups=d_inner, kernel_size=d_conv, padding=d_conv-1) or
// causal_conv1d_fn with activation "silu"; the causal_conv1d package is not
// part of the reference tree and is not installed here):
//   pre[b,d,t] = bias[d] + sum_k w[d,k] * x[b,d,t-(K-1)+k]   (x = 0 before t=0)
//   out[b,d,t] = pre * sigmoid(pre)
// Backward, with g = dout * sigmoid(pre) * (1 + pre * (1 - sigmoid(pre))):
//   dx[b,d,t] = sum_k w[d,k] * g[b,d,t+(K-1)-k]   (terms past L vanish)
//   dw[d,k]   = sum_{b,t} g[b,d,t] * x[b,d,t-(K-1)+k],  dbias[d] = sum_{b,t} g
//
// MI355X design: rows (b, d) of L steps are contiguous. Each thread takes 4
// consecutive steps of one row, read and written as whole 16-byte (fp32) or
// 8-byte (fp16/bf16) vectors when L is a multiple of 4, with the K-1 halo
// steps from the neighbouring vectors (L1 hits), so a wave covers 256
// contiguous steps. The backward recomputes g from x (no saved
// pre-activation); workgroup (d, p) takes every P-th batch row of channel d
// (P chosen to fill the chip), writes dx, and reduces its dw / dbias
// partials in registers and LDS in a fixed order; a small kernel sums the P
// partials in group order (deterministic, no atomics). HBM-bound: x and dout
// read once, out / dx written once.
#include "bcm_common.hpp"

#include <algorithm>
#include <type_traits>

namespace bcm {

constexpr int kConvMaxK = 8;
constexpr int kConvSteps = 4;  // consecutive steps per thread
constexpr int kConvMaxSplit = 64;  // batch groups of the backward

// x[t .. t+3] of a row as floats: one 16-byte (fp32) or 8-byte (fp16/bf16)
// load when VEC (t a multiple of 4, rows aligned), zeros for t < 0 or t >= L
// (whole vectors: L is a multiple of 4 then); else per element with bounds.
template <typename T, bool VEC>
__device__ __forceinline__ void load4(const T* __restrict__ r, int64_t t, int64_t L, float* v) {
  if (VEC) {
    if (t < 0 || t >= L) {
      v[0] = v[1] = v[2] = v[3] = 0.0f;
    } else if constexpr (sizeof(T) == 4) {
      const float4 q = *reinterpret_cast<const float4*>(r + t);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
      const uint2 q = *reinterpret_cast<const uint2*>(r + t);
      const T* e = reinterpret_cast<const T*>(&q);
      v[0] = to_f(e[0]); v[1] = to_f(e[1]); v[2] = to_f(e[2]); v[3] = to_f(e[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (t + i >= 0 && t + i < L) ? to_f(r[t + i]) : 0.0f;
  }
}

template <typename T, bool VEC>
__device__ __forceinline__ void store4(T* __restrict__ r, int64_t t, int64_t L, const float* v) {
  if (VEC) {
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<float4*>(r + t) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      T e[4] = {from_f<T>(v[0]), from_f<T>(v[1]), from_f<T>(v[2]), from_f<T>(v[3])};
      *reinterpret_cast<uint2*>(r + t) = *reinterpret_cast<const uint2*>(e);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (t + i < L) r[t + i] = from_f<T>(v[i]);
  }
}

// KM = 4: width exactly 4 (d_conv's default), straight-line code; KM = 8:
// any width K <= 8 given at run time.
template <typename T, bool SILU, bool VEC, int KM>
__global__ __launch_bounds__(256) void k_conv_fwd(const T* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ bias, T* __restrict__ out, int64_t rows,
                                                  int D, int64_t L, int K_, int64_t chunks) {
  const int K = KM == 4 ? 4 : K_;
  constexpr int PRE = (KM - 1 + 3) / 4 * 4;  // halo steps before t0, whole vectors
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * chunks) return;
  const int64_t row = gid / chunks;
  const int64_t t0 = (gid - row * chunks) * kConvSteps;
  const int d = (int)(row % D);
  const T* xr = x + row * L;
  float wk[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) wk[k] = k < K ? w[(int64_t)d * K + k] : 0.0f;
  const float b0 = bias ? bias[d] : 0.0f;
  // window x[t0-PRE .. t0+3] (xv[i] = x[t0-PRE+i])
  float xv[PRE + 4];
#pragma unroll
  for (int v = 0; v < PRE / 4 + 1; ++v) load4<T, VEC>(xr, t0 - PRE + 4 * v, L, xv + 4 * v);
  float o[kConvSteps];
#pragma unroll
  for (int s = 0; s < kConvSteps; ++s) {
    // step t0+s reads x[t0+s-(K-1)+k] = xv[PRE+s-(K-1)+k]
    float pre = b0;
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (k < K) pre = fmaf(wk[k], xv[PRE + s - (K - 1) + k], pre);
    o[s] = SILU ? pre / (1.0f + __expf(-pre)) : pre;
  }
  store4<T, VEC>(out + row * L, t0, L, o);
}

// Backward of a group of batch rows of channel d: workgroup (d, p) takes the
// rows b = p, p + P, ... (P = gridDim.y); with P > 1 its dw / dbias partials
// go to part[(p * D + d) * (K + 1) ...] for k_conv_bwd_reduce.
template <typename T, bool SILU, bool VEC, int KM>
__global__ __launch_bounds__(256) void k_conv_bwd(const T* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ bias, const T* __restrict__ dout,
                                                  T* __restrict__ dx, float* __restrict__ dw,
                                                  float* __restrict__ dbias, float* __restrict__ part, int B, int D,
                                                  int64_t L, int K_) {
  const int K = KM == 4 ? 4 : K_;  // KM = 4: width exactly 4
  constexpr int PRE = (KM - 1 + 3) / 4 * 4;       // halo steps before t0, whole vectors
  constexpr int NG = kConvSteps + KM - 1;          // g at t0 .. t0+NG-1
  constexpr int NGV = (NG + 3) / 4 * 4;            // ... in whole vectors
  constexpr int NX = PRE + NGV;                    // x at t0-PRE .. t0+NGV-1
  __shared__ float s_red[kConvMaxK + 1][256 / kWave];
  const int d = blockIdx.x, p = blockIdx.y, P = gridDim.y;
  float wk[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) wk[k] = k < K ? w[(int64_t)d * K + k] : 0.0f;
  const float b0 = bias ? bias[d] : 0.0f;
  float aw[kConvMaxK], ab = 0.0f;  // this thread's dw / dbias partials
#pragma unroll
  for (int k = 0; k < kConvMaxK; ++k) aw[k] = 0.0f;
  for (int b = p; b < B; b += P) {
    const int64_t row = (int64_t)b * D + d;
    const T* xr = x + row * L;
    const T* gr = dout + row * L;
    T* dxr = dx + row * L;
    for (int64_t t0 = (int64_t)threadIdx.x * kConvSteps; t0 < L; t0 += (int64_t)blockDim.x * kConvSteps) {
      float xv[NX], go[NGV];  // xv[i] = x[t0-PRE+i], go[i] = dout[t0+i]
#pragma unroll
      for (int v = 0; v < NX / 4; ++v) load4<T, VEC>(xr, t0 - PRE + 4 * v, L, xv + 4 * v);
#pragma unroll
      for (int v = 0; v < NGV / 4; ++v) load4<T, VEC>(gr, t0 + 4 * v, L, go + 4 * v);
      // g at steps t0+i (zero past L: go is zero there)
      float g[NG];
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        float pre = b0;
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (k < K) pre = fmaf(wk[k], xv[PRE + i - (K - 1) + k], pre);
        if (SILU) {
          const float sg = 1.0f / (1.0f + __expf(-pre));
          g[i] = go[i] * sg * fmaf(pre, 1.0f - sg, 1.0f);  // one rounding, in both conv backwards
        } else {
          g[i] = go[i];
        }
      }
      float o[kConvSteps];
#pragma unroll
      for (int s = 0; s < kConvSteps; ++s) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (k < K) acc = fmaf(wk[k], g[s + (K - 1) - k], acc);
        o[s] = acc;
        // dw[k] += g[t] x[t-(K-1)+k] over this thread's own steps (g is 0 past L)
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (k < K) aw[k] = fmaf(g[s], xv[PRE + s - (K - 1) + k], aw[k]);
        ab += g[s];
      }
      store4<T, VEC>(dxr, t0, L, o);
    }
  }
  // fixed-order reduction: butterfly within each wave, then the waves in order
  const int wave = threadIdx.x / kWave, lane = lane_id();
#pragma unroll
  for (int k = 0; k <= kConvMaxK; ++k) {
    float v = k < kConvMaxK ? aw[k] : ab;
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    if (lane == 0) s_red[k][wave] = v;
  }
  __syncthreads();
  if (threadIdx.x <= kConvMaxK) {
    const int k = threadIdx.x;
    float v = 0.0f;
    for (int q = 0; q < (int)(blockDim.x / kWave); ++q) v += s_red[k][q];
    const int slot = k < kConvMaxK ? k : K;  // dbias after the K weights
    if (k < K || k == kConvMaxK) {
      if (P > 1) part[((int64_t)p * D + d) * (K + 1) + slot] = v;
      else if (k < K) dw[(int64_t)d * K + k] = v;
      else if (dbias) dbias[d] = v;
    }
  }
}

// dw / dbias from the P batch groups' partials, summed in group order.
__global__ __launch_bounds__(256) void k_conv_bwd_reduce(const float* __restrict__ part, int P, int D, int K,
                                                         float* __restrict__ dw, float* __restrict__ dbias) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)D * (K + 1)) return;
  float v = 0.0f;
  for (int p0 = 0; p0 < P; p0 += 8) {  // 8 loads in flight, summed in group order
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = p0 + j < P ? part[(int64_t)(p0 + j) * D * (K + 1) + i] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (p0 + j < P) v += q[j];
  }
  const int d = (int)(i / (K + 1)), k = (int)(i % (K + 1));
  if (k < K) dw[(int64_t)d * K + k] = v;
  else if (dbias) dbias[d] = v;
}

// x[t .. t+3] of a row through a buffer resource over the row: vectors
// before the row start or past its end read 0 (no branch, so the loads of a
// window issue back to back). t is a multiple of 4 and L % 4 == 0.
template <typename T>
__device__ __forceinline__ void buf_load4(__amdgpu_buffer_rsrc_t r, int64_t t, int64_t L, float* v) {
  const uint32_t off = (t >= 0 && t < L) ? (uint32_t)(t * (int64_t)sizeof(T)) : kBufOOB;
  if constexpr (sizeof(T) == 4) {
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(q[i]);
  } else {
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    const T* e = reinterpret_cast<const T*>(&q);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = to_f(e[i]);
  }
}

// ---------------------------------------------- backward from the events
// The conv evaluated only at the events (x_events of the fused fill), so its
// gradient arrives as du [E], one value per event. g = du * silu'(pre) lives
// at the events only, and the kernel writes the dense dx row straight from
// it: one wave per row, in windows of kCbWin steps taken from the row's end
// backward. Pass 1 gives every step of the window its g (0 between events;
// pre recomputed from x, the event found from the tile mask and the tile
// table) in LDS and accumulates the lane's dw / dbias terms; pass 2 forms
// dx[t] = sum_k w[k] g[t+(K-1)-k] from LDS, the K-1 slots past the window
// holding the first g of the window after it. dx has x's row strides.
constexpr int kCbWin = 1024;  // steps per window (4 per lane and 256-step segment)

template <typename T, bool SILU, int KM>
__global__ __launch_bounds__(256) void k_conv_bwd_events(
    const T* __restrict__ x, int64_t sb, int64_t sd, int dim, int64_t L, const float* __restrict__ w,
    const float* __restrict__ bias, int K_, const T* __restrict__ du, int64_t n_events,
    const uint32_t* __restrict__ bitmask, int64_t W, int64_t mrd, const int32_t* __restrict__ ts, int64_t nT,
    T* __restrict__ dx, float* __restrict__ part, int64_t rows) {
  const int K = KM == 4 ? 4 : K_;
  constexpr int PRE = (KM - 1 + 3) / 4 * 4;  // halo steps before t0, whole vectors
  __shared__ float s_g[4][kCbWin + kConvMaxK];
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= rows) return;  // no workgroup barrier below
  const int64_t b = row / dim;
  const int d = (int)(row % dim);
  const T* xr = x + b * sb + (int64_t)d * sd;
  T* dr = dx + b * sb + (int64_t)d * sd;
  const uint32_t* mrow = bitmask + (row / mrd) * W;
  const int32_t* tsr = ts + row * (nT + 1);
  float wk[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) wk[k] = k < K ? w[(int64_t)d * K + k] : 0.0f;
  const float b0 = bias ? bias[d] : 0.0f;
  const __amdgpu_buffer_rsrc_t rdu = buf_rsrc(du, n_events * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xr, L * (int64_t)sizeof(T));
  float* sg = s_g[wave];
  float aw[KM], ab = 0.0f;
#pragma unroll
  for (int k = 0; k < KM; ++k) aw[k] = 0.0f;
  if (lane < KM) sg[kCbWin + lane] = 0.0f;  // g past the row's end
  wave_sync();
  constexpr int SEGS = kCbWin / (4 * kWave);
  for (int64_t w0 = (L - 1) / kCbWin * kCbWin; w0 >= 0; w0 -= kCbWin) {
    // pass 1: g at the lane's 4 steps of each segment. Two rounds of loads
    // per window: x, masks and table entries of all segments, then the
    // events' du; lanes past L (L % 4 == 0: whole vectors) get g = 0
    float xv[SEGS][PRE + 4];  // xv[q][i] = x[t0-PRE+i]
    uint64_t m[SEGS];
    int32_t tv[SEGS];
#pragma unroll
    for (int q = 0; q < SEGS; ++q) {
      const int64_t t0 = w0 + 4 * kWave * q + 4 * lane;
#pragma unroll
      for (int v = 0; v < PRE / 4 + 1; ++v) buf_load4<T>(rx, t0 - PRE + 4 * v, L, xv[q] + 4 * v);
      const int64_t tl = (t0 < L ? t0 : 0) / kTile;
      m[q] = tile_mask(mrow, tl);
      tv[q] = tsr[tl];
    }
    float dv[SEGS][4];
    uint32_t nib[SEGS];
#pragma unroll
    for (int q = 0; q < SEGS; ++q) {
      const int64_t t0 = w0 + 4 * kWave * q + 4 * lane;
      const int off = (int)(t0 % kTile);
      nib[q] = t0 < L ? (uint32_t)(m[q] >> off) & 0xFu : 0u;
      uint32_t e = (uint32_t)tv[q] + (uint32_t)__popcll(m[q] & ((1ull << off) - 1ull));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t bit = (nib[q] >> k) & 1u;
        dv[q][k] = buf_load<T>(rdu, bit ? e * (uint32_t)sizeof(T) : kBufOOB);
        e += bit;
      }
    }
#pragma unroll
    for (int q = 0; q < SEGS; ++q) {
      const int lt = 4 * kWave * q + 4 * lane;
      float g[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float pre = b0;
#pragma unroll
        for (int j = 0; j < KM; ++j)
          if (j < K) pre = fmaf(wk[j], xv[q][PRE + k - (K - 1) + j], pre);
        float gv = dv[q][k];
        if (SILU) {
          const float sgm = 1.0f / (1.0f + __expf(-pre));
          gv = dv[q][k] * sgm * fmaf(pre, 1.0f - sgm, 1.0f);  // as k_conv_bwd: one rounding
        }
        g[k] = ((nib[q] >> k) & 1u) ? gv : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int j = 0; j < KM; ++j)
          if (j < K) aw[j] = fmaf(g[k], xv[q][PRE + k - (K - 1) + j], aw[j]);
        ab += g[k];
        sg[lt + k] = g[k];
      }
    }
    wave_sync();
#pragma unroll
    for (int q = 0; q < SEGS; ++q) {  // pass 2: dx at the lane's 4 steps
      const int lt = 4 * kWave * q + 4 * lane;
      const int64_t t0 = w0 + lt;
      if (t0 < L) {
        float gg[4 + KM - 1];  // g[t0 .. t0+3+KM-1]; slots past the window carry the next window's first g
#pragma unroll
        for (int i = 0; i < 4 + KM - 1; ++i) gg[i] = sg[lt + i];
        float o[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k < KM; ++k)
            if (k < K) acc = fmaf(wk[k], gg[s + (K - 1) - k], acc);
          o[s] = acc;
        }
        store4<T, true>(dr, t0, L, o);
      }
    }
    wave_sync();
    const float carry = lane < KM ? sg[lane] : 0.0f;  // this window's first g, for the window before it
    wave_sync();
    if (lane < KM) sg[kCbWin + lane] = carry;
    wave_sync();
  }
  // the row's dw / dbias terms: butterfly over the wave (fixed order)
#pragma unroll
  for (int k = 0; k <= KM; ++k) {
    float v = k < KM ? aw[k] : ab;
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    if (lane == 0 && (k < K || k == KM)) part[row * (K + 1) + (k < KM ? k : K)] = v;
  }
}

// dw / dbias from the rows' terms: channel d sums rows d, d + dim, ... in order.
__global__ __launch_bounds__(256) void k_conv_bwd_events_reduce(const float* __restrict__ part, int64_t nb, int dim,
                                                                int K, float* __restrict__ dw,
                                                                float* __restrict__ dbias) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)dim * (K + 1)) return;
  const int d = (int)(i / (K + 1)), k = (int)(i % (K + 1));
  float v = 0.0f;
  const int64_t stride = (int64_t)dim * (K + 1);
  const float* pr = part + (int64_t)d * (K + 1) + k;
  for (int64_t b0 = 0; b0 < nb; b0 += 8) {  // 8 loads in flight, summed in row order
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = b0 + j < nb ? pr[(b0 + j) * stride] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (b0 + j < nb) v += q[j];
  }
  if (k < K) dw[(int64_t)d * K + k] = v;
  else if (dbias) dbias[d] = v;
}

// Batch groups of the backward: enough workgroups to fill the chip.
inline int conv_split(int64_t B, int64_t D) {
  const int64_t want = (8 * (int64_t)device_cus() + D - 1) / D;
  return (int)std::max<int64_t>(1, std::min<int64_t>({B, want, (int64_t)kConvMaxSplit}));
}

static int conv_checks(const char* fn, int dtype, int64_t B, int64_t D, int64_t L, int K) {
  if (!dtype_ok(dtype)) return set_error(BCM_EINVAL, "%s: x must be fp32/fp16/bf16", fn);
  if (B < 0 || D < 1 || L < 0) return set_error(BCM_EINVAL, "%s: bad shape", fn);
  if (K < 1 || K > kConvMaxK) return set_error(BCM_EINVAL, "%s: kernel width must be in [1, %d]", fn, kConvMaxK);
  if (D > INT32_MAX || B > INT32_MAX) return set_error(BCM_EINVAL, "%s: too many rows", fn);
  return BCM_OK;
}

}  // namespace bcm

extern "C" {

int bcm_causal_conv1d_fwd(const void* x, int dtype, const float* weight, const float* bias, int64_t B, int64_t D,
                          int64_t L, int K, int silu, void* out, bcm_stream_t stream) {
  const char* fn = "bcm_causal_conv1d_fwd";
  int rc = bcm::conv_checks(fn, dtype, B, D, L, K);
  if (rc) return rc;
  if (B == 0 || L == 0) return BCM_OK;
  if (!x || !weight || !out) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  const int64_t rows = B * D, chunks = (L + bcm::kConvSteps - 1) / bcm::kConvSteps;
  const int64_t n = rows * chunks;
  const dim3 grid((unsigned)((n + 255) / 256));
  const bool vec = L % 4 == 0 && bcm::aligned16(x) && bcm::aligned16(out);
  bcm::dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto s_, auto v_) {
      constexpr bool S = decltype(s_)::value, V = decltype(v_)::value;
      if (K == 4)
        hipLaunchKernelGGL((bcm::k_conv_fwd<T, S, V, 4>), grid, dim3(256), 0, bcm::hs(stream),
                           static_cast<const T*>(x), weight, bias, static_cast<T*>(out), rows, (int)D, L, K, chunks);
      else
        hipLaunchKernelGGL((bcm::k_conv_fwd<T, S, V, 8>), grid, dim3(256), 0, bcm::hs(stream),
                           static_cast<const T*>(x), weight, bias, static_cast<T*>(out), rows, (int)D, L, K, chunks);
    };
    if (silu) {
      if (vec) go(std::true_type{}, std::true_type{});
      else go(std::true_type{}, std::false_type{});
    } else {
      if (vec) go(std::false_type{}, std::true_type{});
      else go(std::false_type{}, std::false_type{});
    }
  });
  return bcm::check_launch(fn);
}

int64_t bcm_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K) {
  (void)L;
  if (B < 1 || D < 1 || K < 1 || K > bcm::kConvMaxK) return 0;
  const int P = bcm::conv_split(B, D);
  return P > 1 ? 4 * (int64_t)P * D * (K + 1) : 0;
}

int bcm_causal_conv1d_bwd(const void* x, int dtype, const float* weight, const float* bias, const void* dout,
                          int64_t B, int64_t D, int64_t L, int K, int silu, void* dx, float* dweight, float* dbias,
                          void* workspace, int64_t workspace_bytes, bcm_stream_t stream) {
  const char* fn = "bcm_causal_conv1d_bwd";
  int rc = bcm::conv_checks(fn, dtype, B, D, L, K);
  if (rc) return rc;
  if (!weight || !dweight) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (B > 0 && L > 0 && (!x || !dout || !dx)) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  int P = B > 0 ? bcm::conv_split(B, D) : 1;
  if (P > 1 && (!workspace || workspace_bytes < 4 * (int64_t)P * D * (K + 1))) P = 1;  // no room: one group
  const bool vec = L % 4 == 0 && bcm::aligned16(x) && bcm::aligned16(dout) && bcm::aligned16(dx);
  float* part = static_cast<float*>(workspace);
  bcm::dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto s_, auto v_) {
      constexpr bool S = decltype(s_)::value, V = decltype(v_)::value;
      const dim3 grid((unsigned)D, (unsigned)P);
      if (K == 4)
        hipLaunchKernelGGL((bcm::k_conv_bwd<T, S, V, 4>), grid, dim3(256), 0, bcm::hs(stream),
                           static_cast<const T*>(x), weight, bias, static_cast<const T*>(dout), static_cast<T*>(dx),
                           dweight, dbias, part, (int)B, (int)D, L, K);
      else
        hipLaunchKernelGGL((bcm::k_conv_bwd<T, S, V, 8>), grid, dim3(256), 0, bcm::hs(stream),
                           static_cast<const T*>(x), weight, bias, static_cast<const T*>(dout), static_cast<T*>(dx),
                           dweight, dbias, part, (int)B, (int)D, L, K);
    };
    if (silu) {
      if (vec) go(std::true_type{}, std::true_type{});
      else go(std::true_type{}, std::false_type{});
    } else {
      if (vec) go(std::false_type{}, std::true_type{});
      else go(std::false_type{}, std::false_type{});
    }
  });
  rc = bcm::check_launch(fn);
  if (rc || P == 1) return rc;
  const int64_t n = D * (K + 1);
  hipLaunchKernelGGL(bcm::k_conv_bwd_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, bcm::hs(stream), part,
                     P, (int)D, K, dweight, dbias);
  return bcm::check_launch(fn);
}

int64_t bcm_causal_conv1d_bwd_events_workspace_bytes(int64_t B, int64_t D, int K) {
  if (B < 1 || D < 1 || K < 1 || K > bcm::kConvMaxK) return 0;
  return 4 * B * D * (K + 1);
}

int bcm_causal_conv1d_bwd_events(const void* x, int dtype, int64_t x_batch_stride, int64_t x_dim_stride, int64_t B,
                                 int64_t D, int64_t L, const float* weight, const float* bias, int K, int silu,
                                 const void* du, int64_t n_events, const uint32_t* bitmask, int64_t mask_row_div,
                                 const int32_t* tile_start, void* dx, float* dweight, float* dbias, void* workspace,
                                 int64_t workspace_bytes, bcm_stream_t stream) {
  const char* fn = "bcm_causal_conv1d_bwd_events";
  int rc = bcm::conv_checks(fn, dtype, B, D, L, K);
  if (rc) return rc;
  if (!weight || !dweight) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (B == 0 || L == 0) {  // no rows: the weight gradients are zero
    rc = bcm_zero(dweight, 4 * D * K, stream);
    if (!rc && dbias) rc = bcm_zero(dbias, 4 * D, stream);
    return rc;
  }
  if (!x || !dx || !bitmask || !tile_start || (n_events > 0 && !du))
    return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (n_events < 0 || n_events * 4 > INT32_MAX) return bcm::set_error(BCM_EINVAL, "%s: n_events out of range", fn);
  if (mask_row_div < 1) return bcm::set_error(BCM_EINVAL, "%s: mask_row_div must be >= 1", fn);
  const size_t es = bcm::dtype_size(dtype);
  const uintptr_t va = 4 * es;  // one 4-step vector
  if (L % 4 || x_batch_stride % 4 || x_dim_stride % 4 || x_batch_stride < 0 || x_dim_stride < 0 ||
      reinterpret_cast<uintptr_t>(x) % va || reinterpret_cast<uintptr_t>(dx) % va)
    return bcm::set_error(BCM_EINVAL, "%s: needs L and the row strides multiples of 4 and x, dx aligned to 4 elements",
                          fn);
  if ((reinterpret_cast<uintptr_t>(bitmask) & 7) != 0)
    return bcm::set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  {  // dx is written through the same strides: rows must not overlap
    const bool dim_inner = x_dim_stride <= x_batch_stride;
    const int64_t s_in = dim_inner ? x_dim_stride : x_batch_stride, n_in = dim_inner ? D : B;
    const int64_t s_out = dim_inner ? x_batch_stride : x_dim_stride, n_out = dim_inner ? B : D;
    if ((n_in > 1 && s_in < L) || (n_out > 1 && s_out < s_in * n_in))
      return bcm::set_error(BCM_EINVAL, "%s: the row strides make rows overlap", fn);
  }
  const int64_t rows = B * D;
  if (!workspace || workspace_bytes < 4 * rows * (K + 1))
    return bcm::set_error(BCM_EINVAL, "%s: workspace needs %lld bytes", fn, (long long)(4 * rows * (K + 1)));
  const int64_t W = bcm::bitmask_words(L), nT = bcm::tile_count(L);
  float* part = static_cast<float*>(workspace);
  const dim3 grid((unsigned)((rows + 3) / 4));
  bcm::dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto s_, auto km) {
      constexpr bool S = decltype(s_)::value;
      constexpr int KM = decltype(km)::value;
      hipLaunchKernelGGL((bcm::k_conv_bwd_events<T, S, KM>), grid, dim3(256), 0, bcm::hs(stream),
                         static_cast<const T*>(x), x_batch_stride, x_dim_stride, (int)D, L, weight, bias, K,
                         static_cast<const T*>(du), n_events, bitmask, W, mask_row_div, tile_start, nT,
                         static_cast<T*>(dx), part, rows);
    };
    using K4 = std::integral_constant<int, 4>;
    using K8 = std::integral_constant<int, 8>;
    if (silu) {
      if (K == 4) go(std::true_type{}, K4{});
      else go(std::true_type{}, K8{});
    } else {
      if (K == 4) go(std::false_type{}, K4{});
      else go(std::false_type{}, K8{});
    }
  });
  rc = bcm::check_launch(fn);
  if (rc) return rc;
  const int64_t n = D * (K + 1);
  hipLaunchKernelGGL(bcm::k_conv_bwd_events_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     bcm::hs(stream), part, B, (int)D, K, dweight, dbias);
  return bcm::check_launch(fn);
}

}  // extern "C"
