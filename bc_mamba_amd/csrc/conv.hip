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
// MI355X design: rows (b, d) of L steps are contiguous. The forward gives
// each thread 4 consecutive steps of one row (the K-1 halo values come from
// the neighbouring lanes' lines in L1), so a wave covers 256 contiguous
// steps. The backward runs one workgroup per channel d over its B rows: g is
// recomputed from x (no saved pre-activation), dx is written per row, and
// dw / dbias accumulate in registers and reduce in LDS in a fixed order
// (deterministic, no atomics, no workspace). HBM-bound: x and dout read
// once, out / dx written once.
#include "bcm_common.hpp"

namespace bcm {

constexpr int kConvMaxK = 8;
constexpr int kConvSteps = 4;  // consecutive steps per thread

template <typename T, bool SILU>
__global__ __launch_bounds__(256) void k_conv_fwd(const T* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ bias, T* __restrict__ out, int64_t rows,
                                                  int D, int64_t L, int K, int64_t chunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * chunks) return;
  const int64_t row = gid / chunks;
  const int64_t t0 = (gid - row * chunks) * kConvSteps;
  const int d = (int)(row % D);
  const T* xr = x + row * L;
  float wk[kConvMaxK];
#pragma unroll
  for (int k = 0; k < kConvMaxK; ++k) wk[k] = k < K ? w[(int64_t)d * K + k] : 0.0f;
  const float b0 = bias ? bias[d] : 0.0f;
  // window x[t0-(K-1) .. t0+3]
  float xv[kConvMaxK - 1 + kConvSteps];
#pragma unroll
  for (int i = 0; i < kConvMaxK - 1 + kConvSteps; ++i) {
    const int64_t t = t0 - (K - 1) + i;
    xv[i] = (i < K - 1 + kConvSteps && t >= 0 && t < L) ? to_f(xr[t]) : 0.0f;
  }
  T* orow = out + row * L;
#pragma unroll
  for (int s = 0; s < kConvSteps; ++s) {
    if (t0 + s >= L) break;
    float pre = b0;
#pragma unroll
    for (int k = 0; k < kConvMaxK; ++k)
      if (k < K) pre = fmaf(wk[k], xv[s + k], pre);
    const float v = SILU ? pre / (1.0f + __expf(-pre)) : pre;
    orow[t0 + s] = from_f<T>(v);
  }
}

template <typename T, bool SILU>
__global__ __launch_bounds__(256) void k_conv_bwd(const T* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ bias, const T* __restrict__ dout,
                                                  T* __restrict__ dx, float* __restrict__ dw,
                                                  float* __restrict__ dbias, int B, int D, int64_t L, int K) {
  __shared__ float s_red[kConvMaxK + 1][256 / kWave];
  const int d = blockIdx.x;
  float wk[kConvMaxK];
#pragma unroll
  for (int k = 0; k < kConvMaxK; ++k) wk[k] = k < K ? w[(int64_t)d * K + k] : 0.0f;
  const float b0 = bias ? bias[d] : 0.0f;
  float aw[kConvMaxK], ab = 0.0f;  // this thread's dw / dbias partials
#pragma unroll
  for (int k = 0; k < kConvMaxK; ++k) aw[k] = 0.0f;
  // g at steps t0 .. t0+3+(K-1) needs x at t0-(K-1) .. t0+3+(K-1)
  constexpr int NG = kConvSteps + kConvMaxK - 1;
  constexpr int NX = NG + kConvMaxK - 1;
  for (int b = 0; b < B; ++b) {
    const int64_t row = (int64_t)b * D + d;
    const T* xr = x + row * L;
    const T* gr = dout + row * L;
    T* dxr = dx + row * L;
    for (int64_t t0 = (int64_t)threadIdx.x * kConvSteps; t0 < L; t0 += (int64_t)blockDim.x * kConvSteps) {
      float xv[NX];
#pragma unroll
      for (int i = 0; i < NX; ++i) {
        const int64_t t = t0 - (K - 1) + i;
        xv[i] = (i < NG + K - 1 && t >= 0 && t < L) ? to_f(xr[t]) : 0.0f;
      }
      float g[NG];
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const int64_t t = t0 + i;
        float v = 0.0f;
        if (i < kConvSteps + K - 1 && t < L) {
          float pre = b0;
#pragma unroll
          for (int k = 0; k < kConvMaxK; ++k)
            if (k < K) pre = fmaf(wk[k], xv[i + k], pre);
          const float go = to_f(gr[t]);
          if (SILU) {
            const float sg = 1.0f / (1.0f + __expf(-pre));
            v = go * sg * (1.0f + pre * (1.0f - sg));
          } else {
            v = go;
          }
        }
        g[i] = v;
      }
#pragma unroll
      for (int s = 0; s < kConvSteps; ++s) {
        if (t0 + s >= L) break;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kConvMaxK; ++k)
          if (k < K) acc = fmaf(wk[k], g[s + (K - 1) - k], acc);
        dxr[t0 + s] = from_f<T>(acc);
        // dw[k] += g[t] x[t-(K-1)+k] over this thread's own steps
#pragma unroll
        for (int k = 0; k < kConvMaxK; ++k)
          if (k < K) aw[k] = fmaf(g[s], xv[s + k], aw[k]);
        ab += g[s];
      }
    }
  }
  // fixed-order reduction: waves by DPP-free shuffles, then the 4 wave sums in order
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
    if (k < K) dw[(int64_t)d * K + k] = v;
    else if (k == kConvMaxK && dbias) dbias[d] = v;
  }
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
  bcm::dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (silu)
      hipLaunchKernelGGL((bcm::k_conv_fwd<T, true>), grid, dim3(256), 0, bcm::hs(stream), static_cast<const T*>(x),
                         weight, bias, static_cast<T*>(out), rows, (int)D, L, K, chunks);
    else
      hipLaunchKernelGGL((bcm::k_conv_fwd<T, false>), grid, dim3(256), 0, bcm::hs(stream), static_cast<const T*>(x),
                         weight, bias, static_cast<T*>(out), rows, (int)D, L, K, chunks);
  });
  return bcm::check_launch(fn);
}

int bcm_causal_conv1d_bwd(const void* x, int dtype, const float* weight, const float* bias, const void* dout,
                          int64_t B, int64_t D, int64_t L, int K, int silu, void* dx, float* dweight, float* dbias,
                          bcm_stream_t stream) {
  const char* fn = "bcm_causal_conv1d_bwd";
  int rc = bcm::conv_checks(fn, dtype, B, D, L, K);
  if (rc) return rc;
  if (!weight || !dweight) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  if (B > 0 && L > 0 && (!x || !dout || !dx)) return bcm::set_error(BCM_EINVAL, "%s: null pointer", fn);
  bcm::dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (silu)
      hipLaunchKernelGGL((bcm::k_conv_bwd<T, true>), dim3((unsigned)D), dim3(256), 0, bcm::hs(stream),
                         static_cast<const T*>(x), weight, bias, static_cast<const T*>(dout), static_cast<T*>(dx),
                         dweight, dbias, (int)B, (int)D, L, K);
    else
      hipLaunchKernelGGL((bcm::k_conv_bwd<T, false>), dim3((unsigned)D), dim3(256), 0, bcm::hs(stream),
                         static_cast<const T*>(x), weight, bias, static_cast<const T*>(dout), static_cast<T*>(dx),
                         dweight, dbias, (int)B, (int)D, L, K);
  });
  return bcm::check_launch(fn);
}

}  // extern "C"
