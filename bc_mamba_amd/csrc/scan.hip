// Stage 2: flat per-channel selective scan over packed events, forward and
// backward, depthwise B/C mode.
//
// Reference behaviour: csrc/selective_scan/selective_scan_fwd_kernel.cuh
// :403-728 (forward), selective_scan_bwd_kernel.cuh:635-1169 (backward),
// selective_scan_common.h:43-52 (exponent clamp), :156-190 (scan operator
// (a0,b0)∘(a1,b1) = (a1·a0, a1·b0 + b1) and the running prefix).
//
// MI355X design
//   * One workgroup per model channel d = ch % dim; its waves take the
//     channels ch = d + b·dim for all b. The per-d parameters live in LDS and
//     the parameter gradients (dA, dW_B, dW_C, ddt_*, dD) are reduced inside
//     the workgroup in a fixed order: no atomics, no zero-init, bit-stable.
//   * A channel's events are split into chunks of C = G·R events; each of the
//     G lanes of a lane group owns R consecutive events (items) in registers.
//     u, k and dout are staged through LDS with coalesced loads and read back
//     with an odd lane stride (R+1) so the transposed reads are conflict-free.
//   * The state loop is outermost: per state s every lane computes its R
//     decays a = exp2(clamp(Δ·A·log2e)), folds its items into a local
//     (prod a, h) pair, the G lanes combine the pairs with an inclusive scan
//     (wave shuffles), and a second register pass produces the exact states.
//     y (forward) and du / dΔ (backward) accumulate per item across states in
//     registers, so no per-event cross-lane reduction is needed.
//   * Chunks longer than one workgroup pass (max_seqlen > 2048 uses C = 2048,
//     the reference's chunk) carry (prod a, h) forward in LDS; the backward
//     starts each chunk from the saved state x[ch, c-1] like the reference and
//     carries a·dx backward in LDS.
//   * No MFMA: the work is a first-order recurrence, not a contraction.
#include "bcm_common.hpp"

#include <climits>

namespace bcm {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kScanThreads = 512;  // workgroup size bound (8 waves)

struct FwdLds {
  int N, nw, G, R, nslots;
  int64_t bytes() const {
    return 4ll * (3ll * N + (int64_t)nw * kWave * (R + 1) + (int64_t)nslots * 2 * N);
  }
};

struct BwdLds {
  int N, nw, G, R, nslots;
  int64_t bytes() const {
    return 4ll * (4ll * N + 2ll * nw * kWave * (R + 1) + (int64_t)nslots * N + (int64_t)nslots * (3 * N + 3));
  }
};

// Position of chunk item idx in a lane-transposed LDS tile (stride R+1).
template <int R> __device__ __forceinline__ int tpos(int idx) { return (idx / R) * (R + 1) + (idx % R); }

template <int G, int R, typename T, bool HAS_Z>
__global__ __launch_bounds__(kScanThreads) void k_scan_fwd(const bcm_scan_args a) {
  constexpr int CPW = kWave / G;
  constexpr int RS = R + 1;
  constexpr int C = G * R;
  const int N = a.dstate;
  const int d = blockIdx.x;
  const int nw = blockDim.x / kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / G, j = lane % G;
  const int nslots = nw * CPW;
  const int slot = wave * CPW + grp;

  extern __shared__ float smem[];
  float* sAl = smem;
  float* sWB = sAl + N;
  float* sWC = sWB + N;
  float* gst = sWC + N + wave * (kWave * RS) + grp * (G * RS);
  float* carry = smem + 3 * N + nw * kWave * RS + slot * 2 * N;  // [P_run(N), h_run(N)]

  for (int s = threadIdx.x; s < N; s += blockDim.x) {
    sAl[s] = a.A[(int64_t)d * N + s] * kLog2e;
    sWB[s] = a.W_B[(int64_t)d * N + s];
    sWC[s] = a.W_C[(int64_t)d * N + s];
  }
  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  __syncthreads();

  const T* __restrict__ u = static_cast<const T*>(a.u);
  const T* __restrict__ z = static_cast<const T*>(a.z);
  T* __restrict__ out = static_cast<T*>(a.out);
  T* __restrict__ out_z = static_cast<T*>(a.out_z);
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;

  for (int b0 = 0; b0 < n_per_d; b0 += nslots) {
    const int b = b0 + slot;
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    const int e0 = act ? a.cu_seqlens[ch] : 0;
    const int n = act ? a.cu_seqlens[ch + 1] - e0 : 0;
    const int nch = n > 0 ? (n + C - 1) / C : 0;
    const int wmax = wave_max(nch);
    for (int c = 0; c < wmax; ++c) {
      const int cnt = min(max(n - c * C, 0), C);
      const int64_t eb = (int64_t)e0 + (int64_t)c * C;
      // ---- stage u and k through LDS (coalesced global reads)
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        gst[tpos<R>(idx)] = idx < cnt ? to_f(u[eb + idx]) : 0.0f;
      }
      wave_sync();
      float uu[R];
#pragma unroll
      for (int r = 0; r < R; ++r) uu[r] = gst[j * RS + r];
      wave_sync();
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        gst[tpos<R>(idx)] = __int_as_float(idx < cnt ? a.k[eb + idx] : 1);
      }
      wave_sync();
      float dl[R], du2[R], acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int kk = __float_as_int(gst[j * RS + r]);
        // padding items are identities of the scan: Δ = 0 -> a = 1, b = 0
        dl[r] = (j * R + r < cnt) ? fmaf(dti, (float)(kk - 1), dta) : 0.0f;
        du2[r] = dl[r] * uu[r] * uu[r];
        acc[r] = 0.0f;
      }
      wave_sync();
      // ---- state loop
      for (int s = 0; s < N; ++s) {
        const float Al = sAl[s], wb = sWB[s], wc = sWC[s];
        float av[R];
        float P = 1.0f, H = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          av[r] = decay(dl[r] * Al);
          H = fmaf(av[r], H, du2[r] * wb);
          P *= av[r];
        }
#pragma unroll
        for (int o = 1; o < G; o <<= 1) {
          const float Pp = __shfl_up(P, o, G);
          const float Hp = __shfl_up(H, o, G);
          if (j >= o) {
            H = fmaf(P, Hp, H);
            P *= Pp;
          }
        }
        const float h0 = c > 0 ? carry[N + s] : 0.0f;
        const float P0 = c > 0 ? carry[s] : 1.0f;
        const float hend = fmaf(P, h0, H);
        float h = __shfl_up(hend, 1, G);
        if (j == 0) h = h0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          h = fmaf(av[r], h, du2[r] * wb);
          acc[r] = fmaf(h, wc, acc[r]);
        }
        if (j == G - 1 && c < nch) {
          const float Pn = P0 * P;
          carry[s] = Pn;
          carry[N + s] = hend;
          if (c < nck) reinterpret_cast<float2*>(a.x + (ch * nck + c) * 2 * N)[s] = make_float2(Pn, hend);
        }
      }
      // ---- outputs: y = D·u + u·Σ_s h·W_C, staged for a coalesced store
#pragma unroll
      for (int r = 0; r < R; ++r) gst[j * RS + r] = fmaf(Dv, uu[r], uu[r] * acc[r]);
      wave_sync();
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        if (idx < cnt) {
          const float yv = gst[tpos<R>(idx)];
          out[eb + idx] = from_f<T>(yv);
          if (HAS_Z) {
            const float zv = to_f(z[eb + idx]);
            out_z[eb + idx] = from_f<T>(yv * (zv / (1.0f + __expf(-zv))));
          }
        }
      }
      wave_sync();
    }
    // chunks past the channel's end keep the reference's zero state
    if (act) {
      for (int c = nch; c < nck; ++c)
        for (int s = j; s < 2 * N; s += G) a.x[(ch * nck + c) * 2 * N + s] = 0.0f;
    }
  }
}

template <int G, int R, typename T, bool HAS_Z>
__global__ __launch_bounds__(kScanThreads) void k_scan_bwd(const bcm_scan_args a) {
  constexpr int CPW = kWave / G;
  constexpr int RS = R + 1;
  constexpr int C = G * R;
  const int N = a.dstate;
  const int d = blockIdx.x;
  const int nw = blockDim.x / kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / G, j = lane % G;
  const int nslots = nw * CPW;
  const int slot = wave * CPW + grp;
  const int NA = 3 * N + 3;  // accumulators per slot: dA, dW_B, dW_C, ddt_idle, ddt_active, dD

  extern __shared__ float smem[];
  float* sA = smem;
  float* sAl = sA + N;
  float* sWB = sAl + N;
  float* sWC = sWB + N;
  float* wbase = sWC + N + wave * (2 * kWave * RS);
  float* gdt = wbase + grp * (G * RS);            // gated dout, kept for the chunk
  float* gkm = wbase + kWave * RS + grp * (G * RS);  // staging, then k-1 kept for the chunk
  float* sdx = smem + 4 * N + nw * 2 * kWave * RS;   // [nslots][N] a·dx carried to the previous chunk
  float* sacc = sdx + nslots * N;                    // [nslots][NA]
  float* cdx = sdx + slot * N;
  float* cacc = sacc + slot * NA;

  for (int s = threadIdx.x; s < N; s += blockDim.x) {
    const float Av = a.A[(int64_t)d * N + s];
    sA[s] = Av;
    sAl[s] = Av * kLog2e;
    sWB[s] = a.W_B[(int64_t)d * N + s];
    sWC[s] = a.W_C[(int64_t)d * N + s];
  }
  for (int i = threadIdx.x; i < nslots * NA; i += blockDim.x) sacc[i] = 0.0f;
  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  __syncthreads();

  const T* __restrict__ u = static_cast<const T*>(a.u);
  const T* __restrict__ dout = static_cast<const T*>(a.dout);
  const T* __restrict__ z = static_cast<const T*>(a.z);
  const T* __restrict__ outs = static_cast<const T*>(a.out_saved);
  T* __restrict__ du_o = static_cast<T*>(a.du);
  T* __restrict__ dz_o = static_cast<T*>(a.dz);
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;

  for (int b0 = 0; b0 < n_per_d; b0 += nslots) {
    const int b = b0 + slot;
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    const int e0 = act ? a.cu_seqlens[ch] : 0;
    const int n = act ? a.cu_seqlens[ch + 1] - e0 : 0;
    const int nch = n > 0 ? (n + C - 1) / C : 0;
    const int wmax = wave_max(nch);
    float ddti_l = 0.0f, ddta_l = 0.0f, dD_l = 0.0f;
    for (int c = wmax - 1; c >= 0; --c) {
      const bool cact = c < nch;
      const int cnt = min(max(n - c * C, 0), C);
      const int64_t eb = (int64_t)e0 + (int64_t)c * C;
      // ---- stage u
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        gkm[tpos<R>(idx)] = idx < cnt ? to_f(u[eb + idx]) : 0.0f;
      }
      wave_sync();
      float uu[R];
#pragma unroll
      for (int r = 0; r < R; ++r) uu[r] = gkm[j * RS + r];
      wave_sync();
      // ---- stage k-1 (kept) and the gated dout (kept); dz on the way
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        const int p = tpos<R>(idx);
        float km1 = 0.0f, dv = 0.0f;
        if (idx < cnt) {
          km1 = (float)(a.k[eb + idx] - 1);
          dv = to_f(dout[eb + idx]);
          if (HAS_Z) {
            const float zv = to_f(z[eb + idx]);
            const float ov = to_f(outs[eb + idx]);
            const float sg = 1.0f / (1.0f + __expf(-zv));
            dz_o[eb + idx] = from_f<T>(dv * ov * sg * (1.0f + zv * (1.0f - sg)));
            dv *= zv * sg;
          }
        }
        gkm[p] = km1;
        gdt[p] = dv;
      }
      wave_sync();
      float dl[R], du2[R], doutu[R], acc1[R], acc2[R], acc3[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool valid = j * R + r < cnt;
        dl[r] = valid ? fmaf(dti, gkm[j * RS + r], dta) : 0.0f;
        du2[r] = dl[r] * uu[r] * uu[r];
        doutu[r] = gdt[j * RS + r] * uu[r];
        acc1[r] = 0.0f;
        acc2[r] = 0.0f;
        acc3[r] = 0.0f;
      }
      // ---- state loop
      for (int s = 0; s < N; ++s) {
        const float Ar = sA[s], Al = sAl[s], wb = sWB[s], wc = sWC[s];
        const float h0 = (c > 0 && c - 1 < nck) ? a.x_saved[(ch * nck + (c - 1)) * 2 * N + 2 * s + 1] : 0.0f;
        const float dxc = (c < nch - 1) ? cdx[s] : 0.0f;
        float av[R], hh[R];
        // forward: local fold, group scan, exact states
        float P = 1.0f, H = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          av[r] = decay(dl[r] * Al);
          H = fmaf(av[r], H, du2[r] * wb);
          P *= av[r];
        }
#pragma unroll
        for (int o = 1; o < G; o <<= 1) {
          const float Pp = __shfl_up(P, o, G);
          const float Hp = __shfl_up(H, o, G);
          if (j >= o) {
            H = fmaf(P, Hp, H);
            P *= Pp;
          }
        }
        const float hend = fmaf(P, h0, H);
        float hin = __shfl_up(hend, 1, G);
        if (j == 0) hin = h0;
        {
          float h = hin;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            h = fmaf(av[r], h, du2[r] * wb);
            hh[r] = h;
          }
        }
        // reverse: dx_i = dout_i·u_i·W_C + a_{i+1}·dx_{i+1}
        float anext = __shfl_down(av[0], 1, G);
        if (j == G - 1) anext = 1.0f;  // the chunk carry already holds a_next·dx_next
        float Q = 1.0f, Cc = 0.0f;
#pragma unroll
        for (int r = R - 1; r >= 0; --r) {
          const float al = (r == R - 1) ? anext : av[r + 1];
          Cc = fmaf(al, Cc, doutu[r] * wc);
          Q *= al;
        }
#pragma unroll
        for (int o = 1; o < G; o <<= 1) {
          const float Qs = __shfl_down(Q, o, G);
          const float Cs = __shfl_down(Cc, o, G);
          if (j + o < G) {
            Cc = fmaf(Q, Cs, Cc);
            Q *= Qs;
          }
        }
        const float tfirst = fmaf(Q, dxc, Cc);
        float dx = __shfl_down(tfirst, 1, G);
        if (j == G - 1) dx = dxc;
        float dA_l = 0.0f, dWB_l = 0.0f, dWC_l = 0.0f;
#pragma unroll
        for (int r = R - 1; r >= 0; --r) {
          const float al = (r == R - 1) ? anext : av[r + 1];
          dx = fmaf(al, dx, doutu[r] * wc);
          acc1[r] = fmaf(dx, wb, acc1[r]);
          acc2[r] = fmaf(hh[r], wc, acc2[r]);
          const float hp = r > 0 ? hh[r - 1] : hin;
          const float t2 = dx * (av[r] * hp);
          acc3[r] = fmaf(t2, Ar, acc3[r]);
          dA_l = fmaf(t2, dl[r], dA_l);
          dWB_l = fmaf(dx, du2[r], dWB_l);
          dWC_l = fmaf(doutu[r], hh[r], dWC_l);
        }
        if (j == 0 && cact) cdx[s] = av[0] * dx;
        dA_l = group_sum<G>(dA_l);
        dWB_l = group_sum<G>(dWB_l);
        dWC_l = group_sum<G>(dWC_l);
        if (j == 0 && cact) {
          cacc[s] += dA_l;
          cacc[N + s] += dWB_l;
          cacc[2 * N + s] += dWC_l;
        }
      }
      // ---- per item: du, dΔ -> ddt, dD
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float dt = gdt[j * RS + r];
        const float km1 = gkm[j * RS + r];
        const float duv = fmaf(dt, Dv + acc2[r], 2.0f * dl[r] * uu[r] * acc1[r]);
        const float dd = fmaf(uu[r] * uu[r], acc1[r], acc3[r]);
        ddti_l = fmaf(dd, km1, ddti_l);
        ddta_l += dd;
        dD_l += doutu[r];
        gdt[j * RS + r] = duv;
      }
      wave_sync();
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int idx = q * G + j;
        if (idx < cnt) du_o[eb + idx] = from_f<T>(gdt[tpos<R>(idx)]);
      }
      wave_sync();
    }
    ddti_l = group_sum<G>(ddti_l);
    ddta_l = group_sum<G>(ddta_l);
    dD_l = group_sum<G>(dD_l);
    if (j == 0 && act) {
      cacc[3 * N] += ddti_l;
      cacc[3 * N + 1] += ddta_l;
      cacc[3 * N + 2] += dD_l;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NA; i += blockDim.x) {
    float v = 0.0f;
    for (int sl = 0; sl < nslots; ++sl) v += sacc[sl * NA + i];
    if (i < N) a.dA[(int64_t)d * N + i] = v;
    else if (i < 2 * N) a.dW_B[(int64_t)d * N + (i - N)] = v;
    else if (i < 3 * N) a.dW_C[(int64_t)d * N + (i - 2 * N)] = v;
    else if (i == 3 * N) a.ddt_idle[d] = v;
    else if (i == 3 * N + 1) a.ddt_active[d] = v;
    else if (a.dD) a.dD[d] = v;
  }
}

// ------------------------------------------------------------ host dispatch
static int max_lds_bytes() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) return 65536;
  return v;
}

template <int G, int R, typename T, bool Z, bool BWD>
static int launch(const bcm_scan_args& a, hipStream_t s, const char* fn) {
  constexpr int CPW = kWave / G;
  const int per_d = (a.n_channels + a.dim - 1) / a.dim;
  int nw = (per_d + CPW - 1) / CPW;
  nw = nw < 1 ? 1 : (nw > kScanThreads / kWave ? kScanThreads / kWave : nw);
  const int64_t cap = max_lds_bytes();
  int64_t lds = 0;
  for (;;) {
    lds = BWD ? BwdLds{a.dstate, nw, G, R, nw * CPW}.bytes() : FwdLds{a.dstate, nw, G, R, nw * CPW}.bytes();
    if (lds <= cap || nw == 1) break;
    --nw;
  }
  if (lds > cap) return set_error(BCM_EINVAL, "%s: dstate %d needs %lld bytes of LDS (> %lld)", fn, a.dstate,
                                  (long long)lds, (long long)cap);
  if (BWD)
    hipLaunchKernelGGL((k_scan_bwd<G, R, T, Z>), dim3(a.dim), dim3(nw * kWave), (size_t)lds, s, a);
  else
    hipLaunchKernelGGL((k_scan_fwd<G, R, T, Z>), dim3(a.dim), dim3(nw * kWave), (size_t)lds, s, a);
  return check_launch(fn);
}

template <typename T, bool Z, bool BWD>
static int dispatch_shape(const bcm_scan_args& a, hipStream_t s, const char* fn) {
  const int m = a.max_seqlen;
  if (a.dstate <= 64) {
    if (m <= 64) return launch<16, 4, T, Z, BWD>(a, s, fn);
    if (m <= 128) return launch<16, 8, T, Z, BWD>(a, s, fn);
    if (m <= 256) return launch<16, 16, T, Z, BWD>(a, s, fn);
    if (m <= 384) return launch<16, 24, T, Z, BWD>(a, s, fn);
    if (m <= 512) return launch<32, 16, T, Z, BWD>(a, s, fn);
  } else {
    if (m <= 256) return launch<64, 4, T, Z, BWD>(a, s, fn);
    if (m <= 512) return launch<64, 8, T, Z, BWD>(a, s, fn);
  }
  if (m <= 1024) return launch<64, 16, T, Z, BWD>(a, s, fn);
  return launch<64, 32, T, Z, BWD>(a, s, fn);
}

template <bool BWD>
static int scan_entry(const bcm_scan_args* ap, bcm_stream_t stream, const char* fn) {
  if (!ap) return set_error(BCM_EINVAL, "%s: null args", fn);
  const bcm_scan_args& a = *ap;
  if (!dtype_ok(a.dtype)) return set_error(BCM_EINVAL, "%s: u_flat must be fp16/bf16/fp32", fn);
  if (a.n_channels < 1) return set_error(BCM_EINVAL, "%s: cu_seqlens must have at least 2 elements", fn);
  if (a.dim < 1) return set_error(BCM_EINVAL, "%s: dim must be >= 1", fn);
  if (a.dstate < 1 || a.dstate > 256) return set_error(BCM_EINVAL, "%s: dstate must be in [1, 256]", fn);
  if (a.max_seqlen < 0) return set_error(BCM_EINVAL, "%s: max_seqlen must be non-negative", fn);
  const int want = a.max_seqlen > 0 ? (a.max_seqlen + 2047) / 2048 : 1;
  if (a.n_chunks != want) return set_error(BCM_EINVAL, "%s: n_chunks must equal max(1, ceil(max_seqlen/2048))", fn);
  if (a.n_events < 0 || a.n_events > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_events out of range", fn);
  if (!a.cu_seqlens || !a.dt_idle || !a.dt_active || !a.A || !a.W_B || !a.W_C)
    return set_error(BCM_EINVAL, "%s: null input pointer", fn);
  if (a.n_events > 0 && (!a.u || !a.k)) return set_error(BCM_EINVAL, "%s: null u/k pointer", fn);
  const bool z = a.z != nullptr;
  if (!BWD) {
    if (!a.x || (a.n_events > 0 && !a.out)) return set_error(BCM_EINVAL, "%s: null output pointer", fn);
    if (z && a.n_events > 0 && !a.out_z) return set_error(BCM_EINVAL, "%s: out_z required with z", fn);
  } else {
    if (!a.dA || !a.dW_B || !a.dW_C || !a.ddt_idle || !a.ddt_active)
      return set_error(BCM_EINVAL, "%s: null gradient pointer", fn);
    if (a.n_events > 0 && (!a.dout || !a.du)) return set_error(BCM_EINVAL, "%s: null dout/du pointer", fn);
    if (a.max_seqlen > 2048 && !a.x_saved) return set_error(BCM_EINVAL, "%s: x required for multi-chunk", fn);
    if (z && a.n_events > 0 && (!a.out_saved || !a.dz))
      return set_error(BCM_EINVAL, "%s: out and dz required with z", fn);
  }
  const hipStream_t s = hs(stream);
  int rc = BCM_OK;
  dispatch_dtype(a.dtype, [&](auto tag) {
    using T = decltype(tag);
    rc = z ? dispatch_shape<T, true, BWD>(a, s, fn) : dispatch_shape<T, false, BWD>(a, s, fn);
  });
  return rc;
}

}  // namespace bcm

extern "C" {

int bcm_scan_fwd(const bcm_scan_args* args, bcm_stream_t stream) {
  return bcm::scan_entry<false>(args, stream, "bcm_scan_fwd");
}

int bcm_scan_bwd(const bcm_scan_args* args, bcm_stream_t stream) {
  return bcm::scan_entry<true>(args, stream, "bcm_scan_bwd");
}

}  // extern "C"
