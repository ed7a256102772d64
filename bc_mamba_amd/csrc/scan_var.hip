// Stage 2b: flat per-channel selective scan whose B and C are operands of
// their own instead of u·W_B / u·W_C: the legacy [dstate, E] (per event) or
// [dstate, dim] (per model channel) layout and the tiled
// [n_tiles, dstate, T] layout of fwd_flat_ch / bwd_flat_ch.
//
// Reference behaviour: selective_scan.cpp:760-776, 840-848 (layouts and
// checks), selective_scan_fwd_kernel.cuh:566-598 (B/C addressing: tiled
// B[tile_offsets[ch] + chunk, s, i], legacy B[s, ev]), :640-686 (h_i =
// a_i h_{i-1} + B_i Δ_i u_i, y_i = D u_i + Σ_s C_i h_i),
// selective_scan_bwd_kernel.cuh:902-1044 (dh recurrence, per-event dB / dC),
// :1087-1112 (constant B / C sums), selective_scan.cpp:1085-1090 (dB / dC
// mirror the B / C layout).
//
// MI355X design: one workgroup per model channel d (its waves take the
// channels b·dim + d, so dA, ddt, dD and the constant-B/C sums reduce in LDS
// in a fixed order: no atomics, deterministic). A channel runs in passes of
// 128 events: 16 lanes (one DPP row) × 8 consecutive events per lane. Per
// pass and state a lane folds its 8 items, the row combines the folds with
// the DPP scan of scan_group.hpp, and a second register pass produces the
// states; (decay product, h) and the backward's a·dh carry to the next pass
// through LDS. B and C are read per (state, event) straight from global
// memory: 8 consecutive events per lane, 512 contiguous bytes per row. The
// backward reads the forward states from a workspace [dstate, E] that a
// forward pass over the same inputs writes first, so it needs no chunk
// re-seeding. These modes are not used by the BC_mamba block; the kernels
// aim at correctness at memory speed, not at the depthwise path's VALU tuning.
#include "bcm_common.hpp"
#include "scan_group.hpp"

#include <climits>

namespace bcm {

namespace {
constexpr int kVG = 16;              // lanes per channel group
constexpr int kVR = 8;               // consecutive events per lane
constexpr int kVPass = kVG * kVR;    // events per pass
constexpr int kVThreads = 256;       // 4 waves, 16 channel groups
constexpr int kXChunk = 2048;        // events per saved-state chunk (selective_scan.cpp:795)
constexpr float kLog2eV = 1.4426950408889634f;
static_assert(kXChunk % kVPass == 0, "passes must tile the saved-state chunks");

struct VarLds {
  int N, nslots;
  bool bwd;
  int64_t bytes() const {
    return 4ll * (4ll * N + (int64_t)nslots * (bwd ? (N + 3 * N + 3) : 2 * N));
  }
};

// Element offsets of one operand for the 8 items of a lane in a pass:
// off(s, r) = base[r] + s * sstride, valid when ok[r].
struct BcOperand {
  const float* p;
  int64_t base[kVR];
  int64_t sstride;
  bool ok[kVR];
};

__device__ __forceinline__ void bc_offsets(BcOperand& o, const float* ptr, bool per_event, bool tiled,
                                           int64_t row_stride, int64_t e_first, int pos_first, int n,
                                           int64_t tile0, int T, int N, int64_t n_tiles) {
  o.p = ptr;
  o.sstride = tiled ? T : row_stride;
#pragma unroll
  for (int r = 0; r < kVR; ++r) {
    const int pos = pos_first + r;
    bool ok = per_event && pos < n;
    int64_t base = e_first + r;
    if (tiled) {
      const int64_t tile = tile0 + pos / T;
      ok = ok && tile >= 0 && tile < n_tiles;
      base = (tile * N) * (int64_t)T + pos % T;
    }
    o.ok[r] = ok;
    o.base[r] = ok ? base : 0;
  }
}

__device__ __forceinline__ float bc_load(const BcOperand& o, int r, int s) {
  return o.ok[r] ? o.p[o.base[r] + (int64_t)s * o.sstride] : 0.0f;
}

}  // namespace

template <typename T, bool HAS_Z, bool VB, bool VC>
__global__ __launch_bounds__(kVThreads) void k_scan_var_fwd(const bcm_scan_args a, const bcm_scan_bc bc,
                                                            float* __restrict__ hws) {
  using Ops = Grp<kVG>;
  const int N = a.dstate;
  const int d = blockIdx.x;
  const int nw = blockDim.x / kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / kVG, j = lane % kVG;
  const int nslots = nw * (kWave / kVG);
  const int slot = wave * (kWave / kVG) + grp;
  const bool tiled = bc.layout == BCM_BC_TILED;

  extern __shared__ float smem[];
  float* sAl = smem;
  float* sB = sAl + N;  // constant B / C column of d
  float* sC = sB + N;
  float* carry = sC + 2 * N + slot * 2 * N;  // [P(N), h(N)] at the end of the previous pass

  for (int s = threadIdx.x; s < N; s += blockDim.x) {
    sAl[s] = a.A[(int64_t)d * N + s] * kLog2eV;
    sB[s] = VB ? 0.0f : bc.B[(int64_t)s * bc.b_row_stride + d];
    sC[s] = VC ? 0.0f : bc.C[(int64_t)s * bc.c_row_stride + d];
  }
  __syncthreads();

  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;
  const int64_t E = a.n_events;
  const T* __restrict__ u = static_cast<const T*>(a.u);
  const T* __restrict__ z = static_cast<const T*>(a.z);
  T* __restrict__ out = static_cast<T*>(a.out);
  T* __restrict__ out_z = static_cast<T*>(a.out_z);

  for (int b0 = 0; b0 < n_per_d; b0 += nslots) {
    const int b = b0 + slot;
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    const int e0 = act ? a.cu_seqlens[ch] : 0;
    // events stay inside [0, E) whatever cu_seqlens holds
    const int n = (act && e0 >= 0) ? (int)max((int64_t)0, min((int64_t)a.cu_seqlens[ch + 1], E) - e0) : 0;
    const int np = (n + kVPass - 1) / kVPass;
    const int npw = wave_max_dpp(np);
    const int64_t tile0 = (tiled && act) ? (int64_t)bc.tile_offsets[ch] : 0;
    for (int p = 0; p < npw; ++p) {
      const int pos0 = p * kVPass + j * kVR;
      float uu[kVR], dl[kVR], dlu[kVR], y[kVR];
      bool valid[kVR];
#pragma unroll
      for (int r = 0; r < kVR; ++r) {
        valid[r] = pos0 + r < n;
        const int64_t e = (int64_t)e0 + pos0 + r;
        uu[r] = valid[r] ? to_f(u[e]) : 0.0f;
        const int kk = valid[r] ? a.k[e] : 1;
        dl[r] = valid[r] ? fmaf(dti, (float)(kk - 1), dta) : 0.0f;
        dlu[r] = dl[r] * uu[r];
        y[r] = Dv * uu[r];
      }
      BcOperand ob, oc;
      bc_offsets(ob, bc.B, VB, tiled, bc.b_row_stride, (int64_t)e0 + pos0, pos0, n, tile0, bc.tile_chunk_size, N,
                 bc.n_tiles);
      bc_offsets(oc, bc.C, VC, tiled, bc.c_row_stride, (int64_t)e0 + pos0, pos0, n, tile0, bc.tile_chunk_size, N,
                 bc.n_tiles);
      // the pass that holds the last event of a saved-state chunk (or of the channel)
      const int pass_end = min(n, (p + 1) * kVPass);
      const bool save_x = a.x && p < np && (pass_end % kXChunk == 0 || pass_end == n);
      const int xc = (pass_end - 1) / kXChunk;
#pragma unroll 1
      for (int s = 0; s < N; ++s) {
        const float Al = sAl[s];
        float av[kVR], xv[kVR], cv[kVR];
        float P = 1.0f, H = 0.0f;
#pragma unroll
        for (int r = 0; r < kVR; ++r) {
          av[r] = valid[r] ? decay(dl[r] * Al) : 1.0f;
          const float bv = VB ? bc_load(ob, r, s) : sB[s];
          xv[r] = valid[r] ? bv * dlu[r] : 0.0f;
          cv[r] = VC ? bc_load(oc, r, s) : sC[s];
          H = fmaf(av[r], H, xv[r]);
          P *= av[r];
        }
        Ops::scan_up(P, H);
        const float h0 = p > 0 ? carry[N + s] : 0.0f;
        const float P0 = p > 0 ? carry[s] : 1.0f;
        const float hend = fmaf(P, h0, H);
        float h = Ops::prev(hend, h0);
#pragma unroll
        for (int r = 0; r < kVR; ++r) {
          h = fmaf(av[r], h, xv[r]);
          y[r] = fmaf(cv[r], h, y[r]);
          if (hws && valid[r]) hws[(int64_t)s * E + e0 + pos0 + r] = h;
        }
        if (j == kVG - 1 && p < np) {
          carry[s] = P0 * P;
          carry[N + s] = hend;
          if (save_x && xc < nck) {
            float* xs = a.x + ((ch * nck + xc) * 2 * N);
            xs[2 * s] = P0 * P;
            xs[2 * s + 1] = hend;
          }
        }
      }
      if (out) {
#pragma unroll
        for (int r = 0; r < kVR; ++r) {
          if (!valid[r]) continue;
          const int64_t e = (int64_t)e0 + pos0 + r;
          out[e] = from_f<T>(y[r]);
          if (HAS_Z) {
            const float zv = to_f(z[e]);
            out_z[e] = from_f<T>(y[r] * (zv / (1.0f + __expf(-zv))));
          }
        }
      }
    }
    // saved-state chunks past the channel's end keep the reference's zero state
    if (act && a.x) {
      const int have = (n + kXChunk - 1) / kXChunk;
      for (int c = have; c < nck; ++c)
        for (int s = j; s < 2 * N; s += kVG) a.x[(ch * nck + c) * 2 * N + s] = 0.0f;
    }
  }
}

template <typename T, bool HAS_Z, bool VB, bool VC>
__global__ __launch_bounds__(kVThreads) void k_scan_var_bwd(const bcm_scan_args a, const bcm_scan_bc bc,
                                                            const float* __restrict__ hws) {
  using Ops = Grp<kVG>;
  const int N = a.dstate;
  const int d = blockIdx.x;
  const int nw = blockDim.x / kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / kVG, j = lane % kVG;
  const int nslots = nw * (kWave / kVG);
  const int slot = wave * (kWave / kVG) + grp;
  const bool tiled = bc.layout == BCM_BC_TILED;
  const int NA = 3 * N + 3;  // per slot: dA, constant dB, constant dC, ddt_idle, ddt_active, dD

  extern __shared__ float smem[];
  float* sAl = smem;
  float* sA = sAl + N;
  float* sB = sA + N;
  float* sC = sB + N;
  float* cdh = sC + N + slot * N;                       // a·dh of the first event of the later pass
  float* sacc = sC + N + nslots * N;                    // [nslots][NA]
  float* cacc = sacc + slot * NA;

  for (int s = threadIdx.x; s < N; s += blockDim.x) {
    const float Av = a.A[(int64_t)d * N + s];
    sA[s] = Av;
    sAl[s] = Av * kLog2eV;
    sB[s] = VB ? 0.0f : bc.B[(int64_t)s * bc.b_row_stride + d];
    sC[s] = VC ? 0.0f : bc.C[(int64_t)s * bc.c_row_stride + d];
  }
  for (int i = threadIdx.x; i < nslots * NA; i += blockDim.x) sacc[i] = 0.0f;
  __syncthreads();

  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  const int NC = a.n_channels, dim = a.dim;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;
  const int64_t E = a.n_events;
  const T* __restrict__ u = static_cast<const T*>(a.u);
  const T* __restrict__ dout = static_cast<const T*>(a.dout);
  const T* __restrict__ z = static_cast<const T*>(a.z);
  const T* __restrict__ osv = static_cast<const T*>(a.out_saved);
  T* __restrict__ du_out = static_cast<T*>(a.du);
  T* __restrict__ dz_out = static_cast<T*>(a.dz);

  for (int b0 = 0; b0 < n_per_d; b0 += nslots) {
    const int b = b0 + slot;
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    const int e0 = act ? a.cu_seqlens[ch] : 0;
    // events stay inside [0, E) whatever cu_seqlens holds
    const int n = (act && e0 >= 0) ? (int)max((int64_t)0, min((int64_t)a.cu_seqlens[ch + 1], E) - e0) : 0;
    const int np = (n + kVPass - 1) / kVPass;
    const int npw = wave_max_dpp(np);
    const int64_t tile0 = (tiled && act) ? (int64_t)bc.tile_offsets[ch] : 0;
    float ddti_l = 0.0f, ddta_l = 0.0f, dD_l = 0.0f;
    for (int p = npw - 1; p >= 0; --p) {
      const int pos0 = p * kVPass + j * kVR;
      const int64_t eb = (int64_t)e0 + pos0;
      float uu[kVR], dl[kVR], dlu[kVR], dov[kVR], du[kVR], ddl[kVR];
      int km1[kVR];
      bool valid[kVR];
#pragma unroll
      for (int r = 0; r < kVR; ++r) {
        valid[r] = pos0 + r < n;
        const int64_t e = eb + r;
        uu[r] = valid[r] ? to_f(u[e]) : 0.0f;
        km1[r] = valid[r] ? a.k[e] - 1 : 0;
        dl[r] = valid[r] ? fmaf(dti, (float)km1[r], dta) : 0.0f;
        dlu[r] = dl[r] * uu[r];
        float g = valid[r] ? to_f(dout[e]) : 0.0f;
        if (HAS_Z && valid[r]) {  // selective_scan_bwd_kernel.cuh:795-801
          const float zv = to_f(z[e]), ov = to_f(osv[e]);
          const float sg = 1.0f / (1.0f + __expf(-zv));
          dz_out[e] = from_f<T>(g * ov * sg * (1.0f + zv * (1.0f - sg)));
          g *= zv * sg;
        }
        dov[r] = g;
        du[r] = Dv * g;
        ddl[r] = 0.0f;
        dD_l = fmaf(g, uu[r], dD_l);
      }
      BcOperand ob, oc, odb, odc;
      bc_offsets(ob, bc.B, VB, tiled, bc.b_row_stride, eb, pos0, n, tile0, bc.tile_chunk_size, N, bc.n_tiles);
      bc_offsets(oc, bc.C, VC, tiled, bc.c_row_stride, eb, pos0, n, tile0, bc.tile_chunk_size, N, bc.n_tiles);
      bc_offsets(odb, bc.dB, VB, tiled, bc.db_row_stride, eb, pos0, n, tile0, bc.tile_chunk_size, N, bc.n_tiles);
      bc_offsets(odc, bc.dC, VC, tiled, bc.dc_row_stride, eb, pos0, n, tile0, bc.tile_chunk_size, N, bc.n_tiles);
#pragma unroll 1
      for (int s = 0; s < N; ++s) {
        const float Al = sAl[s], Av = sA[s];
        const float* hs_ = hws + (int64_t)s * E;
        float av[kVR], bv[kVR], gv[kVR], hv[kVR];
#pragma unroll
        for (int r = 0; r < kVR; ++r) {
          av[r] = valid[r] ? decay(dl[r] * Al) : 1.0f;
          bv[r] = VB ? bc_load(ob, r, s) : sB[s];
          const float cv = VC ? bc_load(oc, r, s) : sC[s];
          gv[r] = valid[r] ? cv * dov[r] : 0.0f;
          hv[r] = valid[r] ? hs_[eb + r] : 0.0f;
        }
        const float hp0 = (valid[0] && pos0 > 0) ? hs_[eb - 1] : 0.0f;  // state before the lane's first item
        // dh_i = C_i dout_i + a_{i+1} dh_{i+1}; the last lane of the group
        // takes the carry a·dh of the later pass (and a "next decay" of 1)
        const float anext = Ops::next(av[0], 1.0f);
        const float ec = (p + 1 < np) ? cdh[s] : 0.0f;
        float Q = 1.0f, Ce = 0.0f;
#pragma unroll
        for (int r = kVR - 1; r >= 0; --r) {
          const float al = r == kVR - 1 ? anext : av[r + 1];
          Ce = fmaf(al, Ce, gv[r]);
          Q *= al;
        }
        Ops::scan_down(Q, Ce);
        float dh = Ops::next(fmaf(Q, ec, Ce), ec);
        float dA_l = 0.0f, dBc_l = 0.0f, dCc_l = 0.0f;
#pragma unroll
        for (int r = kVR - 1; r >= 0; --r) {
          const float al = r == kVR - 1 ? anext : av[r + 1];
          dh = fmaf(al, dh, gv[r]);
          const float hp = r > 0 ? hv[r - 1] : hp0;
          const float t = valid[r] ? dh * av[r] * hp : 0.0f;
          dA_l = fmaf(t, dl[r], dA_l);
          const float dhb = valid[r] ? dh * bv[r] : 0.0f;
          ddl[r] = fmaf(dhb, uu[r], fmaf(Av, t, ddl[r]));
          du[r] = fmaf(dhb, dl[r], du[r]);
          const float dbv = valid[r] ? dh * dlu[r] : 0.0f;
          const float dcv = dov[r] * hv[r];
          if (VB) {
            if (odb.ok[r]) const_cast<float*>(odb.p)[odb.base[r] + (int64_t)s * odb.sstride] = dbv;  // bc.dB
          } else {
            dBc_l += dbv;
          }
          if (VC) {
            if (odc.ok[r]) const_cast<float*>(odc.p)[odc.base[r] + (int64_t)s * odc.sstride] = dcv;  // bc.dC
          } else {
            dCc_l += dcv;
          }
        }
        if (j == 0 && p < np) cdh[s] = av[0] * dh;  // dh of the pass's first event
        dA_l = Ops::sum(dA_l);
        if (!VB) dBc_l = Ops::sum(dBc_l);
        if (!VC) dCc_l = Ops::sum(dCc_l);
        if (j == 0 && act) {
          cacc[s] += dA_l;
          if (!VB) cacc[N + s] += dBc_l;
          if (!VC) cacc[2 * N + s] += dCc_l;
        }
      }
#pragma unroll
      for (int r = 0; r < kVR; ++r) {
        if (valid[r]) du_out[eb + r] = from_f<T>(du[r]);
        ddti_l = fmaf(ddl[r], (float)km1[r], ddti_l);
        ddta_l += ddl[r];
      }
    }
    ddti_l = Ops::sum(ddti_l);
    ddta_l = Ops::sum(ddta_l);
    dD_l = Ops::sum(dD_l);
    if (j == 0 && act) {
      cacc[3 * N] += ddti_l;
      cacc[3 * N + 1] += ddta_l;
      cacc[3 * N + 2] += dD_l;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NA; i += blockDim.x) {
    float v = 0.0f;
    for (int q = 0; q < nslots; ++q) v += sacc[q * NA + i];  // fixed order: deterministic
    if (i < N) {
      a.dA[(int64_t)d * N + i] = v;
    } else if (i < 2 * N) {
      if (!VB) bc.dB[(int64_t)(i - N) * bc.db_row_stride + d] = v;
    } else if (i < 3 * N) {
      if (!VC) bc.dC[(int64_t)(i - 2 * N) * bc.dc_row_stride + d] = v;
    } else if (i == 3 * N) {
      a.ddt_idle[d] = v;
    } else if (i == 3 * N + 1) {
      a.ddt_active[d] = v;
    } else if (a.dD) {
      a.dD[d] = v;
    }
  }
}

static int var_checks(const bcm_scan_args* ap, const bcm_scan_bc* bc, bool bwd, const char* fn) {
  if (!ap || !bc) return set_error(BCM_EINVAL, "%s: null args", fn);
  const bcm_scan_args& a = *ap;
  if (!dtype_ok(a.dtype)) return set_error(BCM_EINVAL, "%s: u_flat must be fp16/bf16/fp32", fn);
  if (a.n_channels < 1) return set_error(BCM_EINVAL, "%s: cu_seqlens must have at least 2 elements", fn);
  if (a.dim < 1) return set_error(BCM_EINVAL, "%s: dim must be >= 1", fn);
  if (a.dstate < 1 || a.dstate > 256) return set_error(BCM_EINVAL, "%s: dstate must be in [1, 256]", fn);
  if (a.max_seqlen < 0) return set_error(BCM_EINVAL, "%s: max_seqlen must be non-negative", fn);
  const int want = a.max_seqlen > 0 ? (a.max_seqlen + kXChunk - 1) / kXChunk : 1;
  if (a.n_chunks != want) return set_error(BCM_EINVAL, "%s: n_chunks must equal max(1, ceil(max_seqlen/2048))", fn);
  if (a.n_events < 0 || a.n_events > INT32_MAX) return set_error(BCM_EINVAL, "%s: n_events out of range", fn);
  if (!a.cu_seqlens || !a.dt_idle || !a.dt_active || !a.A) return set_error(BCM_EINVAL, "%s: null input pointer", fn);
  if (a.n_events > 0 && (!a.u || !a.k)) return set_error(BCM_EINVAL, "%s: null u/k pointer", fn);
  if (bc->layout != BCM_BC_LEGACY && bc->layout != BCM_BC_TILED)
    return set_error(BCM_EINVAL, "%s: B/C layout must be BCM_BC_LEGACY or BCM_BC_TILED", fn);
  if (!bc->B || !bc->C) return set_error(BCM_EINVAL, "%s: null B/C pointer", fn);
  if (bc->layout == BCM_BC_TILED) {
    if (!bc->b_per_event || !bc->c_per_event)
      return set_error(BCM_EINVAL, "%s: tiled B/C are per event", fn);
    if (!bc->tile_offsets || bc->tile_chunk_size < 1 || bc->n_tiles < 0)
      return set_error(BCM_EINVAL, "%s: tiled B/C need tile_offsets, tile_chunk_size >= 1 and n_tiles >= 0", fn);
  } else {
    if (bc->b_row_stride < 1 || bc->c_row_stride < 1)
      return set_error(BCM_EINVAL, "%s: legacy B/C row strides must be >= 1", fn);
  }
  const bool z = a.z != nullptr;
  if (!bwd) {
    if (!a.x || (a.n_events > 0 && !a.out)) return set_error(BCM_EINVAL, "%s: null output pointer", fn);
    if (z && a.n_events > 0 && !a.out_z) return set_error(BCM_EINVAL, "%s: out_z required with z", fn);
  } else {
    if (!a.dA || !a.ddt_idle || !a.ddt_active || !bc->dB || !bc->dC)
      return set_error(BCM_EINVAL, "%s: null gradient pointer", fn);
    if (bc->layout == BCM_BC_LEGACY && (bc->db_row_stride < 1 || bc->dc_row_stride < 1))
      return set_error(BCM_EINVAL, "%s: legacy dB/dC row strides must be >= 1", fn);
    if (a.n_events > 0 && (!a.dout || !a.du)) return set_error(BCM_EINVAL, "%s: null dout/du pointer", fn);
    if (z && a.n_events > 0 && (!a.out_saved || !a.dz))
      return set_error(BCM_EINVAL, "%s: out and dz required with z", fn);
  }
  return BCM_OK;
}

template <bool BWD, typename T, bool Z, bool VB, bool VC>
static int var_launch(const bcm_scan_args& a, const bcm_scan_bc& bc, float* hws, hipStream_t s, const char* fn) {
  const int nw = kVThreads / kWave;
  const int64_t lds = VarLds{a.dstate, nw * (kWave / kVG), BWD}.bytes();
  if (lds > max_lds_bytes())
    return set_error(BCM_EINVAL, "%s: dstate %d needs %lld bytes of LDS", fn, a.dstate, (long long)lds);
  if (BWD)
    hipLaunchKernelGGL((k_scan_var_bwd<T, Z, VB, VC>), dim3(a.dim), dim3(kVThreads), (size_t)lds, s, a, bc, hws);
  else
    hipLaunchKernelGGL((k_scan_var_fwd<T, Z, VB, VC>), dim3(a.dim), dim3(kVThreads), (size_t)lds, s, a, bc, hws);
  return check_launch(fn);
}

template <bool BWD>
static int var_dispatch(const bcm_scan_args& a, const bcm_scan_bc& bc, float* hws, hipStream_t s, const char* fn) {
  int rc = BCM_OK;
  const bool z = a.z != nullptr;
  const int mode = (bc.b_per_event ? 2 : 0) | (bc.c_per_event ? 1 : 0);
  dispatch_dtype(a.dtype, [&](auto tag) {
    using T = decltype(tag);
    auto go = [&](auto zt) {
      constexpr bool Z = decltype(zt)::value;
      switch (mode) {
        case 3: rc = var_launch<BWD, T, Z, true, true>(a, bc, hws, s, fn); break;
        case 2: rc = var_launch<BWD, T, Z, true, false>(a, bc, hws, s, fn); break;
        case 1: rc = var_launch<BWD, T, Z, false, true>(a, bc, hws, s, fn); break;
        default: rc = var_launch<BWD, T, Z, false, false>(a, bc, hws, s, fn); break;
      }
    };
    if (z) go(std::true_type{});
    else go(std::false_type{});
  });
  return rc;
}

}  // namespace bcm

extern "C" {

int64_t bcm_scan_var_workspace_bytes(int64_t n_events, int dstate) {
  return (n_events < 0 || dstate < 1) ? 0 : 4 * n_events * (int64_t)dstate;
}

int bcm_scan_var_fwd(const bcm_scan_args* args, const bcm_scan_bc* bc, bcm_stream_t stream) {
  const char* fn = "bcm_scan_var_fwd";
  int rc = bcm::var_checks(args, bc, false, fn);
  if (rc) return rc;
  return bcm::var_dispatch<false>(*args, *bc, nullptr, bcm::hs(stream), fn);
}

int bcm_scan_var_bwd(const bcm_scan_args* args, const bcm_scan_bc* bc, void* workspace, int64_t workspace_bytes,
                     bcm_stream_t stream) {
  const char* fn = "bcm_scan_var_bwd";
  int rc = bcm::var_checks(args, bc, true, fn);
  if (rc) return rc;
  const int64_t need = bcm_scan_var_workspace_bytes(args->n_events, args->dstate);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return bcm::set_error(BCM_EINVAL, "%s: workspace of %lld bytes needed", fn, (long long)need);
  // forward states h[s, e] of the same inputs (outputs and x not written)
  bcm_scan_args f = *args;
  f.out = nullptr;
  f.out_z = nullptr;
  f.x = nullptr;
  float* hws = static_cast<float*>(workspace);
  rc = bcm::var_dispatch<false>(f, *bc, hws, bcm::hs(stream), fn);
  if (rc) return rc;
  return bcm::var_dispatch<true>(*args, *bc, hws, bcm::hs(stream), fn);
}

}  // extern "C"
