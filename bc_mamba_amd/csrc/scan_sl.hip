// Stage 2, dstate 16 / 32 / 64: the depthwise flat selective scan with one
// lane per (channel, group of states), forward and backward.
//
// Reference behaviour: as scan.hip (selective_scan_fwd_kernel.cuh:403-728,
// selective_scan_bwd_kernel.cuh:635-1169, the exponent clamp of
// selective_scan_common.h:43-52).
//
// MI355X design
//   * The 16 lanes of a DPP row own one channel; lane s holds states
//     s + 16j, j < NL (NL = dstate / 16: one, two or four independent
//     recurrences per lane). A wave holds four channels of one model channel
//     d (one workgroup per d, as in scan.hip, so the per-d decay table and
//     the parameter-gradient sums stay in the workgroup). Each lane walks its
//     channel's events in order: the recurrence costs one table read and one
//     fma per event and state, with no lane scans and no padding beyond a
//     block's tail.
//   * Events come in blocks of 16, one per lane of the row: lane j loads
//     event 16·blk + j (coalesced), forms Δ, Δu², its table offset (and the
//     backward's dout·u, k-1), and DPP row_newbcast:q hands event q's values
//     to the whole row, once for all NL states of a lane. The next blocks'
//     loads are in flight while a block computes (a ring of registers), so
//     memory latency overlaps the VALU.
//   * Sums over the states of one event (y, and the backward's Σ_s W_B W_C e
//     and Σ_s W_B W_C g): each lane forms its states' weighted share for
//     each of the block's 16 events, and a DPP reduce-scatter over the row
//     leaves event j's sum in lane j (four halving steps, no LDS round trip
//     and no wave barrier).
//   * The forward saves the state h at the start of every 32-event pass in
//     chunk_g; the backward walks a channel's passes last to first, rebuilds
//     the pass's states (and, up to two states per lane, decays) in registers
//     from that row, then runs the adjoint recurrence
//     e_i = a_{i+1} e_{i+1} + dout_i u_i backward through them.
//   * Bursty streams (a longest channel of more than twice the mean): the
//     workgroup first ranks its model channel's channels by length, and the
//     four rows of a wave take neighbouring ranks, so a wave's rows end
//     together; the two waves that share a SIMD pair long ranks with short.
//   * Scaled recurrences as in scan.hip: g = h / W_B (g = a·g + Δu²) and
//     e = dh / W_C.

#include "bcm_common.hpp"
#include "scan_common.hpp"

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdlib>

namespace bcm {

constexpr int kSLB = 16;                   // events per block (one per lane of a row)
constexpr int kSLRows = kWave / kSLN;      // channels per wave
constexpr int kSLPF = 4;                   // blocks per load round (a round ahead in flight)

// Shape of the state-lane kernels with NL states per lane (dstate 16·NL).
// The decay table holds two copies interleaved, T[k][m][parity]: lane
// (row g, state m) reads word 2(N k + m) + (g & 1), so the two rows
// (channels) of a half-wave read disjoint banks whatever their gaps k (one
// bank per lane: conflict-free); state m + 16j sits 128 bytes after m.
template <int NL> struct SLShape {
  static constexpr int N = kSLN * NL;            // dstate
  static constexpr int Tab = tab_gaps(N);        // longest gap in the decay table
  static constexpr uint32_t Gap = 2u * N * 4u;   // bytes per gap row of the table
  static constexpr int TabSz = 2 * N * (Tab + 1);  // floats of the table
  static constexpr int NA = 3 * N + 3;           // gradient accumulators per slot
  // the backward keeps a pass's decays in registers beside its states up to
  // two states per lane; with four it reads them from the table again
  static constexpr bool KeepA = NL <= 2;
  // events per table round of the backward: four states per lane read a
  // half block at a time, so fewer decays are live beside the pass's states
  static constexpr int H = NL == 4 ? 8 : 16;
  // events per pass (chunk_g rows, the backward's unit of work): the pass's
  // states stay in registers, four states per lane hold 16 events' worth
  static constexpr int Pass = NL == 4 ? 16 : 32;
};
static_assert(SLShape<1>::Pass == kSLPass, "one state per lane: the scan_common pass length");
__device__ __forceinline__ uint32_t sl_tab_lane(int s, int grp) { return (uint32_t)(2 * s + (grp & 1)) * 4; }

// Value of lane Q of this lane's DPP row.
template <int Q> __device__ __forceinline__ int bcast_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x150 + Q, 0xF, 0xF, true);  // row_newbcast:Q
}
template <int Q> __device__ __forceinline__ float bcast_f(float v) {
  return __int_as_float(bcast_i<Q>(__float_as_int(v)));
}

// Decays of the 16 events of a block for this lane's states: each event's
// byte offset in a table row (lane q's tb) plus the lane's row base, one DPP
// add per event, then one read per state (states 16 apart are 128 bytes
// apart). One s_nop 1 first: a DPP read needs two wait states after the VALU
// write of its source, whichever instruction the compiler placed just
// before; the adds themselves write no source of a later one.
template <int NL>
__device__ __forceinline__ void tab16(float (&av)[NL][16], const float* sT, uint32_t rowb, uint32_t tb) {
  uint32_t o[16];
  asm("s_nop 1\n\t"
      "v_add_u32_dpp %0, %16, %17 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %1, %16, %17 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %2, %16, %17 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %3, %16, %17 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %4, %16, %17 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %5, %16, %17 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %6, %16, %17 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %7, %16, %17 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %8, %16, %17 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %9, %16, %17 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %10, %16, %17 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %11, %16, %17 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %12, %16, %17 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %13, %16, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %14, %16, %17 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
      "v_add_u32_dpp %15, %16, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7]),
        "=&v"(o[8]), "=&v"(o[9]), "=&v"(o[10]), "=&v"(o[11]), "=&v"(o[12]), "=&v"(o[13]), "=&v"(o[14]), "=&v"(o[15])
      : "v"(tb), "v"(rowb));
#pragma unroll
  for (int q = 0; q < 16; ++q)
#pragma unroll
    for (int j = 0; j < NL; ++j)
      av[j][q] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(sT) + o[q] + 128u * (uint32_t)j);
}

// Decays of events Q0..Q0+NQ-1 of a block, as tab16 (a shorter range keeps
// fewer decays live: the four-state backward works in half blocks). The
// s_nop 1 of the first add covers the source's last write; the hazard check
// over the built assembly (tests/test_dpp_hazards.py) keeps it honest.
// One event's table address: tb of lane Q of the row plus the lane's row base.
// volatile: the adds of a range keep their order, so the first (with the
// s_nop) stays first after tb's write. Without it the scheduler may move a
// later add ahead of it: a DPP read two wait states early, whose result
// varies with the other waves' timing (seen in a loop of another shape).
template <int Q, bool NOP> __device__ __forceinline__ uint32_t tab_addr(uint32_t tb, uint32_t rowb) {
  uint32_t o;
  if constexpr (NOP)
    asm volatile("s_nop 1\n\tv_add_u32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "=&v"(o) : "v"(tb), "v"(rowb), "n"(Q));
  else
    asm volatile("v_add_u32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "=&v"(o) : "v"(tb), "v"(rowb), "n"(Q));
  return o;
}
template <int NL, int Q0, int NQ, int... Q>
__device__ __forceinline__ void tabq_impl(float (&av)[NL][16], const float* sT, uint32_t rowb, uint32_t tb,
                                          std::integer_sequence<int, Q...>) {
  const uint32_t o[NQ] = {tab_addr<Q0 + Q, Q == 0>(tb, rowb)...};
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int j = 0; j < NL; ++j)
      av[j][Q0 + q] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(sT) + o[q] + 128u * (uint32_t)j);
}
template <int NL, int Q0, int NQ>
__device__ __forceinline__ void tabq(float (&av)[NL][16], const float* sT, uint32_t rowb, uint32_t tb) {
  tabq_impl<NL, Q0, NQ>(av, sT, rowb, tb, std::make_integer_sequence<int, NQ>{});
}

// acc += (value of lane Q of the row's src) * v as one v_fmac_f32_dpp (the
// compiler keeps a separate move for a float DPP operand). NOP: s_nop 1
// first, for the first use of src after its VALU write.
template <int Q, bool NOP> __device__ __forceinline__ void fmac_bcast(float& acc, float src, float v) {
  if constexpr (NOP)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
        : "+v"(acc) : "v"(src), "v"(v), "n"(Q));
  else
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(src), "v"(v), "n"(Q));
}

// Calls f(std::integral_constant<int, q>) for q = 0..15 (compile-time lane
// indices for the DPP controls).
template <typename F, int... Q> __device__ __forceinline__ void for16_impl(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, Q>{}), ...);
}
template <typename F> __device__ __forceinline__ void for16(F&& f) {
  for16_impl(f, std::make_integer_sequence<int, 16>{});
}
template <typename F, int... Q> __device__ __forceinline__ void rfor16_impl(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, 15 - Q>{}), ...);
}
template <typename F> __device__ __forceinline__ void rfor16(F&& f) {  // q = 15..0
  rfor16_impl(f, std::make_integer_sequence<int, 16>{});
}
// Calls f(std::integral_constant<int, q>) for q = Q0..Q0+NQ-1 (forr) or
// q = Q0+NQ-1..Q0 (rforr).
template <int Q0, typename F, int... Q> __device__ __forceinline__ void forr_impl(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, Q0 + Q>{}), ...);
}
template <int Q0, int NQ, typename F> __device__ __forceinline__ void forr(F&& f) {
  forr_impl<Q0>(f, std::make_integer_sequence<int, NQ>{});
}
template <int Q0, int NQ, typename F, int... Q>
__device__ __forceinline__ void rforr_impl(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, Q0 + NQ - 1 - Q>{}), ...);
}
template <int Q0, int NQ, typename F> __device__ __forceinline__ void rforr(F&& f) {
  rforr_impl<Q0, NQ>(f, std::make_integer_sequence<int, NQ>{});
}

// Sum over the 16 lanes of a row, in every lane of it.
__device__ __forceinline__ float row_sum(float v) {
  v += __uint_as_float(dpp<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp<0x140>(__float_as_uint(v)));  // row_mirror
  return v;
}

// Sums over the 16 lanes of each DPP row of v[Q], Q = 0..15, leaving lane s
// of the row with the sum for Q = s: a reduce-scatter in four halving steps
// (partners s and 15 - s, then mirrors within 8 lanes, then quad xors), each
// lane keeping the half of its values that holds its own index and adding
// its partner's copy of that half. All VALU (DPP), no LDS round trip.
// The first two steps split the lanes by 4-lane bank (s < 8: banks 0-1;
// s & 7 < 4: banks 0 and 2), so each of their outputs is two DPP adds into
// one register, each writing only the banks that keep its half (bank_mask),
// with no selects; the quad steps split inside a bank and select. Each asm
// block starts with s_nop 1 (a DPP read needs two wait states after the
// VALU write of its source, which may be the instruction just before the
// block); inside a block every source was written before the block.
__device__ __forceinline__ float row_reduce_scatter16(const float (&v)[kSLN]) {
  const int s = lane_id() & (kSLN - 1);
  float a[8], b[4], c[2];
#define BCM_MIRROR_PAIR(I, J, K)                                                  \
  "v_add_f32_dpp %" #I ", %" #J ", %" #J " row_mirror row_mask:0xf bank_mask:0x3\n\t" \
  "v_add_f32_dpp %" #I ", %" #K ", %" #K " row_mirror row_mask:0xf bank_mask:0xc\n\t"
  asm("s_nop 1\n\t"
      BCM_MIRROR_PAIR(0, 8, 16) BCM_MIRROR_PAIR(1, 9, 17) BCM_MIRROR_PAIR(2, 10, 18) BCM_MIRROR_PAIR(3, 11, 19)
      BCM_MIRROR_PAIR(4, 12, 20) BCM_MIRROR_PAIR(5, 13, 21) BCM_MIRROR_PAIR(6, 14, 22) BCM_MIRROR_PAIR(7, 15, 23)
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(a[4]), "=&v"(a[5]), "=&v"(a[6]), "=&v"(a[7])
      : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]),
        "v"(v[8]), "v"(v[9]), "v"(v[10]), "v"(v[11]), "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]));
#undef BCM_MIRROR_PAIR
#define BCM_HALF_PAIR(I, J, K)                                                         \
  "v_add_f32_dpp %" #I ", %" #J ", %" #J " row_half_mirror row_mask:0xf bank_mask:0x5\n\t" \
  "v_add_f32_dpp %" #I ", %" #K ", %" #K " row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
  asm("s_nop 1\n\t"
      BCM_HALF_PAIR(0, 4, 8) BCM_HALF_PAIR(1, 5, 9) BCM_HALF_PAIR(2, 6, 10) BCM_HALF_PAIR(3, 7, 11)
      : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
#undef BCM_HALF_PAIR
  auto add_dpp = [](float kp, float snd, auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    return kp + __uint_as_float(dpp<C>(__float_as_uint(snd)));
  };
  const bool l2 = (s & 3) < 2, l1 = (s & 1) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    c[i] = add_dpp(l2 ? b[i] : b[2 + i], l2 ? b[2 + i] : b[i], std::integral_constant<int, kDppXor2>{});
  return add_dpp(l1 ? c[0] : c[1], l1 ? c[1] : c[0], std::integral_constant<int, kDppXor1>{});
}

// Decay table of model channel d: T[m][0] = 1 (padding), T[m][k] = the
// decay of gap k, the same expression as the per-event path. Thread t
// builds the entries of state t % N (consecutive threads: consecutive
// words); its A value is loaded at the kernel's start (al), before the
// first events' loads, so the build waits on no data load.
template <int NL> __device__ __forceinline__ float sl_table_al(const bcm_scan_args& a, int d) {
  constexpr int N = SLShape<NL>::N;
  return a.A[(int64_t)d * N + threadIdx.x % N] * kLog2e;
}
template <int NL> __device__ __forceinline__ void sl_build_table(float* sT, float al, float dti, float dta, int nw) {
  constexpr int N = SLShape<NL>::N;
  const int m = threadIdx.x % N;
  for (int q = threadIdx.x / N; q <= SLShape<NL>::Tab; q += nw * (kWave / N)) {
    const float v = q == 0 ? 1.0f : decay(fmaf(dti, (float)(q - 1), dta) * al);
    reinterpret_cast<float2*>(sT)[q * N + m] = make_float2(v, v);
  }
}

// Where a slot stands in the length order of a ranked workgroup: the four
// rows of a wave take neighbouring places, and of the two waves that share
// a SIMD (w and w + 4 of 8) one takes a long place and the other a short one.
__device__ __forceinline__ int sl_slot_order(int wave, int grp, int nw) {
  const int k = (nw == 8 && wave >= 4) ? 11 - wave : wave;
  return k * kSLRows + grp;
}

// ------------------------------------------------------------------ forward
// rank: rank the model channel's channels by length first (sord: [kSortMax]
// ints of LDS, keys: kSortMax ints of scratch LDS, dead after the ranking).
template <typename T, bool HAS_Z, int NL>
__device__ __forceinline__ void sl_fwd_body(const bcm_scan_args& a, float* sT, int* sord, int* keys, int nw, int S,
                                            int rank) {
#pragma clang fp contract(off)  // fmas are written out where they are meant
  using Sh = SLShape<NL>;
  constexpr uint32_t SZ = sizeof(T);
  constexpr int N = Sh::N;
  // the kernel arguments that the first loads need arrive with the first
  // batch of argument loads (one wait), not on demand one batch later
  asm volatile("" ::"s"(a.u), "s"(a.k), "s"(a.cu_seqlens), "s"(a.n_events), "s"(nw), "s"(S), "s"(a.D));
  const int d = blockIdx.x % a.dim;
  const int sp = blockIdx.x / a.dim;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / kSLN, s = lane % kSLN;  // s: the lane's first state, and its event slot in a block
  const int nslots = nw * kSLRows;
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;
  const int g_rows = (a.max_seqlen + Sh::Pass - 1) / Sh::Pass;

  const int64_t E = a.n_events;
  const __amdgpu_buffer_rsrc_t ru = buf_rsrc(a.u, E * SZ), rk = buf_rsrc(a.k, E * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(a.out, E * SZ);
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(a.z, HAS_Z ? E * SZ : 0), roz = buf_rsrc(a.out_z, HAS_Z ? E * SZ : 0);
  const __amdgpu_buffer_rsrc_t racc = buf_rsrc(a.acc, a.acc ? E * 4 : 0);  // empty: the stores are dropped

  // The slot's first channel leads the kernel's loads: the first events'
  // loads wait for its bounds alone, and their latency overlaps the rest of
  // the set-up (parameters, decay table). A ranked workgroup ranks first.
  const int slot = wave * kSLRows + grp;
  const int sorder = rank ? sl_slot_order(wave, grp, nw) : slot;
  if (rank) rank_channels(a, d, n_per_d, keys, sord, nw * kWave);
  auto chan_at = [&](int r0) {  // channel b of the slot in round r0 (n_per_d: none)
    const int v = r0 + sorder * S + sp;
    return v < n_per_d ? (rank ? sord[v] : v) : n_per_d;
  };
  auto channel = [&](int r0, int& e0, int& n) {  // unconditional loads (a clamped row), then selected
    const int b = chan_at(r0);
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    const int64_t cc = ch < NC ? ch : NC - 1;
    const int c0 = a.cu_seqlens[cc], c1 = a.cu_seqlens[cc + 1];
    e0 = b < n_per_d ? c0 : 0;
    n = b < n_per_d ? c1 - c0 : 0;
    report_seqlen(a, n);
  };
  int e0, n;
  channel(0, e0, n);

  const float al = sl_table_al<NL>(a, d);  // the table build waits for this load alone
  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  float Al[NL], wb[NL], cw[NL], rwc[NL];  // the lane's states s + 16j
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int64_t ix = (int64_t)d * N + s + kSLN * j;
    Al[j] = a.A[ix] * kLog2e;
    wb[j] = a.W_B[ix];
    const float wc = a.W_C[ix];
    cw[j] = wb[j] * wc;  // one state per lane: W_B W_C of the lane's own state
    rwc[j] = 1.0f / wc;
  }
  // One state per lane: the recurrence runs on the state's share of y,
  // q = W_B W_C g (q = a q + W_B W_C Δu², one DPP multiply and one fma per
  // event instead of a DPP move, an fma and a multiply), the saved states
  // being q / W_C. Only where every W_B W_C of the model channel and every
  // 1 / W_C lie within [1e-20, 1e20] in magnitude (finite, far from
  // underflow and overflow; uniform over the workgroup); else on g.
  const bool scaled = NL == 1 && __all(fabsf(cw[0]) >= 1e-20f && fabsf(cw[0]) <= 1e20f && fabsf(rwc[0]) <= 1e20f);
  const uint32_t rowb = sl_tab_lane(s, grp);

  // the loads of a channel's block round r
  auto off = [&](int e0, int bk) { return (uint32_t)(e0 + bk * kSLB + s); };
  float Un[kSLPF], Zn[kSLPF];
  int Kn[kSLPF];
  auto issue = [&](int e0, int r) {  // unconditional: the registers never merge with old values
#pragma unroll
    for (int t = 0; t < kSLPF; ++t) {
      Un[t] = buf_load<T>(ru, off(e0, r * kSLPF + t) * SZ);
      Kn[t] = buf_load_i32(rk, off(e0, r * kSLPF + t) * 4u);
      Zn[t] = HAS_Z ? buf_load<T>(rz, off(e0, r * kSLPF + t) * SZ) : 0.0f;
    }
  };
  issue(e0, 0);
  // a decay exponent that can be positive (A > 0 or Δ < 0): lane products
  // of decays are multiplied out instead of taken as exp2 of a Δ sum (a
  // wave's lanes hold all of A[d]; uniform over the workgroup)
  const bool exact = __any(al > 0.0f) || dti < 0.0f || dta < 0.0f;
  sl_build_table<NL>(sT, al, dti, dta, nw);
  __syncthreads();

  auto run = [&](auto exact_tag, auto scaled_tag) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    constexpr bool SC = decltype(scaled_tag)::value && NL == 1;
    // the lane's saved state h = W_B g from its recurrence variable
    auto state = [&](int j, float v) { return SC ? v * rwc[j] : v * wb[j]; };
    for (int r0 = 0; r0 + sp < n_per_d; r0 += nslots * S) {
      const int b = chan_at(r0);
      const bool act = b < n_per_d;
      const int64_t ch = (int64_t)d + (int64_t)b * dim;
      if (r0 > 0) {
        channel(r0, e0, n);
        issue(e0, 0);
      }
      const int nblk = (n + kSLB - 1) / kSLB;
      const int wblk = wave_max_dpp(nblk);
      // The lane's event of block bk is e0 + 16·bk + s (out of range past the
      // channel's end: the loads read the next channel's values or 0, unused).
      // Blocks go in rounds of kSLPF: a round's loads are issued when the round
      // before it starts, so each has a round of compute to arrive in.
      float g[NL], P[NL];
#pragma unroll
      for (int j = 0; j < NL; ++j) g[j] = 0.0f, P[j] = 1.0f;
      float sdl = 0.0f;
      auto block = [&](const int bk, const float uv, const int kk, const float zv) {
        const int i = bk * kSLB + s;
        const bool valid = i < n;
        // padding events are identities: Δ = 0 -> a = 1 (table entry 0), Δu² = 0
        const float dl = valid ? fmaf(dti, (float)(kk - 1), dta) : 0.0f;
        const float du2 = dl * uv * uv;
        const int big = valid && kk > Sh::Tab;
        sdl += dl;
        float av[NL][kSLB];
        tab16<NL>(av, sT, rowb, valid ? (uint32_t)min(kk, Sh::Tab) * Sh::Gap : 0u);
        if (__builtin_expect(__any(big), 0)) {  // gaps past the table: computed decays
          for16([&](auto q) {
            constexpr int Q = decltype(q)::value;
            const float dq = bcast_f<Q>(dl);  // row-uniform condition: lane Q of the row is active
            if (bcast_i<Q>(big)) {
#pragma unroll
              for (int j = 0; j < NL; ++j) av[j][Q] = decay(dq * Al[j]);
            }
          });
        }
        float wq[kSLN];  // one state per lane: W_B W_C g of the lane's state after each event
        for16([&](auto q) {
          constexpr int Q = decltype(q)::value;
          if constexpr (SC) {
            g[0] = fmaf(av[0][Q], g[0], cw[0] * bcast_f<Q>(du2));  // g holds W_B W_C g
            if (EXACT) P[0] *= av[0][Q];
            wq[Q] = g[0];
          } else if constexpr (NL == 1) {
            g[0] = fmaf(av[0][Q], g[0], bcast_f<Q>(du2));
            if (EXACT) P[0] *= av[0][Q];
            wq[Q] = cw[0] * g[0];
          } else {
            const float x = bcast_f<Q>(du2);
#pragma unroll
            for (int j = 0; j < NL; ++j) {
              g[j] = fmaf(av[j][Q], g[j], x);
              if (EXACT) P[j] *= av[j][Q];
            }
            float w = cw[0] * g[0];  // the lane's states' share of Σ_s W_B W_C g_s
#pragma unroll
            for (int j = 1; j < NL; ++j) w = fmaf(cw[j], g[j], w);
            wq[Q] = w;
          }
        });
        // Σ_s W_B W_C g_s of the lane's event: the row's lanes' shares
        // summed per event across the lanes (DPP)
        const float acc = row_reduce_scatter16(wq);
        const float y = fmaf(Dv, uv, uv * acc);
        const uint32_t eo = valid ? off(e0, bk) * SZ : kBufOOB;
        buf_store<T>(ro, eo, y);
        buf_store_f32(racc, valid ? off(e0, bk) * 4u : kBufOOB, acc);  // for the backward (dropped without acc)
        if (HAS_Z) buf_store<T>(roz, eo, y * (zv / (1.0f + __expf(-zv))));
        // saved states at the block end: x after every 2048 events and after
        // the channel's last one; chunk_g at every pass start
        const int cend = min(n, (bk + 1) * kSLB);
        const int xc = (cend - 1) / kXChunk;
        const bool xsave = bk < nblk && (cend % kXChunk == 0 || cend == n) && xc < nck;
        if (__any(xsave)) {
          const float sd = row_sum(sdl);
          if (xsave) {
#pragma unroll
            for (int j = 0; j < NL; ++j) {
              const float Pn = EXACT ? P[j] : decay(sd * Al[j]);
              reinterpret_cast<float2*>(a.x + (ch * nck + xc) * 2 * N)[s + kSLN * j] = make_float2(Pn, state(j, g[j]));
            }
          }
        }
        const int pend = (bk + 1) * kSLB;  // events before the next pass start, when it is one
        if (a.chunk_g && pend % Sh::Pass == 0 && pend < n && pend / Sh::Pass < g_rows) {
#pragma unroll
          for (int j = 0; j < NL; ++j) a.chunk_g[(ch * g_rows + pend / Sh::Pass) * N + s + kSLN * j] = state(j, g[j]);
        }
      };
      for (int r = 0; r * kSLPF < wblk; ++r) {
        float U[kSLPF], Z[kSLPF];
        int K[kSLPF];
#pragma unroll
        for (int t = 0; t < kSLPF; ++t) {
          U[t] = Un[t];
          K[t] = Kn[t];
          Z[t] = Zn[t];
        }
        issue(e0, r + 1);
#pragma unroll
        for (int t = 0; t < kSLPF; ++t)
          if (r * kSLPF + t < wblk) block(r * kSLPF + t, U[t], K[t], Z[t]);
      }
      // chunks past the channel's end keep the reference's zero state
      if (act) {
        for (int c = (n + kXChunk - 1) / kXChunk; c < nck; ++c) {
#pragma unroll
          for (int j = 0; j < 2 * NL; ++j) a.x[(ch * nck + c) * 2 * N + s + kSLN * j] = 0.0f;
        }
      }
    }
  };
  if (scaled) {
    if (exact) run(std::true_type{}, std::true_type{});
    else run(std::false_type{}, std::true_type{});
  } else {
    if (exact) run(std::true_type{}, std::false_type{});
    else run(std::false_type{}, std::false_type{});
  }
}

// nw: waves per workgroup, S: workgroups per model channel (the launch's
// shape, passed rather than read from blockDim / gridDim, whose loads would
// come before any other work); rank: rank the channels by length first
template <typename T, bool HAS_Z, int NL>
__global__ __launch_bounds__(kScanThreads) void k_scan_fwd_sl(const bcm_scan_args a, int nw, int S, int rank) {
  __shared__ float sT[SLShape<NL>::TabSz];
  __shared__ int sord[kSortMax];
  __shared__ int skeys[kSortMax];  // the ranking's scratch keys
  sl_fwd_body<T, HAS_Z, NL>(a, sT, sord, skeys, nw, S, rank);
}

// ----------------------------------------------------------------- backward
// A channel's passes of kSLPass events, last to first. Each pass rebuilds its
// states g (and decays a) in registers from the pass-start state the forward
// saved (phase A, blocks 0..1), then runs the adjoint backward through them
// (phase B, blocks 1..0): e_i = doutu_i + f, f = a_i e_i carried to the
// event before (and across passes). Per state: T0 = Σ tg, T1 = Σ tg·(k-1)
// with tg = f·g_{i-1}, and Σ e·Δu² (dW_B; dW_C is the same sum, since
// Σ_i dout_i u_i g_i = Σ_i e_i Δ_i u_i² over a channel). Per event lane:
// Σ_s W_B W_C g_s (phase A) and Σ_s W_B W_C e_s (phase B), summed over the
// row (see the file's head), then du, the Δ terms of ddt and dD.
constexpr int kSLRowCap = 512;  // events of one channel kept in LDS for its dense row

// Four steps t0..t0+3 of a channel's dense gradient row (the gather
// backward) from its du in LDS, in event order: each value is the next
// event's du masked by the step's bit (0 / -1), the LDS index advancing one
// slot per set bit. m: the tile's event mask, tv: the index of its first
// event, off = t0 % 64 (the lane's first step in the tile).
template <typename T>
__device__ __forceinline__ void dense_seg(T* dr, const float* sdu, int e0, uint64_t m, int32_t tv, int off, int t0) {
  const uint32_t lo_keep = off >= 32 ? 0xFFFFFFFFu : (1u << off) - 1u;
  const uint32_t hi_keep = off > 32 ? (1u << (off - 32)) - 1u : 0u;
  const uint32_t sh = (uint32_t)off & 31u;
  const uint32_t mlo = (uint32_t)m, mhi = (uint32_t)(m >> 32);
  int e = tv - e0 + (int)(__builtin_popcount(mlo & lo_keep) + __builtin_popcount(mhi & hi_keep));
  const uint32_t w = off >= 32 ? mhi : mlo;
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int32_t mk = __builtin_amdgcn_sbfe((int32_t)w, sh + (uint32_t)k, 1u);
    o[k] = __float_as_uint(sdu[min(max(e, 0), kSLRowCap - 1)]) & (uint32_t)mk;
    e -= mk;
  }
  if constexpr (sizeof(T) == 4) {
    st_stream(u32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<u32x4*>(dr + t0));
  } else {
    T h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = from_f<T>(__uint_as_float(o[k]));
    st_stream(*reinterpret_cast<u32x2*>(h), reinterpret_cast<u32x2*>(dr + t0));
  }
}

// Calls f(std::integral_constant<int, j>) for j = 0..NL-1.
template <int NL, typename F, int... J> __device__ __forceinline__ void forj_impl(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <int NL, typename F> __device__ __forceinline__ void forj(F&& f) {
  forj_impl<NL>(f, std::make_integer_sequence<int, NL>{});
}

// WR: the dense rows are written by the workgroup's row writers
// (sl_row_writer) as the passes finish; the waves here publish, per slot,
// the first event whose du is final in prog.
// The per-event sums over the row's states go by DPP reduce-scatter, not
// through an LDS transpose tile: config 3 scan backward 180 -> 177 us,
// config 2 39.0 -> 36.5 us (one compute wave per SIMD, where nothing hides
// the tile's round trips), config 1 cold step 136.3 -> 134.5 us once the
// reduce-scatter's first halvings needed no selects (before that, the tile
// won at config 1's two waves per SIMD: 38.6 against 39.1 us).
template <typename T, bool HAS_Z, bool DXR, int NL, bool WR>
__device__ __forceinline__ void sl_bwd_body(const bcm_scan_args& a, const ScanRows& rw, float* sT,
                                            float* sacc, float* sdu, int* sord, int* keys, int* prog, int nw, int S,
                                            int rank) {
  // no implicit fma contraction: the instantiations (with and without the
  // dense rows) round alike, so their gradients are bit-equal; fmas are
  // written out where they are meant
#pragma clang fp contract(off)
  static_assert(!DXR || NL == 1, "the dense rows are written by the one-state-per-lane kernel");
  static_assert(!WR || DXR, "row writers write dense rows");
  using Sh = SLShape<NL>;
  constexpr bool KEEPA = Sh::KeepA;
  constexpr uint32_t SZ = sizeof(T);
  constexpr int N = Sh::N;
  constexpr int NA = Sh::NA;  // accumulators per slot: dA, dW_B, dW_C, ddt_idle, ddt_active, dD
  // the arguments of the channel bounds' loads come in the first batch of
  // argument loads (more operands here cost scalar-register spills)
  asm volatile("" ::"s"(a.cu_seqlens), "s"(nw), "s"(S));
  constexpr int NB = Sh::Pass / kSLB;  // blocks per pass
  const int d = blockIdx.x % a.dim;
  const int sp = blockIdx.x / a.dim;
  const int nthr = nw * kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / kSLN, s = lane % kSLN;  // s: the lane's first state, and its event slot in a block
  const int slot = wave * kSLRows + grp, nslots = nw * kSLRows;
  const int NC = a.n_channels, dim = a.dim;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;
  const int g_rows = (a.max_seqlen + Sh::Pass - 1) / Sh::Pass;

  const float al = sl_table_al<NL>(a, d);  // first load of the kernel: the table build waits for it alone
  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  float Al[NL], wb[NL], wc[NL], wbcs[NL], wbca[NL];  // the lane's states s + 16j
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int64_t ix = (int64_t)d * N + s + kSLN * j;
    const float Av = a.A[ix];
    Al[j] = Av * kLog2e;
    wb[j] = a.W_B[ix];
    wc[j] = a.W_C[ix];
    wbcs[j] = wb[j] * wc[j];
    wbca[j] = wbcs[j] * Av;
  }
  const uint32_t rowb = sl_tab_lane(s, grp);

  for (int i = threadIdx.x; i < nslots * NA; i += nthr) sacc[i] = 0.0f;
  float* cacc = sacc + slot * NA;

  const int64_t E = a.n_events;
  const __amdgpu_buffer_rsrc_t ru = buf_rsrc(a.u, E * SZ), rk = buf_rsrc(a.k, E * 4);
  const __amdgpu_buffer_rsrc_t rdo = buf_rsrc(a.dout, E * SZ), rdu = buf_rsrc(a.du, a.du ? E * SZ : 0);  // no du: the dense rows alone (stores dropped)
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(a.z, HAS_Z ? E * SZ : 0), ros = buf_rsrc(a.out_saved, HAS_Z ? E * SZ : 0);
  const __amdgpu_buffer_rsrc_t rdz = buf_rsrc(a.dz, HAS_Z ? E * SZ : 0);
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.chunk_g, a.chunk_g ? a.chunk_g_bytes : 0);
  // the forward's per-event state sums: phase A then rebuilds the states
  // alone, without the transpose of each block (uniform over the launch)
  const bool use_acc = a.acc != nullptr;
  const __amdgpu_buffer_rsrc_t racc = buf_rsrc(a.acc, use_acc ? E * 4 : 0);

  // The lane's events of pass p: e0 + Pass·p + 16t + s (t < NB); loads past
  // the channel's end read the next channel's values or 0 and are unused.
  // A pass's loads are issued when the pass after it (in the walk: before
  // it) starts; unconditional, so the registers never merge with old values.
  float Un[NB], Dn[NB], Zn[NB], On[NB], Gn[NL], An[NB];
  int Kn[NB];
  auto issue = [&](int e0, int64_t ch, int p) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const uint32_t o = (uint32_t)(e0 + p * Sh::Pass + t * kSLB + s);
      Un[t] = buf_load<T>(ru, o * SZ);
      Kn[t] = buf_load_i32(rk, o * 4u);
      Dn[t] = buf_load<T>(rdo, o * SZ);
      An[t] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(racc, o * 4u, 0, 0));
      Zn[t] = HAS_Z ? buf_load<T>(rz, o * SZ) : 0.0f;
      On[t] = HAS_Z ? buf_load<T>(ros, o * SZ) : 0.0f;
    }
    // pass-start state h of pass p (chunk_g row p, written by the forward)
#pragma unroll
    for (int j = 0; j < NL; ++j)
      Gn[j] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
          rg, (uint32_t)(((ch * g_rows + p) * N + s + kSLN * j) * 4), 0, 0));
  };
  // a ranked workgroup ranks its channels first; the keys live in the
  // transpose tiles, which the zeroing above does not touch
  const int sorder = rank ? sl_slot_order(wave, grp, nw) : slot;
  if (rank) rank_channels(a, d, n_per_d, keys, sord, nthr);
  auto chan_at = [&](int r0) {  // channel b of the slot in round r0 (n_per_d: none)
    const int v = r0 + sorder * S + sp;
    return v < n_per_d ? (rank ? sord[v] : v) : n_per_d;
  };
  auto channel = [&](int r0, int& e0, int& n, int64_t& ch) {  // unconditional loads (a clamped row), then selected
    const int b = chan_at(r0);
    ch = (int64_t)d + (int64_t)b * dim;
    const int64_t cc = ch < NC ? ch : NC - 1;
    const int c0 = a.cu_seqlens[cc], c1 = a.cu_seqlens[cc + 1];
    e0 = b < n_per_d ? c0 : 0;
    n = b < n_per_d ? c1 - c0 : 0;
    report_seqlen(a, n);
  };
  int e0, n;
  int64_t ch;
  channel(0, e0, n, ch);
  // a single round with row writers: nothing final yet but the (vacuous)
  // events from n on; an idle slot has nothing to write
  if constexpr (WR) {
    if ((lane & (kSLN - 1)) == 0) prog[slot] = chan_at(0) < n_per_d ? n : 0;
  }
  // at least one pass: the dense rows of empty channels are written by it
  int wp = max(1, wave_max_dpp((n + Sh::Pass - 1) / Sh::Pass));
  issue(e0, ch, wp - 1);
  sl_build_table<NL>(sT, al, dti, dta, nw);
  __syncthreads();

  for (int r0 = 0; r0 + sp < n_per_d; r0 += nslots * S) {
    if (r0 > 0) {
      channel(r0, e0, n, ch);
      wp = max(1, wave_max_dpp((n + Sh::Pass - 1) / Sh::Pass));
      issue(e0, ch, wp - 1);
    }
    const bool act = chan_at(r0) < n_per_d;
    const int np = (n + Sh::Pass - 1) / Sh::Pass;
    float f[NL];  // a·e of the event after the current one
    float T0[NL], T1[NL], dWB[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) f[j] = T0[j] = T1[j] = dWB[j] = 0.0f;
    float ddti_l = 0.0f, ddta_l = 0.0f, dD_l = 0.0f;
    for (int p = wp - 1; p >= 0; --p) {
      float uv[NB], gg[NB], dl[NB], km[NB], du2[NB], doutu[NB], acc2[NB];
      uint32_t tb[NB];
      int big[NB];
      // the lane's own events of the pass: Δ, Δu², the gated dout (and dz)
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const int i = p * Sh::Pass + t * kSLB + s;
        const bool valid = i < n;
        const int kk = Kn[t];
        uv[t] = Un[t];
        float dv = Dn[t];
        if (HAS_Z) {
          const float zv = Zn[t], ov = On[t];
          const float sg = 1.0f / (1.0f + __expf(-zv));
          buf_store<T>(rdz, valid ? (uint32_t)(e0 + i) * SZ : kBufOOB, dv * ov * sg * (1.0f + zv * (1.0f - sg)));
          dv *= zv * sg;
        }
        gg[t] = dv;
        dl[t] = valid ? fmaf(dti, (float)(kk - 1), dta) : 0.0f;
        km[t] = valid ? (float)(kk - 1) : 0.0f;
        du2[t] = dl[t] * uv[t] * uv[t];
        doutu[t] = valid ? dv * uv[t] : 0.0f;
        tb[t] = valid ? (uint32_t)min(kk, Sh::Tab) * Sh::Gap : 0u;
        big[t] = valid && kk > Sh::Tab;
      }
#pragma unroll
      for (int t = 0; t < NB; ++t) acc2[t] = An[t];  // the forward's sums (0 without acc: replaced below)
      float g_in[NL];
#pragma unroll
      for (int j = 0; j < NL; ++j) g_in[j] = (p >= 1 && p < np && p < g_rows && wb[j] != 0.0f) ? Gn[j] / wb[j] : 0.0f;
      issue(e0, ch, p - 1);  // the next pass of the walk (past the start: unused)
      // decays of events Q0..Q0+H-1 of block t for the lane's states, from the
      // table or computed
      constexpr int H = Sh::H;
      auto decays = [&](float (&av)[NL][kSLB], int t, auto q0c) {
        constexpr int Q0 = decltype(q0c)::value;
        tabq<NL, Q0, H>(av, sT, rowb, tb[t]);
        if (__builtin_expect(__any(big[t]), 0)) {  // gaps past the table: computed decays
          forr<Q0, H>([&](auto q) {
            constexpr int Q = decltype(q)::value;
            const float dq = bcast_f<Q>(dl[t]);  // row-uniform condition: lane Q of the row is active
            if (bcast_i<Q>(big[t])) {
#pragma unroll
              for (int j = 0; j < NL; ++j) av[j][Q] = decay(dq * Al[j]);
            }
          });
        }
      };
      // ---- phase A: states (and decays) of the pass, Σ_s W_B W_C g_s per event
      // (USE: taken from the forward's sums instead; uniform, so the two forms
      // are separate code)
      float gb[Sh::Pass][NL], ab[KEEPA ? Sh::Pass : 1][NL];
      auto phase_a = [&](auto use_tag) {
        constexpr bool USE = decltype(use_tag)::value;
        float g[NL];
#pragma unroll
        for (int j = 0; j < NL; ++j) g[j] = g_in[j];
#pragma unroll
        for (int t = 0; t < NB; ++t) {
          float wq[kSLN];  // one state per lane: W_B W_C g of the lane's state after each event
          forr<0, kSLB / H>([&](auto hc) {
            constexpr int Q0 = decltype(hc)::value * H;
            float av[NL][kSLB];
            decays(av, t, std::integral_constant<int, Q0>{});
            forr<Q0, H>([&](auto q) {
              constexpr int Q = decltype(q)::value;
              if constexpr (NL == 1) {
                g[0] = fmaf(av[0][Q], g[0], bcast_f<Q>(du2[t]));
                gb[t * kSLB + Q][0] = g[0];
                ab[t * kSLB + Q][0] = av[0][Q];
                if constexpr (!USE) wq[Q] = wbcs[0] * g[0];
              } else {
                const float x = bcast_f<Q>(du2[t]);
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                  g[j] = fmaf(av[j][Q], g[j], x);
                  gb[t * kSLB + Q][j] = g[j];
                  if constexpr (KEEPA) ab[t * kSLB + Q][j] = av[j][Q];
                }
                if constexpr (!USE) {
                  float w = wbcs[0] * g[0];  // the lane's states' share of Σ_s W_B W_C g_s
#pragma unroll
                  for (int j = 1; j < NL; ++j) w = fmaf(wbcs[j], g[j], w);
                  wq[Q] = w;
                }
              }
            });
          });
          if constexpr (!USE) acc2[t] = row_reduce_scatter16(wq);  // the row's states summed per event (DPP)
        }
      };
      if (use_acc) phase_a(std::true_type{});
      else phase_a(std::false_type{});
      // ---- phase B: the adjoint, blocks and events last to first
#pragma unroll
      for (int tt = 0; tt < NB; ++tt) {
        const int t = NB - 1 - tt;
        float wq[kSLN];  // one state per lane: W_B W_C e of the lane's state at each event
        rforr<0, kSLB / H>([&](auto hc) {
        constexpr int Q0 = decltype(hc)::value * H;
        float av[KEEPA ? 1 : NL][kSLB];  // four states per lane: the block's decays read again
        if constexpr (!KEEPA) decays(av, t, std::integral_constant<int, Q0>{});
        rforr<Q0, H>([&](auto q) {
          constexpr int Q = decltype(q)::value;
          const int I = t * kSLB + Q;
          if constexpr (NL == 1) {
            const float e = f[0] + bcast_f<Q>(doutu[t]);
            f[0] = ab[I][0] * e;
            const float tg = f[0] * (I > 0 ? gb[I > 0 ? I - 1 : 0][0] : g_in[0]);
            T0[0] += tg;
            fmac_bcast<Q, Q == kSLB - 1>(T1[0], km[t], tg);   // T1 += (k-1)·tg
            fmac_bcast<Q, Q == kSLB - 1>(dWB[0], du2[t], e);  // dWB += Δu²·e
            wq[Q] = wbcs[0] * e;
          } else {
            const float dq = bcast_f<Q>(doutu[t]);
            float w = 0.0f;
            forj<NL>([&](auto jc) {
              constexpr int J = decltype(jc)::value;
              const float e = f[J] + dq;
              float aj;
              if constexpr (KEEPA) aj = ab[I][J];
              else aj = av[J][Q];
              f[J] = aj * e;
              const float tg = f[J] * (I > 0 ? gb[I > 0 ? I - 1 : 0][J] : g_in[J]);
              T0[J] += tg;
              fmac_bcast<Q, Q == kSLB - 1 && J == 0>(T1[J], km[t], tg);   // T1 += (k-1)·tg
              fmac_bcast<Q, Q == kSLB - 1 && J == 0>(dWB[J], du2[t], e);  // dWB += Δu²·e
              w = J == 0 ? wbcs[0] * e : fmaf(wbcs[J], e, w);
            });
            wq[Q] = w;
          }
        });
        });
        const float acc1 = row_reduce_scatter16(wq);  // the row's states summed per event (DPP)
        // the lane's own event of block t: du, the Δu² terms of ddt, dD
        const int i = p * Sh::Pass + t * kSLB + s;
        const float duv = fmaf(gg[t], Dv + acc2[t], 2.0f * dl[t] * uv[t] * acc1);
        const float dd = uv[t] * uv[t] * acc1;  // the A-term of dΔ goes into ddt through T0, T1
        ddti_l = fmaf(dd, km[t], ddti_l);
        ddta_l += dd;
        dD_l += doutu[t];
        const bool valid = i < n;
        buf_store<T>(rdu, valid ? (uint32_t)(e0 + i) * SZ : kBufOOB, duv);
        // the channel's du in event order, for its dense row (an understated
        // max_seqlen, flagged in the status word, must not spill into the
        // neighbouring slots' rows)
        if (DXR && valid && i < kSLRowCap) sdu[i] = duv;
      }
      if constexpr (WR) {
        // every du from event p·Pass on is in LDS: the writer may take the
        // tiles whose first event is there (the release orders the du
        // stores before the flag)
        if ((lane & (kSLN - 1)) == 0)
          __hip_atomic_store(&prog[slot], p * Sh::Pass, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    // the channel's parameter-gradient terms into the slot's accumulators
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      ddti_l = fmaf(wbca[j], T1[j], ddti_l);
      ddta_l = fmaf(wbca[j], T0[j], ddta_l);
    }
    ddti_l = row_sum(ddti_l);
    ddta_l = row_sum(ddta_l);
    dD_l = row_sum(dD_l);
    if (act) {
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const int m = s + kSLN * j;
        cacc[m] = fmaf(wbcs[j], fmaf(dti, T1[j], dta * T0[j]), cacc[m]);
        cacc[N + m] = fmaf(dWB[j], wc[j], cacc[N + m]);
        cacc[2 * N + m] = fmaf(dWB[j], wb[j], cacc[2 * N + m]);
      }
      if (s == 0) {
        cacc[3 * N] += ddti_l;
        cacc[3 * N + 1] += ddta_l;
        cacc[3 * N + 2] += dD_l;
      }
    }
    if constexpr (DXR && !WR) {
      // dense gradient row of the channel from its du in LDS (event order):
      // the row's 16 lanes take one 64-step tile per store, lane j writing
      // steps 4j..4j+3, each value the next event's du masked by the step's
      // bit (0 / -1), the LDS index advancing one slot per set bit
      wave_sync();
      if (act) {
        const uint32_t* mrow = rw.bitmask + (ch / rw.mrd) * rw.W;
        const int32_t* tsr = rw.ts + ch * (rw.nT + 1);
        T* dr = static_cast<T*>(rw.dx) + ch * rw.L;
        const int L = (int)rw.L;
        const int off = 4 * s;  // the lane's first step in a tile
        auto seg = [&](uint64_t m, int32_t tv, int t0) { dense_seg<T>(dr, sdu, e0, m, tv, off, t0); };
        const int nfull = L / kTile;  // tiles whose 64 steps are all < L
        constexpr int BAT = 8;
        int q0 = 0;
        for (; q0 + BAT <= nfull; q0 += BAT) {
          uint64_t m[BAT];
          int32_t tv[BAT];
#pragma unroll
          for (int i = 0; i < BAT; ++i) {  // masks and table entries in flight together
            m[i] = tile_mask(mrow, q0 + i);
            tv[i] = tsr[q0 + i];
          }
#pragma unroll
          for (int i = 0; i < BAT; ++i) seg(m[i], tv[i], (q0 + i) * kTile + off);
        }
        for (; q0 < nfull; ++q0) seg(tile_mask(mrow, q0), tsr[q0], q0 * kTile + off);
        // a last partial tile (L % 64 != 0; L % 4 == 0, so a lane's 4 steps
        // are all in range or all past the end)
        if (nfull * kTile < L && nfull * kTile + off < L) seg(tile_mask(mrow, nfull), tsr[nfull], nfull * kTile + off);
      }
      wave_sync();  // the du row is rewritten by the next round's channel
    }
  }
  // the workgroup's parameter gradients: slots summed in a fixed order
  __syncthreads();
  for (int i = threadIdx.x; i < NA; i += nthr) {
    float v = 0.0f;
    for (int sl = 0; sl < nslots; ++sl) v += sacc[sl * NA + i];
    if (S > 1) a.split_ws[((int64_t)sp * a.dim + d) * NA + i] = v;  // summed by k_scan_param_reduce
    else store_param_grad(a, d, N, i, v);
  }
}

// Dense-row writer of a single-round workgroup (one wave per SIMD beside
// the compute waves): writer k writes the rows of compute waves k and k + 4
// (the waves on its SIMD; the host uses writers with at most four compute
// waves, so only wave k), each tile as soon as the du of its events are in
// LDS, so the rows' 4 bytes per step leave during the adjoint loops instead
// of in a burst after them. A tile is ready when its first event is at or
// after the slot's published progress (every published value is a valid
// bound: each event from it on has its final du). Lane l writes steps
// 4(l % 16)..+3 of tile j0 + 4i + l / 16. The wait is bounded: after
// kRowWriterPolls empty polls the writer stops and flags the status word
// (BCM_SCAN_ROWS_INCOMPLETE), so every wave reaches the final barrier.
constexpr int kRowWriterPolls = 1 << 20;
constexpr int kRowWriterTiles = 64;  // most tiles per row (the lane of each tile's table entry)

template <typename T>
__device__ void sl_row_writer(const bcm_scan_args& a, const ScanRows& rw, const float* sdu_all, const int* prog,
                              int nw, int S) {
  constexpr int kC = 2 * kSLRows;  // the rows of two compute waves
  const int d = blockIdx.x % a.dim, sp = blockIdx.x / a.dim;
  const int wk = threadIdx.x / kWave - nw;
  const int lane = lane_id();
  const int NC = a.n_channels, dim = a.dim;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;
  const int L = (int)rw.L;
  const int nfull = L / kTile;
  const int ntile = nfull + (nfull * kTile < L ? 1 : 0);  // at most kRowWriterTiles (the host's condition)
  int hi[kC], e0c[kC];
  int32_t tsv[kC];  // lane j: the tile table entry j of the channel
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    const int w = wk + 4 * (c / kSLRows);
    const int v = (w * kSLRows + c % kSLRows) * S + sp;  // the slot's only channel
    const bool act = w < nw && v < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)(act ? v : 0) * dim;
    e0c[c] = act ? a.cu_seqlens[ch] : 0;
    hi[c] = act ? ntile : 0;  // tiles [0, hi) still to write
    tsv[c] = act && lane < ntile ? rw.ts[ch * (rw.nT + 1) + lane] : INT_MAX;
  }
  __syncthreads();  // the compute waves' set-up: decay table, progress initialised

  auto write_tiles = [&](int c, int j0, int j1) {
    const int w = wk + 4 * (c / kSLRows), slot = w * kSLRows + c % kSLRows;
    const int64_t ch = (int64_t)d + (int64_t)(slot * S + sp) * dim;
    const uint32_t* mrow = rw.bitmask + (ch / rw.mrd) * rw.W;
    const int32_t* tsr = rw.ts + ch * (rw.nT + 1);
    T* dr = static_cast<T*>(rw.dx) + ch * rw.L;
    const float* sdu = sdu_all + slot * kSLRowCap;
    const int sub = lane >> 4, off = 4 * (lane & 15);
    constexpr int BAT = 8;
    for (int jb = j0; jb < j1; jb += 4 * BAT) {
      uint64_t m[BAT];
      int32_t tv[BAT];
#pragma unroll
      for (int i = 0; i < BAT; ++i) {  // masks and table entries in flight together (clamped rows)
        const int jj = min(jb + 4 * i + sub, j1 - 1);
        m[i] = tile_mask(mrow, jj);
        tv[i] = tsr[jj];
      }
#pragma unroll
      for (int i = 0; i < BAT; ++i) {
        const int j = jb + 4 * i + sub;
        if (j < j1 && j * kTile + off < L) dense_seg<T>(dr, sdu, e0c[c], m[i], tv[i], off, j * kTile + off);
      }
    }
  };
  bool done = false;
  for (int it = 0; it < kRowWriterPolls && !done; ++it) {
    done = true;
    bool wrote = false;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      if (hi[c] == 0) continue;
      done = false;
      const int w = wk + 4 * (c / kSLRows);
      const int pg = __hip_atomic_load(&prog[w * kSLRows + c % kSLRows], __ATOMIC_ACQUIRE,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
      // the ready tiles of [0, hi) are a suffix (the table rises with j)
      const uint64_t ready = __ballot(lane < hi[c] && tsv[c] - e0c[c] >= pg);
      const int jlo = ready ? (int)__builtin_ctzll(ready) : hi[c];
      if (jlo < hi[c]) {
        write_tiles(c, jlo, hi[c]);
        hi[c] = jlo;
        wrote = true;
      }
    }
    if (!done && !wrote) __builtin_amdgcn_s_sleep(2);
  }
  if (!done && a.status && lane == 0) a.status[0] = BCM_SCAN_ROWS_INCOMPLETE;
  __syncthreads();  // the compute waves' final barrier
}

template <typename T, bool HAS_Z, bool DXR, int NL, bool WR = false>
__global__ __launch_bounds__(WR ? kScanThreads + 4 * kWave : kScanThreads) void k_scan_bwd_sl(
    const bcm_scan_args a, const ScanRows rw, int nw, int S, int rank) {
  __shared__ float sT[SLShape<NL>::TabSz];
  __shared__ float sacc[kScanThreads / kWave * kSLRows * SLShape<NL>::NA];
  __shared__ int sord[kSortMax];
  __shared__ int skeys[kSortMax];  // the ranking's scratch keys
  __shared__ int sprog[WR ? kScanThreads / kWave * kSLRows : 1];
  extern __shared__ float sdu[];  // DXR: [slots][kSLRowCap] each channel's du in event order
  const int wave = threadIdx.x / kWave, grp = lane_id() / kSLN;
  if constexpr (WR) {
    if (wave >= nw) {
      sl_row_writer<T>(a, rw, sdu, sprog, nw, S);
      return;
    }
  }
  // row writers need a single unranked round (the host's choice); rank 0
  // keeps the barrier count of both kinds of wave equal
  sl_bwd_body<T, HAS_Z, DXR, NL, WR>(a, rw, sT, sacc, sdu + (wave * kSLRows + grp) * kSLRowCap, sord, skeys, sprog,
                                     nw, S, WR ? 0 : rank);
}

// ------------------------------------------------------------------- host
// The process-wide family setting of bcm_set_scan_family: -1 until the first
// scan call, which takes it from BCM_SCAN_KERNEL ("lanes" / "items", else
// automatic). One setting for the process, not one per call: the family
// fixes chunk_g's pass length, which the forward and its backward share.
static std::atomic<int> g_scan_family{-1};

int scan_family() {
  int f = g_scan_family.load(std::memory_order_acquire);
  if (f < 0) {
    const char* v = std::getenv("BCM_SCAN_KERNEL");
    const int e = v && v[0] == 'l' ? BCM_SCAN_LANES : (v && v[0] == 'i' ? BCM_SCAN_ITEMS : BCM_SCAN_AUTO);
    int unset = -1;
    g_scan_family.compare_exchange_strong(unset, e, std::memory_order_acq_rel);
    f = g_scan_family.load(std::memory_order_acquire);
  }
  return f;
}

// Which family runs a depthwise scan of dstate 16, 32 or 64. The state lanes
// give one wave per four channels, so they pay when the channels fill every
// SIMD with at least one wave (config 2, 4096 channels on 256 CUs: 125-127
// against 130-131 µs per step; the forward is 2-3 µs slower there, the
// backward 5-7 µs faster); below that the lane groups of scan.hip, which
// split a channel over 16 lanes, keep more of the chip busy.
// bcm_set_scan_family forces either family (the tests run both on the same
// shapes); other dstates always take the lane groups.
bool sl_applies(const bcm_scan_args& a) {
  if (a.dstate != kSLN && a.dstate != 2 * kSLN && a.dstate != 4 * kSLN) return false;
  const int f = scan_family();
  if (f == BCM_SCAN_LANES) return true;
  if (f == BCM_SCAN_ITEMS) return false;
  return (int64_t)a.n_channels >= (int64_t)kSLRows * 4 * device_cus();
}

// Rank the channels by length when the stream is bursty (the longest
// channel more than twice the mean) and a model channel's channels fill
// more than one wave: the rows of a wave then end together.
static int sl_rank(const bcm_scan_args& a) {
  const int64_t per_d = (a.n_channels + a.dim - 1) / a.dim;
  if (per_d <= kSLRows || per_d > kSortMax || a.n_channels < 1) return 0;
  return 2 * a.n_events < (int64_t)a.max_seqlen * a.n_channels ? 1 : 0;
}

int sl_pass_len(int dstate) { return dstate == 4 * kSLN ? SLShape<4>::Pass : kSLPass; }

int sl_split(const bcm_scan_args& a) {
  const int per_d = (a.n_channels + a.dim - 1) / a.dim;
  const int nslots = (kScanThreads / kWave) * kSLRows;
  const int rounds = (per_d + nslots - 1) / nslots;
  const int cus = device_cus();
  if (a.dim < cus && rounds > 1) return std::min(rounds, std::max(1, cus / a.dim));
  return 1;
}

static int sl_waves(const bcm_scan_args& a) {
  const int per_d = (a.n_channels + a.dim - 1) / a.dim;
  const int nw = (per_d + kSLRows - 1) / kSLRows;
  return std::max(1, std::min(kScanThreads / kWave, nw));
}

template <int NL> static void sl_fwd_nl(const bcm_scan_args& a, hipStream_t st, dim3 grid, dim3 block, int nw, int S,
                                        int rank) {
  dispatch_dtype(a.dtype, [&](auto tag) {
    using T = decltype(tag);
    if (a.z) hipLaunchKernelGGL((k_scan_fwd_sl<T, true, NL>), grid, block, 0, st, a, nw, S, rank);
    else hipLaunchKernelGGL((k_scan_fwd_sl<T, false, NL>), grid, block, 0, st, a, nw, S, rank);
  });
}

int sl_launch_fwd(const bcm_scan_args& a, hipStream_t st, const char* fn) {
  const int S = sl_split(a), nw = sl_waves(a), rank = sl_rank(a);
  const dim3 grid((unsigned)((int64_t)a.dim * S)), block((unsigned)(nw * kWave));
  if (a.dstate == kSLN) sl_fwd_nl<1>(a, st, grid, block, nw, S, rank);
  else if (a.dstate == 2 * kSLN) sl_fwd_nl<2>(a, st, grid, block, nw, S, rank);
  else sl_fwd_nl<4>(a, st, grid, block, nw, S, rank);
  return check_launch(fn);
}

template <int NL> static void sl_bwd_nl(const bcm_scan_args& a, hipStream_t st, dim3 grid, dim3 block, int nw, int S,
                                        int rank, const ScanRows* rw) {
  const ScanRows rows = rw ? *rw : ScanRows{};
  dispatch_dtype(a.dtype, [&](auto tag) {
    using T = decltype(tag);
    if constexpr (NL == 1) {
      auto go = [&](auto z, auto dxr, auto wr, dim3 blk, size_t lds) {
        constexpr bool Z = decltype(z)::value, X = decltype(dxr)::value, W = decltype(wr)::value;
        hipLaunchKernelGGL((k_scan_bwd_sl<T, Z, X, 1, W>), grid, blk, lds, st, a, rows, nw, S, rank);
      };
      using Y = std::true_type;
      using F = std::false_type;
      if (rw) {
        const size_t lds = (size_t)nw * kSLRows * kSLRowCap * 4;
        // one unranked round of channels on rows of at most 64 tiles, one
        // compute wave per SIMD: row writers beside the compute waves (config
        // 2: scan backward 43.5 -> 41.2 us). With two compute waves per SIMD
        // the writers' work slows the adjoint loops more than the rows' burst
        // at the end costs (config 1: 42.5-42.8 -> 45.3-45.7 us, whatever the
        // writers' poll interval), so those shapes write the rows in-wave.
        const int64_t per_d = (a.n_channels + a.dim - 1) / a.dim;
        if (!rank && nw <= 4 && per_d <= (int64_t)nw * kSLRows * S && rows.nT <= kRowWriterTiles)
          go(F{}, Y{}, Y{}, dim3(block.x + 4 * kWave), lds);
        else
          go(F{}, Y{}, F{}, block, lds);
        return;
      }
      if (a.z) go(Y{}, F{}, F{}, block, 0);
      else go(F{}, F{}, F{}, block, 0);
    } else {
      if (a.z) hipLaunchKernelGGL((k_scan_bwd_sl<T, true, false, NL>), grid, block, 0, st, a, rows, nw, S, rank);
      else hipLaunchKernelGGL((k_scan_bwd_sl<T, false, false, NL>), grid, block, 0, st, a, rows, nw, S, rank);
    }
  });
}

int sl_launch_bwd(const bcm_scan_args& a, hipStream_t st, const char* fn, const ScanRows* rw) {
  int S = sl_split(a);
  // no (or too small a) workspace for the partials: one workgroup per model channel
  if (!a.split_ws || a.split_ws_bytes < 4 * (int64_t)S * a.dim * (3 * a.dstate + 3)) S = 1;
  const int nw = sl_waves(a), rank = sl_rank(a);
  const dim3 grid((unsigned)((int64_t)a.dim * S)), block((unsigned)(nw * kWave));
  if (rw && a.dstate != kSLN) return set_error(BCM_EINVAL, "%s: no fused dense rows for dstate %d", fn, a.dstate);
  if (a.dstate == kSLN) sl_bwd_nl<1>(a, st, grid, block, nw, S, rank, rw);
  else if (a.dstate == 2 * kSLN) sl_bwd_nl<2>(a, st, grid, block, nw, S, rank, rw);
  else sl_bwd_nl<4>(a, st, grid, block, nw, S, rank, rw);
  int rc = check_launch(fn);
  if (rc || S == 1) return rc;
  return sl_param_reduce(a, S, st, fn);
}

// The dense rows come from the kernel for channels whose events fit the
// LDS row (max_seqlen <= kSLRowCap), no z, 4-step aligned rows.
bool sl_rows_fusable(const bcm_scan_args& a, const bcm_scan_rows& r) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(r.dx);
  return a.dstate == kSLN && !a.z && a.max_seqlen <= kSLRowCap && r.seqlen % 4 == 0 &&
         p % (4 * dtype_size(a.dtype)) == 0;
}

}  // namespace bcm

extern "C" int bcm_set_scan_family(int family) {
  if (family != BCM_SCAN_AUTO && family != BCM_SCAN_LANES && family != BCM_SCAN_ITEMS) {
    bcm::set_error(BCM_EINVAL, "bcm_set_scan_family: unknown family %d", family);
    return -1;
  }
  const int prev = bcm::scan_family();
  bcm::g_scan_family.store(family, std::memory_order_release);
  return prev;
}
