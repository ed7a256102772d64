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
//   * The state loop is outermost: per state s every lane folds its R items
//     into a local (prod a, h) pair, the G lanes combine the pairs with an
//     inclusive scan, and a second register pass produces the exact states.
//     y (forward) and du / dΔ (backward) accumulate per item across states in
//     registers, so no per-event cross-lane reduction is needed.
//   * Decays come from a per-workgroup LDS table T[s][k] = exp2(clamp(Δ(k)·A
//     ·log2e)) for gaps k <= 64 (built with the same expression as the
//     per-event path, so the values are identical). In the backward, items
//     with a longer gap compute their own decay, state by state, with the
//     same expression; a forward chunk with one runs the exact path.
//   * Scaled recurrences: the forward runs g = h / W_B (g = a·g + Δu²) and the
//     backward e = dx / W_C (e = a'·e' + dout·u), so the per-item multiplies
//     by W_B / W_C leave the inner loops; they reappear once per state in the
//     products W_B·W_C, W_B·W_C·A and in the per-state gradient sums.
//   * A lane's product of decays is exp2(A·log2e·Σ Δ) (one transcendental per
//     lane and state instead of a multiply per item) when every exponent is
//     <= 0 (A <= 0 and Δ >= 0; then the clamp can only shift values below
//     2^-126); otherwise the workgroup multiplies the decays exactly.
//   * 16-lane groups scan with DPP row shifts (VALU, no LDS round trip);
//     wider groups use ds_bpermute shuffles.
//   * Chunks longer than one workgroup pass (max_seqlen > 2048 uses C = 2048,
//     the reference's chunk) carry (prod a, g) forward in LDS; the backward
//     starts each chunk from the saved state x[ch, c-1] like the reference and
//     carries a·e backward in LDS.
//   * No MFMA: the work is a first-order recurrence, not a contraction.
#include "bcm_common.hpp"
#include "scan_common.hpp"
#include "scan_group.hpp"

#include <algorithm>
#include <climits>
#include <type_traits>

namespace bcm {

struct FwdLds {
  int N, nw, G, R, nslots;
  bool tbl;
  int64_t bytes() const {
    (void)tbl;  // the decay table is static LDS
    return 4ll * (3ll * N + 2ll * nw * kWave * (R + 1) +
                  (int64_t)nslots * 2 * N);
  }
};

struct BwdLds {
  int N, nw, G, R, nslots;
  bool tbl;
  int64_t bytes() const {
    (void)tbl;  // the decay table is static LDS
    return 4ll * (6ll * N + 2ll * nw * kWave * (R + 1) +
                  (int64_t)nslots * (2 * N + 3 * N + 3));
  }
};

// Chunk staging: lane j of a G-lane group owns the R consecutive items
// j*R .. j*R+R-1 of the chunk. Global memory is read and written row by row
// (item q*G + j in step q: coalesced) and transposed through the group's LDS
// tile, where item i sits at i + i/R (lane stride R+1: conflict-free reads).
template <int R> __device__ __forceinline__ int tile_pos(int idx) { return idx + idx / R; }

// Byte offsets in a group's tile of the items q*G + j (q = 0..R-1) of lane j.
// They repeat with period P = R / gcd(G, R) in q, shifted by P*G + P*G/R
// slots, so P registers and immediate offsets cover all R of them.
template <int G, int R> struct TilePos {
  static constexpr int gcd(int a, int b) { return b ? gcd(b, a % b) : a; }
  static constexpr int P = R / gcd(G, R);
  static constexpr uint32_t STEP = 4u * (P * G + (P * G) / R);
  uint32_t base[P];
  __device__ __forceinline__ explicit TilePos(int j) {
#pragma unroll
    for (int t = 0; t < P; ++t) base[t] = 4u * (uint32_t)tile_pos<R>(t * G + j);
  }
  __device__ __forceinline__ float& at(float* tile, int q) const {
    return *reinterpret_cast<float*>(reinterpret_cast<char*>(tile) + base[q % P] + (uint32_t)(q / P) * STEP);
  }
};


template <int G, int R, typename T, bool HAS_Z, bool TBL>
__global__ __launch_bounds__((kScanThreadsG<G, false>)) void k_scan_fwd(const bcm_scan_args a, int sort_ch, int nw, int S) {
  using Ops = Grp<G>;
  constexpr int CPW = kWave / G;
  constexpr int C = G * R;
  constexpr int HR = R / 2;  // items per half chain
  static_assert(R % 2 == 0, "R must be even");
  constexpr uint32_t SZ = sizeof(T);
  const int N = a.dstate;
  // longest gap in the decay table (without a table tb only marks valid items)
  const int tabk = TBL ? tab_gaps(N) : kTabK;
  // S workgroups per model channel d (the grid is dim·S workgroups of nw
  // waves; both are arguments, not read from gridDim / blockDim, whose loads
  // would come first). A round covers nslots·S channels: the slot at
  // position pos of workgroup sp takes rank r0 + pos·S + sp of round r0
  // (chan_at below)
  asm volatile("" ::"s"(a.cu_seqlens), "s"(nw), "s"(S));  // in the first batch of argument loads
  const int d = blockIdx.x % a.dim;
  const int sp = blockIdx.x / a.dim;
  const int nthr = nw * kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / G, j = lane % G;
  const int nslots = nw * CPW;
  const int slot = wave * CPW + grp;

  // the decay table is static LDS: its address is a compile-time constant,
  // which the table reads take as their instruction offset
  __shared__ float sTab[TBL ? kTabElems : 1];
  __shared__ int sOrd[kSortMax];  // length order of the channels (sort_ch)
  extern __shared__ float smem[];
  float* sT = sTab;
  float* sAl = smem;
  float* sWB = sAl + N;
  float* sWBC = sWB + N;
  // the group's staging tiles for u and k (the u tile also stages y)
  float* tile = sWBC + N + wave * (kWave * (R + 1)) + grp * (G * (R + 1));
  float* tilek = tile + nw * kWave * (R + 1);
  float* mine = tile + j * (R + 1);  // this lane's R items
  float* minek = tilek + j * (R + 1);
  float* carry = sWBC + N + 2 * nw * kWave * (R + 1) + slot * 2 * N;  // [P_run(N), g_run(N)]

  // per-event arrays as buffer resources: items past a channel's events use
  // an out-of-range offset (loads read 0, stores are dropped)
  const int64_t E = a.n_events;
  const __amdgpu_buffer_rsrc_t ru = buf_rsrc(a.u, E * SZ), rk = buf_rsrc(a.k, E * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(a.out, E * SZ);
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(a.z, HAS_Z ? E * SZ : 0), roz = buf_rsrc(a.out_z, HAS_Z ? E * SZ : 0);
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;

  // Chunk loads, row by row (item q*G + j in step q, coalesced), written
  // into the tiles at their transposed positions (positions recomputed per
  // call: opaque() keeps them from being hoisted and held in registers). The
  // first chunk's loads are issued before the parameter set-up so their
  // latency overlaps it.
  // Items past the channel's events load the next channel's values (or 0
  // past E): they are padding, whose Δ the item set-up forces to 0, and
  // their outputs are never stored.
  float rawu[R];
  int rawk[R];
  const TilePos<G, R> tp(j);
  auto issue = [&](int e0, int n, int c) {
    (void)n;
    const uint32_t eb = (uint32_t)(e0 + c * C) + (uint32_t)opaque(j);
#pragma unroll
    for (int q = 0; q < R; ++q) {
      rawu[q] = buf_load<T>(ru, (eb + (uint32_t)(q * G)) * SZ);
      rawk[q] = buf_load_i32(rk, (eb + (uint32_t)(q * G)) * 4u);
    }
  };
  auto to_tiles = [&]() {
#pragma unroll
    for (int q = 0; q < R; ++q) {
      tp.at(tile, q) = rawu[q];
      tp.at(tilek, q) = __int_as_float(rawk[q]);
    }
  };
  auto channel = [&](int b, int& e0, int& n) {
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    e0 = act ? a.cu_seqlens[ch] : 0;
    n = act ? a.cu_seqlens[ch + 1] - e0 : 0;
    report_seqlen(a, n);
  };
  // Channel b of the slot at position p in round r0 (n_per_d: none). With
  // sort_ch the rank indexes the length order, so the S workgroups take
  // every S-th channel of it and a wave's groups take neighbouring lengths;
  // waves past the first half take positions in reverse, so the two waves
  // of a SIMD (w and w + 4 of 8) pair a long wave with a short one.
  const int hw = (nw + 1) / 2;
  const int pos = (wave < hw ? wave : nw - 1 - (wave - hw)) * CPW + grp;
  auto chan_at = [&](int r0, int p) {
    const int v = r0 + p * S + sp;
    return v < n_per_d ? (sort_ch ? sOrd[v] : v) : n_per_d;
  };
  static_assert(2 * kWave * (R + 1) >= kSortMax, "the staging tiles hold the ranking keys");
  if (sort_ch) rank_channels(a, d, n_per_d, reinterpret_cast<int*>(sWBC + N), sOrd, nthr);  // keys in the tiles
  int e0, n;
  const int b_step = nslots * S;
  channel(chan_at(0, pos), e0, n);
  if (sp < n_per_d) issue(e0, n, 0);

  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  for (int s = threadIdx.x; s < N; s += nthr) {
    const float wb = a.W_B[(int64_t)d * N + s];
    sAl[s] = a.A[(int64_t)d * N + s] * kLog2e;
    sWB[s] = wb;
    sWBC[s] = wb * a.W_C[(int64_t)d * N + s];
  }
  if (TBL) build_decay_table(sT, a, d, dti, dta, nthr);
  if (sp < n_per_d) to_tiles();
  const bool exact_blk = exact_products(sAl, N, dti, dta);  // also the barrier after the LDS set-up

  for (int r0 = 0; r0 + sp < n_per_d; r0 += b_step) {
    const int b = chan_at(r0, pos);
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    if (r0 > 0) channel(b, e0, n);
    const int nch = n > 0 ? (n + C - 1) / C : 0;
    const int wmax = wave_max_dpp(nch);
    for (int c = 0; c < wmax; ++c) {
      const int cnt = min(max(n - c * C, 0), C);
      const int nv = cnt - j * R;                 // events among this lane's R items
      const uint32_t eb = (uint32_t)(e0 + c * C);  // event index of the chunk's first item
      // x holds the state after each 2048-event chunk and after the
      // channel's last event, whatever the pass length C
      const int cend = min(n, (c + 1) * C);
      const int xc = (cend - 1) / kXChunk;
      const bool xsave = c < nch && (cend % kXChunk == 0 || cend == n) && xc < nck;
      if (r0 > 0 || c > 0) {
        issue(e0, n, c);
        to_tiles();
      }
      wave_sync();
      float dl[R], du2[R], acc[R];
      uint32_t tb[R];  // byte offset of the item's gap in a table row (0: padding)
      int big = 0;
      float Sa = 0.0f, Sb = 0.0f;  // Σ Δ of each half chain
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool valid = r < nv;
        const int kk = __float_as_int(minek[r]);
        // padding items are identities of the scan: Δ = 0 -> a = 1, Δu² = 0
        const int km1 = valid ? kk - 1 : -1;
        dl[r] = valid ? fmaf(dti, (float)km1, dta) : 0.0f;
        const float uv = mine[r];  // u stays in the tile (read again for the outputs)
        du2[r] = dl[r] * uv * uv;
        tb[r] = (uint32_t)(km1 + 1) * 4u;
        big |= km1 >= tabk ? 1 : 0;
        if (r < HR) Sa += dl[r];
        else Sb += dl[r];
        acc[r] = 0.0f;
      }
      // ---- state loop. EXACT: decays computed per item, products multiplied
      // out. Otherwise decays come from the table, and the next state's reads
      // are issued before this state's second pass (two register buffers).
      auto state = [&](int s, float (&av)[R], float (&avn)[R], auto exact_tag) {
        constexpr bool EXACT = decltype(exact_tag)::value;
        const float Al = sAl[s], wbc = sWBC[s];
        // two independent half chains (items 0..HR-1 and HR..R-1), interleaved
        // for instruction-level parallelism and joined with the scan operator
        float Pa = 1.0f, Ha = 0.0f, Pb = 1.0f, Hb = 0.0f;
#pragma unroll
        for (int i = 0; i < HR; ++i) {
          if (EXACT) {
            av[i] = decay(dl[i] * Al);
            av[i + HR] = decay(dl[i + HR] * Al);
          }
          Ha = fmaf(av[i], Ha, du2[i]);
          Hb = fmaf(av[i + HR], Hb, du2[i + HR]);
          if (EXACT) {
            Pa *= av[i];
            Pb *= av[i + HR];
          }
        }
        if (!EXACT) {
          Pa = decay(Sa * Al);
          Pb = decay(Sb * Al);
        }
        float P = Pa * Pb, H = fmaf(Pb, Ha, Hb);
        Ops::scan_up(P, H);
        const float g0 = c > 0 ? carry[N + s] : 0.0f;
        const float P0 = c > 0 ? carry[s] : 1.0f;
        const float gend = fmaf(P, g0, H);
        const float gin = Ops::prev(gend, g0);
        if (!EXACT) {
          const int sn = s + 1 < N ? s + 1 : s;
          const uint32_t row = (uint32_t)__builtin_amdgcn_readfirstlane(sn * (tabk + 1) * 4);
#pragma unroll
          for (int r = 0; r < R; ++r) avn[r] = tab(sT, row, tb[r]);
        }
        float ga = gin, gb = fmaf(Pa, gin, Ha);
#pragma unroll
        for (int i = 0; i < HR; ++i) {
          ga = fmaf(av[i], ga, du2[i]);
          gb = fmaf(av[i + HR], gb, du2[i + HR]);
          acc[i] = fmaf(ga, wbc, acc[i]);
          acc[i + HR] = fmaf(gb, wbc, acc[i + HR]);
        }
        if (j == G - 1 && c < nch) {
          const float Pn = P0 * P;
          carry[s] = Pn;
          carry[N + s] = gend;
          if (xsave) reinterpret_cast<float2*>(a.x + (ch * nck + xc) * 2 * N)[s] = make_float2(Pn, gend * sWB[s]);
          // chunk_g has one row per pass of a max_seqlen-long channel: a
          // longer channel (reported through a.status) has no row for its
          // later passes
          const int g_rows = (a.max_seqlen + C - 1) / C;
          if (a.chunk_g && c + 1 < nch && c + 1 < g_rows) a.chunk_g[(ch * g_rows + c + 1) * N + s] = gend * sWB[s];
        }
      };
      auto states = [&](auto exact_tag) {
        constexpr bool EXACT = decltype(exact_tag)::value;
        float av0[R], av1[R];
        if (!EXACT) {
#pragma unroll
          for (int r = 0; r < R; ++r) av0[r] = tab(sT, 0u, tb[r]);
        }
#pragma unroll 1
        for (int s = 0; s < N; s += 2) {
          state(s, av0, av1, exact_tag);
          if (s + 1 < N) state(s + 1, av1, av0, exact_tag);
        }
      };
      // a chunk with a gap longer than the table (rare: 0.85^64 per event
      // at 15 % density) runs the exact path
      if constexpr (TBL) {
        if (exact_blk || __any(big)) states(std::true_type{});
        else states(std::false_type{});
      } else {
        states(std::true_type{});
      }
      // ---- outputs: y = D·u + u·Σ_s g·W_B·W_C (and y·silu(z)), stored row by row
      wave_sync();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float uv = mine[r];
        mine[r] = fmaf(Dv, uv, uv * acc[r]);
      }
      wave_sync();
      {
        const int jo = opaque(j);
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int idx = q * G + jo;
          const uint32_t off = idx < cnt ? (eb + idx) * SZ : kBufOOB;
          const float yv = tp.at(tile, q);
          buf_store<T>(ro, off, yv);
          if (HAS_Z) {
            const float zv = buf_load<T>(rz, off);
            buf_store<T>(roz, off, yv * (zv / (1.0f + __expf(-zv))));
          }
        }
      }
      if (a.acc) {  // the per-event state sums for a backward that reuses them (uniform)
        const __amdgpu_buffer_rsrc_t racc = buf_rsrc(a.acc, E * 4);
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r) mine[r] = acc[r];
        wave_sync();
        const int jo = opaque(j);
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int idx = q * G + jo;
          buf_store_f32(racc, idx < cnt ? (eb + idx) * 4u : kBufOOB, tp.at(tile, q));
        }
      }
      wave_sync();  // the tile and the carry (written by lane G-1) are reused in the next chunk
    }
    // chunks past the channel's end keep the reference's zero state
    if (act) {
      for (int c = (n + kXChunk - 1) / kXChunk; c < nck; ++c)
        for (int s = j; s < 2 * N; s += G) a.x[(ch * nck + c) * 2 * N + s] = 0.0f;
    }
  }
}

template <int G, int R, typename T, bool HAS_Z, bool TBL, bool DXR>
__global__ __launch_bounds__((kScanThreadsG<G, true>)) void k_scan_bwd(const bcm_scan_args a, const ScanRows rw, int nw, int S) {
  using Ops = Grp<G>;
  constexpr int CPW = kWave / G;
  constexpr int RS = R + 1;
  constexpr int C = G * R;
  constexpr int HR = R / 2;  // items per half chain
  static_assert(R % 2 == 0, "R must be even");
  constexpr uint32_t SZ = sizeof(T);
  const int N = a.dstate;
  // longest gap in the decay table (without a table tb only marks valid items)
  const int tabk = TBL ? tab_gaps(N) : kTabK;
  // S workgroups per model channel d (the grid is dim·S workgroups of nw
  // waves; both are arguments, not read from gridDim / blockDim, whose loads
  // would come first). A round covers nslots·S channels: the slot at
  // position pos of workgroup sp takes rank r0 + pos·S + sp of round r0
  // (chan_at below)
  asm volatile("" ::"s"(a.cu_seqlens), "s"(nw), "s"(S));  // in the first batch of argument loads
  const int d = blockIdx.x % a.dim;
  const int sp = blockIdx.x / a.dim;
  const int nthr = nw * kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int grp = lane / G, j = lane % G;
  const int nslots = nw * CPW;
  const int slot = wave * CPW + grp;
  const int NA = 3 * N + 3;  // accumulators per slot: dA, dW_B, dW_C, ddt_idle, ddt_active, dD

  // the decay table is static LDS: its address is a compile-time constant,
  // which the table reads take as their instruction offset
  __shared__ float sTab[TBL ? kTabElems : 1];
  extern __shared__ float smem[];
  float* sT = sTab;
  float* sAl = smem;
  float* sWB = sAl + N;
  float* sWC = sWB + N;
  float* sWBC = sWC + N;
  float* sWBCA = sWBC + N;
  float* sA = sWBCA + N;
  // per lane, stride R+1 (conflict-free): the group's staging tile (u, dout
  // and outputs in transposed order), and the items' gap k-1 (0 for padding)
  float* tile = sA + N + wave * (kWave * RS) + grp * (G * RS);
  float* gg = tile + j * RS;
  float* tilek = tile + nw * kWave * RS;  // the k tile; then k-1 per lane
  float* gkm = tilek + j * RS;
  float* sdx = sA + N + 2 * nw * kWave * RS;  // [nslots][N] a·e carried to the previous chunk
  float* sg0 = sdx + nslots * N;              // [nslots][N] g at the chunk start
  float* sacc = sg0 + nslots * N;             // [nslots][NA]
  float* cdx = sdx + slot * N;
  float* cg0 = sg0 + slot * N;
  float* cacc = sacc + slot * NA;

  const int64_t E = a.n_events;
  const __amdgpu_buffer_rsrc_t ru = buf_rsrc(a.u, E * SZ), rk = buf_rsrc(a.k, E * 4);
  const __amdgpu_buffer_rsrc_t rdo = buf_rsrc(a.dout, E * SZ), rdu = buf_rsrc(a.du, a.du ? E * SZ : 0);  // no du: the dense rows alone (stores dropped)
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(a.z, HAS_Z ? E * SZ : 0), ros = buf_rsrc(a.out_saved, HAS_Z ? E * SZ : 0);
  const __amdgpu_buffer_rsrc_t rdz = buf_rsrc(a.dz, HAS_Z ? E * SZ : 0);
  const int NC = a.n_channels, dim = a.dim, nck = a.n_chunks;
  const int n_per_d = d < NC ? (NC - d + dim - 1) / dim : 0;

  // Chunk loads, row by row (item q*G + j in step q, coalesced): k and u go
  // to their tiles at the transposed positions (opaque(): positions are not
  // hoisted and held in registers); they are issued one chunk ahead (the
  // first before the parameter set-up, the next after a chunk's last use of
  // the tiles), so their latency overlaps other work. dout is loaded with
  // them and held in registers until the chunk's set-up has read u; it then
  // goes through the u tile.
  // Items past the channel's events load the next channel's values (or 0
  // past E): they are padding, whose Δ and dout·u the item set-up forces to
  // 0, and their outputs are never stored.
  float rawu[R], rawd[R];
  int rawk[R];
  const TilePos<G, R> tp(j);
  auto issue = [&](int e0, int n, int c) {
    (void)n;
    const uint32_t eb = (uint32_t)(e0 + c * C) + (uint32_t)opaque(j);
#pragma unroll
    for (int q = 0; q < R; ++q) {
      rawk[q] = buf_load_i32(rk, (eb + (uint32_t)(q * G)) * 4u);
      rawu[q] = buf_load<T>(ru, (eb + (uint32_t)(q * G)) * SZ);
      rawd[q] = buf_load<T>(rdo, (eb + (uint32_t)(q * G)) * SZ);
    }
  };
  auto to_tiles = [&]() {
#pragma unroll
    for (int q = 0; q < R; ++q) {
      tp.at(tilek, q) = __int_as_float(rawk[q]);
      tp.at(tile, q) = rawu[q];
    }
  };
  auto channel = [&](int b, int& e0, int& n) {
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    e0 = act ? a.cu_seqlens[ch] : 0;
    n = act ? a.cu_seqlens[ch + 1] - e0 : 0;
    report_seqlen(a, n);
  };
  // Channel b of the slot at position p in round r0 (n_per_d: none): the
  // forward's slot positions, taken in channel order (the forward's length
  // order measured about 3 % slower here on bursty channels)
  const int hw = (nw + 1) / 2;
  const int pos = (wave < hw ? wave : nw - 1 - (wave - hw)) * CPW + grp;
  auto chan_at = [&](int r0, int p) {
    const int v = r0 + p * S + sp;
    return v < n_per_d ? v : n_per_d;
  };
  int e0, n;
  const int b_step = nslots * S;
  channel(chan_at(0, pos), e0, n);
  int nch = n > 0 ? (n + C - 1) / C : 0;
  int wmax = wave_max_dpp(nch);
  if (sp < n_per_d && wmax > 0) issue(e0, n, wmax - 1);

  const float dti = a.dt_idle[d], dta = a.dt_active[d];
  const float Dv = a.D ? a.D[d] : 0.0f;
  for (int s = threadIdx.x; s < N; s += nthr) {
    const float Av = a.A[(int64_t)d * N + s];
    const float wb = a.W_B[(int64_t)d * N + s], wc = a.W_C[(int64_t)d * N + s];
    sA[s] = Av;
    sAl[s] = Av * kLog2e;
    sWB[s] = wb;
    sWC[s] = wc;
    sWBC[s] = wb * wc;
    sWBCA[s] = wb * wc * Av;
  }
  for (int i = threadIdx.x; i < nslots * NA; i += nthr) sacc[i] = 0.0f;
  if (TBL) build_decay_table(sT, a, d, dti, dta, nthr);
  if (sp < n_per_d && wmax > 0) to_tiles();
  const bool exact_blk = exact_products(sAl, N, dti, dta);  // also the barrier after the LDS set-up

  for (int r0 = 0; r0 + sp < n_per_d; r0 += b_step) {
    const int b = chan_at(r0, pos);
    const bool act = b < n_per_d;
    const int64_t ch = (int64_t)d + (int64_t)b * dim;
    // e0, n, nch, wmax describe this channel, and the loads of its last
    // chunk are in the tiles and rawd: issued before the loop or at the end
    // of the previous channel, so raw registers never span a state loop
    float ddti_l = 0.0f, ddta_l = 0.0f, dD_l = 0.0f;
    for (int c = wmax - 1; c >= 0; --c) {
      const bool cact = c < nch;
      const int cnt = min(max(n - c * C, 0), C);
      const int nv = cnt - j * R;
      const uint32_t eb = (uint32_t)(e0 + c * C);
      // chunk-start state in g = h / W_B form from the h the forward saved:
      // chunk_g (pass-start h, row c) or x (2048-event passes: h after the
      // previous chunk, row c - 1); the source is uniform, one code path
      if (c > 0) {
        const bool pg = a.chunk_g != nullptr;
        const float* src = pg ? a.chunk_g : a.x_saved + 1;
        const int64_t rows = pg ? (a.max_seqlen + C - 1) / C : nck;
        const int64_t row = c - (pg ? 0 : 1);
        const int64_t rstride = pg ? N : 2 * N, sstride = pg ? 1 : 2;
        for (int s = j; s < N; s += G) {
          const float h0 = (cact && row < rows) ? src[(ch * rows + row) * rstride + s * sstride] : 0.0f;
          const float wb = sWB[s];
          cg0[s] = wb != 0.0f ? h0 / wb : 0.0f;
        }
      }
      float du2[R], doutu[R], acc1[R], acc2[R];
      // Δ of each item (0 for padding), kept for the state loop's computed
      // decays where registers allow (the 16-item shapes of up to 32 lanes;
      // 8 items must stay within 128 VGPRs for their fourth wave per SIMD);
      // the others recompute it from k-1 in LDS
      constexpr bool kKeepDl = R == 16 && G <= 32;
      float dlx[kKeepDl ? R : 1];
      uint32_t tb[R];  // byte offset of the item's gap k in a table row (4k; 0: padding)
      int big = 0;
      float Sa = 0.0f, Sb = 0.0f, dl0 = 0.0f, dlh = 0.0f;
      {
        // ---- k (-> k-1 in place) and u from their tiles, then the gated
        // dout through the u tile (dz on the way)
        const int jo = opaque(j);
        float dlv[R], uvv[R];
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const bool valid = r < nv;
          const int kk = __float_as_int(gkm[r]);
          // with the fix-up, gaps past the table read its last entry and the
          // state loop replaces it; without it such a chunk runs the exact path
          tb[r] = valid ? (uint32_t)(R >= kFixMinR ? min(kk, tabk) : kk) * 4u : 0u;
          dlv[r] = valid ? fmaf(dti, (float)(kk - 1), dta) : 0.0f;
          if constexpr (kKeepDl) dlx[r] = dlv[r];
          gkm[r] = valid ? (float)(kk - 1) : 0.0f;
          big |= (valid && kk > tabk) ? (1 << r) : 0;
          if (r < HR) Sa += dlv[r];
          else Sb += dlv[r];
          uvv[r] = gg[r];
        }
        dl0 = dlv[0];
        dlh = dlv[HR];
        wave_sync();
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int idx = q * G + jo;
          const uint32_t off = idx < cnt ? (eb + idx) * SZ : kBufOOB;
          float dv = rawd[q];
          if (HAS_Z) {
            const float zv = buf_load<T>(rz, off);
            const float ov = buf_load<T>(ros, off);
            const float sg = 1.0f / (1.0f + __expf(-zv));
            buf_store<T>(rdz, off, dv * ov * sg * (1.0f + zv * (1.0f - sg)));
            dv *= zv * sg;
          }
          tp.at(tile, q) = dv;
          rawd[q] = 0.0f;  // consumed: not live into the state loop on any path
        }
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r) {
          du2[r] = dlv[r] * uvv[r] * uvv[r];
          doutu[r] = r < nv ? gg[r] * uvv[r] : 0.0f;
          acc1[r] = 0.0f;
          acc2[r] = 0.0f;
        }
        wave_sync();  // the staged dout is read; the tile is free until the per-item pass
      }
      // Σ Δ over each half chain's items, and over the items that follow
      // them (the next lane's first; nothing past the chunk: its carry
      // already holds a·e)
      const float S1a = Sa - dl0 + dlh;
      const float S1b = Sb - dlh + Ops::next(dl0, 0.0f);
      // the state loop reads gkm through an index the compiler cannot see
      // through, so it re-reads LDS instead of keeping the stored values live
      const float* km = gkm + opaque(0);
      // items with a gap longer than the table (k > tabk) compute their
      // decays directly, state by state, on the table path; bigm is the
      // wave-uniform set of item slots that hold one in some lane (shapes
      // without the fix-up: nonzero when some lane holds one)
      const uint32_t bigm =
          R >= kFixMinR ? (uint32_t)__builtin_amdgcn_readfirstlane(wave_or(big)) : (uint32_t)__any(big);
      wave_sync();  // cg0 written by the group's lanes
      // ---- state loop; EXACT: decays computed per item, products multiplied out
      // mode: 0 table, 1 table with the long-gap fix-up, 2 exact
      auto states = [&](auto mode_tag) {
        constexpr int MODE = decltype(mode_tag)::value;
        constexpr bool EXACT = MODE == 2;
#pragma unroll 1
        for (int s = 0; s < N; ++s) {
          const float Al = sAl[s], wbc = sWBC[s], wbca = sWBCA[s];
          const uint32_t row = (uint32_t)__builtin_amdgcn_readfirstlane(s * (tabk + 1) * 4);
          const float g0 = c > 0 ? cg0[s] : 0.0f;
          const float ec = (c < nch - 1) ? cdx[s] : 0.0f;
          float av[R];
          // Each lane's R items run as two independent half chains (items
          // 0..HR-1 and HR..R-1), interleaved for instruction-level
          // parallelism and joined with the scan operator.
          // forward: local folds, group scan, exact states (in registers)
          float Pa = 1.0f, Ha = 0.0f, Pb = 1.0f, Hb = 0.0f;
          if (!EXACT) {
#pragma unroll
            for (int r = 0; r < R; ++r) av[r] = tab(sT, row, tb[r]);
            if constexpr (MODE == 1) {
#pragma unroll
              for (int r = 0; r < R; ++r)
                if ((bigm & (1u << r)) && tb[r] && km[r] >= (float)tabk)
                  av[r] = decay((kKeepDl ? dlx[kKeepDl ? r : 0] : fmaf(dti, km[r], dta)) * Al);
            }
          }
#pragma unroll
          for (int i = 0; i < HR; ++i) {
            const int ra = i, rb = i + HR;
            if (EXACT) {
              if constexpr (kKeepDl) {
                av[ra] = decay(dlx[ra] * Al);
                av[rb] = decay(dlx[rb] * Al);
              } else {
                av[ra] = decay((tb[ra] ? fmaf(dti, km[ra], dta) : 0.0f) * Al);
                av[rb] = decay((tb[rb] ? fmaf(dti, km[rb], dta) : 0.0f) * Al);
              }
            }
            Ha = fmaf(av[ra], Ha, du2[ra]);
            Hb = fmaf(av[rb], Hb, du2[rb]);
            if (EXACT) {
              Pa *= av[ra];
              Pb *= av[rb];
            }
          }
          if (!EXACT) {
            Pa = decay(Sa * Al);
            Pb = decay(Sb * Al);
          }
          float P = Pa * Pb, H = fmaf(Pb, Ha, Hb);
          Ops::scan_up(P, H);
          const float gin = Ops::prev(fmaf(P, g0, H), g0);
          float gs[R];  // the exact states of this state's items (registers only)
          {
            float ga = gin, gb = fmaf(Pa, gin, Ha);
#pragma unroll
            for (int i = 0; i < HR; ++i) {
              ga = fmaf(av[i], ga, du2[i]);
              gb = fmaf(av[i + HR], gb, du2[i + HR]);
              gs[i] = ga;
              gs[i + HR] = gb;
            }
          }
          // reverse: e_i = dout_i·u_i + a_{i+1}·e_{i+1}   (dx = W_C·e)
          const float anext = Ops::next(av[0], 1.0f);  // the chunk carry already holds a_next·e_next
          float Qa = 1.0f, Cea = 0.0f, Qb = 1.0f, Ceb = 0.0f;
#pragma unroll
          for (int i = 0; i < HR; ++i) {
            const int ra = HR - 1 - i, rb = R - 1 - i;
            const float ala = av[ra + 1];
            const float alb = (rb == R - 1) ? anext : av[rb + 1];
            Cea = fmaf(ala, Cea, doutu[ra]);
            Ceb = fmaf(alb, Ceb, doutu[rb]);
            if (EXACT) {
              Qa *= ala;
              Qb *= alb;
            }
          }
          if (!EXACT) {
            Qa = decay(S1a * Al);
            Qb = decay(S1b * Al);
          }
          float Q = Qa * Qb, Ce = fmaf(Qa, Ceb, Cea);
          Ops::scan_down(Q, Ce);
          const float ein = Ops::next(fmaf(Q, ec, Ce), ec);
          float eb = ein, ea = fmaf(Qb, ein, Ceb);  // ea starts from e at item HR
          // tg = dx·a·h_prev / (W_B·W_C); with Δ = dt_idle·(k-1) + dt_active the
          // Δ-weighted sums need only T0 = Σ tg and T1 = Σ tg·(k-1)
          float T0a = 0.0f, T1a = 0.0f, dWBa = 0.0f, dWCa = 0.0f;
          float T0b = 0.0f, T1b = 0.0f, dWBb = 0.0f, dWCb = 0.0f;
#pragma unroll
          for (int i = 0; i < HR; ++i) {
            const int ra = HR - 1 - i, rb = R - 1 - i;
            const float ala = av[ra + 1];
            const float alb = (rb == R - 1) ? anext : av[rb + 1];
            const float gra = gs[ra], grb = gs[rb];
            const float gpa = ra > 0 ? gs[ra - 1] : gin;
            const float gpb = gs[rb - 1];
            ea = fmaf(ala, ea, doutu[ra]);
            eb = fmaf(alb, eb, doutu[rb]);
            acc1[ra] = fmaf(ea, wbc, acc1[ra]);       // Σ_s dx·W_B
            acc1[rb] = fmaf(eb, wbc, acc1[rb]);
            acc2[ra] = fmaf(gra, wbc, acc2[ra]);      // Σ_s h·W_C
            acc2[rb] = fmaf(grb, wbc, acc2[rb]);
            const float tga = ea * (av[ra] * gpa);
            const float tgb = eb * (av[rb] * gpb);
            T0a += tga;
            T0b += tgb;
            T1a = fmaf(tga, km[ra], T1a);
            T1b = fmaf(tgb, km[rb], T1b);
            dWBa = fmaf(ea, du2[ra], dWBa);
            dWBb = fmaf(eb, du2[rb], dWBb);
            dWCa = fmaf(doutu[ra], gra, dWCa);
            dWCb = fmaf(doutu[rb], grb, dWCb);
          }
          const float e = ea;  // e of item 0
          const float T0 = T0a + T0b, T1 = T1a + T1b;
          float dWB_l = dWBa + dWBb, dWC_l = dWCa + dWCb;
          if (j == 0 && cact) cdx[s] = av[0] * e;
          // dΔ_i gets Σ_s dx·a·h_prev·A: its ddt sums take T0, T1 lane by lane
          ddta_l = fmaf(wbca, T0, ddta_l);
          ddti_l = fmaf(wbca, T1, ddti_l);
          float dA_l = Ops::sum(fmaf(dti, T1, dta * T0));
          dWB_l = Ops::sum(dWB_l);
          dWC_l = Ops::sum(dWC_l);
          if (j == 0 && cact) {
            cacc[s] += dA_l * wbc;
            cacc[N + s] += dWB_l * sWC[s];
            cacc[2 * N + s] += dWC_l * sWB[s];
          }
        }
      };
      using Table = std::integral_constant<int, 0>;
      using TableFix = std::integral_constant<int, 1>;
      using Exact = std::integral_constant<int, 2>;
      // the fix-up pays per marked slot and state: with many marked slots
      // (bursty events with long gaps) the exact path is cheaper
      if constexpr (TBL && R >= kFixMinR) {
        if (exact_blk || __builtin_popcount(bigm) > kFixSlots) states(Exact{});
        else if (bigm) states(TableFix{});
        else states(Table{});
      } else if constexpr (TBL) {
        if (exact_blk || bigm) states(Exact{});
        else states(Table{});
      } else {
        states(Exact{});
      }
      // ---- per item: du, dΔ -> ddt, dD. The gated dout is still in the u
      // tile from the set-up (the state loop does not touch it); u is loaded
      // again and staged through the k tile once k-1 is in registers.
      wave_sync();
      {
        const int jo = opaque(j);
        float uvv[R], fu[R], kmr[R];
#pragma unroll
        for (int q = 0; q < R; ++q) fu[q] = buf_load<T>(ru, (eb + (uint32_t)(q * G + jo)) * SZ);
#pragma unroll
        for (int r = 0; r < R; ++r) kmr[r] = gkm[r];
        wave_sync();
#pragma unroll
        for (int q = 0; q < R; ++q) tp.at(tilek, q) = fu[q];
        wave_sync();
#pragma unroll
        for (int r = 0; r < R; ++r) uvv[r] = gkm[r];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float uv = uvv[r];
          const float km1 = kmr[r];
          const float dlr = tb[r] ? fmaf(dti, km1, dta) : 0.0f;
          const float duv = fmaf(gg[r], Dv + acc2[r], 2.0f * dlr * uv * acc1[r]);
          const float dd = uv * uv * acc1[r];  // the A-term of dΔ went into ddt in the state loop
          ddti_l = fmaf(dd, km1, ddti_l);
          ddta_l += dd;
          dD_l += doutu[r];
          gg[r] = duv;
        }
        wave_sync();
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int idx = q * G + jo;
          const float v = tp.at(tile, q);
          buf_store<T>(rdu, idx < cnt ? (eb + idx) * SZ : kBufOOB, v);
          if constexpr (DXR) tilek[q * G + j] = v;  // du in event order for the dense row
        }
      }
      if (c > 0) {  // the previous chunk's loads, now that the tiles are free
        wave_sync();
        issue(e0, n, c - 1);
        to_tiles();
      }
      wave_sync();  // cdx (LDS) written by lane 0, read by the group in the previous chunk
    }
    ddti_l = Ops::sum(ddti_l);
    ddta_l = Ops::sum(ddta_l);
    dD_l = Ops::sum(dD_l);
    if (j == 0 && act) {
      cacc[3 * N] += ddti_l;
      cacc[3 * N + 1] += ddta_l;
      cacc[3 * N + 2] += dD_l;
    }
    if constexpr (DXR) {
      // dense gradient row of the channel (one pass: all of its du are in
      // the group's k tile in event order). Each 16 lanes of the group take
      // one 64-step tile per store, lane j writing steps 4(j%16)..+3 of it
      // (TPS tiles per group store), taking its events from the tile's mask
      // and the tile table; 0 between events
      constexpr int TPS = G / 16;
      static_assert(G == 16 || G == 32, "one or two tiles per group store");
      wave_sync();
      if (act) {
        // row and lane constants formed here (opaque: not hoisted into
        // registers that would stay live across the state loop)
        const int64_t row = (int64_t)d + (int64_t)chan_at(r0, opaque(pos)) * dim;
        const uint32_t* mrow = rw.bitmask + (row / rw.mrd) * rw.W;
        const int32_t* tsr = rw.ts + row * (rw.nT + 1);
        T* dr = static_cast<T*>(rw.dx) + row * rw.L;
        const int L = (int)rw.L;
        const int jo = opaque(j);
        const int jt = jo / 16;        // the lane's tile within a group store
        const int off = 4 * (jo % 16);  // the lane's first step in a tile
        const uint32_t lo_keep = off >= 32 ? 0xFFFFFFFFu : (1u << off) - 1u;
        const uint32_t hi_keep = off > 32 ? (1u << (off - 32)) - 1u : 0u;
        const uint32_t sh = (uint32_t)off & 31u;
        const int elo = -e0, ehi = C;  // local event index = table entry - e0, clamped to the tile region
        // one tile: 4 steps, each value the next event's du masked by the
        // step's bit (sign-extended 0 / -1), the LDS address advancing by
        // one slot per set bit; the clamp keeps every read inside the
        // group's region of C + G slots
        auto seg = [&](uint64_t m, int32_t tv, int t0) {
          const uint32_t mlo = (uint32_t)m, mhi = (uint32_t)(m >> 32);
          int e = tv + elo + (int)(__builtin_popcount(mlo & lo_keep) + __builtin_popcount(mhi & hi_keep));
          e = min(max(e, 0), ehi);
          const uint32_t w = off >= 32 ? mhi : mlo;
          uint32_t o[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int32_t mk = __builtin_amdgcn_sbfe((int32_t)w, sh + (uint32_t)k, 1u);
            o[k] = __float_as_uint(tilek[e]) & (uint32_t)mk;
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
        };
        const int nfull = L / kTile;  // tiles whose 64 steps are all < L
        if constexpr (TPS == 1) {
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
        } else {
        constexpr int BAT = 8 / TPS;  // group stores per batch
        const int ngs = (nfull + TPS - 1) / TPS;  // group stores over the full tiles
        // tile of group store g for this lane; past the full tiles it reads
        // the last full tile and stores nothing
        auto tile_of = [&](int g) { return g * TPS + jt; };
        int g0 = 0;
        for (; g0 + BAT <= ngs; g0 += BAT) {
          uint64_t m[BAT];
          int32_t tv[BAT];
#pragma unroll
          for (int i = 0; i < BAT; ++i) {  // masks and table entries in flight together
            const int qt = min(tile_of(g0 + i), nfull - 1);
            m[i] = tile_mask(mrow, qt);
            tv[i] = tsr[qt];
          }
#pragma unroll
          for (int i = 0; i < BAT; ++i)
            if (tile_of(g0 + i) < nfull) seg(m[i], tv[i], tile_of(g0 + i) * kTile + off);
        }
        for (; g0 < ngs; ++g0) {
          const int qt = tile_of(g0);
          if (qt < nfull) seg(tile_mask(mrow, qt), tsr[qt], qt * kTile + off);
        }
        }
        // a last partial tile (L % 64 != 0; L % 4 == 0, so a lane's 4 steps
        // are all in range or all past the end), by the group's first 16 lanes
        if (jt == 0 && nfull * kTile < L && nfull * kTile + off < L)
          seg(tile_mask(mrow, nfull), tsr[nfull], nfull * kTile + off);
      }
    }
    if (r0 + b_step + sp < n_per_d) {  // the next round of this workgroup
      channel(chan_at(r0 + b_step, pos), e0, n);
      nch = n > 0 ? (n + C - 1) / C : 0;
      wmax = wave_max_dpp(nch);
      if (wmax > 0) {
        wave_sync();
        issue(e0, n, wmax - 1);
        to_tiles();
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NA; i += nthr) {
    float v = 0.0f;
    for (int sl = 0; sl < nslots; ++sl) v += sacc[sl * NA + i];
    if (S > 1) a.split_ws[((int64_t)sp * a.dim + d) * NA + i] = v;  // summed by k_scan_param_reduce
    else store_param_grad(a, d, N, i, v);
  }
}

// Parameter gradients of S workgroups per model channel: the S partials of
// each value summed in split order (deterministic).
__global__ __launch_bounds__(256) void k_scan_param_reduce(const bcm_scan_args a, int S) {
  const int N = a.dstate, NA = 3 * N + 3;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)a.dim * NA) return;
  const int d = (int)(t / NA), i = (int)(t % NA);
  float v = 0.0f;
  for (int s0 = 0; s0 < S; s0 += 8) {  // 8 loads in flight, summed in split order
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = s0 + j < S ? a.split_ws[((int64_t)(s0 + j) * a.dim + d) * NA + i] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < S) v += q[j];
  }
  store_param_grad(a, d, N, i, v);
}

// ------------------------------------------------------------ host dispatch
int sl_param_reduce(const bcm_scan_args& a, int S, hipStream_t s, const char* fn) {
  const int64_t tot = (int64_t)a.dim * (3 * a.dstate + 3);
  hipLaunchKernelGGL(k_scan_param_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a, S);
  return check_launch(fn);
}

struct Plan {
  int nw;      // waves per workgroup
  int64_t lds; // dynamic LDS bytes
  int S;       // workgroups per model channel
};

template <int G, int R, typename T, bool Z, bool BWD, bool TBL, bool DXR>
static int launch(const bcm_scan_args& a, hipStream_t s, const char* fn, Plan* query, const ScanRows* rw) {
  constexpr int CPW = kWave / G;
  const int per_d = (a.n_channels + a.dim - 1) / a.dim;
  int nw = (per_d + CPW - 1) / CPW;
  constexpr int kMaxW = kScanThreadsG<G, BWD> / kWave;
  nw = nw < 1 ? 1 : (nw > kMaxW ? kMaxW : nw);
  // the per-workgroup limit covers static and dynamic LDS together
  hipFuncAttributes fa{};
  const void* kfn = BWD ? reinterpret_cast<const void*>(&k_scan_bwd<G, R, T, Z, TBL, DXR>)
                        : reinterpret_cast<const void*>(&k_scan_fwd<G, R, T, Z, TBL>);
  if (hipFuncGetAttributes(&fa, kfn) != hipSuccess) return set_error(BCM_EHIP, "%s: hipFuncGetAttributes failed", fn);
  const int64_t cap = max_lds_bytes() - (int64_t)fa.sharedSizeBytes;
  int64_t lds = 0;
  for (;;) {
    lds = BWD ? BwdLds{a.dstate, nw, G, R, nw * CPW, TBL}.bytes() : FwdLds{a.dstate, nw, G, R, nw * CPW, TBL}.bytes();
    if (lds <= cap || nw == 1) break;
    --nw;
  }
  if (lds > cap) return set_error(BCM_EINVAL, "%s: dstate %d needs %lld bytes of LDS (> %lld)", fn, a.dstate,
                                  (long long)lds, (long long)cap);
  // fewer model channels than CUs and several rounds of channels each:
  // split each model channel's rounds over S workgroups
  const int rounds = (per_d + nw * CPW - 1) / (nw * CPW);
  const int cus = device_cus();
  int S = 1;
  if (a.dim < cus && rounds > 1) S = std::min(rounds, std::max(1, cus / a.dim));
  if (query) {
    *query = Plan{nw, lds, S};
    return BCM_OK;
  }
  // no (or too small a) workspace for the partials: one workgroup per model channel
  if (BWD && (!a.split_ws || a.split_ws_bytes < 4 * (int64_t)S * a.dim * (3 * a.dstate + 3))) S = 1;
  const dim3 grid((unsigned)((int64_t)a.dim * S));
  // forward over channels of several passes: each workgroup ranks its model
  // channel's channels by length, so the groups of a wave (and the
  // workgroups of one model channel) get channels of similar pass counts
  const int sort_ch = !BWD && per_d > 1 && per_d <= kSortMax && a.max_seqlen > G * R;
  if (BWD) {
    hipLaunchKernelGGL((k_scan_bwd<G, R, T, Z, TBL, DXR>), grid, dim3(nw * kWave), (size_t)lds, s, a,
                       rw ? *rw : ScanRows{}, nw, S);
    int rc = check_launch(fn);
    if (rc || S == 1) return rc;
    const int64_t tot = (int64_t)a.dim * (3 * a.dstate + 3);
    hipLaunchKernelGGL(k_scan_param_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a, S);
  } else {
    hipLaunchKernelGGL((k_scan_fwd<G, R, T, Z, TBL>), grid, dim3(nw * kWave), (size_t)lds, s, a, sort_ch, nw, S);
  }
  return check_launch(fn);
}

// Lane-group shape (G lanes x R items per pass of a channel), by a cost
// model in item slots: a single pass of C >= max_seqlen costs C per channel;
// passes of C < max_seqlen (C dividing 2048, so x's chunk ends fall on pass
// ends) cost about (mean/C + 1/2) passes of C per channel. Each pass of a
// state also pays the group scans, sums and lane products, about
// kLaneCost items' worth of VALU per lane, i.e. kLaneCost * G slots.
// Multi-pass shapes shorter than 2048 events need chunk_g in the backward.
enum ShapeId { S16x4, S16x8, S16x16, S16x24, S32x16, S64x4, S64x8, S64x16, S64x32 };
constexpr int kShapeG[] = {16, 16, 16, 16, 32, 64, 64, 64, 64};
constexpr int kShapeR[] = {4, 8, 16, 24, 16, 4, 8, 16, 32};
constexpr double kLaneCost = 6.0;

static ShapeId pick_shape(const bcm_scan_args& a) {
  const int m = a.max_seqlen;
  const bool tbl = a.dstate <= kTabMaxN;
  const double mean = (double)a.n_events / (a.n_channels > 0 ? a.n_channels : 1);
  static const ShapeId tab_shapes[] = {S16x4, S16x8, S16x16, S16x24, S32x16, S64x16, S64x32};
  static const ShapeId plain_shapes[] = {S64x4, S64x8, S64x16, S64x32};
  const ShapeId* cand = tbl ? tab_shapes : plain_shapes;
  const int ncand = tbl ? 7 : 4;
  ShapeId best = cand[ncand - 1];
  double best_cost = 1e300;
  for (int i = 0; i < ncand; ++i) {
    const int C = kShapeG[cand[i]] * kShapeR[cand[i]];
    const double pass = C + kLaneCost * kShapeG[cand[i]];
    double cost;
    if (m <= C) {
      cost = pass;                                             // one pass per channel
    } else {
      if (kXChunk % C != 0) continue;                          // multi-pass needs C | 2048
      cost = (mean / C + 0.5) * pass;
    }
    if (cost < best_cost) {
      best_cost = cost;
      best = cand[i];
    }
  }
  return best;
}

static void chunking(const bcm_scan_args& a, int* pass_len, int* n_pass, int* needs_chunk_g) {
  const ShapeId id = pick_shape(a);
  const int C = sl_applies(a) ? sl_pass_len(a.dstate) : kShapeG[id] * kShapeR[id];
  *pass_len = C;
  *n_pass = a.max_seqlen > 0 ? (a.max_seqlen + C - 1) / C : 1;
  *needs_chunk_g = (*n_pass > 1 && C < kXChunk) ? 1 : 0;
}

// The fused dense-row backward exists for the single-pass 16-lane shapes
// without z (the model's event path); rows_fusable() says when it applies.
template <int G, int R, typename T, bool Z, bool BWD, bool TBL>
static int launch_any(const bcm_scan_args& a, hipStream_t s, const char* fn, Plan* q, const ScanRows* rw) {
  if constexpr (BWD && !Z && (G == 16 || G == 32)) {
    if (rw) return launch<G, R, T, Z, BWD, TBL, true>(a, s, fn, q, rw);
  }
  if (rw) return set_error(BCM_EINVAL, "%s: no fused dense-row backward for this shape", fn);
  return launch<G, R, T, Z, BWD, TBL, false>(a, s, fn, q, nullptr);
}

template <typename T, bool Z, bool BWD>
static int dispatch_shape(const bcm_scan_args& a, hipStream_t s, const char* fn, Plan* q = nullptr,
                          const ScanRows* rw = nullptr) {
  const ShapeId id = pick_shape(a);
  switch (id) {
    case S16x4: return launch_any<16, 4, T, Z, BWD, true>(a, s, fn, q, rw);
    case S16x8: return launch_any<16, 8, T, Z, BWD, true>(a, s, fn, q, rw);
    case S16x16: return launch_any<16, 16, T, Z, BWD, true>(a, s, fn, q, rw);
    case S16x24: return launch_any<16, 24, T, Z, BWD, true>(a, s, fn, q, rw);
    case S32x16: return launch_any<32, 16, T, Z, BWD, true>(a, s, fn, q, rw);
    case S64x4: return launch_any<64, 4, T, Z, BWD, false>(a, s, fn, q, rw);
    case S64x8: return launch_any<64, 8, T, Z, BWD, false>(a, s, fn, q, rw);
    default: break;
  }
  const bool tbl = a.dstate <= kTabMaxN;
  if (id == S64x16)
    return tbl ? launch_any<64, 16, T, Z, BWD, true>(a, s, fn, q, rw)
               : launch_any<64, 16, T, Z, BWD, false>(a, s, fn, q, rw);
  return tbl ? launch_any<64, 32, T, Z, BWD, true>(a, s, fn, q, rw)
             : launch_any<64, 32, T, Z, BWD, false>(a, s, fn, q, rw);
}

// True when bcm_scan_bwd_rows can write the dense rows from the scan kernel:
// a 16-lane shape whose one pass holds every channel, no z, 4-step aligned
// rows.
static bool rows_fusable(const bcm_scan_args& a, const bcm_scan_rows& r) {
  if (sl_applies(a)) return sl_rows_fusable(a, r);
  const ShapeId id = pick_shape(a);
  if ((kShapeG[id] != 16 && kShapeG[id] != 32) || a.max_seqlen > kShapeG[id] * kShapeR[id] || a.z) return false;
  const uintptr_t p = reinterpret_cast<uintptr_t>(r.dx);
  return r.seqlen % 4 == 0 && p % (4 * dtype_size(a.dtype)) == 0;
}

template <bool BWD>
static int scan_entry(const bcm_scan_args* ap, bcm_stream_t stream, const char* fn, const ScanRows* rw = nullptr) {
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
  // per-event arrays are addressed with 32-bit buffer offsets
  if (a.n_events * 4 > INT32_MAX) return set_error(BCM_EINVAL, "%s: per-event arrays must be below 2 GiB", fn);
  if (!a.cu_seqlens || !a.dt_idle || !a.dt_active || !a.A || !a.W_B || !a.W_C)
    return set_error(BCM_EINVAL, "%s: null input pointer", fn);
  if (a.n_events > 0 && (!a.u || !a.k)) return set_error(BCM_EINVAL, "%s: null u/k pointer", fn);
  if (a.chunk_g) {
    int pass_len, n_pass, needs_g;
    chunking(a, &pass_len, &n_pass, &needs_g);
    if (a.chunk_g_pass != pass_len)
      return set_error(BCM_EINVAL,
                       "%s: chunk_g is laid out for passes of %d events, this scan runs passes of %d (size it "
                       "with bcm_scan_chunking under the scan family of both the forward and the backward)",
                       fn, a.chunk_g_pass, pass_len);
    const int64_t need = 4ll * a.n_channels * n_pass * a.dstate;
    if (a.chunk_g_bytes < need)
      return set_error(BCM_EINVAL, "%s: chunk_g needs %lld bytes (n_channels x %d passes x dstate floats)", fn,
                       (long long)need, n_pass);
  }
  const bool z = a.z != nullptr;
  if (!BWD) {
    if (!a.x || (a.n_events > 0 && !a.out)) return set_error(BCM_EINVAL, "%s: null output pointer", fn);
    if (z && a.n_events > 0 && !a.out_z) return set_error(BCM_EINVAL, "%s: out_z required with z", fn);
  } else {
    if (!a.dA || !a.dW_B || !a.dW_C || !a.ddt_idle || !a.ddt_active)
      return set_error(BCM_EINVAL, "%s: null gradient pointer", fn);
    // du may be NULL when the kernel writes the dense rows itself (rw): the
    // rows then carry the only copy of it
    if (a.n_events > 0 && (!a.dout || (!a.du && !rw))) return set_error(BCM_EINVAL, "%s: null dout/du pointer", fn);
    int pass_len, n_pass, needs_g;
    chunking(a, &pass_len, &n_pass, &needs_g);
    if (needs_g && !a.chunk_g)
      return set_error(BCM_EINVAL, "%s: chunk_g required (passes of %d events; run the forward with chunk_g)", fn,
                       pass_len);
    if (n_pass > 1 && !a.chunk_g && !a.x_saved) return set_error(BCM_EINVAL, "%s: x required for multi-chunk", fn);
    if (z && a.n_events > 0 && (!a.out_saved || !a.dz))
      return set_error(BCM_EINVAL, "%s: out and dz required with z", fn);
  }
  const hipStream_t s = hs(stream);
  if (sl_applies(a)) return BWD ? sl_launch_bwd(a, s, fn, rw) : sl_launch_fwd(a, s, fn);
  int rc = BCM_OK;
  dispatch_dtype(a.dtype, [&](auto tag) {
    using T = decltype(tag);
    rc = z ? dispatch_shape<T, true, BWD>(a, s, fn, nullptr, rw) : dispatch_shape<T, false, BWD>(a, s, fn, nullptr, rw);
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

// bcm_scan_bwd_rows' argument checks; *fused: whether it runs as one kernel.
static int rows_plan(const bcm_scan_args* args, const bcm_scan_rows* rows, const char* fn, bool* fused) {
  if (!args || !rows) return bcm::set_error(BCM_EINVAL, "%s: null argument", fn);
  const bcm_scan_rows& r = *rows;
  if (r.seqlen < 0 || r.mask_row_div < 1) return bcm::set_error(BCM_EINVAL, "%s: invalid seqlen / mask_row_div", fn);
  if (args->n_channels >= 1 && r.seqlen > 0) {
    if (!r.bitmask || !r.tile_start || !r.dx) return bcm::set_error(BCM_EINVAL, "%s: null index / dx pointer", fn);
    if ((reinterpret_cast<uintptr_t>(r.bitmask) & 7) != 0)
      return bcm::set_error(BCM_EINVAL, "%s: bitmask must be 8-byte aligned", fn);
  }
  *fused = args->n_channels >= 1 && r.seqlen > 0 && bcm::dtype_ok(args->dtype) && bcm::rows_fusable(*args, r);
  return BCM_OK;
}

int bcm_scan_bwd_rows_fused(const bcm_scan_args* args, const bcm_scan_rows* rows) {
  bool fused = false;
  const int rc = rows_plan(args, rows, "bcm_scan_bwd_rows_fused", &fused);
  return rc ? -rc : (fused ? 1 : 0);
}

int bcm_scan_bwd_rows(const bcm_scan_args* args, const bcm_scan_rows* rows, bcm_stream_t stream) {
  const char* fn = "bcm_scan_bwd_rows";
  bool fused = false;
  if (const int rc = rows_plan(args, rows, fn, &fused)) return rc;
  const bcm_scan_rows& r = *rows;
  if (!fused) {
    // two steps: the scan backward, then the rows from du
    if (args->n_events > 0 && !args->du)
      return bcm::set_error(BCM_EINVAL, "%s: du required where the rows are written from it in a second pass", fn);
    int rc = bcm::scan_entry<true>(args, stream, fn);
    if (rc) return rc;
    return bcm_gather_bwd_rows(args->du, args->dtype, r.bitmask, r.mask_row_div, r.tile_start, args->n_channels,
                               r.seqlen, r.dx, stream);
  }
  const bcm::ScanRows rw{r.bitmask, r.mask_row_div, bcm::bitmask_words(r.seqlen), r.tile_start,
                         bcm::tile_count(r.seqlen), r.seqlen, r.dx};
  return bcm::scan_entry<true>(args, stream, fn, &rw);
}

int64_t bcm_scan_bwd_workspace_bytes(const bcm_scan_args* args) {
  if (!args || !bcm::dtype_ok(args->dtype) || args->dim < 1 || args->dstate < 1 || args->dstate > 256 ||
      args->n_channels < 1)
    return 0;
  if (bcm::sl_applies(*args)) {
    const int S = bcm::sl_split(*args);
    return S > 1 ? 4 * (int64_t)S * args->dim * (3 * args->dstate + 3) : 0;
  }
  bcm::Plan q{1, 0, 1};
  int rc = BCM_OK;
  const bool z = args->z != nullptr;
  bcm::dispatch_dtype(args->dtype, [&](auto tag) {
    using T = decltype(tag);
    rc = z ? bcm::dispatch_shape<T, true, true>(*args, nullptr, "bcm_scan_bwd_workspace_bytes", &q)
           : bcm::dispatch_shape<T, false, true>(*args, nullptr, "bcm_scan_bwd_workspace_bytes", &q);
  });
  if (rc || q.S <= 1) return 0;
  return 4 * (int64_t)q.S * args->dim * (3 * args->dstate + 3);
}

int bcm_scan_chunking(const bcm_scan_args* args, int32_t* pass_len, int32_t* n_pass, int32_t* needs_chunk_g) {
  if (!args || !pass_len || !n_pass || !needs_chunk_g)
    return bcm::set_error(BCM_EINVAL, "bcm_scan_chunking: null argument");
  int p, q, r;
  bcm::chunking(*args, &p, &q, &r);
  *pass_len = p;
  *n_pass = q;
  *needs_chunk_g = r;
  return BCM_OK;
}

}  // extern "C"
