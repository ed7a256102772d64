// Lane-group scans shared by the scan kernels: G consecutive lanes of a
// wave hold one channel's chunk and combine per-lane scan pairs.
#pragma once
#include "bcm_common.hpp"

namespace bcm {

// ------------------------------------------------------------ lane groups
// The G lanes of a group hold one channel's chunk. Scan pairs compose as
// (P1, H1)∘(P2, H2) = (P1·P2, P2·H1 + H2) (selective_scan_common.h:156-161).
template <int G> struct Grp {  // generic width: ds_bpermute shuffles
  static __device__ __forceinline__ int j() { return lane_id() % G; }
  static __device__ __forceinline__ void scan_up(float& P, float& H) {  // inclusive, lanes 0..j
    const int jj = j();
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
      const float Pp = __shfl_up(P, o, G), Hp = __shfl_up(H, o, G);
      if (jj >= o) {
        H = fmaf(P, Hp, H);
        P *= Pp;
      }
    }
  }
  static __device__ __forceinline__ void scan_down(float& Q, float& C) {  // inclusive, lanes j..G-1
    const int jj = j();
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
      const float Qs = __shfl_down(Q, o, G), Cs = __shfl_down(C, o, G);
      if (jj + o < G) {
        C = fmaf(Q, Cs, C);
        Q *= Qs;
      }
    }
  }
  static __device__ __forceinline__ float prev(float v, float first) {  // lane j-1; `first` in lane 0
    const float p = __shfl_up(v, 1, G);
    return j() == 0 ? first : p;
  }
  static __device__ __forceinline__ float next(float v, float last) {  // lane j+1; `last` in lane G-1
    const float p = __shfl_down(v, 1, G);
    return j() == G - 1 ? last : p;
  }
  static __device__ __forceinline__ float sum(float v) { return group_sum<G>(v); }
};

// DPP move inside 16-lane rows; lanes whose source falls outside the row get `old`.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kRowShl = 0x100;     // row_shl:n -> lane i reads lane i+n
constexpr int kRowShr = 0x110;     // row_shr:n -> lane i reads lane i-n
constexpr int kRowMirror = 0x140;  // lane i reads lane 15-i

// DPP move inside 16-lane rows with zero fill for lanes whose source falls
// outside the row (lets the compiler fold the move into the consuming op).
template <int CTRL> __device__ __forceinline__ float dpp_zero(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <> struct Grp<16> {  // one DPP row per group: all cross-lane steps are VALU
  // One scan step is two DPP instructions: H += P·H[lane∓o] with a zero
  // source for a lane without a partner (bound_ctrl), then P *= P[lane∓o]
  // with no write for a lane without a partner (P unchanged: P·1). The
  // compiler does not fold a float DPP move into a v_fmac / v_mul itself
  // (1.0 is not an identity it recognises), which costs three extra moves
  // per step. Each block starts with s_nop 1: a DPP read needs two wait
  // states after the VALU write of its source, whichever instruction the
  // compiler placed just before.
  template <int O> static __device__ __forceinline__ void up(float& P, float& H) {
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:%2 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(H) : "v"(P), "n"(O));
    asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_shr:%1 row_mask:0xf bank_mask:0xf" : "+v"(P) : "n"(O));
  }
  template <int O> static __device__ __forceinline__ void down(float& Q, float& C) {
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shl:%2 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(C) : "v"(Q), "n"(O));
    asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_shl:%1 row_mask:0xf bank_mask:0xf" : "+v"(Q) : "n"(O));
  }
  static __device__ __forceinline__ void scan_up(float& P, float& H) {
    up<1>(P, H);
    up<2>(P, H);
    up<4>(P, H);
    up<8>(P, H);
  }
  static __device__ __forceinline__ void scan_down(float& Q, float& C) {
    down<1>(Q, C);
    down<2>(Q, C);
    down<4>(Q, C);
    down<8>(Q, C);
  }
  static __device__ __forceinline__ float prev(float v, float first) { return dpp_mov<kRowShr + 1>(v, first); }
  static __device__ __forceinline__ float next(float v, float last) { return dpp_mov<kRowShl + 1>(v, last); }
  static __device__ __forceinline__ float sum(float v) {
    v += __uint_as_float(dpp<kDppXor1>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kDppXor2>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kRowMirror>(__float_as_uint(v)));
    return v;
  }
};

// Two DPP rows per group (lanes 0-31 and 32-63 of the wave): the row steps
// of Grp<16>, then one step across the row pair. Forward direction: the odd
// row combines with the last lane of the even row (DPP row_bcast:15, rows 1
// and 3 written). Backward direction: the even row combines with the first
// lane of the odd row, read as a scalar (lanes 16 and 48).
template <> struct Grp<32> {
  static __device__ __forceinline__ int j() { return lane_id() & 31; }
  static __device__ __forceinline__ bool odd_row() { return (lane_id() & 16) != 0; }
  // scalar of lane 16 (group 0) or 48 (group 1), as seen by this lane
  static __device__ __forceinline__ float pair_first(float v) {
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return lane_id() < 32 ? a : b;
  }
  static __device__ __forceinline__ void scan_up(float& P, float& H) {
    Grp<16>::scan_up(P, H);
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_bcast:15 row_mask:0xa bank_mask:0xf" : "+v"(H) : "v"(P));
    asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf" : "+v"(P));
  }
  static __device__ __forceinline__ void scan_down(float& Q, float& C) {
    Grp<16>::scan_down(Q, C);
    const float Qn = pair_first(Q), Cn = pair_first(C);
    if (!odd_row()) {
      C = fmaf(Q, Cn, C);
      Q *= Qn;
    }
  }
  static __device__ __forceinline__ float prev(float v, float first) {  // lane j-1; `first` in lane 0
    const float in_row = dpp_mov<kRowShr + 1>(v, first);  // lane 16 keeps `first` here
    const float from_prev_row = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
    return j() == 16 ? from_prev_row : in_row;
  }
  static __device__ __forceinline__ float next(float v, float last) {  // lane j+1; `last` in lane 31
    const float in_row = dpp_mov<kRowShl + 1>(v, last);  // lane 15 keeps `last` here
    const float from_next_row = pair_first(v);
    return j() == 15 ? from_next_row : in_row;
  }
  // the group's sum in every lane of its even row (lane 0 included)
  static __device__ __forceinline__ float sum(float v) {
    v = Grp<16>::sum(v);
    return v + pair_first(v);
  }
};

}  // namespace bcm
