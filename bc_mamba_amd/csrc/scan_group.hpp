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

}  // namespace bcm
