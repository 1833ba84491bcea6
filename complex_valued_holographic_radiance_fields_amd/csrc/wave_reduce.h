// wave_reduce.h — wave64 reductions for gfx950.
//
// transpose_reduce64: every lane holds 64 values v[0..63]; afterwards lane L
// holds sum over all 64 lanes of v[L].  It is a butterfly in which each step
// pairs lanes with a partner (lane xor 32, 16, 15, 7, 2, 1 — six linearly
// independent masks, so the partner sets tile the wave) and each lane keeps
// the half of its remaining values selected by one of its lane bits while
// handing the other half to its partner.  The two cross-row steps use the
// gfx950 v_permlane32_swap / v_permlane16_swap instructions (a swap plus an
// add per value pair); the in-row steps use DPP row_mirror, row_half_mirror
// and quad_perm.  Cost ~141 VALU instructions for 64 values, versus 6 DPP
// adds plus a broadcast per value for 64 independent reductions.
#pragma once

#include <hip/hip_runtime.h>

namespace hrf {

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}

// Wave64 sum of one value; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_f<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);       // row_half_mirror
  v += dpp_f<0x140>(v);       // row_mirror
  v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

template <int CTRL, int HALF, int N>
__device__ __forceinline__ void butterfly_dpp(float (&v)[N], bool sel) {
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const float lo = v[i], hi = v[i + HALF];
    const float send = sel ? lo : hi;
    const float keep = sel ? hi : lo;
    v[i] = keep + dpp_f<CTRL>(send);
  }
}

__device__ __forceinline__ float transpose_reduce64(float (&v)[64]) {
  const int lane = __lane_id();
  // lane xor 32: lanes 0-31 keep v[i], lanes 32-63 keep v[i+32].
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 32]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  // lane xor 16: rows 0,2 keep v[i], rows 1,3 keep v[i+16].
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 16]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  butterfly_dpp<0x140, 8>(v, (lane >> 3) & 1);  // row_mirror: lane xor 15
  butterfly_dpp<0x141, 4>(v, (lane >> 2) & 1);  // row_half_mirror: lane xor 7
  butterfly_dpp<0x4E, 2>(v, (lane >> 1) & 1);   // quad_perm [2,3,0,1]: lane xor 2
  butterfly_dpp<0xB1, 1>(v, lane & 1);          // quad_perm [1,0,3,2]: lane xor 1
  return v[0];
}

// row_sum16: within each row of 16 lanes, every lane holds NVP values
// v[0..NVP) (NVP a multiple of 4, at most 16); afterwards each lane L holds
// in x[0..NVP/4) the sums over the 16 lanes of its row of values
// (NVP/2) b3 + (NVP/4) b2 + i, with b3, b2 bits 3 and 2 of L: two butterfly
// steps that halve the values (lane xor 15 by DPP row_mirror, lane xor 7 by
// row_half_mirror), then plain DPP adds over the remaining partners (lane
// xor 2, xor 1).  The four lanes of a quad end with the same sums.  Cost
// 3 NVP/2 + 3 NVP/4 + NVP/2 instructions (33 at NVP = 12), against 45 for a
// full 16-value transpose.
template <int NVP>
__device__ __forceinline__ void row_sum16(const float (&v)[NVP], float (&x)[NVP / 4]) {
  static_assert(NVP % 4 == 0 && NVP <= 16, "row_sum16 takes 4, 8, 12 or 16 values");
  constexpr int H = NVP / 2, Q = NVP / 4;
  const int lane = __lane_id();
  const bool b3 = (lane >> 3) & 1, b2 = (lane >> 2) & 1;
  float w[H];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float send = b3 ? v[i] : v[i + H];
    const float keep = b3 ? v[i + H] : v[i];
    w[i] = keep + dpp_f<0x140>(send);  // row_mirror: lane xor 15
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const float send = b2 ? w[i] : w[i + Q];
    const float keep = b2 ? w[i + Q] : w[i];
    x[i] = keep + dpp_f<0x141>(send);  // row_half_mirror: lane xor 7
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) x[i] += dpp_f<0x4E>(x[i]);  // quad_perm [2,3,0,1]
#pragma unroll
  for (int i = 0; i < Q; ++i) x[i] += dpp_f<0xB1>(x[i]);  // quad_perm [1,0,3,2]
}

}  // namespace hrf
