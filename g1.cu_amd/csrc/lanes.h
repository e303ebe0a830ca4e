// Lane-group primitives for the world-per-32-lanes mapping on CDNA4 (wave64 = two worlds).
//
// A "group" is the 32 lanes of one half of a wave64; each group owns one world. Cross-lane
// gathers go through ds_bpermute (__shfl) restricted to the group; the group sum runs on DPP and
// v_permlane16_swap (VALU latency) and gives every lane of the group the bit-identical result.
#pragma once
#include <hip/hip_runtime.h>

namespace g1k {

constexpr int kGroup = 32;

__device__ __forceinline__ int group_lane() { return threadIdx.x & (kGroup - 1); }
__device__ __forceinline__ int group_id() { return threadIdx.x >> 5; }

__device__ __forceinline__ float gshfl(float v, int src) { return __shfl(v, src, kGroup); }
__device__ __forceinline__ int gshfl(int v, int src) { return __shfl(v, src, kGroup); }

// Row rotate (DPP row_ror:N): lane i of each 16-lane row reads lane (i - N) mod 16 of its row.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}

// Sum over the 32 lanes of the group, the same value in every lane. Stage 1 adds the partner
// row (lane i and i^16) with v_permlane16_swap, which exchanges rows 0<->1 and 2<->3 between two
// registers; stages 2-5 add row rotations by 8, 4, 2, 1. After the stage that rotates by m the
// partial sums are periodic with period m within the row, so lane i's partner (i - m) mod 16
// holds the same partial sum as lane i ^ m: every stage adds exactly the operands of the xor
// butterfly (16, 8, 4, 2, 1), and since IEEE addition is commutative the result is bit-identical
// to that butterfly in every lane, without a round trip through the LDS crossbar.
__device__ __forceinline__ float gsum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// gsum when only lanes 0..15 of the group can be nonzero (lanes 16..31 hold +-0): the permlane16
// stage would add those zeros, so it is skipped; the row rotations give every lane of row 0 the
// same sum as gsum's, equal to it except for the sign of an exactly-zero result.
__device__ __forceinline__ float gsum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// gsum when only lanes 0..3 of the group can be nonzero (the others hold +-0): for lanes 0..3 the
// butterfly's stages over 8 and 4 lanes add only zeros, and its last two stages are the quad's xor-2
// and xor-1 exchanges, done here by quad_perm; the same operands in every addition (IEEE addition is
// commutative), so lanes 0..3 get gsum16's result except for the sign of an exactly-zero sum. Lanes
// 4..31 get their own quads' sums.
__device__ __forceinline__ float gsum4(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 2 | (3 << 2) | (0 << 4) | (1 << 6), 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 1 | (0 << 2) | (3 << 4) | (2 << 6), 0xF, 0xF, true));
  return v;
}

// maximum over the wave's two worlds of an int that is uniform within each 32-lane group (a
// per-world count): uniform trip counts for loops whose length depends on per-world data. Read from
// lanes 0 and 32 into scalar registers (no cross-lane LDS round trip), so that the loops and
// branches it bounds compile to scalar compares instead of exec-mask regions.
__device__ __forceinline__ int groups_max(int v) {
  const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 32);
  return a > b ? a : b;
}

// Value of lane I of this lane's aligned 8-lane chain. (Two DPP moves instead of one ds_swizzle:
// the factor's chain levels wait on these broadcasts, and the swizzle's LDS round trip made config 3
// 0.8% slower.)
template <int I>
__device__ __forceinline__ float chain_bcast(float v) {
  static_assert(I >= 0 && I < 8, "lane of the chain");
  // quad_perm [i, i, i, i] (i = I mod 4) gives every quad its lane i; then the quad that does not
  // hold lane I takes the other quad's value (row_shr:4 into banks 1 and 3, or row_shl:4 into
  // banks 0 and 2): two DPP moves, VALU latency instead of an LDS round trip
  constexpr int i = I & 3;
  // (mov_dpp: no old value to materialise; every quad_perm source lane exists)
  const int x = __builtin_amdgcn_mov_dpp(__float_as_int(v), i | (i << 2) | (i << 4) | (i << 6), 0xF, 0xF, true);
  const int y = I < 4 ? __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xA, false)
                      : __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);
  return __int_as_float(y);
}

// DPP moves within 16-lane rows (identical in every row); mov_dpp with bound_ctrl: lanes whose
// source lies outside the row read 0, and no old value has to be materialised
template <int A, int B, int C, int D>
__device__ __forceinline__ float quad_perm(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), A | (B << 2) | (C << 4) | (D << 6), 0xF, 0xF, true));
}

// Chain-to-chain moves at the factor's junctions (chains g on lanes 8g..8g+7 of the group): lane i
// of a 16-lane row takes lane i + 8 (row_shl:8; the upper half of the row reads 0) or lane i - 8
// (row_shr:8; the lower half reads 0), i.e. chain 1 -> 0 and 3 -> 2, or 0 -> 1 and 2 -> 3.
__device__ __forceinline__ float from_next_chain(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x108, 0xF, 0xF, true));
}
__device__ __forceinline__ float from_prev_chain(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x118, 0xF, 0xF, true));
}
// lanes 0..15 of each group take lanes 16..31 (chains 2, 3 -> 0, 1), or lanes 16..31 take lanes
// 0..15 (chains 0, 1 -> 2, 3), by v_permlane16_swap
__device__ __forceinline__ float from_upper_row(float v) {
  return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
}
__device__ __forceinline__ float from_lower_row(float v) {
  return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[0]);
}

// Value of lane I of this lane's group, of its 16-lane row or of its quad, in every lane of that
// unit: W = 32 (I < 32) first makes both 16-lane rows of each group hold the row with lane I (a
// v_permlane16_swap of the value with itself: rows 0 and 2 of the wave in the first result, 1 and
// 3 in the second), then takes lane I mod 16 of each row by DPP row_newbcast; W = 16 (I < 16) the
// row_newbcast alone, W = 4 (I < 4) a quad_perm. No LDS round trip. The DPP move comes last so
// that the compiler can fold it into the instruction that uses the value (a v_fmac_f32 with a DPP
// source operand).
template <int I, int W>
__device__ __forceinline__ float group_bcast(float v) {
  static_assert(I < W && (W == 4 || W == 16 || W == 32), "lane of the unit");
  if constexpr (W == 4) {
    return quad_perm<I, I, I, I>(v);
  } else {
    int x = __float_as_int(v);
    if constexpr (W == 32) {
      const auto p = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
      x = (int)(I < 16 ? p[0] : p[1]);
    }
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x150 + (I & 15), 0xF, 0xF, false));
  }
}

// 8-bit contact mask of this group from a wave ballot
__device__ __forceinline__ unsigned group_ballot8(bool pred) {
  unsigned long long m = __ballot(pred);
  return (unsigned)(m >> (32 * group_id())) & 0xFFu;
}

}  // namespace g1k
