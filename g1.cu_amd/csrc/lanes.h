// Lane-group primitives for the world-per-32-lanes mapping on CDNA4 (wave64 = two worlds).
//
// A "group" is the 32 lanes of one half of a wave64; each group owns one world. Cross-lane
// traffic goes through ds_bpermute (__shfl) restricted to the group, and the butterfly sum gives
// every lane of the group the bit-identical result (IEEE addition is commutative, and each
// butterfly stage combines the same two partial sums on both partner lanes).
#pragma once
#include <hip/hip_runtime.h>

namespace g1k {

constexpr int kGroup = 32;

__device__ __forceinline__ int group_lane() { return threadIdx.x & (kGroup - 1); }
__device__ __forceinline__ int group_id() { return threadIdx.x >> 5; }

__device__ __forceinline__ float gshfl(float v, int src) { return __shfl(v, src, kGroup); }
__device__ __forceinline__ int gshfl(int v, int src) { return __shfl(v, src, kGroup); }

__device__ __forceinline__ float gsum(float v) {
#pragma unroll
  for (int m = kGroup / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kGroup);
  return v;
}

// maximum of an int over the whole wave (both groups): uniform trip counts for loops whose
// length depends on per-world data
__device__ __forceinline__ int wave_max(int v) {
  int o = __shfl_xor(v, 32, 64);
  return v > o ? v : o;
}

// 8-bit contact mask of this group from a wave ballot
__device__ __forceinline__ unsigned group_ballot8(bool pred) {
  unsigned long long m = __ballot(pred);
  return (unsigned)(m >> (32 * group_id())) & 0xFFu;
}

}  // namespace g1k
