// policy.h -- observation, frozen normalisation, policy MLP on fp32 MFMA, Gaussian sampling.
//
// One workgroup (8 waves) owns a tile of 32 worlds. Activations live in LDS ([32][K] row-major,
// padded); each dense layer is a [32 x K] . [K x N] contraction on v_mfma_f32_32x32x2f32 with the
// weights pre-packed k-pair-major (Wp[k/2][n][k%2]) so every B-operand load is one contiguous
// 256-byte line. Waves take 32-column output tiles round-robin. The mu (29) and value (1) heads are
// fused into one 32-wide tile.
//
// Reference: obs src/g1_env.cu:46-81; normalise/clamp :298-302; MLP :219-239 (AC of
// scripts/ppo.py:85-99, packing scripts/ppo_fused.py:35-44); sampling + log-prob :308-318.
#pragma once
#include <hip/hip_runtime.h>

#include "g1_model_tables.h"
#include "physics.h"

namespace g1k {

constexpr int kObs = 100, kAct = 29;
constexpr int kTileWorlds = 32;
constexpr int kPolicyThreads = 512;
constexpr int kPolicyWaves = kPolicyThreads / 64;
constexpr int kMaxHidden = 512;
constexpr int kMaxLayers = 4;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Policy shape: nl hidden layers (ELU or tanh), then the fused [mu | v | pad] head.
struct PolicyShape {
  int nl;
  int hid[kMaxLayers];
  int act;   // 0 tanh, 1 ELU
};

// Offsets of each packed layer inside the packed buffer (floats). Layer l: weights Kp/2 x Np x 2,
// then bias Np. The head is layer nl with Np = 32 (mu 0..28, value 29, zero pad).
struct PackedPolicy {
  const float* Wp;
  long woff[kMaxLayers + 1];
  long boff[kMaxLayers + 1];
  int K[kMaxLayers + 1];   // padded to even
  int Np[kMaxLayers + 1];  // padded to 32
  const float* log_std;    // 29 values (torch order, unpacked tail of W)
};

__device__ __forceinline__ float act_fn(float x, int act) {
  return act == 0 ? tanhf(x) : (x > 0.f ? x : expm1f(x));
}

// obs i of one world (reference: src/g1_env.cu:69-81)
__device__ __forceinline__ float obs_value(const float* qp, const float* qv, const float* pa, int i) {
  if (i < 6) return qv[i];
  if (i < 9) {
    const float w = qp[3], x = qp[4], y = qp[5], z = qp[6];
    // third row of quat2mat(q), negated: R^T (0,0,-1)
    const float r = (i == 6)   ? 2.f * __builtin_fmaf(-w, y, x * z)
                    : (i == 7) ? 2.f * __builtin_fmaf(w, x, y * z)
                               : __builtin_fmaf(-2.f, __builtin_fmaf(y, y, x * x), 1.f);
    return -r;
  }
  if (i < 38) return qp[7 + (i - 9)];
  if (i < 67) return qv[6 + (i - 38)];
  if (i < 96) return pa[i - 67];
  return i == 96 ? 0.8f : 0.f;
}

// ---------------------------------------------------------------- Philox4x32-10 (Salmon et al.,
// "Parallel random numbers: as easy as 1, 2, 3", SC'11): counter-based, so every (world, control
// step, stream, index) draw is reproducible and independent of launch order.
struct U4 { unsigned x, y, z, w; };
__host__ __device__ __forceinline__ U4 philox4x32_10(U4 c, unsigned k0, unsigned k1) {
  const unsigned M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const unsigned long long p0 = (unsigned long long)M0 * c.x;
    const unsigned long long p1 = (unsigned long long)M1 * c.z;
    const unsigned hi0 = (unsigned)(p0 >> 32), lo0 = (unsigned)p0;
    const unsigned hi1 = (unsigned)(p1 >> 32), lo1 = (unsigned)p1;
    c = {hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += W0; k1 += W1;
  }
  return c;
}
// uniform in (0, 1): 24 high bits, offset half an ulp so 0 is never produced
__host__ __device__ __forceinline__ float u01(unsigned v) { return ((v >> 8) + 0.5f) * (1.0f / 16777216.0f); }

enum RngStream : unsigned { kStreamAction = 0, kStreamReset = 1, kStreamInit = 2 };

__device__ __forceinline__ float rng_normal(unsigned long long seed, int w, unsigned step, unsigned stream, int i) {
  U4 r = philox4x32_10(U4{(unsigned)w, step, stream, (unsigned)i}, (unsigned)seed, (unsigned)(seed >> 32));
  const float u1 = u01(r.x), u2 = u01(r.y);
  return sqrtf(-2.f * logf(u1)) * cosf(6.2831853071795864f * u2);
}
__device__ __forceinline__ float rng_pm1(unsigned long long seed, int w, unsigned step, unsigned stream, int i) {
  U4 r = philox4x32_10(U4{(unsigned)w, step, stream, (unsigned)i}, (unsigned)seed, (unsigned)(seed >> 32));
  return u01(r.x) * 2.f - 1.f;
}

// ---------------------------------------------------------------- one dense layer on MFMA
// out[m][n] = act(sum_k in[m][k] W[n][k] + b[n]) for the 32 worlds of the tile.
// in: LDS [32][ldi], out: LDS [32][ldo]; wave wv takes n-tiles wv, wv + kPolicyWaves, ...
__device__ __forceinline__ void mfma_layer(const float* __restrict__ in, int ldi, float* __restrict__ out, int ldo,
                                           const float* __restrict__ Wp, const float* __restrict__ bias, int K,
                                           int Np, int act, bool apply_act) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int mrow = lane & 31, khalf = lane >> 5;
  for (int nt = wv; nt < Np / 32; nt += kPolicyWaves) {
    const int n0 = nt * 32;
    const float bv = bias[n0 + mrow];
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = bv;
    const float* wcol = Wp + (long)(n0 + mrow) * 2 + khalf;
    const float* arow = in + mrow * ldi + khalf;
    // k-pairs in batches of kB: all kB weight loads (L2 latency) are in flight before the first
    // MFMA of the batch waits on them
    constexpr int kB = 16;
    const int K2 = K / 2;
    int kk = 0;
    for (; kk + kB <= K2; kk += kB) {
      float a[kB], b[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        b[u] = wcol[(long)(kk + u) * Np * 2];
        a[u] = arow[2 * (kk + u)];
      }
#pragma unroll
      for (int u = 0; u < kB; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b[u], acc, 0, 0, 0);
    }
    for (; kk < K2; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(arow[2 * kk], wcol[(long)kk * Np * 2], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = (i & 3) + 4 * khalf + 8 * (i >> 2);
      const float v = acc[i];
      out[m * ldo + n0 + mrow] = apply_act ? act_fn(v, act) : v;
    }
  }
}

// The fused 32-wide head has a single output tile: its K range is split over the waves and the
// partial tiles are summed through LDS in wave order (scratch: kPolicyWaves x 32 x 32 floats, not
// aliasing `in`; `out` may alias `in`: every wave has finished reading `in` at the barrier before
// the sum is written).
__device__ __forceinline__ void mfma_head_splitk(const float* in, int ldi, float* out, int ldo,
                                                 float* __restrict__ scratch, const float* __restrict__ Wp,
                                                 const float* __restrict__ bias, int K) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int mrow = lane & 31, khalf = lane >> 5;
  constexpr int Np = 32;
  const int K2 = K / 2;
  const int q = (K2 + kPolicyWaves - 1) / kPolicyWaves;
  const int k0 = wv * q, k1 = min(K2, k0 + q);
  f32x16 acc;
  const float bv = wv == 0 ? bias[mrow] : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = bv;
  const float* wcol = Wp + (long)mrow * 2 + khalf;
  const float* arow = in + mrow * ldi + khalf;
  constexpr int kB = 16;
  int kk = k0;
  for (; kk + kB <= k1; kk += kB) {
    float a[kB], b[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      b[u] = wcol[(long)(kk + u) * Np * 2];
      a[u] = arow[2 * (kk + u)];
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b[u], acc, 0, 0, 0);
  }
  for (; kk < k1; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(arow[2 * kk], wcol[(long)kk * Np * 2], acc, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = (i & 3) + 4 * khalf + 8 * (i >> 2);
    scratch[(wv * 32 + m) * 32 + mrow] = acc[i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * 32; idx += kPolicyThreads) {
    const int m = idx >> 5, n = idx & 31;
    float v = scratch[m * 32 + n];
#pragma unroll
    for (int w = 1; w < kPolicyWaves; ++w) v = v + scratch[(32 * w + m) * 32 + n];
    out[m * ldo + n] = v;
  }
}

}  // namespace g1k
