// policy.h -- observation, frozen normalisation, policy MLP on fp32 MFMA, Gaussian sampling.
//
// One workgroup (8 waves) owns a tile of 32 worlds. Activations live in one LDS buffer per tile
// ([32][ld], k-octet interleaved, padded rows; each layer replaces its input); each dense layer is
// a [32 x K] . [K x N] contraction on v_mfma_f32_32x32x2f32 with the weights pre-packed
// k-octet-major, so the operands of four MFMA steps are one float4 global load (B) and one 16-byte
// LDS read (A) per lane. Waves take 32-column output tiles round-robin. The mu (29) and value (1)
// heads are fused into one 32-wide tile.
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

// Offsets of each packed layer inside the packed buffer (floats). Layer l: weights Kp/8 x Np x 2 x 4
// (k-octet-major, see mfma_layer), then bias Np. The head is layer nl with Np = 32 (mu 0..28,
// value 29, zero pad).
struct PackedPolicy {
  const float* Wp;
  long woff[kMaxLayers + 1];
  long boff[kMaxLayers + 1];
  int K[kMaxLayers + 1];   // padded to a multiple of 8
  int Np[kMaxLayers + 1];  // padded to 32
  const float* log_std;    // 29 values (torch order, unpacked tail of W)
};

// Hidden-layer activations of the policy MLP (k_policy and the one-launch tile), branch-free so
// that they issue between MFMAs. tanh: below |x| = 1/8 the odd series to x^7 (truncation < 2e-10),
// above it 1 - 2 / (e^{2|x|} + 1) with the hardware exp2 (absolute error ~1e-7, no cancellation);
// the sign restored. ELU: x for x > 0, else e^x - 1, below |x| = 1/8 by the series to x^5
// (truncation < 6e-9). A layer's K sums over at most 512 such values, so the outputs stay far
// inside the policy outputs' 1e-5 bound. ACT: 0 tanh, 1 ELU.
template <int ACT>
__device__ __forceinline__ float act_tile(float x) {
  const float a = __builtin_fabsf(x);
  if (ACT == 0) {
    const float a2 = a * a;
    const float ser = __builtin_fmaf(a * a2, __builtin_fmaf(a2, __builtin_fmaf(a2, -17.f / 315.f, 2.f / 15.f), -1.f / 3.f), a);
    const float e = __builtin_amdgcn_exp2f(a * 2.8853900817779268f);   // e^{2a}
    const float big = 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
    const float r = a < 0.125f ? ser : big;
    return __builtin_copysignf(r, x);
  } else {
    const float ser = x * __builtin_fmaf(x, __builtin_fmaf(x, __builtin_fmaf(x, __builtin_fmaf(x, 1.f / 120.f, 1.f / 24.f), 1.f / 6.f), 0.5f), 1.f);
    const float em1 = __builtin_amdgcn_exp2f(x * 1.4426950408889634f) - 1.f;
    const float neg = a < 0.125f ? ser : em1;
    return x > 0.f ? x : neg;
  }
}

__device__ __forceinline__ float act_fn(float x, int act) { return act == 0 ? act_tile<0>(x) : act_tile<1>(x); }

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

// the two standard normals of one Box-Muller draw (counter index i: actions 2i and 2i + 1)
__device__ __forceinline__ void rng_normal2(unsigned long long seed, int w, unsigned step, unsigned stream, int i,
                                            float& z0, float& z1) {
  U4 r = philox4x32_10(U4{(unsigned)w, step, stream, (unsigned)i}, (unsigned)seed, (unsigned)(seed >> 32));
  const float u1 = u01(r.x), u2 = u01(r.y);
  const float rad = sqrtf(-2.f * logf(u1));
  float sn, cs;
  sincosf(6.2831853071795864f * u2, &sn, &cs);
  z0 = rad * cs;
  z1 = rad * sn;
}
__device__ __forceinline__ float rng_pm1(unsigned long long seed, int w, unsigned step, unsigned stream, int i) {
  U4 r = philox4x32_10(U4{(unsigned)w, step, stream, (unsigned)i}, (unsigned)seed, (unsigned)(seed >> 32));
  return u01(r.x) * 2.f - 1.f;
}

// ---------------------------------------------------------------- dense layers on MFMA
// v_mfma_f32_32x32x2f32 step kk: lane (mrow = lane & 31, khalf = lane >> 5) supplies A = x[mrow][2kk
// + khalf] and B = W[n0 + mrow][2kk + khalf]. Four consecutive steps (one k-octet o: k = 8o + 2j +
// khalf, j = 0..3) take their operands from one 16-byte load each:
// * weights packed k-octet-major, Wp[o][n][khalf][j] = W[n][8o + 2j + khalf] (K padded to a multiple
//   of 8 with zero rows): the 64 lanes' float4 loads of one octet are one contiguous 1 KB line;
// * activations in LDS k-octet interleaved, X[m][kperm(k)] with kperm(8o + 2j + khalf) = 8o +
//   4 khalf + j, so a lane's four A operands are one ds_read_b128.
__host__ __device__ __forceinline__ int kperm(int k) { return (k & ~7) | ((k & 1) << 2) | ((k >> 1) & 3); }

// acc += A . B over k-octets [o0, o1) of one 32-column tile (B base at the tile's column), in
// batches of kO octets whose loads are all in flight before the batch's MFMAs
template <int kO>
__device__ __forceinline__ void mfma_octets(f32x16& acc, const float* __restrict__ arow,
                                            const float4* __restrict__ wq, long wstride, int o0, int o1) {
  int o = o0;
  for (; o + kO <= o1; o += kO) {
    float4 b[kO], av[kO];
#pragma unroll
    for (int u = 0; u < kO; ++u) {
      b[u] = wq[(long)(o + u) * wstride];
      av[u] = *reinterpret_cast<const float4*>(arow + 8 * (o + u));
    }
#pragma unroll
    for (int u = 0; u < kO; ++u) {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].x, b[u].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].y, b[u].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].z, b[u].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].w, b[u].w, acc, 0, 0, 0);
    }
  }
  // the last partial batch: its loads are also all issued before its MFMAs (rem is wave-uniform)
  const int rem = o1 - o;
  if (rem > 0) {
    float4 b[kO - 1], av[kO - 1];
#pragma unroll
    for (int u = 0; u < kO - 1; ++u)
      if (u < rem) {
        b[u] = wq[(long)(o + u) * wstride];
        av[u] = *reinterpret_cast<const float4*>(arow + 8 * (o + u));
      }
#pragma unroll
    for (int u = 0; u < kO - 1; ++u)
      if (u < rem) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].x, b[u].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].y, b[u].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].z, b[u].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].w, b[u].w, acc, 0, 0, 0);
      }
  }
}

// mfma_octets for two output tiles of the same input rows (acc0: weights wq0, acc1: wq1): the A
// operands are read once for both, and the two tiles' MFMAs alternate, so consecutive MFMAs do not
// depend on each other. Each tile accumulates its octets in the same order as mfma_octets. The
// weights are double-buffered: the next batch's global loads are issued before the current batch's
// MFMAs (indices clamped to the last octet so every load is issued on every path; the surplus is
// unused).
template <int kO>
__device__ __forceinline__ void mfma_octets2(f32x16& acc0, f32x16& acc1, const float* __restrict__ arow,
                                             const float4* __restrict__ wq0, const float4* __restrict__ wq1,
                                             long wstride, int o0, int o1) {
  if (o0 >= o1) return;
  const int last = o1 - 1;
  float4 b0[kO], b1[kO];
#pragma unroll
  for (int u = 0; u < kO; ++u) {
    b0[u] = wq0[(long)min(o0 + u, last) * wstride];
    b1[u] = wq1[(long)min(o0 + u, last) * wstride];
  }
  for (int o = o0; o < o1; o += kO) {
    float4 n0[kO], n1[kO], av[kO];
#pragma unroll
    for (int u = 0; u < kO; ++u) {
      n0[u] = wq0[(long)min(o + kO + u, last) * wstride];
      n1[u] = wq1[(long)min(o + kO + u, last) * wstride];
    }
#pragma unroll
    for (int u = 0; u < kO; ++u) av[u] = *reinterpret_cast<const float4*>(arow + 8 * min(o + u, last));
#pragma unroll
    for (int u = 0; u < kO; ++u) {
      if (o + u < o1) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].x, b0[u].x, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].x, b1[u].x, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].y, b0[u].y, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].y, b1[u].y, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].z, b0[u].z, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].z, b1[u].z, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].w, b0[u].w, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u].w, b1[u].w, acc1, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < kO; ++u) { b0[u] = n0[u]; b1[u] = n1[u]; }
  }
}

// Columns of a tile row that hold the tile's state during the observation (past the first layer's
// K = 104 interleaved input columns).
constexpr int kPolicyStage = 128;
// and, in rows 0..9, the 3 x 100 normalisation constants (32 per row)
constexpr int kPolicyConst = kPolicyStage + 100;
// output tiles of one wave in a hidden layer (32 columns each, dealt round-robin over the waves)
constexpr int kLayerTiles = (kMaxHidden / 32 + kPolicyWaves - 1) / kPolicyWaves;
// k-octets whose operands one wave holds in flight (two tiles per CU at 4 waves per SIMD: <= 128
// VGPRs per wave)
constexpr int kLayerBatch = 4;
// the same for the two-tile loop, per buffer of its double-buffered weights
constexpr int kPairBatch = 2;

// out[m][n] = act(sum_k in[m][k] W[n][k] + b[n]) for the 32 worlds of the tile, written over its
// input: buf [32][ld] holds the input k-octet interleaved. Wave wv computes the output tiles wv,
// wv + kPolicyWaves, .. into registers, the block barrier ends every read of the input, then the
// activated outputs replace it (columns interleaved for the next layer) and a second barrier
// publishes them.
__device__ __forceinline__ void mfma_layer_inplace(float* buf, int ld, const float* __restrict__ Wp,
                                                   const float* __restrict__ bias, int K, int Np, int act) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int mrow = lane & 31, khalf = lane >> 5;
  static_assert(kLayerTiles == 2, "a wave takes at most two output tiles of a layer");
  f32x16 acc[kLayerTiles];
  const int nt0 = wv, nt1 = wv + kPolicyWaves;
  const float4* wq0 = reinterpret_cast<const float4*>(Wp) + (long)(nt0 * 32 + mrow) * 2 + khalf;
  const float4* wq1 = reinterpret_cast<const float4*>(Wp) + (long)(nt1 * 32 + mrow) * 2 + khalf;
  if (nt0 < Np / 32) {
    const float bv0 = bias[nt0 * 32 + mrow];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][i] = bv0;
    if (nt1 < Np / 32) {
      const float bv1 = bias[nt1 * 32 + mrow];
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[1][i] = bv1;
      mfma_octets2<kPairBatch>(acc[0], acc[1], buf + mrow * ld + 4 * khalf, wq0, wq1, (long)Np * 2, 0, K / 8);
    } else {
      mfma_octets<kLayerBatch>(acc[0], buf + mrow * ld + 4 * khalf, wq0, (long)Np * 2, 0, K / 8);
    }
  }
  __syncthreads();   // every wave has read the layer's input
#pragma unroll
  for (int j = 0; j < kLayerTiles; ++j) {
    const int nt = wv + j * kPolicyWaves;
    if (nt < Np / 32) {
      const int nc = kperm(nt * 32 + mrow);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = (i & 3) + 4 * khalf + 8 * (i >> 2);
        buf[m * ld + nc] = act_fn(acc[j][i], act);
      }
    }
  }
  __syncthreads();
}

// The fused 32-wide head has a single output tile: its k-octets are split over the waves, wave wv's
// partial tile goes to columns scr + 32 wv .. of the tile's rows (scr >= K: past the head's input),
// and after a barrier the partial tiles are summed in wave order into columns 0..31 (natural
// order; the input is dead by then).
__device__ __forceinline__ void mfma_head_splitk(float* buf, int ld, int scr, const float* __restrict__ Wp,
                                                 const float* __restrict__ bias, int K) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int mrow = lane & 31, khalf = lane >> 5;
  constexpr int Np = 32;
  const int K8 = K / 8;
  const int q = (K8 + kPolicyWaves - 1) / kPolicyWaves;
  const int o0 = wv * q, o1 = min(K8, o0 + q);
  f32x16 acc;
  const float bv = wv == 0 ? bias[mrow] : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = bv;
  const float4* wq = reinterpret_cast<const float4*>(Wp) + (long)mrow * 2 + khalf;
  if (o0 < o1) mfma_octets<kLayerBatch>(acc, buf + mrow * ld + 4 * khalf, wq, (long)Np * 2, o0, o1);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = (i & 3) + 4 * khalf + 8 * (i >> 2);
    buf[m * ld + scr + 32 * wv + mrow] = acc[i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * 32; idx += kPolicyThreads) {
    const int m = idx >> 5, n = idx & 31;
    const float* row = buf + m * ld + scr;
    float v = row[n];
#pragma unroll
    for (int w = 1; w < kPolicyWaves; ++w) v = v + row[32 * w + n];
    buf[m * ld + n] = v;
  }
}

}  // namespace g1k
